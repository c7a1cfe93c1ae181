"""Triangle attention with pair bias: validation, padding and autograd facade.

Mirrors the reference facade
``openfold3/core/kernels/turbopairformer/turbopairformer_triangle_attention.py``
(support verdict ``:93-220``, autograd Function ``:223-320``, storage order
``:323-338``, public entry ``:341-472``) on top of the gfx950 kernels in
``csrc/attention.hip``, reached through the C ABI declared in
``include/tpf_amd.h``.

Contract (same as the reference):
  * q, k, v: ``[*B, O, H, N, D]``, q unscaled (the kernels apply 1/sqrt(D));
  * res_mask: additive float ``[*B, O, 1, 1, N]`` (0 keeps, -inf drops);
  * pair_bias: required, ``[*B, 1, H, N, N]``, bf16 or fp32;
  * output: ``[*B, O, N, H, D]``; autograd for q, k, v and pair_bias.

Q/K/V are read in either head-major storage or the sequence-major projection
layout (a contiguous ``[*B, O, N, H, D]`` viewed with ``transpose(-2, -3)``)
without a copy, and their gradients come back in the same storage order.
"""

from __future__ import annotations

import math
import os

import torch

from . import _native

_PAD_QUANTUM = 64  # kernels tile the sequence in 64-key blocks
# Layout bits of the C ABI (include/tpf_amd.h TPF_QKV_SEQ_MAJOR, TPF_BIAS_TRANSPOSED).
_QKV_SEQ_MAJOR = 1
_BIAS_TRANSPOSED = 2
_DBIAS_BF16 = 4  # backward: bf16 dbias in the bias's own storage order
_MAX_HEAD_DIM = 64
_MAX_GRID_YZ = 65_535
_SUPPORT_CACHE: dict = {}
_SUPPORT_CACHE_LIMIT = 4096
_ARCH_CACHE: dict = {}
_INVOCATIONS = 0


def invocation_count() -> int:
    """Number of facade calls (routing regression lock, reference ``:64-66``)."""
    return _INVOCATIONS


def _env_flag(canonical: str, legacy: str, default: str = "1") -> str:
    value = os.environ.get(canonical)
    if value is None:
        value = os.environ.get(legacy, default)
    return value.strip()


def validate_attention_policy() -> None:
    """Backward is always the single-reconstruction kernel; '0' raises.

    Mirrors ``openfold3/core/utils/distributed_contract.py:109-118`` and the
    ``TURBOPAIRFORMER_SR_BACKWARD`` precedence described in ``README.md:84-91``.
    """
    if _env_flag("TURBOPAIRFORMER_SR_BACKWARD", "OPENFOLD3_SR_BACKWARD") == "0":
        raise ValueError(
            "TURBOPAIRFORMER_SR_BACKWARD=0 is not supported: triangle attention "
            "backward always uses single reconstruction"
        )


def shadow_enabled() -> bool:
    """Whether the forward saves the bf16 rounding residual of its output.

    The reference's ``OPENFOLD3_SR_SHADOW`` policy (default ``1``,
    ``openfold3/core/utils/distributed_contract.py:41-44``; read at forward
    time, ``turbopairformer_triangle_attention.py:247-262``): with the
    residual, the backward's row term delta = sum dO * O uses O's f32 value
    instead of its bf16 rounding.  ``TURBOPAIRFORMER_SR_SHADOW`` takes
    precedence over the legacy name; any value other than ``0`` / ``1``
    raises.
    """
    value = _env_flag("TURBOPAIRFORMER_SR_SHADOW", "OPENFOLD3_SR_SHADOW")
    if value not in ("0", "1"):
        raise ValueError(f"OPENFOLD3_SR_SHADOW must be 0 or 1, got {value!r}")
    return value == "1"


def _is_gfx950(device: torch.device) -> bool:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    arch = _ARCH_CACHE.get(idx)
    if arch is None:
        arch = getattr(torch.cuda.get_device_properties(idx), "gcnArchName", "")
        _ARCH_CACHE[idx] = arch
    return arch.split(":")[0] == "gfx950"


def _device_supported(t: torch.Tensor) -> tuple[bool, str]:
    """Device gate: a gfx950 GPU tensor."""
    if t.device.type != "cuda":
        return False, "q/k/v, res_mask, and pair_bias must be GPU tensors"
    if not _is_gfx950(t.device):
        return False, "TurboPairFormer MI355X kernels require a gfx950 device"
    return True, ""


def _device_ctx(device: torch.device):
    return _native.device_ctx(device)


def is_turbopairformer_supported(q, k, v, res_mask, pair_bias) -> tuple[bool, str]:
    """Cached support verdict from metadata only (reference ``:93-220``)."""
    try:
        key = (torch.is_grad_enabled(),) + tuple(
            (tuple(t.shape), t.dtype, t.device, t.requires_grad)
            for t in (q, k, v, res_mask, pair_bias)
        )
    except AttributeError:
        key = None
    if key is not None and key in _SUPPORT_CACHE:
        return _SUPPORT_CACHE[key]
    verdict = _supported_uncached(q, k, v, res_mask, pair_bias)
    if key is not None:
        if len(_SUPPORT_CACHE) >= _SUPPORT_CACHE_LIMIT:
            _SUPPORT_CACHE.clear()
        _SUPPORT_CACHE[key] = verdict
    return verdict


def _supported_uncached(q, k, v, res_mask, pair_bias) -> tuple[bool, str]:
    named = {"q": q, "k": k, "v": v, "res_mask": res_mask, "pair_bias": pair_bias}
    if any(not isinstance(t, torch.Tensor) for t in named.values()):
        return False, "all inputs must be torch.Tensor instances"
    if q.dtype == torch.float32:
        # FP32 q selects the inference implementation and its own contract
        # (reference ``turbopairformer_triangle_attention.py:144-150``).
        from .attention_fp32 import is_attention_fp32_supported

        return is_attention_fp32_supported(q, k, v, res_mask, pair_bias)
    ok, reason = _device_supported(q)
    if not ok:
        return False, reason
    if q.ndim < 5:
        return False, "q must have shape [*B,O,H,N,D]"
    prefix = tuple(q.shape[:-4])
    outer, heads, sequence, head_dim = (int(x) for x in q.shape[-4:])
    if not prefix or any(d <= 0 for d in prefix):
        return False, "requires a positive batch prefix"
    if outer <= 0 or sequence <= 0:
        return False, "requires positive outer and key sequence dimensions"
    if heads < 1 or head_dim < 1 or head_dim > _MAX_HEAD_DIM:
        return False, "requires H>=1 and 1<=D<=64"
    if heads > _MAX_GRID_YZ:
        return False, "head count exceeds the grid-y limit (65535)"
    batch = math.prod(prefix)
    if batch * outer > _MAX_GRID_YZ:
        return False, "flattened batch*outer exceeds the grid-z limit (65535)"
    for name in ("k", "v"):
        if named[name].shape != q.shape:
            return False, f"{name} shape must match q"
    if any(t.dtype != torch.bfloat16 for t in (q, k, v)):
        return False, "q/k/v must be BF16"
    if res_mask.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        return False, "res_mask must be a floating additive mask"
    if tuple(res_mask.shape[-4:]) != (outer, 1, 1, sequence):
        return False, "res_mask tail must be (N,1,1,N)"
    if tuple(pair_bias.shape[-4:]) != (1, heads, sequence, sequence):
        return False, "pair_bias tail must be (1,H,N,N)"
    if pair_bias.dtype not in (torch.bfloat16, torch.float32):
        return False, "pair_bias must be BF16 or FP32"
    if len({t.device for t in named.values()}) != 1:
        return False, "q/k/v, res_mask, and pair_bias must share one device"
    for name in ("res_mask", "pair_bias"):
        t = named[name]
        try:
            bp = torch.broadcast_shapes(prefix, tuple(t.shape[:-4]))
        except RuntimeError:
            return False, f"{name} prefix is not broadcastable to q prefix"
        if tuple(bp) != prefix:
            return False, f"{name} prefix must broadcast exactly to q prefix"
    if res_mask.requires_grad:
        return False, "res_mask must not require gradients"
    return True, "supported"


def _storage_order(t: torch.Tensor) -> str | None:
    """'head_major' (contiguous), 'sequence_major' (transposed projection) or None."""
    if t.is_contiguous():
        return "head_major"
    if t.transpose(-2, -3).is_contiguous() and t.data_ptr() % 16 == 0:
        return "sequence_major"
    return None


# Workspace budget of the backward (bytes).  The reference plans its SR
# backward under a budget too (turbopairformer_triangle_dq_dbias.py:35,
# 150-300); here the budget bounds the dQ partials, the only part of the
# workspace that grows with O * N^2 * H * D / 64: when the full plan exceeds
# it, the reconstruction kernel runs over slabs of outer rows, each slab's dQ
# partials folded before the next slab reuses the space.  Results are
# bitwise equal for every budget.  The default (8 GiB of the MI355X's 288 GB)
# holds config-5 sized problems (N = 768, H = 8, D = 64: a 7.46 GB plan) in
# one slab; larger problems run in slabs (each slab adds a partly filled
# round of workgroups: two slabs at that size cost about 13 %).
DEFAULT_SR_WORKSPACE_BUDGET_BYTES = 8 << 30
_SR_WORKSPACE_BUDGET = DEFAULT_SR_WORKSPACE_BUDGET_BYTES


def set_sr_workspace_budget(budget_bytes: int | None) -> None:
    """Set the backward workspace budget in bytes (None restores the default)."""
    global _SR_WORKSPACE_BUDGET
    if budget_bytes is None:
        _SR_WORKSPACE_BUDGET = DEFAULT_SR_WORKSPACE_BUDGET_BYTES
        return
    budget_bytes = int(budget_bytes)
    if budget_bytes <= 0:
        raise ValueError("workspace_budget_bytes must be positive")
    _SR_WORKSPACE_BUDGET = budget_bytes


def sr_workspace_plan(B: int, O: int, H: int, N: int, D: int,
                      budget_bytes: int | None = None) -> tuple[int, int]:
    """(workspace bytes, slabs) of the backward plan for a kernel-shaped problem
    (N a multiple of 64, D a multiple of 8).  Below the one-run minimum the
    minimum is returned, as the reference's planner does for its irreducible tile."""
    budget = _SR_WORKSPACE_BUDGET if budget_bytes is None else int(budget_bytes)
    ws = int(_native.query("tpf_attn_backward_workspace_bytes_budget", B, O, H, N, D, budget))
    slabs = int(_native.query("tpf_attn_backward_slab_count", B, O, H, N, D, ws))
    return ws, slabs


class _TriangleAttentionFn(torch.autograd.Function):
    """Owns the kernels' saved state (reference ``:223-320``).

    Inputs are the flattened, padded kernel operands; ``bias_k`` is the
    detached kernel bias with ``Bb`` in {1, B} batches, ``source_bias`` keeps
    the autograd edge to the caller's (dtype-converted, padded) bias.
    """

    @staticmethod
    def forward(ctx, q, k, v, mask, bias_k, source_bias, layout, scale, bias_reduce, shadow):
        B, O, H, N, D = (int(x) for x in q.shape)
        out = torch.empty((B, O, N, H, D), device=q.device, dtype=q.dtype)
        lse = torch.empty((B, O, H, N), device=q.device, dtype=torch.float32)
        Bb = int(bias_k.shape[0])
        ws_bytes = int(_native.query("tpf_attn_forward_workspace_bytes", B, H, N, Bb))
        workspace = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8)
        residual = torch.empty_like(out) if shadow else None
        with _device_ctx(q.device):
            if residual is None:
                _native.call(
                    "tpf_attn_forward_bf16",
                    q.data_ptr(), k.data_ptr(), v.data_ptr(), mask.data_ptr(), bias_k.data_ptr(),
                    out.data_ptr(), lse.data_ptr(), workspace.data_ptr(), ws_bytes, B, O, H, N,
                    D, int(layout), Bb, float(scale), _native.stream_of(q),
                )
            else:
                _native.call(
                    "tpf_attn_forward_shadow_bf16",
                    q.data_ptr(), k.data_ptr(), v.data_ptr(), mask.data_ptr(), bias_k.data_ptr(),
                    out.data_ptr(), lse.data_ptr(), residual.data_ptr(), workspace.data_ptr(),
                    ws_bytes, B, O, H, N, D, int(layout), Bb, float(scale),
                    _native.stream_of(q),
                )
        # The residual fixes the delta path for this autograd context; the
        # backward never rereads the environment.
        ctx.save_for_backward(q, k, v, mask, bias_k, out, lse, residual)
        ctx.layout = int(layout)
        ctx.seq_major = bool(layout & _QKV_SEQ_MAJOR)
        ctx.scale = float(scale)
        ctx.bias_reduce = bias_reduce
        ctx.bias_shape = tuple(source_bias.shape)
        ctx.bias_dtype = source_bias.dtype
        return out

    @staticmethod
    def backward(ctx, d_out):
        q, k, v, mask, bias_k, out, lse, residual = ctx.saved_tensors
        B, O, H, N, D = (int(x) for x in q.shape)
        d_out = d_out.contiguous()
        if d_out.dtype != torch.bfloat16:
            d_out = d_out.to(torch.bfloat16)
        with _device_ctx(q.device):
            stream = _native.stream_of(q)
            if ctx.seq_major:
                dq, dk, dv = (
                    torch.empty((B, O, N, H, D), device=q.device, dtype=q.dtype).transpose(2, 3)
                    for _ in range(3)
                )
            else:
                dq, dk, dv = (torch.empty_like(q, memory_format=torch.contiguous_format)
                              for _ in range(3))
            Bb = int(bias_k.shape[0])
            # A bf16 bias gets its gradient from the fold directly: the f32
            # sums rounded once (as the reference's .to(bf16)), stored in the
            # bias's own order (a transposed bias gets a transposed gradient).
            direct = ctx.bias_reduce is None and ctx.bias_dtype == torch.bfloat16
            layout = ctx.layout | (_DBIAS_BF16 if direct else 0)
            dbias = torch.empty((Bb, H, N, N), device=q.device,
                                dtype=torch.bfloat16 if direct else torch.float32)
            ws_bytes = sr_workspace_plan(B, O, H, N, D)[0]
            workspace = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8)
            # delta (with the shadow residual when saved), row statistics and
            # bias preparation in one launch, then reconstruction and folds.
            _native.call(
                "tpf_attn_backward_fused_bf16",
                q.data_ptr(), k.data_ptr(), v.data_ptr(), d_out.data_ptr(), out.data_ptr(),
                0 if residual is None else residual.data_ptr(), lse.data_ptr(),
                mask.data_ptr(), bias_k.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                dbias.data_ptr(), workspace.data_ptr(), ws_bytes,
                B, O, H, N, D, layout, Bb, ctx.scale, stream,
            )
        if direct:
            if ctx.layout & _BIAS_TRANSPOSED:
                dbias = dbias.transpose(-1, -2)
            return dq, dk, dv, None, None, dbias.reshape(ctx.bias_shape), None, None, None, None
        d_bias = dbias
        if ctx.bias_reduce is not None:
            d_bias = ctx.bias_reduce(d_bias)
        d_bias = d_bias.reshape(ctx.bias_shape).to(ctx.bias_dtype)
        return dq, dk, dv, None, None, d_bias, None, None, None, None


def turbopairformer_triangle_attention(q, k, v, res_mask, pair_bias):
    """Validate, pad and run triangle attention, then remove padding.

    Same signature and behaviour as the reference facade
    ``turbopairformer_triangle_attention(q, k, v, res_mask, pair_bias)``
    (``turbopairformer_triangle_attention.py:341-472``).  Unsupported cases raise
    ``ValueError("unsupported TurboPairFormer case: ...")`` before any launch.
    """
    validate_attention_policy()
    ok, reason = is_turbopairformer_supported(q, k, v, res_mask, pair_bias)
    if not ok:
        raise ValueError(f"unsupported TurboPairFormer case: {reason}")
    global _INVOCATIONS
    _INVOCATIONS += 1
    if q.dtype == torch.float32:
        # FP32 inference keeps FP32 storage end to end (reference ``:362-370``).
        from .attention_fp32 import turbopairformer_attention_fp32

        return turbopairformer_attention_fp32(q, k, v, res_mask, pair_bias)
    shadow = shadow_enabled()

    if pair_bias.dtype == torch.float32:
        pair_bias = pair_bias.to(torch.bfloat16)
    prefix = tuple(int(x) for x in q.shape[:-4])
    outer, heads, sequence, head_dim = (int(x) for x in q.shape[-4:])
    batch = math.prod(prefix)
    scale = 1.0 / math.sqrt(head_dim)

    # Head dim: zero-extend to a multiple of 8; the true-D scale is passed to
    # the kernel, so Q is not rescaled (zero channels add nothing to Q.K).
    head_pad = (-head_dim) % 8
    if head_pad:
        q = torch.nn.functional.pad(q, (0, head_pad))
        k = torch.nn.functional.pad(k, (0, head_pad))
        v = torch.nn.functional.pad(v, (0, head_pad))
    # Sequence: pad to the 64-key tile; padded keys get a -inf mask.
    seq_pad = (-sequence) % _PAD_QUANTUM
    if seq_pad:
        pad_qkv = (0, 0, 0, seq_pad)
        q = torch.nn.functional.pad(q, pad_qkv)
        k = torch.nn.functional.pad(k, pad_qkv)
        v = torch.nn.functional.pad(v, pad_qkv)
        pair_bias = torch.nn.functional.pad(pair_bias, (0, seq_pad, 0, seq_pad))
        padded = res_mask.new_full(tuple(res_mask.shape[:-1]) + (sequence + seq_pad,), float("-inf"))
        padded[..., :sequence] = res_mask
        res_mask = padded
    n_k = sequence + seq_pad

    tail = tuple(q.shape[-4:])
    qf, kf, vf = (t.reshape((batch,) + tail) for t in (q, k, v))
    orders = {_storage_order(t) for t in (qf, kf, vf)}
    if len(orders) != 1 or None in orders:
        qf, kf, vf = (t.contiguous() for t in (qf, kf, vf))
        seq_major = False
    else:
        seq_major = orders.pop() == "sequence_major"

    mask_f = (
        res_mask.expand(prefix + tuple(res_mask.shape[-4:]))
        .reshape(batch, outer, n_k)
        .to(torch.float32)
        .contiguous()
    )
    bias_prefix = tuple(int(x) for x in pair_bias.shape[:-4])
    aligned = (1,) * (len(prefix) - len(bias_prefix)) + bias_prefix
    bias_reduce = None
    bias_transposed = False
    if all(x == 1 for x in aligned) or aligned == prefix:
        nbb = 1 if all(x == 1 for x in aligned) else batch
        bias_t = pair_bias.transpose(-1, -2)
        if not pair_bias.is_contiguous() and bias_t.is_contiguous():
            # The ending node's bias.transpose(-1, -2) of a contiguous tensor:
            # the kernels read it in place (TPF_BIAS_TRANSPOSED).
            bias_k = bias_t.reshape(nbb, heads, n_k, n_k).detach()
            bias_transposed = True
        else:
            bias_k = pair_bias.reshape(nbb, heads, n_k, n_k).detach().contiguous()
    else:
        # Partial broadcast: per-batch gradients, then a sum over the
        # broadcast prefix dimensions (reference ``dq_dbias.py:326-376``).
        bias_k = (
            pair_bias.expand(prefix + tuple(pair_bias.shape[-4:]))
            .reshape(batch, heads, n_k, n_k)
            .detach()
            .contiguous()
        )
        red_dims = tuple(i for i, (s, t) in enumerate(zip(aligned, prefix)) if s != t)

        def bias_reduce(d, _p=prefix, _dims=red_dims, _a=aligned):
            d = d.reshape(_p + tuple(d.shape[-3:]))
            return d.sum(dim=_dims, keepdim=True).reshape(_a + tuple(d.shape[-3:]))

    # The kernels use 16-byte vector loads on every operand.
    if mask_f.data_ptr() % 16:
        mask_f = mask_f.clone()
    if bias_k.data_ptr() % 16:
        bias_k = bias_k.clone()
    if any(t.data_ptr() % 16 for t in (qf, kf, vf)):
        qf, kf, vf = (t.contiguous().clone() if t.data_ptr() % 16 else t for t in (qf, kf, vf))
        if len({_storage_order(t) for t in (qf, kf, vf)}) != 1:
            qf, kf, vf = (t.contiguous() for t in (qf, kf, vf))
            seq_major = False
    layout = (_QKV_SEQ_MAJOR if seq_major else 0) | (_BIAS_TRANSPOSED if bias_transposed else 0)
    out = _TriangleAttentionFn.apply(
        qf, kf, vf, mask_f, bias_k, pair_bias, layout, scale, bias_reduce, shadow
    )
    if seq_pad:
        out = out[:, :, :sequence]
    if head_pad:
        out = out[..., :head_dim]
    if not out.is_contiguous():
        out = out.contiguous()
    return out.reshape(prefix + tuple(out.shape[1:]))


def turbo_attention(q, k, v, pair_bias, res_mask=None):
    """Public operator (reference ``README.md:96-115``).

    ``pair_bias`` is required; ``res_mask`` defaults to an all-keep mask.
    """
    if pair_bias is None:
        raise ValueError("pair_bias is required (pass zeros if the model has no bias)")
    if res_mask is None:
        shape = tuple(q.shape[:-3]) + (1, 1, q.shape[-2])
        res_mask = torch.zeros(shape, device=q.device, dtype=torch.float32)
    return turbopairformer_triangle_attention(q, k, v, res_mask, pair_bias)


__all__ = [
    "invocation_count",
    "is_turbopairformer_supported",
    "shadow_enabled",
    "turbo_attention",
    "turbopairformer_triangle_attention",
    "validate_attention_policy",
]
