"""Split backward route of triangle attention, for direct callers.

The public facade (``attention.py``) always runs the single-reconstruction
backward.  The reference keeps two split kernels beside it for callers that
want one half of the gradients from their own ``logsumexp`` and ``delta``:
``turbopairformer_triangle_dkdv`` (dK / dV and an optional recomputed
``delta_true``; ``turbopairformer_triangle_dkdv.py:101-174``) and
``turbopairformer_triangle_dq_dbias`` (dQ and the per-batch FP32 dBias;
``turbopairformer_triangle_dq_dbias.py:379-463``).  Here both run the same
gfx950 reconstruction kernel as the facade (``csrc/attention.hip``,
``attn_bwd_kernel`` in its dK/dV-only or dQ/dBias-only mode), so each half
is bitwise the corresponding output of the single-reconstruction backward
on the same inputs.

Tensor contract (as the reference's split functions): q, k, v, and the
returned dq, dk, dv are bf16 ``[B, O, H, N, D]`` (head-major, or the
sequence-major view of a ``[B, O, N, H, D]`` buffer); ``d_output`` bf16
``[B, O, N, H, D]``; ``logsumexp`` and ``delta`` FP32 with ``B*O*H*N``
elements in ``[B, O, H, N]`` order; ``mask`` FP32 additive ``[B, O, 1, 1, N]``;
``pair_bias`` bf16 ``[B, 1, H, N, N]`` (one shared batch, or an expanded
view of one, is read once).  The kernels need ``N % 64 == 0`` and
``D % 8 == 0``, ``8 <= D <= 64``; the softmax scale is ``1/sqrt(D)``.
"""

from __future__ import annotations

import math

import torch

from . import _native
from .attention import _QKV_SEQ_MAJOR, _device_ctx, _storage_order

_KEY_BLOCK = 64  # keys per delta_true partial (one wave's key range)
_MAX_BUDGET = (1 << 62)


def delta_true_partial_elements(sequence: int, heads: int, batch: int,
                                outer: int | None = None) -> int:
    """FP32 elements of the ``delta_true`` partial workspace: one per query
    row and 64-key block, ``[batch, outer, heads, ceil(sequence / 64),
    sequence]`` (``outer=None`` means ``outer = sequence``), as the
    reference's ``turbopairformer_triangle_dkdv.py:75-91``."""
    if outer is None:
        outer = sequence
    blocks = (sequence + _KEY_BLOCK - 1) // _KEY_BLOCK
    return batch * outer * heads * sequence * blocks


def _operands(q, k, v, d_output, logsumexp, delta, mask, pair_bias, fn):
    """Validate the kernel-format operands; returns (dims, layout, flat
    tensors, bias batch count)."""
    if q.dim() != 5 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError(f"{fn}: q, k, v must share one [B, O, H, N, D] shape")
    B, O, H, N, D = (int(x) for x in q.shape)
    if any(t.dtype != torch.bfloat16 for t in (q, k, v, d_output, pair_bias)):
        raise ValueError(f"{fn}: q, k, v, d_output and pair_bias must be bf16")
    if N % 64 or D % 8 or not 8 <= D <= 64:
        raise ValueError(f"{fn}: needs N % 64 == 0 and D % 8 == 0 with 8 <= D <= 64 "
                         f"(got N={N}, D={D})")
    if not (q.is_cuda and k.device == q.device and v.device == q.device):
        raise ValueError(f"{fn}: inputs must be on one GPU")
    orders = {_storage_order(t) for t in (q, k, v)}
    if len(orders) != 1 or None in orders:
        raise ValueError(f"{fn}: q, k, v must share head-major or sequence-major storage")
    layout = _QKV_SEQ_MAJOR if orders == {"sequence_major"} else 0
    if tuple(d_output.shape) != (B, O, N, H, D):
        raise ValueError(f"{fn}: d_output must be [B, O, N, H, D]")
    rows = B * O * H * N
    if logsumexp.numel() != rows or delta.numel() != rows:
        raise ValueError(f"{fn}: logsumexp and delta must hold B*O*H*N values")
    if mask.numel() != B * O * N:
        raise ValueError(f"{fn}: mask must be [B, O, 1, 1, N]")
    if tuple(pair_bias.shape) != (B, 1, H, N, N):
        raise ValueError(f"{fn}: pair_bias must be [B, 1, H, N, N]")
    if B == 1 or pair_bias.stride(0) == 0:
        bias, bias_batches = pair_bias[:1].contiguous(), 1
    else:
        bias, bias_batches = pair_bias.contiguous(), B
    flat = (d_output.contiguous(), logsumexp.reshape(-1).float().contiguous(),
            delta.reshape(-1).float().contiguous(), mask.reshape(-1).float().contiguous(), bias)
    return (B, O, H, N, D), layout, flat, bias_batches


def turbopairformer_triangle_dkdv(q, k, v, d_output, logsumexp, delta, mask, pair_bias, *,
                                  out_dk=None, out_dv=None, emit_delta_true=False,
                                  delta_true_partials=None, out_delta_true=None):
    """dK and dV from the forward's ``logsumexp`` and the caller's ``delta``
    (dS = P (dP - delta)), optionally with ``delta_true`` = sum_k P dP per
    query row (FP32 ``[B, O, H, N]``, from per-64-key-block partials folded in
    ascending block order; not divided by the recomputed sum of P).  Returns
    ``(dk, dv)`` or ``(dk, dv, delta_true)``; supplied output buffers are
    filled and returned (reference ``turbopairformer_triangle_dkdv.py:101-174``)."""
    fn = "turbopairformer_triangle_dkdv"
    (B, O, H, N, D), layout, (dout, lse, dl, msk, bias), bb = _operands(
        q, k, v, d_output, logsumexp, delta, mask, pair_bias, fn)
    dk = torch.empty_like(q) if out_dk is None else out_dk
    dv = torch.empty_like(q) if out_dv is None else out_dv
    for name, t in (("out_dk", dk), ("out_dv", dv)):
        if t.shape != q.shape or t.dtype != torch.bfloat16 or t.stride() != q.stride():
            raise ValueError(f"{fn}: {name} must match q's shape, dtype and storage")
    parts = dtrue = None
    if emit_delta_true:
        need = delta_true_partial_elements(N, H, B, outer=O)
        if delta_true_partials is None:
            parts = torch.empty(need, device=q.device, dtype=torch.float32)
        else:
            if delta_true_partials.numel() < need:
                raise ValueError(f"delta_true_partials has {delta_true_partials.numel()} "
                                 f"elements, but this shape requires {need}")
            parts = delta_true_partials
            if parts.dtype != torch.float32 or not parts.is_contiguous() or parts.data_ptr() % 16:
                raise ValueError(f"{fn}: delta_true_partials must be contiguous, 16-byte "
                                 "aligned FP32")
        dtrue = (torch.empty((B, O, H, N), device=q.device, dtype=torch.float32)
                 if out_delta_true is None else out_delta_true)
        if dtrue.numel() != B * O * H * N or dtrue.dtype != torch.float32 or \
                not dtrue.is_contiguous():
            raise ValueError(f"{fn}: out_delta_true must be contiguous FP32 [B, O, H, N]")
    ws_bytes = int(_native.query("tpf_attn_dkdv_workspace_bytes", B, O, H, N, D, bb))
    ws = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8)
    with _device_ctx(q.device), torch.no_grad():
        _native.call("tpf_attn_dkdv_bf16", q.data_ptr(), k.data_ptr(), v.data_ptr(),
                     dout.data_ptr(), lse.data_ptr(), dl.data_ptr(), msk.data_ptr(),
                     bias.data_ptr(), dk.data_ptr(), dv.data_ptr(), _native.ptr(parts),
                     _native.ptr(dtrue), ws.data_ptr(), ws_bytes, B, O, H, N, D, layout, bb,
                     1.0 / math.sqrt(D), _native.stream_of(q))
    if emit_delta_true:
        return dk, dv, dtrue
    return dk, dv


def turbopairformer_triangle_dq_dbias(q, k, v, d_output, logsumexp, delta, mask, pair_bias, *,
                                      workspace=None, workspace_budget_bytes=None,
                                      query_span=None, batch_chunk=None, debug_full_plane=False,
                                      out_dq=None, out_dbias=None):
    """bf16 dQ and per-batch FP32 dBias ``[B, 1, H, N, N]`` from the forward's
    ``logsumexp`` and the caller's ``delta``; a broadcast bias still needs
    the caller's reduction over its broadcast axes (reference
    ``turbopairformer_triangle_dq_dbias.py:379-463``).

    The workspace plan is this build's (slabs of outer-row runs under
    ``workspace_budget_bytes``, default the facade's budget; the one-slab
    plan with ``debug_full_plane``).  The reference's ``query_span`` and
    ``batch_chunk`` plan overrides select its own tiling and have no
    counterpart here: they are accepted and unused, and results are bitwise
    the same for every plan.  ``workspace`` (any dtype, contiguous) is used
    when it holds at least the plan's bytes."""
    from .attention import sr_workspace_plan

    del query_span, batch_chunk  # plan overrides of the reference's tiling (see above)
    fn = "turbopairformer_triangle_dq_dbias"
    (B, O, H, N, D), layout, (dout, lse, dl, msk, bias), bb = _operands(
        q, k, v, d_output, logsumexp, delta, mask, pair_bias, fn)
    dq = torch.empty_like(q) if out_dq is None else out_dq
    if dq.shape != q.shape or dq.dtype != torch.bfloat16 or dq.stride() != q.stride():
        raise ValueError(f"{fn}: out_dq must match q's shape, dtype and storage")
    dbias = (torch.empty((B, 1, H, N, N), device=q.device, dtype=torch.float32)
             if out_dbias is None else out_dbias)
    if tuple(dbias.shape) != (B, 1, H, N, N) or dbias.dtype != torch.float32 or \
            not dbias.is_contiguous():
        raise ValueError(f"{fn}: out_dbias must be contiguous FP32 [B, 1, H, N, N]")
    budget = _MAX_BUDGET if debug_full_plane else workspace_budget_bytes
    ws_bytes, _ = sr_workspace_plan(B, O, H, N, D, budget)
    if workspace is not None:
        have = workspace.numel() * workspace.element_size()
        if have < ws_bytes or not workspace.is_contiguous():
            raise ValueError(f"{fn}: workspace holds {have} bytes, but this plan requires "
                             f"{ws_bytes}")
        ws, ws_bytes = workspace, have
    else:
        ws = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8)
    with _device_ctx(q.device), torch.no_grad():
        _native.call("tpf_attn_dq_dbias_bf16", q.data_ptr(), k.data_ptr(), v.data_ptr(),
                     dout.data_ptr(), lse.data_ptr(), dl.data_ptr(), msk.data_ptr(),
                     bias.data_ptr(), dq.data_ptr(), dbias.data_ptr(), ws.data_ptr(), ws_bytes,
                     B, O, H, N, D, layout, bb, 1.0 / math.sqrt(D), _native.stream_of(q))
    return dq, dbias


__all__ = [
    "delta_true_partial_elements",
    "turbopairformer_triangle_dkdv",
    "turbopairformer_triangle_dq_dbias",
]
