"""Inference-only FP32 triangle attention.

Mirrors the reference's FP32 path
``openfold3/core/kernels/turbopairformer/turbopairformer_attention_fp32.py``:
``turbopairformer_attention_fp32(q, k, v, res_mask, pair_bias)`` with raw
(unscaled) q, all inputs FP32, q/k/v ``[*B, O, H, N, D]``, the mask
broadcasting exactly to ``[*B, O, 1, 1, N]`` and the bias to
``[*B, 1, H, N, N]``; returns contiguous FP32 ``[*B, O, N, H, D]``.  No
autograd: calling it with gradients enabled raises.  Products and sums run
in FP32 on the matrix cores (``csrc/attention_f32.hip``); a row whose logits
are all ``-inf`` gives zeros.
"""

from __future__ import annotations

import math

import torch

from . import _native
from .attention import _device_ctx, _device_supported, _storage_order

_PAD_QUANTUM = 64
_DEFAULT_WORKSPACE_BYTES = 64 * 1024 * 1024
_INVOCATIONS = 0


def invocation_count() -> int:
    """Number of completed dispatches through this FP32 implementation."""
    return _INVOCATIONS


def is_attention_fp32_supported(q, k, v, res_mask, pair_bias) -> tuple[bool, str]:
    """Metadata-only verdict (reference ``turbopairformer_attention_fp32.py:45-95``)."""
    if torch.is_grad_enabled():
        return False, "FP32 Triangle Attention is inference-only; use torch.no_grad()"
    named = {"q": q, "k": k, "v": v, "res_mask": res_mask, "pair_bias": pair_bias}
    if any(not isinstance(t, torch.Tensor) for t in named.values()):
        return False, "q/k/v, res_mask, and pair_bias must be tensors"
    if any(t.dtype != torch.float32 for t in named.values()):
        return False, "q/k/v, res_mask, and pair_bias must all be FP32"
    if len({t.device for t in named.values()}) != 1:
        return False, "all inputs must share one device"
    ok, reason = _device_supported(q)
    if not ok:
        return False, reason
    if q.ndim < 5 or any(d <= 0 for d in q.shape):
        return False, "q must have positive shape [*B, O, H, N, D]"
    if k.shape != q.shape or v.shape != q.shape:
        return False, "q/k/v must have identical shapes"
    outer, heads, sequence, head_dim = (int(x) for x in q.shape[-4:])
    if not 1 <= head_dim <= 64:
        return False, "head dimension must be between 1 and 64"
    prefix = tuple(int(x) for x in q.shape[:-4])
    targets = {
        "res_mask": prefix + (outer, 1, 1, sequence),
        "pair_bias": prefix + (1, heads, sequence, sequence),
    }
    for name, target in targets.items():
        try:
            broadcast = torch.broadcast_shapes(tuple(named[name].shape), target)
        except RuntimeError:
            return False, f"{name} does not broadcast to {target}"
        if tuple(broadcast) != target:
            return False, f"{name} must broadcast exactly to {target}"
    return True, "supported inference-only FP32 Triangle Attention"


def validate_inputs(q, k, v, res_mask, pair_bias) -> None:
    """Raise ValueError before any launch if the inference contract is invalid."""
    ok, reason = is_attention_fp32_supported(q, k, v, res_mask, pair_bias)
    if not ok:
        raise ValueError(reason)


def turbopairformer_attention_fp32(q, k, v, res_mask, pair_bias, *,
                                   workspace_bytes: int = _DEFAULT_WORKSPACE_BYTES):
    """Raw-Q FP32 attention, returning contiguous FP32 ``[*B, O, N, H, D]``.

    ``workspace_bytes`` is validated as in the reference
    (``turbopairformer_attention_fp32.py:139-224``); the kernel's own scratch
    (the prescaled bias) is sized by the library.
    """
    validate_inputs(q, k, v, res_mask, pair_bias)
    if isinstance(workspace_bytes, bool) or not isinstance(workspace_bytes, int):
        raise TypeError("workspace_bytes must be an integer")
    outer, heads, sequence, head_dim = (int(x) for x in q.shape[-4:])
    if not 4 * (sequence + head_dim) <= workspace_bytes <= 2**63 - 1:
        raise ValueError("workspace_bytes must hold at least one FP32 score/output row")
    global _INVOCATIONS
    prefix = tuple(int(x) for x in q.shape[:-4])
    batch = math.prod(prefix)
    scale = 1.0 / math.sqrt(head_dim)
    head_pad = (-head_dim) % 4
    seq_pad = (-sequence) % _PAD_QUANTUM
    n_k = sequence + seq_pad
    d_k = head_dim + head_pad
    mask = res_mask.expand(prefix + (outer, 1, 1, sequence)).reshape(batch, outer, sequence)
    bias = pair_bias
    if head_pad:
        q, k, v = (torch.nn.functional.pad(t, (0, head_pad)) for t in (q, k, v))
    if seq_pad:
        q, k, v = (torch.nn.functional.pad(t, (0, 0, 0, seq_pad)) for t in (q, k, v))
        bias = torch.nn.functional.pad(bias, (0, seq_pad, 0, seq_pad))
        mask = torch.nn.functional.pad(mask, (0, seq_pad), value=float("-inf"))
    mask = mask.contiguous()
    tail = tuple(q.shape[-4:])
    qf, kf, vf = (t.reshape((batch,) + tail) for t in (q, k, v))
    orders = {_storage_order(t) for t in (qf, kf, vf)}
    if len(orders) != 1 or None in orders:
        qf, kf, vf = (t.contiguous() for t in (qf, kf, vf))
        seq_major = False
    else:
        seq_major = orders.pop() == "sequence_major"
    bias_prefix = tuple(int(x) for x in bias.shape[:-4])
    aligned = (1,) * (len(prefix) - len(bias_prefix)) + bias_prefix
    if all(x == 1 for x in aligned):
        bias_batches = 1
        bias_k = bias.reshape(1, heads, n_k, n_k).contiguous()
    else:
        bias_batches = batch
        bias_k = bias.expand(prefix + tuple(bias.shape[-4:])).reshape(batch, heads, n_k, n_k).contiguous()
    if any(t.data_ptr() % 16 for t in (qf, kf, vf, mask, bias_k)):
        qf, kf, vf, mask, bias_k = (t.contiguous().clone() for t in (qf, kf, vf, mask, bias_k))
        seq_major = False
    dev = q.device
    out = torch.empty((batch, outer, n_k, heads, d_k), device=dev, dtype=torch.float32)
    ws_bytes = int(_native.query("tpf_attn_forward_f32_workspace_bytes", batch, heads, n_k,
                                 bias_batches))
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
    with _device_ctx(dev):
        _native.call(
            "tpf_attn_forward_f32", qf.data_ptr(), kf.data_ptr(), vf.data_ptr(), mask.data_ptr(),
            bias_k.data_ptr(), out.data_ptr(), None, ws.data_ptr(), ws_bytes, batch, outer, heads,
            n_k, d_k, int(seq_major), bias_batches, scale, _native.stream_of(qf),
        )
    _INVOCATIONS += 1
    if seq_pad or head_pad:
        out = out[:, :, :sequence, :, :head_dim].contiguous()
    return out.reshape(prefix + (outer, sequence, heads, head_dim))


__all__ = [
    "invocation_count",
    "is_attention_fp32_supported",
    "turbopairformer_attention_fp32",
    "validate_inputs",
]
