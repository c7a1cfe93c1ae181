"""Inference-only FP32 triangle multiplicative update.

Mirrors ``run_trimul_fp32(module, z, mask)`` of the reference
(``openfold3/core/kernels/turbopairformer/turbopairformer_trimul_fp32.py:155-400``):
pure FP32 storage and arithmetic for an official OpenFold3 TriMul module
(separate ``linear_{a,b}_{p,g}`` or fused ``linear_ab_{p,g}`` projections,
optional linear biases, optional LayerNorm affine parameters with their eps,
outgoing / incoming from ``module._outgoing``), under ``torch.no_grad()``.
All compute runs in ``csrc/trimul_f32.hip`` (FP32 MFMA).  The reference's
chunking arguments are validated and accepted; one MI355X holds the whole
problem (HBM is 288 GB), so no chunking is applied.
"""

from __future__ import annotations

import torch

from . import _native
from .trimul import _device_ctx

_INVOCATIONS = 0
_MAX_C, _MAX_H = 512, 256


def invocation_count() -> int:
    """Number of completed dispatches through this FP32 implementation."""
    return _INVOCATIONS


def _check_parameter(tensor, shape, device, name, *, optional=False):
    if tensor is None and optional:
        return
    if not isinstance(tensor, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if tensor.dtype != torch.float32 or tensor.device != device:
        raise ValueError(f"{name} must be FP32 on {device}")
    if tuple(tensor.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(tensor.shape)}")


def _linear_parts(layer, rows, channels, device, name):
    _check_parameter(layer.weight, (rows, channels), device, name + ".weight")
    bias = getattr(layer, "bias", None)
    _check_parameter(bias, (rows,), device, name + ".bias", optional=True)
    if getattr(layer, "precision", None) not in (None, torch.float32):
        raise ValueError(f"{name}.precision requests a non-FP32 computation")
    return layer.weight, bias


def _normalization_parts(layer, channels, device, name):
    weight = getattr(layer, "weight", None)
    bias = getattr(layer, "bias", None)
    _check_parameter(weight, (channels,), device, name + ".weight", optional=True)
    _check_parameter(bias, (channels,), device, name + ".bias", optional=True)
    eps = getattr(layer, "eps", None)
    if isinstance(eps, bool) or not isinstance(eps, (int, float)) or not 0 < eps < float("inf"):
        raise ValueError(f"{name}.eps must be finite and positive")
    return weight, bias, float(eps)


def _input_parameters(module, channels, hidden, device):
    """[(weight, bias)] for a_p, a_g, b_p, b_g from either projection layout."""
    unfused = ("linear_a_p", "linear_a_g", "linear_b_p", "linear_b_g")
    has_unfused = all(hasattr(module, n) for n in unfused)
    has_fused = all(hasattr(module, n) for n in ("linear_ab_p", "linear_ab_g"))
    if has_unfused == has_fused:
        raise ValueError("TriMul module must expose exactly one fused or unfused projection layout")
    if has_unfused:
        return [_linear_parts(getattr(module, n), hidden, channels, device, n) for n in unfused]
    p, pb = _linear_parts(module.linear_ab_p, 2 * hidden, channels, device, "linear_ab_p")
    g, gb = _linear_parts(module.linear_ab_g, 2 * hidden, channels, device, "linear_ab_g")

    def half(t, lo):
        return None if t is None else (t[:hidden] if lo else t[hidden:])

    return [(p[:hidden], half(pb, True)), (g[:hidden], half(gb, True)),
            (p[hidden:], half(pb, False)), (g[hidden:], half(gb, False))]


def run_trimul_fp32(module, z, mask=None, *, output_row_chunk_size=None,
                    projection_workspace_bytes: int = 128 * 1024 * 1024,
                    contraction_workspace_bytes: int = 512 * 1024 * 1024):
    """Pure FP32 TriMul update of ``z[*B, N, N, C]`` under no_grad."""
    global _INVOCATIONS
    if torch.is_grad_enabled():
        raise RuntimeError(
            "run_trimul_fp32 is inference-only; enter torch.no_grad() or inference_mode()"
        )
    if not isinstance(z, torch.Tensor) or z.device.type != "cuda" or z.dtype != torch.float32:
        raise ValueError("z must be a CUDA FP32 tensor")
    if z.ndim < 3 or any(d <= 0 for d in z.shape):
        raise ValueError("z must have nonempty shape [*B,N,N,C]")
    sequence, pair_columns, channels = (int(x) for x in z.shape[-3:])
    if sequence != pair_columns:
        raise ValueError("z must have square pair axes")
    hidden = getattr(module, "c_hidden", None)
    if type(hidden) is not int or hidden <= 0 or getattr(module, "c_z", None) != channels:
        raise ValueError("module channels must match z, with positive c_hidden")
    if type(getattr(module, "_outgoing", None)) is not bool:
        raise ValueError("module._outgoing must be a bool")
    if output_row_chunk_size is None:
        if type(contraction_workspace_bytes) is not int or contraction_workspace_bytes <= 0:
            raise ValueError("contraction_workspace_bytes must be a positive integer")
    elif type(output_row_chunk_size) is not int or output_row_chunk_size <= 0:
        raise ValueError("output_row_chunk_size must be a positive integer")
    row_bytes = (channels + 4 * hidden + channels) * z.element_size()
    if type(projection_workspace_bytes) is not int or projection_workspace_bytes < row_bytes:
        raise ValueError("projection_workspace_bytes must fit one FP32 normalized/projected row")
    if channels > _MAX_C or hidden > _MAX_H:
        raise ValueError(f"FP32 TriMul supports C <= {_MAX_C} and c_hidden <= {_MAX_H}")
    if mask is not None:
        if not isinstance(mask, torch.Tensor) or mask.device != z.device:
            raise ValueError("mask must be a tensor on z's device")
        if mask.dtype not in (torch.bool, torch.float32):
            raise ValueError("mask must have dtype bool or FP32")
        try:
            mask = torch.broadcast_to(mask, z.shape[:-1])
        except RuntimeError as error:
            raise ValueError("mask must broadcast exactly to z.shape[:-1]") from error
    dev = z.device
    norm_in = _normalization_parts(module.layer_norm_in, channels, dev, "layer_norm_in")
    norm_out = _normalization_parts(module.layer_norm_out, hidden, dev, "layer_norm_out")
    parts = _input_parameters(module, channels, hidden, dev)
    parts.append(_linear_parts(module.linear_g, channels, channels, dev, "linear_g"))
    parts.append(_linear_parts(module.linear_z, channels, hidden, dev, "linear_z"))

    prefix = tuple(int(x) for x in z.shape[:-3])
    batch = 1
    for d in prefix:
        batch *= d
    zf = z.reshape(batch, sequence, sequence, channels).contiguous()
    if mask is None:
        mf = torch.ones((batch, sequence, sequence), device=dev, dtype=torch.float32)
    else:
        mf = mask.reshape(batch, sequence, sequence).to(torch.float32).contiguous()

    def ptr(t):
        return None if t is None else t.detach().contiguous()

    weights = [ptr(w) for w, _ in parts]
    biases = [ptr(b) for _, b in parts]
    lnw = [ptr(t) for t in (norm_in[0], norm_in[1], norm_out[0], norm_out[1])]
    out = torch.empty((batch, sequence, sequence, channels), device=dev, dtype=torch.float32)
    ws_bytes = int(_native.query("tpf_trimul_forward_f32_workspace_bytes", batch, sequence,
                                 channels, hidden))
    if ws_bytes < 0:
        raise ValueError("FP32 TriMul: problem too large for one call")
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)

    def addr(t):
        return None if t is None else t.data_ptr()

    with torch.autocast("cuda", enabled=False), _device_ctx(dev):
        _native.call(
            "tpf_trimul_forward_f32", zf.data_ptr(), mf.data_ptr(),
            *[addr(w) for w in weights], *[addr(b) for b in biases],
            addr(lnw[0]), addr(lnw[1]), norm_in[2], addr(lnw[2]), addr(lnw[3]), norm_out[2],
            int(module._outgoing), batch, sequence, channels, hidden, out.data_ptr(),
            ws.data_ptr(), ws_bytes, _native.stream_of(zf),
        )
    _INVOCATIONS += 1
    return out.reshape(z.shape)


__all__ = ["invocation_count", "run_trimul_fp32"]
