"""Inference-only FP32 triangle multiplicative update.

Mirrors ``run_trimul_fp32(module, z, mask)`` of the reference
(``openfold3/core/kernels/turbopairformer/turbopairformer_trimul_fp32.py:155-400``):
pure FP32 storage and arithmetic for an official OpenFold3 TriMul module
(separate ``linear_{a,b}_{p,g}`` or fused ``linear_ab_{p,g}`` projections,
optional linear biases, optional LayerNorm affine parameters with their eps,
outgoing / incoming from ``module._outgoing``), under ``torch.no_grad()``.
All compute runs in ``csrc/trimul_f32.hip`` (FP32 MFMA).  As in the
reference, the contraction runs over chunks of output rows: by default as
many rows as fit ``contraction_workspace_bytes`` of FP32 product scratch
([H, rows, N]), or ``output_row_chunk_size`` rows; the LayerNorm and output
projection of a chunk follow it, and the result does not depend on the
chunking (bitwise).  ``projection_workspace_bytes`` is validated as in the
reference; the input projections run over all rows at once.
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


class _ParamError(ValueError):
    """A module parameter that the FP32 kernels cannot take as it is."""


def _fp32_param(owner, attr, shape, device, label, required):
    """``owner.attr`` as an FP32 tensor of ``shape`` on ``device`` (None when
    it is absent and not ``required``); anything else raises _ParamError
    naming ``label``."""
    value = getattr(owner, attr, None)
    if value is None:
        if required:
            raise _ParamError(f"{label} is required")
        return None
    if not isinstance(value, torch.Tensor):
        raise TypeError(f"{label} must be a tensor")
    problems = []
    if value.dtype != torch.float32:
        problems.append(f"dtype {value.dtype}")
    if value.device != device:
        problems.append(f"device {value.device}")
    if problems:
        raise _ParamError(f"{label} must be FP32 on {device} ({', '.join(problems)})")
    if tuple(value.shape) != tuple(shape):
        raise _ParamError(f"{label} must have shape {tuple(shape)}, got {tuple(value.shape)}")
    return value


# The FP32 kernels take six projections: a_p, a_g, b_p, b_g [H, C],
# g [C, C], z [C, H], each with an optional bias.  OpenFold3 modules expose
# the four input projections either as separate layers or as two fused
# [2H, C] layers (a rows first, then b).
_UNFUSED = ("linear_a_p", "linear_a_g", "linear_b_p", "linear_b_g")
_FUSED = ("linear_ab_p", "linear_ab_g")


def _layer(module, name, out_rows, in_cols, device):
    """(weight, bias) of a linear layer, with the FP32-only precision check."""
    layer = getattr(module, name)
    weight = _fp32_param(layer, "weight", (out_rows, in_cols), device, f"{name}.weight", True)
    bias = _fp32_param(layer, "bias", (out_rows,), device, f"{name}.bias", False)
    if getattr(layer, "precision", None) not in (None, torch.float32):
        raise _ParamError(f"{name}.precision requests a non-FP32 computation")
    return weight, bias


def _projections(module, channels, hidden, device):
    """[(weight, bias)] in kernel order a_p, a_g, b_p, b_g, g, z."""
    layouts = [all(hasattr(module, n) for n in names) for names in (_UNFUSED, _FUSED)]
    if layouts.count(True) != 1:
        raise _ParamError("TriMul module must expose exactly one fused or unfused projection layout")
    if layouts[0]:
        inputs = [_layer(module, n, hidden, channels, device) for n in _UNFUSED]
    else:
        (pw, pb), (gw, gb) = (_layer(module, n, 2 * hidden, channels, device) for n in _FUSED)
        rows = (slice(0, hidden), slice(hidden, 2 * hidden))

        def cut(t, r):
            return None if t is None else t[r]

        # Kernel order interleaves projection and gate per branch.
        inputs = [(cut(w, r), cut(b, r)) for r in rows for w, b in ((pw, pb), (gw, gb))]
    return inputs + [_layer(module, "linear_g", channels, channels, device),
                     _layer(module, "linear_z", channels, hidden, device)]


def _norm(module, name, width, device):
    """(weight, bias, eps) of a LayerNorm whose affine parameters may be absent."""
    layer = getattr(module, name)
    weight = _fp32_param(layer, "weight", (width,), device, f"{name}.weight", False)
    bias = _fp32_param(layer, "bias", (width,), device, f"{name}.bias", False)
    eps = getattr(layer, "eps", None)
    ok = isinstance(eps, (int, float)) and not isinstance(eps, bool) and 0 < eps < float("inf")
    if not ok:
        raise _ParamError(f"{name}.eps must be finite and positive")
    return weight, bias, float(eps)


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
    norm_in = _norm(module, "layer_norm_in", channels, dev)
    norm_out = _norm(module, "layer_norm_out", hidden, dev)
    parts = _projections(module, channels, hidden, dev)

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
    if output_row_chunk_size is None:
        # Rows of FP32 product scratch [H, rows, N] that fit the budget
        # (reference turbopairformer_trimul_fp32.py:203-221), at least one.
        row_bytes = hidden * ((sequence + 3) // 4 * 4) * 4
        row_chunk = max(1, min(sequence, contraction_workspace_bytes // row_bytes))
    else:
        row_chunk = min(sequence, output_row_chunk_size)
    ws_bytes = int(_native.query("tpf_trimul_forward_f32_workspace_bytes_chunked", batch,
                                 sequence, channels, hidden, row_chunk))
    if ws_bytes < 0:
        raise ValueError("FP32 TriMul: problem too large for one call")
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)

    def addr(t):
        return None if t is None else t.data_ptr()

    with torch.autocast("cuda", enabled=False), _device_ctx(dev):
        _native.call(
            "tpf_trimul_forward_f32_chunked", zf.data_ptr(), mf.data_ptr(),
            *[addr(w) for w in weights], *[addr(b) for b in biases],
            addr(lnw[0]), addr(lnw[1]), norm_in[2], addr(lnw[2]), addr(lnw[3]), norm_out[2],
            int(module._outgoing), batch, sequence, channels, hidden, row_chunk, out.data_ptr(),
            ws.data_ptr(), ws_bytes, _native.stream_of(zf),
        )
    _INVOCATIONS += 1
    return out.reshape(z.shape)


__all__ = ["invocation_count", "run_trimul_fp32"]
