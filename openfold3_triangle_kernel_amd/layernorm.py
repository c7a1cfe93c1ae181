"""BF16 LayerNorm with FP32 statistics over pair rows (``csrc/layernorm.hip``).

Replaces the torch LayerNorm that OpenFold3's pair-stack modules apply to
their input (``openfold3/core/model/primitives/normalization.py:54-78``:
statistics and affine in FP32, result in the input dtype).  The kernel reads
the rows of a ``[*, I, J, C]`` tensor through its strides, so the transposed
view of the ending-node module is normalised without a copy; the output is
contiguous.  The backward writes dx with the input's own strides and forms
dgamma / dbeta from fixed-order partial sums (deterministic).
"""

from __future__ import annotations

import torch

from . import _native
from .attention import _device_ctx


def _grid_view(x: torch.Tensor) -> torch.Tensor:
    """x as a 4-D [B, I, J, C] view (a copy only when the strides do not allow
    one), channels contiguous, row strides multiples of 8 elements."""
    C = x.shape[-1]
    if x.dim() == 1:
        x = x.reshape(1, 1, 1, C)
    elif x.dim() < 4:
        x = x.reshape((1,) * (4 - x.dim()) + tuple(x.shape))
    elif x.dim() > 4:
        try:
            x = x.view(-1, *x.shape[-3:])
        except RuntimeError:
            x = x.reshape(-1, *x.shape[-3:])
    if (x.stride(-1) != 1 or any(s % 8 for s in x.stride()[:3]) or x.data_ptr() % 16
            or any(s < 0 for s in x.stride())):
        x = x.contiguous()
    return x


def _strides(t: torch.Tensor):
    # A size-1 dimension's stride is never used to address anything.
    return [s if n > 1 else 0 for n, s in zip(t.shape[:3], t.stride()[:3])]


class _LayerNormBf16(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias, eps):
        shape = x.shape
        x4 = _grid_view(x)
        B, I, J, C = x4.shape
        dev = x.device
        w = None if weight is None else weight.detach().float().contiguous()
        b = None if bias is None else bias.detach().float().contiguous()
        y = torch.empty((B, I, J, C), device=dev, dtype=torch.bfloat16)
        mean = torch.empty(B * I * J, device=dev, dtype=torch.float32)
        rstd = torch.empty_like(mean)
        with _device_ctx(dev):
            _native.call("tpf_layer_norm_forward_bf16", x4.data_ptr(), B, I, J, *_strides(x4), C,
                         None if w is None else w.data_ptr(), None if b is None else b.data_ptr(),
                         float(eps), y.data_ptr(), mean.data_ptr(), rstd.data_ptr(),
                         _native.stream_of(x4))
        ctx.save_for_backward(x4, mean, rstd, w)
        ctx.shape = shape
        ctx.param_dtypes = (None if weight is None else weight.dtype,
                            None if bias is None else bias.dtype)
        ctx.set_materialize_grads(False)
        return y.view(shape)

    @staticmethod
    def backward(ctx, dy):
        if dy is None:
            return None, None, None, None
        x4, mean, rstd, w = ctx.saved_tensors
        B, I, J, C = x4.shape
        dev = x4.device
        dy = dy.reshape(B * I * J, C).to(torch.bfloat16).contiguous()
        dx = torch.empty_like(x4)
        want = ctx.needs_input_grad[1] or ctx.needs_input_grad[2]
        dw = db = ws = None
        ws_bytes = 0
        if want:
            dw = torch.empty(C, device=dev, dtype=torch.float32)
            db = torch.empty(C, device=dev, dtype=torch.float32)
            ws_bytes = int(_native.query("tpf_layer_norm_backward_workspace_bytes", B * I * J, C))
            ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
        with _device_ctx(dev):
            _native.call("tpf_layer_norm_backward_bf16", dy.data_ptr(), x4.data_ptr(), B, I, J,
                         *_strides(x4), *_strides(dx), C, mean.data_ptr(), rstd.data_ptr(),
                         None if w is None else w.data_ptr(), dx.data_ptr(),
                         None if dw is None else dw.data_ptr(),
                         None if db is None else db.data_ptr(),
                         None if ws is None else ws.data_ptr(), ws_bytes, _native.stream_of(dy))
        gw = gb = None
        if ctx.needs_input_grad[1] and ctx.param_dtypes[0] is not None:
            gw = dw.to(ctx.param_dtypes[0])
        if ctx.needs_input_grad[2] and ctx.param_dtypes[1] is not None:
            gb = db.to(ctx.param_dtypes[1])
        return dx.view(ctx.shape), gw, gb, None


def layer_norm_bf16(x: torch.Tensor, weight: torch.Tensor | None, bias: torch.Tensor | None,
                    eps: float = 1e-5) -> torch.Tensor:
    """LayerNorm over the last dimension of a CUDA BF16 tensor with FP32
    statistics and FP32 affine parameters; returns contiguous BF16."""
    if not (x.is_cuda and x.dtype == torch.bfloat16):
        raise ValueError("layer_norm_bf16 needs a CUDA bfloat16 tensor")
    C = x.shape[-1]
    if C % 8 or not 8 <= C <= 2048:
        raise ValueError("layer_norm_bf16 needs the channel count to be a multiple of 8 in [8, 2048]")
    for name, p in (("weight", weight), ("bias", bias)):
        if p is not None and tuple(p.shape) != (C,):
            raise ValueError(f"{name} must have shape ({C},)")
    if x.numel() == 0:
        raise ValueError("layer_norm_bf16 needs a nonempty tensor")
    return _LayerNormBf16.apply(x, weight, bias, eps)


__all__ = ["layer_norm_bf16"]
