"""BF16 LayerNorm kernel (csrc/layernorm.hip) against torch's FP32 LayerNorm
on the same bf16 inputs (the FP32-statistics LayerNorm of
openfold3/core/model/primitives/normalization.py:54-78).

Tolerances: the forward output is the FP32 result rounded once to bf16, so
it may differ from torch's by one bf16 rounding step: max-rel <= 8e-3.  dx
is rounded once to bf16 likewise (max-rel <= 8e-3).  dgamma / dbeta are FP32
sums over the same products in another order: max-rel <= 1e-4.  The
parameter gradients are bitwise identical across calls (fixed-order sums).
"""

import pytest
import torch

TOL_BF16 = 8e-3
TOL_PARAM = 1e-4


def _rel(a, b):
    return ((a.float() - b.float()).abs().max() / b.float().abs().max().clamp_min(1e-30)).item()


def _run(x_src, view, C, affine, dev, seed):
    from openfold3_triangle_kernel_amd import layer_norm_bf16

    g = torch.Generator(device=dev).manual_seed(seed)
    w = (1 + 0.2 * torch.randn(C, device=dev, generator=g)) if affine else None
    b = (0.1 * torch.randn(C, device=dev, generator=g)) if affine else None
    x = view(x_src)
    xs = x.detach().requires_grad_(True)
    ws = w.clone().requires_grad_(True) if affine else None
    bs = b.clone().requires_grad_(True) if affine else None
    y = layer_norm_bf16(xs, ws, bs, 1e-5)
    assert y.is_contiguous() and y.dtype == torch.bfloat16 and y.shape == x.shape
    dy = torch.randn(y.shape, device=dev, generator=g).bfloat16()
    grads = torch.autograd.grad(y, [xs] + ([ws, bs] if affine else []), dy)

    xr = x.detach().float().requires_grad_(True)
    wr = w.clone().requires_grad_(True) if affine else None
    br = b.clone().requires_grad_(True) if affine else None
    yr = torch.nn.functional.layer_norm(xr, (C,), wr, br, 1e-5)
    rgrads = torch.autograd.grad(yr, [xr] + ([wr, br] if affine else []), dy.float())

    assert _rel(y, yr) <= TOL_BF16, _rel(y, yr)
    assert grads[0].shape == x.shape and grads[0].dtype == torch.bfloat16
    assert _rel(grads[0], rgrads[0]) <= TOL_BF16, _rel(grads[0], rgrads[0])
    if affine:
        assert _rel(grads[1], rgrads[1]) <= TOL_PARAM, _rel(grads[1], rgrads[1])
        assert _rel(grads[2], rgrads[2]) <= TOL_PARAM, _rel(grads[2], rgrads[2])
        again = torch.autograd.grad(layer_norm_bf16(xs, ws, bs, 1e-5), [ws, bs], dy)
        assert torch.equal(again[0], grads[1]) and torch.equal(again[1], grads[2])
    return grads[0]


@pytest.mark.gpu
@pytest.mark.parametrize("C", [8, 64, 128, 136, 256, 520, 1040, 2048])
def test_layer_norm_channels(gpu, C):
    """Every (lanes, chunks) shape: C/8 = 1 .. 256, ragged chunk counts
    (136 -> 17 chunks on 32 lanes, 520 -> 65 on 64x2, 1040 -> 130 on 64x3)."""
    print(f"layernorm C={C}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(C)
    x = (torch.randn(2, 9, 13, C, device=gpu, generator=g) * 3 + 1).bfloat16()
    _run(x, lambda t: t, C, True, gpu, C)


@pytest.mark.gpu
@pytest.mark.parametrize("affine", [True, False])
def test_layer_norm_transposed_rows(gpu, affine):
    """The ending-node view x.transpose(-2, -3) is read in place and dx keeps
    that view's strides; results equal those of the contiguous copy."""
    print(f"layernorm transposed affine={affine}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(7)
    x = torch.randn(2, 37, 37, 128, device=gpu, generator=g).bfloat16()
    dx_t = _run(x, lambda t: t.transpose(-2, -3), 128, affine, gpu, 11)
    assert dx_t.stride() == x.transpose(-2, -3).stride()
    dx_c = _run(x, lambda t: t.transpose(-2, -3).contiguous(), 128, affine, gpu, 11)
    assert torch.equal(dx_t, dx_c)


@pytest.mark.gpu
def test_layer_norm_shapes(gpu):
    """2-D and 5-D inputs, a row count not a multiple of the rows per
    workgroup, and the pair-stack size N=384 (R = 147456 rows)."""
    print("layernorm shapes", flush=True)
    g = torch.Generator(device=gpu).manual_seed(3)
    for shape in [(1, 64), (1001, 128), (2, 3, 5, 7, 64), (1, 384, 384, 128)]:
        x = torch.randn(shape, device=gpu, generator=g).bfloat16()
        _run(x, lambda t: t, shape[-1], True, gpu, 5)


@pytest.mark.gpu
def test_layer_norm_rejects(gpu):
    from openfold3_triangle_kernel_amd import layer_norm_bf16

    with pytest.raises(ValueError):
        layer_norm_bf16(torch.zeros(4, 12, device=gpu, dtype=torch.bfloat16), None, None)
    with pytest.raises(ValueError):
        layer_norm_bf16(torch.zeros(4, 16, device=gpu), None, None)
