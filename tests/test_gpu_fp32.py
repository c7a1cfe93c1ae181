"""GPU parity of the inference-only FP32 paths against the numpy FP64 oracle.

Tolerance (north star, fp32 mode): every output at max-rel <= 1e-4,
max-rel = max|got - ref| / max|ref|, oracle in float64 on the same f32
inputs (full f32 values, not bf16-rounded).
"""

import numpy as np
import pytest
import torch

from oracle.attention import attention_forward
from tests._util import max_rel

TOL = 1e-4


def _f32_case(B, O, H, N, D, *, mask_tail=0, full_planes=0, bias_batch=1, seed=0):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(B, O, H, N, D, generator=g) for _ in range(3))
    bias = torch.randn(bias_batch, 1, H, N, N, generator=g) * 2
    mask = torch.zeros(B, O, 1, 1, N)
    if mask_tail:
        tails = torch.randint(0, mask_tail + 1, (B, O), generator=g)
        for b in range(B):
            for o in range(O):
                if int(tails[b, o]):
                    mask[b, o, ..., N - int(tails[b, o]):] = float("-inf")
    if full_planes:
        mask[:, :full_planes] = float("-inf")
    return q, k, v, mask, bias


ATTN_CASES = [
    # B, O, H, N, D, mask_tail, full_planes, bias_batch
    (1, 8, 4, 128, 32, 13, 0, 1),
    (1, 16, 4, 384, 32, 32, 0, 1),
    (1, 6, 4, 100, 12, 7, 1, 1),
    (2, 4, 4, 200, 20, 5, 0, 2),
    (1, 6, 4, 256, 64, 0, 2, 1),
    (1, 2, 8, 96, 48, 9, 0, 1),
    (1, 3, 1, 33, 3, 0, 0, 1),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", ATTN_CASES, ids=lambda c: "B{}O{}H{}N{}D{}".format(*c[:5]))
def test_attention_fp32(gpu, case):
    from openfold3_triangle_kernel_amd import turbopairformer_attention_fp32

    B, O, H, N, D, tail, full, bb = case
    q, k, v, mask, bias = _f32_case(B, O, H, N, D, mask_tail=tail, full_planes=full, bias_batch=bb)
    print(f"fp32 attention case={case}", flush=True)
    with torch.no_grad():
        out = turbopairformer_attention_fp32(*(t.to(gpu) for t in (q, k, v, mask, bias)))
    torch.cuda.synchronize()
    assert out.dtype == torch.float32 and out.shape == (B, O, N, H, D)
    ref, _, _ = attention_forward(q.numpy(), k.numpy(), v.numpy(), mask.numpy(), bias.numpy())
    got = out.cpu().numpy()
    if full:
        assert np.all(got[:, :full] == 0)
    err = max_rel(got, ref)
    assert err <= TOL, err


@pytest.mark.gpu
def test_attention_fp32_sequence_major(gpu):
    """The transposed-projection view (sequence-major storage) is read in place."""
    from openfold3_triangle_kernel_amd import turbopairformer_attention_fp32

    q, k, v, mask, bias = _f32_case(1, 4, 4, 128, 32, mask_tail=9)
    qs, ks, vs = (t.transpose(2, 3).contiguous().to(gpu).transpose(2, 3) for t in (q, k, v))
    with torch.no_grad():
        out = turbopairformer_attention_fp32(qs, ks, vs, mask.to(gpu), bias.to(gpu))
    ref, _, _ = attention_forward(q.numpy(), k.numpy(), v.numpy(), mask.numpy(), bias.numpy())
    assert max_rel(out.cpu().numpy(), ref) <= TOL


def _trimul_module(C, H, outgoing, *, biases=False, fused=False, affine=True, seed=0):
    """An object with the official TriMul module's attribute names, FP32 on CPU."""
    from types import SimpleNamespace

    torch.manual_seed(seed)

    def lin(i, o):
        layer = torch.nn.Linear(i, o, bias=biases)
        with torch.no_grad():
            layer.weight.normal_(0, i ** -0.5)
            if biases:
                layer.bias.normal_(0, 0.2)
        return layer

    m = SimpleNamespace(c_z=C, c_hidden=H, _outgoing=outgoing)
    if fused:
        m.linear_ab_p, m.linear_ab_g = lin(C, 2 * H), lin(C, 2 * H)
    else:
        m.linear_a_p, m.linear_a_g, m.linear_b_p, m.linear_b_g = (lin(C, H) for _ in range(4))
    m.linear_g, m.linear_z = lin(C, C), lin(H, C)
    m.layer_norm_in = torch.nn.LayerNorm(C, eps=1e-5, elementwise_affine=affine)
    m.layer_norm_out = torch.nn.LayerNorm(H, eps=1e-5, elementwise_affine=affine)
    if affine:
        with torch.no_grad():
            for ln in (m.layer_norm_in, m.layer_norm_out):
                ln.weight.normal_(1, 0.1)
                ln.bias.normal_(0, 0.1)
    return m


def _oracle_weights(m, C, H):
    def wb(layer, lo=None):
        w = layer.weight.detach().cpu().double().numpy()
        b = None if layer.bias is None else layer.bias.detach().cpu().double().numpy()
        if lo is not None:
            w = w[:H] if lo else w[H:]
            b = None if b is None else (b[:H] if lo else b[H:])
        return w, b

    if hasattr(m, "linear_ab_p"):
        parts = {"ap": wb(m.linear_ab_p, True), "ag": wb(m.linear_ab_g, True),
                 "bp": wb(m.linear_ab_p, False), "bg": wb(m.linear_ab_g, False)}
    else:
        parts = {"ap": wb(m.linear_a_p), "ag": wb(m.linear_a_g), "bp": wb(m.linear_b_p),
                 "bg": wb(m.linear_b_g)}
    parts["g"], parts["z"] = wb(m.linear_g), wb(m.linear_z)
    w = {}
    for n, (wt, b) in parts.items():
        w["w_" + n] = wt
        if b is not None:
            w["bias_" + n] = b

    def aff(ln, n):
        if ln.weight is None:
            return np.ones(n), np.zeros(n)
        return ln.weight.detach().cpu().double().numpy(), ln.bias.detach().cpu().double().numpy()

    w["g_in"], w["b_in"] = aff(m.layer_norm_in, C)
    w["g_out"], w["b_out"] = aff(m.layer_norm_out, H)
    return w


def _to(m, dev):
    from types import SimpleNamespace

    out = SimpleNamespace(**vars(m))
    for name, v in vars(m).items():
        if isinstance(v, torch.nn.Module):
            setattr(out, name, v.to(dev))
    return out


TRIMUL_CASES = [
    # B, N, C, H, outgoing, biases, fused, affine, mask_kind
    (1, 64, 128, 128, True, False, False, True, "float"),
    (1, 64, 128, 128, False, False, False, True, "float"),
    (1, 33, 64, 64, True, True, False, True, "bool"),
    (2, 40, 48, 40, False, True, True, True, "float"),
    (1, 17, 30, 22, True, False, False, False, "none"),
    (1, 96, 128, 96, False, True, False, True, "bool"),
    (1, 36, 64, 150, True, False, False, True, "float"),   # 16 channels per thread, H4 pad
    (1, 32, 48, 30, False, True, False, True, "float"),    # 8 channels per thread, H4 pad
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", TRIMUL_CASES,
                         ids=lambda c: "B{}N{}C{}H{}{}{}{}".format(
                             c[0], c[1], c[2], c[3], "out" if c[4] else "in",
                             "_bias" if c[5] else "", "_fused" if c[6] else ""))
def test_trimul_fp32(gpu, case):
    from oracle.trimul import trimul_forward
    from openfold3_triangle_kernel_amd.trimul_fp32 import run_trimul_fp32

    B, N, C, H, outgoing, biases, fused, affine, mk = case
    m = _trimul_module(C, H, outgoing, biases=biases, fused=fused, affine=affine)
    g = torch.Generator().manual_seed(1)
    z = torch.randn(B, N, N, C, generator=g)
    if mk == "none":
        mask, mask_np = None, np.ones((B, N, N))
    else:
        mb = torch.rand(B, N, N, generator=g) > 0.2
        mask = mb if mk == "bool" else mb.float()
        mask_np = mb.double().numpy()
    print(f"fp32 trimul case={case}", flush=True)
    with torch.no_grad():
        out = run_trimul_fp32(_to(m, gpu), z.to(gpu), None if mask is None else mask.to(gpu))
    torch.cuda.synchronize()
    assert out.dtype == torch.float32 and out.shape == z.shape
    ref, _ = trimul_forward(z.double().numpy(), mask_np, _oracle_weights(m, C, H), outgoing)
    err = max_rel(out.cpu().numpy(), ref)
    assert err <= TOL, err
