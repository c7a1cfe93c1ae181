"""Drop-in modules on the GPU against the reference's committed module
snapshots (``tests/golden/snapshots``, built exactly as the reference's
tests build them: seed 123, every parameter ~ N(0, 0.01) in registration
order, x = rand(2, 22, 22, 128)).

BF16 route (training kernels): max-rel <= 2e-2; FP32 inference route:
max-rel <= 1e-4 (the snapshots are FP32 CPU outputs).
"""

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from tests._util import max_rel

GOLD = Path(__file__).resolve().parent / "golden" / "snapshots"


def _attention_module(starting):
    from openfold3_triangle_kernel_amd import TriangleAttention

    torch.manual_seed(123)
    m = TriangleAttention(128, 12, 4, starting=starting)
    for p in m.parameters():
        p.data.normal_(std=0.01)
    x = torch.rand((2, 22, 22, 128))
    return m, x


@pytest.mark.gpu
@pytest.mark.parametrize("starting", [True, False])
def test_triangle_attention_module_snapshot(gpu, starting):
    m, x = _attention_module(starting)
    ref = np.load(GOLD / f"tri_att_cpu_starting_{starting}.npz")["output"]
    m = m.to(gpu)
    print(f"module tri-att starting={starting}", flush=True)
    with torch.no_grad():
        out32 = m(x.to(gpu))                                   # FP32 inference kernel
    assert max_rel(out32.cpu().numpy(), ref) <= 1e-4
    mb = m.to(torch.bfloat16)
    xb = x.to(gpu, torch.bfloat16).requires_grad_(True)
    outb = mb(xb)                                              # BF16 training kernels
    outb.float().square().mean().backward()
    assert max_rel(outb.detach().float().cpu().numpy(), ref) <= 2e-2
    assert xb.grad is not None and torch.isfinite(xb.grad).all()
    assert all(p.grad is not None for p in mb.parameters())


@pytest.mark.gpu
def test_trimul_module_snapshot_fp32(gpu):
    from openfold3_triangle_kernel_amd import TriangleMultiplicationOutgoing

    torch.manual_seed(123)
    m = TriangleMultiplicationOutgoing(128, 11)
    for p in m.parameters():
        p.data.normal_(std=0.01)
    x = torch.rand((2, 22, 22, 128))
    mask = torch.randint(0, 2, size=(2, 22, 22))
    ref = np.load(GOLD / "tri_mul_outgoing_cpu.npz")["output"]
    m = m.to(gpu)
    with torch.no_grad():
        out = m(x.to(gpu), mask.to(gpu).float())
    assert max_rel(out.cpu().numpy(), ref) <= 1e-4
    # The BF16 training kernels need c_hidden == c_z: this module falls back to
    # the stock math (logged), or raises under strict mode.
    from openfold3_triangle_kernel_amd import set_turbopairformer_strict, stock_invocation_count

    before = stock_invocation_count()
    out_stock = m(x.to(gpu).requires_grad_(True), mask.to(gpu).float())
    assert stock_invocation_count() == before + 1
    assert max_rel(out_stock.detach().cpu().numpy(), ref) <= 1e-4
    set_turbopairformer_strict(True)
    try:
        with pytest.raises(RuntimeError, match="c_hidden == c_z"):
            m(x.to(gpu).requires_grad_(True), mask.to(gpu).float())
    finally:
        set_turbopairformer_strict(False)


def _stock_triangle_attention(m, x, mask, starting, transpose_bias=False):
    """FP32 torch restatement of OpenFold3's TriangleAttention forward
    (triangular_attention.py:352-409, attention.py _prep_qkv / _wrap_up)."""
    import math

    if not starting:
        x = x.transpose(-2, -3)
        mask = mask.transpose(-1, -2)
    x = torch.nn.functional.layer_norm(x, (x.shape[-1],), m.layer_norm.weight, m.layer_norm.bias)
    mask_bias = (m.inf * (mask - 1))[..., :, None, None, :]
    tri = (x @ m.linear_z.weight.t()).permute((0, 3, 2, 1) if transpose_bias else (0, 3, 1, 2))
    tri = tri.unsqueeze(-4)
    H, c = m.mha.no_heads, m.mha.c_hidden

    def heads(t):
        return t.view(t.shape[:-1] + (H, c)).transpose(-2, -3)

    q, k, v = (heads(x @ w.t()) for w in (m.mha.linear_q.weight, m.mha.linear_k.weight,
                                          m.mha.linear_v.weight))
    a = torch.softmax(q @ k.transpose(-1, -2) / math.sqrt(c) + mask_bias + tri, -1)
    o = (a @ v).transpose(-2, -3)
    g = torch.sigmoid(x @ m.mha.linear_g.weight.t()).view(o.shape)
    out = ((o * g).flatten(-2)) @ m.mha.linear_o.weight.t()
    return out.transpose(-2, -3) if not starting else out


def _graph_has(t, name):
    seen, stack = set(), [t.grad_fn]
    while stack:
        f = stack.pop()
        if f is None or f in seen:
            continue
        seen.add(f)
        if type(f).__name__ == name:
            return True
        stack.extend(n for n, _ in f.next_functions)
    return False


@pytest.mark.gpu
@pytest.mark.parametrize("N,transpose_bias,C", [(96, False, 128), (128, False, 128),
                                                (128, True, 128), (128, False, 64)])
@pytest.mark.parametrize("starting", [True, False])
def test_triangle_attention_module_backward(gpu, starting, N, transpose_bias, C):
    """BF16 module forward + every parameter / input gradient vs the FP32
    stock math on the same (bf16-representable) weights.  N = 96 takes the
    per-projection route; N = 128 (a multiple of 64) the pair-row core
    (tpf_attn_pair_*), with the pair bias plain or transposed; C = 128 forms
    the split projection on the row GEMM, C = 64 through the tile GEMM and a
    copy (``_pair_projection``'s other branch).

    The reference's module check (scripts/benchmarks/
    turbopairformer_module_wiring_smoke.py:90-130) gates the output and the
    input gradient (absolute gap < 0.1) and bitwise replay, and only reports
    the parameter gradients.  Here the output, the input gradient and every
    parameter gradient are gated at max-rel <= 2e-2,
    under the default shadow-residual policy; a second pass is bitwise
    identical."""
    from openfold3_triangle_kernel_amd import TriangleAttention

    torch.manual_seed(7)
    m = TriangleAttention(C, 32, 4, starting=starting)
    for p in m.parameters():
        p.data = p.data.normal_(std=0.1 if p.dim() == 2 else 1.0).bfloat16().float()
    m = m.to(gpu)
    x = torch.randn(1, N, N, C, device=gpu).bfloat16().float()
    mask = (torch.rand(1, N, N, device=gpu) > 0.1).float()
    dout = torch.randn(1, N, N, C, device=gpu).bfloat16().float()
    ref_params = {n: p.detach().clone().requires_grad_(True) for n, p in m.named_parameters()}
    xr = x.clone().requires_grad_(True)
    ref_m = TriangleAttention(C, 32, 4, starting=starting).to(gpu)
    ref_m.load_state_dict({n: p for n, p in ref_params.items()})
    for n, p in ref_m.named_parameters():
        p.requires_grad_(True)
    ref = _stock_triangle_attention(ref_m, xr, mask, starting, transpose_bias)
    ref_grads = torch.autograd.grad(ref, [xr] + list(ref_m.parameters()), dout)
    from openfold3_triangle_kernel_amd import stock_invocation_count

    mb = m.to(torch.bfloat16)
    xb = x.bfloat16().requires_grad_(True)
    stock_before = stock_invocation_count()
    out = mb(xb, mask.bfloat16(), transpose_bias=transpose_bias)
    assert _graph_has(out, "_PairAttentionCoreBackward") == (N % 64 == 0)
    grads = torch.autograd.grad(out, [xb] + list(mb.parameters()), dout.bfloat16())
    out2 = mb(xb, mask.bfloat16(), transpose_bias=transpose_bias)
    grads2 = torch.autograd.grad(out2, [xb] + list(mb.parameters()), dout.bfloat16())
    assert torch.equal(out, out2) and all(torch.equal(a, b) for a, b in zip(grads, grads2))
    assert stock_invocation_count() == stock_before  # the kernels ran, never the stock math
    names = ["out", "x"] + [n for n, _ in mb.named_parameters()]
    for name, a, b in zip(names, [out] + list(grads), [ref] + list(ref_grads)):
        err = max_rel(a.detach().float().cpu().numpy(), b.detach().float().cpu().numpy())
        print(f"module starting={starting} N={N} tb={transpose_bias} C={C} {name} max-rel {err:.3e}",
              flush=True)
        assert err <= 2e-2, f"{name}: {err:.3e}"


@pytest.mark.gpu
@pytest.mark.parametrize("N", [64, 50])
@pytest.mark.parametrize("outgoing", [True, False])
def test_trimul_module_backward(gpu, outgoing, N):
    """BF16 TriMul module (run_stable_trimul) forward + input / parameter
    gradients vs the module's stock math in FP32 on the same bf16-representable
    weights (LayerNorm affine perturbed from identity): output, input and
    parameter gradients max-rel <= 2e-2; bitwise replay;
    the stock math never runs on the stable route."""
    from openfold3_triangle_kernel_amd import (
        TriangleMultiplicationIncoming,
        TriangleMultiplicationOutgoing,
        stock_invocation_count,
    )

    cls = TriangleMultiplicationOutgoing if outgoing else TriangleMultiplicationIncoming
    torch.manual_seed(11)
    m = cls(128, 128)
    for name, p in m.named_parameters():
        if p.dim() == 2:
            p.data = (torch.randn_like(p) / math.sqrt(p.shape[1])).bfloat16().float()
        else:
            base = 1.0 if name.endswith("weight") else 0.0
            p.data = (base + 0.1 * torch.randn_like(p)).bfloat16().float()
    m = m.to(gpu)
    x = torch.randn(1, N, N, 128, device=gpu).bfloat16().float()
    mask = (torch.rand(1, N, N, device=gpu) > 0.1).float()
    dout = torch.randn(1, N, N, 128, device=gpu).bfloat16().float()
    xr = x.clone().requires_grad_(True)
    ref = m(xr, mask, use_stable_triangle_multiplicative=False)
    ref_grads = torch.autograd.grad(ref, [xr] + list(m.parameters()), dout)
    mb = m.to(torch.bfloat16)
    xb = x.bfloat16().requires_grad_(True)
    before = stock_invocation_count()
    out = mb(xb, mask.bfloat16())
    grads = torch.autograd.grad(out, [xb] + list(mb.parameters()), dout.bfloat16())
    out2 = mb(xb, mask.bfloat16())
    grads2 = torch.autograd.grad(out2, [xb] + list(mb.parameters()), dout.bfloat16())
    assert stock_invocation_count() == before
    assert torch.equal(out, out2) and all(torch.equal(a, b) for a, b in zip(grads, grads2))
    names = ["out", "x"] + [n for n, _ in mb.named_parameters()]
    for name, a, b in zip(names, [out] + list(grads), [ref] + list(ref_grads)):
        err = max_rel(a.detach().float().cpu().numpy(), b.detach().float().cpu().numpy())
        print(f"trimul module out={outgoing} N={N} {name} max-rel {err:.3e}", flush=True)
        assert err <= 2e-2, f"{name}: {err:.3e}"
