"""Config 1 on the HIP path, the release rel-L2 rule at config 3's full size,
and the backward's workspace budget (slabs of outer rows).

* Config 1: q, k, v ``[1,64,4,64,32]`` ~ N(0,1), q
  unscaled, bias ``[1,1,4,64,64]`` ~ N(0,1), mask zeros, loss mean(out^2).
  The bf16 kernels' output and every gradient against the FP64 oracle at
  max-rel <= 2e-2; the FP32 inference kernel's output at <= 1e-4.
* Config 3 (``[1,384,4,384,32]``, bias 2 N(0,1), random 0-32 key tail per
  outer row), starting and ending node: rel-L2 of out, dq, dk, dv, dbias
  against an FP64 restatement on the GPU must satisfy the reference's release
  rule rel_L2(ours) <= 1.1 * rel_L2(stock) + 1e-6 (tools/aot_numeric_smoke.py:
  174-180), stock = BF16 matmuls with an FP32 softmax (:50-60).
* Workspace budget: a budget that forces several slabs gives results bitwise
  equal to the one-slab plan (config 5's H=8, D=64 attention, and a ragged
  B=2 case whose slabs cross the batch boundary).
"""

import math

import numpy as np
import pytest
import torch

from oracle.attention import attention_backward, attention_forward
from tests._util import max_rel, record, rel_l2

LABELS = ("out", "dq", "dk", "dv", "dbias")


def _config1_inputs():
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(1, 64, 4, 64, 32, generator=g) for _ in range(3))
    bias = torch.randn(1, 1, 4, 64, 64, generator=g)
    mask = torch.zeros(1, 64, 1, 1, 64)
    return q, k, v, bias, mask


@pytest.mark.gpu
def test_config1_bf16_forward_backward(gpu):
    from openfold3_triangle_kernel_amd import turbopairformer_triangle_attention

    q, k, v, bias, mask = (t.bfloat16().float() for t in _config1_inputs())
    xs = [t.to(gpu).bfloat16().requires_grad_(True) for t in (q, k, v, bias)]
    out = turbopairformer_triangle_attention(xs[0], xs[1], xs[2], mask.to(gpu), xs[3])
    loss = out.float().pow(2).mean()
    grads = torch.autograd.grad(loss, xs)
    # The upstream gradient autograd handed the kernel: d mean(out^2) / d out
    # in f32, rounded to the output's bf16.
    dout = (2.0 * out.detach().float() / out.numel()).bfloat16().float().cpu().numpy()
    npf = lambda t: t.detach().float().cpu().numpy()
    ref_out, _, _ = attention_forward(npf(q), npf(k), npf(v), mask.numpy(), npf(bias))
    refs = [ref_out, *attention_backward(npf(q), npf(k), npf(v), mask.numpy(), npf(bias), dout)]
    errs = {}
    for name, got, ref in zip(LABELS, (out, *grads), refs):
        errs[name] = max_rel(npf(got), ref)
        print(f"config1 bf16 {name} max-rel {errs[name]:.3e}", flush=True)
    record("attention_config_gates", "config1 bf16 max-rel vs FP64 oracle", errs)
    for name, e in errs.items():
        assert e <= 2e-2, f"config1 {name}: {e:.3e}"


@pytest.mark.gpu
def test_config1_fp32_forward(gpu):
    from openfold3_triangle_kernel_amd import turbopairformer_triangle_attention

    q, k, v, bias, mask = _config1_inputs()
    with torch.no_grad():  # FP32 mode is inference-only, as the reference's
        out = turbopairformer_triangle_attention(q.to(gpu), k.to(gpu), v.to(gpu), mask.to(gpu),
                                                 bias.to(gpu))
    assert out.dtype == torch.float32
    ref, _, _ = attention_forward(*(t.numpy() for t in (q, k, v, mask, bias)))
    err = max_rel(out.cpu().numpy(), ref)
    print(f"config1 fp32 out max-rel {err:.3e}", flush=True)
    record("attention_config_gates", "config1 fp32 max-rel vs FP64 oracle", {"out": err})
    assert err <= 1e-4


def _config3(dev, node):
    g = torch.Generator(device=dev).manual_seed(0)
    O, H, N, D = 384, 4, 384, 32
    q, k, v = (torch.randn(1, O, H, N, D, device=dev, generator=g).bfloat16() for _ in range(3))
    bias = (torch.randn(1, 1, H, N, N, device=dev, generator=g) * 2).bfloat16()
    tails = torch.randint(0, 33, (1, O), device=dev, generator=g)
    ar = torch.arange(N, device=dev)
    mask = torch.where(ar[None, None, :] >= (N - tails)[..., None], float("-inf"), 0.0)
    mask = mask.reshape(1, O, 1, 1, N).float()
    dout = torch.randn(1, O, N, H, D, device=dev, generator=g).bfloat16()
    if node == "ending":
        q, k, v = (t.transpose(1, 3).contiguous() for t in (q, k, v))
        bias = bias.transpose(-1, -2)
    return q, k, v, bias, mask, dout


def _reference(q, k, v, bias, mask, dout, dtype, stock):
    """FP64 restatement (stock=False) or the stock BF16-matmul / FP32-softmax
    path (stock=True), with autograd."""
    scale = 1.0 / math.sqrt(q.shape[-1])
    if stock:
        xs = [t.detach().clone().requires_grad_(True) for t in (q, k, v, bias)]
        s = torch.matmul(xs[0], xs[1].transpose(-1, -2)).float() * scale + mask + xs[3].float()
        out = torch.matmul(torch.softmax(s, -1).bfloat16(), xs[2]).transpose(-2, -3)
    else:
        xs = [t.detach().to(dtype).requires_grad_(True) for t in (q, k, v, bias)]
        s = torch.matmul(xs[0], xs[1].transpose(-1, -2)) * scale + mask.to(dtype) + xs[3]
        out = torch.matmul(torch.softmax(s, -1), xs[2]).transpose(-2, -3)
    grads = torch.autograd.grad(out, xs, dout.to(out.dtype))
    return [t.detach() for t in (out, *grads)]


def _gpu_rel_l2(a, b):
    a, b = a.double(), b.double()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


@pytest.mark.gpu
@pytest.mark.parametrize("node", ["starting", "ending"])
def test_config3_release_rule_full_size(gpu, node):
    from openfold3_triangle_kernel_amd import turbopairformer_triangle_attention

    q, k, v, bias, mask, dout = _config3(gpu, node)
    xs = [t.detach().requires_grad_(True) for t in (q, k, v, bias)]
    out = turbopairformer_triangle_attention(xs[0], xs[1], xs[2], mask, xs[3])
    got = [out.detach()] + [t.detach() for t in torch.autograd.grad(out, xs, dout)]
    # Rows of the ending node's inputs are already transposed; the bias view
    # is transposed the same way for every path.
    ref = _reference(q, k, v, bias, mask, dout, torch.float64, stock=False)
    st = _reference(q, k, v, bias, mask, dout, None, stock=True)
    rows = {}
    for i, label in enumerate(LABELS):
        e, es = _gpu_rel_l2(got[i], ref[i]), _gpu_rel_l2(st[i], ref[i])
        rows[label] = {"ours": e, "stock": es, "limit": 1.1 * es + 1e-6}
        print(f"config3 {node} {label}: rel-L2 {e:.3e} stock {es:.3e}", flush=True)
    record("attention_config_gates", f"config3 {node} rel-L2 vs FP64", rows)
    for label, r in rows.items():
        assert r["ours"] <= r["limit"], f"config3 {node} {label}: {r}"


def _run_with_budget(q, k, v, bias, mask, dout, budget):
    from openfold3_triangle_kernel_amd import attention as A

    A.set_sr_workspace_budget(budget)
    try:
        xs = [t.detach().requires_grad_(True) for t in (q, k, v, bias)]
        out = A.turbopairformer_triangle_attention(xs[0], xs[1], xs[2], mask, xs[3])
        grads = torch.autograd.grad(out, xs, dout)
        torch.cuda.synchronize()
        return [out.detach()] + [t.detach() for t in grads]
    finally:
        A.set_sr_workspace_budget(None)


def _bitwise(a, b):
    return torch.equal(a.contiguous().view(torch.uint8), b.contiguous().view(torch.uint8))


@pytest.mark.gpu
def test_workspace_budget_slabs_bitwise_config5_d64(gpu):
    from openfold3_triangle_kernel_amd.attention import sr_workspace_plan

    O, H, N, D = 768, 8, 768, 64
    full_bytes, one = sr_workspace_plan(1, O, H, N, D, 1 << 62)
    budget = full_bytes // 3
    small_bytes, slabs = sr_workspace_plan(1, O, H, N, D, budget)
    print(f"[budget] config5 D64: full {full_bytes} B (1 slab), budget {budget} -> "
          f"{small_bytes} B in {slabs} slabs", flush=True)
    assert one == 1 and slabs >= 2 and small_bytes <= budget
    g = torch.Generator(device=gpu).manual_seed(5)
    q, k, v = (torch.randn(1, O, H, N, D, device=gpu, generator=g).bfloat16() for _ in range(3))
    bias = torch.randn(1, 1, H, N, N, device=gpu, generator=g).bfloat16()
    mask = torch.zeros(1, O, 1, 1, N, device=gpu)
    mask[..., -20:] = float("-inf")
    dout = torch.randn(1, O, N, H, D, device=gpu, generator=g).bfloat16()
    a = _run_with_budget(q, k, v, bias, mask, dout, 1 << 62)
    b = _run_with_budget(q, k, v, bias, mask, dout, budget)
    for label, x, y in zip(LABELS, a, b):
        assert _bitwise(x, y), f"{label}: slabbed backward differs from the one-slab plan"


@pytest.mark.gpu
def test_workspace_budget_slabs_cross_batches(gpu):
    """B=2 with a per-batch bias, O=130 (ragged last group): one run per slab,
    slabs crossing the batch boundary; bitwise equal to one slab and within
    the bf16 tolerance of the FP64 oracle."""
    from openfold3_triangle_kernel_amd.attention import sr_workspace_plan

    B, O, H, N, D = 2, 130, 4, 128, 32
    _, slabs = sr_workspace_plan(B, O, H, N, D, 1)
    assert slabs >= 4
    g = torch.Generator().manual_seed(7)
    q, k, v = (torch.randn(B, O, H, N, D, generator=g).bfloat16() for _ in range(3))
    bias = torch.randn(B, 1, H, N, N, generator=g).bfloat16()
    mask = torch.zeros(B, O, 1, 1, N)
    mask[:, :, ..., -9:] = float("-inf")
    dout = torch.randn(B, O, N, H, D, generator=g).bfloat16()
    dev = [t.to(gpu) for t in (q, k, v, bias, mask, dout)]
    a = _run_with_budget(*dev, 1 << 62)
    b = _run_with_budget(*dev, 1)
    for label, x, y in zip(LABELS, a, b):
        assert _bitwise(x, y), f"{label}: slabbed backward differs from the one-slab plan"
    npf = lambda t: t.detach().float().cpu().numpy()
    ref_out, _, _ = attention_forward(npf(q), npf(k), npf(v), npf(mask), npf(bias))
    refs = [ref_out, *attention_backward(npf(q), npf(k), npf(v), npf(mask), npf(bias), npf(dout))]
    for label, got, ref in zip(LABELS, b, refs):
        assert max_rel(npf(got), ref) <= 2e-2, label
