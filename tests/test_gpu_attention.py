"""GPU parity of triangle attention (C-ABI kernels) against the numpy oracle.

Tolerance (north star): bf16 outputs and gradients at max-rel <= 2e-2 against
the FP64 oracle evaluated on the same bf16-rounded inputs, where
max-rel = max|got - ref| / max|ref|.
"""

import numpy as np
import pytest
import torch

from oracle.attention import attention_backward, attention_forward
from tests._util import attention_case, max_rel

TOL = 2e-2

CASES = [
    # (B, O, H, N, D, kwargs)
    ("readme N128", (1, 8, 4, 128, 32), dict(mask_tail=13)),
    ("N100 pad masked", (1, 8, 4, 100, 32), dict(mask_frac=0.3)),
    ("N384 D24", (1, 4, 4, 384, 24), dict(mask_frac=0.2)),
    ("B2 N200 D20", (2, 4, 4, 200, 20), dict(mask_frac=0.2)),
    ("N256 D64 full planes", (1, 6, 4, 256, 64), dict(mask_frac=0.2, full_planes=2)),
    ("N384 D48", (1, 2, 4, 384, 48), dict(mask_frac=0.1)),
    ("N768 D16 H8", (1, 2, 8, 768, 16), dict(mask_frac=0.1)),
    ("O5 ragged group", (1, 5, 2, 64, 32), dict(random_tail=True, mask_tail=32)),
]


def _run(case, dev, seq_major=False):
    from openfold3_triangle_kernel_amd import turbopairformer_triangle_attention

    q, k, v, mask, bias, dout = case
    if seq_major:
        tq, tk, tv = (t.transpose(-2, -3).contiguous().to(dev, torch.bfloat16).transpose(-2, -3)
                      for t in (q, k, v))
    else:
        tq, tk, tv = (t.to(dev, torch.bfloat16) for t in (q, k, v))
    tq, tk, tv = (t.detach().requires_grad_(True) for t in (tq, tk, tv))
    tb = bias.to(dev, torch.bfloat16).requires_grad_(True)
    out = turbopairformer_triangle_attention(tq, tk, tv, mask.to(dev), tb)
    out.backward(dout.to(dev, torch.bfloat16))
    torch.cuda.synchronize()
    return [t.detach().float().cpu().numpy() for t in (out, tq.grad, tk.grad, tv.grad, tb.grad)]


@pytest.mark.gpu
@pytest.mark.parametrize("name,shape,kw", CASES, ids=[c[0] for c in CASES])
def test_attention_matches_oracle(gpu, name, shape, kw):
    print(f"[attn parity] {name} shape={shape} {kw}", flush=True)
    case = attention_case(*shape, **kw)
    q, k, v, mask, bias, dout = (t.numpy() for t in case)
    ref_out, _, _ = attention_forward(q, k, v, mask, bias)
    ref = [ref_out, *attention_backward(q, k, v, mask, bias, dout)]
    got = _run(case, gpu)
    names = ["out", "dq", "dk", "dv", "dbias"]
    errs = {n: max_rel(g, r) for n, g, r in zip(names, got, ref)}
    print(errs, flush=True)
    for n, e in errs.items():
        assert e <= TOL, f"{name}: {n} max-rel {e:.3e} > {TOL}"
    if kw.get("full_planes"):
        fp = kw["full_planes"]
        assert np.all(got[0][:, :fp] == 0), "fully masked planes must give exact zeros"
        for gr in got[1:4]:
            assert np.all(gr[:, :fp] == 0)


@pytest.mark.gpu
def test_attention_sequence_major_storage(gpu):
    case = attention_case(1, 4, 4, 128, 32, mask_tail=7, seed=3)
    a = _run(case, gpu, seq_major=False)
    b = _run(case, gpu, seq_major=True)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


@pytest.mark.gpu
def test_attention_bitwise_replay(gpu):
    case = attention_case(1, 8, 4, 192, 32, mask_frac=0.2, seed=5)
    a = _run(case, gpu)
    b = _run(case, gpu)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


@pytest.mark.gpu
def test_config2_readme_shape(gpu):
    """Config 2 exactly: q/k/v [1,128,4,128,32], bias [1,1,4,128,128] N(0,1),
    the last 13 keys masked, every output and gradient against the FP64
    oracle (dBias folds all 128 outer rows)."""
    print("[attn parity] config 2 [1,128,4,128,32] mask tail 13", flush=True)
    case = attention_case(1, 128, 4, 128, 32, mask_tail=13, seed=2)
    q, k, v, mask, bias, dout = (t.numpy() for t in case)
    ref_out, _, _ = attention_forward(q, k, v, mask, bias)
    ref = [ref_out, *attention_backward(q, k, v, mask, bias, dout)]
    got = _run(case, gpu)
    for n, g_, r in zip(["out", "dq", "dk", "dv", "dbias"], got, ref):
        e = max_rel(g_, r)
        print(n, f"{e:.3e}", flush=True)
        assert e <= TOL, f"config 2: {n} max-rel {e:.3e} > {TOL}"


def _bias_variant(gpu, B, O, H, N, D, bias_shape, bias_dtype, seed):
    from openfold3_triangle_kernel_amd import turbopairformer_triangle_attention

    q, k, v, mask, _, dout = attention_case(B, O, H, N, D, mask_frac=0.15, seed=seed)
    g = torch.Generator().manual_seed(seed + 100)
    bias = torch.randn(bias_shape, generator=g).to(torch.bfloat16).float()
    tq, tk, tv = (t.to(gpu, torch.bfloat16).requires_grad_(True) for t in (q, k, v))
    tb = bias.to(gpu, bias_dtype).requires_grad_(True)
    out = turbopairformer_triangle_attention(tq, tk, tv, mask.to(gpu), tb)
    out.backward(dout.to(gpu, torch.bfloat16))
    torch.cuda.synchronize()
    assert tb.grad.dtype == bias_dtype and tuple(tb.grad.shape) == tuple(bias_shape)
    ref_out, _, _ = attention_forward(q.numpy(), k.numpy(), v.numpy(), mask.numpy(), bias.numpy())
    ref = [ref_out, *attention_backward(q.numpy(), k.numpy(), v.numpy(), mask.numpy(),
                                        bias.numpy(), dout.numpy())]
    got = [t.detach().float().cpu().numpy() for t in (out, tq.grad, tk.grad, tv.grad, tb.grad)]
    for n, g_, r in zip(["out", "dq", "dk", "dv", "dbias"], got, ref):
        assert g_.shape == r.shape, (n, g_.shape, r.shape)
        e = max_rel(g_, r)
        print(n, f"{e:.3e}", flush=True)
        assert e <= TOL, f"{n} max-rel {e:.3e} > {TOL}"


@pytest.mark.gpu
def test_per_batch_bf16_bias_backward(gpu):
    """A bias per batch element ([B,1,H,N,N], Bb = B): each batch's dBias is
    folded over its own outer rows only."""
    print("[attn parity] per-batch bias B=2", flush=True)
    _bias_variant(gpu, 2, 6, 2, 128, 32, (2, 1, 2, 128, 128), torch.bfloat16, seed=11)


@pytest.mark.gpu
def test_runs_of_outer_groups_idle_rows_per_batch_bias(gpu):
    """B=2, O=130, H=4, N=128 on a 256-CU device gives 264 one-group
    workgroups, so the backward walks runs of 2 outer groups per workgroup:
    the last run of each batch holds the ragged group (2 of 4 rows idle) alone,
    and each batch's dBias is folded from its own runs.  Checked against the
    oracle and for bitwise replay."""
    print("[attn parity] runs of outer groups, O=130 ragged, per-batch bias B=2", flush=True)
    _bias_variant(gpu, 2, 130, 4, 128, 32, (2, 1, 4, 128, 128), torch.bfloat16, seed=13)
    from openfold3_triangle_kernel_amd import turbopairformer_triangle_attention

    q, k, v, mask, _, dout = attention_case(2, 130, 4, 128, 32, mask_frac=0.15, seed=13)
    bias = torch.randn((2, 1, 4, 128, 128), generator=torch.Generator().manual_seed(113))

    def grads():
        tq, tk, tv = (t.to(gpu, torch.bfloat16).requires_grad_(True) for t in (q, k, v))
        tb = bias.to(gpu, torch.bfloat16).requires_grad_(True)
        out = turbopairformer_triangle_attention(tq, tk, tv, mask.to(gpu), tb)
        out.backward(dout.to(gpu, torch.bfloat16))
        torch.cuda.synchronize()
        return [t.detach().cpu() for t in (tq.grad, tk.grad, tv.grad, tb.grad)]

    a, b = grads(), grads()
    for x, y in zip(a, b):
        assert torch.equal(x, y)


@pytest.mark.gpu
def test_partially_broadcast_bias_backward(gpu):
    """Prefix [2, 3] with a bias prefix [1, 3]: per-batch gradients summed over
    the broadcast dimension (reference dq_dbias.py:326-376)."""
    print("[attn parity] partial broadcast bias prefix (1,3) of (2,3)", flush=True)
    from openfold3_triangle_kernel_amd import turbopairformer_triangle_attention

    P0, P1, O, H, N, D = 2, 3, 4, 2, 64, 16
    g = torch.Generator().manual_seed(21)
    q, k, v = (torch.randn(P0, P1, O, H, N, D, generator=g).to(torch.bfloat16).float()
               for _ in range(3))
    mask = torch.zeros(P0, P1, O, 1, 1, N)
    mask[torch.rand(P0, P1, O, 1, 1, N, generator=g) < 0.2] = float("-inf")
    bias = torch.randn(1, P1, 1, H, N, N, generator=g).to(torch.bfloat16).float()
    dout = torch.randn(P0, P1, O, N, H, D, generator=g).to(torch.bfloat16).float()
    tq, tk, tv = (t.to(gpu, torch.bfloat16).requires_grad_(True) for t in (q, k, v))
    tb = bias.to(gpu, torch.bfloat16).requires_grad_(True)
    out = turbopairformer_triangle_attention(tq, tk, tv, mask.to(gpu), tb)
    out.backward(dout.to(gpu, torch.bfloat16))
    torch.cuda.synchronize()
    ref_out, _, _ = attention_forward(q.numpy(), k.numpy(), v.numpy(), mask.numpy(), bias.numpy())
    ref = [ref_out, *attention_backward(q.numpy(), k.numpy(), v.numpy(), mask.numpy(),
                                        bias.numpy(), dout.numpy())]
    got = [t.detach().float().cpu().numpy() for t in (out, tq.grad, tk.grad, tv.grad, tb.grad)]
    for n, g_, r in zip(["out", "dq", "dk", "dv", "dbias"], got, ref):
        assert g_.shape == r.shape, (n, g_.shape, r.shape)
        e = max_rel(g_, r)
        print(n, f"{e:.3e}", flush=True)
        assert e <= TOL, f"{n} max-rel {e:.3e} > {TOL}"


@pytest.mark.gpu
def test_fp32_pair_bias_gets_fp32_gradient(gpu):
    """An FP32 pair_bias is rounded to bf16 for the kernels and its gradient
    comes back in FP32 (reference turbopairformer_triangle_attention.py:371-377)."""
    print("[attn parity] fp32 pair bias", flush=True)
    _bias_variant(gpu, 1, 8, 4, 192, 32, (1, 1, 4, 192, 192), torch.float32, seed=12)


@pytest.mark.gpu
def test_transposed_bias_in_place_matches_copy(gpu):
    """bias.transpose(-1, -2) of a contiguous bias (the ending node) is read in
    place (TPF_BIAS_TRANSPOSED); outputs and gradients equal, bit for bit,
    those of the same values passed as a contiguous tensor."""
    from openfold3_triangle_kernel_amd import turbopairformer_triangle_attention

    print("[attn parity] transposed bias view vs contiguous copy", flush=True)
    q, k, v, mask, bias, dout = attention_case(1, 8, 4, 192, 32, mask_frac=0.1, seed=23)
    base = bias.transpose(-1, -2).contiguous().to(gpu, torch.bfloat16)
    res = []
    for contiguous in (False, True):
        b0 = base.clone().requires_grad_(True)
        view = b0.transpose(-1, -2)
        if contiguous:
            view = view.contiguous()
        tq, tk, tv = (t.to(gpu, torch.bfloat16).requires_grad_(True) for t in (q, k, v))
        out = turbopairformer_triangle_attention(tq, tk, tv, mask.to(gpu), view)
        out.backward(dout.to(gpu, torch.bfloat16))
        torch.cuda.synchronize()
        res.append([t.detach().float().cpu() for t in (out, tq.grad, tk.grad, tv.grad, b0.grad)])
    for a, b in zip(*res):
        assert torch.equal(a, b)
    ref_out, _, _ = attention_forward(q.numpy(), k.numpy(), v.numpy(), mask.numpy(), bias.numpy())
    assert max_rel(res[0][0].numpy(), ref_out) <= TOL
