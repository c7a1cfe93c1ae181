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
