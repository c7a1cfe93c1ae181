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
