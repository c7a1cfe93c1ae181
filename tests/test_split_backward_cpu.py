"""Host checks of the split backward route (no GPU): the partial-workspace
size formula and argument validation before any launch."""

import pytest
import torch

from openfold3_triangle_kernel_amd.split_backward import (
    delta_true_partial_elements,
    turbopairformer_triangle_dkdv,
    turbopairformer_triangle_dq_dbias,
)


def test_delta_true_partial_elements():
    # [batch, outer, heads, ceil(N / 64), N] (turbopairformer_triangle_dkdv.py:75-91)
    assert delta_true_partial_elements(128, 4, 1) == 1 * 128 * 4 * 2 * 128
    assert delta_true_partial_elements(100, 2, 3, outer=5) == 3 * 5 * 2 * 2 * 100


def _args(B=1, O=2, H=4, N=128, D=32):
    bf = torch.bfloat16
    q = torch.zeros(B, O, H, N, D, dtype=bf)
    return (q, q.clone(), q.clone(), torch.zeros(B, O, N, H, D, dtype=bf),
            torch.zeros(B, O, H, N), torch.zeros(B, O, H, N), torch.zeros(B, O, 1, 1, N),
            torch.zeros(B, 1, H, N, N, dtype=bf))


def test_rejects_cpu_tensors_and_bad_shapes():
    with pytest.raises(ValueError, match="one GPU"):
        turbopairformer_triangle_dkdv(*_args())
    with pytest.raises(ValueError, match="N % 64"):
        turbopairformer_triangle_dq_dbias(*_args(N=100))
    a = list(_args())
    a[0] = a[0].float()
    with pytest.raises(ValueError, match="bf16"):
        turbopairformer_triangle_dkdv(*a)
