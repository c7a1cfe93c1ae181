"""The TriMul FP32 weight-gradient fold contract of the reference's release
smoke (tools/aot_numeric_smoke.py:201-222): for C in {32, 64, 96, 128},
seed 9187 + C, partials ~ N(0, 1) of shape [17, 5C, C], the fold equals an
ascending FP32 add_ over the chunks bit for bit, and returns the accumulator
it was given."""

import pytest
import torch


@pytest.mark.gpu
@pytest.mark.parametrize("channels", [32, 64, 96, 128])
def test_wgrad_fixed_fold_bitwise(gpu, channels):
    from openfold3_triangle_kernel_amd import trimul_wgrad_fixed_fold

    print(f"[trimul fold] C={channels}", flush=True)
    torch.manual_seed(9187 + channels)
    partials = torch.randn(17, 5 * channels, channels, dtype=torch.float32)
    expected = torch.zeros_like(partials[0])
    for chunk in partials.unbind(0):
        expected.add_(chunk)
    dev_partials = partials.to(gpu)
    actual = torch.full_like(dev_partials[0], float("nan"))
    returned = trimul_wgrad_fixed_fold(dev_partials, actual, True)
    torch.cuda.synchronize()
    assert returned.data_ptr() == actual.data_ptr()
    assert torch.equal(actual.cpu().view(torch.int32), expected.view(torch.int32))
    # Continuing from the accumulator: a second fold adds the same chunks.
    expected2 = expected.clone()
    for chunk in partials.unbind(0):
        expected2.add_(chunk)
    trimul_wgrad_fixed_fold(dev_partials, actual, False)
    torch.cuda.synchronize()
    assert torch.equal(actual.cpu().view(torch.int32), expected2.view(torch.int32))


@pytest.mark.gpu
def test_wgrad_fixed_fold_rejects_overlap(gpu):
    from openfold3_triangle_kernel_amd import trimul_wgrad_fixed_fold

    partials = torch.zeros(3, 8, 8, device=gpu)
    with pytest.raises(RuntimeError, match="overlap"):
        trimul_wgrad_fixed_fold(partials, partials[1], True)
