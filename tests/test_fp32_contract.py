"""Host-side contract of the FP32 entry points (no GPU needed)."""

import pytest
import torch


def test_attention_fp32_rejects_grad_mode_and_dtypes():
    from openfold3_triangle_kernel_amd.attention_fp32 import is_attention_fp32_supported

    q = torch.zeros(1, 2, 4, 8, 16)
    mask = torch.zeros(1, 2, 1, 1, 8)
    bias = torch.zeros(1, 1, 4, 8, 8)
    ok, reason = is_attention_fp32_supported(q, q, q, mask, bias)
    assert not ok and "inference-only" in reason
    with torch.no_grad():
        ok, reason = is_attention_fp32_supported(q.bfloat16(), q, q, mask, bias)
        assert not ok and "FP32" in reason
        ok, reason = is_attention_fp32_supported(q, q, q, mask, bias)
        assert not ok  # CPU tensors are not a gfx950 device


def test_attention_fp32_raises_before_launch():
    from openfold3_triangle_kernel_amd import turbopairformer_attention_fp32

    q = torch.zeros(1, 2, 4, 8, 16)
    with pytest.raises(ValueError, match="inference-only"):
        turbopairformer_attention_fp32(q, q, q, torch.zeros(1, 2, 1, 1, 8), torch.zeros(1, 1, 4, 8, 8))


def test_trimul_fp32_contract():
    from types import SimpleNamespace

    from openfold3_triangle_kernel_amd.trimul_fp32 import run_trimul_fp32

    m = SimpleNamespace(c_z=8, c_hidden=8, _outgoing=True)
    z = torch.zeros(1, 4, 4, 8)
    with pytest.raises(RuntimeError, match="inference-only"):
        run_trimul_fp32(m, z)
    with torch.no_grad(), pytest.raises(ValueError, match="CUDA FP32"):
        run_trimul_fp32(m, z)
