"""Outer-row chunking of the inference paths (reference
``openfold3/core/model/layers/triangular_attention.py:114-158, 322-327`` and
``turbopairformer_trimul_fp32.py:203-221, 344-345``): chunked outputs are
bitwise the unchunked ones, and chunking with gradients raises, as the
reference's stable route does."""

import pytest
import torch

from tests.test_gpu_fp32 import _to, _trimul_module


def _fp32_attention_module(starting, device, seed):
    from openfold3_triangle_kernel_amd import TriangleAttention

    torch.manual_seed(seed)
    m = TriangleAttention(64, 16, 4, starting=starting)
    with torch.no_grad():
        for p in m.parameters():
            p.normal_(std=0.1)
    return m.to(device).eval()


@pytest.mark.gpu
@pytest.mark.parametrize("N", [64, 96])
@pytest.mark.parametrize("starting", [True, False])
def test_fp32_attention_module_chunked_bitwise(gpu, N, starting):
    m = _fp32_attention_module(starting, gpu, 3 + N)
    g = torch.Generator(device=gpu).manual_seed(N)
    x = torch.randn(1, N, N, 64, device=gpu, generator=g)
    mask = (torch.rand(1, N, N, device=gpu, generator=g) > 0.1).float()
    with torch.no_grad():
        ref = m(x, mask)
        for chunk in (1, 7, 32, N + 5):
            print(f"[chunk] fp32 attention N={N} starting={starting} chunk={chunk}", flush=True)
            out = m(x, mask, chunk_size=chunk)
            assert out.dtype == torch.float32
            assert torch.equal(ref, out), f"chunk_size={chunk}"


@pytest.mark.gpu
def test_attention_chunking_with_gradients_raises(gpu):
    m = _fp32_attention_module(True, gpu, 5).to(torch.bfloat16).train()
    x = torch.randn(1, 64, 64, 64, device=gpu, dtype=torch.bfloat16, requires_grad=True)
    with pytest.raises(ValueError, match="inference-only"):
        m(x, None, chunk_size=16)


@pytest.mark.gpu
@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("B,N", [(1, 64), (2, 37)])
def test_fp32_trimul_output_row_chunks_bitwise(gpu, outgoing, B, N):
    from openfold3_triangle_kernel_amd.trimul_fp32 import run_trimul_fp32

    C, H = 64, 64
    m = _to(_trimul_module(C, H, outgoing, biases=True, seed=B + N), gpu)
    g = torch.Generator().manual_seed(N)
    z = torch.randn(B, N, N, C, generator=g).to(gpu)
    mask = (torch.rand(B, N, N, generator=g) > 0.2).to(gpu)
    with torch.no_grad():
        ref = run_trimul_fp32(m, z, mask)
        for chunk in (1, 5, 16, N):
            print(f"[chunk] fp32 trimul B={B} N={N} out={outgoing} chunk={chunk}", flush=True)
            out = run_trimul_fp32(m, z, mask, output_row_chunk_size=chunk)
            assert torch.equal(ref, out), f"output_row_chunk_size={chunk}"
        # The default plan chunks when the product scratch budget is small.
        row_bytes = H * ((N + 3) // 4 * 4) * 4
        out = run_trimul_fp32(m, z, mask, contraction_workspace_bytes=3 * row_bytes)
        assert torch.equal(ref, out)
