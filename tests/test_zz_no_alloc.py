"""The allocation-free attention forward (tpf_attn_forward_noalloc_bf16)
against the workspace entry point it shares its kernels with
(tpf_attn_forward_bf16), through the C ABI: bitwise-equal out and lse on two
calls in a row, the second smaller, and a too-large bias rejected before any
launch."""

import math

import pytest
import torch

from tests._util import attention_case


def _inputs(B, O, H, N, D, seed, dev):
    q, k, v, mask, bias, _ = attention_case(B, O, H, N, D, mask_frac=0.1, seed=seed)
    q, k, v = (t.to(dev, torch.bfloat16).contiguous() for t in (q, k, v))
    mask = mask.reshape(B, O, N).to(dev).contiguous()
    bias = bias.reshape(1, H, N, N).to(dev, torch.bfloat16).contiguous()
    return q, k, v, mask, bias


def _forward(name, ins, B, O, H, N, D, ws=None):
    from openfold3_triangle_kernel_amd import _native

    q, k, v, mask, bias = ins
    dev = q.device
    out = torch.full((B, O, N, H, D), float("nan"), device=dev, dtype=torch.bfloat16)
    lse = torch.full((B, O, H, N), float("nan"), device=dev, dtype=torch.float32)
    scale = 1.0 / math.sqrt(D)
    stream = _native.stream_of(q)
    if name == "tpf_attn_forward_bf16":
        _native.call(name, q.data_ptr(), k.data_ptr(), v.data_ptr(), mask.data_ptr(),
                     bias.data_ptr(), out.data_ptr(), lse.data_ptr(), ws.data_ptr(), ws.numel(),
                     B, O, H, N, D, 0, 1, scale, stream)
    else:
        _native.call(name, q.data_ptr(), k.data_ptr(), v.data_ptr(), mask.data_ptr(),
                     bias.data_ptr(), out.data_ptr(), lse.data_ptr(), B, O, H, N, D, 0, 1, scale,
                     stream)
    torch.cuda.synchronize()
    return out, lse


@pytest.mark.gpu
def test_noalloc_forward_matches_workspace_forward(gpu):
    from openfold3_triangle_kernel_amd import _native

    for B, O, H, N, D, seed in ((1, 8, 4, 384, 32, 1), (1, 4, 2, 128, 16, 2)):
        print(f"[no-alloc] forward B={B} O={O} H={H} N={N} D={D}", flush=True)
        ins = _inputs(B, O, H, N, D, seed, gpu)
        ws = torch.empty(int(_native.query("tpf_attn_forward_workspace_bytes", B, H, N, 1)),
                         device=gpu, dtype=torch.uint8)
        ref_out, ref_lse = _forward("tpf_attn_forward_bf16", ins, B, O, H, N, D, ws)
        out, lse = _forward("tpf_attn_forward_noalloc_bf16", ins, B, O, H, N, D)
        assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16))
        assert torch.equal(lse.view(torch.int32), ref_lse.view(torch.int32))


@pytest.mark.gpu
def test_noalloc_forward_rejects_oversized_bias(gpu):
    from openfold3_triangle_kernel_amd import _native

    # H * N * N = 8 * 768 * 768 = 4,718,592 > 4,194,304 f32 values of scratch.
    # Every operand is a real device tensor of the declared shape, so even a
    # host check that failed to fire could not launch on a bogus address.
    B, O, H, N, D = 1, 1, 8, 768, 32
    q, k, v = (torch.zeros(B, O, H, N, D, device=gpu, dtype=torch.bfloat16) for _ in range(3))
    mask = torch.zeros(B, O, N, device=gpu)
    bias = torch.zeros(1, H, N, N, device=gpu, dtype=torch.bfloat16)
    out = torch.empty(B, O, N, H, D, device=gpu, dtype=torch.bfloat16)
    lse = torch.empty(B, O, H, N, device=gpu)
    with pytest.raises(RuntimeError, match="static scratch"):
        _native.call("tpf_attn_forward_noalloc_bf16", q.data_ptr(), k.data_ptr(), v.data_ptr(),
                     mask.data_ptr(), bias.data_ptr(), out.data_ptr(), lse.data_ptr(),
                     B, O, H, N, D, 0, 1, 1.0 / D ** 0.5, None)
