"""GPU parity of the batched MFMA GEMM (tpf_gemm_bf16) against torch fp32.

C[z] = alpha * A[z] B[z]^T with each operand K-contiguous or MN-contiguous;
ragged M / N / K (not multiples of the 128 x 128 x 64 tile), batches, and f32
or bf16 output.  Tolerance: bf16 inputs are exact in fp32, so the only error
is the f32 accumulation order (and the bf16 rounding of a bf16 output):
max-rel <= 1e-5 for f32 output, <= 8e-3 for bf16 output.
"""

import pytest
import torch

from tests._util import max_rel


def _operand(x, kc):
    """Return (tensor, ld) of the [rows, K] matrix x in the requested layout."""
    if kc:
        return x.contiguous(), x.shape[-1]
    rows = x.shape[-2]
    ld = (rows + 7) // 8 * 8
    t = torch.zeros(*x.shape[:-2], x.shape[-1], ld, dtype=x.dtype, device=x.device)
    t[..., :rows] = x.transpose(-1, -2)
    return t, ld


CASES = [
    # batch, M, N, K
    (1, 128, 128, 64),
    (3, 384, 384, 384),
    (2, 200, 72, 136),
    (1, 33, 17, 8),
    (1, 640, 128, 4096),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
@pytest.mark.parametrize("a_kc,b_kc", [(1, 1), (1, 0), (0, 1), (0, 0)], ids=["KK", "KM", "MK", "MM"])
@pytest.mark.parametrize("out_f32", [1, 0], ids=["f32", "bf16"])
def test_gemm(gpu, case, a_kc, b_kc, out_f32):
    from openfold3_triangle_kernel_amd import _native

    bz, M, N, K = case
    g = torch.Generator(device="cpu").manual_seed(M * 7 + N * 3 + K)
    a = torch.randn(bz, M, K, generator=g).to(torch.bfloat16).to(gpu)
    b = torch.randn(bz, N, K, generator=g).to(torch.bfloat16).to(gpu)
    ta, lda = _operand(a, a_kc)
    tb, ldb = _operand(b, b_kc)
    c = torch.full((bz, M, N), float("nan"), device=gpu,
                   dtype=torch.float32 if out_f32 else torch.bfloat16)
    alpha = 0.5
    stream = torch.cuda.current_stream().cuda_stream
    print(f"gemm case={case} a_kc={a_kc} b_kc={b_kc} out_f32={out_f32}", flush=True)
    _native.call("tpf_gemm_bf16", ta.data_ptr(), a_kc, lda, ta[0].numel(), tb.data_ptr(), b_kc,
                 ldb, tb[0].numel(), c.data_ptr(), out_f32, N, M * N, M, N, K, bz, alpha, stream)
    torch.cuda.synchronize()
    ref = alpha * torch.bmm(a.double().cpu(), b.double().cpu().transpose(1, 2))
    err = max_rel(c.float().cpu().numpy(), ref.cpu().numpy())
    assert err <= (1e-5 if out_f32 else 8e-3), err


@pytest.mark.gpu
@pytest.mark.parametrize("R,M,N", [(147456, 520, 128), (4096, 128, 128), (300, 24, 40)])
def test_wgrad_split_k(gpu, R, M, N):
    """tpf_wgrad_bf16: dW = dy^T x over R rows (split-K + fixed-order fold)."""
    from openfold3_triangle_kernel_amd import _native

    g = torch.Generator(device="cpu").manual_seed(R + M)
    dy = torch.randn(R, M, generator=g).to(torch.bfloat16).to(gpu)
    x = torch.randn(R, N, generator=g).to(torch.bfloat16).to(gpu)
    dw = torch.empty(M, N, device=gpu)
    ws_bytes = int(_native.query("tpf_wgrad_bf16_workspace_bytes", R, M, N))
    ws = torch.empty(ws_bytes, device=gpu, dtype=torch.uint8)
    stream = torch.cuda.current_stream().cuda_stream
    _native.call("tpf_wgrad_bf16", dy.data_ptr(), M, x.data_ptr(), N, R, M, N, dw.data_ptr(),
                 ws.data_ptr(), ws_bytes, stream)
    torch.cuda.synchronize()
    ref = dy.double().t() @ x.double()
    assert max_rel(dw.cpu().numpy(), ref.cpu().numpy()) <= 1e-5
    dw2 = torch.empty_like(dw)
    _native.call("tpf_wgrad_bf16", dy.data_ptr(), M, x.data_ptr(), N, R, M, N, dw2.data_ptr(),
                 ws.data_ptr(), ws_bytes, stream)
    torch.cuda.synchronize()
    assert torch.equal(dw, dw2)  # fixed-order fold: bitwise replay


# Tall products with a small weight (the pair-row projections) dispatch to the
# weight-stationary row kernel: batch 1, K-contiguous x, bf16 out, alpha 1,
# K = 128, N a multiple of 16 up to 640 (W K- or MN-contiguous); the K = 576
# cases (dx = dproj W_all) take the tile GEMM through the same entry point.
ROW_CASES = [
    # R, N, K
    (1, 16, 128),
    (31, 128, 128),
    (1000, 576, 128),
    (4133, 48, 128),
    (70000, 576, 128),
    (9999, 128, 576),
    (33, 112, 576),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", ROW_CASES, ids=lambda c: "x".join(map(str, c)))
@pytest.mark.parametrize("w_kc", [1, 0], ids=["W_NK", "W_KN"])
def test_row_gemm(gpu, case, w_kc):
    """Against the FP64 product (bf16 output: <= 8e-3 max-rel) and row-chunk
    invariance: rows computed in a separate call give the same bits."""
    from openfold3_triangle_kernel_amd import _native

    R, N, K = case
    print(f"row gemm R={R} N={N} K={K} w_kc={w_kc}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(R + N + K)
    x = torch.randn(R, K, generator=g).to(torch.bfloat16).to(gpu)
    w = torch.randn(N, K, generator=g).to(torch.bfloat16).to(gpu)
    tw, ldw = _operand(w, w_kc)
    stream = torch.cuda.current_stream().cuda_stream

    def run(xs):
        y = torch.full((xs.shape[0], N), float("nan"), device=gpu, dtype=torch.bfloat16)
        _native.call("tpf_gemm_bf16", xs.data_ptr(), 1, K, 0, tw.data_ptr(), w_kc, ldw, 0,
                     y.data_ptr(), 0, N, 0, xs.shape[0], N, K, 1, 1.0, stream)
        return y

    y = run(x)
    lo, hi = R // 3, R // 3 + max(1, R // 2)
    part = run(x[lo:hi].contiguous())
    torch.cuda.synchronize()
    ref = x.double().cpu() @ w.double().cpu().t()
    assert max_rel(y.float().cpu().numpy(), ref.numpy()) <= 8e-3
    assert torch.equal(part.view(torch.int16), y[lo:hi].view(torch.int16)), "row chunk differs"


@pytest.mark.gpu
def test_row_gemm_output_beyond_2gib(gpu):
    """An output larger than 2 GiB (buffer offsets are per 32-row block):
    the last rows match a separate call on them bitwise and the FP32
    product within the bf16 tolerance."""
    from openfold3_triangle_kernel_amd import _native

    R, N, K = 1_900_000, 576, 128
    assert R * N * 2 > 2**31
    g = torch.Generator(device=gpu).manual_seed(11)
    x = torch.randn(R, K, device=gpu, generator=g).to(torch.bfloat16)
    w = torch.randn(N, K, device=gpu, generator=g).to(torch.bfloat16)
    stream = torch.cuda.current_stream().cuda_stream
    print(f"row gemm R={R} N={N} K={K} (> 2 GiB output)", flush=True)

    def run(xs):
        y = torch.empty((xs.shape[0], N), device=gpu, dtype=torch.bfloat16)
        _native.call("tpf_gemm_bf16", xs.data_ptr(), 1, K, 0, w.data_ptr(), 1, K, 0, y.data_ptr(), 0,
                     N, 0, xs.shape[0], N, K, 1, 1.0, stream)
        return y

    y = run(x)
    tail = run(x[R - 1000:].contiguous())
    torch.cuda.synchronize()
    assert torch.equal(tail.view(torch.int16), y[R - 1000:].view(torch.int16))
    ref = x[R - 1000:].float() @ w.float().t()
    assert max_rel(y[R - 1000:].float().cpu().numpy(), ref.cpu().numpy()) <= 8e-3
    del y


@pytest.mark.gpu
@pytest.mark.parametrize("B,N,H,D", [(1, 64, 4, 32), (2, 96, 2, 16), (1, 128, 4, 24)])
def test_pair_projection_split(gpu, B, N, H, D):
    """tpf_pair_projection_bf16: x W^T with q | k | v written as head-major
    planes [3, B, N(i), H, N(j), D] and the remaining columns as rows, bitwise
    equal to the row GEMM's plain output rearranged."""
    from openfold3_triangle_kernel_amd import _native

    C, hc = 128, H * D
    P = (4 * hc + H + 63) // 64 * 64
    R = B * N * N
    assert _native.query("tpf_pair_projection_supported", P, C, N, H, D)
    g = torch.Generator(device="cpu").manual_seed(B + N + H + D)
    x = torch.randn(R, C, generator=g).to(torch.bfloat16).to(gpu)
    w = torch.randn(P, C, generator=g).to(torch.bfloat16).to(gpu)
    qkv = torch.full((3, B, N, H, N, D), float("nan"), device=gpu, dtype=torch.bfloat16)
    rest = torch.full((R, P - 3 * hc), float("nan"), device=gpu, dtype=torch.bfloat16)
    y = torch.empty((R, P), device=gpu, dtype=torch.bfloat16)
    stream = torch.cuda.current_stream().cuda_stream
    print(f"pair projection B={B} N={N} H={H} D={D} P={P}", flush=True)
    _native.call("tpf_pair_projection_bf16", x.data_ptr(), w.data_ptr(), B, N, C, P, H, D,
                 qkv.data_ptr(), rest.data_ptr(), stream)
    _native.call("tpf_gemm_bf16", x.data_ptr(), 1, C, 0, w.data_ptr(), 1, C, 0, y.data_ptr(), 0, P,
                 0, R, P, C, 1, 1.0, stream)
    torch.cuda.synchronize()
    want_qkv = y[:, :3 * hc].reshape(B, N, N, 3, H, D).permute(3, 0, 1, 4, 2, 5)
    assert torch.equal(qkv.view(torch.int16), want_qkv.contiguous().view(torch.int16))
    assert torch.equal(rest.view(torch.int16), y[:, 3 * hc:].contiguous().view(torch.int16))
    ref = x.double().cpu() @ w.double().cpu().t()
    assert max_rel(y.float().cpu().numpy(), ref.numpy()) <= 8e-3
