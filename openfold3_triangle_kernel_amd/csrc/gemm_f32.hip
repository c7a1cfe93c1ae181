// Batched FP32 GEMM on gfx950 MFMA (inference-only FP32 paths):
//
//   C[z][m][n] = alpha * sum_k A[z](m, k) * B[z](n, k) + bias[n]
//
// A and B are K-contiguous ("KC": X[r * ld + k]) or MN-contiguous ("MN":
// X[k * ld + r]); C is row-major f32.  The main loop is gemm_core_f32.hpp.
// Replaces the reference's strict-FP32 cuBLAS products of the FP32 TriMul
// (openfold3/core/kernels/turbopairformer/turbopairformer_trimul_fp32.py:336-360).
#include "common.hpp"
#include "gemm_core.hpp"
#include "gemm_core_f32.hpp"
#include "tpf_gemm.hpp"
#include "tpf_status.hpp"

namespace tpf {

template <bool A_KC, bool B_KC>
__global__ __launch_bounds__(256, 2) void gemm_f32_kernel(GemmArgsF32 g) {
  __shared__ __attribute__((aligned(1024))) char smem[kFMainLdsBytes];
  const int tm = (g.M + kFM - 1) / kFM, tn = (g.N + kFN - 1) / kFN;
  const int64_t T = xcd_order((int64_t)tm * tn * g.batch);
  if (T < 0) return;
  const int nt = (int)(T % tn);
  const int64_t r = T / tn;
  const int mt = (int)(r % tm);
  const int z = (int)(r / tm);
  const int m0 = mt * kFM, n0 = nt * kFN;
  GemmOperandF32 A{g.A + (int64_t)z * g.a_bs, g.a_ld, g.M, g.a_gather_n, g.a_div_n, g.a_div_nn};
  GemmOperandF32 B{g.B + (int64_t)z * g.b_bs, g.b_ld, g.N, 0, {}, {}};
  f32x16 acc[2][2];
  gemm_tile_f32<A_KC, B_KC>(A, B, m0, n0, 0, g.K, smem, acc);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int rl = lane & 31, hl = lane >> 5, wm = w >> 1, wn = w & 1;
  float* C = g.C + (int64_t)z * g.c_bs;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int col = n0 + wn * 64 + j * 32 + rl;
    if (col >= g.N) continue;
    const float bv = g.bias ? g.bias[col] : 0.f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) {
        const int row = m0 + wm * 64 + i * 32 + 8 * (rr >> 2) + 4 * hl + (rr & 3);
        if (row < g.M) C[(int64_t)row * g.c_ld + col] = fmaf(acc[i][j][rr], g.alpha, bv);
      }
  }
}

int gemm_f32_launch(const GemmArgsF32& g0, int a_kc, int b_kc, int batch, hipStream_t stream,
                    const char* fn) {
  GemmArgsF32 g = g0;
  g.batch = batch;
  if (g.M < 1 || g.N < 1 || g.K < 1 || batch < 1)
    return set_error(TPF_ERR_SHAPE, "%s: bad GEMM shape M=%d N=%d K=%d", fn, g.M, g.N, g.K);
  // 16-byte loads: leading dimensions are multiples of 4 elements; a KC
  // operand needs K % 4 == 0, an MN operand may read up to 3 elements past
  // M (or N) inside its row pitch.
  if (g.a_ld % 4 || g.b_ld % 4 || (a_kc && g.K % 4) || (b_kc && g.K % 4) ||
      (!a_kc && g.a_ld < (g.M + 3) / 4 * 4) || (!b_kc && g.b_ld < (g.N + 3) / 4 * 4) ||
      ((uintptr_t)g.A % 16) || ((uintptr_t)g.B % 16) || (g.a_bs % 4) || (g.b_bs % 4))
    return set_error(TPF_ERR_SHAPE, "%s: GEMM operand pitch/padding/alignment requirement violated",
                     fn);
  if (g.a_gather_n > 0 && !a_kc)
    return set_error(TPF_ERR_ARG, "%s: row gather needs a K-contiguous A", fn);
  if (g.a_gather_n > 0) {
    g.a_div_n = make_fastdiv((uint32_t)g.a_gather_n);
    g.a_div_nn = make_fastdiv((uint32_t)g.a_gather_n * (uint32_t)g.a_gather_n);
  }
  const int64_t a_span = a_kc ? (int64_t)g.M * g.a_ld : (int64_t)g.K * g.a_ld;
  const int64_t b_span = b_kc ? (int64_t)g.N * g.b_ld : (int64_t)g.K * g.b_ld;
  if (a_span * 4 >= (int64_t)kBufOOB || b_span * 4 >= (int64_t)kBufOOB)
    return set_error(TPF_ERR_SHAPE, "%s: GEMM operand exceeds 2 GiB per batch item", fn);
  const int64_t total = (int64_t)((g.M + kFM - 1) / kFM) * ((g.N + kFN - 1) / kFN) * batch;
  const int64_t blocks = (total + 7) / 8 * 8;
  if (blocks > INT32_MAX) return set_error(TPF_ERR_SHAPE, "%s: GEMM grid too large", fn);
  dim3 grid((unsigned)blocks);
  if (a_kc && b_kc) hipLaunchKernelGGL((gemm_f32_kernel<true, true>), grid, dim3(256), 0, stream, g);
  else if (a_kc) hipLaunchKernelGGL((gemm_f32_kernel<true, false>), grid, dim3(256), 0, stream, g);
  else if (b_kc) hipLaunchKernelGGL((gemm_f32_kernel<false, true>), grid, dim3(256), 0, stream, g);
  else hipLaunchKernelGGL((gemm_f32_kernel<false, false>), grid, dim3(256), 0, stream, g);
  return check_launch(fn);
}

}  // namespace tpf

extern "C" int tpf_gemm_f32(const float* A, int a_kc, int64_t a_ld, int64_t a_bs, const float* B,
                            int b_kc, int64_t b_ld, int64_t b_bs, float* C, int64_t c_ld,
                            int64_t c_bs, int64_t M, int64_t N, int64_t K, int64_t batch,
                            double alpha, const float* bias, void* stream) {
  if (!A || !B || !C) return tpf::set_error(TPF_ERR_ARG, "tpf_gemm_f32: null pointer");
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX || batch > INT32_MAX)
    return tpf::set_error(TPF_ERR_SHAPE, "tpf_gemm_f32: dimension exceeds int32");
  tpf::GemmArgsF32 g{};
  g.A = A; g.a_ld = a_ld; g.a_bs = a_bs;
  g.B = B; g.b_ld = b_ld; g.b_bs = b_bs;
  g.C = C; g.c_ld = c_ld; g.c_bs = c_bs;
  g.M = (int)M; g.N = (int)N; g.K = (int)K;
  g.alpha = (float)alpha; g.bias = bias;
  return tpf::gemm_f32_launch(g, a_kc, b_kc, (int)batch, (hipStream_t)stream, "tpf_gemm_f32");
}
