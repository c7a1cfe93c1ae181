// Split-K weight-gradient products (MN-contiguous operands, f32 partials
// folded in fixed order): the TriMul dW5 / dW_z pair and the pair-stack
// projection weight gradients.  Own translation unit for its stage shape:
// 64-deep k-steps, two stages (measured best for these long-K, few-tile
// products; the contraction shape in gemm.hip is 32 deep, three stages).
#define TPF_GEMM_IMPL gk64
#include "gemm_impl.hpp"

namespace tpf {

using namespace gk64;

int gemm_launch_wgrad(const GemmArgs& g0, hipStream_t stream, const char* fn) {
  GemmArgs g = g0;
  int rc = gemm_prepare(g, 0, 0, 1, g0.batch > 0 ? g0.batch : 1, fn);
  if (rc) return rc;
  dim3 grid((unsigned)((gemm_tiles(g) + 7) / 8 * 8));
  hipLaunchKernelGGL((gemm_bf16_kernel<false, false, true>), grid, dim3(256), 0, stream, g);
  return check_launch(fn);
}

int gemm_launch_pair_wgrad(const GemmArgs& p0, const GemmArgs& p1, hipStream_t stream,
                           const char* fn) {
  GemmArgs g0 = p0, g1 = p1;
  int rc = gemm_prepare(g0, 0, 0, 1, p0.batch > 0 ? p0.batch : 1, fn);
  if (rc) return rc;
  if ((rc = gemm_prepare(g1, 0, 0, 1, p1.batch > 0 ? p1.batch : 1, fn))) return rc;
  const int64_t blocks = (gemm_tiles(g0) + 7) / 8 * 8 + (gemm_tiles(g1) + 7) / 8 * 8;
  if (blocks > INT32_MAX) return set_error(TPF_ERR_SHAPE, "%s: GEMM grid too large", fn);
  hipLaunchKernelGGL((gemm_bf16_pair_kernel<false, false, false, false, true>), dim3((unsigned)blocks),
                     dim3(256), 0, stream, g0, g1);
  return check_launch(fn);
}

}  // namespace tpf

// Weight gradient of a linear layer over many rows: dW[m][n] = sum_r dy[r][m] x[r][n]
// (dy [R][M] and x [R][N] row-major bf16, both read MN-contiguous), split over
// R with f32 partials and the fixed-order fold (deterministic).  The shape
// of every projection weight gradient of the pair stack (K = B*N^2 rows).
// The split count fills one round of 512 workgroups (two per CU on 256 CUs)
// without spilling into a second: a launch of 515 for 5 output tiles ran
// its last 3 workgroups as a round of their own, doubling the time.  At
// most 256 splits: a one-tile product gains nothing from 512 (its fold of
// twice the partials cost more, 9 -> 25 us at 128 x 128).  The count depends
// on the shape only (fixed fold order on every device).
static int wgrad_splits(int64_t R, int64_t M, int64_t N) {
  const int64_t tiles = ((M + tpf::kGM - 1) / tpf::kGM) * ((N + tpf::kGN - 1) / tpf::kGN);
  int64_t s = 512 / tiles;
  if (s > R / 256) s = R / 256;
  if (s > 256) s = 256;
  if (s < 1) s = 1;
  return (int)s;
}

extern "C" int64_t tpf_wgrad_bf16_workspace_bytes(int64_t R, int64_t M, int64_t N) {
  return (int64_t)wgrad_splits(R, M, N) * M * N * 4;
}

extern "C" int tpf_wgrad_bf16(const void* dy, int64_t ld_dy, const void* x, int64_t ld_x,
                              int64_t R, int64_t M, int64_t N, float* dw, void* workspace,
                              int64_t workspace_bytes, void* stream) {
  const char* fn = "tpf_wgrad_bf16";
  if (!dy || !x || !dw || !workspace) return tpf::set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  if (R < 1 || M < 1 || N < 1 || R > INT32_MAX || M > INT32_MAX || N > INT32_MAX)
    return tpf::set_error(TPF_ERR_SHAPE, "%s: bad shape", fn);
  if (workspace_bytes < tpf_wgrad_bf16_workspace_bytes(R, M, N))
    return tpf::set_error(TPF_ERR_ARG, "%s: workspace too small", fn);
  const int splits = wgrad_splits(R, M, N);
  tpf::GemmArgs g{};
  g.A = (const __bf16*)dy; g.a_ld = ld_dy; g.a_bs = 0;
  g.B = (const __bf16*)x; g.b_ld = ld_x; g.b_bs = 0;
  g.C = workspace; g.c_ld = N; g.c_bs = 0; g.c_split = M * N;
  g.M = (int)M; g.N = (int)N; g.K = (int)R; g.ksplit = splits;
  g.k_chunk = (int)((R + splits - 1) / splits); g.alpha = 1.f;
  hipStream_t s = (hipStream_t)stream;
  int rc = tpf::gemm_launch_wgrad(g, s, fn);
  if (rc) return rc;
  return tpf::fold_launch((const float*)workspace, dw, M * N, M * N, splits, s, fn);
}
