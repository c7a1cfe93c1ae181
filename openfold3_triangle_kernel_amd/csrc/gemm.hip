// Batched bf16 GEMM on gfx950 MFMA for the TriMul channel contraction, its
// backward products and the split-K weight-gradient products.
//
//   C[z][m][n] = alpha * sum_k A[z](m, k) * B[z](n, k)
//
// A and B are each given either K-contiguous ("KC": X[r * ld + k]) or
// MN-contiguous ("MN": X[k * ld + r]); the LDS tiles are always K-contiguous,
// so every layout feeds the MFMA the same way.  C is row-major (n contiguous)
// in bf16 or f32.  Split-K writes f32 partials at C + split * c_split and a
// fixed-order fold kernel sums them (deterministic, no atomics).
//
// Tile: 128 x 128 x 32 per 256-thread workgroup, 4 waves in a 2 x 2 grid of
// 64 x 64 sub-tiles (2 x 2 MFMA 32x32x16 tiles each).  The next K tile is
// fetched into registers while the current one is multiplied.
#include "common.hpp"
#include "tpf_gemm.hpp"
#include "tpf_status.hpp"

namespace tpf {

constexpr int GBM = 128, GBN = 128, GBK = 32, GPITCH = GBK + 8;

template <bool KC>
__device__ __forceinline__ void gemm_load(const __bf16* __restrict__ X, int64_t ld, int r0,
                                          int R, int k0, int kend, int tid, bf16x8 (&reg)[2]) {
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int idx = it * 256 + tid;
    if (KC) {
      const int r = idx >> 2, kc = (idx & 3) * 8;
      const bool ok = (r0 + r < R) && (k0 + kc < kend);
      reg[it] = ok ? ld8(X + (int64_t)(r0 + r) * ld + k0 + kc) : zero8();
    } else {
      const int k = idx >> 4, rc = (idx & 15) * 8;
      const bool ok = (r0 + rc < R) && (k0 + k < kend);
      reg[it] = ok ? ld8(X + (int64_t)(k0 + k) * ld + r0 + rc) : zero8();
    }
  }
}

template <bool KC>
__device__ __forceinline__ void gemm_store_lds(__bf16* S, int tid, const bf16x8 (&reg)[2]) {
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int idx = it * 256 + tid;
    if (KC) {
      const int r = idx >> 2, kc = (idx & 3) * 8;
      *reinterpret_cast<bf16x8*>(&S[r * GPITCH + kc]) = reg[it];
    } else {
      const int k = idx >> 4, rc = (idx & 15) * 8;
#pragma unroll
      for (int e = 0; e < 8; ++e) S[(rc + e) * GPITCH + k] = reg[it][e];
    }
  }
}

template <bool A_KC, bool B_KC, bool OUT_F32>
__global__ __launch_bounds__(256) void gemm_bf16_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) __bf16 As[GBM * GPITCH];
  __shared__ __attribute__((aligned(16))) __bf16 Bs[GBN * GPITCH];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int rl = lane & 31, hl = lane >> 5;
  const int wm = w >> 1, wn = w & 1;
  const int n0 = blockIdx.x * GBN, m0 = blockIdx.y * GBM;
  const int z = blockIdx.z / g.ksplit, split = blockIdx.z % g.ksplit;
  const int kbeg = split * g.k_chunk;
  const int kend = min(g.K, kbeg + g.k_chunk);
  const __bf16* A = g.A + (int64_t)z * g.a_bs;
  const __bf16* B = g.B + (int64_t)z * g.b_bs;

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = zero16();

  bf16x8 ra[2], rb[2];
  gemm_load<A_KC>(A, g.a_ld, m0, g.M, kbeg, kend, tid, ra);
  gemm_load<B_KC>(B, g.b_ld, n0, g.N, kbeg, kend, tid, rb);
  for (int k0 = kbeg; k0 < kend; k0 += GBK) {
    __syncthreads();
    gemm_store_lds<A_KC>(As, tid, ra);
    gemm_store_lds<B_KC>(Bs, tid, rb);
    __syncthreads();
    if (k0 + GBK < kend) {
      gemm_load<A_KC>(A, g.a_ld, m0, g.M, k0 + GBK, kend, tid, ra);
      gemm_load<B_KC>(B, g.b_ld, n0, g.N, k0 + GBK, kend, tid, rb);
    }
#pragma unroll
    for (int ks = 0; ks < GBK / 16; ++ks) {
      bf16x8 af[2], bfr[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        af[t] = *reinterpret_cast<const bf16x8*>(&As[(wm * 64 + t * 32 + rl) * GPITCH + ks * 16 + 8 * hl]);
        bfr[t] = *reinterpret_cast<const bf16x8*>(&Bs[(wn * 64 + t * 32 + rl) * GPITCH + ks * 16 + 8 * hl]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma32(af[i], bfr[j], acc[i][j]);
    }
  }

  char* Cb = (char*)g.C + ((int64_t)z * g.c_bs + (int64_t)split * g.c_split) * (OUT_F32 ? 4 : 2);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + wn * 64 + j * 32 + rl;
      if (col >= g.N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * hl + (r & 3);
        if (row < g.M) {
          const float val = acc[i][j][r] * g.alpha;
          const int64_t off = (int64_t)row * g.c_ld + col;
          if (OUT_F32) reinterpret_cast<float*>(Cb)[off] = val;
          else reinterpret_cast<__bf16*>(Cb)[off] = f2bf(val);
        }
      }
    }
}

// Fixed-order fold of split partials: thread (i, j) sums splits
// [j*chunk, min((j+1)*chunk, splits)) in ascending order and writes the
// result to dst + j*dst_stride + i.  Repeated passes (chunk 64) reduce any
// number of splits; the order depends only on the shapes (deterministic).
__global__ __launch_bounds__(256) void fold_f32_kernel(const float* __restrict__ part,
                                                       float* __restrict__ dst, int64_t n,
                                                       int64_t stride, int splits, int chunk,
                                                       int64_t dst_stride) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int j = blockIdx.y;
  if (i >= n) return;
  const int s0 = j * chunk, s1 = min(splits, s0 + chunk);
  float acc = part[(int64_t)s0 * stride + i];
  for (int s = s0 + 1; s < s1; ++s) acc += part[(int64_t)s * stride + i];
  dst[(int64_t)j * dst_stride + i] = acc;
}

int gemm_launch(const GemmArgs& g0, int a_kc, int b_kc, int out_f32, int batch,
                hipStream_t stream, const char* fn) {
  GemmArgs g = g0;
  if (g.M < 1 || g.N < 1 || g.K < 1 || batch < 1 || g.ksplit < 1)
    return set_error(TPF_ERR_SHAPE, "%s: bad GEMM shape M=%d N=%d K=%d", fn, g.M, g.N, g.K);
  // 16-byte vector loads: leading dimensions are multiples of 8 elements.  A
  // K-contiguous operand needs K % 8 == 0 (callers zero-pad); an MN-contiguous
  // operand may read up to 7 elements past M (or N) inside its row pitch.
  if (g.a_ld % 8 || g.b_ld % 8 || (a_kc && g.K % 8) || (b_kc && g.K % 8) ||
      (!a_kc && g.a_ld < (g.M + 7) / 8 * 8) || (!b_kc && g.b_ld < (g.N + 7) / 8 * 8))
    return set_error(TPF_ERR_SHAPE, "%s: GEMM operand pitch/padding requirement violated", fn);
  if (g.ksplit > 1 && !out_f32)
    return set_error(TPF_ERR_ARG, "%s: split-K needs f32 output", fn);
  if (g.k_chunk <= 0) g.k_chunk = g.K;
  g.k_chunk = ((g.k_chunk + GBK - 1) / GBK) * GBK;
  dim3 grid((g.N + GBN - 1) / GBN, (g.M + GBM - 1) / GBM, (unsigned)(batch * g.ksplit));
  if (grid.z > 65535 || grid.y > 65535) return set_error(TPF_ERR_SHAPE, "%s: GEMM grid too large", fn);
#define TPF_GEMM_CASE(AK, BK, OF)                                                            \
  if (a_kc == AK && b_kc == BK && out_f32 == OF) {                                            \
    hipLaunchKernelGGL((gemm_bf16_kernel<AK, BK, OF>), grid, dim3(256), 0, stream, g);         \
    return check_launch(fn);                                                                  \
  }
  TPF_GEMM_CASE(1, 1, 0)
  TPF_GEMM_CASE(1, 1, 1)
  TPF_GEMM_CASE(1, 0, 0)
  TPF_GEMM_CASE(1, 0, 1)
  TPF_GEMM_CASE(0, 1, 0)
  TPF_GEMM_CASE(0, 1, 1)
  TPF_GEMM_CASE(0, 0, 0)
  TPF_GEMM_CASE(0, 0, 1)
#undef TPF_GEMM_CASE
  return set_error(TPF_ERR_ARG, "%s: bad GEMM layout flags", fn);
}

int fold_launch(const float* part, float* out, int64_t n, int64_t stride, int splits,
                hipStream_t stream, const char* fn) {
  // Passes of 64-way chunks, written in place into each chunk's first slot.
  constexpr int kChunk = 64;
  float* buf = const_cast<float*>(part);
  int64_t st = stride;
  while (splits > kChunk) {
    const int groups = (splits + kChunk - 1) / kChunk;
    hipLaunchKernelGGL(fold_f32_kernel, dim3((unsigned)((n + 255) / 256), (unsigned)groups),
                       dim3(256), 0, stream, buf, buf, n, st, splits, kChunk, st * kChunk);
    int rc = check_launch(fn);
    if (rc) return rc;
    splits = groups;
    st *= kChunk;
  }
  hipLaunchKernelGGL(fold_f32_kernel, dim3((unsigned)((n + 255) / 256), 1), dim3(256), 0, stream,
                     buf, out, n, st, splits, splits, (int64_t)0);
  return check_launch(fn);
}

}  // namespace tpf

extern "C" int tpf_gemm_bf16(const void* A, int a_kc, int64_t a_ld, int64_t a_bs, const void* B,
                             int b_kc, int64_t b_ld, int64_t b_bs, void* C, int out_f32,
                             int64_t c_ld, int64_t c_bs, int64_t M, int64_t N, int64_t K,
                             int64_t batch, double alpha, void* stream) {
  if (!A || !B || !C) return tpf::set_error(TPF_ERR_ARG, "tpf_gemm_bf16: null pointer");
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
    return tpf::set_error(TPF_ERR_SHAPE, "tpf_gemm_bf16: dimension exceeds int32");
  tpf::GemmArgs g{};
  g.A = (const __bf16*)A; g.a_ld = a_ld; g.a_bs = a_bs;
  g.B = (const __bf16*)B; g.b_ld = b_ld; g.b_bs = b_bs;
  g.C = C; g.c_ld = c_ld; g.c_bs = c_bs; g.c_split = 0;
  g.M = (int)M; g.N = (int)N; g.K = (int)K; g.ksplit = 1; g.k_chunk = (int)K;
  g.alpha = (float)alpha;
  return tpf::gemm_launch(g, a_kc, b_kc, out_f32, (int)batch, (hipStream_t)stream, "tpf_gemm_bf16");
}
