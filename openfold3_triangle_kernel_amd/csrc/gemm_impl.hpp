// Batched bf16 GEMM tiles, kernels and argument checks, compiled by each
// translation unit that includes this header with its own stage shape
// (TPF_GEMM_GK / TPF_GEMM_NS) into its own namespace TPF_GEMM_IMPL, so that
// kernels of different stage shapes never share a name.
#pragma once

#include "common.hpp"
#include "gemm_core.hpp"
#include "tpf_gemm.hpp"
#include "tpf_status.hpp"

#ifndef TPF_GEMM_IMPL
#error "define TPF_GEMM_IMPL (the namespace of this stage shape) before including gemm_impl.hpp"
#endif

namespace tpf {
namespace TPF_GEMM_IMPL {

// Tile T of problem g (T < tiles of g, in (n-tile, m-tile, split, batch)
// order) into C.
// TM: the square tile size (128, or 192 for the TriMul contractions whose
// sizes are multiples of 192).
template <int TM>
constexpr int gemm_smem_bytes() {
  // The ring, and the bf16 epilogue's staging of four TM/2 x TM/2 sub-tiles.
  return gemm_ring_bytes(kGNS, TM) > 4 * (TM / 2) * (TM / 2 + 8) * 2
             ? gemm_ring_bytes(kGNS, TM)
             : 4 * (TM / 2) * (TM / 2 + 8) * 2;
}

template <bool A_KC, bool B_KC, bool OUT_F32, int TM = kGM>
__device__ __forceinline__ void gemm_bf16_tile(const GemmArgs& g, int64_t T, char* smem) {
  constexpr int NB = TM / 64, HT = TM / 2;
  const int tm = (g.M + TM - 1) / TM, tn = (g.N + TM - 1) / TM;
  const int nt = (int)(T % tn);
  int64_t r = T / tn;
  const int mt = (int)(r % tm);
  r /= tm;
  const int split = (int)(r % g.ksplit);
  const int z = (int)(r / g.ksplit);
  const int m0 = mt * TM, n0 = nt * TM;
  const int kbeg = split * g.k_chunk;
  const int kend = min(g.K, kbeg + g.k_chunk);
  GemmOperand A{g.A + (int64_t)z * g.a_bs, g.a_ld, g.M, g.a_gather_n, g.a_div_n, g.a_div_nn};
  GemmOperand B{g.B + (int64_t)z * g.b_bs, g.b_ld, g.N, 0, {}, {}, g.b_kmax > 0 ? g.b_kmax : 0x7fffffff};
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int rl = lane & 31, hl = lane >> 5, wm = w >> 1, wn = w & 1;
  char* Cb = (char*)g.C + ((int64_t)z * g.c_bs + (int64_t)split * g.c_split) * (OUT_F32 ? 4 : 2);
  f32x16 acc[NB][NB];
  if constexpr (OUT_F32) {
    gemm_tile<A_KC, B_KC, kGNS, TM>(A, B, m0, n0, kbeg, kend, smem, acc);
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int col = n0 + wn * HT + j * 32 + rl;
        if (col >= g.N) continue;
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) {
          const int row = m0 + wm * HT + i * 32 + 8 * (rr >> 2) + 4 * hl + (rr & 3);
          if (row < g.M)
            reinterpret_cast<float*>(Cb)[(int64_t)row * g.c_ld + col] = acc[i][j][rr] * g.alpha;
        }
      }
  } else {
    // bf16 output: the tile is formed transposed (C^T = B A^T), so each lane's
    // four consecutive accumulator registers are four consecutive columns of
    // C; wave w stages its TM/2 x TM/2 sub-tile (rows TM/2 (w & 1), columns
    // TM/2 (w >> 1)) in LDS as bf16 rows and writes it back with 16-byte
    // stores, whole row segments of TM bytes per group of TM / 16 lanes.
    gemm_tile<B_KC, A_KC, kGNS, TM>(B, A, n0, m0, kbeg, kend, smem, acc);
    constexpr int EP = HT + 8;  // staged row pitch (bf16)
    static_assert(4 * HT * EP * 2 <= gemm_smem_bytes<TM>(), "epilogue staging fits");
    __bf16* Ls = reinterpret_cast<__bf16*>(smem) + w * HT * EP;
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          bf16x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = f2bf(acc[i][j][4 * r4 + e] * g.alpha);
          *reinterpret_cast<bf16x4*>(&Ls[(32 * j + rl) * EP + 32 * i + 8 * r4 + 4 * hl]) = v;
        }
    __syncthreads();
    const bool vec = ((g.c_ld | g.c_bs) % 8 == 0) && ((uintptr_t)g.C % 16 == 0);
    __bf16* Cw = reinterpret_cast<__bf16*>(Cb);
    constexpr int CPR = HT / 8;  // 16-byte chunks per staged row
#pragma unroll
    for (int it = 0; it < HT * CPR / 64; ++it) {
      const int q = 64 * it + lane;
      const int rr = q / CPR, ch = q % CPR;
      const int row = m0 + HT * wn + rr, col = n0 + HT * wm + 8 * ch;
      if (row >= g.M || col >= g.N) continue;
      const bf16x8 v = *reinterpret_cast<const bf16x8*>(&Ls[rr * EP + 8 * ch]);
      __bf16* dst = Cw + (int64_t)row * g.c_ld + col;
      if (vec && col + 8 <= g.N) {
        st8(dst, v);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (col + e < g.N) dst[e] = v[e];
      }
    }
  }
}

__host__ __device__ inline int64_t gemm_tiles(const GemmArgs& g, int tm = kGM) {
  return (int64_t)((g.M + tm - 1) / tm) * ((g.N + tm - 1) / tm) * g.batch * g.ksplit;
}

template <bool A_KC, bool B_KC, bool OUT_F32, int TM = kGM>
__global__ __launch_bounds__(256, 2) void gemm_bf16_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) char smem[gemm_smem_bytes<TM>()];
  const int64_t T = xcd_order(gemm_tiles(g, TM));
  if (T < 0) return;
  gemm_bf16_tile<A_KC, B_KC, OUT_F32, TM>(g, T, smem);
}

// Two problems of one layout in one grid: workgroups [0, p0) take the
// tiles of g0 and the rest those of g1 (p0 = g0's tiles rounded up to 8),
// each in its own XCD-aware order, so both problems spread over all XCDs
// and independent small GEMMs stay in flight together.
template <bool AK0, bool BK0, bool AK1, bool BK1, bool OUT_F32, int TM = kGM>
__global__ __launch_bounds__(256, 2) void gemm_bf16_pair_kernel(GemmArgs g0, GemmArgs g1) {
  __shared__ __attribute__((aligned(1024))) char smem[gemm_smem_bytes<TM>()];
  const int64_t t0 = gemm_tiles(g0, TM), p0 = (t0 + 7) / 8 * 8;
  const int64_t L = blockIdx.x;
  if (L < p0) {
    const int64_t T = xcd_order_of(L, t0);
    if (T >= 0) gemm_bf16_tile<AK0, BK0, OUT_F32, TM>(g0, T, smem);
  } else {
    const int64_t T = xcd_order_of(L - p0, gemm_tiles(g1, TM));
    if (T >= 0) gemm_bf16_tile<AK1, BK1, OUT_F32, TM>(g1, T, smem);
  }
}

static inline int gemm_prepare(GemmArgs& g, int a_kc, int b_kc, int out_f32, int batch, const char* fn) {
  g.batch = batch;
  if (g.M < 1 || g.N < 1 || g.K < 1 || batch < 1 || g.ksplit < 1)
    return set_error(TPF_ERR_SHAPE, "%s: bad GEMM shape M=%d N=%d K=%d", fn, g.M, g.N, g.K);
  // 16-byte loads: leading dimensions are multiples of 8 elements.  A
  // K-contiguous operand needs K % 8 == 0 (callers zero-pad); an
  // MN-contiguous operand may read up to 7 elements past M (or N) inside its
  // row pitch.
  if (g.a_ld % 8 || g.b_ld % 8 || (a_kc && g.K % 8) || (b_kc && g.K % 8) ||
      (!a_kc && g.a_ld < (g.M + 7) / 8 * 8) || (!b_kc && g.b_ld < (g.N + 7) / 8 * 8) ||
      ((int64_t)(uintptr_t)g.A % 16) || ((int64_t)(uintptr_t)g.B % 16) || (g.a_bs % 8) ||
      (g.b_bs % 8))
    return set_error(TPF_ERR_SHAPE, "%s: GEMM operand pitch/padding/alignment requirement violated",
                     fn);
  if (g.a_gather_n > 0 && !a_kc)
    return set_error(TPF_ERR_ARG, "%s: row gather needs a K-contiguous A", fn);
  if (g.a_gather_n > 0) {
    g.a_div_n = make_fastdiv((uint32_t)g.a_gather_n);
    g.a_div_nn = make_fastdiv((uint32_t)g.a_gather_n * (uint32_t)g.a_gather_n);
  }
  // Buffer offsets of one batch item must stay below 2^31 bytes.
  const int64_t a_span = a_kc ? (int64_t)g.M * g.a_ld : (int64_t)g.K * g.a_ld;
  const int64_t b_span = b_kc ? (int64_t)g.N * g.b_ld : (int64_t)g.K * g.b_ld;
  if (a_span * 2 >= (int64_t)kBufOOB || b_span * 2 >= (int64_t)kBufOOB)
    return set_error(TPF_ERR_SHAPE, "%s: GEMM operand exceeds 2 GiB per batch item", fn);
  if (g.ksplit > 1 && !out_f32)
    return set_error(TPF_ERR_ARG, "%s: split-K needs f32 output", fn);
  if (g.k_chunk <= 0) g.k_chunk = g.K;
  g.k_chunk = ((g.k_chunk + kGK - 1) / kGK) * kGK;
  if ((gemm_tiles(g) + 7) / 8 * 8 > INT32_MAX)
    return set_error(TPF_ERR_SHAPE, "%s: GEMM grid too large", fn);
  return TPF_OK;
}

}  // namespace TPF_GEMM_IMPL
}  // namespace tpf
