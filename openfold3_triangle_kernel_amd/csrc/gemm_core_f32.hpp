// FP32 MFMA GEMM main loop (gfx950 v_mfma_f32_32x32x2_f32, 256 threads =
// 4 waves per workgroup), for the inference-only FP32 paths.
//
//   acc(m, n) = sum_{k in [kbeg, kend)} A(m, k) * B(n, k)     (all f32)
//
// Tile 128 (m) x 128 (n) x 32 (k); wave w owns the 64 x 64 sub-tile
// (wm, wn) = (w >> 1, w & 1) as 2 x 2 accumulators in the 32x32 MFMA layout
//   acc[i][j] register r <-> m = 64 wm + 32 i + 8 (r / 4) + 4 (lane / 32) + r % 4,
//                            n = 64 wn + 32 j + lane % 32.
// One 32x32x2 MFMA consumes one k value per lane half; the k index is a pure
// summation index, so within every group of 8 k the lanes of the lower half
// supply k = 0..3 and those of the upper half k = 4..7 across four MFMAs,
// each lane feeding all four from one 16-byte LDS read.
//
// Operands are read from HBM straight into LDS (buffer_load ... lds, zeros
// outside the tensor), two k-stages in flight.  Either operand may be
//   KC (K-contiguous): X[row * ld + k] -- LDS tile [128 rows][32 k], the
//      16-byte chunk c of row r stored at slot c ^ (r & 7);
//   MN (MN-contiguous): X[k * ld + row] -- LDS tile [32 k][128 rows],
//      fragments are 4-byte reads of consecutive rows.
// A KC operand may gather its rows (the transposed pair order of the
// incoming TriMul direction, as in gemm_core.hpp).
#pragma once

#include "common.hpp"

namespace tpf {

constexpr int kFM = 128, kFN = 128, kFK = 32;
constexpr int kFTileBytes = kFM * kFK * 4;       // 16 KiB
constexpr int kFStageBytes = 2 * kFTileBytes;
constexpr int kFMainLdsBytes = 2 * kFStageBytes;  // 64 KiB

__device__ __forceinline__ f32x16 mfma32f(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

struct GemmOperandF32 {
  const float* p;  // element (0, 0) of this batch item
  int64_t ld;      // leading dimension in elements
  int rows;        // extent of the m (or n) dimension
  int gather_n;    // KC row gather (0 = none)
  FastDiv div_n, div_nn;
};

template <bool KC>
struct TileLoaderF32 {
  i32x4 rsrc;
  uint32_t row_off[4];  // KC: byte offset of each row start (kBufOOB if absent)
  int sub;              // KC: k offset of this lane; MN: k-row in instruction
  int col_ok;
  uint32_t col_off;
  int64_t ld;

  __device__ __forceinline__ void init(const GemmOperandF32& op, int r0) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    rsrc = buffer_rsrc(op.p);
    ld = op.ld;
    if (KC) {
      const int rin = lane >> 3;                  // 8 rows of 128 bytes per instruction
      sub = 4 * ((lane & 7) ^ (rin & 7));
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int row = r0 + 8 * (4 * w + t) + rin;
        uint32_t off = kBufOOB;
        if (row < op.rows) {
          int64_t prow = row;
          if (op.gather_n > 0) {
            const uint32_t n = op.gather_n, nn = op.div_nn.d;
            const uint32_t b = fdiv((uint32_t)row, op.div_nn), p = (uint32_t)row - b * nn;
            const uint32_t i = fdiv(p, op.div_n), k = p - i * n;
            prow = (int64_t)b * nn + (int64_t)k * n + i;
          }
          off = (uint32_t)(prow * op.ld * 4);
        }
        row_off[t] = off;
      }
    } else {
      sub = lane >> 5;                            // 2 k-rows of 512 bytes per instruction
      const int col = r0 + 4 * (lane & 31);
      col_ok = col < op.rows;
      col_off = (uint32_t)col * 4;
    }
  }

  __device__ __forceinline__ void issue(int k0, int kend, char* tile) const {
    const int w = threadIdx.x >> 6;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int j = 4 * w + t;
      uint32_t off;
      if (KC) {
        const int k = k0 + sub;
        off = (row_off[t] != kBufOOB && k < kend) ? row_off[t] + (uint32_t)k * 4 : kBufOOB;
      } else {
        const int k = k0 + 2 * j + sub;
        off = (col_ok && k < kend) ? (uint32_t)((int64_t)k * ld * 4) + col_off : kBufOOB;
      }
      buf2lds16(rsrc, off, tile + j * 1024);
    }
  }
};

// The four k values (group g of 8) this lane feeds for rows rbase + lane % 32.
template <bool KC>
__device__ __forceinline__ f32x4 tile_frag_f32(const float* T, int rbase, int g) {
  const int lane = threadIdx.x & 63, hl = lane >> 5;
  if (KC) {
    const int r = rbase + (lane & 31);
    const int slot = (2 * g + hl) ^ (r & 7);
    return *reinterpret_cast<const f32x4*>(T + r * kFK + slot * 4);
  } else {
    const int col = rbase + (lane & 31);
    f32x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = T[(8 * g + 4 * hl + e) * kFM + col];
    return v;
  }
}

template <bool A_KC, bool B_KC>
__device__ __forceinline__ void gemm_tile_f32(const GemmOperandF32& A, const GemmOperandF32& B,
                                              int m0, int n0, int kbeg, int kend, char* smem,
                                              f32x16 (&acc)[2][2]) {
  const int w = threadIdx.x >> 6;
  const int wm = w >> 1, wn = w & 1;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = zero16();
  TileLoaderF32<A_KC> la;
  TileLoaderF32<B_KC> lb;
  la.init(A, m0);
  lb.init(B, n0);
  const int nk = (kend - kbeg + kFK - 1) / kFK;
  if (nk <= 0) return;
  la.issue(kbeg, kend, smem);
  lb.issue(kbeg, kend, smem + kFTileBytes);
  for (int kt = 0; kt < nk; ++kt) {
    char* cur = smem + (kt & 1) * kFStageBytes;
    wait_vmcnt<0>();
    lds_barrier();
    if (kt + 1 < nk) {
      char* nxt = smem + ((kt + 1) & 1) * kFStageBytes;
      la.issue(kbeg + (kt + 1) * kFK, kend, nxt);
      lb.issue(kbeg + (kt + 1) * kFK, kend, nxt + kFTileBytes);
    }
    const float* As = reinterpret_cast<const float*>(cur);
    const float* Bs = reinterpret_cast<const float*>(cur + kFTileBytes);
#pragma unroll
    for (int g = 0; g < kFK / 8; ++g) {
      f32x4 af[2], bfr[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        af[t] = tile_frag_f32<A_KC>(As, 64 * wm + 32 * t, g);
        bfr[t] = tile_frag_f32<B_KC>(Bs, 64 * wn + 32 * t, g);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[i][j] = mfma32f(af[i][e], bfr[j][e], acc[i][j]);
    }
  }
  lds_barrier();
}

}  // namespace tpf
