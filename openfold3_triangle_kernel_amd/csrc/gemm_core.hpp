// MFMA GEMM main loop shared by the TriMul kernels and the generic batched
// GEMM (gfx950, 256 threads = 4 waves per workgroup).
//
//   acc(m, n) = sum_{k in [kbeg, kend)} A(m, k) * B(n, k)
//
// Tile 128 (m) x 128 (n) x 64 (k); wave w owns the 64 x 64 sub-tile
// (wm, wn) = (w >> 1, w & 1) as 2 x 2 MFMA 32x32x16 accumulators:
//   acc[i][j] register r <-> m = 64 wm + 32 i + 8 (r / 4) + 4 (lane / 32) + r % 4,
//                            n = 64 wn + 32 j + lane % 32.
//
// Operands are read from HBM straight into LDS (buffer_load ... lds, 16 bytes
// per lane, zeros outside the tensor), two k-stages in flight.  Either
// operand may be
//   KC (K-contiguous): X[row * ld + k] -- LDS tile [128 rows][64 k], the 16-
//      byte chunk c of row r stored at slot c ^ (r & 7); fragments are plain
//      16-byte LDS reads;
//   MN (MN-contiguous): X[k * ld + row] -- LDS tile [64 k][128 rows], chunk c
//      of k-row r stored at slot c ^ ((r & 3) << 1); fragments come from
//      transposing LDS reads (ds_read_b64_tr_b16), so no transposed copy of
//      the operand ever exists in memory.
// A KC operand may gather its rows: row m of batch item m / nn is read from
// physical row (m / nn) * nn + (p % n) * n + p / n, p = m % nn (the
// transposed pair order of the incoming TriMul direction).
#pragma once

#include "common.hpp"

namespace tpf {

constexpr int kGM = 128, kGN = 128, kGK = 64;
constexpr int kGTileBytes = kGM * kGK * 2;        // one operand tile, 16 KiB
constexpr int kGStageBytes = 2 * kGTileBytes;     // A + B
constexpr int kGMainLdsBytes = 2 * kGStageBytes;  // two stages, 64 KiB

struct GemmOperand {
  const __bf16* p;  // element (0, 0) of this batch item
  int64_t ld;       // leading dimension in elements
  int rows;         // extent of the m (or n) dimension
  int gather_n;     // KC row gather (0 = none); nn = gather_n^2
};

// Per-lane loader state of one operand (offsets fixed for the whole k loop).
template <bool KC>
struct TileLoader {
  i32x4 rsrc;
  uint32_t row_off[4];  // KC: byte offset of the row start (kBufOOB if absent)
  int col_ok;           // MN: column chunk inside the tensor
  uint32_t col_off;     // MN: byte offset of the column chunk
  int sub;              // KC: k chunk (elements) of this lane; MN: k-row in instr
  int64_t ld;

  __device__ __forceinline__ void init(const GemmOperand& op, int r0) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    rsrc = buffer_rsrc(op.p);
    ld = op.ld;
    if (KC) {
      const int rin = lane >> 3;                        // row inside instruction
      sub = 8 * ((lane & 7) ^ (rin & 7));               // k offset of this lane
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int row = r0 + 8 * (4 * w + t) + rin;
        uint32_t off = kBufOOB;
        if (row < op.rows) {
          int64_t prow = row;
          if (op.gather_n > 0) {
            const int64_t nn = (int64_t)op.gather_n * op.gather_n;
            const int64_t b = row / nn, p = row % nn;
            prow = b * nn + (p % op.gather_n) * op.gather_n + p / op.gather_n;
          }
          off = (uint32_t)(prow * op.ld * 2);
        }
        row_off[t] = off;
      }
    } else {
      const int kr = lane >> 4;                         // k-row inside instruction
      const int chunk = (lane & 15) ^ ((kr & 3) << 1);
      sub = kr;
      const int col = r0 + 8 * chunk;
      col_ok = col < op.rows;
      col_off = (uint32_t)col * 2;
    }
  }

  // Issue the 4 instructions of this wave for the k-tile at k0 into tile.
  __device__ __forceinline__ void issue(int k0, int kend, char* tile) const {
    const int w = threadIdx.x >> 6;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int j = 4 * w + t;
      uint32_t off;
      if (KC) {
        const int k = k0 + sub;
        off = (row_off[t] != kBufOOB && k < kend) ? row_off[t] + (uint32_t)k * 2 : kBufOOB;
      } else {
        const int k = k0 + 4 * j + sub;
        off = (col_ok && k < kend) ? (uint32_t)((int64_t)k * ld * 2) + col_off : kBufOOB;
      }
      buf2lds16(rsrc, off, tile + j * 1024);
    }
  }
};

// A fragment (rows rbase + lane % 32, k = 16 s + 8 (lane / 32) .. + 8).
template <bool KC>
__device__ __forceinline__ bf16x8 tile_frag(const __bf16* T, int rbase, int s) {
  const int lane = threadIdx.x & 63;
  if (KC) {
    const int r = rbase + (lane & 31);
    const int slot = (2 * s + (lane >> 5)) ^ (r & 7);
    return *reinterpret_cast<const bf16x8*>(T + r * kGK + slot * 8);
  } else {
    const int g = lane >> 4, ip = lane & 15;
    const int col = rbase + 16 * (g & 1) + 4 * (ip & 3);
    bf16x4 h[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int r = 16 * s + 4 * e + 8 * (g >> 1) + (ip >> 2);
      const int slot = (col >> 3) ^ ((r & 3) << 1);
      h[e] = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
          (lds_bf16x4*)(T + r * kGM + slot * 8 + (col & 7)));
    }
    return cat8(h[0], h[1]);
  }
}

// Full k loop of one 128 x 128 tile.  smem holds kGMainLdsBytes; on return
// every wave has finished reading it (callers may reuse it after a barrier).
template <bool A_KC, bool B_KC>
__device__ __forceinline__ void gemm_tile(const GemmOperand& A, const GemmOperand& B, int m0,
                                          int n0, int kbeg, int kend, char* smem,
                                          f32x16 (&acc)[2][2]) {
  const int w = threadIdx.x >> 6;
  const int wm = w >> 1, wn = w & 1;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = zero16();
  TileLoader<A_KC> la;
  TileLoader<B_KC> lb;
  la.init(A, m0);
  lb.init(B, n0);
  const int nk = (kend - kbeg + kGK - 1) / kGK;
  if (nk <= 0) return;
  la.issue(kbeg, kend, smem);
  lb.issue(kbeg, kend, smem + kGTileBytes);
  for (int kt = 0; kt < nk; ++kt) {
    char* cur = smem + (kt & 1) * kGStageBytes;
    wait_vmcnt<0>();
    lds_barrier();
    if (kt + 1 < nk) {
      char* nxt = smem + ((kt + 1) & 1) * kGStageBytes;
      la.issue(kbeg + (kt + 1) * kGK, kend, nxt);
      lb.issue(kbeg + (kt + 1) * kGK, kend, nxt + kGTileBytes);
    }
    const __bf16* As = reinterpret_cast<const __bf16*>(cur);
    const __bf16* Bs = reinterpret_cast<const __bf16*>(cur + kGTileBytes);
#pragma unroll
    for (int s = 0; s < kGK / 16; ++s) {
      bf16x8 af[2], bfr[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        af[t] = tile_frag<A_KC>(As, 64 * wm + 32 * t, s);
        bfr[t] = tile_frag<B_KC>(Bs, 64 * wn + 32 * t, s);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma32(af[i], bfr[j], acc[i][j]);
    }
  }
  lds_barrier();
}

// XCD-aware tile order: workgroup L runs on XCD L % 8; consecutive logical
// tiles T (which share operand rows) are placed on the same XCD so they hit
// the same L2.  Returns -1 for the padding ids of the rounded-up grid.
__device__ __forceinline__ int64_t xcd_order(int64_t total) {
  const int64_t L = blockIdx.x;
  const int64_t per = (total + 7) / 8;
  const int64_t T = (L % 8) * per + L / 8;
  return T < total ? T : -1;
}

}  // namespace tpf
