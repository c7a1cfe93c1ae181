// MFMA GEMM main loop shared by the TriMul kernels and the generic batched
// GEMM (gfx950, 256 threads = 4 waves per workgroup).
//
//   acc(m, n) = sum_{k in [kbeg, kend)} A(m, k) * B(n, k)
//
// Tile TM (m) x TM (n) x kGK (k), TM = 128 (default) or 192; wave w owns the
// TM/2 x TM/2 sub-tile (wm, wn) = (w >> 1, w & 1) as NB x NB (NB = TM / 64)
// MFMA 32x32x16 accumulators:
//   acc[i][j] register r <-> m = TM/2 wm + 32 i + 8 (r / 4) + 4 (lane / 32) + r % 4,
//                            n = TM/2 wn + 32 j + lane % 32.
//
// Operands are read from HBM straight into LDS (buffer_load ... lds, 16 bytes
// per lane, zeros outside the tensor) through a ring of NS stages (a
// template parameter of gemm_tile, default kGNS).  Either
// operand may be
//   KC (K-contiguous): X[row * ld + k] -- LDS tile [TM rows][kGK k], the 16-
//      byte chunk c of row r stored at slot kc_slot(r, c); fragments are plain
//      16-byte LDS reads;
//   MN (MN-contiguous): X[k * ld + row] -- LDS tile [kGK k][TM rows], chunk c
//      of k-row r stored at slot c ^ ((r & 3) << 1); fragments come from
//      transposing LDS reads (ds_read_b64_tr_b16), so no transposed copy of
//      the operand ever exists in memory.
// A KC operand may gather its rows: row m of batch item m / nn is read from
// physical row (m / nn) * nn + (p % n) * n + p / n, p = m % nn (the
// transposed pair order of the incoming TriMul direction).
#pragma once

#include "common.hpp"

namespace tpf {

#ifndef TPF_GEMM_GK
#define TPF_GEMM_GK 64
#endif
#ifndef TPF_GEMM_NS
#define TPF_GEMM_NS 2
#endif
constexpr int kGM = 128, kGN = 128;
constexpr int kGK = TPF_GEMM_GK;                  // k depth of one stage (32 or 64)
constexpr int kGNS = TPF_GEMM_NS;                 // stages in the LDS ring
static_assert(kGK == 32 || kGK == 64, "stage depth");
// One operand tile of a TM-row tile, both operands of a stage, and the 1 KiB
// loads per wave per operand tile.
template <int TM> constexpr int g_tile_bytes() { return TM * kGK * 2; }
template <int TM> constexpr int g_stage_bytes() { return 2 * g_tile_bytes<TM>(); }
template <int TM> constexpr int g_instr() { return g_tile_bytes<TM>() / 1024 / 4; }
constexpr int kGTileBytes = g_tile_bytes<kGM>();
constexpr int kGStageBytes = g_stage_bytes<kGM>();

struct GemmOperand {
  const __bf16* p;  // element (0, 0) of this batch item
  int64_t ld;       // leading dimension in elements
  int rows;         // extent of the m (or n) dimension
  int gather_n;     // KC row gather (0 = none); nn = gather_n^2
  FastDiv div_n, div_nn;  // division by gather_n and gather_n^2 (gather only)
  int kmax = 0x7fffffff;  // MN: k rows that exist (rows past it read zeros)
};

// Slot of 16-byte chunk c in row r of a KC tile.  gfx950's LDS serves 64
// banks (256 bytes) per cycle, i.e. 16 lanes of a 16-byte read: with 64-byte
// rows (kGK = 32) the 16 rows of one lane group fill all banks when the slot
// varies with r / 4 (measured: no bank-conflict cycles).  The 128-byte rows
// of kGK = 64 keep the row-parity swizzle (two-way conflicts remain; the
// loader's per-lane chunk must not change between the 8-row groups of one
// instruction, which excludes an (r / 2)-based slot).
__device__ __forceinline__ int kc_slot(int r, int c) {
  return kGK == 64 ? (c ^ (r & 7)) : (c ^ ((r >> 2) & 3));
}

// Per-lane loader state of one operand (offsets fixed for the whole k loop).
// Load j of a stage (j = g_instr * w + t) fills bytes [1024 j, 1024 j + 1024)
// of the tile, lane l the 16 bytes at chunk position p = 64 j + l.
template <bool KC, int TM = kGM>
struct TileLoader {
  static constexpr int NI = g_instr<TM>();
  i32x4 rsrc;
  uint32_t row_off[KC ? NI : 1];  // KC: byte offset of the row start (kBufOOB if absent)
  uint32_t col_off[KC ? 1 : NI];  // MN: byte offset of the column chunk (kBufOOB if absent)
  int kr[KC ? 1 : NI];            // MN: k-row of the chunk in the tile
  int kmax;                       // MN: k rows that exist
  int sub;                        // KC: k offset of this lane
  int64_t ld;

  __device__ __forceinline__ void init(const GemmOperand& op, int r0) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    rsrc = buffer_rsrc(op.p);
    ld = op.ld;
    if (KC) {
      constexpr int cpr = kGK / 8, rpi = 64 / cpr;  // chunks per row, rows per instruction
      const int rin = lane / cpr;
      sub = 8 * kc_slot(rin, lane % cpr);             // rows of one lane differ by rpi (even)
#pragma unroll
      for (int t = 0; t < NI; ++t) {
        const int row = r0 + rpi * (NI * w + t) + rin;
        uint32_t off = kBufOOB;
        if (row < op.rows) {
          int64_t prow = row;
          if (op.gather_n > 0) {
            const uint32_t n = op.gather_n, nn = op.div_nn.d;
            const uint32_t b = fdiv((uint32_t)row, op.div_nn), p = (uint32_t)row - b * nn;
            const uint32_t i = fdiv(p, op.div_n), k = p - i * n;
            prow = (int64_t)b * nn + (int64_t)k * n + i;
          }
          off = (uint32_t)(prow * op.ld * 2);
        }
        row_off[t] = off;
      }
    } else {
      // Chunk position p holds k-row p / (TM / 8), slot p % (TM / 8), i.e.
      // column chunk slot ^ ((k-row & 3) << 1) (the XOR stays inside the
      // 8-chunk group, so inside the row for TM a multiple of 64).
      constexpr int cpr = TM / 8;
#pragma unroll
      for (int t = 0; t < NI; ++t) {
        // With 64 % cpr == 0 (TM = 128) every load of a lane has the same
        // chunk, and its k-row advances by 64 / cpr per load: the loop's
        // values then differ only by constants.
        const int p = 64 * (NI * w + t) + lane;
        const int r = 64 % cpr == 0 ? (64 / cpr) * (NI * w + t) + lane / cpr : p / cpr;
        const int slot = 64 % cpr == 0 ? lane % cpr : p % cpr;
        const int chunk = slot ^ ((r & 3) << 1);
        const int col = r0 + 8 * chunk;
        kr[t] = r;
        col_off[t] = col < op.rows ? (uint32_t)col * 2 : kBufOOB;
      }
      kmax = op.kmax;
    }
  }

  // Issue this wave's instructions for the k-tile at k0 into tile.
  __device__ __forceinline__ void issue(int k0, int kend, char* tile) const {
    const int w = threadIdx.x >> 6;
#pragma unroll
    for (int t = 0; t < NI; ++t) {
      const int j = NI * w + t;
      uint32_t off;
      if (KC) {
        const int k = k0 + sub;
        off = (row_off[t] != kBufOOB && k < kend) ? row_off[t] + (uint32_t)k * 2 : kBufOOB;
      } else {
        const int k = k0 + kr[t];
        off = (col_off[t] != kBufOOB && k < kend && k < kmax)
                  ? (uint32_t)((int64_t)k * ld * 2) + col_off[t]
                  : kBufOOB;
      }
      buf2lds16(rsrc, off, tile + j * 1024);
    }
  }
};

// A fragment (rows rbase + lane % 32, k = 16 s + 8 (lane / 32) .. + 8).
template <bool KC, int TM = kGM>
__device__ __forceinline__ bf16x8 tile_frag(const __bf16* T, int rbase, int s) {
  const int lane = threadIdx.x & 63;
  if (KC) {
    const int r = rbase + (lane & 31);
    const int slot = kc_slot(r, 2 * s + (lane >> 5));
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
          (lds_bf16x4*)(T + r * TM + slot * 8 + (col & 7)));
    }
    return cat8(h[0], h[1]);
  }
}

// LDS bytes of an NS-stage ring.
constexpr int gemm_ring_bytes(int ns, int tm = kGM) { return ns * 2 * tm * kGK * 2; }

// Full k loop of one 128 x 128 tile.  smem holds gemm_ring_bytes(NS); on
// return every wave has finished reading it (callers may reuse it after a
// barrier).  NS - 1 stages are in flight while one is multiplied: deeper
// rings hide more load latency per workgroup at the cost of LDS.
template <bool A_KC, bool B_KC, int NS = kGNS, int TM = kGM>
__device__ __forceinline__ void gemm_tile(const GemmOperand& A, const GemmOperand& B, int m0,
                                          int n0, int kbeg, int kend, char* smem,
                                          f32x16 (&acc)[TM / 64][TM / 64]) {
  constexpr int NB = TM / 64, SB = g_stage_bytes<TM>(), TB = g_tile_bytes<TM>();
  const int w = threadIdx.x >> 6;
  const int wm = w >> 1, wn = w & 1;
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[i][j] = zero16();
  TileLoader<A_KC, TM> la;
  TileLoader<B_KC, TM> lb;
  la.init(A, m0);
  lb.init(B, n0);
  const int nk = (kend - kbeg + kGK - 1) / kGK;
  if (nk <= 0) return;
#pragma unroll
  for (int st = 0; st < NS - 1; ++st) {
    if (st < nk) {
      la.issue(kbeg + st * kGK, kend, smem + st * SB);
      lb.issue(kbeg + st * kGK, kend, smem + st * SB + TB);
    }
  }
  for (int kt = 0; kt < nk; ++kt) {
    char* cur = smem + (kt % NS) * SB;
    // Stage kt has landed once at most the later stages' loads are pending.
    if (kt + NS - 2 < nk) wait_vmcnt<(NS - 2) * 2 * g_instr<TM>()>();
    else wait_vmcnt<0>();
    lds_barrier();
    if (kt + NS - 1 < nk) {
      char* nxt = smem + ((kt + NS - 1) % NS) * SB;
      la.issue(kbeg + (kt + NS - 1) * kGK, kend, nxt);
      lb.issue(kbeg + (kt + NS - 1) * kGK, kend, nxt + TB);
    }
    const __bf16* As = reinterpret_cast<const __bf16*>(cur);
    const __bf16* Bs = reinterpret_cast<const __bf16*>(cur + TB);
#pragma unroll
    for (int s = 0; s < kGK / 16; ++s) {
      bf16x8 af[NB], bfr[NB];
#pragma unroll
      for (int t = 0; t < NB; ++t) {
        af[t] = tile_frag<A_KC, TM>(As, (TM / 2) * wm + 32 * t, s);
        bfr[t] = tile_frag<B_KC, TM>(Bs, (TM / 2) * wn + 32 * t, s);
      }
#pragma unroll
      for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = mfma32(af[i], bfr[j], acc[i][j]);
    }
  }
  lds_barrier();
}

// XCD-aware tile order: workgroup L runs on XCD L % 8; consecutive logical
// tiles T (which share operand rows) are placed on the same XCD so they hit
// the same L2.  Returns -1 for the padding ids of the rounded-up grid.
__device__ __forceinline__ int64_t xcd_order_of(int64_t L, int64_t total) {
  const int64_t per = (total + 7) / 8;
  const int64_t T = (L % 8) * per + L / 8;
  return T < total ? T : -1;
}

// The same order for this workgroup.
__device__ __forceinline__ int64_t xcd_order(int64_t total) { return xcd_order_of(blockIdx.x, total); }

}  // namespace tpf
