// Triangle attention with pair bias on gfx950: forward, delta, single-pass
// backward and fixed-order reducers.
//
// Math (per plane p = (b, o, h), q/k index the N sequence positions):
//   S[q,k]   = scale * <Q[q], K[k]> + mask[b,o,k] + bias[h,q,k]
//   P        = softmax_k(S),   O[q] = sum_k P[q,k] V[k]
//   LSE[q]   = log sum_k exp(S[q,k])      (-inf for a fully masked row)
//   delta[q] = <dO[q], O[q]>
//   dS       = P * (dO V^T - delta)
//   dQ = scale * dS K,  dK = scale * dS^T Q,  dV = P^T dO,
//   dBias[h,q,k] = sum over (b, o) sharing the bias of dS[q,k]
// Reference behaviour: turbopairformer_triangle_forward.cu:414-441 (online
// softmax recurrence, -inf rows -> O = 0 and LSE = -inf) and
// turbopairformer_triangle_dq_dbias.cu:1-46 (single reconstruction of P per
// tile for all four gradients, fixed non-atomic reduction orders).
//
// Layouts in HBM:
//   Q/K/V  [B, O, H, N, D] with one shared storage order: row stride s_row
//          between sequence positions and s_head between heads (head-major
//          s_row = D, s_head = N*D; sequence-major s_row = H*D, s_head = D);
//          plane stride s_plane (H*N*D for the standalone op; the pair
//          projection layout uses N * row pitch, see the tpf_attn_pair_* entry
//          points).
//   mask   [B, O, N] f32 additive.    bias [Bb, H, N, N] bf16, Bb in {1, B}.
//   out    [B, O, N, H, D] bf16.      lse / delta [B, O, H, N] f32.
// N must be a multiple of 64 (the host pads) and D a multiple of 8, D <= 64.
#include <algorithm>
#include <mutex>

#include "common.hpp"
#include "tpf_gemm.hpp"
#include "tpf_status.hpp"

namespace tpf {

struct AttnGeom {
  int B, O, H, N, D;
  int64_t s_row, s_head;   // Q/K/V element strides
  int64_t s_plane;         // elements between (b, o) planes of Q/K/V
  int64_t o_row, o_head;   // dQ/dK/dV element strides (the Q/K/V ones unless the
  int64_t o_plane;         //   pair-row core writes the gradients into its projection rows)
  int64_t bias_bstride;    // elements between bias batches (0 = broadcast)
  float scale;             // softmax scale (1/sqrt(D_true))
  int og_t;                // pair-row core: og rows in transposed pair order (O == N)
  int64_t gate_pitch;      // pair-row core: row pitch of the gate rows [B*O*N][gate_pitch]
};

// Element strides of a pair bias bias[bb, h, q, k]: the standalone op's
// contiguous [Bb, H, N, N] (s_k = 1), or the pair-bias columns of the
// projection rows (s_h = 1, s_q / s_k = N * pitch and pitch, swapped for the
// transposed bias).
struct BiasView {
  int64_t s_bb, s_h, s_q, s_k;
  int H;
};

// Output item of thread item i of a fragment-major bias pass (items per
// (batch, head) block: per_bh).  With the heads adjacent in memory (the
// projection rows' bias columns, s_h = 1) the heads are the fastest thread
// index, so the lanes of one pair row read its one sector together instead
// of H workgroups fetching it apart; a wave then still writes 256-byte runs
// of each head's block.
__device__ __forceinline__ int64_t bias_item_order(int64_t i, int64_t per_bh, const BiasView& bv) {
  if (bv.s_h != 1 || bv.H == 1) return i;
  const int64_t h = i % bv.H, r = i / bv.H;
  const int64_t bb = r / per_bh;
  return (bb * bv.H + h) * per_bh + (r - bb * per_bh);
}

__device__ __forceinline__ const __bf16* bias_at(const __bf16* bias, const BiasView& bv,
                                                 int64_t bh, int64_t q, int64_t k) {
  const int64_t bb = bh / bv.H, h = bh - bb * bv.H;
  return bias + bb * bv.s_bb + h * bv.s_h + q * bv.s_q + k * bv.s_k;
}

// XCD-aware tile order.  Workgroups are dispatched round-robin over the 8
// XCDs (linear id L goes to XCD L % 8), each with its own L2.  Logical tile
// T = (h * planes + plane) * qtiles + qtile is head-major, and XCD x takes
// the contiguous range [x * per, (x + 1) * per): every XCD then touches one
// head's bias (L2-resident) and walks neighbouring query tiles of a plane
// back to back (K/V reuse).  Returns false for the padding ids past total.
struct TileId { int qt, h, plane; };
__device__ __forceinline__ bool xcd_tile(int64_t total, int qtiles, int planes, TileId* t) {
  const int64_t L = blockIdx.x;
  const int64_t per = (total + 7) / 8;
  const int64_t T = (L % 8) * per + L / 8;
  if (T >= total) return false;
  t->qt = (int)(T % qtiles);
  const int64_t r = T / qtiles;
  t->plane = (int)(r % planes);
  t->h = (int)(r / planes);
  return true;
}

// ---------------------------------------------------------------------------
// Bias pre-pass: bias_s = f32(bias) / scale, so that
//   scale * <Q, K> + bias = scale * (<Q, K> + bias_s)
// and the bias seeds the S^T accumulator; the softmax then needs one FMA per
// score.  bias_s is stored fragment-major: for every 32-query x 32-key block
// (qb, kb) of head h, 1024 floats laid out as [j][lane][i] where lane
// (ql + 32*hl) register 4*j + i of the S^T = K Q^T accumulator holds
// (query 32*qb + ql, key 32*kb + 8*j + 4*hl + i).  Each 16-byte load
// instruction of a wave then reads one contiguous kilobyte.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void attn_bias_prescale_kernel(const __bf16* __restrict__ bias,
                                                                 float* __restrict__ out,
                                                                 int64_t items, int N,
                                                                 float inv_scale, BiasView bv) {
  const int64_t it = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (it >= items) return;
  const int64_t i = bias_item_order(it, (int64_t)(N / 32) * (N / 32) * 256, bv);  // (block, j, lane)
  const int lane = (int)(i & 63), j = (int)((i >> 6) & 3);
  const int64_t blk = i >> 8;
  const int nkb = N / 32;
  const int kb = (int)(blk % nkb);
  const int64_t hq = blk / nkb;            // (bb * H + h) * (N / 32) + qb
  const int qb = (int)(hq % (N / 32));
  const int64_t bh = hq / (N / 32);
  const int ql = lane & 31, hl = lane >> 5;
  const __bf16* src = bias_at(bias, bv, bh, qb * 32 + ql, kb * 32 + 8 * j + 4 * hl);
  f32x4 o;
  if (bv.s_k == 1) {
    const bf16x4 v = ld4(src);
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = bf2f(v[e]) * inv_scale;
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = bf2f(src[e * bv.s_k]) * inv_scale;
  }
  *reinterpret_cast<f32x4*>(out + i * 4) = o;
}

// Longest mask row the forward stages in LDS (up to 2 rows, 64 KiB of dynamic LDS).
constexpr int kFwdMaskLdsMaxN = 8192;

// ---------------------------------------------------------------------------
// Forward.  One workgroup = NW waves = 32*NW queries of one plane (NW = 4:
// 2, 3 and 6 measured slower at N = 384); each wave owns 32 queries and
// walks all keys in 64-key tiles that the workgroup stages in LDS.
// Scores are produced transposed (S^T = K Q^T) so each lane owns one query
// column: row max / sum need only the lane^32 exchange, and the C-layout P^T
// block is fed directly as the B operand of O^T += V^T P^T.
//
// Memory pipeline.  K and V tiles are staged row-major in LDS (16-byte
// chunks XOR-swizzled per row) and double-buffered; each wave fetches its
// share of tile t+1 into registers (buffer loads) between the two 32-key
// blocks of tile t and writes it to the other LDS buffer at the end of tile
// t, so the loads have one block of compute to arrive.  V^T operands come
// from the row-major V tile through transposing LDS reads.  The prescaled
// bias of a 32-key block (fragment-major, one 4 KiB read per wave) seeds
// the S^T accumulator; the next block's bias is loaded into the same
// registers as soon as the current block's S MFMAs have consumed them.  Every load is issued unconditionally (past the last
// tile or block it reloads the last one, whose copy is never consumed; lane
// chunks past D read zeros through the buffer range check) and is visible
// to the compiler's wait counting, and loads are issued in the
// order they are consumed, so waiting for block b's bias never waits for a
// K / V tile issued after it.
//
// Softmax works on 32-key blocks.  Scores stay in raw units
// r = <Q,K> + bias_s (+ mask / scale), and p = exp2(r * c2 - m * c2) with
// c2 = scale * log2(e): one FMA + one exp per score.  Row sums use packed
// bf16 dot products of the rounded P (the values that also enter P V).  The
// running max is raised only when a block exceeds it by more than 8 in log2
// units (p <= 256 otherwise), so the O rescale is rare.
// ---------------------------------------------------------------------------
// Swizzle of the 16-byte chunks of K / V tile rows: a 16-byte row read by 8
// consecutive rows (8 lanes = 128 bytes) and an 8-byte transposing read of 4
// consecutive rows x 2 chunks (16 lanes = 128 bytes) each cover all 32
// banks once.  DP = 32 (64-byte rows): rows 0..7 -> 0, 0, 2, 2, 1, 1, 3, 3;
// DP = 64 (128-byte rows): 0, 2, 4, 6, 1, 3, 5, 7.
template <int DP>
__device__ __forceinline__ int kv_swz(int r) {
  return (DP == 32) ? ((((r >> 1) & 1) << 1) | ((r >> 2) & 1)) : (((r & 3) << 1) | ((r >> 2) & 1));
}
template <int DP>
__device__ __forceinline__ int kv_off(int r, int col) {  // element offset of (row, col)
  return r * DP + (((col >> 3) ^ kv_swz<DP>(r)) << 3) + (col & 7);
}

// tr_col4 (common.hpp) on a swizzled K / V tile: lane l receives
// { M[r0 + e][c0 + l % 32] : e = 0..3 }, r0 = rbase_lo (l < 32) or rbase_hi.
template <int DP>
__device__ __forceinline__ bf16x4 kv_tr_col4(const __bf16* M, int rbase_lo, int rbase_hi, int c0) {
  const int l = threadIdx.x & 63, gq = l >> 4, ip = l & 15;
  const int r = ((gq >> 1) ? rbase_hi : rbase_lo) + (ip >> 2);
  const __bf16* p = M + kv_off<DP>(r, c0 + 16 * (gq & 1) + 4 * (ip & 3));
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p);
}

template <int DP, int NW, int PL>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(3, 8))) void attn_fwd_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k,
    const __bf16* __restrict__ v, const float* __restrict__ mask,
    const float* __restrict__ bias_s, __bf16* __restrict__ out,
    float* __restrict__ lse, __bf16* __restrict__ res, const __bf16* __restrict__ gate,
    __bf16* __restrict__ og, AttnGeom g) {
  constexpr int TE = 64 * DP;                  // elements of one K (or V) tile
  constexpr int REG = TE / 8;                  // 16-byte chunks of one K (or V) tile
  constexpr int CPT = 2 * PL * REG / (64 * NW);  // chunks per thread per tile
  static_assert(REG % (64 * NW) == 0, "a thread's chunks split evenly over K / V tiles");
  constexpr int QT = 32 * NW;                  // queries per workgroup
  // [buffer][plane][K, V] tiles.
  __shared__ __attribute__((aligned(16))) __bf16 KVs[2][PL][2][TE];
  // The planes' mask rows divided by the scale (dynamic LDS of PL * N floats).
  extern __shared__ __attribute__((aligned(16))) float Ms[];

  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int ql = lane & 31, hl = lane >> 5;
  const int N = g.N, D = g.D;
  // Groups of PL consecutive outer rows of one batch (the last group of a
  // batch may hold fewer: its missing planes recompute the first one and
  // store nothing).
  const int groups = (g.O + PL - 1) / PL;
  TileId tile;
  const int qtiles = (N + QT - 1) / QT;
  if (!xcd_tile((int64_t)qtiles * g.H * g.B * groups, qtiles, g.B * groups, &tile)) return;
  const int h = tile.h;
  const int b = tile.plane / groups;
  const int o0 = (tile.plane - b * groups) * PL;
  const int q0 = tile.qt * QT + w * 32;
  const bool active = q0 < N;
  const int qi = q0 + ql;
  int plane[PL];
  bool pvalid[PL];
#pragma unroll
  for (int p = 0; p < PL; ++p) {
    pvalid[p] = o0 + p < g.O;
    plane[p] = b * g.O + (pvalid[p] ? o0 + p : o0);
  }

  const float c2 = g.scale * kLog2e;
  const float inv_scale = 1.f / g.scale;
  const float thr = 8.f / c2;  // lazy-rescale threshold in raw units
  const int ntiles = N / 64, nblk = N / 32;

  // Q rows of this wave for every plane (B operand of S^T = K Q^T), zeros
  // past D.
  bf16x8 qreg[PL][DP / 16];
#pragma unroll
  for (int p = 0; p < PL; ++p) {
    const __amdgpu_buffer_rsrc_t rq = raw_rsrc(q + (int64_t)plane[p] * g.s_plane + (int64_t)h * g.s_head);
#pragma unroll
    for (int s2 = 0; s2 < DP / 16; ++s2) {
      const int d0 = 16 * s2 + 8 * hl;
      qreg[p][s2] = buf_ld8(rq, (active && d0 < D) ? (uint32_t)(((int64_t)qi * g.s_row + d0) * 2) : kBufOOB);
    }
  }

  // K / V chunks of a thread: chunk n = tid + 64 NW i of the tile group,
  // region n / REG = (plane, K or V); LDS chunk position -> (row, physical
  // chunk), reading the logical chunk the swizzle stores there.  Per-lane
  // byte offsets are fixed; a tile adds 64 rows.
  __amdgpu_buffer_rsrc_t rkv[2 * PL];
#pragma unroll
  for (int p = 0; p < PL; ++p) {
    const int64_t off = (int64_t)plane[p] * g.s_plane + (int64_t)h * g.s_head;
    rkv[2 * p] = raw_rsrc(k + off);
    rkv[2 * p + 1] = raw_rsrc(v + off);
  }
  uint32_t vkv[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int e = ((tid + 64 * NW * i) % REG) * 8;  // element offset within its tile
    const int r = e / DP, c = ((e % DP) / 8) ^ kv_swz<DP>(r);
    vkv[i] = c * 8 < D ? (uint32_t)(((int64_t)r * g.s_row + c * 8) * 2) : kBufOOB;
  }
  const uint32_t tile_bytes = (uint32_t)(64 * g.s_row * 2);
  auto load_kv = [&](int t, bf16x8* dst) {
    // Tiles past the last one reload the last one (never consumed); the
    // tile offset is a scalar, the lane offsets fixed.
    const uint32_t so = (uint32_t)min(t, ntiles - 1) * tile_bytes;
#pragma unroll
    for (int i = 0; i < CPT; ++i)
      dst[i] = __builtin_bit_cast(
          bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rkv[64 * NW * i / REG], vkv[i], so, 0));
  };
  auto store_kv = [&](int buf, const bf16x8* src) {
#pragma unroll
    for (int i = 0; i < CPT; ++i)
      *reinterpret_cast<bf16x8*>(&KVs[buf][0][0][0] + (tid + 64 * NW * i) * 8) = src[i];
  };

  // Fragment-major bias blocks of this wave's 32 queries: 1024 floats per
  // 32-key block, lane-interleaved (see attn_bias_prescale_kernel); shared by
  // the PL planes.
  const __amdgpu_buffer_rsrc_t rs_b = raw_rsrc(
      bias_s + (int64_t)b * g.bias_bstride +
      ((int64_t)h * (N / 32) + (active ? q0 / 32 : 0)) * (int64_t)(N / 32) * 1024);
  const uint32_t vb_lane = (uint32_t)lane * 16;
  auto load_bias = [&](int blk) {
    // Blocks past the last one reload the last one (never consumed).
    const uint32_t so = (uint32_t)min(blk, nblk - 1) * 4096;
    f32x16 r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 x = __builtin_bit_cast(
          f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_b, vb_lane + j * 1024, so, 0));
#pragma unroll
      for (int i = 0; i < 4; ++i) r[4 * j + i] = x[i];
    }
    return r;
  };

  // Pipeline fill issued first: K / V of tile 0 and the bias of block 0 are
  // in flight while the mask rows are staged (−0.7 us at N = 384).
  bf16x8 kvr[CPT];
  load_kv(0, kvr);
  f32x16 bset = load_bias(0);
  // Tiles whose 64 mask entries are all zero in every plane skip the mask
  // add (uniform flags); computed up front so no wait on the mask sits
  // inside the pipelined loop.  Each wave ballots the 64-key tiles it
  // stages (its 64 lanes take one tile per pass; N % 64 == 0), so the flags
  // cost no round trips to memory beyond the staging loads (one ballot
  // load per tile and plane measured 3 us slower at N = 384); the waves'
  // words meet after the first barrier of the tile loop.
  __shared__ uint64_t Mw[NW];
  uint64_t wbits = 0ull;
#pragma unroll
  for (int p = 0; p < PL; ++p) {
    const float* mrow = mask + (int64_t)plane[p] * N;
    for (int i = tid; i < N; i += 64 * NW) {
      const float mv = mrow[i];
      Ms[p * N + i] = mv * inv_scale;
      if (__any(mv != 0.f)) wbits |= 1ull << ((i >> 6) & 63);
    }
  }
  if (lane == 0) Mw[w] = ntiles <= 64 ? wbits : ~0ull;
  uint64_t mbits = ~0ull;
  bool mbits_ready = false;

  store_kv(0, kvr);

  f32x16 acc[PL][DP / 32];
  float m[PL], l[PL], nm[PL];
#pragma unroll
  for (int p = 0; p < PL; ++p) {
#pragma unroll
    for (int i = 0; i < DP / 32; ++i) acc[p][i] = zero16();
    m[p] = -INFINITY;
    l[p] = 0.f;
    nm[p] = 0.f;
  }
  const bf16x2 ones = {static_cast<__bf16>(1.f), static_cast<__bf16>(1.f)};

  // One 32-key block for every plane: S^T seeded with the shared bias (whose
  // registers then take block blk + 1's bias), mask, online softmax (one
  // rescale branch for all planes), O^T += V^T P^T.  The planes' chains are
  // independent, so their MFMA and VALU work interleave.
  auto block = [&](int buf, int sb, int blk, bool masked, int kt) {
    // Every K fragment of the block is read before the first MFMA, so the
    // LDS latency is paid once.
    bf16x8 ka[PL][DP / 16];
#pragma unroll
    for (int p = 0; p < PL; ++p)
#pragma unroll
      for (int ks = 0; ks < DP / 16; ++ks)
        ka[p][ks] = *reinterpret_cast<const bf16x8*>(
            &KVs[buf][p][0][kv_off<DP>(sb * 32 + ql, 16 * ks + 8 * hl)]);
    f32x16 s[PL];
#pragma unroll
    for (int p = 0; p < PL; ++p) {
      s[p] = mfma32(ka[p][0], qreg[p][0], bset);
#pragma unroll
      for (int ks = 1; ks < DP / 16; ++ks) s[p] = mfma32(ka[p][ks], qreg[p][ks], s[p]);
    }
    bset = load_bias(blk + 1);
    if (masked) {
#pragma unroll
      for (int p = 0; p < PL; ++p)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const f32x4 mv = *reinterpret_cast<const f32x4*>(&Ms[p * N + kt + sb * 32 + 8 * j + 4 * hl]);
#pragma unroll
          for (int i = 0; i < 4; ++i) s[p][4 * j + i] += mv[i];
        }
    }
    float mx[PL];
    bool up = false;
#pragma unroll
    for (int p = 0; p < PL; ++p) {
      float x = fmaxf(s[p][0], s[p][1]);
#pragma unroll
      for (int r = 2; r < 16; ++r) x = fmaxf(x, s[p][r]);
      mx[p] = xor32_max(x);
      up = up || (mx[p] > m[p] + thr);
    }
    if (__any(up)) {
#pragma unroll
      for (int p = 0; p < PL; ++p) {
        const float m_new = fmaxf(m[p], mx[p]);
        const float alpha = (m_new == -INFINITY) ? 1.f : fast_exp2((m[p] - m_new) * c2);
        l[p] *= alpha;
#pragma unroll
        for (int db = 0; db < DP / 32; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[p][db][r] *= alpha;
        m[p] = m_new;
        nm[p] = (m_new == -INFINITY) ? 0.f : -m_new * c2;
      }
    }
#pragma unroll
    for (int p = 0; p < PL; ++p) {
      const __bf16* Vt = &KVs[buf][p][1][0];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        // P in packed bf16 pairs (one v_cvt_pk each), summed by v_dot2 and
        // reassembled into the B operand without permutes.
        uint32_t pw[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          f32x2 f;
          f[0] = fast_exp2(fmaf(s[p][8 * t + 2 * e], c2, nm[p]));
          f[1] = fast_exp2(fmaf(s[p][8 * t + 2 * e + 1], c2, nm[p]));
          const bf16x2 pr = __builtin_convertvector(f, bf16x2);
          l[p] = __builtin_amdgcn_fdot2_f32_bf16(pr, ones, l[p], false);
          pw[e] = __builtin_bit_cast(uint32_t, pr);
        }
        u32x4 pwv = {pw[0], pw[1], pw[2], pw[3]};
        const bf16x8 pb = __builtin_bit_cast(bf16x8, pwv);
        // V^T operand: keys {16t + 4hl .. +3, 16t + 8 + 4hl .. +3} of the
        // block (the key order of the P^T registers), channel 32 db + ql.
        const int k0 = sb * 32 + 16 * t;
#pragma unroll
        for (int db = 0; db < DP / 32; ++db) {
          const bf16x8 va = cat8(kv_tr_col4<DP>(Vt, k0, k0 + 4, 32 * db),
                                 kv_tr_col4<DP>(Vt, k0 + 8, k0 + 12, 32 * db));
          acc[p][db] = mfma32(va, pb, acc[p][db]);
        }
      }
    }
  };

  // Tile t: in LDS buffer t % 2 (written before the barrier); tile t+1 is
  // loaded into registers during the tile's first block and written to the
  // other buffer at its end.  Waves past N (the last query tile when
  // N % (32 NW) != 0) compute on zero Q rows and store nothing: no branch
  // splits the loads' register state.
#pragma unroll 1
  for (int t = 0; t < ntiles; ++t) {
    __syncthreads();
    if (!mbits_ready) {  // after the loop's first barrier: every wave's word is in
      mbits = 0ull;
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) mbits |= Mw[ww];
      mbits_ready = true;
    }
    const bool masked = (mbits >> (t & 63)) & 1ull;
    block(t & 1, 0, 2 * t, masked, t * 64);
    load_kv(t + 1, kvr);
    block(t & 1, 1, 2 * t + 1, masked, t * 64);
    // Buffer (t+1) % 2 was last read in tile t-1, before the barrier above.
    store_kv((t + 1) & 1, kvr);
  }
  if (!active) return;

#pragma unroll
  for (int p = 0; p < PL; ++p) {
    if (!pvalid[p]) continue;
    const float l_tot = xor32_sum(l[p]);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    const int64_t orow_off = (((int64_t)plane[p] * N + qi) * g.H + h) * D;
    __bf16* orow = out + orow_off;
    // A lane holds channels 8j + 4hl .. +3 (j = 0..3) of its query; one
    // exchange with lane l ^ 32 per register pair (j, j + 1) gives it 8
    // consecutive channels, 16p + 8hl .. +7, stored as one 16-byte chunk
    // (out, residual and gated output: 8-byte stores measured 85 against
    // 77 us at N = 384).
    int64_t og_off = orow_off;
    if (gate && g.og_t) {
      const int64_t ob = plane[p] % g.O;
      og_off = ((((int64_t)plane[p] - ob) * N + (int64_t)qi * N + ob) * g.H + h) * D;
    }
#pragma unroll
    for (int db = 0; db < DP / 32; ++db) {
      uint32_t po[4][2], pr[4][2];  // [j][pair] packed bf16 of out and residual
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const float a0 = acc[p][db][4 * j + 2 * e], a1 = acc[p][db][4 * j + 2 * e + 1];
          const bf16x2 o2 = {f2bf(a0 * inv), f2bf(a1 * inv)};
          // Shadow residual: the part of the f32 output the bf16 store drops.
          const bf16x2 r2 = {f2bf(fmaf(a0, inv, -bf2f(o2[0]))), f2bf(fmaf(a1, inv, -bf2f(o2[1])))};
          po[j][e] = __builtin_bit_cast(uint32_t, o2);
          pr[j][e] = __builtin_bit_cast(uint32_t, r2);
        }
#pragma unroll
      for (int pp = 0; pp < 2; ++pp) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          auto ro = __builtin_amdgcn_permlane32_swap(po[2 * pp][e], po[2 * pp + 1][e], false, false);
          po[2 * pp][e] = ro[0];
          po[2 * pp + 1][e] = ro[1];
          auto rr = __builtin_amdgcn_permlane32_swap(pr[2 * pp][e], pr[2 * pp + 1][e], false, false);
          pr[2 * pp][e] = rr[0];
          pr[2 * pp + 1][e] = rr[1];
        }
        const int d0 = db * 32 + 16 * pp + 8 * hl;
        if (d0 < D) {
          const u32x4 ov = {po[2 * pp][0], po[2 * pp][1], po[2 * pp + 1][0], po[2 * pp + 1][1]};
          *reinterpret_cast<u32x4*>(orow + d0) = ov;
          if (res) {
            const u32x4 rv = {pr[2 * pp][0], pr[2 * pp][1], pr[2 * pp + 1][0], pr[2 * pp + 1][1]};
            *reinterpret_cast<u32x4*>(res + orow_off + d0) = rv;
          }
          if (gate) {
            // Output gate of the pair-row module: og = o * sigmoid(g), with g
            // in Q's storage order (the gate columns of the projection rows).
            const bf16x8 g8 = ld8(gate + ((int64_t)plane[p] * N + qi) * g.gate_pitch + h * D + d0);
            const bf16x8 o8 = __builtin_bit_cast(bf16x8, ov);
            bf16x8 og8;
#pragma unroll
            for (int i = 0; i < 8; ++i) og8[i] = f2bf(bf2f(o8[i]) * sigmoidf(bf2f(g8[i])));
            // og_t: the row of pair (o, qi) is stored at (b, qi, o) (O == N).
            st8(og + og_off + d0, og8);
          }
        }
      }
    }
    if (hl == 0) {
      lse[((int64_t)plane[p] * g.H + h) * N + qi] =
          l_tot > 0.f ? (m[p] * c2 + log2f(l_tot)) * kLn2 : -INFINITY;
    }
  }
}

// ---------------------------------------------------------------------------
// delta[b,o,h,q] = sum_d f32(dO) * f32(O), both [B,O,N,H,D] contiguous; with
// SHADOW, sum_d f32(dO) * (f32(O) + f32(res)) where res is the forward's bf16
// rounding residual of O (reference: turbopairformer_triangle_delta.cu:343-416).
// One thread per (row, 8-channel chunk), rows r = (plane, q, h): consecutive
// lanes read consecutive 16 bytes.  A row's D/8 chunk products meet in LDS
// (workgroup w takes items [w * per, (w + 1) * per), per a multiple of D/8)
// and are added in chunk order.
// ---------------------------------------------------------------------------
// Row sums of one workgroup's items: returns the delta index [plane][h][q]
// of the row the calling thread finalises, with its sum in *sum (-1 for
// every other thread).
template <bool SHADOW>
__device__ __forceinline__ int64_t delta_row(const __bf16* __restrict__ dout,
                                             const __bf16* __restrict__ out,
                                             const __bf16* __restrict__ res, int64_t items,
                                             int per, int H, int N, int D, float* sum) {
  __shared__ float part[256];
  const int tid = threadIdx.x;
  const int64_t t = (int64_t)blockIdx.x * per + tid;
  const bool act = tid < per && t < items;
  float s = 0.f;
  if (act) {
    const bf16x8 x = ld8(dout + t * 8), y = ld8(out + t * 8);
    if (SHADOW) {
      // O_f32 ~ O_bf16 + residual, summed in f32 before the product.
      const bf16x8 r = ld8(res + t * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) s = fmaf(bf2f(x[e]), bf2f(y[e]) + bf2f(r[e]), s);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) s = fmaf(bf2f(x[e]), bf2f(y[e]), s);
    }
  }
  part[tid] = s;
  __syncthreads();
  const int d8 = D / 8;
  if (!act || (t % d8) != 0) return -1;
  float acc = 0.f;
  for (int u = 0; u < d8; ++u) acc += part[tid + u];
  *sum = acc;
  // r enumerates [plane][q][h]; delta is [plane][h][q].
  const int64_t r = t / d8;
  const int hh = (int)(r % H);
  const int64_t pq = r / H;
  const int qq = (int)(pq % N);
  const int64_t plane = pq / N;
  return (plane * H + hh) * N + qq;
}

template <bool SHADOW>
__global__ __launch_bounds__(256) void attn_delta_kernel(
    const __bf16* __restrict__ dout, const __bf16* __restrict__ out,
    const __bf16* __restrict__ res, float* __restrict__ delta, int64_t items, int per, int H,
    int N, int D) {
  float sum;
  const int64_t idx = delta_row<SHADOW>(dout, out, res, items, per, H, N, D, &sum);
  if (idx >= 0) delta[idx] = sum;
}

// ---------------------------------------------------------------------------
// Backward preparation.
//   rowprep: nl2 = -lse * log2(e) (-inf for fully masked rows, whose P is 0)
//            and nd = -delta, so that in the reconstruction kernel
//              P = exp2(S_raw * c2 + nl2),  dP - delta = MFMA(dO, V^T; C = nd).
//   bias_bwd: bias / scale in the fragment-major layout of the S = Q K^T
//            accumulator: for every 32-key x 32-query block (kb, qb) of head
//            h, [j][lane][i] holds (query 32*qb + 8*j + 4*hl + i,
//            key 32*kb + (lane % 32)), hl = lane / 32.
// ---------------------------------------------------------------------------
// One launch for both: workgroups [0, row_blocks) take rowprep items, the
// rest take bias items (256 items per workgroup each).
// One bias item: 4 values of the fragment-major prescaled bias (item i =
// (fragment block, j, lane)).
__device__ __forceinline__ void bwd_bias_item(const __bf16* __restrict__ bias,
                                              float* __restrict__ out, int64_t it, int N,
                                              float inv_scale, const BiasView& bv) {
  const int64_t i = bias_item_order(it, (int64_t)(N / 32) * (N / 32) * 256, bv);
  const int lane = (int)(i & 63), j = (int)((i >> 6) & 3);
  const int64_t blk = i >> 8;
  const int nb = N / 32;
  const int qb = (int)(blk % nb);
  const int64_t bk = blk / nb;             // (bh) * nb + kb
  const int kb = (int)(bk % nb);
  const int64_t bh = bk / nb;
  const int kl = lane & 31, hl = lane >> 5;
  const __bf16* src = bias_at(bias, bv, bh, qb * 32 + 8 * j + 4 * hl, kb * 32 + kl);
  f32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = bf2f(src[(int64_t)e * bv.s_q]) * inv_scale;
  *reinterpret_cast<f32x4*>(out + i * 4) = o;
}

__device__ __forceinline__ float neg_lse_log2(float l) {
  return (l == -INFINITY) ? -INFINITY : -l * kLog2e;
}

// One launch for both: workgroups [0, row_blocks) take rowprep items, the
// rest take bias items (256 items per workgroup each).
__global__ __launch_bounds__(256) void attn_bwd_prep_kernel(const float* __restrict__ lse,
                                                            const float* __restrict__ delta,
                                                            float* __restrict__ nl2,
                                                            float* __restrict__ nd, int64_t rows,
                                                            int64_t row_blocks,
                                                            const __bf16* __restrict__ bias,
                                                            float* __restrict__ out, int64_t items,
                                                            int N, float inv_scale, BiasView bv) {
  if ((int64_t)blockIdx.x < row_blocks) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows) return;
    nl2[i] = neg_lse_log2(lse[i]);
    nd[i] = -delta[i];
    return;
  }
  const int64_t i = ((int64_t)blockIdx.x - row_blocks) * 256 + threadIdx.x;
  if (i < items) bwd_bias_item(bias, out, i, N, inv_scale, bv);
}

// Delta and the backward preparation in one launch (the fused backward
// entry point): workgroups [0, delta_blocks) compute delta rows as
// attn_delta_kernel does and write nd = -delta and nl2 = -lse * log2(e) for
// them; the rest take bias items.
template <bool SHADOW>
__global__ __launch_bounds__(256) void attn_bwd_rows_kernel(
    const __bf16* __restrict__ dout, const __bf16* __restrict__ out,
    const __bf16* __restrict__ res, const float* __restrict__ lse, float* __restrict__ nl2,
    float* __restrict__ nd, int64_t items, int per, int H, int N, int D, int64_t delta_blocks,
    const __bf16* __restrict__ bias, float* __restrict__ bias_out, int64_t bias_items,
    float inv_scale, BiasView bv) {
  if ((int64_t)blockIdx.x >= delta_blocks) {
    const int64_t i = ((int64_t)blockIdx.x - delta_blocks) * 256 + threadIdx.x;
    if (i < bias_items) bwd_bias_item(bias, bias_out, i, N, inv_scale, bv);
    return;
  }
  float sum;
  const int64_t idx = delta_row<SHADOW>(dout, out, res, items, per, H, N, D, &sum);
  if (idx >= 0) {
    nd[idx] = -sum;
    nl2[idx] = neg_lse_log2(lse[idx]);
  }
}

// ---------------------------------------------------------------------------
// Backward.  One workgroup = (key block of 64*KH keys, head, group of 4 outer
// rows), KH = 2 for D <= 32 (8 waves) and 1 for D = 64 (4 waves, LDS-bound);
// wave w owns outer row o = 4*group + (w % 4) and key half w / 4 and keeps its
// dK / dV accumulators for those 64 keys in registers while streaming all
// queries in 32-row steps.  Scores are
// formed as S = Q K^T (lane = key column) so the C-layout P and dS tiles are
// the B operands of dV^T += dO^T P and dK^T += Q^T dS without data movement;
// the transposed A operands (dO^T, Q^T) and dS^T for dQ^T = K^T dS^T come
// from row-major LDS tiles through transposing reads.  The S accumulator is
// seeded with the prescaled bias and the dP accumulator with -delta, so
//   P = exp2(S * c2 + nl2),  dS = P * dP            (one FMA, one mul).
// Inputs of step i+1 (the bias fragments shared by the 4 waves, each wave's
// Q / dO rows and row statistics) stream into the other half of a double
// buffer with direct global->LDS loads while step i computes.
// The two key halves of an outer row add their f32 dQ tiles through LDS
// (half 0 + half 1), and dQ leaves as one bf16 partial per key block; dBias
// sums the 4 outer rows' bf16 dS^T tiles in LDS (fixed order) into an f32
// partial per outer group (one bf16 rounding fewer than a bf16 partial: the
// reference's error envelope on dBias needs it).  Fixed-order reducers finish both.  Tiles are
// ordered XCD-aware by (head, outer group, key block).
// ---------------------------------------------------------------------------
constexpr int kBwdGroup = 4;
// What one backward launch produces: every gradient (the single-
// reconstruction route), or one half of the split route of direct callers:
// dK / dV (optionally with the per-64-key-block partials of
// delta_true = sum_k P dP), or the dQ / dBias partials.
constexpr int kBwdSR = 0, kBwdDKDV = 1, kBwdDQDB = 2;
// A slab of the backward: the flattened runs [brun0, brun0 + nbrun) of
// outer groups (run index b * runs + r) and the planes they cover, whose dQ
// partials [key block][planes][H][N][D] sit in the workspace at once.
struct BwdSlab {
  int brun0, nbrun;
  int64_t plane0, planes;
};
// Key halves per backward workgroup (keys per workgroup = 64 * KH).
__host__ __device__ constexpr int bwd_kh(int dp) { return dp == 32 ? 2 : 1; }
// Backward key blocks (= dQ partials) for head dimension D.
static inline int64_t bwd_key_blocks(int64_t N, int64_t D) {
  const int64_t kw = 64 * bwd_kh(D <= 32 ? 32 : 64);
  return (N + kw - 1) / kw;
}

// Q / dO tile of 32 rows x DP bf16 stored unpadded, 16-byte chunks permuted
// per row (phys = c ^ swz(r)) so transposing reads of 4 consecutive rows and
// row reads of 8 consecutive rows avoid bank conflicts.
template <int DP>
__device__ __forceinline__ int qd_swz(int r) {
  return (DP == 32) ? (((r >> 1) & 1) << 1) : ((r & 3) << 1);
}
template <int DP>
__device__ __forceinline__ int qd_off(int r, int col) {  // element offset of (row, col)
  return r * DP + (((col >> 3) ^ qd_swz<DP>(r)) << 3) + (col & 7);
}
// tr_col4 on a swizzled Q / dO tile (see tr_col4 in common.hpp).
template <int DP>
__device__ __forceinline__ bf16x4 qd_tr_col4(const __bf16* M, int rbase_lo, int rbase_hi, int c0) {
  const int l = threadIdx.x & 63, gq = l >> 4, ip = l & 15;
  const int r = ((gq >> 1) ? rbase_hi : rbase_lo) + (ip >> 2);
  const __bf16* p = M + qd_off<DP>(r, c0 + 16 * (gq & 1) + 4 * (ip & 3));
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p);
}

// Batched LDS reads for the register-starved backward loop: the reads of a
// group go out back to back and are waited for once (the compiler, at full
// register pressure, reuses one destination pair and waits after each read).
// Outputs are early-clobber so no read overwrites a later read's address.
typedef uint32_t u32x16 __attribute__((ext_vector_type(16)));
// 16 dwords at a + 256 r (r = 0..15): one lane's column of a [16][64] f32 tile.
__device__ __forceinline__ u32x16 lds_read_col16(unsigned a) {
  u32x2 v0, v1, v2, v3, v4, v5, v6, v7;
  asm volatile(
      "ds_read2st64_b32 %0, %8 offset1:1\n\t"
      "ds_read2st64_b32 %1, %8 offset0:2 offset1:3\n\t"
      "ds_read2st64_b32 %2, %8 offset0:4 offset1:5\n\t"
      "ds_read2st64_b32 %3, %8 offset0:6 offset1:7\n\t"
      "ds_read2st64_b32 %4, %8 offset0:8 offset1:9\n\t"
      "ds_read2st64_b32 %5, %8 offset0:10 offset1:11\n\t"
      "ds_read2st64_b32 %6, %8 offset0:12 offset1:13\n\t"
      "ds_read2st64_b32 %7, %8 offset0:14 offset1:15\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(v0), "=&v"(v1), "=&v"(v2), "=&v"(v3), "=&v"(v4), "=&v"(v5), "=&v"(v6), "=&v"(v7)
      : "v"(a)
      : "memory");
  const u32x2 vs[8] = {v0, v1, v2, v3, v4, v5, v6, v7};
  u32x16 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) { r[2 * i] = vs[i][0]; r[2 * i + 1] = vs[i][1]; }
  return r;
}
// 16 bytes (as two 8-byte halves) at each of four 8-byte aligned addresses.
typedef uint32_t u32x4v __attribute__((__vector_size__(16)));
__device__ __forceinline__ void lds_read_rows4(u32x4* out, unsigned a0, unsigned a1, unsigned a2,
                                               unsigned a3) {
  u32x4v r0, r1, r2, r3;
  asm volatile(
      "ds_read2_b64 %0, %4 offset1:1\n\t"
      "ds_read2_b64 %1, %5 offset1:1\n\t"
      "ds_read2_b64 %2, %6 offset1:1\n\t"
      "ds_read2_b64 %3, %7 offset1:1\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3)
      : "v"(a0), "v"(a1), "v"(a2), "v"(a3)
      : "memory");
  const u32x4v rs[4] = {r0, r1, r2, r3};
#pragma unroll
  for (int i = 0; i < 4; ++i) out[i] = u32x4{rs[i][0], rs[i][1], rs[i][2], rs[i][3]};
}

template <int DP, int MODE>
__global__ __launch_bounds__(256 * bwd_kh(DP), 1) void attn_bwd_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k,
    const __bf16* __restrict__ v, const __bf16* __restrict__ dout,
    const float* __restrict__ nl2_g, const float* __restrict__ nd_g,
    const float* __restrict__ mask, const float* __restrict__ bias_f,
    __bf16* __restrict__ dk, __bf16* __restrict__ dv,
    __bf16* __restrict__ dq_part, float* __restrict__ dbias_part, AttnGeom g, int run,
    BwdSlab sl, float* __restrict__ dtrue_part) {
  constexpr int KT = DP + 16;  // K tile pitch at setup (bf16)
  constexpr int SP = 32 + 4;   // dS^T tile [64 keys][32 queries] pitch (bf16): the
                               // 8-byte row writes of 32 lanes cover all banks once
  constexpr int KH = bwd_kh(DP);               // key halves of 64 keys
  constexpr int NW = 4 * KH;                    // waves
  constexpr int NT = 64 * NW;                   // threads
  constexpr int QDE = 32 * DP;                 // elements of one Q (or dO) tile
  constexpr int QDI = QDE * 2 / 1024;          // 1 KB async loads per Q (or dO) tile
  static_assert(QDI % KH == 0, "Q / dO loads split over the key halves");
  // Double buffers [parity]; one loop body serves both parities, so the
  // resident accumulators keep one register assignment across steps.
  __shared__ __attribute__((aligned(16))) float Bfb[2][2 * KH][1024];  // bias fragments [32-key block]
  __shared__ __attribute__((aligned(16))) __bf16 QDb[2][4][2 * QDE];   // [outer row] Q | dO rows
  __shared__ __attribute__((aligned(16))) float RSb[2][4][64];         // [outer row] nl2 | nd
  // The waves' dS^T tiles [64 keys][SP]; at setup their K tiles [64 keys][KT].
  constexpr int SSE = 64 * (KT > SP ? KT : SP);
  __shared__ __attribute__((aligned(16))) __bf16 dSs[NW * SSE];
  __bf16* const dSbase = dSs;
  // Key half 1's dQ^T tiles for key half 0 [outer row][d block][16 regs][lane].
  __shared__ __attribute__((aligned(16))) float Xq[KH == 2 ? 4 : 1][DP / 32][16][64];

  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int pw = w & 3, kh = w >> 2;            // outer row in the group, key half
  const int kl = lane & 31, hl = lane >> 5;
  const int N = g.N, D = g.D, H = g.H;
  const int nkb = (N + 64 * KH - 1) / (64 * KH);
  const int groups = (g.O + kBwdGroup - 1) / kBwdGroup;
  const int runs = (groups + run - 1) / run;
  const int64_t total = (int64_t)H * nkb * sl.nbrun;
  int64_t T;
  {
    const int64_t L = blockIdx.x, per = (total + 7) / 8;
    T = (L % 8) * per + L / 8;
    if (T >= total) return;
  }
  // Tile order (head, batch and run of outer groups, key block): the nkb
  // workgroups that share one group's Q / dO rows run side by side on one
  // XCD (L2 reuse).  A workgroup walks the `run` consecutive outer groups of
  // its run and accumulates their dBias into one partial (slot brun).
  const int kblk = (int)(T % nkb);
  const int64_t hb = T / nkb;
  const int brun = sl.brun0 + (int)(hb % sl.nbrun);
  const int h = (int)(hb / sl.nbrun);
  const int b = brun / runs;
  const int og_lo = (brun % runs) * run, og_hi = min(groups, og_lo + run);
  const int key_base = kblk * 64 * KH + 64 * kh;
  // A key half past N (N % 128 == 64) runs with every key masked: P = dS = 0.
  const bool keys_ok = key_base < N;
  const float c2 = g.scale * kLog2e;
  const float inv_scale = 1.f / g.scale;
  __bf16* const Ss = dSbase + w * SSE;  // this wave's dS^T tile, and its K tile at setup
  __bf16* const Kt = Ss;
  float* const dbp = dbias_part + ((int64_t)brun * H + h) * N * N;

#pragma unroll 1
  for (int og = og_lo; og < og_hi; ++og) {
  const bool first = og == og_lo;
  // Every wave's LDS reads of the previous group are done before this
  // group's setup writes the K tiles, statistics and first loads.
  if (!first) __syncthreads();
  const int o = og * kBwdGroup + pw;
  const bool plane_ok = o < g.O;
  const int plane = b * g.O + (plane_ok ? o : 0);
  const int64_t plane_off = (int64_t)plane * g.s_plane + (int64_t)h * g.s_head;
  const bool active = plane_ok && keys_ok;

  if (!plane_ok && kh == 0) {  // statistics of an idle outer row: P = 0 everywhere
    RSb[0][pw][lane] = lane < 32 ? -INFINITY : 0.f;
    RSb[1][pw][lane] = lane < 32 ? -INFINITY : 0.f;
  }

  const int64_t bb = (g.bias_bstride == 0) ? 0 : b;
  const int nb32 = N / 32;
  // Fragment blocks (kb32, qb) of this head: [(bb*H + h)*nb32 + kb32][qb][1024].
  const float* bfrag = bias_f + ((bb * H + h) * nb32 + kblk * 2 * KH) * (int64_t)nb32 * 1024;
  const int64_t do_plane = (int64_t)plane * N * H * D + (int64_t)h * D;  // dO is [B,O,N,H,D]
  const int64_t st_plane = ((int64_t)plane * H + h) * N;                // row statistics
  // dQ partials of the slab's planes [key block][plane - plane0][h][q][D].
  __bf16* dqp = dq_part + ((int64_t)kblk * sl.planes + (plane_ok ? plane - sl.plane0 : 0)) * H * N * D +
                (int64_t)h * N * D;
  const int key_blk0 = kblk * 64 * KH;  // first key of the workgroup
  // Partial stores through buffer resources: per-lane offsets fixed for the
  // walk, the step's offset in a scalar.  dQ: this wave's outer row and
  // head; dBias: the (run, head) N x N block, which the first group of the
  // run writes and the later ones read back (range 0: reads give zeros) and
  // rewrite with their rows added.
  const __amdgpu_buffer_rsrc_t rs_dq = __builtin_amdgcn_make_buffer_rsrc(dqp, 0, 0x7FFFFFFF, 0x00020000);
  const uint32_t vdq = (uint32_t)(kl * D * 2);  // query row kl of the step
  const __amdgpu_buffer_rsrc_t rs_db = __builtin_amdgcn_make_buffer_rsrc(dbp, 0, 0x7FFFFFFF, 0x00020000);
  const int dbkey = tid % (64 * KH), dbqb = tid / (64 * KH);
  const uint32_t vdb = key_blk0 + dbkey < N ? (uint32_t)((8 * dbqb * N + key_blk0 + dbkey) * 4) : kBufOOB;
  // The run's partial so far: read back by the thread that writes it
  // (range 0 for the run's first group: zeros), at device scope (sc1), so
  // the load misses the CU's L1, which may hold an older copy of the line.
  const __amdgpu_buffer_rsrc_t rs_dbr =
      __builtin_amdgcn_make_buffer_rsrc(dbp, 0, first ? 0 : 0x7FFFFFFF, 0x00020000);

  // Issue the direct-to-LDS loads of step q0 into buffer `buf`.
  typedef float BfT[2 * KH][1024];
  typedef __bf16 QDT[4][2 * QDE];
  typedef float RST[4][64];
  // bf16 pair (1, 0) for the dBias sum, materialised in a register: as an
  // operand of v_dot2c_f32_bf16 the compiler would encode it as the inline
  // constant 1.0, which the hardware reads as the f32 pattern 0x3f800000,
  // i.e. the pair (0, 1).
  uint32_t sel_lo_bits;
  asm volatile("v_mov_b32 %0, 0x3f80" : "=v"(sel_lo_bits));
  // Buffer loads with per-lane byte offsets fixed for the whole walk; each
  // step advances only a scalar offset.  Lanes past D and the lanes of an
  // idle wave read zeros (kBufOOB).
  const i32x4 rs_bias = buffer_rsrc(bfrag);
  const i32x4 rs_q = buffer_rsrc(q + plane_off);
  const i32x4 rs_do = buffer_rsrc(dout + do_plane);
  // Bias: wave w loads kilobytes 2w and 2w+1 of the step's 8*KH KB (32-key
  // blocks past N read zeros).  Q / dO: key half kh loads its share of its
  // outer row's tiles.
  constexpr int QDH = QDI / KH;
  uint32_t vb[2], vq[QDH], vdo[QDH];
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    const int kbx = 2 * w + x, cb = kbx >> 2, j = kbx & 3;
    vb[x] = key_blk0 + 32 * cb < N ? (uint32_t)((cb * nb32 * 1024 + j * 256 + lane * 4) * 4)
                                   : kBufOOB;
  }
#pragma unroll
  for (int n = 0; n < QDH; ++n) {
    const int gc = (kh * QDH + n) * 64 + lane, r = gc / (DP / 8), c = (gc % (DP / 8)) ^ qd_swz<DP>(r);
    const bool ld = plane_ok && c * 8 < D;
    vq[n] = ld ? (uint32_t)((r * g.s_row + c * 8) * 2) : kBufOOB;
    vdo[n] = ld ? (uint32_t)((r * H * D + c * 8) * 2) : kBufOOB;
  }
  auto issue = [&](int q0, BfT& Bf, QDT& QDs, RST& RS) {
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const int kbx = 2 * w + x, cb = kbx >> 2, j = kbx & 3;
      buf2lds16_so(rs_bias, vb[x], (uint32_t)q0 * 128u, &Bf[cb][j * 256]);
    }
    // Q and dO rows, swizzled.
#pragma unroll
    for (int n = 0; n < QDH; ++n) {
      const int nn = kh * QDH + n;
      buf2lds16_so(rs_q, vq[n], (uint32_t)(q0 * g.s_row * 2), &QDs[pw][nn * 512]);
      buf2lds16_so(rs_do, vdo[n], (uint32_t)(q0 * H * D * 2), &QDs[pw][QDE + nn * 512]);
    }
    // An idle outer row keeps the -inf / 0 statistics written at setup, so
    // its P and dS are exactly zero and it adds nothing to the dBias sum.
    if (plane_ok && kh == 0 && lane < 16) {
      const float* src = (lane < 8 ? nl2_g : nd_g) + st_plane + q0 + (lane & 7) * 4;
      g2lds16(src, &RS[pw][0]);
    }
  };

  // The first step's loads go out before the key block's setup loads, so
  // the two latencies overlap (Q / dO chunks past D and idle rows read
  // zeros through the buffer range check).
  issue(0, Bfb[0], QDb[0], RSb[0]);

  // Per-wave constant operands for this key block.
  bf16x8 kB[2][DP / 16], vB[2][DP / 16];  // B operands of S and dP (lane = key)
  bf16x8 kA[DP / 32][4];                  // A operand of dQ^T = K^T dS^T
  float mk2[2];
  {
    // All loads first (branch-free, zeros outside the tensor), one wait.
    const __amdgpu_buffer_rsrc_t rk = raw_rsrc(k + plane_off), rv = raw_rsrc(v + plane_off);
    const __amdgpu_buffer_rsrc_t rm = raw_rsrc(mask + (int64_t)plane * N);
    float mraw[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int key = key_base + cb * 32 + kl;
#pragma unroll
      for (int s = 0; s < DP / 16; ++s) {
        const int d0 = 16 * s + 8 * hl;
        const uint32_t off = (active && d0 < D) ? (uint32_t)(((int64_t)key * g.s_row + d0) * 2) : kBufOOB;
        kB[cb][s] = buf_ld8(rk, off);
        vB[cb][s] = buf_ld8(rv, off);
      }
      mraw[cb] = buf_ldf(rm, active ? (uint32_t)(key * 4) : kBufOOB);
    }
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
#pragma unroll
      for (int s = 0; s < DP / 16; ++s)
        *reinterpret_cast<bf16x8*>(&Kt[(cb * 32 + kl) * KT + 16 * s + 8 * hl]) = kB[cb][s];
      mk2[cb] = active ? mraw[cb] * inv_scale : (keys_ok ? 0.f : -INFINITY);
    }
  }
  const bool wmask = __any(mk2[0] != 0.f || mk2[1] != 0.f);
  __syncthreads();
#pragma unroll
  for (int db = 0; db < DP / 32; ++db)
#pragma unroll
    for (int t = 0; t < 4; ++t)
      kA[db][t] = cat8(tr_col4(Kt, KT, 16 * t, 16 * t + 8, 32 * db),
                       tr_col4(Kt, KT, 16 * t + 4, 16 * t + 12, 32 * db));

  f32x16 dKacc[DP / 32][2], dVacc[DP / 32][2];
#pragma unroll
  for (int db = 0; db < DP / 32; ++db)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) { dKacc[db][cb] = zero16(); dVacc[db][cb] = zero16(); }

  __syncthreads();  // zero fill and K-tile reads done before the first loads land
  // One query step: prefetch step q0+32 into the other buffers, wait for this
  // step's loads, compute.  Barriers are bare s_barrier with an explicit LDS
  // counter wait, so the prefetch stays in flight across them.
  auto step = [&](int q0, BfT& Bc, QDT& QDc, RST& RSc, BfT& Bn, QDT& QDn, RST& RSn) {
    float dbprev[8];
    auto load_dbprev = [&] {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        dbprev[e] = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(rs_dbr, vdb, (q0 + e) * N * 4, 16));
    };
    // This step's loads were issued one step ago; wait for them, read the
    // shared bias fragments and the row statistics, then start the next
    // step's loads so they overlap this step's compute.
    // Younger than those loads: this wave's previous-step partial loads
    // (8 read-backs) and stores (8 dBias, plus dQ on key half 0), all issued
    // by every wave; with two key halves they may stay in flight (different
    // rows from this step's; measured faster), with one (D = 64) waiting for
    // them measured faster.  The first step of a group waits for
    // everything: its setup loads are younger, and the last group's partial
    // stores must land before this group reads the same addresses back.
    if (q0 == 0 || KH == 1 || MODE == kBwdDKDV)
      wait_vmcnt<0>();
    else
      wait_vmcnt<16>();
    lds_barrier();
    f32x16 sinit[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f32x4 x = *reinterpret_cast<const f32x4*>(&Bc[2 * kh + cb][j * 256 + lane * 4]);
#pragma unroll
        for (int i = 0; i < 4; ++i) sinit[cb][4 * j + i] = x[i];
      }
    f32x16 nl2v, ndv;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f32x4 a4 = *reinterpret_cast<const f32x4*>(&RSc[pw][8 * j + 4 * hl]);
      f32x4 d4 = *reinterpret_cast<const f32x4*>(&RSc[pw][32 + 8 * j + 4 * hl]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        nl2v[4 * j + i] = a4[i];
        ndv[4 * j + i] = d4[i];
      }
    }
    const __bf16* Qs = QDc[pw];
    const __bf16* dOs = QDc[pw] + QDE;
    bf16x8 qA[DP / 16], doA[DP / 16];
#pragma unroll
    for (int s = 0; s < DP / 16; ++s) {
      const int c = 16 * s + 8 * hl;
      qA[s] = *reinterpret_cast<const bf16x8*>(&Qs[qd_off<DP>(kl, c)]);
      doA[s] = *reinterpret_cast<const bf16x8*>(&dOs[qd_off<DP>(kl, c)]);
    }
    // The other buffers were last read before the barrier above.
    if (q0 + 32 < N) issue(q0 + 32, Bn, QDn, RSn);
    f32x16 P[2], dS[2];
    float tsum[16];  // delta_true: this lane's sum over its keys of P dP per query row
#pragma unroll
    for (int r = 0; r < 16; ++r) tsum[r] = 0.f;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      f32x16 sacc = sinit[cb];
      f32x16 dp = ndv;
#pragma unroll
      for (int ks = 0; ks < DP / 16; ++ks) {
        sacc = mfma32(qA[ks], kB[cb][ks], sacc);
        dp = mfma32(doA[ks], vB[cb][ks], dp);
      }
      if (wmask) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[r] += mk2[cb];
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(fmaf(sacc[r], c2, nl2v[r]));
        P[cb][r] = p;
        dS[cb][r] = p * dp[r];
        // dP itself is the accumulator minus its -delta seed.
        if constexpr (MODE == kBwdDKDV) tsum[r] = fmaf(p, dp[r] - ndv[r], tsum[r]);
      }
    }
    if constexpr (MODE == kBwdDKDV) {
      // delta_true partial of this wave's 64 keys: the 32 key lanes of each
      // half summed on DPP / permlane (fixed order), written by lanes 0 / 32
      // as the 16 query rows 8j + 4hl + i.
      if (dtrue_part && active) {
#pragma unroll
        for (int r = 0; r < 16; ++r) tsum[r] = lanes_sum<32>(tsum[r]);
        if (kl == 0) {
          const int nkb64 = (N + 63) / 64;
          float* dst = dtrue_part + (((int64_t)plane * H + h) * nkb64 + kblk * KH + kh) * N + q0;
#pragma unroll
          for (int j = 0; j < 4; ++j)
            *reinterpret_cast<f32x4*>(dst + 8 * j + 4 * hl) =
                f32x4{tsum[4 * j], tsum[4 * j + 1], tsum[4 * j + 2], tsum[4 * j + 3]};
        }
      }
    }
    // P and dS in bf16, packed once: B operands of dV^T += dO^T P and
    // dK^T += Q^T dS (16-query k-steps, C-layout order) and the dS^T tile.
    bf16x8 pP[2][2], pS[2][2];  // [cb][t]
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        pP[cb][t] = pack8(P[cb], 8 * t);
        pS[cb][t] = pack8(dS[cb], 8 * t);
      }
    if constexpr (MODE != kBwdDQDB) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int db = 0; db < DP / 32; ++db) {
        const bf16x8 da = cat8(qd_tr_col4<DP>(dOs, 16 * t, 16 * t + 4, 32 * db),
                               qd_tr_col4<DP>(dOs, 16 * t + 8, 16 * t + 12, 32 * db));
        const bf16x8 qa = cat8(qd_tr_col4<DP>(Qs, 16 * t, 16 * t + 4, 32 * db),
                               qd_tr_col4<DP>(Qs, 16 * t + 8, 16 * t + 12, 32 * db));
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          dVacc[db][cb] = mfma32(da, pP[cb][t], dVacc[db][cb]);
          dKacc[db][cb] = mfma32(qa, pS[cb][t], dKacc[db][cb]);
        }
      }
    }
    }  // dK / dV
    if constexpr (MODE != kBwdDKDV) {
    // dS -> LDS as bf16 [key][query]: the dQ operand and the dBias sum.
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bf16x8 h = pS[cb][j >> 1];
        bf16x4 s4;
#pragma unroll
        for (int i = 0; i < 4; ++i) s4[i] = h[4 * (j & 1) + i];
        *reinterpret_cast<bf16x4*>(&Ss[(cb * 32 + kl) * SP + 8 * j + 4 * hl]) = s4;
      }
    // The run's partial so far for this step's dBias outputs, loaded here
    // so the dQ phase and its barrier cover the latency.
    load_dbprev();
    // dQ^T (d x 32 queries) = K^T dS^T over this wave's 64 keys; key half 1
    // hands its tile to key half 0 through LDS (read after the barrier).
    f32x16 dqacc[DP / 32];
#pragma unroll
    for (int db = 0; db < DP / 32; ++db) {
      f32x16 acc = zero16();
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const bf16x8 sb = cat8(tr_col4(Ss, SP, 16 * t, 16 * t + 8, 0),
                               tr_col4(Ss, SP, 16 * t + 4, 16 * t + 12, 0));
        acc = mfma32(kA[db][t], sb, acc);
      }
      dqacc[db] = acc;
      if (KH == 2 && kh == 1) {
#pragma unroll
        for (int r = 0; r < 16; ++r) Xq[pw][db][r][lane] = acc[r];
      }
    }
    lds_barrier();
    // dQ partial over the workgroup's keys: (half 0 + half 1) -> bf16.
    if (kh == 0 && plane_ok) {
#pragma unroll
      for (int db = 0; db < DP / 32; ++db) {
        f32x16 acc = dqacc[db];
        if (KH == 2) {
          // All 16 values in one batch of LDS reads and one wait (at full
          // register pressure the compiler issues them one pair at a time).
          const u32x16 x = lds_read_col16(lds_offset(&Xq[pw][db][0][lane]));
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[r] += __uint_as_float(x[r]);
        }
        // Lane-pair exchange as for dK / dV below: 16-byte stores of
        // channels 16p + 8hl .. +7 (chunks past D dropped by the range check).
        uint32_t pq[4][2];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int e = 0; e < 2; ++e)
            pq[j][e] = __builtin_bit_cast(
                uint32_t, bf16x2{f2bf(acc[4 * j + 2 * e]), f2bf(acc[4 * j + 2 * e + 1])});
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            auto r = __builtin_amdgcn_permlane32_swap(pq[2 * pp][e], pq[2 * pp + 1][e], false, false);
            pq[2 * pp][e] = r[0];
            pq[2 * pp + 1][e] = r[1];
          }
          const int d0 = db * 32 + 16 * pp + 8 * hl;
          const u32x4 o = {pq[2 * pp][0], pq[2 * pp][1], pq[2 * pp + 1][0], pq[2 * pp + 1][1]};
          __builtin_amdgcn_raw_buffer_store_b128(o, rs_dq, d0 < D ? vdq + (uint32_t)d0 * 2 : kBufOOB,
                                                 q0 * D * 2, 0);
        }
      }
    }
    // dBias partial (f32): the 4 outer rows' bf16 dS^T tiles summed in the fixed
    // order ((o0 + o1) + o2) + o3.  Thread = (key, 8-query block): 8-byte
    // reads of each wave's row, and each store instruction of a wave writes
    // 64 consecutive keys of one query row (128 bytes).
    {
      const int key = dbkey, qb = dbqb;
      const int kw = 4 * (key >> 6);  // first wave of this key's half
      // Each add is one v_dot2 with a one-hot selector: x * 1 + y * 0 + acc
      // is the f32 sum acc + x (unpack and add in one instruction).
      const bf16x2 sel[2] = {__builtin_bit_cast(bf16x2, sel_lo_bits),
                             {static_cast<__bf16>(0.f), static_cast<__bf16>(1.f)}};
      float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      // The 4 rows' chunks in one batch of LDS reads and one wait.
      const __bf16* src = dSbase + kw * SSE + (key & 63) * SP + 8 * qb;
      u32x4 rows[4];
      lds_read_rows4(rows, lds_offset(src), lds_offset(src + SSE), lds_offset(src + 2 * SSE),
                     lds_offset(src + 3 * SSE));
#pragma unroll
      for (int ww = 0; ww < 4; ++ww) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          // (A vector element is copied to a scalar before the bit cast:
          // hipcc 7.2 folds a bit cast of an element expression to element 0.)
          acc[e] = __builtin_amdgcn_fdot2_f32_bf16(
              __builtin_bit_cast(bf16x2, (uint32_t)rows[ww][e >> 1]), sel[e & 1], acc[e], false);
      }
      // The run's partial: earlier groups first, then this group's rows.
#pragma unroll
      for (int e = 0; e < 8; ++e)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(dbprev[e] + acc[e]), rs_db, vdb,
                                              (q0 + e) * N * 4, 0);
    }
    }  // dQ / dBias
  };
#pragma unroll 1
  for (int q0 = 0; q0 < N; q0 += 32) {
    const int cur = (q0 >> 5) & 1;
    step(q0, Bfb[cur], QDb[cur], RSb[cur], Bfb[cur ^ 1], QDb[cur ^ 1], RSb[cur ^ 1]);
  }
  // dK (scaled) and dV, in Q/K/V storage order.  A lane holds channels
  // 8j + 4hl .. +3 (j = 0..3) of its key; one exchange with lane l ^ 32 per
  // register pair (j, j + 1) gives it 8 consecutive channels, 16j + 8hl ..
  // +7, so each store instruction writes 32 contiguous bytes per key (two
  // 16-byte stores per key and tensor instead of four 8-byte ones).
  if (MODE != kBwdDQDB && active) {
#pragma unroll
  for (int db = 0; db < DP / 32; ++db)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int key = key_base + cb * 32 + kl;
      const int64_t row = (int64_t)plane * g.o_plane + (int64_t)h * g.o_head + (int64_t)key * g.o_row;
      uint32_t pk[4][2], pv[4][2];  // [j][pair] packed bf16
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const bf16x2 a = {f2bf(dKacc[db][cb][4 * j + 2 * e] * g.scale),
                            f2bf(dKacc[db][cb][4 * j + 2 * e + 1] * g.scale)};
          const bf16x2 v2 = {f2bf(dVacc[db][cb][4 * j + 2 * e]), f2bf(dVacc[db][cb][4 * j + 2 * e + 1])};
          pk[j][e] = __builtin_bit_cast(uint32_t, a);
          pv[j][e] = __builtin_bit_cast(uint32_t, v2);
        }
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        // Lanes < 32 keep chunk 2p and receive chunk 2p of lane l + 32;
        // lanes >= 32 receive chunk 2p + 1 of lane l - 32 and keep theirs.
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          auto rk = __builtin_amdgcn_permlane32_swap(pk[2 * p][e], pk[2 * p + 1][e], false, false);
          pk[2 * p][e] = rk[0];
          pk[2 * p + 1][e] = rk[1];
          auto rv = __builtin_amdgcn_permlane32_swap(pv[2 * p][e], pv[2 * p + 1][e], false, false);
          pv[2 * p][e] = rv[0];
          pv[2 * p + 1][e] = rv[1];
        }
        const int d0 = db * 32 + 16 * p + 8 * hl;
        if (d0 < D) {
          const u32x4 ok = {pk[2 * p][0], pk[2 * p][1], pk[2 * p + 1][0], pk[2 * p + 1][1]};
          const u32x4 ov = {pv[2 * p][0], pv[2 * p][1], pv[2 * p + 1][0], pv[2 * p + 1][1]};
          *reinterpret_cast<u32x4*>(dk + row + d0) = ok;
          *reinterpret_cast<u32x4*>(dv + row + d0) = ov;
        }
      }
    }
  }
  }  // outer groups of the run
}

// dQ = bf16(scale * sum_kb partial[kb]) in ascending key-block order; bf16
// partials [kb][plane][h][q][D], output in Q's storage order.  One call
// folds 256 (query, 8-channel chunk) items, chunk bx, of (plane, head) block
// ph.  Up to 8 partial loads are in flight; they are added in key-block order.
__device__ __forceinline__ void dq_fold_block(const __bf16* __restrict__ part,
                                              __bf16* __restrict__ dq, const AttnGeom& g, int nkb,
                                              int bx, int64_t ph, int64_t plane0, int64_t planes) {
  const int D8 = g.D / 8;
  const int t = bx * 256 + threadIdx.x;
  if (t >= g.N * D8) return;
  const int qq = t / D8, d0 = (t - qq * D8) * 8;
  const int64_t stride = planes * g.H * g.N * g.D;
  const int64_t lp = ph / g.H;  // plane within the slab
  const int hh = (int)(ph - lp * g.H);
  const int64_t plane = plane0 + lp;
  const __bf16* src = part + (ph * g.N + qq) * g.D + d0;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  for (int k0 = 0; k0 < nkb; k0 += 8) {
    bf16x8 x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (k0 + u < nkb) x[u] = ld8_nt(src + (int64_t)(k0 + u) * stride);
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (k0 + u < nkb) {
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = (k0 + u == 0) ? bf2f(x[u][e]) : acc[e] + bf2f(x[u][e]);
      }
  }
  bf16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = f2bf(acc[e] * g.scale);
  st8(dq + plane * g.o_plane + hh * g.o_head + (int64_t)qq * g.o_row + d0, o);
}

// Grid: x = 256-item chunk, y = plane * H + h (strided past the grid limit).
__global__ __launch_bounds__(256) void attn_dq_reduce_kernel(
    const __bf16* __restrict__ part, __bf16* __restrict__ dq, AttnGeom g, int nkb) {
  const int64_t nph = (int64_t)g.B * g.O * g.H;
  for (int64_t ph = blockIdx.y; ph < nph; ph += gridDim.y)
    dq_fold_block(part, dq, g, nkb, blockIdx.x, ph, 0, (int64_t)g.B * g.O);
}

// dBias[bb,h,q,k] = fold over the f32 (b, outer group) partials that share
// bias batch bb (Bb == 1 folds every batch; Bb == B folds per batch).
// Workgroup = 512 outputs x 4 ranges of partials: thread (range s, chunk c)
// sums its range for 8 consecutive keys in ascending order (4 partials, 8
// loads in flight; each load instruction of a wave reads 1 KB, or 8 x 128 B
// for a tile), and the four range sums are added in the fixed order
// ((s0 + s1) + s2) + s3.  Output: f32 in [Bb, H, N, N] order, or (out_bf16)
// rounded to bf16, either in that order or (transposed) in the order of a
// transposed bias, dbias[bb, h, k, q]: then the workgroup covers an 8-query
// x 64-key tile and writes it transposed through LDS, 16 bytes per key.
__device__ __forceinline__ void dbias_fold_block(const float* __restrict__ part,
                                                 void* __restrict__ dbias, int B, int Bb,
                                                 int groups, int H, int N, int64_t blk,
                                                 bool out_bf16, bool transposed) {
  __shared__ float red[4][64][9];
  const int c = threadIdx.x & 63, sl = threadIdx.x >> 6;
  const int64_t hnn = (int64_t)H * N * N;
  bool act;
  int bb;
  int64_t e;  // offset of the thread's first output in the [H, N, N] block
  int th = 0, tq0 = 0, tk0 = 0;  // transposed tile: head, first query, first key
  if (!transposed) {
    const int64_t idx = blk * 64 + c;
    act = idx < (int64_t)Bb * (hnn / 8);
    bb = act ? (int)(idx / (hnn / 8)) : 0;
    e = act ? (idx % (hnn / 8)) * 8 : 0;
  } else {
    // Tiles of 8 queries x 64 keys (N % 64 == 0): thread c -> query c / 8,
    // keys 8 (c % 8) .. +7.
    const int kt_n = N / 64, tiles = (N / 8) * kt_n;
    const int64_t bh = blk / tiles;
    const int r = (int)(blk % tiles), qt = r / kt_n, kt = r % kt_n;
    act = bh < (int64_t)Bb * H;
    bb = act ? (int)(bh / H) : 0;
    th = (int)(bh % H);
    tq0 = qt * 8;
    tk0 = kt * 64;
    e = act ? (int64_t)th * N * N + (int64_t)(tq0 + c / 8) * N + tk0 + (c % 8) * 8 : 0;
  }
  const int b_lo = (Bb == 1) ? 0 : bb, b_hi = (Bb == 1) ? B : bb + 1;
  const int n = (b_hi - b_lo) * groups;
  const int per = (n + 3) / 4;
  const int s0 = sl * per, s1 = min(n, s0 + per);
  const float* src = part + (int64_t)b_lo * groups * hnn + e;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;
  if (act) {
    for (int s = s0; s < s1; s += 4) {
      f32x4 x[4][2];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (s + u < s1) {
          const float* p = src + (int64_t)(s + u) * hnn;
          x[u][0] = ld4f_nt(p);
          x[u][1] = ld4f_nt(p + 4);
        }
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (s + u < s1) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float xv = x[u][i >> 2][i & 3];
            acc[i] = (s + u == s0) ? xv : acc[i] + xv;
          }
        }
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) red[sl][c][i] = acc[i];
  __syncthreads();
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    v[i] = red[0][c][i];
    for (int r = 1; r < 4; ++r)
      if (r * per < n) v[i] += red[r][c][i];
  }
  if (!transposed) {
    if (sl != 0 || !act) return;
    if (out_bf16) {
      bf16x8 o;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = f2bf(v[i]);
      st8((__bf16*)dbias + (int64_t)bb * hnn + e, o);
    } else {
      float* d = (float*)dbias + (int64_t)bb * hnn + e;
      *reinterpret_cast<f32x4*>(d) = f32x4{v[0], v[1], v[2], v[3]};
      *reinterpret_cast<f32x4*>(d + 4) = f32x4{v[4], v[5], v[6], v[7]};
    }
    return;
  }
  // Transposed bf16 tile: T[query][key] in LDS, then thread c writes key c's
  // 8 queries as one 16-byte chunk of dbias[bb, h, key, qt*8 .. +7].
  __shared__ __bf16 T[8][64 + 8];
  __syncthreads();  // every range's red reads done (sl > 0 threads read too)
  if (sl == 0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) T[c / 8][(c % 8) * 8 + i] = f2bf(v[i]);
  }
  __syncthreads();
  if (sl != 0 || !act) return;
  bf16x8 o;
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = T[i][c];
  st8((__bf16*)dbias + (int64_t)bb * hnn + (int64_t)th * N * N + (int64_t)(tk0 + c) * N + tq0, o);
}

__global__ __launch_bounds__(256) void attn_fold_kernel(
    const __bf16* __restrict__ dq_part, __bf16* __restrict__ dq, AttnGeom g, int nkb, int dq_bx,
    const float* __restrict__ db_part, void* __restrict__ dbias, int Bb, int groups,
    int64_t n_db, int db_mode, int64_t plane0, int64_t planes) {
  const int64_t b = blockIdx.x;
  if (b < n_db) {
    dbias_fold_block(db_part, dbias, g.B, Bb, groups, g.H, g.N, b, db_mode != 0, db_mode == 2);
  } else {
    const int64_t r = b - n_db;
    dq_fold_block(dq_part, dq, g, nkb, (int)(r % dq_bx), r / dq_bx, plane0, planes);
  }
}

// ---------------------------------------------------------------------------
// Output gate of the pair-row module core (the forward applies it in the
// attention forward's epilogue, og = o * sigmoid(g)).  Backward: one thread
// per (pair row, 8-channel chunk), so consecutive lanes touch consecutive 16
// bytes:
//   d_o = d_og * sigmoid(g),  dg = d_og * o * s * (1 - s), and
//             delta[b,i,h,j] = sum_d d_o * o (the softmax backward's row term;
//             the D/8 chunk partials of a head meet in LDS), with o + res when
//             the forward saved the shadow residual res of o.
// o / og / d_og / d_o are [B, N, N, H*D] rows; g and dg sit at the gate
// columns (offset 3*H*D) of the projection rows (row pitch `pitch`).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float gate_sigmoid(float x) { return sigmoidf(x); }

// Workgroup w takes items [w * per, (w + 1) * per) with per a multiple of
// D/8, so a head's chunks never straddle two workgroups.
template <bool SHADOW>
__global__ __launch_bounds__(256) void attn_gate_bwd_kernel(
    const __bf16* __restrict__ d_og, const __bf16* __restrict__ o,
    const __bf16* __restrict__ res, const __bf16* __restrict__ gate, int64_t gpitch,
    __bf16* __restrict__ d_o,
    float* __restrict__ delta, __bf16* __restrict__ dgate, int64_t dpitch, int64_t items, int per,
    FastDiv fN, int H, int D, FastDiv fhc8, int og_t) {
  // items < 2^31 (checked on the host): 32-bit item index; element offsets
  // (8 per item) are formed in 64 bits.
  __shared__ float part[256];
  const int tid = threadIdx.x;
  const uint32_t t = blockIdx.x * (uint32_t)per + tid;  // (row, chunk)
  const int d8 = D / 8;
  const bool act = tid < per && t < (uint32_t)items;
  const uint32_t row = fdiv(t, fhc8);
  const int c = (int)(t - row * fhc8.d);
  float sdot = 0.f;
  if (act) {
    // og_t: d_og of pair row (b, i, j) is stored at row (b, j, i).
    size_t dog = (size_t)t * 8;
    if (og_t) {
      const uint32_t pl = fdiv(row, fN), j = row - pl * fN.d;
      const uint32_t bb = fdiv(pl, fN), i = pl - bb * fN.d;
      dog = (((size_t)bb * fN.d + j) * fN.d + i) * (8 * (size_t)fhc8.d) + (size_t)c * 8;
    }
    const bf16x8 dv = ld8(d_og + dog), ov = ld8(o + (size_t)t * 8),
                 gv = ld8(gate + (size_t)row * gpitch + c * 8);
    bf16x8 rv;
    if (SHADOW) rv = ld8(res + (size_t)t * 8);
    bf16x8 r_do, r_dg;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float sg = gate_sigmoid(bf2f(gv[e]));
      const float dd = bf2f(dv[e]), oo = bf2f(ov[e]);
      r_do[e] = f2bf(dd * sg);
      r_dg[e] = f2bf(dd * oo * sg * (1.f - sg));
      // delta pairs the bf16 dO that the backward kernel reads with O (with
      // SHADOW, with O + its rounding residual, summed in f32).
      sdot = fmaf(bf2f(r_do[e]), SHADOW ? oo + bf2f(rv[e]) : oo, sdot);
    }
    st8(d_o + (size_t)t * 8, r_do);
    st8(dgate + (size_t)row * dpitch + c * 8, r_dg);
  }
  part[tid] = sdot;
  __syncthreads();
  if (!act) return;
  if (c % d8 != 0) return;
  float s = 0.f;
  for (int u = 0; u < d8; ++u) s += part[tid + u];
  // row = (b, i, j): plane (b, i), query j; delta is [plane][h][j].
  const int h = c / d8;
  const uint32_t plane = fdiv(row, fN);
  const int j = (int)(row - plane * fN.d);
  delta[((int64_t)plane * H + h) * fN.d + j] = s;
}

// Pair-bias gradient into the projection gradient rows.  Workgroup = 512
// consecutive (query, key) elements of one bias batch bb x 4 head slots:
// thread (slot s, lane c) owns elements 4c..4c+3 and 256+4c..256+4c+3 (each
// load instruction of a wave reads 1 KB contiguous) and folds heads s, s + 4,
// ... < H, each over the f32 (b, outer group) partials that share bb in
// ascending order (8 partials' loads in flight, nontemporal: the partials are
// read once).  The H sums of an element meet in LDS, and the workgroup then
// writes the row tails [4*H*D, pitch) of its 512 key rows (H values, zeros
// after them) in 16-byte chunks, consecutive lanes on consecutive chunks.
__global__ __launch_bounds__(256) void attn_dbias_pair_kernel(
    const float* __restrict__ part, int B, int Bb, int groups, int H, int N,
    __bf16* __restrict__ dproj, int64_t pitch, int64_t tail_off, int transpose_bias) {
  __shared__ float red[16][516];
  const int tid = threadIdx.x, c = tid & 63, slot = tid >> 6;
  const int64_t nn = (int64_t)N * N;  // a multiple of 512 (N % 64 == 0)
  const int64_t el0 = (int64_t)blockIdx.x * 512;  // over Bb * nn
  const int bb = (int)(el0 / nn);
  const int64_t e = el0 - (int64_t)bb * nn;
  const int b_lo = (Bb == 1) ? 0 : bb, b_hi = (Bb == 1) ? B : bb + 1;
  const int64_t stride = (int64_t)H * nn;
  const int n = (b_hi - b_lo) * groups;
  const int o0 = 4 * c, o1 = 256 + 4 * c;
  for (int h = slot; h < H; h += 4) {
    const float* src = part + (int64_t)b_lo * groups * stride + (int64_t)h * nn + e;
    f32x4 a0 = ld4f_nt(src + o0), a1 = ld4f_nt(src + o1);
    int s = 1;
    for (; s + 8 <= n; s += 8) {
      f32x4 x[8][2];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float* p = src + (int64_t)(s + u) * stride;
        x[u][0] = ld4f_nt(p + o0);
        x[u][1] = ld4f_nt(p + o1);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) { a0 += x[u][0]; a1 += x[u][1]; }
    }
    for (; s < n; ++s) {
      const float* p = src + (int64_t)s * stride;
      a0 += ld4f_nt(p + o0);
      a1 += ld4f_nt(p + o1);
    }
    *reinterpret_cast<f32x4*>(&red[h][o0]) = a0;
    *reinterpret_cast<f32x4*>(&red[h][o1]) = a1;
  }
  __syncthreads();
  // Row tails: 512 key rows x tail8 chunks of 8 bf16 (chunk u of a row holds
  // heads 8u .. 8u+7).
  const int tail8 = (int)((pitch - tail_off) / 8);
  for (int t = tid; t < 512 * tail8; t += 256) {
    const int j = t / tail8, ch = t - j * tail8;
    const int64_t el = e + j;
    const int q = (int)(el / N), k = (int)(el % N);
    const int64_t r = (int64_t)bb * nn + (transpose_bias ? (int64_t)k * N + q : (int64_t)q * N + k);
    bf16x8 v;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int h = ch * 8 + u;
      v[u] = f2bf(h < H ? red[h][j] : 0.f);
    }
    st8(dproj + r * pitch + tail_off + ch * 8, v);
  }
}

}  // namespace tpf

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
using namespace tpf;

static int check_geom(const AttnGeom& g, const char* fn) {
  if (g.B < 1 || g.O < 1 || g.H < 1 || g.N < 1)
    return set_error(TPF_ERR_SHAPE, "%s: B, O, H and N must be positive", fn);
  if (g.N % 64 != 0)
    return set_error(TPF_ERR_SHAPE, "%s: N=%d must be a multiple of 64 (pad on the host)", fn, g.N);
  if (g.D < 8 || g.D > 64 || g.D % 8 != 0)
    return set_error(TPF_ERR_SHAPE, "%s: D=%d must be a multiple of 8 in [8, 64]", fn, g.D);
  if (g.H > 65535) return set_error(TPF_ERR_SHAPE, "%s: H=%d exceeds the grid-y limit", fn, g.H);
  return TPF_OK;
}

static int make_geom(AttnGeom* g, int64_t B, int64_t O, int64_t H, int64_t N, int64_t D,
                     int layout, int64_t bias_batches, double scale, const char* fn) {
  if (B > INT32_MAX || O > INT32_MAX || N > INT32_MAX)
    return set_error(TPF_ERR_SHAPE, "%s: dimension exceeds int32", fn);
  if (layout & ~(TPF_QKV_SEQ_MAJOR | TPF_BIAS_TRANSPOSED | TPF_DBIAS_BF16))
    return set_error(TPF_ERR_ARG, "%s: unknown layout flags 0x%x", fn, layout);
  const bool seq_major = layout & TPF_QKV_SEQ_MAJOR;
  g->B = (int)B; g->O = (int)O; g->H = (int)H; g->N = (int)N; g->D = (int)D;
  g->s_row = seq_major ? H * D : D;
  g->s_head = seq_major ? D : N * D;
  g->s_plane = H * N * D;
  if (bias_batches != 1 && bias_batches != B)
    return set_error(TPF_ERR_SHAPE, "%s: bias batch count %lld must be 1 or B=%lld", fn,
                     (long long)bias_batches, (long long)B);
  g->bias_bstride = (bias_batches == 1) ? 0 : H * N * N;
  g->o_row = g->s_row;
  g->o_head = g->s_head;
  g->o_plane = g->s_plane;
  g->scale = (float)scale;
  g->og_t = 0;
  g->gate_pitch = 0;
  return check_geom(*g, fn);
}

// Contiguous [Bb, H, N, N] bias, or (TPF_BIAS_TRANSPOSED in layout) the
// transpose over its last two axes of a contiguous one: bias[bb, h, q, k]
// stored at bb*H*N*N + h*N*N + k*N + q.
static BiasView dense_bias(int64_t H, int64_t N, int64_t bias_batches, int layout = 0) {
  const bool t = layout & TPF_BIAS_TRANSPOSED;
  BiasView bv;
  bv.s_bb = bias_batches == 1 ? 0 : H * N * N;
  bv.s_h = N * N;
  bv.s_q = t ? 1 : N;
  bv.s_k = t ? N : 1;
  bv.H = (int)H;
  return bv;
}

static int attn_prescale_bias(const AttnGeom& g, const void* bias, const BiasView& bv,
                              float* bias_s, int64_t bias_batches, hipStream_t s,
                              const char* fn) {
  const int64_t items = bias_batches * g.H * (int64_t)g.N * g.N / 4;
  hipLaunchKernelGGL(attn_bias_prescale_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256),
                     0, s, (const __bf16*)bias, bias_s, items, g.N, 1.f / g.scale, bv);
  return check_launch(fn);
}

static int attn_forward_impl(AttnGeom g, const void* q, const void* k, const void* v,
                             const float* mask, const void* bias, const BiasView& bv,
                             int64_t bias_batches, void* out, float* lse, void* res,
                             void* workspace, hipStream_t s, const char* fn,
                             const void* gate = nullptr, void* og = nullptr) {
  // Waves (32 queries each) per workgroup, and outer rows per wave (planes
  // sharing one bias load).
  constexpr int kFwdWaves = 4, kFwdPlanes32 = 2, kFwdPlanes64 = 1;
  const int pl = g.D <= 32 ? kFwdPlanes32 : kFwdPlanes64;
  const int64_t total = ((g.N + 32 * kFwdWaves - 1) / (32 * kFwdWaves)) * (int64_t)g.H * g.B *
                        ((g.O + pl - 1) / pl);
  if ((total + 7) / 8 * 8 > INT32_MAX)
    return set_error(TPF_ERR_SHAPE, "%s: too many query tiles", fn);
  if (g.N > kFwdMaskLdsMaxN)
    return set_error(TPF_ERR_SHAPE, "%s: N=%d exceeds the forward's mask staging limit %d", fn, g.N,
                     kFwdMaskLdsMaxN);
  float* bias_s = (float*)workspace;
  int rc = attn_prescale_bias(g, bias, bv, bias_s, bias_batches, s, fn);
  if (rc) return rc;
  g.bias_bstride = (bias_batches == 1) ? 0 : (int64_t)g.H * g.N * g.N;
  dim3 grid((unsigned)((total + 7) / 8 * 8));
  const unsigned mask_lds = (unsigned)(pl * g.N) * 4u;
  if (g.D <= 32)
    hipLaunchKernelGGL((attn_fwd_kernel<32, kFwdWaves, kFwdPlanes32>), grid, dim3(64 * kFwdWaves),
                       mask_lds, s, (const __bf16*)q, (const __bf16*)k, (const __bf16*)v, mask,
                       bias_s, (__bf16*)out, lse, (__bf16*)res, (const __bf16*)gate, (__bf16*)og,
                       g);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<64, kFwdWaves, kFwdPlanes64>), grid, dim3(64 * kFwdWaves),
                       mask_lds, s, (const __bf16*)q, (const __bf16*)k, (const __bf16*)v, mask,
                       bias_s, (__bf16*)out, lse, (__bf16*)res, (const __bf16*)gate, (__bf16*)og,
                       g);
  return check_launch(fn);
}

// Outer groups per backward workgroup (the run whose dBias it accumulates
// into one partial): the largest run length that keeps the whole backward in
// the fewest rounds of one workgroup per CU, i.e. minimises
// ceil(workgroups / CUs) * run.  run = 1 gives one partial per group.  The
// run length fixes the dBias summation order, so it is chosen for a fixed
// 256-CU device (MI355X) from the problem shape alone: the same inputs give
// the same bits on every device.
constexpr int64_t kBwdPlanCus = 256;
static int bwd_run_len(int64_t B, int64_t O, int64_t H, int64_t N, int64_t D) {
  const int64_t groups = (O + kBwdGroup - 1) / kBwdGroup;
  const int64_t per_run = H * bwd_key_blocks(N, D) * B;
  int64_t best = 1, best_cost = INT64_MAX;
  for (int64_t r = 1; r <= groups; ++r) {
    const int64_t wgs = per_run * ((groups + r - 1) / r);
    const int64_t cost = (wgs + kBwdPlanCus - 1) / kBwdPlanCus * r;
    if (cost <= best_cost) { best = r; best_cost = cost; }
  }
  return (int)best;
}
static int64_t bwd_runs(int64_t O, int run) {
  return ((O + kBwdGroup - 1) / kBwdGroup + run - 1) / run;
}

// Backward workspace: bf16 dQ partials [key blocks][slab planes][H,N,D] |
// f32 dBias partials [B * runs][H,N,N] (one per run of outer groups) | f32
// fragment-major bias [<=B][H,N,N] | f32 row statistics nl2, nd [B,O,H,N];
// each region 256-byte aligned.  Only the dQ partials depend on the slab.
struct BwdParts {
  __bf16* dq;
  float* db;
  float* bias_f;
  float* nl2;
  float* nd;
};

static int64_t a256(int64_t v) { return (v + 255) / 256 * 256; }

static int64_t bwd_layout(int64_t B, int64_t O, int64_t H, int64_t N, int64_t D,
                          int64_t slab_planes, char* base, BwdParts* parts) {
  const int64_t runs = bwd_runs(O, bwd_run_len(B, O, H, N, D));
  const int64_t rows = B * O * H * N;
  int64_t off = 0;
  auto take = [&](int64_t bytes) { char* p = base ? base + off : nullptr; off += a256(bytes); return p; };
  char* dq = take(bwd_key_blocks(N, D) * slab_planes * H * N * D * 2);
  char* db = take(B * runs * H * N * N * 4);
  char* bf = take(B * H * N * N * 4);
  char* nl = take(rows * 4);
  char* nd = take(rows * 4);
  if (parts) {
    parts->dq = (__bf16*)dq; parts->db = (float*)db; parts->bias_f = (float*)bf;
    parts->nl2 = (float*)nl; parts->nd = (float*)nd;
  }
  return off;
}
static int64_t bwd_full_bytes(int64_t B, int64_t O, int64_t H, int64_t N, int64_t D) {
  return bwd_layout(B, O, H, N, D, B * O, nullptr, nullptr);
}

// Slab plan for a workspace of `bytes`: every slab holds `per` consecutive
// flattened runs (the last one fewer), sized evenly so the slabs' grids
// are alike.  One slab when the full plan fits; per = 0 when not even one
// run's dQ partials fit.  Slabs change where the dQ partials live, not any
// summation order: results are bitwise equal to the one-slab plan.
struct BwdPlan {
  int run;       // outer groups per run
  int runs;      // runs per batch
  int per;       // flattened runs per slab
  int slabs;
};
static int64_t bwd_slab_planes(int64_t B, int64_t O, int per_runs, int run) {
  // Upper bound of the planes of any `per_runs` consecutive runs.
  return std::min<int64_t>(B * O, (int64_t)per_runs * run * kBwdGroup);
}
static BwdPlan bwd_plan(int64_t B, int64_t O, int64_t H, int64_t N, int64_t D, int64_t bytes) {
  BwdPlan p;
  p.run = bwd_run_len(B, O, H, N, D);
  p.runs = (int)bwd_runs(O, p.run);
  const int fr = (int)(B * p.runs);
  if (bytes >= bwd_full_bytes(B, O, H, N, D)) {
    p.per = fr;
    p.slabs = 1;
    return p;
  }
  int lo = 0, hi = fr;  // largest per whose layout fits
  while (lo < hi) {
    const int mid = (lo + hi + 1) / 2;
    if (bwd_layout(B, O, H, N, D, bwd_slab_planes(B, O, mid, p.run), nullptr, nullptr) <= bytes)
      lo = mid;
    else
      hi = mid - 1;
  }
  if (lo == 0) { p.per = 0; p.slabs = 0; return p; }
  // Among the slab sizes that fit, the one with the fewest rounds of
  // workgroups over a 256-CU device (a slab's last round may be partly
  // empty), then the largest.
  const int64_t wpr = H * bwd_key_blocks(N, D);  // workgroups per run
  int64_t best_rounds = INT64_MAX;
  for (int per = lo; per >= 1; --per) {
    const int slabs = (fr + per - 1) / per, last = fr - (slabs - 1) * per;
    const int64_t rounds = (int64_t)(slabs - 1) * ((per * wpr + kBwdPlanCus - 1) / kBwdPlanCus) +
                           (last * wpr + kBwdPlanCus - 1) / kBwdPlanCus;
    if (rounds < best_rounds) { best_rounds = rounds; p.per = per; p.slabs = slabs; }
  }
  return p;
}
// Slab s of a plan: its flattened runs and the contiguous planes they cover.
static BwdSlab bwd_slab(const BwdPlan& p, int64_t B, int64_t O, int s) {
  BwdSlab sl;
  const int fr = (int)(B * p.runs);
  sl.brun0 = s * p.per;
  sl.nbrun = std::min(fr, sl.brun0 + p.per) - sl.brun0;
  auto plane_of = [&](int frun) {  // first plane of flattened run frun (frun <= fr)
    if (frun >= fr) return B * O;
    const int64_t b = frun / p.runs, r = frun % p.runs;
    return b * O + std::min<int64_t>(O, r * p.run * kBwdGroup);
  };
  sl.plane0 = plane_of(sl.brun0);
  sl.planes = plane_of(sl.brun0 + sl.nbrun) - sl.plane0;
  return sl;
}

// Delta, row statistics and the prescaled bias in one launch (fused
// backward); attn_backward_main_impl then runs with rows_ready.
static int attn_backward_rows_impl(const AttnGeom& g, const void* dout, const void* out,
                                   const void* res, const float* lse, const void* bias,
                                   const BiasView& bv, int64_t bias_batches, void* workspace,
                                   int64_t slab_planes, hipStream_t s, const char* fn) {
  const int64_t B = g.B, O = g.O, H = g.H, N = g.N, D = g.D;
  BwdParts pt;
  bwd_layout(B, O, H, N, D, slab_planes, (char*)workspace, &pt);
  const int64_t items = B * O * N * H * (D / 8);
  const int per = 256 - 256 % (int)(D / 8);
  const int64_t delta_blocks = (items + per - 1) / per;
  const int64_t bias_items = bias_batches * H * N * N / 4;
  const int64_t blocks = delta_blocks + (bias_items + 255) / 256;
  if (blocks > INT32_MAX) return set_error(TPF_ERR_SHAPE, "%s: row grid too large", fn);
  if (res)
    hipLaunchKernelGGL(attn_bwd_rows_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, s,
                       (const __bf16*)dout, (const __bf16*)out, (const __bf16*)res, lse, pt.nl2,
                       pt.nd, items, per, (int)H, (int)N, (int)D, delta_blocks,
                       (const __bf16*)bias, pt.bias_f, bias_items, 1.f / g.scale, bv);
  else
    hipLaunchKernelGGL(attn_bwd_rows_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, s,
                       (const __bf16*)dout, (const __bf16*)out, (const __bf16*)nullptr, lse,
                       pt.nl2, pt.nd, items, per, (int)H, (int)N, (int)D, delta_blocks,
                       (const __bf16*)bias, pt.bias_f, bias_items, 1.f / g.scale, bv);
  return check_launch(fn);
}

// Row statistics and the prescaled bias from lse and delta (when the rows
// kernel has not run).
static int attn_backward_prep_impl(const AttnGeom& g, const float* lse, const float* delta,
                                   const void* bias, const BiasView& bv, int64_t bias_batches,
                                   const BwdParts& pt, hipStream_t s, const char* fn) {
  const int64_t rows = (int64_t)g.B * g.O * g.H * g.N;
  const int64_t items = bias_batches * g.H * (int64_t)g.N * g.N / 4;
  const int64_t row_blocks = (rows + 255) / 256;
  if (row_blocks + (items + 255) / 256 > INT32_MAX)
    return set_error(TPF_ERR_SHAPE, "%s: backward preparation grid too large", fn);
  hipLaunchKernelGGL(attn_bwd_prep_kernel, dim3((unsigned)(row_blocks + (items + 255) / 256)),
                     dim3(256), 0, s, lse, delta, pt.nl2, pt.nd, rows, row_blocks,
                     (const __bf16*)bias, pt.bias_f, items, (int)g.N, 1.f / g.scale, bv);
  return check_launch(fn);
}

// The reconstruction kernel over one slab (dK, dV of its planes and their
// dQ / dBias partials).
template <int DP, int MODE>
static void bwd_kernel_launch(dim3 grid, const AttnGeom& g, const void* q, const void* k,
                              const void* v, const void* dout, const float* mask, void* dk,
                              void* dv, const BwdParts& pt, const BwdPlan& plan,
                              const BwdSlab& sl, float* dtrue, hipStream_t s) {
  hipLaunchKernelGGL((attn_bwd_kernel<DP, MODE>), grid, dim3(256 * bwd_kh(DP)), 0, s,
                     (const __bf16*)q, (const __bf16*)k, (const __bf16*)v, (const __bf16*)dout,
                     pt.nl2, pt.nd, mask, pt.bias_f, (__bf16*)dk, (__bf16*)dv, pt.dq, pt.db, g,
                     plan.run, sl, dtrue);
}
static int attn_backward_slab_impl(const AttnGeom& g, const void* q, const void* k,
                                   const void* v, const void* dout, const float* mask,
                                   void* dk, void* dv, const BwdParts& pt, const BwdPlan& plan,
                                   const BwdSlab& sl, hipStream_t s, const char* fn,
                                   int mode = kBwdSR, float* dtrue = nullptr) {
  const int64_t H = g.H, N = g.N, D = g.D;
  const int64_t total = H * bwd_key_blocks(N, D) * sl.nbrun;
  if ((total + 7) / 8 * 8 > INT32_MAX)
    return set_error(TPF_ERR_SHAPE, "%s: too many backward tiles", fn);
  dim3 grid((unsigned)((total + 7) / 8 * 8));
#define TPF_BWD_LAUNCH(DP, MODE) \
  bwd_kernel_launch<DP, MODE>(grid, g, q, k, v, dout, mask, dk, dv, pt, plan, sl, dtrue, s)
  if (D <= 32) {
    if (mode == kBwdDKDV) TPF_BWD_LAUNCH(32, kBwdDKDV);
    else if (mode == kBwdDQDB) TPF_BWD_LAUNCH(32, kBwdDQDB);
    else TPF_BWD_LAUNCH(32, kBwdSR);
  } else {
    if (mode == kBwdDKDV) TPF_BWD_LAUNCH(64, kBwdDKDV);
    else if (mode == kBwdDQDB) TPF_BWD_LAUNCH(64, kBwdDQDB);
    else TPF_BWD_LAUNCH(64, kBwdSR);
  }
#undef TPF_BWD_LAUNCH
  return check_launch(fn);
}

// Folds of one slab: its planes' dQ, and (with_dbias, after the last slab)
// every dBias partial.  db_mode: 0 = f32 dBias, 1 = bf16, 2 = bf16 in
// transposed-bias order.
static int attn_backward_fold_impl(const AttnGeom& g, void* dq, void* dbias,
                                   int64_t bias_batches, const BwdParts& pt, const BwdPlan& plan,
                                   const BwdSlab& sl, bool with_dbias, hipStream_t s,
                                   const char* fn, int db_mode) {
  const int64_t H = g.H, N = g.N, D = g.D;
  const int64_t nph = sl.planes * H;
  const int64_t dq_bx = (N * (D / 8) + 255) / 256;
  const int64_t n_db = with_dbias ? (bias_batches * H * N * N / 8 + 63) / 64 : 0;
  if (n_db + dq_bx * nph > 0x7fffffff)
    return set_error(TPF_ERR_ARG, "%s: fold grid too large", fn);
  if (n_db + dq_bx * nph == 0) return TPF_OK;
  hipLaunchKernelGGL(attn_fold_kernel, dim3((unsigned)(n_db + dq_bx * nph)), dim3(256), 0, s,
                     pt.dq, (__bf16*)dq, g, (int)bwd_key_blocks(N, D), (int)dq_bx, pt.db, dbias,
                     (int)bias_batches, plan.runs, n_db, db_mode, sl.plane0, sl.planes);
  return check_launch(fn);
}

// delta_true[row] = sum over the 64-key blocks kb (ascending) of
// part[row][kb], row = (plane, head), query; part is [B, O, H, kb, N].
__global__ __launch_bounds__(256) void attn_delta_true_fold_kernel(const float* __restrict__ part,
                                                                   float* __restrict__ out,
                                                                   int64_t rows, int N, int nkb) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= rows) return;
  const int64_t ph = r / N;
  const int qq = (int)(r - ph * N);
  const float* src = part + ph * nkb * N + qq;
  float acc = src[0];
  for (int kb = 1; kb < nkb; ++kb) acc += src[(int64_t)kb * N];
  out[r] = acc;
}

extern "C" {

int64_t tpf_attn_forward_workspace_bytes(int64_t B, int64_t H, int64_t N,
                                         int64_t bias_batches) {
  (void)B;
  return bias_batches * H * N * N * 4;
}

int tpf_attn_forward_bf16(const void* q, const void* k, const void* v, const float* mask,
                          const void* bias, void* out, float* lse, void* workspace,
                          int64_t workspace_bytes, int64_t B, int64_t O, int64_t H, int64_t N,
                          int64_t D, int layout, int64_t bias_batches, double scale,
                          void* stream) {
  const char* fn = "tpf_attn_forward_bf16";
  AttnGeom g;
  int rc = make_geom(&g, B, O, H, N, D, layout, bias_batches, scale, fn);
  if (rc) return rc;
  if (!q || !k || !v || !mask || !bias || !out || !lse || !workspace)
    return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  if (workspace_bytes < tpf_attn_forward_workspace_bytes(B, H, N, bias_batches))
    return set_error(TPF_ERR_ARG, "%s: workspace too small", fn);
  return attn_forward_impl(g, q, k, v, mask, bias, dense_bias(H, N, bias_batches, layout), bias_batches,
                           out, lse, nullptr, workspace, (hipStream_t)stream, fn);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free forward: the prescaled-bias scratch lives in a file-scope
// device array instead of a caller workspace.  Each GPU holds its own copy
// of the array (at its own address) until the process ends; its address is
// looked up once per device with that device current and kept per device.
// Every call on a GPU shares that GPU's array: calls that overlap on one GPU
// (two streams) race on it.  The prescale kernel writes every scratch word
// the forward kernel then reads, so nothing needs clearing between calls.
// ---------------------------------------------------------------------------
static constexpr int64_t kNoAllocScratchBytes = 16ll << 20;  // 4M f32 bias values
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / 4];
static constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];

static int noalloc_scratch(void** out, const char* fn) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(TPF_ERR_LAUNCH, "%s: no current HIP device (or device index >= %d)", fn,
                     kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(TPF_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s",
                       fn, dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return TPF_OK;
}

extern "C" {

int tpf_attn_forward_noalloc_bf16(const void* q, const void* k, const void* v, const float* mask,
                                  const void* bias, void* out, float* lse, int64_t B, int64_t O,
                                  int64_t H, int64_t N, int64_t D, int layout,
                                  int64_t bias_batches, double scale, void* stream) {
  const char* fn = "tpf_attn_forward_noalloc_bf16";
  AttnGeom g;
  int rc = make_geom(&g, B, O, H, N, D, layout, bias_batches, scale, fn);
  if (rc) return rc;
  if (!q || !k || !v || !mask || !bias || !out || !lse)
    return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  const int64_t need = tpf_attn_forward_workspace_bytes(B, H, N, bias_batches);
  if (need > kNoAllocScratchBytes)
    return set_error(TPF_ERR_SHAPE,
                     "%s: bias_batches*H*N*N = %lld exceeds the static scratch of %lld f32 values "
                     "(use tpf_attn_forward_bf16 with a workspace)",
                     fn, (long long)(need / 4), (long long)(kNoAllocScratchBytes / 4));
  void* ws = nullptr;
  if ((rc = noalloc_scratch(&ws, fn))) return rc;
  return attn_forward_impl(g, q, k, v, mask, bias, dense_bias(H, N, bias_batches, layout), bias_batches,
                           out, lse, nullptr, ws, (hipStream_t)stream, fn);
}

int tpf_attn_forward_shadow_bf16(const void* q, const void* k, const void* v, const float* mask,
                                 const void* bias, void* out, float* lse, void* residual,
                                 void* workspace, int64_t workspace_bytes, int64_t B, int64_t O,
                                 int64_t H, int64_t N, int64_t D, int layout,
                                 int64_t bias_batches, double scale, void* stream) {
  const char* fn = "tpf_attn_forward_shadow_bf16";
  AttnGeom g;
  int rc = make_geom(&g, B, O, H, N, D, layout, bias_batches, scale, fn);
  if (rc) return rc;
  if (!q || !k || !v || !mask || !bias || !out || !lse || !residual || !workspace)
    return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  if (workspace_bytes < tpf_attn_forward_workspace_bytes(B, H, N, bias_batches))
    return set_error(TPF_ERR_ARG, "%s: workspace too small", fn);
  return attn_forward_impl(g, q, k, v, mask, bias, dense_bias(H, N, bias_batches, layout), bias_batches,
                           out, lse, residual, workspace, (hipStream_t)stream, fn);
}

static int attn_delta_launch(const void* dout, const void* out, const void* res, float* delta,
                             int64_t B, int64_t O, int64_t H, int64_t N, int64_t D,
                             void* stream, const char* fn) {
  if (!dout || !out || !delta) return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  if (B < 1 || O < 1 || H < 1 || N < 1 || D < 8 || D > 64 || D % 8)
    return set_error(TPF_ERR_SHAPE, "%s: bad shape", fn);
  const int64_t items = B * O * N * H * (D / 8);
  const int per = 256 - 256 % (int)(D / 8);
  const dim3 grid((unsigned)((items + per - 1) / per));
  if (res)
    hipLaunchKernelGGL(attn_delta_kernel<true>, grid, dim3(256), 0, (hipStream_t)stream,
                       (const __bf16*)dout, (const __bf16*)out, (const __bf16*)res, delta, items,
                       per, (int)H, (int)N, (int)D);
  else
    hipLaunchKernelGGL(attn_delta_kernel<false>, grid, dim3(256), 0, (hipStream_t)stream,
                       (const __bf16*)dout, (const __bf16*)out, (const __bf16*)nullptr, delta,
                       items, per, (int)H, (int)N, (int)D);
  return check_launch(fn);
}

int tpf_attn_delta_bf16(const void* dout, const void* out, float* delta, int64_t B, int64_t O,
                        int64_t H, int64_t N, int64_t D, void* stream) {
  return attn_delta_launch(dout, out, nullptr, delta, B, O, H, N, D, stream,
                           "tpf_attn_delta_bf16");
}

int tpf_attn_delta_shadow_bf16(const void* dout, const void* out, const void* residual,
                               float* delta, int64_t B, int64_t O, int64_t H, int64_t N,
                               int64_t D, void* stream) {
  if (!residual) return set_error(TPF_ERR_ARG, "tpf_attn_delta_shadow_bf16: null pointer");
  return attn_delta_launch(dout, out, residual, delta, B, O, H, N, D, stream,
                           "tpf_attn_delta_shadow_bf16");
}

int64_t tpf_attn_backward_workspace_bytes(int64_t B, int64_t O, int64_t H, int64_t N,
                                          int64_t D) {
  return bwd_full_bytes(B, O, H, N, D);
}

int64_t tpf_attn_backward_workspace_bytes_budget(int64_t B, int64_t O, int64_t H, int64_t N,
                                                 int64_t D, int64_t budget_bytes) {
  if (B < 1 || O < 1 || H < 1 || N < 1 || D < 1) return -1;
  const int64_t full = bwd_full_bytes(B, O, H, N, D);
  if (budget_bytes >= full) return full;
  BwdPlan p = bwd_plan(B, O, H, N, D, budget_bytes);
  // Below the one-run minimum the minimum is returned (it exceeds the budget).
  const int per = p.per > 0 ? p.per : 1;
  const int slabs = (int)((B * p.runs + per - 1) / per);
  const int even = (int)((B * p.runs + slabs - 1) / slabs);
  return bwd_layout(B, O, H, N, D, bwd_slab_planes(B, O, even, p.run), nullptr, nullptr);
}

int tpf_attn_backward_slab_count(int64_t B, int64_t O, int64_t H, int64_t N, int64_t D,
                                 int64_t workspace_bytes) {
  if (B < 1 || O < 1 || H < 1 || N < 1 || D < 1) return -1;
  return bwd_plan(B, O, H, N, D, workspace_bytes).slabs;
}

// full_only: the split main / finish stages need the one-slab plan.
static int attn_bwd_prepare(AttnGeom* g, BwdPlan* plan, const char* fn, const void* q,
                            const void* k, const void* v, const void* dout, const float* lse,
                            const float* delta, const float* mask, const void* bias,
                            const void* workspace, int64_t workspace_bytes, int64_t B, int64_t O,
                            int64_t H, int64_t N, int64_t D, int layout, int64_t bias_batches,
                            double scale, bool full_only) {
  int rc = make_geom(g, B, O, H, N, D, layout, bias_batches, scale, fn);
  if (rc) return rc;
  if (!q || !k || !v || !dout || !lse || !delta || !mask || !bias || !workspace)
    return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  const int64_t need = full_only ? bwd_full_bytes(B, O, H, N, D)
                                 : tpf_attn_backward_workspace_bytes_budget(B, O, H, N, D, 0);
  if (workspace_bytes < need)
    return set_error(TPF_ERR_ARG, "%s: workspace %lld < required %lld", fn,
                     (long long)workspace_bytes, (long long)need);
  *plan = bwd_plan(B, O, H, N, D, workspace_bytes);
  if (plan->slabs < 1) return set_error(TPF_ERR_ARG, "%s: workspace too small", fn);
  return TPF_OK;
}

// Stage 1 of the backward: row statistics and bias preparation, then the
// single-reconstruction kernel writing dK, dV and the dQ / dBias partials.
int tpf_attn_backward_main_bf16(const void* q, const void* k, const void* v, const void* dout,
                                const float* lse, const float* delta, const float* mask,
                                const void* bias, void* dk, void* dv, void* workspace,
                                int64_t workspace_bytes, int64_t B, int64_t O, int64_t H,
                                int64_t N, int64_t D, int layout, int64_t bias_batches,
                                double scale, void* stream) {
  const char* fn = "tpf_attn_backward_main_bf16";
  AttnGeom g;
  BwdPlan plan;
  int rc = attn_bwd_prepare(&g, &plan, fn, q, k, v, dout, lse, delta, mask, bias, workspace,
                            workspace_bytes, B, O, H, N, D, layout, bias_batches, scale, true);
  if (rc) return rc;
  if (!dk || !dv) return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  hipStream_t s = (hipStream_t)stream;
  BwdParts pt;
  bwd_layout(B, O, H, N, D, B * O, (char*)workspace, &pt);
  if ((rc = attn_backward_prep_impl(g, lse, delta, bias, dense_bias(H, N, bias_batches, layout),
                                    bias_batches, pt, s, fn)))
    return rc;
  return attn_backward_slab_impl(g, q, k, v, dout, mask, dk, dv, pt, plan, bwd_slab(plan, B, O, 0),
                                 s, fn);
}

// Stage 2 of the backward: fixed-order folds of the dQ and dBias partials.
int tpf_attn_backward_finish_bf16(void* dq, void* dbias, const void* workspace, int64_t B,
                                  int64_t O, int64_t H, int64_t N, int64_t D, int layout,
                                  int64_t bias_batches, double scale, void* stream) {
  const char* fn = "tpf_attn_backward_finish_bf16";
  AttnGeom g;
  int rc = make_geom(&g, B, O, H, N, D, layout, bias_batches, scale, fn);
  if (rc) return rc;
  if (!dq || !dbias || !workspace) return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  const int db_mode = !(layout & TPF_DBIAS_BF16) ? 0 : (layout & TPF_BIAS_TRANSPOSED) ? 2 : 1;
  const BwdPlan plan = bwd_plan(B, O, H, N, D, INT64_MAX);
  BwdParts pt;
  bwd_layout(B, O, H, N, D, B * O, (char*)workspace, &pt);
  return attn_backward_fold_impl(g, dq, dbias, bias_batches, pt, plan, bwd_slab(plan, B, O, 0),
                                 true, (hipStream_t)stream, fn, db_mode);
}

// Every slab of a plan: reconstruction, then that slab's dQ fold; the dBias
// fold joins the last slab's fold launch.
static int attn_backward_slabs(const AttnGeom& g, const BwdPlan& plan, const void* q,
                               const void* k, const void* v, const void* dout, const float* mask,
                               void* dq, void* dk, void* dv, void* dbias, int64_t bias_batches,
                               const BwdParts& pt, hipStream_t s, const char* fn, int db_mode,
                               int mode = kBwdSR) {
  for (int i = 0; i < plan.slabs; ++i) {
    const BwdSlab sl = bwd_slab(plan, g.B, g.O, i);
    int rc = attn_backward_slab_impl(g, q, k, v, dout, mask, dk, dv, pt, plan, sl, s, fn, mode);
    if (rc) return rc;
    rc = attn_backward_fold_impl(g, dq, dbias, bias_batches, pt, plan, sl, i + 1 == plan.slabs, s,
                                 fn, db_mode);
    if (rc) return rc;
  }
  return TPF_OK;
}

int tpf_attn_backward_bf16(const void* q, const void* k, const void* v, const void* dout,
                           const float* lse, const float* delta, const float* mask,
                           const void* bias, void* dq, void* dk, void* dv, void* dbias,
                           void* workspace, int64_t workspace_bytes, int64_t B, int64_t O,
                           int64_t H, int64_t N, int64_t D, int layout, int64_t bias_batches,
                           double scale, void* stream) {
  const char* fn = "tpf_attn_backward_bf16";
  AttnGeom g;
  BwdPlan plan;
  int rc = attn_bwd_prepare(&g, &plan, fn, q, k, v, dout, lse, delta, mask, bias, workspace,
                            workspace_bytes, B, O, H, N, D, layout, bias_batches, scale, false);
  if (rc) return rc;
  if (!dq || !dk || !dv || !dbias) return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  hipStream_t s = (hipStream_t)stream;
  BwdParts pt;
  bwd_layout(B, O, H, N, D, bwd_slab_planes(B, O, plan.per, plan.run), (char*)workspace, &pt);
  if ((rc = attn_backward_prep_impl(g, lse, delta, bias, dense_bias(H, N, bias_batches, layout),
                                    bias_batches, pt, s, fn)))
    return rc;
  const int db_mode = !(layout & TPF_DBIAS_BF16) ? 0 : (layout & TPF_BIAS_TRANSPOSED) ? 2 : 1;
  return attn_backward_slabs(g, plan, q, k, v, dout, mask, dq, dk, dv, dbias, bias_batches, pt, s,
                             fn, db_mode);
}

// Whole backward from the forward's outputs: delta (with the shadow residual
// when given), row statistics and bias preparation in one launch, then the
// reconstruction kernel and the folds, slab by slab.
int tpf_attn_backward_fused_bf16(const void* q, const void* k, const void* v, const void* dout,
                                 const void* out, const void* residual, const float* lse,
                                 const float* mask, const void* bias, void* dq, void* dk,
                                 void* dv, void* dbias, void* workspace, int64_t workspace_bytes,
                                 int64_t B, int64_t O, int64_t H, int64_t N, int64_t D,
                                 int layout, int64_t bias_batches, double scale, void* stream) {
  const char* fn = "tpf_attn_backward_fused_bf16";
  AttnGeom g;
  BwdPlan plan;
  // delta is computed in the workspace: the prepare check's delta slot gets lse.
  int rc = attn_bwd_prepare(&g, &plan, fn, q, k, v, dout, lse, lse, mask, bias, workspace,
                            workspace_bytes, B, O, H, N, D, layout, bias_batches, scale, false);
  if (rc) return rc;
  if (!out || !dq || !dk || !dv || !dbias) return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  const BiasView bv = dense_bias(H, N, bias_batches, layout);
  hipStream_t s = (hipStream_t)stream;
  const int64_t slab_planes = bwd_slab_planes(B, O, plan.per, plan.run);
  rc = attn_backward_rows_impl(g, dout, out, residual, lse, bias, bv, bias_batches, workspace,
                               slab_planes, s, fn);
  if (rc) return rc;
  BwdParts pt;
  bwd_layout(B, O, H, N, D, slab_planes, (char*)workspace, &pt);
  const int db_mode = !(layout & TPF_DBIAS_BF16) ? 0 : (layout & TPF_BIAS_TRANSPOSED) ? 2 : 1;
  return attn_backward_slabs(g, plan, q, k, v, dout, mask, dq, dk, dv, dbias, bias_batches, pt, s,
                             fn, db_mode);
}

// ---------------------------------------------------------------------------
// Split backward route of direct callers: the reconstruction kernel in a
// mode that produces one half of the gradients from caller-supplied lse and
// delta.  dK / dV (with optional delta_true = sum_k P dP per query row, from
// per-64-key-block f32 partials folded in ascending block order); dQ and the
// per-batch f32 dBias through the same partials and folds as the single-
// reconstruction route, so each half is bitwise that route's output.
// ---------------------------------------------------------------------------
static int64_t dkdv_layout(int64_t B, int64_t O, int64_t H, int64_t N, int64_t bias_batches,
                           char* base, BwdParts* parts) {
  const int64_t rows = B * O * H * N;
  int64_t off = 0;
  auto take = [&](int64_t bytes) { char* p = base ? base + off : nullptr; off += a256(bytes); return p; };
  char* bf = take(bias_batches * H * N * N * 4);
  char* nl = take(rows * 4);
  char* nd = take(rows * 4);
  if (parts) {
    parts->dq = nullptr; parts->db = nullptr; parts->bias_f = (float*)bf;
    parts->nl2 = (float*)nl; parts->nd = (float*)nd;
  }
  return off;
}

int64_t tpf_attn_dkdv_workspace_bytes(int64_t B, int64_t O, int64_t H, int64_t N, int64_t D,
                                      int64_t bias_batches) {
  (void)D;
  if (B < 1 || O < 1 || H < 1 || N < 1 || bias_batches < 1) return -1;
  return dkdv_layout(B, O, H, N, bias_batches, nullptr, nullptr);
}

int64_t tpf_attn_dkdv_delta_true_partial_elements(int64_t B, int64_t O, int64_t H, int64_t N) {
  if (B < 1 || O < 1 || H < 1 || N < 1) return -1;
  return B * O * H * N * ((N + 63) / 64);
}

int tpf_attn_dkdv_bf16(const void* q, const void* k, const void* v, const void* dout,
                       const float* lse, const float* delta, const float* mask, const void* bias,
                       void* dk, void* dv, float* delta_true_partials, float* delta_true,
                       void* workspace, int64_t workspace_bytes, int64_t B, int64_t O, int64_t H,
                       int64_t N, int64_t D, int layout, int64_t bias_batches, double scale,
                       void* stream) {
  const char* fn = "tpf_attn_dkdv_bf16";
  AttnGeom g;
  int rc = make_geom(&g, B, O, H, N, D, layout, bias_batches, scale, fn);
  if (rc) return rc;
  if (layout & TPF_DBIAS_BF16) return set_error(TPF_ERR_ARG, "%s: TPF_DBIAS_BF16 has no meaning here", fn);
  if (!q || !k || !v || !dout || !lse || !delta || !mask || !bias || !dk || !dv || !workspace)
    return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  if ((delta_true_partials == nullptr) != (delta_true == nullptr))
    return set_error(TPF_ERR_ARG, "%s: delta_true and its partials are given together", fn);
  if (delta_true_partials && ((uintptr_t)delta_true_partials % 16))
    return set_error(TPF_ERR_ARG, "%s: delta_true partials must be 16-byte aligned", fn);
  if (workspace_bytes < tpf_attn_dkdv_workspace_bytes(B, O, H, N, D, bias_batches))
    return set_error(TPF_ERR_ARG, "%s: workspace too small", fn);
  hipStream_t s = (hipStream_t)stream;
  BwdParts pt;
  dkdv_layout(B, O, H, N, bias_batches, (char*)workspace, &pt);
  if ((rc = attn_backward_prep_impl(g, lse, delta, bias, dense_bias(H, N, bias_batches, layout),
                                    bias_batches, pt, s, fn)))
    return rc;
  const BwdPlan plan = bwd_plan(B, O, H, N, D, INT64_MAX);
  for (int i = 0; i < plan.slabs; ++i)
    if ((rc = attn_backward_slab_impl(g, q, k, v, dout, mask, dk, dv, pt, plan,
                                      bwd_slab(plan, B, O, i), s, fn, kBwdDKDV,
                                      delta_true_partials)))
      return rc;
  if (delta_true) {
    const int64_t rows = B * O * H * N;
    hipLaunchKernelGGL(attn_delta_true_fold_kernel, dim3((unsigned)((rows + 255) / 256)),
                       dim3(256), 0, s, delta_true_partials, delta_true, rows, (int)N,
                       (int)((N + 63) / 64));
    return check_launch(fn);
  }
  return TPF_OK;
}

int64_t tpf_attn_dq_dbias_workspace_bytes(int64_t B, int64_t O, int64_t H, int64_t N, int64_t D) {
  if (B < 1 || O < 1 || H < 1 || N < 1 || D < 1) return -1;
  return bwd_full_bytes(B, O, H, N, D);
}

int tpf_attn_dq_dbias_bf16(const void* q, const void* k, const void* v, const void* dout,
                           const float* lse, const float* delta, const float* mask,
                           const void* bias, void* dq, float* dbias, void* workspace,
                           int64_t workspace_bytes, int64_t B, int64_t O, int64_t H, int64_t N,
                           int64_t D, int layout, int64_t bias_batches, double scale,
                           void* stream) {
  const char* fn = "tpf_attn_dq_dbias_bf16";
  AttnGeom g;
  BwdPlan plan;
  int rc = attn_bwd_prepare(&g, &plan, fn, q, k, v, dout, lse, delta, mask, bias, workspace,
                            workspace_bytes, B, O, H, N, D, layout, bias_batches, scale, false);
  if (rc) return rc;
  if (layout & TPF_DBIAS_BF16) return set_error(TPF_ERR_ARG, "%s: dbias is f32 here", fn);
  if (!dq || !dbias) return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  hipStream_t s = (hipStream_t)stream;
  BwdParts pt;
  bwd_layout(B, O, H, N, D, bwd_slab_planes(B, O, plan.per, plan.run), (char*)workspace, &pt);
  if ((rc = attn_backward_prep_impl(g, lse, delta, bias, dense_bias(H, N, bias_batches, layout),
                                    bias_batches, pt, s, fn)))
    return rc;
  // dBias per batch item (B output batches), whatever the bias's batch count.
  return attn_backward_slabs(g, plan, q, k, v, dout, mask, dq, nullptr, nullptr, dbias, B, pt, s,
                             fn, 0, kBwdDQDB);
}

// ---------------------------------------------------------------------------
// Pair-row entry points: the attention core of the triangle-attention module.
// q, k, v come as head-major planes qkv[part][b][i][h][j][d] (written so by
// the projection, tpf_pair_projection_bf16), the gate and the pair bias as
// rows rest[b][i][j][rest_pitch] = gate (H*D) | bias (H) | pad, and the
// gradients go to rows dproj[b][i][j][dproj_pitch] = q | k | v | gate | bias
// | pad.  Row (b, i, j) is pair (i, j); plane i attends over j.
// ---------------------------------------------------------------------------

static int pair_geom(AttnGeom* g, BiasView* bv, int64_t rest_pitch, int64_t dproj_pitch,
                     int flags, int64_t B, int64_t N, int64_t H, int64_t D, double scale,
                     const char* fn) {
  if (flags & ~(TPF_PAIR_BIAS_TRANSPOSED | TPF_PAIR_OG_TRANSPOSED))
    return set_error(TPF_ERR_ARG, "%s: unknown flags 0x%x", fn, flags);
  int rc = make_geom(g, B, N, H, N, D, 0, B, scale, fn);  // head-major q / k / v
  if (rc) return rc;
  const int transpose_bias = (flags & TPF_PAIR_BIAS_TRANSPOSED) != 0;
  g->og_t = (flags & TPF_PAIR_OG_TRANSPOSED) != 0;
  const int64_t hc = H * D;
  if (rest_pitch < hc + H || rest_pitch % 8 != 0)
    return set_error(TPF_ERR_SHAPE, "%s: rest pitch %lld must be a multiple of 8 >= H*D + H", fn,
                     (long long)rest_pitch);
  if (dproj_pitch && (dproj_pitch < 4 * hc + H || dproj_pitch % 8 != 0))
    return set_error(TPF_ERR_SHAPE, "%s: dproj pitch %lld must be a multiple of 8 >= 4*H*D + H",
                     fn, (long long)dproj_pitch);
  if (H > 16) return set_error(TPF_ERR_SHAPE, "%s: H=%lld exceeds 16", fn, (long long)H);
  // Gradients into the projection-gradient rows.
  g->o_row = dproj_pitch;
  g->o_head = D;
  g->o_plane = N * dproj_pitch;
  g->gate_pitch = rest_pitch;
  bv->s_bb = N * N * rest_pitch;
  bv->s_h = 1;
  bv->s_q = transpose_bias ? rest_pitch : N * rest_pitch;
  bv->s_k = transpose_bias ? N * rest_pitch : rest_pitch;
  bv->H = (int)H;
  return TPF_OK;
}

int64_t tpf_attn_pair_forward_workspace_bytes(int64_t B, int64_t N, int64_t H) {
  return B * H * N * N * 4;
}

int tpf_attn_pair_forward_bf16(const void* qkv, const void* rest, int64_t rest_pitch,
                               const float* mask, int flags, void* o, float* lse, void* og,
                               void* residual, void* workspace, int64_t workspace_bytes,
                               int64_t B, int64_t N, int64_t H, int64_t D, double scale,
                               void* stream) {
  const char* fn = "tpf_attn_pair_forward_bf16";
  AttnGeom g;
  BiasView bv;
  int rc = pair_geom(&g, &bv, rest_pitch, 0, flags, B, N, H, D, scale, fn);
  if (rc) return rc;
  if (!qkv || !rest || !mask || !o || !lse || !og || !workspace)
    return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  if (((uintptr_t)qkv | (uintptr_t)rest | (uintptr_t)o | (uintptr_t)og) % 16)
    return set_error(TPF_ERR_ARG, "%s: qkv, rest, o and og must be 16-byte aligned", fn);
  if (workspace_bytes < tpf_attn_pair_forward_workspace_bytes(B, N, H))
    return set_error(TPF_ERR_ARG, "%s: workspace too small", fn);
  const int64_t hc = H * D, part = B * N * H * N * D;
  const __bf16* q = (const __bf16*)qkv;
  const __bf16* r = (const __bf16*)rest;
  hipStream_t s = (hipStream_t)stream;
  if (residual && (uintptr_t)residual % 16)
    return set_error(TPF_ERR_ARG, "%s: residual must be 16-byte aligned", fn);
  // The forward's epilogue applies the output gate (og = o * sigmoid(g)).
  return attn_forward_impl(g, q, q + part, q + 2 * part, mask, r + hc, bv, B, o, lse, residual,
                           workspace, s, fn, r, og);
}

// Workspace: the attention backward's, then d_o [B, N, N, H*D] bf16 and
// delta [B, N, H, N] f32.
int64_t tpf_attn_pair_backward_workspace_bytes(int64_t B, int64_t N, int64_t H, int64_t D) {
  return bwd_full_bytes(B, N, H, N, D) + a256(B * N * N * H * D * 2) +
         a256(B * N * H * N * 4);
}

}  // extern "C"

namespace tpf {
// The pair-row backward from d_og (d_og set) or, fused, from the module's
// upstream gradient dout [R, C] and W_o [C, H*D] (d_og null): the d_og
// product then runs with the gate backward in its epilogue
// (rowgemm_gate_bwd) and d_og never reaches memory.
static int pair_backward_impl(const void* qkv, const void* rest, int64_t rest_pitch,
                              const float* mask, int flags, const void* o, const float* lse,
                              const void* residual, const void* d_og, const void* dout,
                              const void* w_o, int64_t C, void* dproj, int64_t dproj_pitch,
                              void* workspace, int64_t workspace_bytes, int64_t B, int64_t N,
                              int64_t H, int64_t D, double scale, void* stream, const char* fn) {
  AttnGeom g;
  BiasView bv;
  if (dproj_pitch < 1) return set_error(TPF_ERR_SHAPE, "%s: dproj pitch must be positive", fn);
  int rc = pair_geom(&g, &bv, rest_pitch, dproj_pitch, flags, B, N, H, D, scale, fn);
  if (rc) return rc;
  if (!qkv || !rest || !mask || !o || !lse || !(d_og || (dout && w_o)) || !dproj || !workspace)
    return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  if (((uintptr_t)qkv | (uintptr_t)rest | (uintptr_t)o | (uintptr_t)d_og | (uintptr_t)dout |
       (uintptr_t)w_o | (uintptr_t)dproj) % 16)
    return set_error(TPF_ERR_ARG, "%s: qkv, rest, o, the gradients and dproj must be 16-byte "
                     "aligned", fn);
  if (workspace_bytes < tpf_attn_pair_backward_workspace_bytes(B, N, H, D))
    return set_error(TPF_ERR_ARG, "%s: workspace too small", fn);
  const int64_t hc = H * D, part = B * N * H * N * D;
  const int64_t main_bytes = bwd_full_bytes(B, N, H, N, D);
  __bf16* d_o = (__bf16*)((char*)workspace + main_bytes);
  float* delta = (float*)((char*)workspace + main_bytes + a256(B * N * N * hc * 2));
  const __bf16* q = (const __bf16*)qkv;
  const __bf16* r = (const __bf16*)rest;
  __bf16* dp = (__bf16*)dproj;
  hipStream_t s = (hipStream_t)stream;
  const int64_t items = B * N * N * (hc / 8);
  if (items >= (int64_t)kBufOOB - 256)
    return set_error(TPF_ERR_SHAPE, "%s: %lld gate chunks exceed 2^31", fn, (long long)items);
  const int per = 256 - 256 % (int)(D / 8);
  const dim3 ggrid((unsigned)((items + per - 1) / per));
  const FastDiv fN = make_fastdiv((uint32_t)N), fhc8 = make_fastdiv((uint32_t)(hc / 8));
  if (!d_og) {
    if ((rc = rowgemm_gate_bwd((const __bf16*)dout, (const __bf16*)w_o, C, (const __bf16*)o,
                               (const __bf16*)residual, r, rest_pitch, d_o, delta, dp + 3 * hc,
                               dproj_pitch, B, N, H, D, g.og_t, s, fn)))
      return rc;
  } else if (residual)
    hipLaunchKernelGGL(attn_gate_bwd_kernel<true>, ggrid, dim3(256), 0, s, (const __bf16*)d_og,
                       (const __bf16*)o, (const __bf16*)residual, r, rest_pitch, d_o, delta,
                       dp + 3 * hc, dproj_pitch, items, per, fN, (int)H, (int)D, fhc8, g.og_t);
  else
    hipLaunchKernelGGL(attn_gate_bwd_kernel<false>, ggrid, dim3(256), 0, s, (const __bf16*)d_og,
                       (const __bf16*)o, (const __bf16*)nullptr, r, rest_pitch, d_o, delta,
                       dp + 3 * hc, dproj_pitch, items, per, fN, (int)H, (int)D, fhc8, g.og_t);
  if (d_og && (rc = check_launch(fn))) return rc;
  BwdParts pt;
  bwd_layout(B, N, H, N, D, B * N, (char*)workspace, &pt);
  const BwdPlan plan = bwd_plan(B, N, H, N, D, INT64_MAX);
  if ((rc = attn_backward_prep_impl(g, lse, delta, r + hc, bv, B, pt, s, fn))) return rc;
  if ((rc = attn_backward_slab_impl(g, q, q + part, q + 2 * part, d_o, mask, dp + hc, dp + 2 * hc,
                                    pt, plan, bwd_slab(plan, B, N, 0), s, fn)))
    return rc;
  const int64_t nph = B * N * H;
  hipLaunchKernelGGL(attn_dq_reduce_kernel,
                     dim3((unsigned)((N * (D / 8) + 255) / 256), (unsigned)(nph < 65535 ? nph : 65535)),
                     dim3(256), 0, s, pt.dq, dp, g, (int)bwd_key_blocks(N, D));
  if ((rc = check_launch(fn))) return rc;
  const int64_t groups = plan.runs;
  const dim3 db_grid((unsigned)(B * N * N / 512));
  hipLaunchKernelGGL(attn_dbias_pair_kernel, db_grid, dim3(256), 0, s, pt.db, (int)B, (int)B,
                     (int)groups, (int)H, (int)N, dp, dproj_pitch, 4 * hc,
                     (flags & TPF_PAIR_BIAS_TRANSPOSED) != 0);
  return check_launch(fn);
}
}  // namespace tpf

extern "C" {

int tpf_attn_pair_backward_bf16(const void* qkv, const void* rest, int64_t rest_pitch,
                                const float* mask, int flags, const void* o, const float* lse,
                                const void* residual, const void* d_og, void* dproj,
                                int64_t dproj_pitch, void* workspace, int64_t workspace_bytes,
                                int64_t B, int64_t N, int64_t H, int64_t D, double scale,
                                void* stream) {
  const char* fn = "tpf_attn_pair_backward_bf16";
  if (!d_og) return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  return pair_backward_impl(qkv, rest, rest_pitch, mask, flags, o, lse, residual, d_og, nullptr,
                            nullptr, 0, dproj, dproj_pitch, workspace, workspace_bytes, B, N, H,
                            D, scale, stream, fn);
}

int tpf_attn_pair_backward_dout_supported(int64_t C, int64_t H, int64_t D) {
  return rowgemm_gate_supported(C, H, D) ? 1 : 0;
}

int tpf_attn_pair_backward_dout_bf16(const void* qkv, const void* rest, int64_t rest_pitch,
                                     const float* mask, int flags, const void* o,
                                     const float* lse, const void* residual, const void* dout,
                                     const void* w_o, int64_t C, void* dproj, int64_t dproj_pitch,
                                     void* workspace, int64_t workspace_bytes, int64_t B,
                                     int64_t N, int64_t H, int64_t D, double scale, void* stream) {
  const char* fn = "tpf_attn_pair_backward_dout_bf16";
  if (!dout || !w_o) return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  if (!rowgemm_gate_supported(C, H, D))
    return set_error(TPF_ERR_SHAPE, "%s: no fused instance for C=%lld H=%lld D=%lld", fn,
                     (long long)C, (long long)H, (long long)D);
  return pair_backward_impl(qkv, rest, rest_pitch, mask, flags, o, lse, residual, nullptr, dout,
                            w_o, C, dproj, dproj_pitch, workspace, workspace_bytes, B, N, H, D,
                            scale, stream, fn);
}

}  // extern "C"
