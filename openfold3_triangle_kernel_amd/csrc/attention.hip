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
//          plane stride is always H*N*D.
//   mask   [B, O, N] f32 additive.    bias [Bb, H, N, N] bf16, Bb in {1, B}.
//   out    [B, O, N, H, D] bf16.      lse / delta [B, O, H, N] f32.
// N must be a multiple of 64 (the host pads) and D a multiple of 8, D <= 64.
#include "common.hpp"
#include "tpf_status.hpp"

namespace tpf {

struct AttnGeom {
  int B, O, H, N, D;
  int64_t s_row, s_head;   // Q/K/V/dQ/dK/dV element strides
  int64_t bias_bstride;    // elements between bias batches (0 = broadcast)
  float scale;             // softmax scale (1/sqrt(D_true))
};

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
                                                                 float inv_scale) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (block, j, lane)
  if (i >= items) return;
  const int lane = (int)(i & 63), j = (int)((i >> 6) & 3);
  const int64_t blk = i >> 8;
  const int nkb = N / 32;
  const int kb = (int)(blk % nkb);
  const int64_t hq = blk / nkb;            // (bb * H + h) * (N / 32) + qb
  const int qb = (int)(hq % (N / 32));
  const int64_t bh = hq / (N / 32);
  const int ql = lane & 31, hl = lane >> 5;
  const __bf16* src = bias + (bh * N + qb * 32 + ql) * (int64_t)N + kb * 32 + 8 * j + 4 * hl;
  bf16x4 v = ld4(src);
  f32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = bf2f(v[e]) * inv_scale;
  *reinterpret_cast<f32x4*>(out + i * 4) = o;
}

// ---------------------------------------------------------------------------
// Forward.  One workgroup = 4 waves = 128 queries of one plane; each wave owns
// 32 queries and walks all keys in 64-key tiles staged in LDS (double
// buffered, fetched into registers one tile ahead).  Scores are produced
// transposed (S^T = K Q^T) so each lane owns one query column: row max / sum
// need only the lane^32 exchange, and the C-layout P^T block is fed directly
// as the B operand of O^T += V^T P^T.
// Softmax works on 32-key blocks.  The S^T accumulator is seeded with the
// prescaled bias (loaded one block ahead), scores stay in raw units
// r = <Q,K> + bias_s (+ mask / scale), and p = exp2(r * c2 - m * c2) with
// c2 = scale * log2(e): one FMA + one exp per score.  Row sums use packed
// bf16 dot products of the rounded P (the values that also enter P V).  The
// running max is raised only when a block exceeds it by more than 8 in log2
// units (p <= 256 otherwise), so the O rescale is rare.
// ---------------------------------------------------------------------------
template <int DP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DP == 32 ? 4 : 2, 8))) void attn_fwd_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k,
    const __bf16* __restrict__ v, const float* __restrict__ mask,
    const float* __restrict__ bias_s, __bf16* __restrict__ out,
    float* __restrict__ lse, AttnGeom g) {
  constexpr int KP = DP + 8;     // K tile pitch (bf16): conflict-free 16-byte reads
  constexpr int VP = 64 + 4;     // V^T tile pitch (bf16): conflict-free 8-byte reads
  constexpr int KITEMS = 64 * DP / 8;   // 16-byte K chunks per tile (one per thread)
  constexpr int VITEMS = 16 * DP / 8;   // (4-key group, 8-channel chunk) V items
  __shared__ __attribute__((aligned(16))) __bf16 Ks[2][64 * KP];
  __shared__ __attribute__((aligned(16))) __bf16 Vt[2][DP * VP];

  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int ql = lane & 31, hl = lane >> 5;
  const int N = g.N, D = g.D;
  TileId tile;
  const int qtiles = (N + 127) / 128;
  if (!xcd_tile((int64_t)qtiles * g.H * g.B * g.O, qtiles, g.B * g.O, &tile)) return;
  const int h = tile.h, plane = tile.plane;
  const int b = plane / g.O;
  const int q0 = tile.qt * 128 + w * 32;
  const bool active = q0 < N;
  const int qi = q0 + ql;

  const int64_t plane_off = (int64_t)plane * g.H * N * D + (int64_t)h * g.s_head;
  const __bf16* qb = q + plane_off;
  const __bf16* kb = k + plane_off;
  const __bf16* vb = v + plane_off;
  const float* mrow = mask + (int64_t)plane * N;
  // Fragment-major bias blocks of this wave's 32 queries: 1024 floats per
  // 32-key block, lane-interleaved.
  const float* brow = bias_s + (int64_t)b * g.bias_bstride +
                      ((int64_t)h * (N / 32) + (active ? q0 / 32 : 0)) * (int64_t)(N / 32) * 1024 + lane * 4;
  const float c2 = g.scale * kLog2e;
  const float inv_scale = 1.f / g.scale;
  const float thr = 8.f / c2;  // lazy-rescale threshold in raw units

  bf16x8 qreg[DP / 16];
#pragma unroll
  for (int s = 0; s < DP / 16; ++s) {
    const int d0 = 16 * s + 8 * hl;
    qreg[s] = (active && d0 < D) ? ld8(qb + (int64_t)qi * g.s_row + d0) : zero8();
  }

  // K: thread -> (key, 8-channel chunk) items; V: thread -> (4-key group,
  // chunk), transposed into Vt[d][key] with 8-byte stores.
  constexpr int KPT = (KITEMS + 255) / 256;  // K items per thread
  const int vgrp = tid % 16, vc = tid / 16;
  const bool vthread = tid < VITEMS;
  const bool vload = vthread && vc * 8 < D;
  bf16x8 kr[KPT], vr[4];
  auto load_kv = [&](int kt) {
#pragma unroll
    for (int it = 0; it < KPT; ++it) {
      const int idx = it * 256 + tid;
      const int kkey = idx / (DP / 8), kc = idx % (DP / 8);
      kr[it] = (idx < KITEMS && kc * 8 < D) ? ld8(kb + (int64_t)(kt + kkey) * g.s_row + kc * 8) : zero8();
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
      vr[r] = vload ? ld8(vb + (int64_t)(kt + vgrp * 4 + r) * g.s_row + vc * 8) : zero8();
  };
  auto store_kv = [&](int buf) {
#pragma unroll
    for (int it = 0; it < KPT; ++it) {
      const int idx = it * 256 + tid;
      const int kkey = idx / (DP / 8), kc = idx % (DP / 8);
      if (idx < KITEMS) *reinterpret_cast<bf16x8*>(&Ks[buf][kkey * KP + kc * 8]) = kr[it];
    }
    if (vthread) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        bf16x4 col;
#pragma unroll
        for (int r = 0; r < 4; ++r) col[r] = vr[r][e];
        *reinterpret_cast<bf16x4*>(&Vt[buf][(vc * 8 + e) * VP + vgrp * 4]) = col;
      }
    }
  };

  // Tiles whose 64 mask entries are all zero skip the mask add (the mask
  // is per plane, so the flag is uniform); computed up front so no wait on
  // the mask sits inside the pipelined loop.
  const int ntiles = N / 64;
  uint64_t mbits = ~0ull;
  if (ntiles <= 64) {
    mbits = 0ull;
    for (int t = 0; t < ntiles; ++t)
      if (__any(mrow[t * 64 + lane] != 0.f)) mbits |= 1ull << t;
  }

  f32x16 acc[DP / 32];
#pragma unroll
  for (int i = 0; i < DP / 32; ++i) acc[i] = zero16();
  float m = -INFINITY, l = 0.f, nm = 0.f;
  const bf16x2 ones = {static_cast<__bf16>(1.f), static_cast<__bf16>(1.f)};

  // The bias block for the next 32 keys is fetched while the current block
  // is processed; K/V for the next tile are fetched at the start of a tile
  // and stored to the other LDS buffer at its end.
  auto load_bias = [&](int blk) {
    f32x16 r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f32x4 x = *reinterpret_cast<const f32x4*>(brow + (int64_t)blk * 1024 + j * 256);
#pragma unroll
      for (int i = 0; i < 4; ++i) r[4 * j + i] = x[i];
    }
    return r;
  };
  f32x16 bnext = load_bias(0);
  load_kv(0);
  store_kv(0);
  __syncthreads();
  const int nblk = N / 32;
  for (int kt = 0, buf = 0; kt < N; kt += 64, buf ^= 1) {
    const bool more = kt + 64 < N;
    if (more) load_kv(kt + 64);
    const bool masked = (mbits >> ((kt >> 6) & 63)) & 1ull;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      const int blk = (kt >> 5) + sb;
      f32x16 s = bnext;
      if (blk + 1 < nblk) bnext = load_bias(blk + 1);
      if (!active) continue;
#pragma unroll
      for (int ks = 0; ks < DP / 16; ++ks) {
        bf16x8 ka = *reinterpret_cast<const bf16x8*>(&Ks[buf][(sb * 32 + ql) * KP + 16 * ks + 8 * hl]);
        s = mfma32(ka, qreg[ks], s);
      }
      if (masked) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          f32x4 mv = *reinterpret_cast<const f32x4*>(mrow + kt + sb * 32 + 8 * j + 4 * hl);
#pragma unroll
          for (int i = 0; i < 4; ++i) s[4 * j + i] = fmaf(mv[i], inv_scale, s[4 * j + i]);
        }
      }
      float mx = s[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
      mx = xor32_max(mx);
      if (__any(mx > m + thr)) {
        const float m_new = fmaxf(m, mx);
        const float alpha = (m_new == -INFINITY) ? 1.f : fast_exp2((m - m_new) * c2);
        l *= alpha;
#pragma unroll
        for (int db = 0; db < DP / 32; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[db][r] *= alpha;
        m = m_new;
        nm = (m == -INFINITY) ? 0.f : -m * c2;
      }
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        bf16x8 pb;
#pragma unroll
        for (int e = 0; e < 8; ++e) pb[e] = f2bf(fast_exp2(fmaf(s[8 * t + e], c2, nm)));
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          bf16x2 pr = {pb[e], pb[e + 1]};
          l = __builtin_amdgcn_fdot2_f32_bf16(pr, ones, l, false);
        }
        const int key0 = sb * 32 + 16 * t + 4 * hl;
#pragma unroll
        for (int db = 0; db < DP / 32; ++db) {
          const __bf16* vr2 = &Vt[buf][(db * 32 + ql) * VP + key0];
          bf16x4 lo = *reinterpret_cast<const bf16x4*>(vr2);
          bf16x4 hi = *reinterpret_cast<const bf16x4*>(vr2 + 8);
          bf16x8 va;
#pragma unroll
          for (int e = 0; e < 4; ++e) { va[e] = lo[e]; va[4 + e] = hi[e]; }
          acc[db] = mfma32(va, pb, acc[db]);
        }
      }
    }
    if (more) store_kv(buf ^ 1);
    __syncthreads();
  }
  if (!active) return;

  const float l_tot = xor32_sum(l);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  __bf16* orow = out + (((int64_t)plane * N + qi) * g.H + h) * D;
#pragma unroll
  for (int db = 0; db < DP / 32; ++db)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d0 = db * 32 + 8 * j + 4 * hl;
      if (d0 < D) {
        bf16x4 o4;
#pragma unroll
        for (int i = 0; i < 4; ++i) o4[i] = f2bf(acc[db][4 * j + i] * inv);
        *reinterpret_cast<bf16x4*>(orow + d0) = o4;
      }
    }
  if (hl == 0) {
    lse[((int64_t)plane * g.H + h) * N + qi] =
        l_tot > 0.f ? (m * c2 + log2f(l_tot)) * kLn2 : -INFINITY;
  }
}

// ---------------------------------------------------------------------------
// delta[b,o,h,q] = sum_d f32(dO) * f32(O), both [B,O,N,H,D] contiguous.
// One thread per (plane, q, h) row; rows of one (plane, q) are adjacent.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void attn_delta_kernel(
    const __bf16* __restrict__ dout, const __bf16* __restrict__ out,
    float* __restrict__ delta, int64_t rows, int H, int N, int D) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= rows) return;
  const __bf16* a = dout + r * D;
  const __bf16* o = out + r * D;
  float s = 0.f;
  for (int d = 0; d < D; d += 8) {
    bf16x8 x = ld8(a + d), y = ld8(o + d);
#pragma unroll
    for (int e = 0; e < 8; ++e) s = fmaf(bf2f(x[e]), bf2f(y[e]), s);
  }
  // r enumerates [plane][q][h]; delta is [plane][h][q].
  const int hh = (int)(r % H);
  const int64_t pq = r / H;
  const int qq = (int)(pq % N);
  const int64_t plane = pq / N;
  delta[(plane * H + hh) * N + qq] = s;
}

// ---------------------------------------------------------------------------
// Backward.  One workgroup = (64-key block, head, group of 4 outer rows); wave
// w owns outer row o = 4*group + w and keeps its dK / dV accumulators for the
// 64 keys in registers while streaming all queries in 32-row steps.  Scores are
// formed as S = Q K^T (lane = key column) so the C-layout P and dS tiles are
// the B operands of dV^T += dO^T P and dK^T += Q^T dS without data movement.
// dS goes through LDS once per step for (a) dQ^T = K^T dS^T, written as a
// per-key-block f32 partial, and (b) the dBias sum over the 4 waves, written
// as a per-outer-group f32 partial.  Fixed-order reducers finish both.
// ---------------------------------------------------------------------------
constexpr int kBwdGroup = 4;

template <int DP>
__global__ __launch_bounds__(256, 1) void attn_bwd_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k,
    const __bf16* __restrict__ v, const __bf16* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ delta,
    const float* __restrict__ mask, const __bf16* __restrict__ bias,
    __bf16* __restrict__ dk, __bf16* __restrict__ dv,
    float* __restrict__ dq_part, float* __restrict__ dbias_part, AttnGeom g) {
  constexpr int TP = 32 + 8;  // pitch of transposed Q / dO tiles (bf16)
  constexpr int SP = 64 + 8;  // pitch of the dS tile (bf16)
  constexpr int BP = 32 + 4;  // pitch of the transposed bias tile (f32)
  __shared__ __attribute__((aligned(16))) __bf16 Qt[4][DP * TP];
  __shared__ __attribute__((aligned(16))) __bf16 dOt[4][DP * TP];
  __shared__ __attribute__((aligned(16))) __bf16 dSs[4][32 * SP];
  __shared__ __attribute__((aligned(16))) float Bt[64 * BP];
  __shared__ __attribute__((aligned(16))) float Red[4][32 * 64];

  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int kl = lane & 31, hl = lane >> 5;
  const int kblk = blockIdx.x, h = blockIdx.y;
  const int groups = (g.O + kBwdGroup - 1) / kBwdGroup;
  const int b = blockIdx.z / groups, og = blockIdx.z % groups;
  const int o = og * kBwdGroup + w;
  const bool active = o < g.O;
  const int N = g.N, D = g.D, H = g.H;
  const int plane = b * g.O + (active ? o : 0);
  const int64_t plane_off = (int64_t)plane * H * N * D + (int64_t)h * g.s_head;
  const int key_base = kblk * 64;
  const float c2 = g.scale * kLog2e;

  // Per-wave constant operands for this key block.
  bf16x8 kB[2][DP / 16], vB[2][DP / 16];  // B operands: lane = key column
  bf16x8 kA[DP / 32][4];                  // A operand of dQ^T = K^T dS^T
  float mask2[2];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    const int key = key_base + cb * 32 + kl;
#pragma unroll
    for (int s = 0; s < DP / 16; ++s) {
      const int d0 = 16 * s + 8 * hl;
      const int64_t off = plane_off + (int64_t)key * g.s_row + d0;
      kB[cb][s] = (active && d0 < D) ? ld8(k + off) : zero8();
      vB[cb][s] = (active && d0 < D) ? ld8(v + off) : zero8();
    }
    mask2[cb] = active ? mask[(int64_t)plane * N + key] * kLog2e : -INFINITY;
  }
#pragma unroll
  for (int db = 0; db < DP / 32; ++db)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int d = db * 32 + kl;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int key = key_base + 16 * t + 8 * hl + e;
        kA[db][t][e] = (active && d < D) ? k[plane_off + (int64_t)key * g.s_row + d]
                                         : static_cast<__bf16>(0.f);
      }
    }

  f32x16 dKacc[DP / 32][2], dVacc[DP / 32][2];
#pragma unroll
  for (int db = 0; db < DP / 32; ++db)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) { dKacc[db][cb] = zero16(); dVacc[db][cb] = zero16(); }

  const __bf16* bias_h = bias + (int64_t)b * g.bias_bstride + (int64_t)h * N * N;
  const int64_t do_plane = (int64_t)plane * N * H * D + (int64_t)h * D;  // dO is [B,O,N,H,D]
  const int64_t st_plane = ((int64_t)plane * H + h) * N;                // lse / delta
  const int nkb = N / 64;
  float* dqp = dq_part + ((int64_t)kblk * g.B * g.O + plane) * H * N * D + (int64_t)h * N * D;

  for (int q0 = 0; q0 < N; q0 += 32) {
    // Stage the bias tile (32 queries x 64 keys) transposed, scaled by log2 e.
    {
      const int qr = tid >> 3, c = tid & 7;  // 32 rows x 8 chunks of 8 keys
      bf16x8 bv = ld8(bias_h + (int64_t)(q0 + qr) * N + key_base + c * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) Bt[(c * 8 + e) * BP + qr] = bf2f(bv[e]) * kLog2e;
    }
    // Q and dO rows (A operands of S and dP), also staged transposed.
    bf16x8 qA[DP / 16], doA[DP / 16];
#pragma unroll
    for (int s = 0; s < DP / 16; ++s) {
      const int d0 = 16 * s + 8 * hl;
      const bool ok = active && d0 < D;
      qA[s] = ok ? ld8(q + plane_off + (int64_t)(q0 + kl) * g.s_row + d0) : zero8();
      doA[s] = ok ? ld8(dout + do_plane + (int64_t)(q0 + kl) * H * D + d0) : zero8();
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        Qt[w][(d0 + e) * TP + kl] = qA[s][e];
        dOt[w][(d0 + e) * TP + kl] = doA[s][e];
      }
    }
    f32x4 lse4[4], del4[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int qq = q0 + 8 * j + 4 * hl;
      if (active) {
        lse4[j] = *reinterpret_cast<const f32x4*>(lse + st_plane + qq);
        del4[j] = *reinterpret_cast<const f32x4*>(delta + st_plane + qq);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) { lse4[j][i] = INFINITY; del4[j][i] = 0.f; }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
        lse4[j][i] = (lse4[j][i] == -INFINITY) ? INFINITY : lse4[j][i] * kLog2e;
    }
    __syncthreads();

    f32x16 P[2], dS[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      f32x16 s = zero16(), dp = zero16();
#pragma unroll
      for (int ks = 0; ks < DP / 16; ++ks) {
        s = mfma32(qA[ks], kB[cb][ks], s);
        dp = mfma32(doA[ks], vB[cb][ks], dp);
      }
      const float* bcol = &Bt[(cb * 32 + kl) * BP];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f32x4 bt = *reinterpret_cast<const f32x4*>(bcol + 8 * j + 4 * hl);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 4 * j + i;
          const float x = fmaf(s[r], c2, bt[i]) + (mask2[cb] - lse4[j][i]);
          const float p = fast_exp2(x);
          P[cb][r] = p;
          dS[cb][r] = p * (dp[r] - del4[j][i]);
        }
      }
    }
    // dV^T += dO^T P, dK^T += Q^T dS (16-query k-steps, permuted order).
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int db = 0; db < DP / 32; ++db) {
        const int row = (db * 32 + kl) * TP + 16 * t + 4 * hl;
        bf16x8 da, qa;
        {
          bf16x4 lo = *reinterpret_cast<const bf16x4*>(&dOt[w][row]);
          bf16x4 hi = *reinterpret_cast<const bf16x4*>(&dOt[w][row + 8]);
          bf16x4 lo2 = *reinterpret_cast<const bf16x4*>(&Qt[w][row]);
          bf16x4 hi2 = *reinterpret_cast<const bf16x4*>(&Qt[w][row + 8]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            da[e] = lo[e]; da[4 + e] = hi[e];
            qa[e] = lo2[e]; qa[4 + e] = hi2[e];
          }
        }
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          dVacc[db][cb] = mfma32(da, pack8(P[cb], 8 * t), dVacc[db][cb]);
          dKacc[db][cb] = mfma32(qa, pack8(dS[cb], 8 * t), dKacc[db][cb]);
        }
      }
    }
    // dS -> LDS: bf16 copy for dQ, f32 copy for the dBias wave sum.
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int qq = 8 * (r >> 2) + 4 * hl + (r & 3);
        const int key = cb * 32 + kl;
        dSs[w][qq * SP + key] = f2bf(dS[cb][r]);
        Red[w][qq * 64 + key] = dS[cb][r];
      }
    __syncthreads();
    // dQ^T (d x 32 queries) = K^T dS^T over this block's 64 keys.
    if (active) {
#pragma unroll
      for (int db = 0; db < DP / 32; ++db) {
        f32x16 acc = zero16();
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          bf16x8 sb = *reinterpret_cast<const bf16x8*>(&dSs[w][kl * SP + 16 * t + 8 * hl]);
          acc = mfma32(kA[db][t], sb, acc);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int d0 = db * 32 + 8 * j + 4 * hl;
          if (d0 < D) {
            f32x4 o4;
#pragma unroll
            for (int i = 0; i < 4; ++i) o4[i] = acc[4 * j + i];
            *reinterpret_cast<f32x4*>(dqp + (int64_t)(q0 + kl) * D + d0) = o4;
          }
        }
      }
    }
    // dBias partial: fixed wave order ((w0 + w1) + w2) + w3.
    {
      float* dst = dbias_part + (((int64_t)blockIdx.z * H + h) * N + q0) * N + key_base;
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        const int idx = it * 256 + tid;          // 32 rows x 16 float4 chunks
        const int qr = idx >> 4, c4 = (idx & 15) * 4;
        f32x4 acc = *reinterpret_cast<const f32x4*>(&Red[0][qr * 64 + c4]);
#pragma unroll
        for (int ww = 1; ww < 4; ++ww) {
          f32x4 x = *reinterpret_cast<const f32x4*>(&Red[ww][qr * 64 + c4]);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[i] += x[i];
        }
        *reinterpret_cast<f32x4*>(dst + (int64_t)qr * N + c4) = acc;
      }
    }
    (void)nkb;
  }
  if (!active) return;
  // dK (scaled) and dV, in Q/K/V storage order.
#pragma unroll
  for (int db = 0; db < DP / 32; ++db)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int key = key_base + cb * 32 + kl;
      const int64_t row = plane_off + (int64_t)key * g.s_row;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d0 = db * 32 + 8 * j + 4 * hl;
        if (d0 < D) {
          bf16x4 a4, b4;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            a4[i] = f2bf(dKacc[db][cb][4 * j + i] * g.scale);
            b4[i] = f2bf(dVacc[db][cb][4 * j + i]);
          }
          *reinterpret_cast<bf16x4*>(dk + row + d0) = a4;
          *reinterpret_cast<bf16x4*>(dv + row + d0) = b4;
        }
      }
    }
}

// dQ = bf16(scale * sum_kb partial[kb]) in ascending key-block order; written
// in Q's storage order.  One thread per 4 consecutive d of one row.
__global__ __launch_bounds__(256) void attn_dq_reduce_kernel(
    const float* __restrict__ part, __bf16* __restrict__ dq, AttnGeom g, int nkb) {
  const int D4 = g.D / 4;
  const int64_t total = (int64_t)g.B * g.O * g.H * g.N * D4;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= total) return;
  const int d0 = (int)(idx % D4) * 4;
  int64_t r = idx / D4;                 // [plane][h][q]
  const int qq = (int)(r % g.N); r /= g.N;
  const int hh = (int)(r % g.H);
  const int64_t plane = r / g.H;
  const int64_t stride = (int64_t)g.B * g.O * g.H * g.N * g.D;
  const float* src = part + ((plane * g.H + hh) * g.N + qq) * g.D + d0;
  f32x4 acc = *reinterpret_cast<const f32x4*>(src);
  for (int kb = 1; kb < nkb; ++kb) {
    f32x4 x = *reinterpret_cast<const f32x4*>(src + kb * stride);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] += x[i];
  }
  bf16x4 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = f2bf(acc[i] * g.scale);
  *reinterpret_cast<bf16x4*>(dq + plane * g.H * g.N * g.D + hh * g.s_head + (int64_t)qq * g.s_row + d0) = o;
}

// dBias[bb,h,q,k] (f32) = ascending fold over (b, outer group) partials that
// share bias batch bb.  Bb == 1 folds every batch; Bb == B folds per batch.
__global__ __launch_bounds__(256) void attn_dbias_reduce_kernel(
    const float* __restrict__ part, float* __restrict__ dbias, int B, int Bb,
    int groups, int H, int N) {
  const int64_t hnn4 = (int64_t)H * N * N / 4;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)Bb * hnn4) return;
  const int bb = (int)(idx / hnn4);
  const int64_t e = (idx % hnn4) * 4;
  const int b_lo = (Bb == 1) ? 0 : bb, b_hi = (Bb == 1) ? B : bb + 1;
  f32x4 acc;
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = 0.f;
  bool first = true;
  for (int bi = b_lo; bi < b_hi; ++bi)
    for (int gi = 0; gi < groups; ++gi) {
      f32x4 x = *reinterpret_cast<const f32x4*>(part + ((int64_t)bi * groups + gi) * H * N * N + e);
      if (first) { acc = x; first = false; }
      else {
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] += x[i];
      }
    }
  *reinterpret_cast<f32x4*>(dbias + (int64_t)bb * H * N * N + e) = acc;
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
                     int seq_major, int64_t bias_batches, double scale, const char* fn) {
  if (B > INT32_MAX || O > INT32_MAX || N > INT32_MAX)
    return set_error(TPF_ERR_SHAPE, "%s: dimension exceeds int32", fn);
  g->B = (int)B; g->O = (int)O; g->H = (int)H; g->N = (int)N; g->D = (int)D;
  g->s_row = seq_major ? H * D : D;
  g->s_head = seq_major ? D : N * D;
  if (bias_batches != 1 && bias_batches != B)
    return set_error(TPF_ERR_SHAPE, "%s: bias batch count %lld must be 1 or B=%lld", fn,
                     (long long)bias_batches, (long long)B);
  g->bias_bstride = (bias_batches == 1) ? 0 : H * N * N;
  g->scale = (float)scale;
  return check_geom(*g, fn);
}

extern "C" {

int64_t tpf_attn_forward_workspace_bytes(int64_t B, int64_t H, int64_t N,
                                         int64_t bias_batches) {
  (void)B;
  return bias_batches * H * N * N * 4;
}

static int attn_prescale_bias(const AttnGeom& g, const void* bias, float* bias_s,
                              int64_t bias_batches, hipStream_t s, const char* fn) {
  const int64_t items = bias_batches * g.H * (int64_t)g.N * g.N / 4;
  hipLaunchKernelGGL(attn_bias_prescale_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256),
                     0, s, (const __bf16*)bias, bias_s, items, g.N, 1.f / g.scale);
  return check_launch(fn);
}

int tpf_attn_forward_bf16(const void* q, const void* k, const void* v, const float* mask,
                          const void* bias, void* out, float* lse, void* workspace,
                          int64_t workspace_bytes, int64_t B, int64_t O, int64_t H, int64_t N,
                          int64_t D, int seq_major, int64_t bias_batches, double scale,
                          void* stream) {
  const char* fn = "tpf_attn_forward_bf16";
  AttnGeom g;
  int rc = make_geom(&g, B, O, H, N, D, seq_major, bias_batches, scale, fn);
  if (rc) return rc;
  if (!q || !k || !v || !mask || !bias || !out || !lse || !workspace)
    return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  if (workspace_bytes < tpf_attn_forward_workspace_bytes(B, H, N, bias_batches))
    return set_error(TPF_ERR_ARG, "%s: workspace too small", fn);
  const int64_t total = ((N + 127) / 128) * H * B * O;
  if ((total + 7) / 8 * 8 > INT32_MAX)
    return set_error(TPF_ERR_SHAPE, "%s: too many query tiles", fn);
  hipStream_t s = (hipStream_t)stream;
  float* bias_s = (float*)workspace;
  if ((rc = attn_prescale_bias(g, bias, bias_s, bias_batches, s, fn))) return rc;
  g.bias_bstride = (bias_batches == 1) ? 0 : H * N * N;
  dim3 grid((unsigned)((total + 7) / 8 * 8));
  if (D <= 32)
    hipLaunchKernelGGL(attn_fwd_kernel<32>, grid, dim3(256), 0, s, (const __bf16*)q,
                       (const __bf16*)k, (const __bf16*)v, mask, bias_s, (__bf16*)out, lse, g);
  else
    hipLaunchKernelGGL(attn_fwd_kernel<64>, grid, dim3(256), 0, s, (const __bf16*)q,
                       (const __bf16*)k, (const __bf16*)v, mask, bias_s, (__bf16*)out, lse, g);
  return check_launch(fn);
}

int tpf_attn_delta_bf16(const void* dout, const void* out, float* delta, int64_t B, int64_t O,
                        int64_t H, int64_t N, int64_t D, void* stream) {
  if (!dout || !out || !delta) return set_error(TPF_ERR_ARG, "tpf_attn_delta_bf16: null pointer");
  if (B < 1 || O < 1 || H < 1 || N < 1 || D < 8 || D > 64 || D % 8)
    return set_error(TPF_ERR_SHAPE, "tpf_attn_delta_bf16: bad shape");
  const int64_t rows = B * O * N * H;
  hipLaunchKernelGGL(attn_delta_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const __bf16*)dout, (const __bf16*)out, delta, rows,
                     (int)H, (int)N, (int)D);
  return check_launch("tpf_attn_delta_bf16");
}

int64_t tpf_attn_backward_workspace_bytes(int64_t B, int64_t O, int64_t H, int64_t N,
                                          int64_t D) {
  const int64_t groups = (O + kBwdGroup - 1) / kBwdGroup;
  const int64_t dq = (N / 64) * B * O * H * N * D * 4;
  const int64_t db = B * groups * H * N * N * 4;
  return ((dq + 255) / 256) * 256 + db;
}

static int attn_bwd_prepare(AttnGeom* g, const char* fn, const void* q, const void* k,
                            const void* v, const void* dout, const float* lse, const float* delta,
                            const float* mask, const void* bias, const void* workspace,
                            int64_t workspace_bytes, int64_t B, int64_t O, int64_t H, int64_t N,
                            int64_t D, int seq_major, int64_t bias_batches, double scale) {
  int rc = make_geom(g, B, O, H, N, D, seq_major, bias_batches, scale, fn);
  if (rc) return rc;
  if (!q || !k || !v || !dout || !lse || !delta || !mask || !bias || !workspace)
    return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  const int64_t need = tpf_attn_backward_workspace_bytes(B, O, H, N, D);
  if (workspace_bytes < need)
    return set_error(TPF_ERR_ARG, "%s: workspace %lld < required %lld", fn,
                     (long long)workspace_bytes, (long long)need);
  const int64_t groups = (O + kBwdGroup - 1) / kBwdGroup;
  if (B * groups > 65535) return set_error(TPF_ERR_SHAPE, "%s: B*ceil(O/4) exceeds grid-z", fn);
  return TPF_OK;
}

static void attn_bwd_parts(const AttnGeom& g, void* workspace, float** dq_part, float** db_part) {
  const int64_t dq_bytes = (int64_t)(g.N / 64) * g.B * g.O * g.H * g.N * g.D * 4;
  *dq_part = (float*)workspace;
  *db_part = (float*)((char*)workspace + ((dq_bytes + 255) / 256) * 256);
}

// Stage 1 of the backward: the single-reconstruction kernel writing dK, dV
// and the dQ / dBias partials into the workspace.
int tpf_attn_backward_main_bf16(const void* q, const void* k, const void* v, const void* dout,
                                const float* lse, const float* delta, const float* mask,
                                const void* bias, void* dk, void* dv, void* workspace,
                                int64_t workspace_bytes, int64_t B, int64_t O, int64_t H,
                                int64_t N, int64_t D, int seq_major, int64_t bias_batches,
                                double scale, void* stream) {
  const char* fn = "tpf_attn_backward_main_bf16";
  AttnGeom g;
  int rc = attn_bwd_prepare(&g, fn, q, k, v, dout, lse, delta, mask, bias, workspace,
                            workspace_bytes, B, O, H, N, D, seq_major, bias_batches, scale);
  if (rc) return rc;
  if (!dk || !dv) return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  float *dq_part, *db_part;
  attn_bwd_parts(g, workspace, &dq_part, &db_part);
  const int64_t groups = (O + kBwdGroup - 1) / kBwdGroup;
  dim3 grid((unsigned)(N / 64), (unsigned)H, (unsigned)(B * groups));
  hipStream_t s = (hipStream_t)stream;
  if (D <= 32)
    hipLaunchKernelGGL(attn_bwd_kernel<32>, grid, dim3(256), 0, s, (const __bf16*)q,
                       (const __bf16*)k, (const __bf16*)v, (const __bf16*)dout, lse, delta, mask,
                       (const __bf16*)bias, (__bf16*)dk, (__bf16*)dv, dq_part, db_part, g);
  else
    hipLaunchKernelGGL(attn_bwd_kernel<64>, grid, dim3(256), 0, s, (const __bf16*)q,
                       (const __bf16*)k, (const __bf16*)v, (const __bf16*)dout, lse, delta, mask,
                       (const __bf16*)bias, (__bf16*)dk, (__bf16*)dv, dq_part, db_part, g);
  return check_launch(fn);
}

// Stage 2 of the backward: fixed-order folds of the dQ and dBias partials.
int tpf_attn_backward_finish_bf16(void* dq, float* dbias, const void* workspace, int64_t B,
                                  int64_t O, int64_t H, int64_t N, int64_t D, int seq_major,
                                  int64_t bias_batches, double scale, void* stream) {
  const char* fn = "tpf_attn_backward_finish_bf16";
  AttnGeom g;
  int rc = make_geom(&g, B, O, H, N, D, seq_major, bias_batches, scale, fn);
  if (rc) return rc;
  if (!dq || !dbias || !workspace) return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  float *dq_part, *db_part;
  attn_bwd_parts(g, (void*)workspace, &dq_part, &db_part);
  hipStream_t s = (hipStream_t)stream;
  const int64_t groups = (O + kBwdGroup - 1) / kBwdGroup;
  const int64_t dq_items = B * O * H * N * (D / 4);
  hipLaunchKernelGGL(attn_dq_reduce_kernel, dim3((unsigned)((dq_items + 255) / 256)), dim3(256),
                     0, s, dq_part, (__bf16*)dq, g, (int)(N / 64));
  if ((rc = check_launch(fn))) return rc;
  const int64_t db_items = bias_batches * H * N * N / 4;
  hipLaunchKernelGGL(attn_dbias_reduce_kernel, dim3((unsigned)((db_items + 255) / 256)),
                     dim3(256), 0, s, db_part, dbias, (int)B, (int)bias_batches, (int)groups,
                     (int)H, (int)N);
  return check_launch(fn);
}

int tpf_attn_backward_bf16(const void* q, const void* k, const void* v, const void* dout,
                           const float* lse, const float* delta, const float* mask,
                           const void* bias, void* dq, void* dk, void* dv, float* dbias,
                           void* workspace, int64_t workspace_bytes, int64_t B, int64_t O,
                           int64_t H, int64_t N, int64_t D, int seq_major, int64_t bias_batches,
                           double scale, void* stream) {
  if (!dq || !dbias) return set_error(TPF_ERR_ARG, "tpf_attn_backward_bf16: null pointer");
  int rc = tpf_attn_backward_main_bf16(q, k, v, dout, lse, delta, mask, bias, dk, dv, workspace,
                                       workspace_bytes, B, O, H, N, D, seq_major, bias_batches,
                                       scale, stream);
  if (rc) return rc;
  return tpf_attn_backward_finish_bf16(dq, dbias, workspace, B, O, H, N, D, seq_major,
                                       bias_batches, scale, stream);
}

}  // extern "C"
