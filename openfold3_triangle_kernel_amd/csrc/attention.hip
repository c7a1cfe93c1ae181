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

// ---------------------------------------------------------------------------
// Forward.  One workgroup = 4 waves = 128 queries of one plane; each wave owns
// 32 queries and walks all keys in 64-key tiles staged in LDS.  Scores are
// produced transposed (S^T = K Q^T) so each lane owns one query column: row
// max / sum need only the lane^32 exchange, and the C-layout P^T tile is fed
// directly as the B operand of O^T += V^T P^T.
// ---------------------------------------------------------------------------
template <int DP>
__global__ __launch_bounds__(256) void attn_fwd_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k,
    const __bf16* __restrict__ v, const float* __restrict__ mask,
    const __bf16* __restrict__ bias, __bf16* __restrict__ out,
    float* __restrict__ lse, AttnGeom g) {
  constexpr int KP = DP + 8;     // K tile pitch (bf16)
  constexpr int VP = 64 + 8;     // V^T tile pitch (bf16)
  __shared__ __attribute__((aligned(16))) __bf16 Ks[64 * KP];
  __shared__ __attribute__((aligned(16))) __bf16 Vt[DP * VP];

  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int ql = lane & 31, hl = lane >> 5;
  const int h = blockIdx.y, plane = blockIdx.z;
  const int b = plane / g.O;
  const int N = g.N, D = g.D;
  const int q0 = blockIdx.x * 128 + w * 32;
  const bool active = q0 < N;
  const int qi = q0 + ql;

  const int64_t plane_off = (int64_t)plane * g.H * N * D + (int64_t)h * g.s_head;
  const __bf16* qb = q + plane_off;
  const __bf16* kb = k + plane_off;
  const __bf16* vb = v + plane_off;
  const float* mrow = mask + (int64_t)plane * N;
  const __bf16* brow = bias + (int64_t)b * g.bias_bstride + ((int64_t)h * N + (active ? qi : 0)) * N;
  const float c2 = g.scale * kLog2e;

  bf16x8 qreg[DP / 16];
#pragma unroll
  for (int s = 0; s < DP / 16; ++s) {
    const int d0 = 16 * s + 8 * hl;
    qreg[s] = (active && d0 < D) ? ld8(qb + (int64_t)qi * g.s_row + d0) : zero8();
  }

  f32x16 acc[DP / 32];
#pragma unroll
  for (int i = 0; i < DP / 32; ++i) acc[i] = zero16();
  float m = -INFINITY, l = 0.f;

  for (int kt = 0; kt < N; kt += 64) {
    __syncthreads();
    // Stage K (row-major) and V^T for keys kt..kt+63.
#pragma unroll
    for (int it = 0; it < (64 * DP / 8 + 255) / 256; ++it) {
      const int idx = it * 256 + tid;
      if (idx < 64 * DP / 8) {
        const int key = idx / (DP / 8), c = idx % (DP / 8);
        const int64_t off = (int64_t)(kt + key) * g.s_row + c * 8;
        bf16x8 kv = zero8(), vv = zero8();
        if (c * 8 < D) { kv = ld8(kb + off); vv = ld8(vb + off); }
        *reinterpret_cast<bf16x8*>(&Ks[key * KP + c * 8]) = kv;
#pragma unroll
        for (int e = 0; e < 8; ++e) Vt[(c * 8 + e) * VP + key] = vv[e];
      }
    }
    __syncthreads();
    if (!active) continue;

    f32x16 st[2];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      f32x16 s = zero16();
#pragma unroll
      for (int ks = 0; ks < DP / 16; ++ks) {
        bf16x8 ka = *reinterpret_cast<const bf16x8*>(&Ks[(sb * 32 + ql) * KP + 16 * ks + 8 * hl]);
        s = mfma32(ka, qreg[ks], s);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int key = kt + sb * 32 + 8 * j + 4 * hl;
        bf16x4 bv = ld4(brow + key);
        f32x4 mv = *reinterpret_cast<const f32x4*>(mrow + key);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float add = (bf2f(bv[i]) + mv[i]) * kLog2e;
          s[4 * j + i] = fmaf(s[4 * j + i], c2, add);
        }
      }
      st[sb] = s;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, st[sb][r]);
    mx = xor32_max(mx);
    const float m_new = fmaxf(m, mx);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = fast_exp2(m - m_use);
    float lsum = 0.f;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(st[sb][r] - m_use);
        st[sb][r] = p;
        lsum += p;
      }
    l = l * alpha + lsum;
    m = m_new;
#pragma unroll
    for (int db = 0; db < DP / 32; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[db][r] *= alpha;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        bf16x8 pb = pack8(st[sb], 8 * t);
        const int key0 = sb * 32 + 16 * t + 4 * hl;
#pragma unroll
        for (int db = 0; db < DP / 32; ++db) {
          const __bf16* vr = &Vt[(db * 32 + ql) * VP + key0];
          bf16x4 lo = *reinterpret_cast<const bf16x4*>(vr);
          bf16x4 hi = *reinterpret_cast<const bf16x4*>(vr + 8);
          bf16x8 va;
#pragma unroll
          for (int e = 0; e < 4; ++e) { va[e] = lo[e]; va[4 + e] = hi[e]; }
          acc[db] = mfma32(va, pb, acc[db]);
        }
      }
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
        l_tot > 0.f ? (m + log2f(l_tot)) * kLn2 : -INFINITY;
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

int tpf_attn_forward_bf16(const void* q, const void* k, const void* v, const float* mask,
                          const void* bias, void* out, float* lse, int64_t B, int64_t O,
                          int64_t H, int64_t N, int64_t D, int seq_major,
                          int64_t bias_batches, double scale, void* stream) {
  AttnGeom g;
  int rc = make_geom(&g, B, O, H, N, D, seq_major, bias_batches, scale, "tpf_attn_forward_bf16");
  if (rc) return rc;
  if (!q || !k || !v || !mask || !bias || !out || !lse)
    return set_error(TPF_ERR_ARG, "tpf_attn_forward_bf16: null pointer");
  if (B * O > 65535)
    return set_error(TPF_ERR_SHAPE, "tpf_attn_forward_bf16: B*O=%lld exceeds grid-z", (long long)(B * O));
  dim3 grid((unsigned)((N + 127) / 128), (unsigned)H, (unsigned)(B * O));
  hipStream_t s = (hipStream_t)stream;
  if (D <= 32)
    hipLaunchKernelGGL(attn_fwd_kernel<32>, grid, dim3(256), 0, s, (const __bf16*)q,
                       (const __bf16*)k, (const __bf16*)v, mask, (const __bf16*)bias,
                       (__bf16*)out, lse, g);
  else
    hipLaunchKernelGGL(attn_fwd_kernel<64>, grid, dim3(256), 0, s, (const __bf16*)q,
                       (const __bf16*)k, (const __bf16*)v, mask, (const __bf16*)bias,
                       (__bf16*)out, lse, g);
  return check_launch("tpf_attn_forward_bf16");
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
