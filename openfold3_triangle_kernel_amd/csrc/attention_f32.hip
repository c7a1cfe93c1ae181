// FP32 triangle attention forward (inference) on gfx950 MFMA.
//
//   out[b,o,q,h,:] = sum_k softmax_k(scale <q, k> + mask[b,o,k] + bias[bb,h,q,k]) v[k,:]
//
// all in FP32 (v_mfma_f32_32x32x2_f32 products and sums, f32 softmax), the
// contract of the reference's inference-only FP32 path
// (openfold3/core/kernels/turbopairformer/turbopairformer_attention_fp32.py:139-224):
// a row whose logits are all -inf produces zeros.
//
// Same schedule as the bf16 forward (csrc/attention.hip): one workgroup = 4
// waves x 32 queries of one plane, 64-key tiles double-buffered in LDS, the
// S^T = K Q^T accumulator of each 32-key block seeded with the prescaled,
// fragment-major bias, online softmax with a lazily raised running max.
// The 32x32x2 MFMA takes one k value per lane half: within each group of 8
// channels the lower half supplies channels 0..3 and the upper half 4..7
// over four MFMAs; in O^T += V^T P^T the key of register r of P^T is
// 8 (r / 4) + 4 (lane / 32) + r % 4, so P feeds the MFMA straight from
// registers and V^T is read for the same keys.
#include "common.hpp"
#include "tpf_status.hpp"

namespace tpf {

struct AttnGeomF {
  int B, O, H, N, D;
  int64_t s_row;         // element stride between sequence rows of q/k/v
  int64_t s_head;        // element stride between heads of q/k/v
  int64_t bias_bstride;  // elements between bias batches (0 = shared)
  float scale;
};

__device__ __forceinline__ f32x16 mfma32f_a(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// f32 bias -> f32 bias / scale in the fragment-major S^T layout (see the
// bf16 pre-pass in csrc/attention.hip).
__global__ __launch_bounds__(256) void attn_bias_prescale_f32_kernel(const float* __restrict__ bias,
                                                                     float* __restrict__ out,
                                                                     int64_t items, int N,
                                                                     float inv_scale) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (block, j, lane)
  if (i >= items) return;
  const int lane = (int)(i & 63), j = (int)((i >> 6) & 3);
  const int64_t blk = i >> 8;
  const int nkb = N / 32;
  const int kb = (int)(blk % nkb);
  const int64_t hq = blk / nkb;
  const int qb = (int)(hq % (N / 32));
  const int64_t bh = hq / (N / 32);
  const int ql = lane & 31, hl = lane >> 5;
  const float* src = bias + (bh * N + qb * 32 + ql) * (int64_t)N + kb * 32 + 8 * j + 4 * hl;
  f32x4 v = *reinterpret_cast<const f32x4*>(src);
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] *= inv_scale;
  *reinterpret_cast<f32x4*>(out + i * 4) = v;
}

template <int DP>
__global__ __launch_bounds__(256) void attn_fwd_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ mask, const float* __restrict__ bias_s, float* __restrict__ out,
    float* __restrict__ lse, AttnGeomF g) {
  constexpr int KP = DP + 4;  // K tile pitch (f32): conflict-free 16-byte reads
  constexpr int VP = 64 + 4;  // V^T tile pitch (f32)
  constexpr int CH = DP / 4;  // 16-byte chunks per row
  constexpr int PER = 64 * CH / 256;  // K (and V) chunks per thread per tile
  __shared__ __attribute__((aligned(16))) float Ks[2][64 * KP];
  __shared__ __attribute__((aligned(16))) float Vt[2][DP * VP];

  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int ql = lane & 31, hl = lane >> 5;
  const int N = g.N, D = g.D;
  const int qtiles = (N + 127) / 128;
  int64_t T;
  {
    const int64_t total = (int64_t)qtiles * g.H * g.B * g.O;
    const int64_t L = blockIdx.x, per = (total + 7) / 8;
    T = (L % 8) * per + L / 8;
    if (T >= total) return;
  }
  const int qt = (int)(T % qtiles);
  const int64_t rr = T / qtiles;
  const int plane = (int)(rr % ((int64_t)g.B * g.O));
  const int h = (int)(rr / ((int64_t)g.B * g.O));
  const int b = plane / g.O;
  const int q0 = qt * 128 + w * 32;
  const bool active = q0 < N;
  const int qi = q0 + ql;

  const int64_t plane_off = (int64_t)plane * g.H * N * D + (int64_t)h * g.s_head;
  const float* qb = q + plane_off;
  const float* kb = k + plane_off;
  const float* vb = v + plane_off;
  const float* mrow = mask + (int64_t)plane * N;
  const float* brow = bias_s + (int64_t)b * g.bias_bstride +
                      ((int64_t)h * (N / 32) + (active ? q0 / 32 : 0)) * (int64_t)(N / 32) * 1024 + lane * 4;
  const float c2 = g.scale * kLog2e;
  const float inv_scale = 1.f / g.scale;
  const float thr = 8.f / c2;

  f32x4 qv[DP / 8];
#pragma unroll
  for (int gg = 0; gg < DP / 8; ++gg) {
    const int d0 = 8 * gg + 4 * hl;
    qv[gg] = (active && d0 < D) ? *reinterpret_cast<const f32x4*>(qb + (int64_t)qi * g.s_row + d0)
                                : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  f32x4 kr[PER], vr[PER];
  auto load_kv = [&](int kt) {
#pragma unroll
    for (int it = 0; it < PER; ++it) {
      const int idx = it * 256 + tid;
      const int key = idx / CH, c = idx % CH;
      kr[it] = c * 4 < D ? *reinterpret_cast<const f32x4*>(kb + (int64_t)(kt + key) * g.s_row + c * 4)
                         : f32x4{0.f, 0.f, 0.f, 0.f};
      const int vkey = idx % 64, vc = idx / 64;
      vr[it] = vc * 4 < D ? *reinterpret_cast<const f32x4*>(vb + (int64_t)(kt + vkey) * g.s_row + vc * 4)
                          : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  auto store_kv = [&](int buf) {
#pragma unroll
    for (int it = 0; it < PER; ++it) {
      const int idx = it * 256 + tid;
      *reinterpret_cast<f32x4*>(&Ks[buf][(idx / CH) * KP + (idx % CH) * 4]) = kr[it];
      // V items run key-fastest, so the transposing stores hit consecutive banks.
      const int key = idx % 64, c = idx / 64;
#pragma unroll
      for (int e = 0; e < 4; ++e) Vt[buf][(c * 4 + e) * VP + key] = vr[it][e];
    }
  };
  const int ntiles = N / 64;
  uint64_t mbits = ~0ull;
  if (ntiles <= 64) {
    // Four tiles' mask loads in flight per ballot round.
    mbits = 0ull;
    for (int t = 0; t < ntiles; t += 4) {
      float mv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) mv[u] = t + u < ntiles ? mrow[(t + u) * 64 + lane] : 0.f;
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (__any(mv[u] != 0.f)) mbits |= 1ull << (t + u);
    }
  }
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

  f32x16 acc[DP / 32];
#pragma unroll
  for (int i = 0; i < DP / 32; ++i) acc[i] = zero16();
  float m = -INFINITY, l = 0.f, nm = 0.f;
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
      for (int gg = 0; gg < DP / 8; ++gg) {
        const f32x4 kf = *reinterpret_cast<const f32x4*>(&Ks[buf][(sb * 32 + ql) * KP + 8 * gg + 4 * hl]);
#pragma unroll
        for (int e = 0; e < 4; ++e) s = mfma32f_a(kf[e], qv[gg][e], s);
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
      f32x16 p;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        p[r] = fast_exp2(fmaf(s[r], c2, nm));
        l += p[r];
      }
#pragma unroll
      for (int db = 0; db < DP / 32; ++db) {
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const f32x4 va = *reinterpret_cast<const f32x4*>(
              &Vt[buf][(db * 32 + ql) * VP + sb * 32 + 8 * qq + 4 * hl]);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[db] = mfma32f_a(va[e], p[4 * qq + e], acc[db]);
        }
      }
    }
    if (more) store_kv(buf ^ 1);
    __syncthreads();
  }
  if (!active) return;
  const float l_tot = xor32_sum(l);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  float* orow = out + (((int64_t)plane * N + qi) * g.H + h) * D;
#pragma unroll
  for (int db = 0; db < DP / 32; ++db)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d0 = db * 32 + 8 * j + 4 * hl;
      if (d0 < D) {
        f32x4 o4;
#pragma unroll
        for (int i = 0; i < 4; ++i) o4[i] = acc[db][4 * j + i] * inv;
        *reinterpret_cast<f32x4*>(orow + d0) = o4;
      }
    }
  if (hl == 0 && lse) {
    lse[((int64_t)plane * g.H + h) * N + qi] =
        l_tot > 0.f ? (m * c2 + log2f(l_tot)) * kLn2 : -INFINITY;
  }
}

}  // namespace tpf

using namespace tpf;

extern "C" {

int64_t tpf_attn_forward_f32_workspace_bytes(int64_t B, int64_t H, int64_t N,
                                             int64_t bias_batches) {
  (void)B;
  return bias_batches * H * N * N * 4;
}

int tpf_attn_forward_f32(const float* q, const float* k, const float* v, const float* mask,
                         const float* bias, float* out, float* lse, void* workspace,
                         int64_t workspace_bytes, int64_t B, int64_t O, int64_t H, int64_t N,
                         int64_t D, int layout, int64_t bias_batches, double scale,
                         void* stream) {
  const char* fn = "tpf_attn_forward_f32";
  if (layout & ~TPF_QKV_SEQ_MAJOR)
    return set_error(TPF_ERR_ARG, "%s: layout flags 0x%x: only TPF_QKV_SEQ_MAJOR is supported", fn,
                     layout);
  const bool seq_major = layout & TPF_QKV_SEQ_MAJOR;
  if (!q || !k || !v || !mask || !bias || !out || !workspace)
    return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  if (B < 1 || O < 1 || H < 1 || N < 1)
    return set_error(TPF_ERR_SHAPE, "%s: B, O, H and N must be positive", fn);
  if (N % 64 != 0)
    return set_error(TPF_ERR_SHAPE, "%s: N=%lld must be a multiple of 64 (pad on the host)", fn,
                     (long long)N);
  if (D < 4 || D > 64 || D % 4 != 0)
    return set_error(TPF_ERR_SHAPE, "%s: D=%lld must be a multiple of 4 in [4, 64]", fn,
                     (long long)D);
  if (bias_batches != 1 && bias_batches != B)
    return set_error(TPF_ERR_SHAPE, "%s: bias batch %lld must be 1 or B", fn,
                     (long long)bias_batches);
  if (workspace_bytes < tpf_attn_forward_f32_workspace_bytes(B, H, N, bias_batches))
    return set_error(TPF_ERR_ARG, "%s: workspace too small", fn);
  const int64_t total = ((N + 127) / 128) * H * B * O;
  if ((total + 7) / 8 * 8 > INT32_MAX || B * O > INT32_MAX)
    return set_error(TPF_ERR_SHAPE, "%s: too many query tiles", fn);
  AttnGeomF g;
  g.B = (int)B; g.O = (int)O; g.H = (int)H; g.N = (int)N; g.D = (int)D;
  g.s_row = seq_major ? H * D : D;
  g.s_head = seq_major ? D : N * D;
  g.bias_bstride = (bias_batches == 1) ? 0 : H * N * N;
  g.scale = (float)scale;
  hipStream_t s = (hipStream_t)stream;
  float* bias_s = (float*)workspace;
  const int64_t items = bias_batches * H * N * N / 4;
  hipLaunchKernelGGL(attn_bias_prescale_f32_kernel, dim3((unsigned)((items + 255) / 256)),
                     dim3(256), 0, s, bias, bias_s, items, (int)N, (float)(1.0 / scale));
  int rc = check_launch(fn);
  if (rc) return rc;
  dim3 grid((unsigned)((total + 7) / 8 * 8));
  if (D <= 32)
    hipLaunchKernelGGL(attn_fwd_f32_kernel<32>, grid, dim3(256), 0, s, q, k, v, mask, bias_s, out,
                       lse, g);
  else
    hipLaunchKernelGGL(attn_fwd_f32_kernel<64>, grid, dim3(256), 0, s, q, k, v, mask, bias_s, out,
                       lse, g);
  return check_launch(fn);
}

}  // extern "C"
