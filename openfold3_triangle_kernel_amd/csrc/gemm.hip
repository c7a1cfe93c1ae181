// Batched bf16 GEMM on gfx950 MFMA for the TriMul channel contraction, its
// backward products and the split-K weight-gradient products.
//
//   C[z][m][n] = alpha * sum_k A[z](m, k) * B[z](n, k)
//
// A and B are each given either K-contiguous ("KC": X[r * ld + k]) or
// MN-contiguous ("MN": X[k * ld + r]); the main loop (gemm_core.hpp) reads
// both layouts straight into LDS and feeds the MFMA from there.  C is
// row-major (n contiguous) in bf16 or f32.  Split-K writes f32 partials at
// C + split * c_split and a fixed-order fold kernel sums them
// (deterministic, no atomics).
#include "common.hpp"
#include "gemm_core.hpp"
#include "tpf_gemm.hpp"
#include "tpf_status.hpp"

namespace tpf {

// Tile T of problem g (T < tiles of g, in (n-tile, m-tile, split, batch)
// order) into C.
template <bool A_KC, bool B_KC, bool OUT_F32>
__device__ __forceinline__ void gemm_bf16_tile(const GemmArgs& g, int64_t T, char* smem) {
  const int tm = (g.M + kGM - 1) / kGM, tn = (g.N + kGN - 1) / kGN;
  const int nt = (int)(T % tn);
  int64_t r = T / tn;
  const int mt = (int)(r % tm);
  r /= tm;
  const int split = (int)(r % g.ksplit);
  const int z = (int)(r / g.ksplit);
  const int m0 = mt * kGM, n0 = nt * kGN;
  const int kbeg = split * g.k_chunk;
  const int kend = min(g.K, kbeg + g.k_chunk);
  GemmOperand A{g.A + (int64_t)z * g.a_bs, g.a_ld, g.M, g.a_gather_n, g.a_div_n, g.a_div_nn};
  GemmOperand B{g.B + (int64_t)z * g.b_bs, g.b_ld, g.N, 0, {}, {}};
  f32x16 acc[2][2];
  gemm_tile<A_KC, B_KC>(A, B, m0, n0, kbeg, kend, smem, acc);

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int rl = lane & 31, hl = lane >> 5, wm = w >> 1, wn = w & 1;
  char* Cb = (char*)g.C + ((int64_t)z * g.c_bs + (int64_t)split * g.c_split) * (OUT_F32 ? 4 : 2);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + wn * 64 + j * 32 + rl;
      if (col >= g.N) continue;
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) {
        const int row = m0 + wm * 64 + i * 32 + 8 * (rr >> 2) + 4 * hl + (rr & 3);
        if (row < g.M) {
          const float val = acc[i][j][rr] * g.alpha;
          const int64_t off = (int64_t)row * g.c_ld + col;
          if (OUT_F32) reinterpret_cast<float*>(Cb)[off] = val;
          else reinterpret_cast<__bf16*>(Cb)[off] = f2bf(val);
        }
      }
    }
}

__host__ __device__ inline int64_t gemm_tiles(const GemmArgs& g) {
  return (int64_t)((g.M + kGM - 1) / kGM) * ((g.N + kGN - 1) / kGN) * g.batch * g.ksplit;
}

template <bool A_KC, bool B_KC, bool OUT_F32>
__global__ __launch_bounds__(256, 2) void gemm_bf16_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) char smem[kGMainLdsBytes];
  const int64_t T = xcd_order(gemm_tiles(g));
  if (T < 0) return;
  gemm_bf16_tile<A_KC, B_KC, OUT_F32>(g, T, smem);
}

// Two problems of one layout in one grid: workgroups [0, p0) take the
// tiles of g0 and the rest those of g1 (p0 = g0's tiles rounded up to 8),
// each in its own XCD-aware order, so both problems spread over all XCDs
// and independent small GEMMs stay in flight together.
template <bool AK0, bool BK0, bool AK1, bool BK1, bool OUT_F32>
__global__ __launch_bounds__(256, 2) void gemm_bf16_pair_kernel(GemmArgs g0, GemmArgs g1) {
  __shared__ __attribute__((aligned(1024))) char smem[kGMainLdsBytes];
  const int64_t t0 = gemm_tiles(g0), p0 = (t0 + 7) / 8 * 8;
  const int64_t L = blockIdx.x;
  if (L < p0) {
    const int64_t T = xcd_order_of(L, t0);
    if (T >= 0) gemm_bf16_tile<AK0, BK0, OUT_F32>(g0, T, smem);
  } else {
    const int64_t T = xcd_order_of(L - p0, gemm_tiles(g1));
    if (T >= 0) gemm_bf16_tile<AK1, BK1, OUT_F32>(g1, T, smem);
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
  int s = s0 + 1;
  for (; s + 8 <= s1; s += 8) {  // 8 loads in flight, added in ascending order
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = part[(int64_t)(s + e) * stride + i];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc += v[e];
  }
  for (; s < s1; ++s) acc += part[(int64_t)s * stride + i];
  dst[(int64_t)j * dst_stride + i] = acc;
}

// Several folds in one launch per pass: blockIdx.y runs over the (segment,
// chunk) pairs.  Intermediate passes fold 64-split chunks in place (as
// fold_launch does); the final pass writes element i of a segment to
// dst[i / piece][i % piece], so one segment can land in up to 4 outputs.
__global__ __launch_bounds__(256) void fold_multi_kernel(FoldSegs f, int final_pass) {
  int sg = 0;
  while (sg + 1 < f.nseg && (int)blockIdx.y >= f.gbase[sg + 1]) ++sg;
  const int j = (int)blockIdx.y - f.gbase[sg];
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= f.n[sg]) return;
  const float* part = f.part[sg];
  const int64_t stride = f.stride[sg];
  const int chunk = final_pass ? f.splits[sg] : 64;
  const int s0 = j * chunk, s1 = min(f.splits[sg], s0 + chunk);
  float acc = part[(int64_t)s0 * stride + i];
  int s = s0 + 1;
  for (; s + 8 <= s1; s += 8) {
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = part[(int64_t)(s + e) * stride + i];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc += v[e];
  }
  for (; s < s1; ++s) acc += part[(int64_t)s * stride + i];
  if (final_pass) {
    const int64_t pc = i / f.piece[sg];
    f.dst[sg][pc][i - pc * f.piece[sg]] = acc;
  } else {
    const_cast<float*>(part)[(int64_t)j * 64 * stride + i] = acc;
  }
}

int fold_multi(FoldSegs f, hipStream_t stream, const char* fn) {
  if (f.nseg < 1 || f.nseg > kFoldMaxSegs) return set_error(TPF_ERR_ARG, "%s: bad fold segments", fn);
  for (;;) {
    // Segments with more than 64 splits take a 64-chunk pass; the others wait.
    FoldSegs p = f;
    p.nseg = 0;
    int groups = 0;
    int64_t maxn = 0;
    for (int sg = 0; sg < f.nseg; ++sg) {
      if (f.splits[sg] <= 64) continue;
      const int k = p.nseg++;
      p.part[k] = f.part[sg]; p.n[k] = f.n[sg]; p.stride[k] = f.stride[sg];
      p.splits[k] = f.splits[sg]; p.gbase[k] = groups;
      groups += (f.splits[sg] + 63) / 64;
      maxn = f.n[sg] > maxn ? f.n[sg] : maxn;
    }
    if (p.nseg == 0) break;
    hipLaunchKernelGGL(fold_multi_kernel, dim3((unsigned)((maxn + 255) / 256), (unsigned)groups),
                       dim3(256), 0, stream, p, 0);
    int rc = check_launch(fn);
    if (rc) return rc;
    for (int sg = 0; sg < f.nseg; ++sg)
      if (f.splits[sg] > 64) {
        f.splits[sg] = (f.splits[sg] + 63) / 64;
        f.stride[sg] *= 64;
      }
  }
  int64_t maxn = 0;
  for (int sg = 0; sg < f.nseg; ++sg) {
    f.gbase[sg] = sg;
    maxn = f.n[sg] > maxn ? f.n[sg] : maxn;
  }
  hipLaunchKernelGGL(fold_multi_kernel, dim3((unsigned)((maxn + 255) / 256), (unsigned)f.nseg),
                     dim3(256), 0, stream, f, 1);
  return check_launch(fn);
}

static int gemm_prepare(GemmArgs& g, int a_kc, int b_kc, int out_f32, int batch, const char* fn) {
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

int gemm_launch(const GemmArgs& g0, int a_kc, int b_kc, int out_f32, int batch,
                hipStream_t stream, const char* fn) {
  GemmArgs g = g0;
  int rc = gemm_prepare(g, a_kc, b_kc, out_f32, batch, fn);
  if (rc) return rc;
  dim3 grid((unsigned)((gemm_tiles(g) + 7) / 8 * 8));
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

int gemm_launch_pair(const GemmArgs& p0, int a_kc0, int b_kc0, const GemmArgs& p1, int a_kc1,
                     int b_kc1, int out_f32, hipStream_t stream, const char* fn) {
  GemmArgs g0 = p0, g1 = p1;
  int rc = gemm_prepare(g0, a_kc0, b_kc0, out_f32, p0.batch > 0 ? p0.batch : 1, fn);
  if (rc) return rc;
  if ((rc = gemm_prepare(g1, a_kc1, b_kc1, out_f32, p1.batch > 0 ? p1.batch : 1, fn))) return rc;
  const int64_t blocks = (gemm_tiles(g0) + 7) / 8 * 8 + (gemm_tiles(g1) + 7) / 8 * 8;
  if (blocks > INT32_MAX) return set_error(TPF_ERR_SHAPE, "%s: GEMM grid too large", fn);
  dim3 grid((unsigned)blocks);
#define TPF_GEMM_PAIR_CASE(A0, B0, A1, B1, OF)                                                \
  if (a_kc0 == A0 && b_kc0 == B0 && a_kc1 == A1 && b_kc1 == B1 && out_f32 == OF) {             \
    hipLaunchKernelGGL((gemm_bf16_pair_kernel<A0, B0, A1, B1, OF>), grid, dim3(256), 0, stream,  \
                       g0, g1);                                                               \
    return check_launch(fn);                                                                  \
  }
  TPF_GEMM_PAIR_CASE(0, 0, 0, 0, 1)  // TriMul weight gradients
  TPF_GEMM_PAIR_CASE(1, 0, 0, 0, 0)  // TriMul contraction backward (dA, dB)
#undef TPF_GEMM_PAIR_CASE
  return set_error(TPF_ERR_ARG, "%s: GEMM pair layout not instantiated", fn);
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

// Weight gradient of a linear layer over many rows: dW[m][n] = sum_r dy[r][m] x[r][n]
// (dy [R][M] and x [R][N] row-major bf16, both read MN-contiguous), split over
// R with f32 partials and the fixed-order fold (deterministic).  The shape
// of every projection weight gradient of the pair stack (K = B*N^2 rows).
static int wgrad_splits(int64_t R, int64_t M, int64_t N) {
  const int64_t tiles = ((M + tpf::kGM - 1) / tpf::kGM) * ((N + tpf::kGN - 1) / tpf::kGN);
  int64_t s = (512 + tiles - 1) / tiles;
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
  int rc = tpf::gemm_launch(g, 0, 0, 1, 1, s, fn);
  if (rc) return rc;
  return tpf::fold_launch((const float*)workspace, dw, M * N, M * N, splits, s, fn);
}
