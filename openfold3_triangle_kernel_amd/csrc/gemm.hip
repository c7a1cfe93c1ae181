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
// Stage shape of this translation unit (measured on the TriMul contraction
// and its dA / dB products: 32-deep k-steps, three stages in flight); the
// split-K weight-gradient products use their own shape (gemm_wgrad.hip).
#define TPF_GEMM_GK 32
#define TPF_GEMM_NS 3
#define TPF_GEMM_IMPL gk32
#include "gemm_impl.hpp"

namespace tpf {

using namespace gk32;

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

// The weight-gradient fold contract of the reference
// (trimul_wgrad_fixed_fold, turbopairformer_trimul_cuda.cu:200-217, 2050-2089):
// accumulator[e] = (((init + p[0][e]) + p[1][e]) + ...) + p[chunks-1][e] in
// round-to-nearest FP32, init = 0 (initialize) or the accumulator's value.
template <bool INIT>
__global__ __launch_bounds__(256) void wgrad_fixed_fold_kernel(const float* __restrict__ part,
                                                               int chunks, int64_t n,
                                                               float* __restrict__ acc) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float sum = INIT ? 0.f : acc[i];
  int c = 0;
  for (; c + 8 <= chunks; c += 8) {  // 8 loads in flight, added in ascending order
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = part[(int64_t)(c + e) * n + i];
#pragma unroll
    for (int e = 0; e < 8; ++e) sum = __fadd_rn(sum, v[e]);
  }
  for (; c < chunks; ++c) sum = __fadd_rn(sum, part[(int64_t)c * n + i]);
  acc[i] = sum;
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


extern "C" int tpf_trimul_wgrad_fixed_fold(const float* partials, int64_t chunks, int64_t elements,
                                           float* accumulator, int initialize, void* stream) {
  const char* fn = "tpf_trimul_wgrad_fixed_fold";
  if (!partials || !accumulator) return tpf::set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  if (chunks < 1 || chunks > INT32_MAX || elements < 1)
    return tpf::set_error(TPF_ERR_SHAPE, "%s: chunks and elements must be positive", fn);
  if ((elements + 255) / 256 > INT32_MAX)
    return tpf::set_error(TPF_ERR_SHAPE, "%s: too many elements", fn);
  const char* pa = (const char*)partials;
  const char* ac = (const char*)accumulator;
  if (ac < pa + chunks * elements * 4 && pa < ac + elements * 4)
    return tpf::set_error(TPF_ERR_ARG, "%s: accumulator overlaps the partials", fn);
  const dim3 grid((unsigned)((elements + 255) / 256));
  if (initialize)
    hipLaunchKernelGGL(tpf::wgrad_fixed_fold_kernel<true>, grid, dim3(256), 0, (hipStream_t)stream,
                       partials, (int)chunks, elements, accumulator);
  else
    hipLaunchKernelGGL(tpf::wgrad_fixed_fold_kernel<false>, grid, dim3(256), 0,
                       (hipStream_t)stream, partials, (int)chunks, elements, accumulator);
  return tpf::check_launch(fn);
}
