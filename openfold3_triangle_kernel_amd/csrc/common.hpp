// Shared device helpers for the gfx950 (CDNA4) TurboPairFormer kernels.
//
// Everything here is written for 64-lane wavefronts and the gfx950 bf16 MFMA
// instructions (v_mfma_f32_32x32x16_bf16).  Operand layouts of that
// instruction, as used by every kernel in this library:
//
//   A (32 x 16, row-major in k):  lane l holds A[l % 32][8*(l/32) .. +8]
//   B (16 x 32, col-major in k):  lane l holds B[8*(l/32) .. +8][l % 32]
//   C (32 x 32):                  lane l, register r holds
//                                 C[8*(r/4) + 4*(l/32) + (r%4)][l % 32]
//
// The k index is a pure summation index, so any permutation applied to both
// A and B gives the same product; the attention kernels use this to feed a
// C-layout tile straight back in as a B operand without moving data.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tpf {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

__device__ __forceinline__ float bf2f(u16 h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
__device__ __forceinline__ float bf2f(__bf16 h) { return static_cast<float>(h); }

// Round-to-nearest-even f32 -> bf16 (hardware v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ __bf16 f2bf(float f) { return static_cast<__bf16>(f); }
typedef uint32_t u32x2 __attribute__((__vector_size__(8)));
__device__ __forceinline__ u16 f2bf_bits(float f) {
  __bf16 h = static_cast<__bf16>(f);
  return *reinterpret_cast<u16*>(&h);
}

// Exchange with lane l ^ 32 through v_permlane32_swap; returns the pair
// (lower-half value, upper-half value) so symmetric reductions combine the
// two in the same order on both halves (bitwise identical results).
__device__ __forceinline__ float xor32_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                            false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                            false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Exchange with lane l ^ 16 through v_permlane16_swap (rows of 16 lanes
// swapped pairwise), summed in the order (even row) + (odd row) on both rows.
__device__ __forceinline__ float xor16_sum(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                            false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Cross-lane moves on the VALU (DPP), no LDS round trip.  Controls used:
// quad_perm [1,0,3,2] (lane ^ 1), quad_perm [2,3,0,1] (lane ^ 2),
// row_half_mirror (lane ^ 7 within 8-lane blocks), row_ror:8 (lane ^ 8
// within rows of 16).
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppXor8 = 0x128;
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of L lanes (L a power of two <= 64); every lane
// of a group ends with the same bits (each level adds a lane pair's values,
// a + b on one lane and b + a on the other).
template <int L>
__device__ __forceinline__ float lanes_sum(float x) {
  static_assert(L >= 1 && L <= 64 && (L & (L - 1)) == 0, "lane group");
  if constexpr (L >= 2) x += dpp_f<kDppXor1>(x);
  if constexpr (L >= 4) x += dpp_f<kDppXor2>(x);
  if constexpr (L >= 8) x += dpp_f<kDppHalfMirror>(x);
  if constexpr (L >= 16) x += dpp_f<kDppXor8>(x);
  if constexpr (L >= 32) x = xor16_sum(x);
  if constexpr (L >= 64) x = xor32_sum(x);
  return x;
}
__device__ __forceinline__ float row16_sum(float x) { return lanes_sum<16>(x); }

// Partner value for one level of a transposing butterfly over lanes: a lane
// whose level bit H differs and whose bits above H agree (exact xor for
// H = 1, 2, 8, 16, 32; for H = 4 the mirror lane ^ 7 of its 8-lane block).
template <int H>
__device__ __forceinline__ float butterfly_partner(float x, int lane) {
  if constexpr (H == 1) {
    return dpp_f<kDppXor1>(x);
  } else if constexpr (H == 2) {
    return dpp_f<kDppXor2>(x);
  } else if constexpr (H == 4) {
    return dpp_f<kDppHalfMirror>(x);
  } else if constexpr (H == 8) {
    return dpp_f<kDppXor8>(x);
  } else if constexpr (H == 16) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float((lane & 16) ? r[0] : r[1]);
  } else {
    static_assert(H == 32, "butterfly level");
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float((lane & 32) ? r[0] : r[1]);
  }
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Logistic function with the hardware reciprocal (v_rcp_f32, 1 ulp): the
// IEEE division of 1 / (1 + e^-x) costs about ten VALU instructions, and every
// consumer rounds the result (or its products) to bf16.  x = -inf gives
// rcp(inf) = 0, x = +inf gives 1.
__device__ __forceinline__ float sigmoidf(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }

// 16-byte global load/store of 8 bf16 values.
__device__ __forceinline__ bf16x8 ld8(const __bf16* p) {
  return *reinterpret_cast<const bf16x8*>(p);
}
// Streaming loads of data read once (fold partials): nontemporal, so they do
// not displace reused lines from the caches.
__device__ __forceinline__ bf16x8 ld8_nt(const __bf16* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(p));
}
__device__ __forceinline__ f32x4 ld4f_nt(const float* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
}
__device__ __forceinline__ void st8(__bf16* p, bf16x8 v) {
  *reinterpret_cast<bf16x8*>(p) = v;
}
__device__ __forceinline__ bf16x4 ld4(const __bf16* p) {
  return *reinterpret_cast<const bf16x4*>(p);
}

__device__ __forceinline__ bf16x8 zero8() {
  bf16x8 z;
#pragma unroll
  for (int i = 0; i < 8; ++i) z[i] = static_cast<__bf16>(0.f);
  return z;
}

// Transposing LDS read (ds_read_b64_tr_b16).  In each 16-lane group every
// lane supplies the address of 4 consecutive bf16; lane j of the group
// receives element j % 4 of the chunks supplied by lanes 4e + j / 4
// (e = 0..3).  tr_col4 uses it to fetch a column fragment of a row-major LDS
// matrix M (pitch in elements): lane l receives
//   { M[r0 + e][c0 + (l % 32)] : e = 0..3 },  r0 = rbase_lo (l < 32) or rbase_hi.
// Rows are 8-byte aligned when pitch and c0 are multiples of 4.
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
__device__ __forceinline__ bf16x4 tr_col4(const __bf16* M, int pitch, int rbase_lo, int rbase_hi,
                                          int c0) {
  const int l = threadIdx.x & 63, g = l >> 4, ip = l & 15;
  const int r = ((g >> 1) ? rbase_hi : rbase_lo) + (ip >> 2);
  const __bf16* p = M + r * pitch + c0 + 16 * (g & 1) + 4 * (ip & 3);
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p);
}

__device__ __forceinline__ bf16x8 cat8(bf16x4 lo, bf16x4 hi) {
  bf16x8 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) { o[e] = lo[e]; o[4 + e] = hi[e]; }
  return o;
}

// Pack registers r0..r0+7 of a C-layout tile into a bf16 B operand.
__device__ __forceinline__ bf16x8 pack8(const f32x16& c, int r0) {
  bf16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = f2bf(c[r0 + e]);
  return o;
}

// LDS byte offset of a generic pointer into LDS: its low 32 bits (the flat
// LDS aperture keeps the offset there).  Truncating the generic address
// instead of an address-space cast avoids the cast's null-pointer select.
__device__ __forceinline__ unsigned lds_offset(const void* p) {
  return (unsigned)(uintptr_t)p;
}

// Direct 16-byte global -> LDS load (global_load_lds_dwordx4): lane i writes
// dst_base + 16*i.  Issued through inline assembly so the compiler does not
// guard every later LDS read with a full vmcnt wait; callers wait explicitly
// (wait_vmcnt) before reading the destination.  dst_base must be uniform.
__device__ __forceinline__ void g2lds16(const void* src, void* dst_base) {
  const unsigned lds = __builtin_amdgcn_readfirstlane(lds_offset(dst_base));
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :: "v"(src), "s"(lds) : "memory", "m0");
}

// s_waitcnt vmcnt(n) leaving the other counters untouched (gfx9 encoding).
template <int n>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(n >= 0 && n < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier that waits only for this wave's LDS operations (the
// memory clobbers keep the compiler from moving memory accesses across it).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt / expcnt untouched
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Buffer resource of a raw (unstructured) buffer starting at base.  The
// range is 2^31 - 1 bytes, so an offset of kBufOOB (2^31) reads as zeros:
// loaders use it for elements outside the tensor instead of branching.
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t kBufOOB = 0x80000000u;
__device__ __forceinline__ i32x4 buffer_rsrc(const void* base) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xFFFFu));
  r[2] = 0x7FFFFFFF;
  r[3] = 0x00020000;
  return r;
}

// Direct 16-byte buffer -> LDS load (buffer_load_dwordx4 ... lds): lane i
// writes dst_base + 16*i with the 16 bytes at byte offset voff of the
// buffer (zeros when voff is out of range).  Same waiting rules as g2lds16.
__device__ __forceinline__ void buf2lds16(i32x4 rsrc, uint32_t voff, void* dst_base) {
  const unsigned lds = __builtin_amdgcn_readfirstlane(lds_offset(dst_base));
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :: "s"(lds), "v"(voff), "s"(rsrc) : "memory", "m0");
}

// buf2lds16 with a uniform byte offset `soff` (an SGPR) added to every
// lane's voff: a loop advances soff on the scalar unit while the per-lane
// offsets stay fixed.  voff = kBufOOB still reads zeros.
__device__ __forceinline__ void buf2lds16_so(i32x4 rsrc, uint32_t voff, uint32_t soff,
                                             void* dst_base) {
  const unsigned lds = __builtin_amdgcn_readfirstlane(lds_offset(dst_base));
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :: "s"(lds), "v"(voff), "s"(rsrc), "s"(soff) : "memory", "m0");
}

// Raw buffer resource over [base, base + 2^31 - 1) for the load/store
// builtins; a byte offset of kBufOOB reads zeros and drops stores.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7FFFFFFF, 0x00020000);
}
// Branch-free 16-byte / 4-byte loads through a buffer resource (zeros at
// kBufOOB): a run of them issues back to back and is waited on once.
__device__ __forceinline__ bf16x8 buf_ld8(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0));
}
__device__ __forceinline__ float buf_ldf(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, 0, 0));
}

// Division by a run-time invariant d (Granlund-Montgomery): for n < 2^31,
// n / d = (umulhi(n, m) + n) >> s with s = ceil(log2 d),
// m = floor(2^32 (2^s - d) / d) + 1.  Replaces 32/64-bit integer division
// (dozens of instructions each) in index arithmetic.
struct FastDiv {
  uint32_t d, m, s;
};
inline FastDiv make_fastdiv(uint32_t d) {
  uint32_t s = 0;
  while ((1ull << s) < d) ++s;
  const uint64_t m = ((1ull << 32) * ((1ull << s) - d)) / d + 1;
  return FastDiv{d, (uint32_t)m, s};
}
__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
  return (__umulhi(n, f.m) + n) >> f.s;
}

}  // namespace tpf
