// Weight-stationary row GEMM on gfx950: y[R, N] = x[R, K] W^T for a tall x
// (R = the pair rows of a module, up to millions) and a small weight W
// (N x K bf16, N and K at most a few hundred), bf16 in and out, f32
// accumulation.  These are the projections of the triangle-attention module
// (x_ln W_all^T, og W_o^T, dout W_o; K = 128): the 128 x 128 tile GEMM
// spends most of a short-K tile in its prologue and epilogue and re-reads
// each x tile once per output tile column, while here every workgroup keeps
// its slice of W in registers for the whole launch and streams x once.
//
// Launch: one persistent workgroup of 8 waves per CU walks 32-row blocks
// strided by the grid size.  Wave w owns the output tiles t = w, w + 8, ... (16
// channels each, t < N / 16) and holds their weight rows as the A operands
// of v_mfma_f32_16x16x32_bf16 (MT x KS registers of 8 bf16, K = 32 KS).
// Waves 0-3 stream x blocks into a DEPTH-deep LDS ring with direct
// buffer->LDS loads (rows chunk-rotated, so the 16 rows of a fragment read
// hit distinct banks); waves 4-7 store: each block's outputs are staged in
// LDS as [row][N] bf16 (two buffers) and leave as 16-byte row chunks.  The
// loading waves issue only loads and the storing waves only stores, so each
// side's vmcnt waits count its own operations.
//
// Each output element is sum_k x[r, k] W[n, k] in one fixed MFMA order
// (k-steps ascending), whatever the row's block or position in it, so a row
// gives the same bits in any launch (row chunks equal the whole).

#include "common.hpp"
#include "tpf_gemm.hpp"
#include "tpf_status.hpp"

namespace tpf {

constexpr int kRowNW = 8;  // waves per workgroup

template <int KS>
constexpr int row_depth() { return KS <= 4 ? 4 : 3; }
// (K = 576, the dx = dproj W_all product, measured slower here than on the
// tile GEMM, 216 against 197 us at 589,824 rows, and is left to it.)

// Split destination of the triangle-attention projection (SPLIT = true):
// output columns [0, 3 H D) are q | k | v and go to head-major planes
// qkv[part][b][i][h][j][d] (the layout the attention kernels stream as
// contiguous 2 KB tiles), the rest (gate | bias | pad) to rows of pitch
// ldy in y.  Row r = (b, i, j) of the pair grid; a 32-row block lies in one
// (b, i) because the sequence length is a multiple of 32.
struct RowSplit {
  __bf16* qkv;
  int64_t part_elems;  // B * N * H * N * D
  int Nseq, H, D;
};

// Gate-backward epilogue of the triangle-attention module (MODE = kRowGate /
// kRowGateShadow): the product is d_og = dout W_o (hc = H D columns) of the
// pair rows r = (b, i, j), and instead of storing it the kernel applies the
// backward of og = o * sigmoid(g):
//   d_o   = d_og * s                      (bf16, rows [R, hc])
//   dgate = d_og * o * s * (1 - s)        (bf16, columns [0, hc) of rows of
//                                          pitch dpitch)
//   delta[b, i, h, j] = sum_d d_o * o~    (f32; o~ = o, or o + its rounding
//                                          residual res with the shadow)
// with s = sigmoid(gate).  o, res and the gate rows (pitch gpitch) stream
// through the LDS ring beside x.  og_t: dout holds pair row (b, i, j) at row
// (b, j, i) (the ending node's caller order), gathered by the loader.
struct RowGate {
  const __bf16* o;
  const __bf16* res;
  const __bf16* gate;
  int64_t gpitch;
  __bf16* d_o;
  float* delta;
  __bf16* dgate;
  int64_t dpitch;
  int Nseq, H, D, og_t;
  FastDiv fbp, fN;  // 32-row blocks per (b, i) plane (N / 32), and N
};

constexpr int kRowPlain = 0, kRowSplit = 1, kRowGate = 2, kRowGateShadow = 3;

template <int KS, int MT, int MODE>
__global__ __launch_bounds__(64 * kRowNW) void rowgemm_ws_kernel(
    const __bf16* __restrict__ x, int64_t ldx, const __bf16* __restrict__ w, int w_kc,
    int64_t ldw, __bf16* __restrict__ y, int64_t ldy, int64_t R, int N, int64_t nblocks,
    RowSplit sp, RowGate gt) {
  constexpr bool SPLIT = MODE == kRowSplit;
  constexpr bool GATE = MODE >= kRowGate;
  constexpr int K = 32 * KS;
  constexpr int CPR = K / 8;               // 16-byte chunks per x row
  constexpr int DEPTH = row_depth<KS>();
  constexpr int XCH = 32 * CPR;            // chunks of one x block
  static_assert(XCH % 256 == 0, "x block splits evenly over the loading waves");
  constexpr int NMAX = 16 * kRowNW * MT;  // widest output the instance serves
  // Gate mode: side arrays o, gate (and res) of a block, N / 8 chunks per row.
  constexpr int NSIDE = MODE == kRowGateShadow ? 3 : 2;
  constexpr int LPS = GATE ? 32 * NMAX / 8 / 256 : 0;  // side loads per array and thread
  static_assert(!GATE || MT == 1, "the gate epilogue serves N <= 128");
  constexpr int LPT = XCH / 256 + (GATE ? NSIDE * LPS : 0);  // loads per loading thread per block
  __shared__ __attribute__((aligned(1024))) __bf16 Xs[DEPTH][32 * K];
  __shared__ __attribute__((aligned(16))) __bf16 Ys[2 * 32 * (NMAX + 8)];  // [2][32][N + 8]
  __shared__ __attribute__((aligned(16))) __bf16 Ss[GATE ? DEPTH * NSIDE : 1][GATE ? 32 * NMAX : 8];
  const int YP = N + 8;

  const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int l16 = lane & 15, lg = lane >> 4;
  const bool loader = wv < kRowNW / 2;
  const int tiles = N / 16;

  // Stationary A operands: channel 16 t + l16, k chunk 4 ks + lg.
  bf16x8 wf[MT][KS];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const int t = wv + kRowNW * m;
    const int ch = 16 * (t < tiles ? t : 0) + l16;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int k0 = 8 * (4 * ks + lg);
      if (w_kc) {
        wf[m][ks] = ld8(w + (int64_t)ch * ldw + k0);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) wf[m][ks][e] = w[(int64_t)(k0 + e) * ldw + ch];
      }
    }
  }

  // Workgroup g takes blocks g, g + G, g + 2 G, ... (G = grid size), so at
  // any time the grid works on a compact window of consecutive blocks (DRAM
  // pages shared across workgroups): measured 56 -> 51 us on the plain
  // product and 219 -> 207 us on the gate epilogue at 589,824 rows, against
  // one contiguous range per workgroup.  Buffer resources are based at each
  // block's first row (64-bit address arithmetic on the scalar unit), so the
  // 32-bit lane offsets stay small for any row count.
  const int64_t nit =
      blockIdx.x < nblocks ? (nblocks - blockIdx.x + gridDim.x - 1) / gridDim.x : 0;
  auto gb = [&](int64_t it) { return (int64_t)blockIdx.x + it * gridDim.x; };
  // Loading thread i of 256 takes chunks ci = 256 j + i of the block: row
  // r = ci / CPR, stored at slot (c + r) % CPR of its row.
  // Gate mode: a loading thread's side chunks ci = 256 j + tid are (row
  // ci / (N / 8), chunk ci % (N / 8)) of the block, stored unrotated at
  // element 8 ci of the stage; their byte offsets are the same every block.
  uint32_t side_o[GATE ? LPS : 1], side_g[GATE ? LPS : 1];
  if constexpr (GATE) {
    const int cpr = N / 8;
#pragma unroll
    for (int j = 0; j < LPS; ++j) {
      const int ci = 256 * j + tid, r = ci / cpr, c = ci - r * cpr;
      const bool ok = loader && ci < 32 * cpr;
      side_o[j] = ok ? (uint32_t)((r * N + 8 * c) * 2) : kBufOOB;
      side_g[j] = ok ? (uint32_t)((r * gt.gpitch + 8 * c) * 2) : kBufOOB;
    }
  }
  auto issue = [&](int64_t it) {
    const int stage = (int)(it % DEPTH);
    const bool vb = it < nit;
    const int64_t bb = vb ? gb(it) : 0;
    // x rows of the block: consecutive, or (og_t) the pair rows
    // (b, i, j0 + r) at dout rows (b, j0 + r, i), N rows apart.
    int64_t xrow0 = bb * 32, xstride = ldx;
    if constexpr (GATE) {
      if (gt.og_t) {
        const uint32_t bi = fdiv((uint32_t)bb, gt.fbp), j0 = ((uint32_t)bb - bi * gt.fbp.d) * 32;
        const uint32_t b = fdiv(bi, gt.fN), i = bi - b * gt.fN.d;
        xrow0 = ((int64_t)b * gt.Nseq + j0) * gt.Nseq + i;
        xstride = gt.Nseq * ldx;
      }
    }
    const i32x4 rs_x = buffer_rsrc(x + xrow0 * ldx);
#pragma unroll
    for (int j = 0; j < XCH / 256; ++j) {
      const int ci = 256 * j + tid;
      const int r = ci / CPR, slot = ci % CPR;
      const int gc = (slot - r % CPR + CPR) % CPR;
      const bool ok = vb && bb * 32 + r < R;
      buf2lds16(rs_x, ok ? (uint32_t)((r * xstride + 8 * gc) * 2) : kBufOOB,
                &Xs[stage][(256 * j + 64 * wv) * 8]);
    }
    if constexpr (GATE) {
      const bool ok = vb;
      const i32x4 rs_o = buffer_rsrc(gt.o + bb * 32 * N);
      const i32x4 rs_g = buffer_rsrc(gt.gate + bb * 32 * gt.gpitch);
#pragma unroll
      for (int j = 0; j < LPS; ++j) {
        const int dst = (256 * j + 64 * wv) * 8;
        buf2lds16(rs_o, ok ? side_o[j] : kBufOOB, &Ss[stage * NSIDE][dst]);
        buf2lds16(rs_g, ok ? side_g[j] : kBufOOB, &Ss[stage * NSIDE + 1][dst]);
        if constexpr (NSIDE == 3)
          buf2lds16(buffer_rsrc(gt.res + bb * 32 * N), ok ? side_o[j] : kBufOOB,
                    &Ss[stage * NSIDE + 2][dst]);
      }
    }
  };
  // Split destination: storing thread st's chunks i (q = st + 256 i of the
  // block) are numbered so that consecutive lanes write consecutive
  // addresses: first the q | k | v segments (part, head) of 32 rows x D (2 KB
  // contiguous in a plane at D = 32), a row's chunks fastest; then the rest
  // rows (contiguous: their pitch is the rest width).  The map is the same
  // for every block (offsets relative to the block's plane and row bases),
  // so it is formed once, off the block loop.
  struct SplitChunk { int64_t off; int lds, row; bool rest; };
  constexpr int SIT = (32 * NMAX / 8 + 255) / 256;
  SplitChunk smap[SPLIT ? SIT : 1];
  if constexpr (SPLIT) {
    const int st = tid - 256, cpr = N / 8, nch = 32 * cpr;
    const int hc = sp.H * sp.D, dch = sp.D / 8;
    const int seg_ch = 32 * dch, nq = 3 * sp.H * seg_ch, rcpr = cpr - 3 * hc / 8;
#pragma unroll
    for (int i = 0; i < SIT; ++i) {
      const int q = st + 256 * i;
      SplitChunk m{0, -1, 0, false};
      if (!loader && q < nch) {
        if (q < nq) {
          const int seg = q / seg_ch, in = q - seg * seg_ch;
          const int part = seg / sp.H, h = seg - part * sp.H;
          const int row = in / dch, dc = in - row * dch;
          m = SplitChunk{part * sp.part_elems + ((int64_t)h * sp.Nseq + row) * sp.D + 8 * dc,
                         row * YP + part * hc + h * sp.D + 8 * dc, row, false};
        } else {
          const int u = q - nq, row = u / rcpr, k = u - row * rcpr;
          m = SplitChunk{row * ldy + 8 * k, row * YP + 3 * hc + 8 * k, row, true};
        }
      }
      smap[i] = m;
    }
  }
  if (loader) {
#pragma unroll
    for (int d = 0; d < DEPTH - 1; ++d) issue(d);
    wait_vmcnt<LPT * (DEPTH - 2)>();  // the first block landed
  }
  __syncthreads();
#pragma unroll 1
  for (int64_t it = 0; it < nit; ++it) {
    const int64_t blk = gb(it);
    const int stage = (int)(it % DEPTH);
    __bf16* Yb = Ys + (int)(it & 1) * 32 * YP;
    if (loader) issue(it + DEPTH - 1);
    const __bf16* Xb = Xs[stage];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const int t = wv + kRowNW * m;
      if (t >= tiles) break;  // wave-uniform
      f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
          const int row = 16 * rt + l16;
          const bf16x8 af =
              *reinterpret_cast<const bf16x8*>(&Xb[row * K + 8 * ((4 * ks + lg + row) % CPR)]);
          acc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[m][ks], af, acc[rt], 0, 0, 0);
        }
      // The weight rows are the A operand, so the tile comes out transposed:
      // register e of lane l holds row 16 rt + l16, channel 16 t + 4 lg + e,
      // and each lane writes 4 consecutive channels of one row at once.
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        bf16x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = f2bf(acc[rt][e]);
        *reinterpret_cast<bf16x4*>(&Yb[(16 * rt + l16) * YP + 16 * t + 4 * lg]) = o;
      }
    }
    // Gate mode: the storing waves take block blk's side chunks out of the
    // ring now, before the barrier after which the loaders refill the stage.
    constexpr int GIT = GATE ? 32 * NMAX / 8 / 256 : 1;
    bf16x8 so[GIT], sg[GIT], sr[GIT];
    if constexpr (GATE) {
      if (!loader) {
#pragma unroll
        for (int i = 0; i < GIT; ++i) {
          const int e = 8 * (tid - 256 + 256 * i);
          so[i] = *reinterpret_cast<const bf16x8*>(&Ss[stage * NSIDE][e]);
          sg[i] = *reinterpret_cast<const bf16x8*>(&Ss[stage * NSIDE + 1][e]);
          if constexpr (NSIDE == 3) sr[i] = *reinterpret_cast<const bf16x8*>(&Ss[stage * NSIDE + 2][e]);
        }
      }
    }
    if (loader) wait_vmcnt<LPT * (DEPTH - 2)>();  // block blk + 1 landed
    __syncthreads();
    if constexpr (GATE) {
      if (!loader) {
        // Block rows r0 .. r0 + 31 = (b, i, j0 .. j0 + 31); chunk q = st +
        // 256 i is (row q / (N / 8), chunk c = q % (N / 8)); the D / 8
        // chunks of head h = c / (D / 8) are consecutive lanes of one wave
        // (D / 8 divides 64), so the head's sum gathers them by lane.
        const int st = tid - 256, cpr = N / 8, d8 = gt.D / 8;
        const int64_t r0 = blk * 32;
        const uint32_t bi = fdiv((uint32_t)blk, gt.fbp);
        const int j0 = (int)((uint32_t)blk - bi * gt.fbp.d) * 32;
#pragma unroll
        for (int i = 0; i < GIT; ++i) {
          const int q = st + 256 * i, row = q / cpr, c = q - row * cpr;
          const bool act = q < 32 * cpr;
          float sdot = 0.f;
          if (act) {
            const bf16x8 dv = *reinterpret_cast<const bf16x8*>(&Yb[row * YP + 8 * c]);
            bf16x8 r_do, r_dg;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const float sgm = sigmoidf(bf2f(sg[i][e]));
              const float dd = bf2f(dv[e]), oo = bf2f(so[i][e]);
              r_do[e] = f2bf(dd * sgm);
              r_dg[e] = f2bf(dd * oo * sgm * (1.f - sgm));
              // delta pairs the bf16 d_o the attention backward reads with
              // o (with the shadow, o + its residual, summed in f32).
              sdot = fmaf(bf2f(r_do[e]), NSIDE == 3 ? oo + bf2f(sr[i][e]) : oo, sdot);
            }
            st8(gt.d_o + (r0 + row) * N + 8 * c, r_do);
            st8(gt.dgate + (r0 + row) * gt.dpitch + 8 * c, r_dg);
          }
          const int lane_q = lane;
          float hs = 0.f;
          for (int u = 0; u < d8; ++u) hs += __shfl(sdot, lane_q + u);
          if (act && c % d8 == 0)
            gt.delta[((int64_t)bi * gt.H + c / d8) * gt.Nseq + j0 + row] = hs;
        }
      }
    } else if (!loader) {
      // 32 rows x N / 8 chunks over the 256 storing threads: every LDS read
      // first, then the stores back to back.
      constexpr int SIT = (32 * NMAX / 8 + 255) / 256;
      const int st = tid - 256, cpr = N / 8;
      const int nch = 32 * cpr;
      if constexpr (!SPLIT) {
        const __amdgpu_buffer_rsrc_t rs_y =
            __builtin_amdgcn_make_buffer_rsrc(y + blk * 32 * ldy, 0, 0x7FFFFFFF, 0x00020000);
        bf16x8 v[SIT];
        uint32_t off[SIT];
#pragma unroll
        for (int i = 0; i < SIT; ++i) {
          const int q = st + 256 * i;
          const int row = q / cpr, k = q - row * cpr;
          const bool ok = q < nch && blk * 32 + row < R;
          v[i] = *reinterpret_cast<const bf16x8*>(&Yb[(q < nch ? row * YP + 8 * k : 0)]);
          off[i] = ok ? (uint32_t)((row * ldy + 8 * k) * 2) : kBufOOB;
        }
#pragma unroll
        for (int i = 0; i < SIT; ++i)
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v[i]), rs_y, off[i], 0, 0);
      } else {
        // Block rows r0 .. r0 + 31 = (b, i, j0 .. j0 + 31).
        const int64_t r0 = blk * 32;
        const int64_t bi = r0 / sp.Nseq;               // b * N + i
        const int j0 = (int)(r0 - bi * sp.Nseq);
        // Per-thread chunk map (the same for every block): see split_map.
        __bf16* const qbase = sp.qkv + (bi * sp.H * sp.Nseq + j0) * sp.D;
        __bf16* const rbase = y + r0 * ldy;
        bf16x8 v[SIT];
        __bf16* dst[SIT];
#pragma unroll
        for (int i = 0; i < SIT; ++i) {
          const bool ok = smap[i].lds >= 0 && r0 + smap[i].row < R;
          v[i] = *reinterpret_cast<const bf16x8*>(&Yb[ok ? smap[i].lds : 0]);
          dst[i] = ok ? (smap[i].rest ? rbase : qbase) + smap[i].off : nullptr;
        }
#pragma unroll
        for (int i = 0; i < SIT; ++i)
          if (dst[i]) st8(dst[i], v[i]);
      }
    }
  }
  // The ring loads issued past the last block still write LDS: let them land
  // before the workgroup releases its LDS.
  if (loader) wait_vmcnt<0>();
}

// Runs y = x W^T on the row kernel when the shape has an instance (K = 128,
// N a multiple of 16 with N / 16 <= 8 MT, 16-byte aligned rows and
// row pitches below 2^26 bytes); returns false (nothing launched) otherwise.
bool rowgemm_try(const __bf16* x, int64_t ldx, const __bf16* w, int w_kc, int64_t ldw, __bf16* y,
                 int64_t ldy, int64_t R, int64_t N, int64_t K, hipStream_t stream, int* rc,
                 const char* fn) {
  if (R < 1 || N < 16 || N % 16 || N > 640 || ldx % 8 || ldy % 8 || ldx < K || ldy < N ||
      (uintptr_t)x % 16 || (uintptr_t)y % 16 || (w_kc && (ldw % 8 || (uintptr_t)w % 16)) ||
      ldw < (w_kc ? K : N))
    return false;
  // Lane offsets inside one 32-row block stay below 2^31 bytes.
  if (32 * ldx * 2 >= (int64_t)kBufOOB || 32 * ldy * 2 >= (int64_t)kBufOOB) return false;
  const int tiles = (int)(N / 16);
  const int64_t nblocks = (R + 31) / 32;
  const unsigned grid = (unsigned)(nblocks < device_cus() ? nblocks : device_cus());
#define TPF_ROW_CASE(KS, MT)                                                                   \
  if (K == 32 * KS && tiles <= kRowNW * MT) {                                                  \
    hipLaunchKernelGGL((rowgemm_ws_kernel<KS, MT, kRowPlain>), dim3(grid), dim3(64 * kRowNW),  \
                       0, stream, x, ldx, w, w_kc, ldw, y, ldy, R, (int)N, nblocks, RowSplit{}, \
                       RowGate{});                                                             \
    *rc = check_launch(fn);                                                                    \
    return true;                                                                               \
  }
  TPF_ROW_CASE(4, 1)   // K = 128, N <= 128: linear_o, d_og
  TPF_ROW_CASE(4, 5)   // K = 128, N <= 640: the q | k | v | gate | bias projection
#undef TPF_ROW_CASE
  return false;
}

bool rowgemm_gate_supported(int64_t C, int64_t H, int64_t D) {
  const int64_t hc = H * D;
  return C == 128 && (D == 8 || D == 16 || D == 32 || D == 64) && hc % 16 == 0 && hc <= 128;
}

int rowgemm_gate_bwd(const __bf16* dout, const __bf16* w_o, int64_t C, const __bf16* o,
                     const __bf16* res, const __bf16* gate, int64_t gpitch, __bf16* d_o,
                     float* delta, __bf16* dgate, int64_t dpitch, int64_t B, int64_t N, int64_t H,
                     int64_t D, int og_t, hipStream_t stream, const char* fn) {
  const int64_t hc = H * D, R = B * N * N;
  if (!rowgemm_gate_supported(C, H, D) || N % 32 || gpitch % 8 || dpitch % 8)
    return set_error(TPF_ERR_SHAPE, "%s: no fused gate-backward instance for C=%lld H=%lld D=%lld",
                     fn, (long long)C, (long long)H, (long long)D);
  if (((uintptr_t)dout | (uintptr_t)w_o | (uintptr_t)o | (uintptr_t)res | (uintptr_t)gate |
       (uintptr_t)d_o | (uintptr_t)dgate) % 16)
    return set_error(TPF_ERR_ARG, "%s: operands must be 16-byte aligned", fn);
  // Lane offsets within one 32-row block (dout rows N apart with og_t).
  if (32 * (og_t ? N : 1) * C * 2 >= (int64_t)kBufOOB || 32 * gpitch * 2 >= (int64_t)kBufOOB)
    return set_error(TPF_ERR_SHAPE, "%s: N=%lld too large for 32-bit block offsets", fn,
                     (long long)N);
  const int64_t nblocks = R / 32;
  if (nblocks >= (int64_t)1 << 31)
    return set_error(TPF_ERR_SHAPE, "%s: %lld row blocks exceed 2^31", fn, (long long)nblocks);
  const unsigned grid = (unsigned)(nblocks < device_cus() ? nblocks : device_cus());
  const RowGate gt{o, res, gate, gpitch, d_o, delta, dgate, dpitch, (int)N, (int)H, (int)D, og_t,
                   make_fastdiv((uint32_t)(N / 32)), make_fastdiv((uint32_t)N)};
  if (res)
    hipLaunchKernelGGL((rowgemm_ws_kernel<4, 1, kRowGateShadow>), dim3(grid), dim3(64 * kRowNW),
                       0, stream, dout, C, w_o, 0, hc, (__bf16*)nullptr, hc, R, (int)hc, nblocks,
                       RowSplit{}, gt);
  else
    hipLaunchKernelGGL((rowgemm_ws_kernel<4, 1, kRowGate>), dim3(grid), dim3(64 * kRowNW), 0,
                       stream, dout, C, w_o, 0, hc, (__bf16*)nullptr, hc, R, (int)hc, nblocks,
                       RowSplit{}, gt);
  return check_launch(fn);
}

}  // namespace tpf

using namespace tpf;

extern "C" int tpf_pair_projection_supported(int64_t P, int64_t K, int64_t N, int64_t H,
                                             int64_t D) {
  return K == 128 && P % 16 == 0 && P <= 640 && N % 32 == 0 && D % 8 == 0 && H >= 1 &&
         P >= 3 * H * D + 8 && (P - 3 * H * D) % 8 == 0;
}

extern "C" int tpf_pair_projection_bf16(const void* x, const void* w, int64_t B, int64_t N,
                                        int64_t C, int64_t P, int64_t H, int64_t D, void* qkv,
                                        void* rest, void* stream) {
  const char* fn = "tpf_pair_projection_bf16";
  if (!x || !w || !qkv || !rest) return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  if (B < 1 || N < 1 || !tpf_pair_projection_supported(P, C, N, H, D))
    return set_error(TPF_ERR_SHAPE, "%s: unsupported shape (C=%lld P=%lld N=%lld H=%lld D=%lld)",
                     fn, (long long)C, (long long)P, (long long)N, (long long)H, (long long)D);
  if (((uintptr_t)x | (uintptr_t)w | (uintptr_t)qkv | (uintptr_t)rest) % 16)
    return set_error(TPF_ERR_ARG, "%s: pointers must be 16-byte aligned", fn);
  const int64_t R = B * N * N, rest_pitch = P - 3 * H * D;
  const int64_t nblocks = (R + 31) / 32;
  const unsigned grid = (unsigned)(nblocks < device_cus() ? nblocks : device_cus());
  const RowSplit sp{(__bf16*)qkv, B * N * H * N * D, (int)N, (int)H, (int)D};
  hipLaunchKernelGGL((rowgemm_ws_kernel<4, 5, kRowSplit>), dim3(grid), dim3(64 * kRowNW), 0,
                     (hipStream_t)stream, (const __bf16*)x, C, (const __bf16*)w, 1, C,
                     (__bf16*)rest, rest_pitch, R, (int)P, nblocks, sp, RowGate{});
  return check_launch(fn);
}
