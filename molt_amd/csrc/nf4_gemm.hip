// NF4-fused bf16 MFMA GEMMs for the NF4+LoRA linear (gfx950).
//
// Forward   Y[M,N]  = X[M,K] . deq(W[N,K])^T + T[M,r] . bf16(s B[N,r])^T
// Backward  dX[M,K] = dY[M,N] . deq(W[N,K])  + U[M,r] . bf16(A[r,K])
//
// The NF4 weight is dequantised while it is staged into LDS: packed bytes are
// read with 16-byte (forward) or 2-byte-per-row patch (backward) loads, each
// byte is looked up in a 256-entry LDS table of fp32 code pairs, multiplied by
// the block's fp32 scale and rounded to bf16 (the same bf16 values
// bitsandbytes.functional.dequantize_4bit produces), then fed to
// v_mfma_f32_32x32x16_bf16 with fp32 accumulation. The backward stages an
// 8-row x 4-column patch per thread and transposes it in registers, so the
// contraction index (a row of W) becomes contiguous in LDS.
//
// The rank-r LoRA term is folded into the same accumulator as extra
// contraction steps: the A-side operand is T (or U) and the W-side operand is
// the fp32 adapter matrix scaled and rounded to bf16, so the output is rounded
// to bf16 exactly once.
//
// Gate/up pairing (forward): one workgroup computes gate and up for the same
// 64 intermediate columns. Each wave's 64-row W sub-tile holds 32 gate rows
// then the 32 up rows of the same columns, so a lane owns gate and up of the
// same (m, i) and the epilogue writes g, u and h = bf16(bf16(silu(g)) u).
#include <stdlib.h>

#include <algorithm>

#include "mfma_core.h"

namespace molt {
namespace {

constexpr int BM = 128;        // X rows per workgroup tile
constexpr int BN = 128;        // W rows (forward) / output columns (backward) per tile
constexpr int WAVES_M = 2, WAVES_N = 2;
constexpr int NT = 64 * WAVES_M * WAVES_N;
constexpr int WROWS = BN / WAVES_N;   // 64
constexpr int WCOLS = BM / WAVES_M;   // 64
constexpr int TM = WROWS / 32, TN = WCOLS / 32;
constexpr int GROUP_M = 8;

enum { EPI_STORE = 0, EPI_GATEUP = 1, EPI_SWIGLU_BWD = 2 };

struct FwdParams {
  const uint16_t* x; int64_t ldx; int64_t M; int64_t K;
  const uint8_t* packed[2]; const float* scales[2];
  int64_t N;                 // rows of each weight
  const float* code; int order; int block_size;
  const uint16_t* t; int64_t ldt; int lr;      // LoRA contraction length (0 = none)
  const float* lb[2]; int64_t ldlb; int r; float s[2];
  uint16_t* y[3]; int64_t ldy;                 // single: y[0]; pair: g, u, h
  int vec_out;
  // split-K (large-tile single-output kernel only): blockIdx.y = split, each
  // split runs split_steps (even) 64-deep steps and writes an fp32 partial
  // tile to part[split][M][N]; null part = no split
  int split_steps; float* part;
  // staged weights (large-tile kernels): bf16 deq(W) [N, K] of each weight,
  // row stride ldw, read by DMA instead of dequantising packed bytes
  const uint16_t* wst[2]; int64_t ldw;
  // LoRA steps through the staged kernel's DMA ring: bf16(s B) rows of each
  // weight [N, lora_ring] (lr rounded up to 64, zeros past the adapter's
  // ranks), the pair's block-diagonal layout; 0 = no ring
  const uint16_t* lbst[2]; int lora_ring;
  // staged kernels: also write deq(W)^T [K, N] of each weight (row stride N,
  // N % 8 == 0) for the input gradient of the same weights; null = do not
  uint16_t* wt_out[2];
};

struct BwdParams {
  const uint16_t* dy[2]; int64_t lddy; int64_t M;
  const uint8_t* packed[2]; const float* scales[2];
  int64_t Nw;                // contraction length per segment (rows of W)
  int64_t Kw;                // output columns (cols of W)
  const float* code; int order; int block_size; int nseg;
  const uint16_t* u[2]; int64_t ldu; int r;
  const float* la[2]; int64_t ldla; float la_scale;
  uint16_t* dx; int64_t lddx;
  const uint16_t* gate; const uint16_t* up; uint16_t* dg; uint16_t* du; int64_t ldg;
  int vec_out;
  int split_steps; float* part;   // split-K of the plain-store large-tile kernel (see FwdParams)
  // staged weights (large-tile kernels): bf16 deq(W)^T [Kw, Nw] of each
  // segment, row stride ldw: row k holds the contraction elements of output column k
  const uint16_t* wst[2]; int64_t ldw;
};

struct Smem {
  uint16_t xs[2][BM * LDSW];
  uint16_t ws[2][BN * LDSW];
  float2 tab[256];
  float code16[16];
};

MOLT_DEV float silu_f32(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

// Two-way select of a kernel-argument array element. Indexing the argument
// struct with a lane-dependent index makes the compiler fetch the pointer
// with a vector memory load (and wait for every outstanding load before
// using it); a select of the two scalar values keeps it in registers.
template <typename T>
MOLT_DEV T sel2(T a, T b, int i) { return i ? b : a; }
#define sel(arr, i) sel2((arr)[0], (arr)[1], (i))

MOLT_DEV uint32_t dequant_pair(const float2* tab, uint32_t byte, float sc) {
  const float2 c = tab[byte];
  return pack_bf16x2(c.x * sc, c.y * sc);
}

// ------------------------------------------------------------ X-side staging
struct AReg { u32x4_t v[BM * BK / 8 / NT]; };
constexpr int A_PT = BM * BK / 8 / NT;  // 16-byte chunks per thread (4)

MOLT_DEV void a_issue(AReg& ar, const uint16_t* __restrict__ a, int64_t lda, int64_t m0,
                      int64_t M, int64_t k0, int tid) {
#pragma unroll
  for (int c = 0; c < A_PT; ++c) {
    const int idx = tid + c * NT;
    const int row = idx >> 3, col = (idx & 7) * 8;
    const int64_t m = m0 + row;
    u32x4_t v = {0u, 0u, 0u, 0u};
    if (m < M) v = *reinterpret_cast<const u32x4_t*>(a + m * lda + k0 + col);
    ar.v[c] = v;
  }
}

MOLT_DEV void a_commit(const AReg& ar, uint16_t* xs, int tid) {
#pragma unroll
  for (int c = 0; c < A_PT; ++c) {
    const int idx = tid + c * NT;
    const int row = idx >> 3, col = (idx & 7) * 8;
    *reinterpret_cast<u32x4_t*>(xs + row * LDSW + col) = ar.v[c];
  }
}

// Element-wise X-side staging with full bounds checks (tails, odd strides, LoRA steps).
MOLT_DEV void a_generic(uint16_t* xs, const uint16_t* __restrict__ a, int64_t lda, int64_t m0,
                        int64_t M, int64_t k0, int64_t L, int tid) {
  for (int e = tid; e < BM * BK; e += NT) {
    const int row = e / BK, j = e % BK;
    const int64_t m = m0 + row, k = k0 + j;
    xs[row * LDSW + j] = (m < M && k < L) ? a[m * lda + k] : (uint16_t)0;
  }
}

// X side of a LoRA contraction step (T or U, [M, L] bf16): the thread's four
// 8-element chunks as 32 element loads from clamped addresses, all issued
// before the first use (a load behind a bounds branch would make the compiler
// wait for every load issued before it), zeros outside the operand.
MOLT_DEV void a_lora(uint16_t* xs, const uint16_t* __restrict__ a, int64_t lda, int64_t m0, int64_t M, int64_t k0,
                     int64_t L, int tid) {
  uint16_t e[A_PT][8];
#pragma unroll
  for (int c = 0; c < A_PT; ++c) {
    const int idx = tid + c * NT;
    const int64_t m = m0 + (idx >> 3), k = k0 + (idx & 7) * 8;
    const int64_t mc = m < M ? m : M - 1;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t kc = k + i < L ? k + i : L - 1;
      e[c][i] = a[mc * lda + kc];
    }
  }
#pragma unroll
  for (int c = 0; c < A_PT; ++c) {
    const int idx = tid + c * NT;
    const int64_t m = m0 + (idx >> 3), k = k0 + (idx & 7) * 8;
    uint16_t v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = m < M && k + i < L ? e[c][i] : (uint16_t)0;
    *reinterpret_cast<u32x4_t*>(xs + (idx >> 3) * LDSW + (idx & 7) * 8) = __builtin_bit_cast(u32x4_t, v);
  }
}

// ------------------------------------------------ forward W-side (row-contract)
// LDS row R of the W tile -> (weight index, weight row).
MOLT_DEV void fwd_row(int R, int64_t tn, bool pair, int& which, int64_t& n) {
  if (pair) {
    which = (R >> 5) & 1;
    n = tn * (BN / 2) + (R >> 6) * 32 + (R & 31);
  } else {
    which = 0;
    n = tn * BN + R;
  }
}

struct WRowReg { u32x4_t q; float sc; };

MOLT_DEV void wrow_issue(WRowReg& wr, const FwdParams& p, int64_t tn, bool pair, int64_t k0, int tid) {
  const int R = tid >> 1, half = tid & 1;
  int which; int64_t n;
  fwd_row(R, tn, pair, which, n);
  const int64_t k = k0 + 32 * half;
  u32x4_t q = {0u, 0u, 0u, 0u};
  float sc = 0.0f;
  if (n < p.N) {
    const int64_t flat = n * p.K + k;
    q = *reinterpret_cast<const u32x4_t*>(sel(p.packed, which) + (flat >> 1));
    sc = sel(p.scales, which)[flat >> 6];
  }
  wr.q = q;
  wr.sc = sc;
}

MOLT_DEV void wrow_commit(const WRowReg& wr, uint16_t* ws, const float2* tab, int tid) {
  const int R = tid >> 1, half = tid & 1;
  uint16_t* dst = ws + R * LDSW + 32 * half;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const uint32_t w = wr.q[d];
    u32x4_t o;
    o[0] = dequant_pair(tab, w & 0xffu, wr.sc);
    o[1] = dequant_pair(tab, (w >> 8) & 0xffu, wr.sc);
    o[2] = dequant_pair(tab, (w >> 16) & 0xffu, wr.sc);
    o[3] = dequant_pair(tab, w >> 24, wr.sc);
    *reinterpret_cast<u32x4_t*>(dst + 8 * d) = o;
  }
}

MOLT_DEV void wrow_generic(uint16_t* ws, const FwdParams& p, int64_t tn, bool pair, int64_t k0,
                           const float* code16, int tid) {
  for (int e = tid; e < BN * BK; e += NT) {
    const int R = e / BK, j = e % BK;
    int which; int64_t n;
    fwd_row(R, tn, pair, which, n);
    const int64_t k = k0 + j;
    uint16_t v = 0;
    if (n < p.N && k < p.K) {
      const int64_t f = n * p.K + k;
      const int nib = nf4_nibble(sel(p.packed, which), f, p.order);
      v = bf16_bits(code16[nib] * sel(p.scales, which)[f / p.block_size]);
    }
    ws[R * LDSW + j] = v;
  }
}

// LoRA step (forward): W-side row R holds bf16(s * B[n, j - off]) for its
// window. A thread owns 32 consecutive columns of one row (as wrow_issue);
// its loads come from clamped addresses and are all issued before any use.
MOLT_DEV void wrow_lora(uint16_t* ws, const FwdParams& p, int64_t tn, bool pair, int64_t k0, int tid) {
  const int R = tid >> 1, half = tid & 1;
  int which; int64_t n;
  fwd_row(R, tn, pair, which, n);
  const float s = which ? p.s[1] : p.s[0];
  const float* brow = sel(p.lb, which) + (n < p.N ? n : p.N - 1) * p.ldlb;
  const int64_t c0 = k0 + 32 * half - (int64_t)which * p.r;   // adapter column of the first element
  float f[32];
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    const int64_t c = c0 + j;
    f[j] = brow[c < 0 ? 0 : (c < p.r ? c : p.r - 1)];
  }
  uint16_t* dst = ws + R * LDSW + 32 * half;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    u32x4_t o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = 8 * d + 2 * i;
      const bool ok0 = n < p.N && c0 + j >= 0 && c0 + j < p.r;
      const bool ok1 = n < p.N && c0 + j + 1 >= 0 && c0 + j + 1 < p.r;
      o[i] = pack_bf16x2(ok0 ? s * f[j] : 0.0f, ok1 ? s * f[j + 1] : 0.0f);
    }
    *reinterpret_cast<u32x4_t*>(dst + 8 * d) = o;
  }
}

// --------------------------------------------- backward W-side (column-contract)
// Thread patch: 8 contraction rows x 4 output columns.
constexpr int CG = BN / 4;  // 32 column groups
static_assert(CG * 8 == NT, "backward patch layout needs BN/4 * 8 == threads");

struct WColReg { uint32_t q[8]; float sc[8]; };

MOLT_DEV void wcol_issue(WColReg& wr, const BwdParams& p, int seg, int64_t tn, int64_t c0, int tid) {
  const int cg = tid % CG, rg = tid / CG;
  const int64_t col = tn * BN + 4 * cg;
  const bool ok = col < p.Kw;
  const uint8_t* packed = sel(p.packed, seg);
  const float* scales = sel(p.scales, seg);
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int64_t c = c0 + 8 * rg + r;
    uint32_t q = 0;
    float sc = 0.0f;
    if (ok) {
      const int64_t flat = c * p.Kw + col;
      q = *reinterpret_cast<const uint16_t*>(packed + (flat >> 1));
      sc = scales[flat >> 6];
    }
    wr.q[r] = q;
    wr.sc[r] = sc;
  }
}

MOLT_DEV void wcol_commit(const WColReg& wr, uint16_t* ws, const float2* tab, int tid) {
  const int cg = tid % CG, rg = tid / CG;
  float v[8][4];
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const float2 p0 = tab[wr.q[r] & 0xffu];
    const float2 p1 = tab[(wr.q[r] >> 8) & 0xffu];
    v[r][0] = p0.x * wr.sc[r];
    v[r][1] = p0.y * wr.sc[r];
    v[r][2] = p1.x * wr.sc[r];
    v[r][3] = p1.y * wr.sc[r];
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    u32x4_t o;
    o[0] = pack_bf16x2(v[0][j], v[1][j]);
    o[1] = pack_bf16x2(v[2][j], v[3][j]);
    o[2] = pack_bf16x2(v[4][j], v[5][j]);
    o[3] = pack_bf16x2(v[6][j], v[7][j]);
    *reinterpret_cast<u32x4_t*>(ws + (4 * cg + j) * LDSW + 8 * rg) = o;
  }
}

MOLT_DEV void wcol_generic(uint16_t* ws, const BwdParams& p, int seg, int64_t tn, int64_t c0,
                           const float* code16, int tid) {
  for (int e = tid; e < BN * BK; e += NT) {
    const int R = e % BN, j = e / BN;   // consecutive threads walk the contiguous output dim
    const int64_t col = tn * BN + R, c = c0 + j;
    uint16_t v = 0;
    if (col < p.Kw && c < p.Nw) {
      const int64_t f = c * p.Kw + col;
      const int nib = nf4_nibble(sel(p.packed, seg), f, p.order);
      v = bf16_bits(code16[nib] * sel(p.scales, seg)[f / p.block_size]);
    }
    ws[R * LDSW + j] = v;
  }
}

// LoRA step (backward): W-side row R (output column) holds bf16(la_scale *
// A[c0 + j, col]). A thread owns the patch of wcol_commit (8 contraction rows
// x 4 columns); its loads come from clamped addresses and are all issued
// before any use.
MOLT_DEV void wcol_lora(uint16_t* ws, const BwdParams& p, int seg, int64_t tn, int64_t c0, int tid) {
  const float* a = sel(p.la, seg);
  const int cg = tid % CG, rg = tid / CG;
  const int64_t col = tn * BN + 4 * cg;
  float f[8][4];
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int64_t c = c0 + 8 * rg + r;
    const int64_t cc = c < p.r ? c : p.r - 1;
#pragma unroll
    for (int j = 0; j < 4; ++j) f[r][j] = a[cc * p.ldla + (col + j < p.Kw ? col + j : p.Kw - 1)];
  }
  float v[8][4];
#pragma unroll
  for (int r = 0; r < 8; ++r)
#pragma unroll
    for (int j = 0; j < 4; ++j) v[r][j] = c0 + 8 * rg + r < p.r && col + j < p.Kw ? p.la_scale * f[r][j] : 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    u32x4_t o;
    o[0] = pack_bf16x2(v[0][j], v[1][j]);
    o[1] = pack_bf16x2(v[2][j], v[3][j]);
    o[2] = pack_bf16x2(v[4][j], v[5][j]);
    o[3] = pack_bf16x2(v[6][j], v[7][j]);
    *reinterpret_cast<u32x4_t*>(ws + (4 * cg + j) * LDSW + 8 * rg) = o;
  }
}

// ------------------------------------------- pipelined main steps (aligned)
// Workgroup barrier without __syncthreads()'s release fence (the fence makes
// the compiler drain every outstanding vector-memory op, including register
// loads that are only used steps later); this wave's LDS accesses are waited
// for, and the empty asm statements keep the compiler from moving memory
// accesses across the barrier.
MOLT_DEV void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);              // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// The register loads of one forward main step (aligned operands): X rows and
// W rows past the matrix re-read the last row, so every load is issued
// unconditionally (a load behind a bounds branch makes the compiler wait for
// all earlier loads at the join). Those rows only feed output rows and
// columns that are never stored.
struct FwdStage { AReg a; WRowReg w; };

MOLT_DEV void fwd_issue(FwdStage& st, const FwdParams& p, int64_t m0, int64_t tn, bool pair, int s, int tid) {
  const int64_t k0 = (int64_t)s * BK;
#pragma unroll
  for (int c = 0; c < A_PT; ++c) {
    const int idx = tid + c * NT;
    const int64_t m = m0 + (idx >> 3) < p.M ? m0 + (idx >> 3) : p.M - 1;
    st.a.v[c] = *reinterpret_cast<const u32x4_t*>(p.x + m * p.ldx + k0 + (idx & 7) * 8);
  }
  const int R = tid >> 1, half = tid & 1;
  int which; int64_t n;
  fwd_row(R, tn, pair, which, n);
  const int64_t flat = (n < p.N ? n : p.N - 1) * p.K + k0 + 32 * half;
  st.w.q = *reinterpret_cast<const u32x4_t*>(sel(p.packed, which) + (flat >> 1));
  st.w.sc = sel(p.scales, which)[flat >> 6];
}

// Main steps sbeg .. sbeg + n - 1 of the aligned forward kernels. Three
// register sets rotate: while step i's MFMAs run from LDS buffer i % 2, step
// i + 1 is committed from its set to the other buffer and that set is refilled
// with step i + 4, so the loads of two to three steps are in flight at every
// step boundary (one step of lookahead left the kernel waiting on memory
// latency at these short contractions). Steps past the range re-load the
// last one and are never committed.
template <bool PAIR>
MOLT_DEV void fwd_main(const FwdParams& p, Smem& sm, int64_t m0, int64_t tn, int sbeg, int n,
                       f32x16_t (&acc)[TM][TN], int tid, int lane, int wm, int wn) {
  const int last = n - 1;
  auto S = [&](int i) { return sbeg + (i < last ? i : last); };
  FwdStage s0, s1, s2;
  fwd_issue(s0, p, m0, tn, PAIR, S(0), tid);
  fwd_issue(s1, p, m0, tn, PAIR, S(1), tid);
  fwd_issue(s2, p, m0, tn, PAIR, S(2), tid);
  a_commit(s0.a, sm.xs[0], tid);
  wrow_commit(s0.w, sm.ws[0], sm.tab, tid);
  fwd_issue(s0, p, m0, tn, PAIR, S(3), tid);
  lds_barrier();
#define MOLT_FWD_ITER(K, SET)                                                        \
  mfma_step<TM, TN>(sm.ws[(K) & 1], sm.xs[(K) & 1], wn * WROWS, wm * WCOLS, acc, lane); \
  if (i + (K) + 1 >= n) break;                                                       \
  a_commit(SET.a, sm.xs[((K) + 1) & 1], tid);                                        \
  wrow_commit(SET.w, sm.ws[((K) + 1) & 1], sm.tab, tid);                             \
  fwd_issue(SET, p, m0, tn, PAIR, S(i + (K) + 4), tid);                              \
  lds_barrier();
  for (int i = 0; i < n; i += 6) {
    MOLT_FWD_ITER(0, s1)
    MOLT_FWD_ITER(1, s2)
    MOLT_FWD_ITER(2, s0)
    MOLT_FWD_ITER(3, s1)
    MOLT_FWD_ITER(4, s2)
    MOLT_FWD_ITER(5, s0)
  }
#undef MOLT_FWD_ITER
  __syncthreads();   // every wave is done with the LDS buffers
}

// --------------------------------------------------------------- epilogues
// Vector stores of output tiles. NT: non-temporal (used by the 256 x 256
// kernels, whose outputs are hundreds of MB): the tiles stream to HBM while
// the GEMM runs instead of staying dirty in the last-level cache, where the
// next, memory-bound kernel would pay for writing them back.
template <bool NT, typename V>
MOLT_DEV void st_vec(uint16_t* dst, const V& v) {
  if constexpr (NT) __builtin_nontemporal_store(v, reinterpret_cast<V*>(dst));
  else *reinterpret_cast<V*>(dst) = v;
}

template <bool NT = false>
MOLT_DEV void store4(uint16_t* __restrict__ out, int64_t ld, int64_t m, int64_t n, int64_t N,
                     const float* v, bool vec) {
  uint16_t* dst = out + m * ld + n;
  if (vec && n + 3 < N) {
    u32x2_t o = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    st_vec<NT>(dst, o);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (n + e < N) dst[e] = bf16_bits(v[e]);
  }
}

MOLT_DEV void load4(const uint16_t* __restrict__ src, int64_t ld, int64_t m, int64_t n, int64_t N,
                    float* v, bool vec) {
  const uint16_t* s = src + m * ld + n;
  if (vec && n + 3 < N) {
    const u32x2_t w = *reinterpret_cast<const u32x2_t*>(s);
    v[0] = bf16_lo(w[0]); v[1] = bf16_hi(w[0]); v[2] = bf16_lo(w[1]); v[3] = bf16_hi(w[1]);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = (n + e < N) ? bf16_to_f32(s[e]) : 0.0f;
  }
}

// fp32 partial tile of a split-K launch of the 128 x 128 kernels:
// part[m][n0 ..] (row stride N, N % 4 == 0), rows past M and columns past N
// skipped.
MOLT_DEV void store_partial128(float* part, int64_t M, int64_t N, const f32x16_t (&acc)[TM][TN], int64_t m0,
                               int64_t n0, int wm, int wn, int lane) {
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t m = m0 + wm * WCOLS + j * 32 + (lane & 31);
    if (m >= M) continue;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int64_t n = n0 + wn * WROWS + i * 32 + 8 * g + 4 * (lane >> 5);
        if (n >= N) continue;
        const f32x4_t v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
        *reinterpret_cast<f32x4_t*>(part + m * N + n) = v;
      }
  }
}

// ------------------------------------------------------------------ kernels
template <bool PAIR, bool ALIGNED>
__global__ __launch_bounds__(NT, 2) void nf4_fwd_kernel(const FwdParams p) {
  __shared__ Smem sm;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WAVES_M, wn = wave / WAVES_M;

  const int64_t cols_per_tile = PAIR ? BN / 2 : BN;
  const int64_t nt_m = ceil_div64(p.M, BM), nt_n = ceil_div64(p.N, cols_per_tile);
  int64_t tm, tn;
  grouped_tile(xcd_tile(blockIdx.x, nt_m * nt_n), nt_m, nt_n, GROUP_M, tm, tn);
  const int64_t m0 = tm * BM;

  build_pair_table(sm.tab, p.code, p.order);
  if (tid < 16) sm.code16[tid] = p.code[tid];

  const int ks = (int)ceil_div64(p.K, BK);
  // split-K (single output only): this workgroup runs main steps
  // [sbeg, send); the LoRA steps belong to the last split
  const bool split = !PAIR && p.part != nullptr;
  const int sbeg = split ? (int)blockIdx.y * p.split_steps : 0;
  const int send = split ? min(ks, sbeg + p.split_steps) : ks;
  const int ls = p.lr > 0 && (!split || blockIdx.y + 1 == gridDim.y) ? (int)ceil_div64(p.lr, BK) : 0;
  const int nmain = send - sbeg;
  const int total = nmain + ls;
  // virtual step v -> main step sbeg + v, then LoRA step ks + (v - nmain)
  auto step_of = [&](int v) { return v < nmain ? sbeg + v : ks + (v - nmain); };

  f32x16_t acc[TM][TN];
  zero_acc(acc);
  AReg ar;
  WRowReg wr;

  auto issue = [&](int s) {
    if (ALIGNED && s < ks) {
      a_issue(ar, p.x, p.ldx, m0, p.M, (int64_t)s * BK, tid);
      wrow_issue(wr, p, tn, PAIR, (int64_t)s * BK, tid);
    }
  };
  auto commit = [&](int s, int buf) {
    uint16_t* xs = sm.xs[buf];
    uint16_t* ws = sm.ws[buf];
    if (s < ks) {
      if (ALIGNED) {
        a_commit(ar, xs, tid);
        wrow_commit(wr, ws, sm.tab, tid);
      } else {
        a_generic(xs, p.x, p.ldx, m0, p.M, (int64_t)s * BK, p.K, tid);
        wrow_generic(ws, p, tn, PAIR, (int64_t)s * BK, sm.code16, tid);
      }
    } else {
      const int64_t c0 = (int64_t)(s - ks) * BK;
      a_lora(xs, p.t, p.ldt, m0, p.M, c0, p.lr, tid);
      wrow_lora(ws, p, tn, PAIR, c0, tid);
    }
  };

  __syncthreads();  // pair table ready
  int v0 = 0;       // first virtual step of the loop below
  if constexpr (ALIGNED) {
    if (nmain > 0) fwd_main<PAIR>(p, sm, m0, tn, sbeg, nmain, acc, tid, lane, wm, wn);
    v0 = nmain;     // the loop runs the LoRA steps only
  }
  if (v0 < total) {
    issue(step_of(v0));
    commit(step_of(v0), 0);
    __syncthreads();
  }
  for (int v = v0; v < total; ++v) {
    const int cur = (v - v0) & 1;
    if (v + 1 < total) issue(step_of(v + 1));
    mfma_step<TM, TN>(sm.ws[cur], sm.xs[cur], wn * WROWS, wm * WCOLS, acc, lane);
    if (v + 1 < total) commit(step_of(v + 1), cur ^ 1);
    __syncthreads();
  }

  if (split) {
    store_partial128(p.part + (int64_t)blockIdx.y * p.M * p.N, p.M, p.N, acc, m0, tn * BN, wm, wn, lane);
    return;
  }
  const bool vec = p.vec_out != 0;
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t m = m0 + wm * WCOLS + j * 32 + (lane & 31);
    if (m >= p.M) continue;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      if (!PAIR) {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const int64_t n = tn * BN + wn * WROWS + i * 32 + 8 * g + 4 * (lane >> 5);
          float v[4] = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
          store4(p.y[0], p.ldy, m, n, p.N, v, vec);
        }
      } else {
        const int64_t n = tn * (BN / 2) + wn * 32 + 8 * g + 4 * (lane >> 5);
        float gv[4], uv[4], hv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          gv[e] = round_bf16(acc[0][j][4 * g + e]);
          uv[e] = round_bf16(acc[1][j][4 * g + e]);
          hv[e] = round_bf16(silu_f32(gv[e])) * uv[e];
        }
        store4(p.y[0], p.ldy, m, n, p.N, gv, vec);
        store4(p.y[1], p.ldy, m, n, p.N, uv, vec);
        store4(p.y[2], p.ldy, m, n, p.N, hv, vec);
      }
    }
  }
}

template <int EPI, bool ALIGNED>
__global__ __launch_bounds__(NT) void nf4_bwd_kernel(const BwdParams p) {
  __shared__ Smem sm;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WAVES_M, wn = wave / WAVES_M;

  const int64_t nt_m = ceil_div64(p.M, BM), nt_n = ceil_div64(p.Kw, BN);
  int64_t tm, tn;
  grouped_tile(xcd_tile(blockIdx.x, nt_m * nt_n), nt_m, nt_n, GROUP_M, tm, tn);
  const int64_t m0 = tm * BM;

  build_pair_table(sm.tab, p.code, p.order);
  if (tid < 16) sm.code16[tid] = p.code[tid];

  const int ks = (int)ceil_div64(p.Nw, BK);        // steps per NF4 segment
  const int lsteps = p.r > 0 ? (int)ceil_div64(p.r, BK) : 0;
  // split-K (plain store only): main steps [sbeg, send) of the nseg * ks,
  // the LoRA steps in the last split
  const bool split = EPI == EPI_STORE && p.part != nullptr;
  const int sbeg = split ? (int)blockIdx.y * p.split_steps : 0;
  const int send = split ? min(p.nseg * ks, sbeg + p.split_steps) : p.nseg * ks;
  const int nmain = send - sbeg;
  const int nl = !split || blockIdx.y + 1 == gridDim.y ? p.nseg * lsteps : 0;
  const int total = nmain + nl;
  auto step_of = [&](int v) { return v < nmain ? sbeg + v : p.nseg * ks + (v - nmain); };

  f32x16_t acc[TM][TN];
  zero_acc(acc);
  AReg ar;
  WColReg wr;

  auto issue = [&](int s) {
    if (ALIGNED && s < p.nseg * ks) {
      const int seg = s / ks;
      const int64_t c0 = (int64_t)(s % ks) * BK;
      a_issue(ar, sel(p.dy, seg), p.lddy, m0, p.M, c0, tid);
      wcol_issue(wr, p, seg, tn, c0, tid);
    }
  };
  auto commit = [&](int s, int buf) {
    uint16_t* xs = sm.xs[buf];
    uint16_t* ws = sm.ws[buf];
    if (s < p.nseg * ks) {
      const int seg = s / ks;
      const int64_t c0 = (int64_t)(s % ks) * BK;
      if (ALIGNED) {
        a_commit(ar, xs, tid);
        wcol_commit(wr, ws, sm.tab, tid);
      } else {
        a_generic(xs, sel(p.dy, seg), p.lddy, m0, p.M, c0, p.Nw, tid);
        wcol_generic(ws, p, seg, tn, c0, sm.code16, tid);
      }
    } else {
      const int ls = s - p.nseg * ks;
      const int seg = ls / lsteps;
      const int64_t c0 = (int64_t)(ls % lsteps) * BK;
      a_lora(xs, sel(p.u, seg), p.ldu, m0, p.M, c0, p.r, tid);
      wcol_lora(ws, p, seg, tn, c0, tid);
    }
  };

  __syncthreads();
  issue(step_of(0));
  commit(step_of(0), 0);
  __syncthreads();
  for (int v = 0; v < total; ++v) {
    const int cur = v & 1;
    if (v + 1 < total) issue(step_of(v + 1));
    mfma_step<TM, TN>(sm.ws[cur], sm.xs[cur], wn * WROWS, wm * WCOLS, acc, lane);
    if (v + 1 < total) commit(step_of(v + 1), cur ^ 1);
    __syncthreads();
  }

  if (split) {
    store_partial128(p.part + (int64_t)blockIdx.y * p.M * p.Kw, p.M, p.Kw, acc, m0, tn * BN, wm, wn, lane);
    return;
  }
  const bool vec = p.vec_out != 0;
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t m = m0 + wm * WCOLS + j * 32 + (lane & 31);
    if (m >= p.M) continue;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int64_t n = tn * BN + wn * WROWS + i * 32 + 8 * g + 4 * (lane >> 5);
        float v[4] = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
        if (EPI == EPI_STORE) {
          store4(p.dx, p.lddx, m, n, p.Kw, v, vec);
        } else {
          float gv[4], uv[4], dgv[4], duv[4];
          load4(p.gate, p.ldg, m, n, p.Kw, gv, vec);
          load4(p.up, p.ldg, m, n, p.Kw, uv, vec);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float dh = round_bf16(v[e]);
            const float sg = __builtin_amdgcn_rcpf(1.0f + __expf(-gv[e]));
            duv[e] = dh * round_bf16(gv[e] * sg);
            dgv[e] = round_bf16(dh * uv[e]) * (sg * (1.0f + gv[e] * (1.0f - sg)));
          }
          store4(p.dg, p.ldg, m, n, p.Kw, dgv, vec);
          store4(p.du, p.ldg, m, n, p.Kw, duv, vec);
        }
      }
    }
  }
}

// ======================================================================
// Large-tile kernels for aligned shapes (K, contraction and output widths
// multiples of 64, NF4 block 64): 256 x 256 workgroup tile, 8 waves of
// 128 W rows x 64 X rows (8 accumulator tiles, 128 registers per wave), so
// two waves share each SIMD and one's memory or dequantisation work fills
// the other's MFMA gaps. The next step's loads are spread over the MFMA
// sub-steps of the current one (X straight into LDS, the packed NF4 bytes
// into registers, dequantised into the other LDS buffer during the last
// sub-step), and the LDS layout is unpadded with 16-byte chunks XOR-swizzled
// by (row ^ row/8) & 7, so fragment reads, row-major stores and the
// backward's transposed patch stores are all bank-conflict free.
// ======================================================================
namespace big {

// outputs by non-temporal stores (st_vec)
constexpr bool kStreamOut = true;

constexpr int BM = 256, BN = 256, NT = 512, WAVES_M = 4;
constexpr int WROWS = 128, WCOLS = 64, TM = 4, TN = 2, LD = 64;
constexpr int GROUP_M = 4;
constexpr int BUF = BM * LD;     // bf16 elements of one operand buffer (32 KB)
constexpr int TABC = 16;         // interleaved copies of the code-pair table
constexpr int EP_LD = 256 + 8;   // (128 x 128 path and backward) epilogue tile row stride

// Operand buffer layout. A tile row holds its 64 contraction elements as 8
// chunks of 16 B in one 128-byte line, row R at 128 R, chunk c at position
// c ^ f(R) with f(R) = (R ^ ((R >> 3) & 3)) & 7. Then
//  * a ds_read_b128 of one chunk over 16 consecutive rows (served 16 lanes per
//    cycle over 64 banks) hits 16 distinct 16-byte bank groups: rows R and
//    R + 8 of the group differ in R & 1 or in f (the fragment reads);
//  * a 1 KB DMA block is 8 whole rows, so each 128-byte line of X is one
//    request (half-line requests doubled the L1 traffic);
//  * f(R + 32) = f(R), so the subtiles of a fragment read are one per-lane
//    base offset (XOR-ed with the sub-step) plus an immediate of 32 rows.
MOLT_DEV int lswz(int R) { return (R ^ ((R >> 3) & 3)) & 7; }
MOLT_DEV int loff(int R, int c) { return R * 64 + ((c ^ lswz(R)) << 3); }

// Global -> LDS DMA writes lane l's 16 bytes to (block base + 16 l): block blk
// (1 KB) of a buffer holds rows 8 blk .. 8 blk + 7, lane l filling position
// l % 8 of row 8 blk + l / 8. Returns the tile row and first contraction
// element the lane must fetch.
// DMA instructions that fill one operand buffer (16 bytes per lane each).
constexpr int kStageDma = BUF * 2 / (NT * 16);
static_assert(kStageDma == 4, "x_load and the staged W DMA issue 4 instructions per buffer");

// Value selects for the staged kernels' per-step sources. A conditional
// expression over two lvalues (captured variables, array elements) selects an
// address and loads through it, from scratch memory, which also makes the
// result look divergent; by-value parameters keep it a register select.
template <typename T>
MOLT_DEV T pick(bool c, T a, T b) { return c ? a : b; }

// Steps 0 .. n - 1 of a staged kernel: step j reads X buffer j % 3 and W
// buffer j % 2 and loads X(j + 2), W(j + 1) into the buffers read at step
// j - 1. The pattern repeats every 6 steps; every call names its buffers
// statically (the compiler then tells the LDS reads of one buffer from the
// DMA into another and inserts no waits between them).
template <typename Step>
MOLT_DEV void ring_steps(int n, Step& step, uint16_t* x0, uint16_t* x1, uint16_t* x2, uint16_t* w0, uint16_t* w1) {
  int j = 0;
  for (; j + 6 <= n; j += 6) {
    step(j, x0, w0, x2, w1);
    step(j + 1, x1, w1, x0, w0);
    step(j + 2, x2, w0, x1, w1);
    step(j + 3, x0, w1, x2, w0);
    step(j + 4, x1, w0, x0, w1);
    step(j + 5, x2, w1, x1, w0);
  }
  if (j < n) step(j, x0, w0, x2, w1);
  if (j + 1 < n) step(j + 1, x1, w1, x0, w0);
  if (j + 2 < n) step(j + 2, x2, w0, x1, w1);
  if (j + 3 < n) step(j + 3, x0, w1, x2, w0);
  if (j + 4 < n) step(j + 4, x1, w0, x0, w1);
}

MOLT_DEV void dma_slot(int blk, int lane, int& R, int& k) {
  R = 8 * blk + (lane >> 3);
  k = 8 * ((lane & 7) ^ lswz(R));
}

// Kernel-argument pointers and the 16 codes stay in scalar registers or are
// read once; see build_tab.
typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Buffer resource over [p, p + bytes): loads through it are bounds-checked by
// the hardware (out-of-range lanes read zero) and take a 32-bit per-lane byte
// offset plus a uniform scalar offset, so no per-step 64-bit address math.
MOLT_DEV __amdgpu_buffer_rsrc_t make_rsrc(const void* p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
MOLT_DEV u32x4_t buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, soff, 0);
}
MOLT_DEV uint32_t buf_load4(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, soff, 0);
}
// 16 bytes per lane from global straight into LDS at dst + 16 * lane (dst uniform).
MOLT_DEV void buf_load_lds16(__amdgpu_buffer_rsrc_t r, void* dst, uint32_t off, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)dst, 16, off, soff, 0, 0);
}
// vmcnt(N) with the other counters untouched: wait until at most N of this
// wave's vector-memory operations (loads, buffer-to-LDS DMA) are outstanding.
template <int N>
MOLT_DEV void wait_vm_at_most() {
  static_assert(N >= 0 && N < 16, "vmcnt immediate is 4 bits here");
  __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}
MOLT_DEV void wait_vm0() { wait_vm_at_most<0>(); }

// The end of a step waits with a partial vmcnt that counts the register loads
// of the next-but-one step as the only ones allowed to stay in flight; that
// holds only if every DMA of the step is issued before them. vmcnt counts in
// issue order, so the scheduler must not move a register load above a DMA
// (it did: two X DMA blocks then landed after the barrier, and other waves
// read stale LDS rows). Compiler and scheduling barrier between the two groups.
MOLT_DEV void dma_then_loads() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Workgroup barrier without __syncthreads()'s release fence: the fence makes
// the compiler drain every outstanding vector-memory op, including register
// loads of packed weight bytes that are only used a step later. The caller
// waits explicitly (vmcnt) for the DMA other waves will read; this wave's own
// LDS stores are waited for here, and the empty asm statements keep the
// compiler from moving memory accesses across the barrier.
MOLT_DEV void step_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);              // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Code-pair table, TABC interleaved copies: entry (byte b, copy c) at b * TABC + c
// holds (code[first nibble], code[second nibble]). Lane l reads copy l % TABC,
// which spreads the data-dependent lookups of a wave over TABC bank pairs.
MOLT_DEV void build_tab(float2* tab, const float* __restrict__ code, int order, int tid) {
  const float cv = code[tid & 15];
#pragma unroll
  for (int k = 0; k < 256 * TABC / NT; ++k) {
    const int i = tid + k * NT, b = i / TABC;
    const float ch = __shfl(cv, b >> 4), cl = __shfl(cv, b & 15);
    tab[i] = order ? make_float2(ch, cl) : make_float2(cl, ch);
  }
}

// Per-lane fragment offsets: lane l supplies row (l % 32) of each 32-row
// subtile and the 8-element half (l / 32) of a 16-deep sub-step. Sub-step kk
// reads chunk 2 kk + l / 32, whose position is (h ^ f(R)) ^ 2 kk: its offset
// is base ^ (kk << 4) (the XOR touches only the position bits); subtile i adds
// 32 rows = 2048 elements.
struct FragOff { int a, b; };

MOLT_DEV void frag_offsets(FragOff& f, int arow0, int brow0, int lane) {
  const int h = lane >> 5;
  f.a = loff(arow0 + (lane & 31), h);
  f.b = loff(brow0 + (lane & 31), h);
}

MOLT_DEV void load_frags(const uint16_t* __restrict__ ws, const uint16_t* __restrict__ xs, const FragOff& f, int kk,
                         bf16x8_t (&a)[TM], bf16x8_t (&b)[TN]) {
  const int ao = f.a ^ (kk << 4), bo = f.b ^ (kk << 4);
#pragma unroll
  for (int i = 0; i < TM; ++i)
    a[i] = *reinterpret_cast<const bf16x8_t*>(ws + ao + 2048 * i);
#pragma unroll
  for (int j = 0; j < TN; ++j)
    b[j] = *reinterpret_cast<const bf16x8_t*>(xs + bo + 2048 * j);
}

MOLT_DEV void mfma_set(const bf16x8_t (&a)[TM], const bf16x8_t (&b)[TN], f32x16_t (&acc)[TM][TN]) {
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
}

// One BK step from LDS (used by the LoRA steps): four 16-deep sub-steps, the
// fragment reads of sub-step kk+1 issued before the MFMAs of kk.
MOLT_DEV void compute(const uint16_t* __restrict__ ws, const uint16_t* __restrict__ xs, const FragOff& f,
                      f32x16_t (&acc)[TM][TN]) {
  bf16x8_t a[2][TM], b[2][TN];
  load_frags(ws, xs, f, 0, a[0], b[0]);
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    if (kk < 3) load_frags(ws, xs, f, kk + 1, a[(kk + 1) & 1], b[(kk + 1) & 1]);
    mfma_set(a[kk & 1], b[kk & 1], acc);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Instruction interleave of one 16-deep sub-step: each of the 8 MFMAs is
// followed by one or two LDS reads and a few VALU instructions, so the LDS
// queue and the VALU stay busy in the shadow of the matrix core instead of
// stalling the wave in bursts.
MOLT_DEV void interleave_substep() {
#define MOLT_SGB(nds)                                   \
  __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    \
  __builtin_amdgcn_sched_group_barrier(0x100, nds, 0);  \
  __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
  MOLT_SGB(2) MOLT_SGB(2) MOLT_SGB(1) MOLT_SGB(1) MOLT_SGB(1) MOLT_SGB(1) MOLT_SGB(1) MOLT_SGB(1)
#undef MOLT_SGB
  __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
}

// ---- forward W side (row-contract): 16 packed bytes (32 elements of one row) per thread
MOLT_DEV void fwd_row(int R, int64_t tn, bool pair, int& which, int64_t& n) {
  if (pair) {
    const int sub = (R >> 5) & 3;
    which = sub >> 1;
    n = tn * (BN / 2) + (R >> 7) * 64 + (sub & 1) * 32 + (R & 31);
  } else {
    which = 0;
    n = tn * BN + R;
  }
}

// deq(W)^T from the W tile of a staged forward step (FwdParams::wt_out).
// Thread q owns tile rows 4 (q % 64) .. + 3, four consecutive rows n of one
// weight, and the 8 contraction elements of chunk q / 64 of the step; per half
// chunk: four 8-byte LDS reads, a half-word exchange (v_perm) into 4 rows of
// W^T (one per contraction element, 4 consecutive n each) and four 8-byte
// non-temporal stores. The 64 lanes of a wave write one contraction element of
// all 256 tile rows per store: whole 256-byte runs of W^T rows. (Fewer live
// registers than 16-byte rows of 8 n, which the GEMM's budget does not leave.)
MOLT_DEV void wt_tile_write(const FwdParams& p, const uint16_t* __restrict__ wc, int64_t tn, int64_t k0, bool pair,
                            int tid) {
  const int g = tid & 63, c = tid >> 6;
  int which;
  int64_t n0;
  fwd_row(4 * g, tn, pair, which, n0);
  if (n0 >= p.N) return;   // rows past the weight (clamped copies of its last row)
  uint16_t* dst = sel(p.wt_out, which) + (k0 + 8 * c) * p.N + n0;
#pragma unroll
  for (int hk = 0; hk < 2; ++hk) {
    u32x2_t v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = *reinterpret_cast<const u32x2_t*>(wc + loff(4 * g + i, c) + 4 * hk);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t pick_half = (e & 1) ? 0x07060302u : 0x05040100u;
      const u32x2_t o = {__builtin_amdgcn_perm(v[1][e >> 1], v[0][e >> 1], pick_half),
                         __builtin_amdgcn_perm(v[3][e >> 1], v[2][e >> 1], pick_half)};
      st_vec<kStreamOut>(dst + (4 * hk + e) * p.N, o);
    }
  }
}

// One thread's packed W bytes and block scale for one forward step. w_load
// fetches them with exactly kLoads vector-memory instructions, issued after the
// step's X DMA (dma_then_loads); the step's closing wait leaves exactly these in
// flight, so kLoads is also that wait's vmcnt.
struct WBytes {
  u32x4_t q;
  float sc;
  static constexpr int kQLoads = sizeof(u32x4_t) / 16;   // 16 bytes per buffer_load_dwordx4
  static constexpr int kLoads = kQLoads + 1;             // + the scale
};
static_assert(WBytes::kQLoads == 1 && WBytes::kLoads == 2, "w_load issues one 16-byte and one 4-byte load");

MOLT_DEV void w_lookup(const WBytes& w, const float2* tabc, int d, float2 (&c)[4]) {
  const uint32_t q = w.q[d];
  c[0] = tabc[(q & 0xffu) * TABC];
  c[1] = tabc[((q >> 8) & 0xffu) * TABC];
  c[2] = tabc[((q >> 16) & 0xffu) * TABC];
  c[3] = tabc[(q >> 24) * TABC];
}

// Forward dequant slot of a thread: tile row R and 16-byte half of the row's
// 32-byte slice of the step. A ds_write_b128 is served 8 consecutive lanes
// per cycle over 32 banks, i.e. by the lane's 16-byte slot (its chunk
// position c ^ f(R)) mod 8. The 8 lanes of a group take 8 consecutive rows of
// one half, whose f(R) all differ; the two halves of a row sit in lanes l and
// l + 8, so the global load of a row's 32 bytes stays within one instruction.
MOLT_DEV void wslot(int tid, int& R, int& half) {
  const int l = tid & 63;
  half = (l >> 3) & 1;
  R = 32 * (tid >> 6) + 8 * (l >> 4) + (l & 7);
}

// bf16(code * scale) of 8 elements (the rounding of dequantize_4bit) into chunk 4 * half + d of row R.
MOLT_DEV void w_finish(const float2 (&c)[4], float sc, uint16_t* ws, int R, int half, int d) {
  u32x4_t o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = pack_bf16x2(c[e].x * sc, c[e].y * sc);
  *reinterpret_cast<u32x4_t*>(ws + loff(R, 4 * half + d)) = o;
}

// ---- staging of the LoRA contraction steps (swizzled layout). Each thread
// handles whole 8-element chunks: all of its global loads are issued before
// any LDS store, 16-byte vector loads where the chunk lies inside the operand
// and is aligned, element loads (with zeros outside) otherwise.
MOLT_DEV bool al16(const void* q) { return ((uintptr_t)q & 15) == 0; }

MOLT_DEV void lora_a_stage(uint16_t* xs, const uint16_t* __restrict__ t, int64_t ldt, int64_t m0, int64_t M,
                           int64_t c0, int64_t L, int tid) {
  constexpr int CH = BM * (BK / 8) / NT;
  const bool vec = al16(t) && ldt % 8 == 0;
  u32x4_t v[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int q = tid + NT * c, R = q >> 3, ch = q & 7;
    const int64_t m = m0 + R, k = c0 + 8 * ch;
    if (vec && m < M && k + 8 <= L) {
      v[c] = *reinterpret_cast<const u32x4_t*>(t + m * ldt + k);
    } else {
      uint16_t e[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) e[i] = (m < M && k + i < L) ? t[m * ldt + k + i] : (uint16_t)0;
      v[c] = __builtin_bit_cast(u32x4_t, e);
    }
  }
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int q = tid + NT * c;
    *reinterpret_cast<u32x4_t*>(xs + loff(q >> 3, q & 7)) = v[c];
  }
}

MOLT_DEV void lora_wrow_stage(uint16_t* ws, const FwdParams& p, int64_t tn, bool pair, int64_t c0, int tid) {
  constexpr int CH = BN * (BK / 8) / NT;
  u32x4_t o[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int q = tid + NT * c, R = q >> 3, ch = q & 7;
    int which; int64_t n;
    fwd_row(R, tn, pair, which, n);
    const float* lb = sel(p.lb, which);
    const float s = which ? p.s[1] : p.s[0];
    const int64_t cc = c0 + 8 * ch - (int64_t)which * p.r;   // first rank of the chunk
    float f[8];
    if (n < p.N && cc >= 0 && cc + 8 <= p.r && al16(lb + n * p.ldlb + cc)) {
      const f32x4_t lo = *reinterpret_cast<const f32x4_t*>(lb + n * p.ldlb + cc);
      const f32x4_t hi = *reinterpret_cast<const f32x4_t*>(lb + n * p.ldlb + cc + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) { f[i] = lo[i]; f[4 + i] = hi[i]; }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] = (n < p.N && cc + i >= 0 && cc + i < p.r) ? lb[n * p.ldlb + cc + i] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) o[c][i] = pack_bf16x2(s * f[2 * i], s * f[2 * i + 1]);
  }
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int q = tid + NT * c;
    *reinterpret_cast<u32x4_t*>(ws + loff(q >> 3, q & 7)) = o[c];
  }
}

// ---- epilogue staging of the 256 x 256 output tile in the four operand
// buffers (64 rows each, unpadded), 16-byte chunks XOR-swizzled by row so the
// column-strided fragment writes and the row-wise 16-byte reads are both
// conflict-free.
struct EpTile { uint16_t* b0; uint16_t* b1; uint16_t* b2; uint16_t* b3; };

MOLT_DEV uint16_t* ep_at(const EpTile& e, int row, int col) {
  const int c = row >> 6;
  uint16_t* base = c == 0 ? e.b0 : c == 1 ? e.b1 : c == 2 ? e.b2 : e.b3;
  return base + (row & 63) * 256 + ((((col >> 3) ^ (row & 31)) << 3) | (col & 7));
}

// Pair layout: subtiles 0,1 of a wave are gate and 2,3 the up rows of the same
// 64 intermediate columns. Staged as [X row][c] with c in 0..127 = gate of
// intermediate column tn*128 + c and 128 + c = up of the same column.
MOLT_DEV void stage_acc_pair(const EpTile& ep, const f32x16_t (&acc)[TM][TN], int wm, int wn, int lane) {
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int row = wm * WCOLS + j * 32 + (lane & 31);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int col = (i >> 1) * 128 + wn * 64 + (i & 1) * 32 + 8 * g + 4 * (lane >> 5);
        u32x2_t o = {pack_bf16x2(acc[i][j][4 * g], acc[i][j][4 * g + 1]),
                     pack_bf16x2(acc[i][j][4 * g + 2], acc[i][j][4 * g + 3])};
        *reinterpret_cast<u32x2_t*>(ep_at(ep, row, col)) = o;
      }
  }
}

MOLT_DEV void gateup_store(const EpTile& ep, const FwdParams& p, int64_t m0, int64_t tn, int tid) {
  // 256 rows x 16 chunks of 8 intermediate columns
#pragma unroll
  for (int it = 0; it < BM * 16 / NT; ++it) {
    const int q = tid + it * NT;
    const int row = q >> 4, ch = q & 15;
    const int64_t m = m0 + row, n = tn * (BN / 2) + 8 * ch;
    if (m >= p.M || n >= p.N) continue;
    const u32x4_t gw = *reinterpret_cast<const u32x4_t*>(ep_at(ep, row, 8 * ch));
    const u32x4_t uw = *reinterpret_cast<const u32x4_t*>(ep_at(ep, row, 128 + 8 * ch));
    u32x4_t hw;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float h0 = round_bf16(silu_f32(bf16_lo(gw[e]))) * bf16_lo(uw[e]);
      const float h1 = round_bf16(silu_f32(bf16_hi(gw[e]))) * bf16_hi(uw[e]);
      hw[e] = pack_bf16x2(h0, h1);
    }
    const int64_t off = m * p.ldy + n;
    if (p.vec_out && n + 8 <= p.N) {
      st_vec<kStreamOut>(p.y[0] + off, gw);
      st_vec<kStreamOut>(p.y[1] + off, uw);
      st_vec<kStreamOut>(p.y[2] + off, hw);
    } else {
      for (int e = 0; e < 8 && n + e < p.N; ++e) {
        const int w = e >> 1, sh = (e & 1) * 16;
        p.y[0][off + e] = (uint16_t)(gw[w] >> sh);
        p.y[1][off + e] = (uint16_t)(uw[w] >> sh);
        p.y[2][off + e] = (uint16_t)(hw[w] >> sh);
      }
    }
  }
}

// fp32 partial tile of a split-K launch: part[m][n0 ..] (row stride N, N a
// multiple of 256 so every 4-element group is inside the row), rows past M skipped.
MOLT_DEV void store_partial(float* part, int64_t M, int64_t N, const f32x16_t (&acc)[TM][TN], int64_t m0, int64_t n0,
                            int wm, int wn, int lane) {
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t m = m0 + wm * WCOLS + j * 32 + (lane & 31);
    if (m >= M) continue;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int64_t n = n0 + wn * WROWS + i * 32 + 8 * g + 4 * (lane >> 5);
        const f32x4_t v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
        *reinterpret_cast<f32x4_t*>(part + m * N + n) = v;
      }
  }
}

// Forward NF4 GEMM, 256 x 256 tile, 8 waves of 128 (W rows) x 64 (X rows).
//
// Pipeline of step s (BK = 64 contraction elements), all from LDS buffer s&1:
//  * the fragments of sub-step 0 are read while the MFMAs of the previous
//    step's last sub-step run (those fragments were held in registers across
//    the barrier, so the matrix core does not drain at every step);
//  * X(s+1) streams global -> LDS (buffer-load DMA) into the other buffer;
//  * the packed bytes of W(s+2) load into one register set while W(s+1), in
//    the other, is dequantised into the other W buffer a quarter per
//    sub-step, each quarter's table lookups one sub-step ahead of its use;
//  * one vmcnt(0) + barrier at the end of the step.
// Each operand buffer is its own __shared__ array and the loop is unrolled so
// that buffer choice is static: the compiler can then tell the LDS reads of
// one buffer from the DMA into the other and inserts no waits between them.
// Requires K % 128 == 0 (an even number of steps) and block size 64.
// STAGED: W arrives as the bf16 copy p.wst (the values the dequant would
// produce) by the same DMA as X, so a step is DMA, fragment reads and MFMAs
// only and the code-pair table is not needed.
template <bool PAIR, bool STAGED>
__global__ __launch_bounds__(NT) void fwd_kernel(const FwdParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t xb0[BUF], xb1[BUF], wb0[BUF], wb1[BUF];
  __shared__ float2 tab[STAGED ? 1 : 256 * TABC];
  __shared__ __attribute__((aligned(16))) uint16_t xb2[STAGED ? BUF : 8];   // the table's space
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WAVES_M, wn = wave / WAVES_M;
  const int64_t cols_per_tile = PAIR ? BN / 2 : BN;
  const int64_t nt_m = ceil_div64(p.M, BM), nt_n = ceil_div64(p.N, cols_per_tile);
  int64_t tm, tn;
  grouped_tile(xcd_tile(blockIdx.x, nt_m * nt_n), nt_m, nt_n, GROUP_M, tm, tn);
  const int64_t m0 = tm * BM;
  if constexpr (!STAGED) build_tab(tab, p.code, p.order, tid);
  const float2* tabc = tab + (lane & (TABC - 1));

  FragOff fo;
  frag_offsets(fo, wn * WROWS, wm * WCOLS, lane);
  f32x16_t acc[TM][TN];
  zero_acc(acc);

  // X: the 16-byte slot each lane fills in the 1 KB blocks its wave owns.
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.x, ((p.M - 1) * p.ldx + p.K) * 2);
  uint32_t xoff[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    int R, k;
    dma_slot(wave * 4 + c, lane, R, k);
    xoff[c] = (uint32_t)((min(m0 + R, p.M - 1) * p.ldx + k) * 2);
  }
  // W: row wR, bytes [16 * wh, +16) of the row's 32-byte slice of the step
  // (wslot); a wave covers 32 rows, so the weight (gate or up) is uniform over it.
  int wR, wh;
  wslot(tid, wR, wh);
  int which; int64_t n;
  fwd_row(wR, tn, PAIR, which, n);
  which = __builtin_amdgcn_readfirstlane(which);
  n = min(n, p.N - 1);
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(which ? p.packed[1] : p.packed[0], p.N * p.K / 2);
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(which ? p.scales[1] : p.scales[0], p.N * p.K / 64 * 4);
  const uint32_t woff = (uint32_t)(n * p.K / 2 + 16 * wh);
  const uint32_t soff = (uint32_t)(n * p.K / 64 * 4);

  auto x_load = [&](uint16_t* dst, int64_t k0) {
#pragma unroll
    for (int c = 0; c < 4; ++c) buf_load_lds16(xr, dst + (wave * 4 + c) * 512, xoff[c], (uint32_t)(k0 * 2));
  };
  auto w_load = [&](WBytes& w, int64_t k0) {
    w.q = buf_load16(wr, woff, (uint32_t)(k0 >> 1));
    w.sc = __builtin_bit_cast(float, buf_load4(sr, soff, (uint32_t)((k0 >> 6) * 4)));
  };
  const int ks = (int)(p.K / BK);
  const int64_t klast = p.K - BK;
  // this workgroup's steps: all of them, or split blockIdx.y's range (an even count)
  const int sbeg = p.part ? (int)blockIdx.y * p.split_steps : 0;
  const int send = p.part ? min(ks, sbeg + p.split_steps) : ks;

  bf16x8_t a[2][TM], b[2][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i) a[1][i] = bf16x8_t{};
#pragma unroll
  for (int j = 0; j < TN; ++j) b[1][j] = bf16x8_t{};

  if constexpr (STAGED) {
    // W tile row R by DMA from row n of its weight's bf16 copy; a DMA block is
    // 8 rows of one weight (gate and up alternate every 64 rows), so the
    // buffer resource is uniform per instruction. With p.lora_ring the LoRA
    // contraction follows as extra steps of the same ring: X from T (rank
    // columns), W from the weight's staged bf16(s B) rows [N, lrs], lrs = lr
    // rounded up to 64. A shorter lr is one step whose chunks past lr re-read
    // the row's own T columns (k mod lr): the staged rows are zero there, so
    // they add exact zeros, and a non-finite T value meets only its own row,
    // whose output it already makes non-finite. (A lane select of an
    // out-of-range offset instead made the compiler rebuild every step's DMA
    // offsets: +167 instructions.)
    const bool ring = p.lora_ring && (!p.part || blockIdx.y + 1 == gridDim.y);
    const int64_t lrs = ring ? p.lora_ring : 0;
    const int64_t xbytes = ((p.M - 1) * p.ldx + p.K) * 2, tbytes = ring ? ((p.M - 1) * p.ldt + p.lr) * 2 : 0;
    const int64_t wbytes = p.N * p.ldw * 2, bbytes = p.N * lrs * 2;
    uint32_t wdoff[4], toff[4], bdoff[4];
    int wsel[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      int R, k, which;
      int64_t nr;
      dma_slot(wave * 4 + c, lane, R, k);
      fwd_row(R, tn, PAIR, which, nr);
      wsel[c] = __builtin_amdgcn_readfirstlane(which);
      wdoff[c] = (uint32_t)((min(nr, p.N - 1) * p.ldw + k) * 2);
      bdoff[c] = (uint32_t)((min(nr, p.N - 1) * lrs + k) * 2);
      toff[c] = (uint32_t)((min(m0 + R, p.M - 1) * p.ldt + k % max(p.lr, 1)) * 2);
    }
    // step j of this workgroup: the contraction step sbeg + j, then the LoRA
    // steps; indices past the end repeat the last step (loads never read).
    const int n_main = send - sbeg, n_all = n_main + (int)(lrs / BK);
    // (buffer resources built from selected base pointers: a select of two
    // resources is lowered through memory)
    auto x_src = [&](uint16_t* dst, int j) {
      j = __builtin_amdgcn_readfirstlane(min(j, n_all - 1));
      const bool lo = j >= n_main;
      const __amdgpu_buffer_rsrc_t r = make_rsrc(pick<const void*>(lo, p.t, p.x), pick<int64_t>(lo, tbytes, xbytes));
      const uint32_t so = __builtin_amdgcn_readfirstlane(
          (uint32_t)((lo ? (int64_t)(j - n_main) * BK : (int64_t)(sbeg + j) * BK) * 2));
#pragma unroll
      for (int c = 0; c < 4; ++c) buf_load_lds16(r, dst + (wave * 4 + c) * 512, pick(lo, toff[c], xoff[c]), so);
    };
    auto w_src = [&](uint16_t* dst, int j) {
      j = __builtin_amdgcn_readfirstlane(min(j, n_all - 1));
      const bool lo = j >= n_main;
      const uint32_t so = __builtin_amdgcn_readfirstlane(
          (uint32_t)((lo ? (int64_t)(j - n_main) * BK : (int64_t)(sbeg + j) * BK) * 2));
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int w = PAIR ? wsel[c] : 0;
        const void* base = pick<const void*>(lo, sel(p.lbst, w), sel(p.wst, w));
        buf_load_lds16(make_rsrc(base, pick<int64_t>(lo, bbytes, wbytes)), dst + (wave * 4 + c) * 512,
                       pick(lo, bdoff[c], wdoff[c]), so);
      }
    };
    // X in a ring of three buffers, loaded two steps ahead; W in two, one
    // step ahead (its tiles are shared by every row block, mostly from L2).
    x_src(xb0, 0);
    w_src(wb0, 0);
    x_src(xb1, 1);
    wait_vm_at_most<kStageDma>();                    // X(0), W(0) landed; X(1) may fly
    step_barrier();
    // deq(W)^T for the input gradient: main step s of column tile tn is
    // written by the row block tm = s % nt_m, so each step's tile is written
    // once and the work is spread evenly over the row blocks. The stores are
    // issued before the step's DMA, so the closing wait (which leaves only
    // X(j + 2) in flight) also covers them and every step ends in the same
    // state. (Issuing them after the DMA and leaving them in flight into the
    // next step needs a different wait in those steps; the compiler then
    // waits more in the steps that follow, and it measured no faster.)
    const bool keep_t = p.wt_out[0] != nullptr;
    const int ntm = (int)nt_m, tm32 = (int)tm;
    auto step = [&](int j, const uint16_t* xc, const uint16_t* wc, uint16_t* x2, uint16_t* wnx) {
      if (keep_t && j < n_main && (sbeg + j) % ntm == tm32) {
        wt_tile_write(p, wc, tn, (int64_t)(sbeg + j) * BK, PAIR, tid);
        __builtin_amdgcn_sched_barrier(0);           // the stores stay ahead of the step's DMA
      }
      load_frags(wc, xc, fo, 0, a[0], b[0]);
      mfma_set(a[1], b[1], acc);
      w_src(wnx, j + 1);
      dma_then_loads();                              // keep W(j + 1) issued before X(j + 2)
      x_src(x2, j + 2);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kk = 0; kk < 3; ++kk) {
        load_frags(wc, xc, fo, kk + 1, a[(kk + 1) & 1], b[(kk + 1) & 1]);
        mfma_set(a[kk & 1], b[kk & 1], acc);
        __builtin_amdgcn_sched_barrier(0);
      }
      wait_vm_at_most<kStageDma>();                  // W(j + 1), X(j + 1) landed; X(j + 2) may fly
      step_barrier();
    };
    ring_steps(n_all, step, xb0, xb1, xb2, wb0, wb1);
    wait_vm0();                                      // the last step's X(j + 2), never read
    __syncthreads();
  } else {
    WBytes r0, r1;
    x_load(xb0, (int64_t)sbeg * BK);
    w_load(r0, (int64_t)sbeg * BK);
    wait_vm0();
    __syncthreads();  // table, X(sbeg)
    {
      float2 c[4];
#pragma unroll
      for (int d = 0; d < 4; ++d) { w_lookup(r0, tabc, d, c); w_finish(c, r0.sc, wb0, wR, wh, d); }
    }
    w_load(r0, min((int64_t)(sbeg + 1) * BK, klast));
    wait_vm0();
    __syncthreads();

    auto step = [&](int s, const WBytes& cw, WBytes& nw, const uint16_t* xc, const uint16_t* wc, uint16_t* xn,
                    uint16_t* wnx) {
      const int64_t k1 = min((int64_t)(s + 1) * BK, klast), k2 = min((int64_t)(s + 2) * BK, klast);
      float2 c[4];
      load_frags(wc, xc, fo, 0, a[0], b[0]);
      mfma_set(a[1], b[1], acc);
      x_load(xn, k1);
      dma_then_loads();
      w_load(nw, k2);
      w_lookup(cw, tabc, 0, c);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kk = 0; kk < 3; ++kk) {
        load_frags(wc, xc, fo, kk + 1, a[(kk + 1) & 1], b[(kk + 1) & 1]);
        mfma_set(a[kk & 1], b[kk & 1], acc);
        w_finish(c, cw.sc, wnx, wR, wh, kk);
        w_lookup(cw, tabc, kk + 1, c);
        interleave_substep();
        __builtin_amdgcn_sched_barrier(0);
      }
      w_finish(c, cw.sc, wnx, wR, wh, 3);
      wait_vm_at_most<WBytes::kLoads>();            // X(s + 1) landed; only W(s + 2)'s loads may fly
      step_barrier();
    };
    // W(s + 1) sits in r0 during even steps and in r1 during odd ones; the LDS buffers alternate likewise.
    for (int s = sbeg; s < send; s += 2) {
      step(s, r0, r1, xb0, wb0, xb1, wb1);
      step(s + 1, r1, r0, xb1, wb1, xb0, wb0);
    }
  }
  mfma_set(a[1], b[1], acc);
  // the LoRA steps belong to the last split (uniform per workgroup)
  const int64_t lr = (!p.part || blockIdx.y + 1 == gridDim.y) && !(STAGED && p.lora_ring) ? p.lr : 0;
  for (int64_t c0 = 0; c0 < lr; c0 += BK) {
    lora_a_stage(xb0, p.t, p.ldt, m0, p.M, c0, p.lr, tid);
    lora_wrow_stage(wb0, p, tn, PAIR, c0, tid);
    __syncthreads();
    compute(wb0, xb0, fo, acc);
    __syncthreads();
  }

  if (!PAIR) {
    if (p.part) {
      store_partial(p.part + (int64_t)blockIdx.y * p.M * p.N, p.M, p.N, acc, m0, tn * BN, wm, wn, lane);
      return;
    }
    const bool vec = p.vec_out != 0;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t m = m0 + wm * WCOLS + j * 32 + (lane & 31);
      if (m >= p.M) continue;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int64_t nn = tn * BN + wn * WROWS + i * 32 + 8 * g + 4 * (lane >> 5);
          float v[4] = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
          store4(p.y[0], p.ldy, m, nn, p.N, v, vec);
        }
      }
    }
    return;
  }
  // Gate/up pair: stage bf16 gate and up of the tile in LDS, then form
  // h = bf16(bf16(silu(g)) u) cooperatively with 16-byte loads and stores.
  const EpTile ep{xb0, xb1, wb0, wb1};
  stage_acc_pair(ep, acc, wm, wn, lane);
  __syncthreads();
  gateup_store(ep, p, m0, tn, tid);
}

// ===== backward (column-contract) kernel =====
// dX[M, Kw] = sum over segments of dY_seg[M, Nw] . deq(W_seg[Nw, Kw]) (+ LoRA).
// A tile row on the W side is an output column (a column of W); the
// contraction runs over rows of W. A thread dequantises a 4-row x 8-column
// patch (four 4-byte loads, one scale per row) and writes it transposed: rows
// (0, 1) and (2, 3) of the patch become bf16 pairs in 8 consecutive tile rows.
// One thread's backward W patch for one step: kRows rows of 8 packed codes
// (4 bytes) and each row's block scale. w_load issues two 4-byte loads per row,
// after the step's dY DMA, so kLoads is the closing wait's vmcnt.
struct WPatch {
  static constexpr int kRows = 4;
  static constexpr int kLoads = 2 * kRows;
  uint32_t q[kRows];
  float sc[kRows];
};

// Column group of a lane's 4 x 8 patch (the row group is tid / 32, so lanes l
// and l + 32 share a column group).
MOLT_DEV int patch_cg(int lane) {
  return (lane & 1) | (((lane >> 2) & 1) << 1) | (((lane >> 3) & 3) << 2) | (((lane >> 1) & 1) << 4);
}

// Lookups of byte b of the four patch rows: columns 2b, 2b + 1.
MOLT_DEV void wp_lookup(const WPatch& w, const float2* tabc, int b, float2 (&c)[4]) {
#pragma unroll
  for (int r = 0; r < 4; ++r) c[r] = tabc[((w.q[r] >> (8 * b)) & 0xffu) * TABC];
}

// bf16(code * scale) of columns 2b and 2b + 1, each as two bf16 pairs (patch rows 0,1 and 2,3).
MOLT_DEV void wp_finish(const float2 (&c)[4], const float (&sc)[4], u32x2_t& ce, u32x2_t& co) {
  ce[0] = pack_bf16x2(c[0].x * sc[0], c[1].x * sc[1]);
  ce[1] = pack_bf16x2(c[2].x * sc[2], c[3].x * sc[3]);
  co[0] = pack_bf16x2(c[0].y * sc[0], c[1].y * sc[1]);
  co[1] = pack_bf16x2(c[2].y * sc[2], c[3].y * sc[3]);
}

// Columns k and k + 4 of the thread's patch. Lanes l and l + 32 hold the two
// 4-row halves (rg even / odd) of the same 8 contraction rows: one
// v_permlane32_swap per dword gives lane l all 8 rows of column k and lane
// l + 32 all 8 rows of column k + 4, written as one 16-byte chunk each.
MOLT_DEV void wp_swap_write(const u32x2_t& lo, const u32x2_t& hi, uint16_t* ws, int cg, int rg, int k) {
  u32x4_t o;
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    const auto r = __builtin_amdgcn_permlane32_swap(lo[d], hi[d], false, false);
    o[d] = r[0];
    o[2 + d] = r[1];
  }
  *reinterpret_cast<u32x4_t*>(ws + loff(8 * cg + k + 4 * (rg & 1), rg >> 1)) = o;
}

// Whole patch (prologue): all four column pairs.
MOLT_DEV void wp_commit(const WPatch& w, const float2* tabc, uint16_t* ws, int cg, int rg) {
  float2 c[4];
  u32x2_t col[8];
#pragma unroll
  for (int b = 0; b < 4; ++b) { wp_lookup(w, tabc, b, c); wp_finish(c, w.sc, col[2 * b], col[2 * b + 1]); }
#pragma unroll
  for (int k = 0; k < 4; ++k) wp_swap_write(col[k], col[k + 4], ws, cg, rg, k);
}

// Backward W side of a LoRA step: element (output column R, rank c0 + k) =
// bf16(scale * A[c0 + k][col]). A thread loads a 4-rank x 8-column patch of A
// (16-byte loads along the columns) and transposes it so the ranks become
// contiguous in LDS.
MOLT_DEV void lora_wcol_stage(uint16_t* ws, const BwdParams& p, int seg, int64_t tn, int64_t c0, int tid) {
  static_assert(NT == 512, "one 4 x 8 patch per thread");
  const float* a = sel(p.la, seg);
  const int cg = tid & 31, rg = tid >> 5;            // 32 column groups of 8, 16 rank groups of 4
  const int64_t col = tn * BN + 8 * cg;
  float v[4][8];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t c = c0 + 4 * rg + r;
    const float* row = a + c * p.ldla + col;
    if (c < p.r && col + 8 <= p.Kw && al16(row)) {
      const f32x4_t lo = *reinterpret_cast<const f32x4_t*>(row);
      const f32x4_t hi = *reinterpret_cast<const f32x4_t*>(row + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) { v[r][i] = lo[i]; v[r][4 + i] = hi[i]; }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[r][i] = (c < p.r && col + i < p.Kw) ? row[i] : 0.0f;
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    u32x2_t o;
    o[0] = pack_bf16x2(p.la_scale * v[0][j], p.la_scale * v[1][j]);
    o[1] = pack_bf16x2(p.la_scale * v[2][j], p.la_scale * v[3][j]);
    *reinterpret_cast<u32x2_t*>(ws + loff(8 * cg + j, rg >> 1) + 4 * (rg & 1)) = o;
  }
}

// acc[i][j] holds C[W row][X row]: W row = wn*WROWS + 32i + 8(e/4) + 4(lane/32) + e%4,
// X row = wm*WCOLS + 32j + lane%32. Staged as [X row][W row] in bf16.
MOLT_DEV void stage_acc(const EpTile& ep, const f32x16_t (&acc)[TM][TN], int wm, int wn, int lane) {
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int row = wm * WCOLS + j * 32 + (lane & 31);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int col = wn * WROWS + i * 32 + 8 * g + 4 * (lane >> 5);
        u32x2_t o = {pack_bf16x2(acc[i][j][4 * g], acc[i][j][4 * g + 1]),
                     pack_bf16x2(acc[i][j][4 * g + 2], acc[i][j][4 * g + 3])};
        *reinterpret_cast<u32x2_t*>(ep_at(ep, row, col)) = o;
      }
  }
}

// SwiGLU backward epilogue (kernels/gated_activation.py:47-51 with MOLT's bf16
// rounding points): dh comes from the staged tile, gate/up from HBM. A thread
// owns SW_IT chunks of 8 intermediate columns (rows q / 32, chunk q % 32 for
// q = tid + NT * it); swiglu_load issues all of its gate/up loads at once, so
// they are in flight while the tile is staged and the workgroup synchronises.
constexpr int SW_IT = BM * 32 / NT;
struct SwigluIn { u32x4_t g[SW_IT], u[SW_IT]; };

template <int IT0 = 0, int NIT = SW_IT>
MOLT_DEV void swiglu_load(SwigluIn& in, const BwdParams& p, int64_t m0, int64_t tn, int tid) {
#pragma unroll
  for (int it = IT0; it < IT0 + NIT; ++it) {
    const int q = tid + it * NT;
    const int64_t m = m0 + (q >> 5), n = tn * BN + 8 * (q & 31);
    const int64_t off = m * p.ldg + n;
    if (m < p.M && p.vec_out && n + 8 <= p.Kw) {
      in.g[it] = *reinterpret_cast<const u32x4_t*>(p.gate + off);
      in.u[it] = *reinterpret_cast<const u32x4_t*>(p.up + off);
    } else {
      uint16_t gt[8], ut[8];
      for (int e = 0; e < 8; ++e) {
        const bool ok = m < p.M && n + e < p.Kw;
        gt[e] = ok ? p.gate[off + e] : (uint16_t)0;
        ut[e] = ok ? p.up[off + e] : (uint16_t)0;
      }
      in.g[it] = __builtin_bit_cast(u32x4_t, gt);
      in.u[it] = __builtin_bit_cast(u32x4_t, ut);
    }
  }
}

// gate/up loads of iterations IT0 .. IT0 + NIT - 1 for full 16-byte chunks
// (Kw and ldg multiples of 8, 16-byte aligned gate/up): every load is issued,
// chunks past M or Kw reading the first chunk instead (their results are not
// stored), so the loads are straight-line code and a later wait can leave the
// other batch in flight.
template <int IT0, int NIT>
MOLT_DEV void swiglu_load16(SwigluIn& in, const BwdParams& p, int64_t m0, int64_t tn, int tid) {
#pragma unroll
  for (int it = IT0; it < IT0 + NIT; ++it) {
    const int q = tid + it * NT;
    const int64_t m = m0 + (q >> 5), n = tn * BN + 8 * (q & 31);
    const int64_t off = m < p.M && n < p.Kw ? m * p.ldg + n : 0;
    in.g[it] = *reinterpret_cast<const u32x4_t*>(p.gate + off);
    in.u[it] = *reinterpret_cast<const u32x4_t*>(p.up + off);
  }
}

template <int IT0 = 0, int NIT = SW_IT>
MOLT_DEV void swiglu_bwd_store(const EpTile& ep, const BwdParams& p, int64_t m0, int64_t tn, int tid,
                               const SwigluIn& in) {
#pragma unroll
  for (int it = IT0; it < IT0 + NIT; ++it) {
    const int q = tid + it * NT;
    const int row = q >> 5, ch = q & 31;
    const int64_t m = m0 + row, n = tn * BN + 8 * ch;
    if (m >= p.M || n >= p.Kw) continue;
    const u32x4_t dh = *reinterpret_cast<const u32x4_t*>(ep_at(ep, row, 8 * ch));
    const u32x4_t gw = in.g[it], uw = in.u[it];
    const int64_t off = m * p.ldg + n;
    u32x4_t dgw, duw;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float dgo[2], duo[2];
      const float dhv[2] = {bf16_lo(dh[e]), bf16_hi(dh[e])};
      const float gv[2] = {bf16_lo(gw[e]), bf16_hi(gw[e])};
      const float uv[2] = {bf16_lo(uw[e]), bf16_hi(uw[e])};
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const float sg = __builtin_amdgcn_rcpf(1.0f + __expf(-gv[t]));
        duo[t] = dhv[t] * round_bf16(gv[t] * sg);
        dgo[t] = round_bf16(dhv[t] * uv[t]) * (sg * (1.0f + gv[t] * (1.0f - sg)));
      }
      dgw[e] = pack_bf16x2(dgo[0], dgo[1]);
      duw[e] = pack_bf16x2(duo[0], duo[1]);
    }
    if (p.vec_out && n + 8 <= p.Kw) {
      st_vec<kStreamOut>(p.dg + off, dgw);
      st_vec<kStreamOut>(p.du + off, duw);
    } else {
      for (int e = 0; e < 8 && n + e < p.Kw; ++e) {
        const int w = e >> 1, sh = (e & 1) * 16;
        p.dg[off + e] = (uint16_t)(dgw[w] >> sh);
        p.du[off + e] = (uint16_t)(duw[w] >> sh);
      }
    }
  }
}

// dg/du of iterations IT0 .. IT0 + NIT - 1 in the full-chunk case, as
// straight-line code: every lane issues its two 16-byte buffer stores
// (non-temporal), those of chunks past M or Kw with an offset past the end of
// the buffer, where the hardware drops them. With per-lane branches around
// the stores the compiler cannot count the stores in flight and waits for all
// of them before the next iteration's gate/up values, which serialises the
// epilogue on store latency.
template <int IT0, int NIT>
MOLT_DEV void swiglu_bwd_store16(const EpTile& ep, const BwdParams& p, int64_t m0, int64_t tn, int tid,
                                 const SwigluIn& in) {
  const int64_t bytes = ((p.M - 1) * p.ldg + p.Kw) * 2;
  const __amdgpu_buffer_rsrc_t rg = make_rsrc(p.dg, bytes), ru = make_rsrc(p.du, bytes);
#pragma unroll
  for (int it = IT0; it < IT0 + NIT; ++it) {
    const int q = tid + it * NT;
    const int row = q >> 5, ch = q & 31;
    const int64_t m = m0 + row, n = tn * BN + 8 * ch;
    const uint32_t off = m < p.M && n < p.Kw ? (uint32_t)((m * p.ldg + n) * 2) : 0x80000000u;
    const u32x4_t dh = *reinterpret_cast<const u32x4_t*>(ep_at(ep, row, 8 * ch));
    const u32x4_t gw = in.g[it], uw = in.u[it];
    u32x4_t dgw, duw;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float dgo[2], duo[2];
      const float dhv[2] = {bf16_lo(dh[e]), bf16_hi(dh[e])};
      const float gv[2] = {bf16_lo(gw[e]), bf16_hi(gw[e])};
      const float uv[2] = {bf16_lo(uw[e]), bf16_hi(uw[e])};
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const float sg = __builtin_amdgcn_rcpf(1.0f + __expf(-gv[t]));
        duo[t] = dhv[t] * round_bf16(gv[t] * sg);
        dgo[t] = round_bf16(dhv[t] * uv[t]) * (sg * (1.0f + gv[t] * (1.0f - sg)));
      }
      dgw[e] = pack_bf16x2(dgo[0], dgo[1]);
      duw[e] = pack_bf16x2(duo[0], duo[1]);
    }
    __builtin_amdgcn_raw_buffer_store_b128(dgw, rg, off, 0, kStreamOut ? 2 : 0);
    __builtin_amdgcn_raw_buffer_store_b128(duw, ru, off, 0, kStreamOut ? 2 : 0);
  }
}

// Interleave of one backward sub-step: 8 MFMAs, their LDS reads and VALU,
// then NW transposed-patch writes.
template <int NW>
MOLT_DEV void interleave_substep_bwd() {
#define MOLT_SGB(nds)                                   \
  __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    \
  __builtin_amdgcn_sched_group_barrier(0x100, nds, 0);  \
  __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
  MOLT_SGB(2) MOLT_SGB(2) MOLT_SGB(1) MOLT_SGB(1) MOLT_SGB(1) MOLT_SGB(1) MOLT_SGB(1) MOLT_SGB(1)
#undef MOLT_SGB
  if (NW) __builtin_amdgcn_sched_group_barrier(0x200, NW, 0);
}

// Backward NF4 GEMM, 256 (X rows) x 256 (output columns) tile, 8 waves of
// 128 x 64, the same pipeline as the forward kernel: X = dY of the step's
// segment by buffer-load DMA one step ahead, the W patch bytes one step ahead
// in registers, dequantised (one patch row per sub-step) into the other W
// buffer, last sub-step's MFMAs carried across the barrier. Requires
// Nw % 64 == 0, Kw % 8 == 0, an even number of steps and block size 64.
// STAGED: the W tile arrives by DMA from the transposed bf16 copy p.wst of
// each segment (row = output column, as the tile stores it), like the
// forward's staged variant.
template <int EPI, bool STAGED>
__global__ __launch_bounds__(NT) void bwd_kernel(const BwdParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t xb0[BUF], xb1[BUF], wb0[BUF], wb1[BUF];
  __shared__ float2 tab[STAGED ? 1 : 256 * TABC];
  __shared__ __attribute__((aligned(16))) uint16_t xb2[STAGED ? BUF : 8];   // the table's space
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WAVES_M, wn = wave / WAVES_M;
  const int64_t nt_m = ceil_div64(p.M, BM), nt_n = ceil_div64(p.Kw, BN);
  int64_t tm, tn;
  grouped_tile(xcd_tile(blockIdx.x, nt_m * nt_n), nt_m, nt_n, GROUP_M, tm, tn);
  const int64_t m0 = tm * BM;
  if constexpr (!STAGED) build_tab(tab, p.code, p.order, tid);
  const float2* tabc = tab + (lane & (TABC - 1));

  FragOff fo;
  frag_offsets(fo, wn * WROWS, wm * WCOLS, lane);
  f32x16_t acc[TM][TN];
  zero_acc(acc);

  // X (dY of a segment): per-lane DMA slots, one resource per segment.
  const int64_t xbytes = ((p.M - 1) * p.lddy + p.Nw) * 2;
  const __amdgpu_buffer_rsrc_t xr0 = make_rsrc(p.dy[0], xbytes), xr1 = make_rsrc(p.dy[1], xbytes);
  uint32_t xoff[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    int R, k;
    dma_slot(wave * 4 + c, lane, R, k);
    xoff[c] = (uint32_t)((min(m0 + R, p.M - 1) * p.lddy + k) * 2);
  }
  // W patch: rows c0 + 4 rg + r (r = 0..3), columns col .. col + 7; lanes l and
  // l + 32 take rank groups 2m and 2m + 1 of the same columns (the permlane32
  // swap pairs them) and a wave's 32 column groups cover 256 contiguous columns,
  // so each 4-byte load instruction reads 128 contiguous bytes of two rows.
  // A ds_write_b128 is served 8 consecutive lanes per cycle by the lane's
  // 16-byte slot (chunk position) mod 8; for the transposed store of row
  // R = 8 cg + k (+4) the position is m ^ f(R) and f(R) varies with cg & 3
  // only, so lane bits 0 and 2 carry those (two lanes per slot).
  const int cg = patch_cg(lane), rg = tid >> 5;
  const int64_t col = min(tn * BN + 8 * cg, p.Kw - 8);
  const int64_t wbytes = p.Nw * p.Kw / 2, sbytes = p.Nw * p.Kw / 16;
  const __amdgpu_buffer_rsrc_t wr0 = make_rsrc(p.packed[0], wbytes), wr1 = make_rsrc(p.packed[1], wbytes);
  const __amdgpu_buffer_rsrc_t sr0 = make_rsrc(p.scales[0], sbytes), sr1 = make_rsrc(p.scales[1], sbytes);
  const uint32_t woff = (uint32_t)(4 * rg * (p.Kw / 2) + col / 2);
  const uint32_t soff = (uint32_t)((4 * rg * (p.Kw / 64) + col / 64) * 4);

  const int kseg = (int)(p.Nw / BK);
  const int ks = p.nseg * kseg;
  // step -> (segment, first contraction row), clamped to the last step; at
  // most two segments, so a compare instead of a scalar division
  auto seg_of = [&](int s) { return min(s, ks - 1) >= kseg ? 1 : 0; };
  auto c0_of = [&](int s) { const int t = min(s, ks - 1); return (int64_t)(t - (t >= kseg ? kseg : 0)) * BK; };
  auto x_load = [&](uint16_t* dst, int s) {
    const __amdgpu_buffer_rsrc_t xr = seg_of(s) ? xr1 : xr0;
    const uint32_t so = (uint32_t)(c0_of(s) * 2);
#pragma unroll
    for (int c = 0; c < 4; ++c) buf_load_lds16(xr, dst + (wave * 4 + c) * 512, xoff[c], so);
  };
  auto w_load = [&](WPatch& w, int s) {
    const int sg = seg_of(s);
    const __amdgpu_buffer_rsrc_t wr = sg ? wr1 : wr0, sr = sg ? sr1 : sr0;
    const int64_t c0 = c0_of(s);
#pragma unroll
    for (int r = 0; r < WPatch::kRows; ++r) {   // WPatch::kLoads loads: two per row
      w.q[r] = buf_load4(wr, woff, (uint32_t)((c0 + r) * (p.Kw / 2)));
      w.sc[r] = __builtin_bit_cast(float, buf_load4(sr, soff, (uint32_t)((c0 + r) * (p.Kw / 64) * 4)));
    }
  };

  // this workgroup's steps: all of them, or split blockIdx.y's range (an even count)
  const int sbeg = p.part ? (int)blockIdx.y * p.split_steps : 0;
  const int send = p.part ? min(ks, sbeg + p.split_steps) : ks;

  bf16x8_t a[2][TM], b[2][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i) a[1][i] = bf16x8_t{};
#pragma unroll
  for (int j = 0; j < TN; ++j) b[1][j] = bf16x8_t{};

  if constexpr (STAGED) {
    // W tile row R = output column tn * BN + R, the row of the segment's
    // transposed copy; the step's contraction rows are its columns c0 .. c0 + 63.
    const int64_t wtbytes = p.Kw * p.ldw * 2;
    const __amdgpu_buffer_rsrc_t ws0 = make_rsrc(p.wst[0], wtbytes), ws1 = make_rsrc(p.wst[1], wtbytes);
    uint32_t wdoff[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      int R, k;
      dma_slot(wave * 4 + c, lane, R, k);
      wdoff[c] = (uint32_t)((min(tn * BN + R, p.Kw - 1) * p.ldw + k) * 2);
    }
    auto w_dma = [&](uint16_t* dst, int s) {
      const __amdgpu_buffer_rsrc_t wr = seg_of(s) ? ws1 : ws0;
      const uint32_t so = (uint32_t)(c0_of(s) * 2);
#pragma unroll
      for (int c = 0; c < 4; ++c) buf_load_lds16(wr, dst + (wave * 4 + c) * 512, wdoff[c], so);
    };
    // dY in a ring of three buffers, loaded two steps ahead; W in two, one
    // step ahead (as in the staged forward kernel).
    x_load(xb0, sbeg);
    w_dma(wb0, sbeg);
    x_load(xb1, sbeg + 1);
    wait_vm_at_most<kStageDma>();                    // dY(sbeg), W(sbeg) landed; dY(sbeg + 1) may fly
    step_barrier();
    auto step = [&](int s, const uint16_t* xc, const uint16_t* wc, uint16_t* x2, uint16_t* wnx) {
      load_frags(wc, xc, fo, 0, a[0], b[0]);
      mfma_set(a[1], b[1], acc);
      w_dma(wnx, s + 1);
      dma_then_loads();                              // keep W(s + 1) issued before dY(s + 2)
      x_load(x2, s + 2);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kk = 0; kk < 3; ++kk) {
        load_frags(wc, xc, fo, kk + 1, a[(kk + 1) & 1], b[(kk + 1) & 1]);
        mfma_set(a[kk & 1], b[kk & 1], acc);
        __builtin_amdgcn_sched_barrier(0);
      }
      wait_vm_at_most<kStageDma>();                  // W(s + 1), dY(s + 1) landed; dY(s + 2) may fly
      step_barrier();
    };
    // buffers of step s: dY s % 3, W s % 2, so the pattern repeats every 6 steps
    int s = sbeg;
    for (; s + 6 <= send; s += 6) {
      step(s, xb0, wb0, xb2, wb1);
      step(s + 1, xb1, wb1, xb0, wb0);
      step(s + 2, xb2, wb0, xb1, wb1);
      step(s + 3, xb0, wb1, xb2, wb0);
      step(s + 4, xb1, wb0, xb0, wb1);
      step(s + 5, xb2, wb1, xb1, wb0);
    }
    if (s + 2 <= send) {
      step(s, xb0, wb0, xb2, wb1);
      step(s + 1, xb1, wb1, xb0, wb0);
      s += 2;
    }
    if (s + 2 <= send) {
      step(s, xb2, wb0, xb1, wb1);
      step(s + 1, xb0, wb1, xb2, wb0);
    }
    wait_vm0();                                      // the last step's dY(s + 2), never read
    __syncthreads();
  } else {
    WPatch r0, r1;
    x_load(xb0, sbeg);
    w_load(r0, sbeg);
    wait_vm0();
    __syncthreads();  // table, X(sbeg)
    wp_commit(r0, tabc, wb0, cg, rg);
    w_load(r0, sbeg + 1);
    wait_vm0();
    __syncthreads();

    // Dequant of W(s+1) across the sub-steps: column pairs (0,1), (4,5) then
    // (2,3), (6,7), each pair's lookups one sub-step ahead; columns k and k + 4
    // are written together after the lane exchange.
    auto step = [&](int s, const WPatch& cw, WPatch& nw, const uint16_t* xc, const uint16_t* wc, uint16_t* xn,
                    uint16_t* wnx) {
      float2 c[4];
      u32x2_t c0, c1, c4, c5;
      load_frags(wc, xc, fo, 0, a[0], b[0]);
      mfma_set(a[1], b[1], acc);
      x_load(xn, s + 1);
      dma_then_loads();
      w_load(nw, s + 2);
      wp_lookup(cw, tabc, 0, c);
      __builtin_amdgcn_sched_barrier(0);
      load_frags(wc, xc, fo, 1, a[1], b[1]);
      mfma_set(a[0], b[0], acc);
      wp_finish(c, cw.sc, c0, c1);
      wp_lookup(cw, tabc, 2, c);
      interleave_substep_bwd<0>();
      __builtin_amdgcn_sched_barrier(0);
      load_frags(wc, xc, fo, 2, a[0], b[0]);
      mfma_set(a[1], b[1], acc);
      wp_finish(c, cw.sc, c4, c5);
      wp_swap_write(c0, c4, wnx, cg, rg, 0);
      wp_swap_write(c1, c5, wnx, cg, rg, 1);
      wp_lookup(cw, tabc, 1, c);
      interleave_substep_bwd<2>();
      __builtin_amdgcn_sched_barrier(0);
      load_frags(wc, xc, fo, 3, a[1], b[1]);
      mfma_set(a[0], b[0], acc);
      wp_finish(c, cw.sc, c0, c1);
      wp_lookup(cw, tabc, 3, c);
      interleave_substep_bwd<0>();
      __builtin_amdgcn_sched_barrier(0);
      wp_finish(c, cw.sc, c4, c5);
      wp_swap_write(c0, c4, wnx, cg, rg, 2);
      wp_swap_write(c1, c5, wnx, cg, rg, 3);
      wait_vm_at_most<WPatch::kLoads>();            // dY(s + 1) landed; only W(s + 2)'s loads may fly
      step_barrier();
    };
    for (int s = sbeg; s < send; s += 2) {
      step(s, r0, r1, xb0, wb0, xb1, wb1);
      step(s + 1, r1, r0, xb1, wb1, xb0, wb0);
    }
  }
  mfma_set(a[1], b[1], acc);
  // the LoRA steps belong to the last split (uniform per workgroup)
  const int lr = !p.part || blockIdx.y + 1 == gridDim.y ? p.r : 0;
  for (int seg = 0; seg < p.nseg && lr > 0; ++seg) {
    for (int64_t c0 = 0; c0 < p.r; c0 += BK) {
      lora_a_stage(xb0, sel(p.u, seg), p.ldu, m0, p.M, c0, p.r, tid);
      lora_wcol_stage(wb0, p, seg, tn, c0, tid);
      __syncthreads();
      compute(wb0, xb0, fo, acc);
      __syncthreads();
    }
  }

  if (EPI == EPI_STORE && p.part) {
    store_partial(p.part + (int64_t)blockIdx.y * p.M * p.Kw, p.M, p.Kw, acc, m0, tn * BN, wm, wn, lane);
    return;
  }
  if (EPI == EPI_STORE) {
    const bool vec = p.vec_out != 0;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t m = m0 + wm * WCOLS + j * 32 + (lane & 31);
      if (m >= p.M) continue;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int64_t n = tn * BN + wn * WROWS + i * 32 + 8 * g + 4 * (lane >> 5);
          float v[4] = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
          store4(p.dx, p.lddx, m, n, p.Kw, v, vec);
        }
      }
    }
    return;
  }
  // SwiGLU backward: stage dh = bf16(acc) of the tile, then compute dgate/dup
  // cooperatively with 16-byte loads of gate/up and 16-byte stores.
  const EpTile ep{xb0, xb1, wb0, wb1};
  SwigluIn in;
  if constexpr (!STAGED) {   // (the fused kernel's registers leave no room for the batches below)
    stage_acc(ep, acc, wm, wn, lane);
    swiglu_load(in, p, m0, tn, tid);
    __syncthreads();
    swiglu_bwd_store(ep, p, m0, tn, tid, in);
    return;
  }
  // full 16-byte chunks (and byte offsets that fit the buffer resources):
  // gate/up in two batches, the first in flight while dh is staged, the
  // second while the first half's outputs are formed and stored
  const bool full16 = p.vec_out && p.ldg % 8 == 0 && p.Kw % 8 == 0 &&
                      ((((uintptr_t)p.gate | (uintptr_t)p.up | (uintptr_t)p.dg | (uintptr_t)p.du) & 15) == 0) &&
                      ((p.M - 1) * p.ldg + p.Kw) * 2 < ((int64_t)1 << 31);
  constexpr int H = SW_IT / 2;
  if (full16) swiglu_load16<0, H>(in, p, m0, tn, tid);
  else swiglu_load<0, H>(in, p, m0, tn, tid);
  stage_acc(ep, acc, wm, wn, lane);
  __syncthreads();
  if (full16) {
    swiglu_load16<H, H>(in, p, m0, tn, tid);
    swiglu_bwd_store16<0, H>(ep, p, m0, tn, tid, in);
    swiglu_bwd_store16<H, H>(ep, p, m0, tn, tid, in);
  } else {
    swiglu_load<H, H>(in, p, m0, tn, tid);
    swiglu_bwd_store<0, H>(ep, p, m0, tn, tid, in);
    swiglu_bwd_store<H, H>(ep, p, m0, tn, tid, in);
  }
}

// Transposed bf16 copy of one or two weights for the staged input-gradient
// kernels: wt[k][n] = bf16(code(W[n][k]) * scale(n, k / 64)), the values the
// fused kernel dequantises into its W tile. A workgroup converts tiles of 64
// weight rows x 256 columns with the fused kernel's 4 x 8 patches and lane
// exchange into an LDS tile in the operand layout (row = column k of W), then
// writes the tile's 256 rows of 128 bytes, 8 lanes per row, as whole-line
// 16-byte stores. blockIdx.z selects the weight. Requires Nw % 64 == 0,
// Kw % 256 == 0 and 4-byte aligned packed data.
struct StageTParams {
  const uint8_t* packed[2]; const float* scales[2]; uint16_t* wt[2];
  const float* code; int order; int64_t Nw, Kw, ldw;
};

__global__ __launch_bounds__(NT) void stage_wt_kernel(const StageTParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[BUF];
  __shared__ float2 tab[256 * TABC];
  const int tid = threadIdx.x, lane = tid & 63;
  build_tab(tab, p.code, p.order, tid);
  const float2* tabc = tab + (lane & (TABC - 1));
  const int seg = blockIdx.z;
  const uint8_t* packed = sel(p.packed, seg);
  const float* scales = sel(p.scales, seg);
  uint16_t* wt = sel(p.wt, seg);
  const int cg = patch_cg(lane), rg = tid >> 5;
  const int64_t col = (int64_t)blockIdx.x * BN + 8 * cg;
  const int64_t n_tiles = p.Nw / 64;
  __syncthreads();  // table
  for (int64_t nt = blockIdx.y; nt < n_tiles; nt += gridDim.y) {
    WPatch w;
#pragma unroll
    for (int r = 0; r < WPatch::kRows; ++r) {
      const int64_t n = nt * 64 + 4 * rg + r;
      w.q[r] = *reinterpret_cast<const uint32_t*>(packed + n * (p.Kw / 2) + col / 2);
      w.sc[r] = scales[n * (p.Kw / 64) + col / 64];
    }
    wp_commit(w, tabc, tile, cg, rg);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < BUF / 8 / NT; ++i) {
      const int q = tid + NT * i, R = q >> 3, c = q & 7;
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(tile + loff(R, c));
      *reinterpret_cast<u32x4_t*>(wt + ((int64_t)blockIdx.x * BN + R) * p.ldw + nt * 64 + 8 * c) = v;
    }
    __syncthreads();
  }
}

// Everything a staged forward GEMM reads besides X and T, in one launch: the
// bf16 rows of each weight and the ring's bf16(s B) rows. Job j takes blocks
// first[j] .. first[j + 1] - 1 (uniform per block).
//  * kind 0, a weight of `units` 8-element units with block size 64 and
//    resolved fp32 scales: bf16(code * scale) per element, the values (and
//    the code-pair table, arithmetic and rounding) of molt_nf4_dequantize's
//    flat-scale path, so the staged copy is bitwise that call's output. A
//    thread takes 4 units, all loads issued before any use, and 16-byte
//    non-temporal stores.
//  * kind 1, the bf16 LoRA operand of one weight for the ring's LoRA steps
//    (the values the fused kernel stages into LDS): o[n][c] for c < lr is
//    bf16(s B[n][c - woff]) where 0 <= c - woff < r, else bf16(s 0). One
//    weight has woff = 0; in the gate/up pair the up rows have woff = r (gate
//    ranks first); lr is r, 2r, or 64 when that is shorter. One thread per 8
//    consecutive columns.
constexpr int kStageJobs = 10;
constexpr int kStageUnits = 4;
struct StageJobs {
  const void* src[kStageJobs];      // packed bytes (kind 0) or fp32 B (kind 1)
  const float* scales[kStageJobs];  // kind 0: resolved scales
  const float* code[kStageJobs];    // kind 0: the 16 codes
  uint16_t* out[kStageJobs];
  int64_t count[kStageJobs];        // kind 0: units; kind 1: B rows
  int64_t ldb[kStageJobs];
  float s[kStageJobs];
  int kind[kStageJobs], order[kStageJobs], r[kStageJobs], woff[kStageJobs], lr[kStageJobs];
  int first[kStageJobs + 1];
  int n;
};

__global__ __launch_bounds__(256) void stage_kernel(const StageJobs J) {
  __shared__ float2 tab[256];
  int j = 0;
#pragma unroll
  for (int k = 1; k < kStageJobs; ++k) j += (k < J.n && (int)blockIdx.x >= J.first[k]) ? 1 : 0;
  const int64_t blk = (int64_t)blockIdx.x - J.first[j];
  if (J.kind[j] == 0) {
    {
      const float* code = J.code[j];
      const int b = threadIdx.x, hi = b >> 4, lo = b & 15, order = J.order[j];
      tab[b] = make_float2(code[order ? hi : lo], code[order ? lo : hi]);
    }
    __syncthreads();
    const uint8_t* packed = static_cast<const uint8_t*>(J.src[j]);
    const float* scales = J.scales[j];
    const int64_t units = J.count[j];
    uint32_t q[kStageUnits];
    float sc[kStageUnits];
#pragma unroll
    for (int i = 0; i < kStageUnits; ++i) {
      const int64_t u = min(blk * 256 * kStageUnits + i * 256 + threadIdx.x, units - 1);
      q[i] = *reinterpret_cast<const uint32_t*>(packed + 4 * u);
    }
#pragma unroll
    for (int i = 0; i < kStageUnits; ++i) {
      const int64_t u = min(blk * 256 * kStageUnits + i * 256 + threadIdx.x, units - 1);
      sc[i] = scales[(8 * u) >> 6];
    }
#pragma unroll
    for (int i = 0; i < kStageUnits; ++i) {
      const int64_t u = blk * 256 * kStageUnits + i * 256 + threadIdx.x;
      if (u >= units) continue;
      u32x4_t w;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float2 pr = tab[(q[i] >> (8 * e)) & 0xffu];
        w[e] = pack_bf16x2(pr.x * sc[i], pr.y * sc[i]);
      }
      __builtin_nontemporal_store(w, reinterpret_cast<u32x4_t*>(J.out[j] + 8 * u));
    }
  } else {
    const int lr = J.lr[j], chunks = lr / 8, r = J.r[j];
    const int64_t q = blk * 256 + threadIdx.x;
    if (q >= J.count[j] * chunks) return;
    const int64_t n = q / chunks;
    const int c0 = (int)(q - n * chunks) * 8 - J.woff[j];
    const float* b = static_cast<const float*>(J.src[j]);
    const float s = J.s[j];
    float f[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (c0 + i >= 0 && c0 + i < r) ? b[n * J.ldb[j] + c0 + i] : 0.0f;
    u32x4_t v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = pack_bf16x2(s * f[2 * i], s * f[2 * i + 1]);
    *reinterpret_cast<u32x4_t*>(J.out[j] + n * lr + (q - n * chunks) * 8) = v;
  }
}

// Host-side list of stage_kernel jobs, launched once.
struct Stager {
  StageJobs J{};
  int blocks = 0;
  void add(int kind, int64_t count, int64_t nblocks) {
    J.kind[J.n] = kind;
    J.count[J.n] = count;
    J.first[J.n] = blocks;
    blocks += (int)nblocks;
    J.first[++J.n] = blocks;
  }
  // a weight with resolved scales, block size 64 and rows * cols % 8 == 0
  void weight(const molt_nf4_weight& w, uint16_t* out) {
    const int i = J.n;
    J.src[i] = w.packed; J.scales[i] = w.scales; J.code[i] = w.code; J.order[i] = w.nibble_order; J.out[i] = out;
    const int64_t units = w.rows * w.cols / 8;
    add(0, units, ceil_div64(units, 256 * kStageUnits));
  }
  void lora_b(const float* b, int64_t ldb, int r, int woff, float s, int64_t rows, int lr, uint16_t* out) {
    const int i = J.n;
    J.src[i] = b; J.ldb[i] = ldb; J.r[i] = r; J.woff[i] = woff; J.s[i] = s; J.lr[i] = lr; J.out[i] = out;
    add(1, rows, ceil_div64(rows * (lr / 8), 256));
  }
  void launch(hipStream_t stream) const {
    if (J.n) hipLaunchKernelGGL(stage_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, J);
  }
};

}  // namespace big

// y[m, n] = bf16(sum over splits s = 0, 1, .. of part[s][m][n]): the splits
// are added in order, so the result does not depend on which workgroup of the
// split-K launch finished first. Four consecutive n per thread (N % 4 == 0).
__global__ void split_sum_kernel(const float* __restrict__ part, int splits, int64_t M, int64_t N,
                                 uint16_t* __restrict__ y, int64_t ldy) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= M * (N / 4)) return;
  const int64_t m = q / (N / 4), n = 4 * (q - m * (N / 4));
  f32x4_t v = *reinterpret_cast<const f32x4_t*>(part + m * N + n);
  for (int s = 1; s < splits; ++s) {
    const f32x4_t w = *reinterpret_cast<const f32x4_t*>(part + (int64_t)s * M * N + m * N + n);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] += w[e];
  }
  uint16_t* dst = y + m * ldy + n;
  if (((uintptr_t)dst & 7) == 0) {
    const u32x2_t o = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    *reinterpret_cast<u32x2_t*>(dst) = o;
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) dst[e] = bf16_bits(v[e]);
  }
}

// ------------------------------------------------------------- host helpers
bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// Below this many 256 x 256 tiles the 128 x 128 kernels fill the 256 CUs
// better. The MOLT_TUNE_BIG_TILE_MIN setting overrides the threshold (tests use
// it to run the large-tile kernels at small shapes).
int64_t big_tile_min() { return molt::tuning_value(MOLT_TUNE_BIG_TILE_MIN); }

// Split-K: a plain-store GEMM whose output has too few tiles to fill the CUs
// but a long contraction runs S workgroups per tile over contiguous ranges of
// split_steps 64-deep steps, S the largest with tiles * S <= CUs (at most 8)
// that leaves every range at least min_steps steps (an even count for the
// large-tile kernel, which runs steps in pairs). Returns S (1 = no split).
int plan_splits(int64_t tiles, int64_t steps, int64_t min_steps, bool even, int& split_steps) {
  split_steps = (int)steps;
  if (molt::tuning_value(MOLT_TUNE_SPLIT_K) == 0) return 1;
  int S = (int)std::min<int64_t>(8, molt::device_cus() / std::max<int64_t>(tiles, 1));
  while (S > 1 && steps / S < min_steps) --S;
  if (S <= 1) return 1;
  const int64_t per = ceil_div64(steps, S);
  split_steps = (int)(even ? 2 * ceil_div64(per, 2) : per);
  return (int)ceil_div64(steps, split_steps);
}

// The fewest steps per range: MOLT_TUNE_SPLIT_MIN_STEPS for a 256 x 256 tile;
// a 128 x 128 step is a quarter of the work, so a quarter of that for the
// small kernels.
int64_t split_min_big() { return molt::tuning_value(MOLT_TUNE_SPLIT_MIN_STEPS); }
int64_t split_min_small() { return std::max<int64_t>(1, split_min_big() / 4); }

// The 256 x 256 kernels run an even number of 64-deep steps and address X
// (dY), the packed bytes and the scales through 32-bit buffer offsets.
bool fwd_big_ok(int64_t M, int64_t ldx, int64_t N, int64_t K, bool al) {
  const int64_t lim = 0x7fffffffll;
  return al && K % 128 == 0 && ((M - 1) * ldx + K) * 2 <= lim && N * K / 2 <= lim && N * K / 16 <= lim;
}
bool bwd_big_ok(int64_t M, int64_t lddy, int64_t Nw, int64_t Kw, int nseg) {
  const int64_t lim = 0x7fffffffll;
  return (nseg * (Nw / 64)) % 2 == 0 && ((M - 1) * lddy + Nw) * 2 <= lim && Nw * Kw / 2 <= lim && Nw * Kw / 16 <= lim;
}

// A split large-tile launch is taken only when its workgroups occupy at least
// half the CUs; a narrower output (the 1536 -> 256 grouped-query projections)
// fills the GPU better as 128 x 128 tiles, split or not.
bool fills_half(int64_t workgroups) { return 2 * workgroups >= molt::device_cus(); }

// Kernel choice of one GEMM: the 256 x 256 kernels (unsplit or split-K), or
// the 128 x 128 kernels (split-K or unsplit).
enum { PLAN_BIG = 0, PLAN_BIG_SPLIT = 1, PLAN_SMALL_SPLIT = 2, PLAN_SMALL = 3 };
struct GemmPlan { int kind, S, split_steps; };

// Forward Y[M, N] over K: big_ok / al say whether the operands qualify for the
// large-tile kernels / the 128 x 128 kernels' aligned path.
GemmPlan fwd_plan(int64_t M, int64_t N, int64_t K, bool pair, bool big_ok, bool al) {
  const int64_t big_tiles = ceil_div64(M, big::BM) * ceil_div64(N, pair ? big::BN / 2 : big::BN);
  if (big_ok && big_tiles >= big_tile_min()) return {PLAN_BIG, 1, 0};
  int ss = 0;
  if (big_ok && !pair && N % big::BN == 0) {
    const int S = plan_splits(big_tiles, K / BK, split_min_big(), true, ss);
    if (S > 1 && fills_half(big_tiles * S)) return {PLAN_BIG_SPLIT, S, ss};
  }
  if (al && !pair && N % 4 == 0) {
    const int S = plan_splits(ceil_div64(M, BM) * ceil_div64(N, BN), ceil_div64(K, BK), split_min_small(), false, ss);
    if (S > 1) return {PLAN_SMALL_SPLIT, S, ss};
  }
  return {PLAN_SMALL, 1, 0};
}

// Input gradient dX[M, Kw] over nseg segments of Nw (EPI_SWIGLU_BWD never splits).
GemmPlan bwd_plan(int64_t M, int64_t Nw, int64_t Kw, int nseg, bool swiglu, bool big_ok, bool al) {
  const int64_t big_tiles = ceil_div64(M, big::BM) * ceil_div64(Kw, big::BN);
  if (big_ok && big_tiles >= big_tile_min()) return {PLAN_BIG, 1, 0};
  int ss = 0;
  if (big_ok && !swiglu && Kw % big::BN == 0) {
    const int S = plan_splits(big_tiles, nseg * (Nw / BK), split_min_big(), true, ss);
    if (S > 1 && fills_half(big_tiles * S)) return {PLAN_BIG_SPLIT, S, ss};
  }
  if (al && !swiglu && Kw % 4 == 0) {
    const int S = plan_splits(ceil_div64(M, BM) * ceil_div64(Kw, BN), nseg * ceil_div64(Nw, BK), split_min_small(),
                              false, ss);
    if (S > 1) return {PLAN_SMALL_SPLIT, S, ss};
  }
  return {PLAN_SMALL, 1, 0};
}

size_t split_bytes(int S, int64_t M, int64_t N) { return S > 1 ? (size_t)S * M * N * sizeof(float) : 0; }

// Staged weights: a 256 x 256 GEMM over many 256-row blocks of X (dY)
// dequantises each weight tile once per row block. From
// MOLT_TUNE_STAGE_MIN_MTILES row blocks on, one pass writes the bf16 weight
// (transposed for the input gradient) to the caller's workspace and the
// kernels read it by DMA; the weight tile values, and so the results, are the
// same. The copy is addressed with 32-bit offsets.
bool stage_wanted(int kind, int64_t M, int64_t rows, int64_t cols) {
  const int64_t t = molt::tuning_value(MOLT_TUNE_STAGE_MIN_MTILES);
  return (kind == PLAN_BIG || kind == PLAN_BIG_SPLIT) && t > 0 && ceil_div64(M, big::BM) >= t &&
         rows * cols * 2 < 0x7fffffffll;
}
size_t stage_one(int64_t rows, int64_t cols) { return (size_t)(rows * cols * 2 + 255) / 256 * 256; }

// Columns of the staged bf16(s B) rows the forward ring streams for a LoRA
// contraction of length lr, or 0 when the ring does not take it: a multiple of
// 64 runs as lr / 64 ring steps; a shorter one (a multiple of 8: 16 for one
// rank-16 adapter, 32 for the gate/up pair) as one step over rows padded with
// zeros to 64, its T columns past lr read as zeros.
int64_t ring_cols(int64_t lr) {
  if (lr > 0 && lr % BK == 0) return lr;
  return lr > 0 && lr < BK && lr % 8 == 0 ? BK : 0;
}

// molt_amd_time_next_gemm: a GEMM entry point takes (and so disarms) the
// events as it starts, whatever it then does; a call that returns early leaves
// them unrecorded instead of passing them on to a later, unrelated GEMM.
struct GemmEvents {
  void* start = nullptr;
  void* end = nullptr;
  GemmEvents() { molt::take_gemm_events(&start, &end); }
};

// The taken events are recorded right around the GEMM kernel's launch
// (construct before, finish() after).
struct KernelEvents {
  const GemmEvents& ev;
  hipStream_t stream;
  KernelEvents(const GemmEvents& e, hipStream_t s) : ev(e), stream(s) {
    if (ev.start) (void)hipEventRecord(static_cast<hipEvent_t>(ev.start), stream);
  }
  void finish() {
    if (ev.end) (void)hipEventRecord(static_cast<hipEvent_t>(ev.end), stream);
  }
};

// Workspace layout of the GEMM entry points: the staged weights (if any),
// their bf16 LoRA operands for the ring (if any: lora_rows x
// ring_cols(lora_cols) per weight), then the split-K partials (if any). A
// workspace too small for the LoRA copies stages the weights alone.
struct GemmWorkspace { bool stage, ring, split; size_t stage_bytes, lora_bytes; };
GemmWorkspace place_workspace(const GemmPlan& plan, bool want_stage, int weights, int64_t rows, int64_t cols,
                              int64_t lora_rows, int64_t lora_cols, int64_t M, int64_t out_n, const void* ws,
                              size_t ws_bytes) {
  GemmWorkspace g{false, false, false, 0, 0};
  const size_t sb = want_stage ? weights * stage_one(rows, cols) : 0;
  const bool want_ring = want_stage && ring_cols(lora_cols) > 0;
  const size_t lb = want_ring ? weights * stage_one(lora_rows, ring_cols(lora_cols)) : 0;
  const size_t pb = split_bytes(plan.S, M, out_n);
  const bool usable = ws && aligned(ws, 256);
  g.stage = want_stage && usable && ws_bytes >= sb + pb;
  g.ring = g.stage && want_ring && ws_bytes >= sb + lb + pb;
  g.stage_bytes = g.stage ? sb : 0;
  g.lora_bytes = g.ring ? lb : 0;
  g.split = plan.S > 1 && usable && ws_bytes >= g.stage_bytes + g.lora_bytes + pb;
  return g;
}

int check_weight_for_gemm(const molt_nf4_weight* w, const char* who) {
  MOLT_REQUIRE(w && w->packed && w->code, MOLT_EINVAL, "%s: weight, packed and code are required", who);
  MOLT_REQUIRE(w->scales, MOLT_EINVAL, "%s: resolved fp32 scales are required (molt_nf4_resolve_scales)", who);
  MOLT_REQUIRE(w->rows > 0 && w->cols > 0, MOLT_EINVAL, "%s: empty weight", who);
  MOLT_REQUIRE(w->block_size >= 2 && w->block_size % 2 == 0, MOLT_EINVAL, "%s: bad block size %d", who, w->block_size);
  MOLT_REQUIRE(w->nibble_order == 0 || w->nibble_order == 1, MOLT_EINVAL, "%s: bad nibble order", who);
  return MOLT_OK;
}

bool same_format(const molt_nf4_weight* a, const molt_nf4_weight* b) {
  return a->rows == b->rows && a->cols == b->cols && a->block_size == b->block_size &&
         a->nibble_order == b->nibble_order && a->code == b->code;
}

}  // namespace
}  // namespace molt

using namespace molt;

extern "C" int molt_nf4_lora_forward_impl(const uint16_t* x, int64_t ldx, int64_t M,
                                          const molt_nf4_weight* w0, const molt_nf4_weight* w1,
                                          const uint16_t* t, int64_t ldt, int lr,
                                          const float* b0, const float* b1, int64_t ldb, int r,
                                          float s0, float s1, uint16_t* y0, uint16_t* y1,
                                          uint16_t* y2, int64_t ldy, const molt::WtHandoff* wt,
                                          void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const char* who = "molt_nf4_lora_forward";
  const GemmEvents armed;
  int rc = check_weight_for_gemm(w0, who);
  if (rc) return rc;
  const bool pair = w1 != nullptr;
  if (pair) {
    rc = check_weight_for_gemm(w1, who);
    if (rc) return rc;
    MOLT_REQUIRE(same_format(w0, w1), MOLT_EINVAL, "%s: gate and up weights must share shape and format", who);
  }
  MOLT_REQUIRE(M >= 0 && ldx >= w0->cols, MOLT_EINVAL, "%s: bad X", who);
  MOLT_REQUIRE(ldy >= w0->rows, MOLT_EINVAL, "%s: bad Y", who);
  MOLT_REQUIRE(lr == 0 || (ldt >= lr && b0 && (!pair || b1) && r > 0 && ldb >= r), MOLT_EINVAL,
               "%s: bad LoRA operands", who);
  if (M == 0) return MOLT_OK;   // an empty token batch: no pointers are read (they may be null)
  MOLT_REQUIRE(x && y0 && (!pair || (y1 && y2)) && (lr == 0 || t), MOLT_EINVAL, "%s: null X, Y or T", who);

  FwdParams p{};
  p.x = x; p.ldx = ldx; p.M = M; p.K = w0->cols;
  p.packed[0] = w0->packed; p.scales[0] = w0->scales;
  p.packed[1] = pair ? w1->packed : w0->packed; p.scales[1] = pair ? w1->scales : w0->scales;
  p.N = w0->rows; p.code = w0->code; p.order = w0->nibble_order; p.block_size = w0->block_size;
  p.t = t; p.ldt = ldt; p.lr = lr;
  p.lb[0] = b0; p.lb[1] = pair ? b1 : b0; p.ldlb = ldb; p.r = r; p.s[0] = s0; p.s[1] = s1;
  p.y[0] = y0; p.y[1] = y1; p.y[2] = y2; p.ldy = ldy;
  p.vec_out = (ldy % 4 == 0) && aligned(y0, 8) && (!pair || (aligned(y1, 8) && aligned(y2, 8)));

  const bool al = (p.K % 64 == 0) && p.block_size == 64 && ldx % 8 == 0 && aligned(x, 16) &&
                  aligned(w0->packed, 16) && (!pair || aligned(w1->packed, 16));
  const int64_t big_tiles = ceil_div64(M, big::BM) * ceil_div64(p.N, pair ? big::BN / 2 : big::BN);
  const GemmPlan plan = fwd_plan(M, p.N, p.K, pair, fwd_big_ok(M, ldx, p.N, p.K, al), al);
  // the LoRA ring reads T by DMA: 16-byte aligned rows
  const bool t_dma = lr > 0 && t && aligned(t, 16) && ldt % 8 == 0;
  const GemmWorkspace gw = place_workspace(plan, stage_wanted(plan.kind, M, p.N, p.K), pair ? 2 : 1, p.N, p.K, p.N,
                                           t_dma ? lr : 0, M, p.N, workspace, workspace_bytes);
  char* wsb = static_cast<char*>(workspace);
  const bool split = gw.split;
  if (plan.kind == PLAN_BIG || (plan.kind == PLAN_BIG_SPLIT && split)) {
    MOLT_REQUIRE(big_tiles < (1ll << 31), MOLT_EINVAL, "%s: problem too large", who);
    if (plan.kind == PLAN_BIG_SPLIT) {
      p.split_steps = plan.split_steps;
      p.part = reinterpret_cast<float*>(wsb + gw.stage_bytes + gw.lora_bytes);
    }
    // the staged operands in one launch: the bf16 weight rows (resolved
    // scales, the flat-scale dequant) and the ring's bf16(s B) rows
    big::Stager stager;
    if (gw.ring) {
      const int nw = pair ? 2 : 1;
      const int lrc = (int)ring_cols(lr);   // staged row length (lr, or 64 for a shorter lr)
      for (int i = 0; i < 2; ++i) p.lbst[i] = reinterpret_cast<uint16_t*>(wsb + gw.stage_bytes + (i < nw ? i : 0) *
                                                                           stage_one(p.N, lrc));
      for (int i = 0; i < nw; ++i)
        stager.lora_b(i ? b1 : b0, ldb, r, i * r, i ? s1 : s0, p.N, lrc, const_cast<uint16_t*>(p.lbst[i]));
      p.lora_ring = lrc;
    }
    if (gw.stage) {
      for (int i = 0; i < (pair ? 2 : 1); ++i) {
        uint16_t* dst = reinterpret_cast<uint16_t*>(wsb + i * stage_one(p.N, p.K));
        stager.weight(*(i ? w1 : w0), dst);
        p.wst[i] = dst;
      }
      if (!pair) p.wst[1] = p.wst[0];
      p.ldw = p.K;
      // deq(W)^T for the input gradient, written by the GEMM from its W tiles
      if (wt && wt->out[0] && (!pair || wt->out[1]) && p.N % 8 == 0 && aligned(wt->out[0], 16) &&
          (!pair || aligned(wt->out[1], 16))) {
        p.wt_out[0] = wt->out[0];
        p.wt_out[1] = pair ? wt->out[1] : wt->out[0];
      }
    }
    stager.launch(stream);
    rc = check_launch(who);
    if (rc) return rc;
    dim3 grid((unsigned)big_tiles, (unsigned)plan.S), block(big::NT);
    KernelEvents kev(armed, stream);
    if (gw.stage) {
      if (pair) hipLaunchKernelGGL((big::fwd_kernel<true, true>), grid, block, 0, stream, p);
      else hipLaunchKernelGGL((big::fwd_kernel<false, true>), grid, block, 0, stream, p);
    } else {
      if (pair) hipLaunchKernelGGL((big::fwd_kernel<true, false>), grid, block, 0, stream, p);
      else hipLaunchKernelGGL((big::fwd_kernel<false, false>), grid, block, 0, stream, p);
    }
    kev.finish();
  } else {
    const int64_t cols_per_tile = pair ? BN / 2 : BN;
    const int64_t tiles = ceil_div64(M, BM) * ceil_div64(p.N, cols_per_tile);
    MOLT_REQUIRE(tiles < (1ll << 31), MOLT_EINVAL, "%s: problem too large", who);
    const bool small_split = plan.kind == PLAN_SMALL_SPLIT && split;
    if (small_split) {
      p.split_steps = plan.split_steps;
      p.part = static_cast<float*>(workspace);
    }
    dim3 grid((unsigned)tiles, small_split ? (unsigned)plan.S : 1u), block(NT);
    KernelEvents kev(armed, stream);
    if (pair) {
      if (al) hipLaunchKernelGGL((nf4_fwd_kernel<true, true>), grid, block, 0, stream, p);
      else hipLaunchKernelGGL((nf4_fwd_kernel<true, false>), grid, block, 0, stream, p);
    } else {
      if (al) hipLaunchKernelGGL((nf4_fwd_kernel<false, true>), grid, block, 0, stream, p);
      else hipLaunchKernelGGL((nf4_fwd_kernel<false, false>), grid, block, 0, stream, p);
    }
    kev.finish();
  }
  if (p.part) {
    rc = check_launch(who);
    if (rc) return rc;
    const int64_t q = M * (p.N / 4);
    hipLaunchKernelGGL(split_sum_kernel, dim3((unsigned)ceil_div64(q, 256)), dim3(256), 0, stream, p.part, plan.S, M,
                       p.N, y0, ldy);
  }
  rc = check_launch(who);
  if (rc == MOLT_OK && p.wt_out[0] && wt->written) *wt->written = 1;
  return rc;
}

// Y[M, N] = bf16(X . deq(W)^T + T . bf16(s B)^T) over a weight stacked from
// nw NF4 weights along the output rows, W = [W_0; W_1; ..] (N the sum of their
// rows): each is dequantised into its rows of the staged bf16 copy and one
// staged big-tile GEMM runs over the whole, so projections that share an input
// take one GEMM launch. B fp32 [N, lr] (row stride ldb) and T bf16 [M, lr] with
// lr 0 or a multiple of 64 (the LoRA steps of the DMA ring). Only the staged
// plan applies: any other is refused before a launch (MOLT_EUNSUPPORTED).
extern "C" int molt_nf4_stacked_forward_impl(const uint16_t* x, int64_t ldx, int64_t M, int32_t nw,
                                             const molt_nf4_weight* w, const uint16_t* t, int64_t ldt, int32_t lr,
                                             const float* b, int64_t ldb, float s, uint16_t* y, int64_t ldy,
                                             uint16_t* wt_out, int32_t* wt_written, void* workspace,
                                             size_t workspace_bytes, hipStream_t stream) {
  const char* who = "molt_nf4_stacked_forward";
  const GemmEvents armed;
  if (wt_written) *wt_written = 0;
  MOLT_REQUIRE(w && nw >= 1 && nw <= 8, MOLT_EINVAL, "%s: 1..8 weights", who);
  int64_t N = 0;
  for (int i = 0; i < nw; ++i) {
    const int rc = check_weight_for_gemm(&w[i], who);
    if (rc) return rc;
    MOLT_REQUIRE(w[i].cols == w[0].cols && w[i].block_size == w[0].block_size &&
                 w[i].nibble_order == w[0].nibble_order && w[i].code == w[0].code, MOLT_EINVAL,
                 "%s: stacked weights must share columns, block size, nibble order and code table", who);
    N += w[i].rows;
  }
  const int64_t K = w[0].cols;
  MOLT_REQUIRE(M >= 0 && ldx >= K && ldy >= N, MOLT_EINVAL, "%s: bad X or Y stride", who);
  MOLT_REQUIRE(lr == 0 || (lr % BK == 0 && t && b && ldt >= lr && ldb >= lr), MOLT_EINVAL,
               "%s: bad LoRA operands (lr=%d must be a multiple of %d)", who, lr, BK);
  if (M == 0) return MOLT_OK;
  MOLT_REQUIRE(x && y, MOLT_EINVAL, "%s: null X or Y", who);
  bool al = K % 64 == 0 && w[0].block_size == 64 && ldx % 8 == 0 && aligned(x, 16);
  for (int i = 0; i < nw; ++i) al = al && aligned(w[i].packed, 16);
  const GemmPlan plan = fwd_plan(M, N, K, false, fwd_big_ok(M, ldx, N, K, al), al);
  const bool t_dma = lr > 0 && aligned(t, 16) && ldt % 8 == 0;
  MOLT_REQUIRE(stage_wanted(plan.kind, M, N, K) && (lr == 0 || t_dma), MOLT_EUNSUPPORTED,
               "%s: needs the staged big-tile plan (M=%lld, N=%lld, K=%lld) and 16-byte aligned T rows", who,
               (long long)M, (long long)N, (long long)K);
  const GemmWorkspace gw = place_workspace(plan, true, 1, N, K, N, lr, M, N, workspace, workspace_bytes);
  MOLT_REQUIRE(gw.stage && (lr == 0 || gw.ring) && (plan.kind != PLAN_BIG_SPLIT || gw.split), MOLT_EWORKSPACE,
               "%s: workspace of %zu bytes (256-byte aligned) needed, got %zu", who,
               molt_nf4_lora_forward_workspace(M, N, K, lr), workspace_bytes);

  FwdParams p{};
  p.x = x; p.ldx = ldx; p.M = M; p.K = K; p.N = N;
  p.packed[0] = p.packed[1] = w[0].packed; p.scales[0] = p.scales[1] = w[0].scales;
  p.code = w[0].code; p.order = w[0].nibble_order; p.block_size = w[0].block_size;
  p.t = t; p.ldt = ldt; p.lr = lr;
  p.lb[0] = p.lb[1] = b; p.ldlb = ldb; p.r = lr; p.s[0] = p.s[1] = s;
  p.y[0] = y; p.ldy = ldy;
  p.vec_out = (ldy % 4 == 0) && aligned(y, 8);
  char* wsb = static_cast<char*>(workspace);
  if (plan.kind == PLAN_BIG_SPLIT) {
    p.split_steps = plan.split_steps;
    p.part = reinterpret_cast<float*>(wsb + gw.stage_bytes + gw.lora_bytes);
  }
  // one staging launch: each weight's bf16 rows at its place in the stack
  // (resolved scales: the flat-scale dequant) and the ring's bf16(s B) rows
  big::Stager stager;
  if (lr > 0) {
    p.lbst[0] = p.lbst[1] = reinterpret_cast<uint16_t*>(wsb + gw.stage_bytes);
    stager.lora_b(b, ldb, lr, 0, s, N, lr, const_cast<uint16_t*>(p.lbst[0]));
    p.lora_ring = lr;
  }
  int64_t row0 = 0;
  for (int i = 0; i < nw; ++i) {
    stager.weight(w[i], reinterpret_cast<uint16_t*>(wsb) + row0 * K);
    row0 += w[i].rows;
  }
  stager.launch(stream);
  int rc = check_launch(who);
  if (rc) return rc;
  p.wst[0] = p.wst[1] = reinterpret_cast<const uint16_t*>(wsb);
  p.ldw = K;
  if (wt_out && N % 8 == 0 && aligned(wt_out, 16)) p.wt_out[0] = p.wt_out[1] = wt_out;
  const int64_t big_tiles = ceil_div64(M, big::BM) * ceil_div64(N, big::BN);
  MOLT_REQUIRE(big_tiles < (1ll << 31), MOLT_EINVAL, "%s: problem too large", who);
  {
    KernelEvents kev(armed, stream);
    hipLaunchKernelGGL((big::fwd_kernel<false, true>), dim3((unsigned)big_tiles, (unsigned)plan.S), dim3(big::NT), 0,
                       stream, p);
    kev.finish();
  }
  if (p.part) {
    rc = check_launch(who);
    if (rc) return rc;
    const int64_t q = M * (N / 4);
    hipLaunchKernelGGL(split_sum_kernel, dim3((unsigned)ceil_div64(q, 256)), dim3(256), 0, stream, p.part, plan.S, M,
                       N, y, ldy);
  }
  rc = check_launch(who);
  if (rc == MOLT_OK && p.wt_out[0] && wt_written) *wt_written = 1;
  return rc;
}

extern "C" int molt_nf4_lora_backward_impl(const uint16_t* dy0, const uint16_t* dy1, int64_t lddy,
                                           int64_t M, const molt_nf4_weight* w0,
                                           const molt_nf4_weight* w1, const uint16_t* u0,
                                           const uint16_t* u1, int64_t ldu, const float* a0,
                                           const float* a1, int64_t lda, int r, float lora_scale,
                                           uint16_t* dx, int64_t lddx, const uint16_t* gate, const uint16_t* up,
                                           uint16_t* dg, uint16_t* du, int64_t ldg, const molt::WtHandoff* wt,
                                           void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const char* who = "molt_nf4_lora_backward_input";
  const GemmEvents armed;
  int rc = check_weight_for_gemm(w0, who);
  if (rc) return rc;
  const int nseg = w1 ? 2 : 1;
  if (w1) {
    rc = check_weight_for_gemm(w1, who);
    if (rc) return rc;
    MOLT_REQUIRE(same_format(w0, w1), MOLT_EINVAL, "%s: paired weights must share shape and format", who);
  }
  const bool swiglu = dg != nullptr;
  MOLT_REQUIRE(M >= 0 && lddy >= w0->rows, MOLT_EINVAL, "%s: bad dY", who);
  MOLT_REQUIRE(r == 0 || (ldu >= r && a0 && lda >= w0->cols && (nseg == 1 || a1)), MOLT_EINVAL,
               "%s: bad LoRA operands", who);
  if (swiglu) {
    MOLT_REQUIRE(ldg >= w0->cols && nseg == 1, MOLT_EINVAL, "%s: bad SwiGLU operands", who);
  } else {
    MOLT_REQUIRE(lddx >= w0->cols, MOLT_EINVAL, "%s: bad dX", who);
  }
  if (M == 0) return MOLT_OK;   // an empty token batch: no pointers are read (they may be null)
  MOLT_REQUIRE(dy0 && (nseg == 1 || dy1), MOLT_EINVAL, "%s: null gradient", who);
  MOLT_REQUIRE(r == 0 || (u0 && (nseg == 1 || u1)), MOLT_EINVAL, "%s: null LoRA gradient", who);
  MOLT_REQUIRE(swiglu ? (gate && up && du) : dx != nullptr, MOLT_EINVAL, "%s: null output", who);

  BwdParams p{};
  p.dy[0] = dy0; p.dy[1] = w1 ? dy1 : dy0; p.lddy = lddy; p.M = M;
  p.packed[0] = w0->packed; p.scales[0] = w0->scales;
  p.packed[1] = w1 ? w1->packed : w0->packed; p.scales[1] = w1 ? w1->scales : w0->scales;
  p.Nw = w0->rows; p.Kw = w0->cols;
  p.code = w0->code; p.order = w0->nibble_order; p.block_size = w0->block_size; p.nseg = nseg;
  p.u[0] = u0; p.u[1] = w1 ? u1 : u0; p.ldu = ldu; p.r = r;
  p.la[0] = a0; p.la[1] = w1 ? a1 : a0; p.ldla = lda; p.la_scale = lora_scale;
  p.dx = dx; p.lddx = lddx;
  p.gate = gate; p.up = up; p.dg = dg; p.du = du; p.ldg = ldg;
  if (swiglu)
    p.vec_out = ldg % 4 == 0 && aligned(gate, 8) && aligned(up, 8) && aligned(dg, 8) && aligned(du, 8);
  else
    p.vec_out = lddx % 4 == 0 && aligned(dx, 8);

  const bool al = (p.Nw % 64 == 0) && (p.Kw % 64 == 0) && p.block_size == 64 && lddy % 8 == 0 &&
                  aligned(dy0, 16) && (nseg == 1 || aligned(dy1, 16)) && aligned(w0->packed, 2) &&
                  (nseg == 1 || aligned(w1->packed, 2));
  const int64_t big_tiles = ceil_div64(M, big::BM) * ceil_div64(p.Kw, big::BN);
  const bool big_ok = al && aligned(w0->packed, 4) && (nseg == 1 || aligned(w1->packed, 4)) &&
                      bwd_big_ok(M, lddy, p.Nw, p.Kw, nseg);
  const GemmPlan plan = bwd_plan(M, p.Nw, p.Kw, nseg, swiglu, big_ok, al);
  const bool want_stage = stage_wanted(plan.kind, M, p.Nw, p.Kw) && p.Kw % big::BN == 0;
  // deq(W)^T of each segment handed over by the forward: read instead of staged
  const bool use_wt = want_stage && wt && wt->in[0] && (nseg == 1 || wt->in[1]) && aligned(wt->in[0], 16) &&
                      (nseg == 1 || aligned(wt->in[1], 16));
  const GemmWorkspace gw = place_workspace(plan, want_stage && !use_wt, nseg, p.Nw, p.Kw, 0, 0, M, p.Kw, workspace,
                                           workspace_bytes);
  const bool staged = gw.stage || use_wt;
  char* wsb = static_cast<char*>(workspace);
  const bool split = gw.split;
  if (wt && wt->required)
    MOLT_REQUIRE(use_wt && (plan.kind == PLAN_BIG || (plan.kind == PLAN_BIG_SPLIT && split)), MOLT_EUNSUPPORTED,
                 "%s: this input gradient reads the forward's transposed weight, which needs the staged big-tile "
                 "plan (M=%lld, N=%lld, K=%lld) and a workspace for its split", who, (long long)M,
                 (long long)p.Nw, (long long)p.Kw);
  if (plan.kind == PLAN_BIG || (plan.kind == PLAN_BIG_SPLIT && split)) {
    MOLT_REQUIRE(big_tiles < (1ll << 31), MOLT_EINVAL, "%s: problem too large", who);
    if (plan.kind == PLAN_BIG_SPLIT) {
      p.split_steps = plan.split_steps;
      p.part = reinterpret_cast<float*>(wsb + gw.stage_bytes + gw.lora_bytes);
    }
    if (use_wt) {
      p.wst[0] = wt->in[0];
      p.wst[1] = nseg == 2 ? wt->in[1] : wt->in[0];
      p.ldw = p.Nw;
    } else if (gw.stage) {
      big::StageTParams sp{};
      for (int i = 0; i < 2; ++i) {
        const molt_nf4_weight* w = (i && w1) ? w1 : w0;
        sp.packed[i] = w->packed;
        sp.scales[i] = w->scales;
        sp.wt[i] = reinterpret_cast<uint16_t*>(wsb + (i < nseg ? i : 0) * stage_one(p.Nw, p.Kw));
        p.wst[i] = sp.wt[i];
      }
      sp.code = w0->code; sp.order = w0->nibble_order;
      sp.Nw = p.Nw; sp.Kw = p.Kw; sp.ldw = p.ldw = p.Nw;
      const int64_t col_tiles = p.Kw / big::BN, row_tiles = p.Nw / 64;
      const int64_t per_col = std::max<int64_t>(1, std::min<int64_t>(row_tiles, ceil_div64(4 * molt::device_cus(),
                                                                                        col_tiles * nseg)));
      hipLaunchKernelGGL(big::stage_wt_kernel, dim3((unsigned)col_tiles, (unsigned)per_col, (unsigned)nseg),
                         dim3(big::NT), 0, stream, sp);
      rc = check_launch(who);
      if (rc) return rc;
    }
    dim3 grid((unsigned)big_tiles, (unsigned)plan.S), block(big::NT);
    KernelEvents kev(armed, stream);
    if (staged) {
      if (swiglu) hipLaunchKernelGGL((big::bwd_kernel<EPI_SWIGLU_BWD, true>), grid, block, 0, stream, p);
      else hipLaunchKernelGGL((big::bwd_kernel<EPI_STORE, true>), grid, block, 0, stream, p);
    } else {
      if (swiglu) hipLaunchKernelGGL((big::bwd_kernel<EPI_SWIGLU_BWD, false>), grid, block, 0, stream, p);
      else hipLaunchKernelGGL((big::bwd_kernel<EPI_STORE, false>), grid, block, 0, stream, p);
    }
    kev.finish();
  } else {
    const int64_t tiles = ceil_div64(M, BM) * ceil_div64(p.Kw, BN);
    MOLT_REQUIRE(tiles < (1ll << 31), MOLT_EINVAL, "%s: problem too large", who);
    const bool small_split = plan.kind == PLAN_SMALL_SPLIT && split;
    if (small_split) {
      p.split_steps = plan.split_steps;
      p.part = static_cast<float*>(workspace);
    }
    dim3 grid((unsigned)tiles, small_split ? (unsigned)plan.S : 1u), block(NT);
    KernelEvents kev(armed, stream);
    if (swiglu) {
      if (al) hipLaunchKernelGGL((nf4_bwd_kernel<EPI_SWIGLU_BWD, true>), grid, block, 0, stream, p);
      else hipLaunchKernelGGL((nf4_bwd_kernel<EPI_SWIGLU_BWD, false>), grid, block, 0, stream, p);
    } else {
      if (al) hipLaunchKernelGGL((nf4_bwd_kernel<EPI_STORE, true>), grid, block, 0, stream, p);
      else hipLaunchKernelGGL((nf4_bwd_kernel<EPI_STORE, false>), grid, block, 0, stream, p);
    }
    kev.finish();
  }
  if (p.part) {
    rc = check_launch(who);
    if (rc) return rc;
    const int64_t q = M * (p.Kw / 4);
    hipLaunchKernelGGL(split_sum_kernel, dim3((unsigned)ceil_div64(q, 256)), dim3(256), 0, stream, p.part, plan.S, M,
                       p.Kw, dx, lddx);
  }
  return check_launch(who);
}

// Workspace of molt_nf4_lora_forward / molt_nf4_lora_backward_input(_pair): the
// split-K partials when the plan for 16-byte aligned operands splits (see
// plan_splits), else 0. Calls whose operands do not qualify, or whose
// workspace is smaller, run unsplit.
// Staged weights, their LoRA copies (rank a multiple of 64) and split partials.
size_t gemm_workspace(const GemmPlan& plan, bool stage, int weights, int64_t rows, int64_t cols, int64_t lora_rows,
                      int64_t lora_cols, int64_t M, int64_t out_n) {
  size_t b = split_bytes(plan.S, M, out_n);
  if (stage) {
    b += weights * stage_one(rows, cols);
    if (ring_cols(lora_cols) > 0) b += weights * stage_one(lora_rows, ring_cols(lora_cols));
  }
  return b;
}

extern "C" size_t molt_nf4_lora_forward_workspace(int64_t M, int64_t N, int64_t K, int32_t r) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 64 != 0 || r < 0) return 0;
  const GemmPlan plan = fwd_plan(M, N, K, false, fwd_big_ok(M, K, N, K, true), true);
  return gemm_workspace(plan, stage_wanted(plan.kind, M, N, K), 1, N, K, N, r, M, N);
}

extern "C" size_t molt_nf4_gateup_forward_workspace(int64_t M, int64_t N, int64_t K, int32_t r) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 64 != 0 || r < 0) return 0;
  const GemmPlan plan = fwd_plan(M, N, K, true, fwd_big_ok(M, K, N, K, true), true);
  return gemm_workspace(plan, stage_wanted(plan.kind, M, N, K), 2, N, K, N, 2 * (int64_t)r, M, N);
}

extern "C" size_t molt_nf4_lora_backward_workspace(int64_t M, int64_t Nw, int64_t Kw, int32_t nseg) {
  if (M <= 0 || Nw <= 0 || Kw <= 0 || Nw % 64 != 0 || Kw % 64 != 0 || nseg < 1 || nseg > 2) return 0;
  const GemmPlan plan = bwd_plan(M, Nw, Kw, nseg, false, bwd_big_ok(M, Nw, Nw, Kw, nseg), true);
  const bool stage = stage_wanted(plan.kind, M, Nw, Kw) && Kw % big::BN == 0;
  return gemm_workspace(plan, stage, nseg, Nw, Kw, 0, 0, M, Kw);
}

// Workspace of the input-gradient entry points given deq(W)^T (the *_wt
// variants): only the split partials, the weights are not staged.
extern "C" size_t molt_nf4_lora_backward_workspace_wt(int64_t M, int64_t Nw, int64_t Kw, int32_t nseg) {
  if (M <= 0 || Nw <= 0 || Kw <= 0 || Nw % 64 != 0 || Kw % 64 != 0 || nseg < 1 || nseg > 2) return 0;
  const GemmPlan plan = bwd_plan(M, Nw, Kw, nseg, false, bwd_big_ok(M, Nw, Nw, Kw, nseg), true);
  return gemm_workspace(plan, false, nseg, Nw, Kw, 0, 0, M, Kw);
}

// 1 when a *_keep_wt forward of M token rows over N x K weights (16-byte
// aligned X with row stride K) writes deq(W)^T: its plan stages the weights
// and N % 8 == 0; and when the input gradient of the same weights over the
// same rows would read it (its plan stages them too).
extern "C" int32_t molt_nf4_keeps_wt(int64_t M, int64_t N, int64_t K, int32_t weights) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 64 != 0 || N % 64 != 0 || weights < 1 || weights > 2) return 0;
  const GemmPlan fp = fwd_plan(M, N, K, weights == 2, fwd_big_ok(M, K, N, K, true), true);
  const GemmPlan bp = bwd_plan(M, N, K, weights, false, bwd_big_ok(M, N, N, K, weights), true);
  return stage_wanted(fp.kind, M, N, K) && stage_wanted(bp.kind, M, N, K) && K % big::BN == 0 ? 1 : 0;
}
