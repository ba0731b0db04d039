// Skinny-M (M <= 16) NF4 GEMV with the rank-r LoRA add-on (gfx950), HBM-bound.
//
// Y[m, n] = sum_b scale(n, b) * sum_{k in block b} X[m, k] * code[W(n, k)]
//           + sum_j T[m, j] * bf16(s * B[n, j])
//
// v_mfma_f32_16x16x32_bf16 with X as the 16-row operand (rows >= M repeat
// row 0 and are never stored) and the NF4 codes as the 16-column operand.
// Lane group g = lane/16 owns the contiguous 16 elements [64b + 16g, +16) of
// block b (8 packed bytes, one 8-byte load per row), split over two 32-deep
// MFMAs, so each MFMA pair sums exactly one block and the block scale is
// applied once to its 16x16 result instead of to every weight.
//
// A workgroup (8 waves) owns 16 rows of W and all of K; its waves take
// contiguous slices of K, keep a whole chunk of blocks in flight (8 blocks
// when the u8 codes of 4 blocks can be read as one 4-byte load and share an
// absmax2 entry, else 4), and are summed in wave order through LDS, so no
// cross-workgroup reduction (and no device-scope fence) is needed. Codes come
// from an LDS table of bf16 code pairs indexed by the packed byte, replicated
// 32 times with the copy chosen by lane % 32, so the data-dependent lookups of
// a half-wave hit 32 distinct banks. The LoRA term is one more MFMA step per
// 32 ranks; its B rows are copied into LDS by direct global->LDS loads and T
// is held in registers, both issued with the first weight chunk.
#include <algorithm>
#include <mutex>

#include "common.h"

#include <stdlib.h>

namespace molt {
namespace {

constexpr int GV_WAVES = 8;
constexpr int GV_NT = 64 * GV_WAVES;
constexpr int GV_TILES = 1;              // 16-row MFMA tiles per wave
constexpr int GV_ROWS = 16 * GV_TILES;   // weight rows per workgroup
// Blocks per wave chunk (all loads of a chunk are in flight together).
template <bool Q4> constexpr int gv_u() { return Q4 ? 8 : 4; }
constexpr int GV_RMAX = 128;             // largest LoRA rank
constexpr int GV_TABW = 32;              // table copies (one per lane of a half-wave)
constexpr int GV_LT = 16 * GV_RMAX / GV_NT;   // T elements per thread

typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(1))) const void* gptr_t;
typedef __attribute__((address_space(3))) void* lptr_t;

struct GemvParams {
  const uint16_t* x; int64_t ldx; int M;
  const uint8_t* packed; int64_t N; int K;
  const float* scales;                                   // resolved, or null when nested
  const uint8_t* q; const float* absmax2; const float* code2; float offset; int dq_shift;
  const float* code; int order;
  const uint16_t* t; int64_t ldt; const float* lb; int r; float s;
  uint16_t* y; int64_t ldy;
};

// One chunk of gv_u<Q4>() blocks. Q4 (nested statistics, 4-aligned blocks): the
// u8 codes of a row's four blocks are one 4-byte load and share one absmax2
// entry; otherwise one code (or resolved scale) load per block.
template <bool Q4>
struct GvChunk {
  static constexpr int U = gv_u<Q4>();
  u32x2_t w[U][GV_TILES];
  u32x4_t xa[U], xb[U];
  uint32_t q[Q4 ? U / 4 : U][GV_TILES];
  float s[Q4 ? U / 4 : U][GV_TILES];
};

// Loads of one chunk. Every address is clamped into its tensor (past-the-end
// blocks repeat the last one and are not consumed; rows past N or M feed only
// outputs that are never stored), so no load is predicated. Offsets are 32-bit
// (a weight holds < 2^31 bytes and blocks), added to the uniform base pointers.
template <bool Q4>
MOLT_DEV void gv_load(GvChunk<Q4>& c, const GemvParams& p, const uint32_t (&wofs)[GV_TILES],
                      const uint32_t (&blk0)[GV_TILES], uint32_t xofs, int b, int b1) {
#pragma unroll
  for (int u = 0; u < gv_u<Q4>(); ++u) {
    const uint32_t bb = (uint32_t)(b + u < b1 ? b + u : b1 - 1);
    c.xa[u] = *reinterpret_cast<const u32x4_t*>(p.x + (xofs + 64u * bb));
    c.xb[u] = *reinterpret_cast<const u32x4_t*>(p.x + (xofs + 64u * bb + 8u));
#pragma unroll
    for (int t = 0; t < GV_TILES; ++t) {
      c.w[u][t] = *reinterpret_cast<const u32x2_t*>(p.packed + (wofs[t] + 32u * bb));
      const uint32_t blk = blk0[t] + bb;
      if (Q4) {
        if (u % 4 == 0) {
          // Whole 4-block units: a unit past the end repeats the last one
          // (b1 - 4 is unit-aligned), so the 4-byte code load stays inside
          // the row's codes.
          const uint32_t qblk = blk0[t] + (uint32_t)(b + u < b1 ? b + u : b1 - 4);
          c.q[u / 4][t] = *reinterpret_cast<const uint32_t*>(p.q + qblk);
          c.s[u / 4][t] = p.absmax2[qblk >> p.dq_shift];
        }
      } else if (p.scales) {
        c.s[u][t] = p.scales[blk];
      } else {
        c.q[u][t] = p.q[blk];
        c.s[u][t] = p.absmax2[blk >> p.dq_shift];
      }
    }
  }
}

MOLT_DEV float gv_scale(const GemvParams& p, const float* code2s, uint32_t q, float s) {
#pragma clang fp contract(off)
  if (p.scales) return s;
  const float prod = code2s[q & 0xffu] * s;
  return prod + p.offset;
}

struct GvSmem {
  union {
    uint32_t tab[256 * GV_TABW];                          // bf16 code pair of byte b at [b * 32 + copy]
    f32x4_t red[GV_WAVES - 1][GV_TILES][64];
  };
  float code2s[256];
  float lb[GV_ROWS * GV_RMAX];                            // raw fp32 LoRA B rows n0.., row stride r
  uint16_t lt[16 * GV_RMAX];                              // T rows 0..15, row stride r
};

// With gridDim.y > 1 (narrow outputs: few 16-row groups) K is split over
// gridDim.y workgroups per group, contiguous ranges of whole units; each writes
// its fp32 partial to `part` (slice-major) and gm_reduce_kernel sums them in
// slice order. The LoRA term belongs to slice 0.
template <bool Q4>
__global__ __launch_bounds__(GV_NT) __attribute__((amdgpu_waves_per_eu(4)))
void nf4_gemv_kernel(const GemvParams p, float* part) {
  __shared__ GvSmem sm;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t n0 = (int64_t)blockIdx.x * GV_ROWS;
  const int col = lane & 15, g = lane >> 4;
  const int KB = p.K >> 6;
  // Waves take contiguous slices of whole units (4 blocks under Q4) of this
  // workgroup's K range.
  constexpr int unit = Q4 ? 4 : 1;
  const int all_units = KB / unit, ns = (int)gridDim.y, sl = (int)blockIdx.y;
  const int u0 = sl * all_units / ns, units = (sl + 1) * all_units / ns - u0;
  const int b0 = unit * (u0 + wave * units / GV_WAVES), b1 = unit * (u0 + (wave + 1) * units / GV_WAVES);
  const int mc = col < p.M ? col : p.M - 1;
  const uint32_t xofs = (uint32_t)(mc * p.ldx + 16 * g);
  uint32_t wofs[GV_TILES], blk0[GV_TILES];
#pragma unroll
  for (int t = 0; t < GV_TILES; ++t) {
    const int64_t n = n0 + 16 * t + col;
    const int64_t nc = n < p.N ? n : p.N - 1;
    wofs[t] = (uint32_t)(nc * (p.K >> 1) + 8 * g);
    blk0[t] = (uint32_t)(nc * KB);
  }

  // Issue order: the codebooks (tiny, L2-resident), the first weight chunk,
  // then the LoRA operands straight into LDS. Nothing waits until all of
  // them are in flight.
  // The codebook is read through the constant address space (scalar loads
  // into SGPRs: one copy per wave instead of per lane).
  typedef __attribute__((address_space(4))) const f32x4_t* cptr_t;
  const cptr_t cbp = (cptr_t)p.code;
  const f32x4_t cb0 = cbp[0], cb1 = cbp[1], cb2 = cbp[2], cb3 = cbp[3];
  const float c2 = (p.code2 ? p.code2 : p.code)[p.code2 ? (tid & 255) : 0];
  GvChunk<Q4> c;
  if (b0 < b1) gv_load<Q4>(c, p, wofs, blk0, xofs, b0, b1);
  const bool lora = p.r > 0 && sl == 0;
  if (lora) {
    // B rows n0 .. n0+63 are contiguous (row stride r): 4-byte copies.
    const int nb = GV_ROWS * p.r;
    const int64_t bmax = p.N * p.r - 1;
    for (int base = wave * 64; base < nb; base += GV_NT) {
      int64_t e = n0 * p.r + base + lane;
      e = e < bmax ? e : bmax;
      __builtin_amdgcn_global_load_lds((gptr_t)(p.lb + e), (lptr_t)(sm.lb + base), 4, 0, 0);
    }
  }
  // T rows 0 .. 15 (rows >= M repeat row 0) into registers; stored below.
  uint32_t traw[GV_LT];
#pragma unroll
  for (int k = 0; k < GV_LT; ++k) {
    traw[k] = 0;
    if (lora) {
      int i = tid + k * GV_NT;
      i = i < 16 * p.r ? i : 0;
      const int m = i / p.r, j = i - m * p.r;
      traw[k] = p.t[(int64_t)(m < p.M ? m : 0) * p.ldt + j];
    }
  }

  // Replicated code-pair table: this thread writes byte values b with low
  // nibble tid / 32 (copy tid % 32) for every high nibble.
  {
    const float cv[16] = {cb0[0], cb0[1], cb0[2], cb0[3], cb1[0], cb1[1], cb1[2], cb1[3],
                          cb2[0], cb2[1], cb2[2], cb2[3], cb3[0], cb3[1], cb3[2], cb3[3]};
    const int lo = tid >> 5, copy = tid & 31;
    float clo = cv[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) clo = lo == i ? cv[i] : clo;
#pragma unroll
    for (int hi = 0; hi < 16; ++hi) {
      const float first = p.order ? cv[hi] : clo, second = p.order ? clo : cv[hi];
      sm.tab[(hi * 16 + lo) * GV_TABW + copy] = pack_bf16x2(first, second);
    }
    if (tid < 256) sm.code2s[tid] = c2;
  }
  if (lora) {
#pragma unroll
    for (int k = 0; k < GV_LT; ++k) {
      const int i = tid + k * GV_NT;
      if (i < 16 * p.r) sm.lt[i] = (uint16_t)traw[k];
    }
  }
  __syncthreads();

  const uint32_t* tab = sm.tab + (lane & 31);
  f32x4_t acc[GV_TILES];
#pragma unroll
  for (int t = 0; t < GV_TILES; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int b = b0; b < b1;) {
#pragma unroll
    for (int u = 0; u < gv_u<Q4>(); ++u) {
      if (b + u >= b1) break;
      const bf16x8v xa = __builtin_bit_cast(bf16x8v, c.xa[u]);
      const bf16x8v xb = __builtin_bit_cast(bf16x8v, c.xb[u]);
#pragma unroll
      for (int t = 0; t < GV_TILES; ++t) {
        u32x4_t w0, w1;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          w0[j] = tab[((c.w[u][t][0] >> (8 * j)) & 0xffu) * GV_TABW];
          w1[j] = tab[((c.w[u][t][1] >> (8 * j)) & 0xffu) * GV_TABW];
        }
        f32x4_t tmp = {0.f, 0.f, 0.f, 0.f};
        tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa, __builtin_bit_cast(bf16x8v, w0), tmp, 0, 0, 0);
        tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xb, __builtin_bit_cast(bf16x8v, w1), tmp, 0, 0, 0);
        const float sc = Q4 ? gv_scale(p, sm.code2s, c.q[u / 4][t] >> (8 * (u % 4)), c.s[u / 4][t])
                            : gv_scale(p, sm.code2s, c.q[u][t], c.s[u][t]);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[t][e] += sc * tmp[e];
      }
    }
    b += gv_u<Q4>();
    if (b < b1) gv_load<Q4>(c, p, wofs, blk0, xofs, b, b1);
  }

  __syncthreads();                       // the table area becomes the reduction area
  if (wave > 0) {
#pragma unroll
    for (int t = 0; t < GV_TILES; ++t) sm.red[wave - 1][t][lane] = acc[t];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < GV_WAVES - 1; ++w)
#pragma unroll
    for (int t = 0; t < GV_TILES; ++t) acc[t] += sm.red[w][t][lane];

  if (lora) {
    // acc += T . bf16(s B)^T, 32 ranks per MFMA step (ranks past r are zero).
    for (int j0 = 0; j0 < p.r; j0 += 32) {
      u32x4_t ta;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int j = j0 + 8 * g + 2 * e;
        const uint32_t lo = j < p.r ? sm.lt[col * p.r + j] : 0u;
        const uint32_t hi = j + 1 < p.r ? sm.lt[col * p.r + j + 1] : 0u;
        ta[e] = lo | (hi << 16);
      }
#pragma unroll
      for (int t = 0; t < GV_TILES; ++t) {
        const float* brow = sm.lb + (16 * t + col) * p.r;
        u32x4_t bw;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = j0 + 8 * g + 2 * e;
          const float lo = j < p.r ? round_bf16(p.s * brow[j]) : 0.0f;
          const float hi = j + 1 < p.r ? round_bf16(p.s * brow[j + 1]) : 0.0f;
          bw[e] = pack_bf16x2(lo, hi);
        }
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8v, ta),
                                                         __builtin_bit_cast(bf16x8v, bw), acc[t], 0, 0, 0);
      }
    }
  }

  // acc[t][e] is C[m][n] with m = 4 (lane / 16) + e, n = n0 + 16 t + lane % 16.
#pragma unroll
  for (int t = 0; t < GV_TILES; ++t) {
    const int64_t n = n0 + 16 * t + col;
    if (n >= p.N) continue;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = 4 * g + e;
      if (m >= p.M) continue;
      if (ns == 1) p.y[(int64_t)m * p.ldy + n] = bf16_bits(acc[t][e]);
      else part[((int64_t)sl * p.M + m) * p.N + n] = acc[t][e];
    }
  }
}


// ---------------------------------------------------------------------------
// Streaming dot-product variant for M <= 4 (decode). Each wave walks rows of W
// in rounds: round j covers RW rows at j * (grid waves * RW) + (this wave's
// index) * RW, so every round of the grid reads a contiguous band of W. A
// lane reads 16 contiguous packed bytes (32 elements, half a block) of each
// 1 KB piece of a row, so each load instruction is 1 KB of one row. The loads
// of a round (weight pieces, block statistics, LoRA B entries) are issued two
// rounds ahead into three rotating register sets, so the dot-product work of
// round j overlaps the HBM stream of rounds j + 1 and j + 2. Codes come from
// the replicated LDS table of bf16 code pairs and meet X (staged once per
// workgroup in LDS) through v_dot2_f32_bf16; the block scale multiplies each
// lane's half-block sum, lane j < r adds T[j] bf16(s B[n, j]), and the 64
// lanes of a row are summed by DPP row reductions and scalar reads. MX rows of X (the tokens,
// M <= MX; rows past M repeat row M - 1 and are not stored) share each code
// lookup, one dot2 per token. K is any multiple of 64 up to 7 x 2048: the last
// piece of a row may be partial (its lanes past the row end are masked).
constexpr int GD_WAVES = 8;
constexpr int GD_NT = 64 * GD_WAVES;
constexpr int GD_XPAD = 8;                // bf16 elements of X row padding

// Code-pair table of the dot kernel: entry (byte b, copy c) at b * TS + c.
// With TS = 64 (256 bytes per entry, copies in the first 128) a lane's
// lookup address is one v_perm_b32 of the packed dword: the byte lands in
// bits 8-15 beside the lane's copy offset (lane % 32) * 4 in bits 0-7, where
// the 32-dword stride takes a bit-field extract and a shift-add per byte.
// It doubles the table's footprint (64 KB), so it is used where the LDS
// allows (see gd_perm).
template <int TS>
struct GdSmem {
  uint32_t tab[256 * TS];
  float code2s[256];
};
template <int IPR, int MX>
constexpr bool gd_perm() { return IPR == 2 ? MX == 1 : MX <= 2; }

typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));

template <int RW, int IPR>
struct GdRound {
  u32x4_t w[RW * IPR];
  uint32_t q[RW * IPR];
  float s[RW * IPR];
  float lb[RW][2];
};

// Loads of one round (rows n0 .. n0 + RW - 1, clamped to the matrix). Every
// load is unconditional (statistics layout and LoRA presence are template
// parameters, out-of-range indices are clamped and their values masked), so
// each round issues the same fixed number of loads and the compiler's vmcnt
// wait before a round's arithmetic counts exactly the two later rounds as
// still in flight; a load under a run-time branch made it wait for those too.
// Rows past the matrix read row `fallback` instead (the wave's own first row,
// already on its way to the cache; one shared row would be a hot spot).
template <int RW, int IPR, bool NESTED, bool LORA, bool FULL>
MOLT_DEV void gd_load(GdRound<RW, IPR>& R, const GemvParams& p, int64_t n0, int lane, int KB, int64_t fallback) {
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int64_t n = n0 + r < p.N ? n0 + r : fallback;
#pragma unroll
    for (int i = 0; i < IPR; ++i) {
      const int j = r * IPR + i;
      // the last piece may end inside the row: its lanes past the end re-read
      // the row's last 16 bytes and block (their products are dropped)
      const int wo = FULL || i + 1 < IPR ? 1024 * i + 16 * lane : min(1024 * i + 16 * lane, (p.K >> 1) - 16);
      const int bo = FULL || i + 1 < IPR ? 32 * i + (lane >> 1) : min(32 * i + (lane >> 1), KB - 1);
      R.w[j] = *reinterpret_cast<const u32x4_t*>(p.packed + (uint32_t)(n * (p.K >> 1) + wo));
      const uint32_t blk = (uint32_t)(n * KB + bo);
      if constexpr (NESTED) {
        R.q[j] = p.q[blk];
        R.s[j] = p.absmax2[blk >> p.dq_shift];
      } else {
        R.q[j] = 0;
        R.s[j] = p.scales[blk];
      }
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int jr = lane + 64 * q;
      if constexpr (LORA) {
        const float v = p.lb[n * p.r + (jr < p.r ? jr : p.r - 1)];
        R.lb[r][q] = jr < p.r ? v : 0.0f;
      } else {
        R.lb[r][q] = 0.0f;
      }
    }
  }
}

// Sum over the 64 lanes of a wave with no LDS traffic (a shuffle becomes an
// LDS permute whose wait also drains the round's outstanding table lookups):
// DPP within each row of 16 lanes (swap neighbours, swap pairs, half-row
// mirror, row mirror), then the four row sums read into scalars and added in
// row order. The result is wave-uniform.
MOLT_DEV float gd_wave_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
  const int iv = __builtin_bit_cast(int, v);
  return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 16))) +
         (__builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 32)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 48)));
}

// Dot products of one round; returns the value lane r * MX + m stores (row r
// of token m, see gd_store). X row m sits at
// xs + m * xstride (elements); with XREG (one token) the lane's X chunks are
// xg[4 i + h] in registers instead.
template <int RW, int IPR, int MX, bool XREG, bool PERM, bool FULL>
MOLT_DEV float gd_compute(const GdRound<RW, IPR>& R, const GemvParams& p, const uint32_t* tab, const uint16_t* xs,
                         int xstride, const u32x4_t* xg, const float* code2s, const float (&lt)[MX][2], int64_t n0,
                         int lane) {
  const uint32_t lb = (uint32_t)(lane & 31) * 4;     // PERM: byte offset of the lane's copy
  float acc[RW][MX];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int m = 0; m < MX; ++m) acc[r][m] = 0.0f;
#pragma unroll
  for (int i = 0; i < IPR; ++i) {                                      // piece i of every row: X read once
    float bs[RW][MX];
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
      for (int m = 0; m < MX; ++m) bs[r][m] = 0.0f;
#pragma unroll
    for (int h = 0; h < 4; ++h) {                                      // 4 bytes per dword, 8 elements
      u32x4_t xv[MX];
#pragma unroll
      for (int m = 0; m < MX; ++m)
        xv[m] = XREG ? xg[4 * i + h] : *reinterpret_cast<const u32x4_t*>(xs + m * xstride + 8 * (256 * i + 64 * h + lane));
#pragma unroll
      for (int b = 0; b < 4; ++b) {
#pragma unroll
        for (int r = 0; r < RW; ++r) {
          uint32_t pair;
          if constexpr (PERM) {
            // bits 15:8 = byte b of the dword, bits 7:0 = lb: selectors 4 + b (S0), 0 (S1), 12 (zero)
            const uint32_t off = __builtin_amdgcn_perm(R.w[r * IPR + i][h], lb, 0x0C0C0400u | ((uint32_t)b << 8));
            pair = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(tab) + off);
          } else {
            pair = tab[((R.w[r * IPR + i][h] >> (8 * b)) & 0xffu) * GV_TABW];
          }
#pragma unroll
          for (int m = 0; m < MX; ++m) {
            // copy the element out first: __builtin_bit_cast of a vector-element
            // lvalue reads element 0 with this compiler
            const uint32_t xw = xv[m][b];
            bs[r][m] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, pair),
                                                       __builtin_bit_cast(bf16x2v, xw), bs[r][m], false);
          }
        }
      }
    }
    // lanes past the end of a row in its last piece contribute nothing
    const bool live = FULL || i + 1 < IPR || 1024 * i + 16 * lane < (p.K >> 1);
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const float sc = gv_scale(p, code2s, R.q[r * IPR + i], R.s[r * IPR + i]);
#pragma unroll
      for (int m = 0; m < MX; ++m) {
        acc[r][m] += live ? sc * bs[r][m] : 0.0f;
        asm volatile("" : "+v"(acc[r][m]));                           // keeps each piece's lookups short-lived
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  // LoRA partials join the row sums; sum over the wave (gd_wave_sum); lane
  // r * MX + m stores row r of token m
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const float b0 = round_bf16(p.s * R.lb[r][0]), b1 = round_bf16(p.s * R.lb[r][1]);
#pragma unroll
    for (int m = 0; m < MX; ++m) acc[r][m] = gd_wave_sum(acc[r][m] + (lt[m][0] * b0 + lt[m][1] * b1));
  }
  float v = acc[0][0];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int m = 0; m < MX; ++m) v = lane == r * MX + m ? acc[r][m] : v;
  return v;
}

// Store of one round's results: lane r * MX + m holds row n0 + r of token m.
template <int RW, int MX>
MOLT_DEV void gd_store(const GemvParams& p, float v, int64_t n0, int lane) {
  if (lane < RW * MX) {
    const int rr = lane / MX, m = lane % MX;
    const int64_t n = n0 + rr;
    if (n < p.N && m < p.M) p.y[(int64_t)m * p.ldy + n] = bf16_bits(v);
  }
}

// At K = 4096 with up to two X rows the kernel is held to 128 registers, so two
// workgroups fit on a CU.
//
// MAXR > 0: at most MAXR rounds per wave, all issued up front in straight-line
// code (rounds past `rounds` load the clamped last row and are not computed),
// each round's arithmetic starting as soon as its own loads have landed, and
// every store after the last round: with no branch between a load and its use
// the compiler's waits count exactly the later loads still in flight. MAXR = 0:
// any number of rounds, loaded two ahead in three rotating register sets.
template <int RW, int IPR, int MX, bool NESTED, bool LORA, int MAXR, bool FULL>
__global__ __launch_bounds__(GD_NT) __attribute__((amdgpu_waves_per_eu(IPR <= 2 && MX <= 2 ? 4 : 1)))
void nf4_gemv_dot_kernel(const GemvParams p, int rounds) {
  constexpr bool PERM = gd_perm<IPR, MX>();
  constexpr int TS = PERM ? 64 : GV_TABW;
  __shared__ GdSmem<TS> sm;
  extern __shared__ __attribute__((aligned(16))) uint16_t gd_xs[];      // X, MX rows of K + GD_XPAD elements
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t stride = (int64_t)gridDim.x * GD_WAVES * RW;          // rows per round of the grid
  const int64_t nb = ((int64_t)blockIdx.x * GD_WAVES + wave) * RW;    // first row of round 0
  const int KB = p.K >> 6;

  typedef __attribute__((address_space(4))) const f32x4_t* cptr_t;
  const cptr_t cbp = (cptr_t)p.code;
  const f32x4_t cb0 = cbp[0], cb1 = cbp[1], cb2 = cbp[2], cb3 = cbp[3];

  // X first (16-byte chunks into registers), so that the wait before its LDS
  // stores, and the barrier after them, do not wait for the weight stream.
  // One token at K = 4096: the lane's 64 elements of X (16-byte chunks
  // 256 i + 4 lane + h, the elements its weight bytes multiply) stay in
  // registers, read straight from memory; otherwise X is staged in LDS. (At
  // K = 14336 with two rounds per wave the 112 registers fit, but the decode
  // measured slower: 11.3 -> 12.5 us at 4096 x 14336.)
  constexpr bool XREG = IPR == 2 && MX == 1;
  constexpr int XCH = IPR * 256, XIT = XREG ? 0 : (MX * XCH + GD_NT - 1) / GD_NT;   // 16-byte chunks of X
  // X rows in LDS take whole pieces (IPR x 2048 elements); chunks past the end
  // of a row (a partial last piece) re-read its last chunk, whose products
  // the compute drops
  const int xstride = IPR * 2048 + GD_XPAD;
  const int xlast = (p.K >> 3) - 1;                                   // last 16-byte chunk of a row
  u32x4_t xr[XIT > 0 ? XIT : 1];
  u32x4_t xg[XREG ? 4 * IPR : 1];
  if constexpr (XREG) {
#pragma unroll
    for (int c = 0; c < 4 * IPR; ++c)
      xg[c] = *reinterpret_cast<const u32x4_t*>(p.x + 8 * min(256 * (c >> 2) + 4 * lane + (c & 3), xlast));
  }
#pragma unroll
  for (int it = 0; it < XIT; ++it) {
    const int c = tid + it * GD_NT < MX * XCH ? tid + it * GD_NT : MX * XCH - 1;
    const int m = c / XCH < p.M ? c / XCH : p.M - 1;
    xr[it] = *reinterpret_cast<const u32x4_t*>(p.x + m * p.ldx + 8 * min(c % XCH, xlast));
  }
  // unconditional loads here too (clamped, then masked): see gd_load
  float c2 = 0.0f;
  if constexpr (NESTED) c2 = p.code2[tid & 255];
  float lt[MX][2];
#pragma unroll
  for (int m = 0; m < MX; ++m) {
    const int mm = m < p.M ? m : p.M - 1;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int jr = lane + 64 * q;
      lt[m][q] = 0.0f;
      if constexpr (LORA) {
        const float v = bf16_to_f32(p.t[mm * p.ldt + (jr < p.r ? jr : p.r - 1)]);
        lt[m][q] = jr < p.r ? v : 0.0f;
      }
    }
  }

  // The small loads above (X, the nested code table, T) are issued before any
  // weight load and must stay there: a wait for one of them placed after the
  // weight loads would wait for the whole weight stream too.
  __builtin_amdgcn_sched_barrier(0);
  constexpr int NB = MAXR > 0 ? MAXR : 3;
  const int64_t nf = nb < p.N ? nb : p.N - 1;
  GdRound<RW, IPR> b[NB];
  gd_load<RW, IPR, NESTED, LORA, FULL>(b[0], p, nb, lane, KB, nf);
#pragma unroll
  for (int j = 1; j < (MAXR > 0 ? MAXR : 2); ++j) gd_load<RW, IPR, NESTED, LORA, FULL>(b[j], p, nb + j * stride, lane, KB, nf);

  // X in LDS by (piece, dword, lane): 16-byte chunk c = 256 i + 4 l + h (elements
  // 2048 i + 32 l + 8 h ..) sits at 256 i + 64 h + l, so the reads of a piece's
  // dword h by the 64 lanes are 1 KB contiguous (bank-conflict free).
#pragma unroll
  for (int it = 0; it < XIT; ++it) {
    const int c = tid + it * GD_NT;
    const int m = c / XCH, cc = c % XCH;
    if (c < MX * XCH)
      *reinterpret_cast<u32x4_t*>(gd_xs + m * xstride + 8 * ((cc & ~255) | ((cc & 3) << 6) | ((cc >> 2) & 63))) =
          xr[it];
  }
  {
    const float cv[16] = {cb0[0], cb0[1], cb0[2], cb0[3], cb1[0], cb1[1], cb1[2], cb1[3],
                          cb2[0], cb2[1], cb2[2], cb2[3], cb3[0], cb3[1], cb3[2], cb3[3]};
    static_assert(GV_TABW == 32 && GD_NT % 512 == 0 && GD_NT <= 8192, "table build covers 256 x 32 entries");
    constexpr int HS = GD_NT / 512;                                    // high nibbles per pass
    const int lo = (tid >> 5) & 15, copy = tid & 31, h0 = tid >> 9;
    float clo = cv[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) clo = lo == i ? cv[i] : clo;
#pragma unroll
    for (int k = 0; k < 16 / HS; ++k) {
      const int hi = h0 + HS * k;
      float chi = cv[0];
#pragma unroll
      for (int i = 1; i < 16; ++i) chi = hi == i ? cv[i] : chi;
      const float first = p.order ? chi : clo, second = p.order ? clo : chi;
      sm.tab[(hi * 16 + lo) * TS + copy] = pack_bf16x2(first, second);
    }
    sm.code2s[tid & 255] = c2;                       // every thread: no branch around the load
  }
  __syncthreads();

  const uint32_t* tab = PERM ? sm.tab : sm.tab + (lane & 31);
  if constexpr (MAXR > 0) {
    float out[MAXR];
#pragma unroll
    for (int j = 0; j < MAXR; ++j)
      out[j] = gd_compute<RW, IPR, MX, XREG, PERM, FULL>(b[j], p, tab, gd_xs, xstride, xg, sm.code2s, lt, nb + j * stride, lane);
#pragma unroll
    for (int j = 0; j < MAXR; ++j)
      if (j < rounds) gd_store<RW, MX>(p, out[j], nb + j * stride, lane);
  } else {
    // Rounds past the last one load the (clamped) last row again and are never
    // computed: unconditional loads keep the waits exact (see gd_load).
    for (int j = 0; j < rounds; j += 3) {
      gd_load<RW, IPR, NESTED, LORA, FULL>(b[2], p, nb + (j + 2) * stride, lane, KB, nf);
      gd_store<RW, MX>(p, gd_compute<RW, IPR, MX, XREG, PERM, FULL>(b[0], p, tab, gd_xs, xstride, xg, sm.code2s, lt,
                                                          nb + j * stride, lane), nb + j * stride, lane);
      if (j + 1 >= rounds) break;
      gd_load<RW, IPR, NESTED, LORA, FULL>(b[0], p, nb + (j + 3) * stride, lane, KB, nf);
      gd_store<RW, MX>(p, gd_compute<RW, IPR, MX, XREG, PERM, FULL>(b[1], p, tab, gd_xs, xstride, xg, sm.code2s, lt,
                                                          nb + (j + 1) * stride, lane), nb + (j + 1) * stride, lane);
      if (j + 2 >= rounds) break;
      gd_load<RW, IPR, NESTED, LORA, FULL>(b[1], p, nb + (j + 4) * stride, lane, KB, nf);
      gd_store<RW, MX>(p, gd_compute<RW, IPR, MX, XREG, PERM, FULL>(b[2], p, tab, gd_xs, xstride, xg, sm.code2s, lt,
                                                          nb + (j + 2) * stride, lane), nb + (j + 2) * stride, lane);
    }
  }
}

// ---------------------------------------------------------------------------
// Streaming MFMA variant for 2 <= M <= 16 and K a multiple of 3584 or 4096.
// A workgroup walks 16-row groups of W (group blockIdx.x + j * gridDim.x in
// round j) over one K slice of NW * 512 elements (slice blockIdx.y); its
// first NW waves split the slice, wave w owning blocks 8w .. 8w + 7 of the
// slice in every row, so each wave's X fragments (16 rows of X, 128 bytes
// per lane) are loaded once and stay in registers. With one slice the
// outputs are stored as bf16; with several (K = 14336: four slices of 3584)
// each slice writes fp32 partials that gm_reduce_kernel sums in slice order.
// A round's loads (16 bytes per lane per pair of blocks, the block
// statistics, the LoRA B entries of the wave's rank chunk) are issued two
// rounds ahead into three rotating register sets (with one round per
// workgroup, ONE, only that round is loaded). Per block, two
// v_mfma_f32_16x16x32_bf16 over bf16 code pairs from the replicated LDS table
// give the block's partial products, scaled by the block scale in fp32 (as in
// nf4_gemv_kernel); the 8 waves' 16 x 16 partials are summed through a
// double-buffered LDS area, one barrier per round.
constexpr int GM_WAVES = 8;
constexpr int GM_NT = 64 * GM_WAVES;

// mode 0: resolved fp32 scales; 1: nested, one u8 code per block; 2: nested,
// the codes of 4 blocks in one 4-byte load sharing one absmax2 entry.
// LV: 0 no LoRA; 1 LoRA B rows read as 16-byte vectors (r % 4 == 0, 16-byte
// aligned); 2 LoRA B rows read one float at a time.
template <int SM, int LV>
struct GmRound {
  static constexpr int NS = SM == 2 ? 2 : 8;
  static constexpr int NL = LV == 0 ? 1 : 8;
  u32x4_t w[4];                                           // blocks 2i, 2i + 1: see gm_load
  uint32_t q[NS];
  float s[NS];
  float lb[NL];
};

// Code-pair table at a 256-byte entry stride (see GdSmem): a lookup address is
// one v_perm_b32 of the packed dword.
struct GmSmem {
  uint32_t tab[256 * 64];
  float code2s[256];
  f32x4_t red[2][GM_WAVES][64];
};

// Loads of one round: 16-row group `grp` (clamped to the last group by the
// caller, so every address is in bounds) over the wave's 512 elements at kw.
// Every load is unconditional, so each round issues the same fixed number of
// loads and the compiler's vmcnt wait before a round's arithmetic counts the
// two later rounds as still in flight (a load under a branch made it wait for
// them too). The LoRA B entries of rank chunk jc (8 ranks per lane group g)
// are clamped into the row; the T fragment is zero for the ranks past r.
template <int SM, int LV>
MOLT_DEV void gm_load(GmRound<SM, LV>& R, const GemvParams& p, int64_t grp, int kw, int col, int g, int jc) {
  const int64_t n = 16 * grp + col < p.N ? 16 * grp + col : p.N - 1;
  const uint32_t blk0 = (uint32_t)(n * (p.K >> 6) + (kw >> 6));
  // 16 bytes per lane: lane groups g = 0, 1 read bytes 16 g .. 16 g + 15 of
  // block 2i, groups 2, 3 bytes 16 (g - 2) .. of block 2i + 1, so one load
  // instruction covers 64 contiguous bytes of each of its 16 rows
  const uint32_t wofs = (uint32_t)(n * (p.K >> 1) + (kw >> 1) + 16 * g);
#pragma unroll
  for (int i = 0; i < 4; ++i) R.w[i] = *reinterpret_cast<const u32x4_t*>(p.packed + wofs + 64u * i);
  if constexpr (SM == 2) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      R.q[u] = *reinterpret_cast<const uint32_t*>(p.q + blk0 + 4 * u);
      R.s[u] = p.absmax2[(blk0 + 4 * u) >> p.dq_shift];
    }
  } else {
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      if constexpr (SM == 0) {
        R.q[b] = 0;
        R.s[b] = p.scales[blk0 + b];
      } else {
        R.q[b] = p.q[blk0 + b];
        R.s[b] = p.absmax2[(blk0 + b) >> p.dq_shift];
      }
    }
  }
  const int j = jc + 8 * g;                                            // first rank of the lane's 8
  if constexpr (LV == 1) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int jj = j + 4 * h;
      const f32x4_t v = *reinterpret_cast<const f32x4_t*>(p.lb + n * p.r + (jj < p.r ? jj : p.r - 4));
#pragma unroll
      for (int e = 0; e < 4; ++e) R.lb[4 * h + e] = v[e];
    }
  } else if constexpr (LV == 2) {
#pragma unroll
    for (int e = 0; e < 8; ++e) R.lb[e] = p.lb[n * p.r + (j + e < p.r ? j + e : p.r - 1)];
  }
}

// Block scale: the resolved fp32 scale, or code2[u8 code] * absmax2 + offset
// (the nested statistics, as gv_scale computes them).
template <int SM>
MOLT_DEV float gm_scale(const GemvParams& p, const float* code2s, uint32_t q, float s) {
#pragma clang fp contract(off)
  if constexpr (SM == 0) {
    return s;
  } else {
    const float prod = code2s[q & 0xffu] * s;
    return prod + p.offset;
  }
}

// One round of one wave: 8 blocks of 64 elements of 16 rows. Each block's two
// MFMAs go to an accumulator of their own and the block scales are applied
// after all 16 MFMAs, so no MFMA result is waited for inside the loop; the sum
// over blocks runs in block order (acc += scale * block partial).
template <int SM, int LV>
MOLT_DEV f32x4_t gm_compute(const GmRound<SM, LV>& R, const GemvParams& p, const char* tab, uint32_t lb,
                            const float* code2s, const u32x4_t (&xf)[8][2], const u32x4_t& tf) {
  float sc[8];
#pragma unroll
  for (int b = 0; b < 8; ++b)
    sc[b] = SM == 2 ? gm_scale<SM>(p, code2s, R.q[b / 4] >> (8 * (b % 4)), R.s[b / 4])
                    : gm_scale<SM>(p, code2s, R.q[b % GmRound<SM, LV>::NS], R.s[b % GmRound<SM, LV>::NS]);
  // Each lane holds 16 bytes of block 2i (lane groups 0, 1) or 2i + 1 (groups
  // 2, 3). Swapping dwords 2, 3 of the lower 32 lanes with dwords 0, 1 of the
  // upper 32 (v_permlane32_swap) leaves every lane two dwords of each block:
  // dword t of block 2i + e sits in wd[i][2 e + t], and in lane group g it holds
  // the block's elements 16 gk(g) + 8 t .. + 7, gk = {0, 2, 1, 3}[g] (the X
  // fragments follow the same order), so both MFMAs of a block sum only that
  // block.
  u32x4_t wd[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const auto s02 = __builtin_amdgcn_permlane32_swap(R.w[i][0], R.w[i][2], false, false);
    const auto s13 = __builtin_amdgcn_permlane32_swap(R.w[i][1], R.w[i][3], false, false);
    wd[i][0] = s02[0]; wd[i][2] = s02[1]; wd[i][1] = s13[0]; wd[i][3] = s13[1];
  }
  // The lookups of block b + 1 are issued before the MFMAs of block b (the
  // scheduling barriers keep that order), so each block's LDS latency hides
  // behind the previous block's MFMAs.
  u32x4_t wl[2][2];
  auto look = [&](int b, u32x4_t (&w)[2]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // bits 15:8 = byte j of the dword, bits 7:0 = the lane's copy offset
      const uint32_t sel = 0x0C0C0400u | ((uint32_t)j << 8);
      w[0][j] = *reinterpret_cast<const uint32_t*>(tab + __builtin_amdgcn_perm(wd[b >> 1][2 * (b & 1)], lb, sel));
      w[1][j] = *reinterpret_cast<const uint32_t*>(tab + __builtin_amdgcn_perm(wd[b >> 1][2 * (b & 1) + 1], lb, sel));
    }
  };
  f32x4_t tmp[8];
  look(0, wl[0]);
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    if (b + 1 < 8) look(b + 1, wl[(b + 1) & 1]);
    __builtin_amdgcn_sched_barrier(0);
    const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
    tmp[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8v, xf[b][0]),
                                                     __builtin_bit_cast(bf16x8v, wl[b & 1][0]), zero, 0, 0, 0);
    tmp[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8v, xf[b][1]),
                                                     __builtin_bit_cast(bf16x8v, wl[b & 1][1]), tmp[b], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  }
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int b = 0; b < 8; ++b)
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] += sc[b] * tmp[b][e];
  if constexpr (LV != 0) {
    // every wave runs the LoRA step, so each round consumes its B loads (a
    // load whose value one path never reads made the compiler wait for the
    // whole stream at the loop head). T is zero for the ranks past r and on
    // waves holding no rank of slice 0, so the clamped B entries there (finite
    // entries of the same row) add nothing; B itself is not masked, which would
    // place a wait right after its load.
    u32x4_t bw;
#pragma unroll
    for (int e = 0; e < 4; ++e) bw[e] = pack_bf16x2(p.s * R.lb[2 * e], p.s * R.lb[2 * e + 1]);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8v, tf), __builtin_bit_cast(bf16x8v, bw),
                                                  acc, 0, 0, 0);
  }
  return acc;
}

template <int SM, int NW, int LV, bool ONE>
__global__ __launch_bounds__(GM_NT) void nf4_gemv_ms_kernel(const GemvParams p, int rounds, float* part) {
  static_assert(NW >= 3 && NW <= GM_WAVES, "K slice of NW x 512 elements");
  __shared__ GmSmem sm;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, g = lane >> 4;
  const bool active = NW == GM_WAVES || wave < NW;                     // waves >= NW only help reduce
  // the wave's K range (a wave past NW loads wave 0's range and discards it)
  const int kw = (int)blockIdx.y * NW * 512 + 512 * (active ? wave : 0);
  const int jc = 32 * (active ? wave : 0);                             // the wave's LoRA rank chunk
  const bool lora = LV != 0 && active && blockIdx.y == 0 && jc < p.r;  // slice 0 only

  typedef __attribute__((address_space(4))) const f32x4_t* cptr_t;
  const cptr_t cbp = (cptr_t)p.code;
  const f32x4_t cb0 = cbp[0], cb1 = cbp[1], cb2 = cbp[2], cb3 = cbp[3];
  float c2 = 0.0f;
  if constexpr (SM != 0) c2 = p.code2[tid & 255];

  // X fragments of the wave's K slice (rows >= M repeat row M - 1; their
  // outputs are never stored) and the wave's T fragment (ranks past r: 0).
  const int mc = col < p.M ? col : p.M - 1;
  u32x4_t xf[8][2];
  {
    const uint16_t* xr = p.x + (int64_t)mc * p.ldx + kw + 32 * (g & 1) + 16 * (g >> 1);
#pragma unroll
    for (int b = 0; b < 8; ++b)
#pragma unroll
      for (int h = 0; h < 2; ++h) xf[b][h] = *reinterpret_cast<const u32x4_t*>(xr + 64 * b + 8 * h);   // see gm_compute
  }
  u32x4_t tf = {0u, 0u, 0u, 0u};
  if constexpr (LV != 0) {
    uint16_t e[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int j = jc + 8 * g + i;
      const uint16_t v = p.t[(int64_t)mc * p.ldt + (j < p.r ? j : p.r - 1)];
      e[i] = lora && j < p.r ? v : (uint16_t)0;
    }
    tf = __builtin_bit_cast(u32x4_t, e);
  }
  // the small loads above stay ahead of the weight stream (a wait for one of
  // them placed after the weight loads would wait for the stream too)
  __builtin_amdgcn_sched_barrier(0);

  GmRound<SM, LV> b0, b1, b2;
  const int64_t g0 = blockIdx.x, gs = gridDim.x, glast = (p.N - 1) >> 4;
  auto grp = [&](int j) { const int64_t v = g0 + (int64_t)j * gs; return v < glast ? v : glast; };
  gm_load(b0, p, grp(0), kw, col, g, jc);
  if constexpr (!ONE) gm_load(b1, p, grp(1), kw, col, g, jc);

  {
    const float cv[16] = {cb0[0], cb0[1], cb0[2], cb0[3], cb1[0], cb1[1], cb1[2], cb1[3],
                          cb2[0], cb2[1], cb2[2], cb2[3], cb3[0], cb3[1], cb3[2], cb3[3]};
    static_assert(GM_NT == 512, "table build covers 256 x 32 entries");
    const int lo = (tid >> 5) & 15, copy = tid & 31;
    float clo = cv[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) clo = lo == i ? cv[i] : clo;
#pragma unroll
    for (int hi = 0; hi < 16; ++hi) {
      const float first = p.order ? cv[hi] : clo, second = p.order ? clo : cv[hi];
      sm.tab[(hi * 16 + lo) * 64 + copy] = pack_bf16x2(first, second);
    }
    sm.code2s[tid & 255] = c2;                       // every thread: no branch around the load
  }
  __syncthreads();
  const char* tab = reinterpret_cast<const char*>(sm.tab);
  const uint32_t lb = (uint32_t)(lane & 31) * 4;

  // Round j: partials into red[j & 1], barrier, threads 0..255 sum (in wave
  // order) and store bf16, or an fp32 partial of this K slice. The barrier
  // waits for the LDS stores only (no fence), so the weight loads of the next
  // two rounds stay in flight across it. red[j & 1] is written again in round
  // j + 2, after every thread has passed round j + 1's barrier, which each
  // reaches only after its reads of round j have completed.
  auto finish = [&](const f32x4_t& acc, int j) {
    sm.red[j & 1][wave][lane] = acc;
    __builtin_amdgcn_s_waitcnt(0xC07F);              // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    if (tid < 256) {
      const int ln = tid >> 2, e = tid & 3;
      float v = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) v += sm.red[j & 1][w][ln][e];
      const int m = 4 * (ln >> 4) + e;
      const int64_t n = 16 * (g0 + (int64_t)j * gs) + (ln & 15);
      if (m < p.M && n < p.N) {
        if (gridDim.y == 1) p.y[(int64_t)m * p.ldy + n] = bf16_bits(v);
        else part[((int64_t)blockIdx.y * p.M + m) * p.N + n] = v;
      }
    }
  };
  const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
  // Rounds past the last one load the (clamped) last group again and are never
  // computed: unconditional loads keep the waits exact. Whole groups of three
  // rounds run in the loop (no exit inside it, which made the compiler drain
  // the stream at the loop head); the last one or two after it, from the
  // rounds the loop has already loaded into b0 and b1.
  if constexpr (ONE) {
    finish(active ? gm_compute(b0, p, tab, lb, sm.code2s, xf, tf) : zero, 0);
    return;
  }
  int j = 0;
  for (; j + 3 <= rounds; j += 3) {
    gm_load(b2, p, grp(j + 2), kw, col, g, jc);
    finish(active ? gm_compute(b0, p, tab, lb, sm.code2s, xf, tf) : zero, j);
    gm_load(b0, p, grp(j + 3), kw, col, g, jc);
    finish(active ? gm_compute(b1, p, tab, lb, sm.code2s, xf, tf) : zero, j + 1);
    gm_load(b1, p, grp(j + 4), kw, col, g, jc);
    finish(active ? gm_compute(b2, p, tab, lb, sm.code2s, xf, tf) : zero, j + 2);
  }
  if (j < rounds) finish(active ? gm_compute(b0, p, tab, lb, sm.code2s, xf, tf) : zero, j);
  if (j + 1 < rounds) finish(active ? gm_compute(b1, p, tab, lb, sm.code2s, xf, tf) : zero, j + 1);
}

// Y[m, n] = bf16(sum over K slices of the fp32 partials), slices in order.
__global__ void gm_reduce_kernel(const float* __restrict__ part, int slices, int M, int64_t N,
                                 uint16_t* __restrict__ y, int64_t ldy) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)M * N) return;
  const int m = (int)(i / N);
  const int64_t n = i - (int64_t)m * N;
  float v = 0.0f;
  for (int k = 0; k < slices; ++k) v += part[(int64_t)k * M * N + i];
  y[(int64_t)m * ldy + n] = bf16_bits(v);
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

}  // namespace
}  // namespace molt

using namespace molt;

namespace molt {
namespace {
// K slices of the streaming MFMA kernel (2 <= M <= 16): 0 when it does not apply.
int gm_slices(int64_t M, int64_t K, int& nw) {
  nw = 8;
  if (M < 2 || M > 16 || K % 512 != 0) return 0;
  const int64_t chunks = K / 512;
  if (chunks == 8) return 1;
  if (chunks % 7 == 0 && chunks / 7 <= 8) { nw = 7; return (int)(chunks / 7); }
  if (chunks % 8 == 0 && chunks / 8 <= 8) return (int)(chunks / 8);
  return 0;
}
// K slices of the fallback MFMA kernel (nf4_gemv_kernel): narrow outputs (at
// most 128 groups of 16 rows) split K over up to 8 workgroups per group, as
// many as keep two workgroups per CU and whole 4-block units for every wave.
int gv_slices(int64_t N, int64_t K) {
  const int64_t groups = ceil_div64(N, GV_ROWS);
  if (groups > 128 || K % 256 != 0) return 1;
  const int64_t units = K / 256;                        // 4-block units
  const int64_t s = std::min<int64_t>(std::min<int64_t>(8, units / GV_WAVES), 2 * molt::device_cus() / groups);
  return s < 2 ? 1 : (int)s;
}
}  // namespace
}  // namespace molt

extern "C" size_t molt_nf4_gemv_workspace(int64_t M, int64_t N, int64_t K) {
  // fp32 partials of the K slices when the streaming MFMA kernel, or the
  // fallback kernel of a narrow output, splits K
  int nw = 8;
  const int ks = gm_slices(M, K, nw);
  const int vs = gv_slices(N, K);
  const int s = std::max(ks, vs);
  return s > 1 ? (size_t)s * (size_t)M * (size_t)N * sizeof(float) : 0;
}

extern "C" int molt_nf4_gemv(const uint16_t* x, int64_t ldx, int64_t M, const molt_nf4_weight* w,
                             const uint16_t* t, int64_t ldt, const float* lora_b, int32_t r, float scaling,
                             uint16_t* y, int64_t ldy, void* workspace, size_t workspace_bytes,
                             void* stream) {
  const char* who = "molt_nf4_gemv";
  MOLT_REQUIRE(w && w->packed && w->code && x && y, MOLT_EINVAL, "%s: null argument", who);
  MOLT_REQUIRE(M >= 1 && M <= 16, MOLT_EUNSUPPORTED, "%s: M=%lld outside 1..16", who, (long long)M);
  MOLT_REQUIRE(w->block_size == 64 && w->cols % 64 == 0, MOLT_EUNSUPPORTED,
               "%s: needs block_size 64 and cols %% 64 == 0", who);
  MOLT_REQUIRE(w->cols < (1ll << 30), MOLT_EUNSUPPORTED, "%s: cols too large", who);
  MOLT_REQUIRE(w->rows * (w->cols / 2) < (1ll << 31) && M * ldx < (1ll << 30), MOLT_EUNSUPPORTED,
               "%s: weight or activations too large for 32-bit offsets", who);
  MOLT_REQUIRE(w->rows > 0 && ldx >= w->cols && ldy >= w->rows, MOLT_EINVAL, "%s: bad shape/stride", who);
  MOLT_REQUIRE(ldx % 8 == 0 && aligned(x, 16) && aligned(w->packed, 8) && aligned(w->code, 16), MOLT_EINVAL,
               "%s: X rows and the codebook must be 16-byte aligned and packed data 8-byte aligned", who);
  MOLT_REQUIRE(r >= 0 && (r == 0 || (t && lora_b && ldt >= r)), MOLT_EINVAL, "%s: bad LoRA operands", who);
  MOLT_REQUIRE(r <= GV_RMAX, MOLT_EUNSUPPORTED, "%s: LoRA rank %d > %d", who, r, GV_RMAX);
  const bool nested = w->nested != 0;
  MOLT_REQUIRE(nested ? (w->absmax_q && w->absmax2 && w->code2 && w->dq_block > 0) : (w->scales != nullptr),
               MOLT_EINVAL, "%s: scale statistics missing", who);
  int shift = 0;
  if (nested) {
    MOLT_REQUIRE((w->dq_block & (w->dq_block - 1)) == 0, MOLT_EUNSUPPORTED,
                 "%s: nested block %d is not a power of two", who, w->dq_block);
    while ((1 << shift) < w->dq_block) ++shift;
  }
  GemvParams p{};
  p.x = x; p.ldx = ldx; p.M = (int)M; p.packed = w->packed; p.N = w->rows; p.K = (int)w->cols;
  p.scales = nested ? nullptr : w->scales;
  p.q = w->absmax_q; p.absmax2 = w->absmax2; p.code2 = nested ? w->code2 : nullptr; p.offset = w->offset;
  p.dq_shift = shift;
  p.code = w->code; p.order = w->nibble_order;
  p.t = t; p.ldt = ldt; p.lb = lora_b; p.r = r; p.s = scaling; p.y = y; p.ldy = ldy;
  const int64_t groups = ceil_div64(p.N, GV_ROWS);
  MOLT_REQUIRE(groups < (1ll << 31), MOLT_EINVAL, "%s: problem too large", who);
  hipStream_t st = (hipStream_t)stream;
  // Decode: streaming dot-product kernel, one row per wave per round, as many
  // workgroups as fit on the GPU at once (two per CU at K = 4096 with up to two
  // tokens, else one; at K = 14336 three rounds of 7 KB per wave need ~190
  // registers); the waves loop over the rounds. M = 2 runs with two X rows, 3
  // and 4 with four. It serves M <= 2, and M = 3, 4 where it measured faster
  // than the MFMA kernel (K = 14336, or at most 2048 rows); the
  // MOLT_TUNE_GEMV_DOT_M setting (0..4) replaces that rule by a plain bound on M.
  // Any K (a multiple of 64, at most 7 pieces of 2048): a row is IPR pieces of
  // 1 KB, the last possibly partial; IPR is rounded up to an instantiated
  // value (a wholly idle piece re-reads the row's last bytes and is dropped).
  // Where the MFMA kernel does not take K (not 8, or a multiple of 7 or 8,
  // chunks of 512), the dot kernel also serves M = 3, 4.
  // M = 5..8 over at most 2048 rows and K <= 4096 (eight X rows of at most
  // two pieces fit in LDS beside the code table): eight tokens per lookup,
  // where the MFMA kernel, with one 16-row group per workgroup, leaves most
  // CUs idle.
  int gm_nw_probe = 8;
  const bool gm_takes_k = gm_slices(4, w->cols, gm_nw_probe) > 0;
  const int ipr_need = (int)ceil_div64(w->cols, 2048);
  const int dot_max_m = (int)molt::tuning_value(MOLT_TUNE_GEMV_DOT_M);
  const bool dot_m = (dot_max_m >= 0 ? M <= dot_max_m
                                     : (M <= 2 || (M <= 4 && (w->cols == 14336 || w->rows <= 2048 || !gm_takes_k)) ||
                                        (M <= 8 && w->rows <= 2048))) &&
                     (M <= 4 || ipr_need <= 2);
  if (dot_m && ipr_need <= 7 && aligned(w->packed, 16)) {
    const int ipr = ipr_need <= 3 ? ipr_need : (ipr_need <= 5 ? 5 : 7);
    const int cus = molt::device_cus();
    const int rw = 1;                                         // rows per wave per round
    const int mx = M == 1 ? 1 : (M == 2 ? 2 : (M <= 4 ? 4 : 8));   // X rows held by the kernel
    // One workgroup per CU, so that each wave has more rounds over the same
    // set-up work (code table, X, LoRA operands): one token 4096^2 5.2 -> 4.95
    // us, 14336 x 4096 10.5-11.2 -> 10.1-10.2 us, 8960 x 1536 6.4 -> 5.4 us;
    // two tokens 14336 x 4096 12.8-13.1 -> 12.1-12.5 us, 8960 x 1536 7.6 ->
    // 6.4 us. Two (the kernel then fits in 128 registers) for two tokens over
    // at most 4096 rows, where one measured slower (4096^2: 5.35 -> 5.6 us).
    const int per_cu = ipr <= 2 && mx == 2 && w->rows <= 4096 ? 2 : 1;
    const int64_t waves = std::min<int64_t>(ceil_div64(w->rows, rw), (int64_t)cus * GD_WAVES * per_cu);
    const int64_t wgs = ceil_div64(waves, GD_WAVES);
    const int rounds = (int)ceil_div64(w->rows, wgs * GD_WAVES * rw);
    const size_t dyn = ipr == 2 && mx == 1 ? 0 : (size_t)mx * (ipr * 2048 + GD_XPAD) * 2;   // X in registers
    // rows of whole pieces (K = 4096, 14336) skip the partial-piece clamps and masks
    const bool full = w->cols == (int64_t)ipr * 2048;
#define MOLT_GDK(IPRv, MXv, NE, LO, MR)                                                                        \
  do {                                                                                                          \
    if ((IPRv == 2 || IPRv == 7) && full)                                                                       \
      hipLaunchKernelGGL((nf4_gemv_dot_kernel<1, IPRv, MXv, NE, LO, MR, (IPRv == 2 || IPRv == 7)>),             \
                         dim3((unsigned)wgs), dim3(GD_NT), dyn, st, p, rounds);                                 \
    else                                                                                                        \
      hipLaunchKernelGGL((nf4_gemv_dot_kernel<1, IPRv, MXv, NE, LO, MR, false>), dim3((unsigned)wgs), dim3(GD_NT), \
                         dyn, st, p, rounds);                                                                   \
  } while (0)
    // nested statistics with at most 4 rounds per wave (every cfg5 decode shape): straight-line rounds
#define MOLT_GDS(IPRv, MXv, LO)                                                   \
  do {                                                                            \
    if (rounds == 1) MOLT_GDK(IPRv, MXv, true, LO, 1);                                       \
    else if (rounds == 2) MOLT_GDK(IPRv, MXv, true, LO, 2); else MOLT_GDK(IPRv, MXv, true, LO, 4); \
  } while (0)
#define MOLT_GD(IPRv, MXv)                                                                                  \
  do {                                                                                                      \
    if (nested && rounds <= 4) { if (r > 0) MOLT_GDS(IPRv, MXv, true); else MOLT_GDS(IPRv, MXv, false); } \
    else if (nested) { if (r > 0) MOLT_GDK(IPRv, MXv, true, true, 0); else MOLT_GDK(IPRv, MXv, true, false, 0); } \
    else { if (r > 0) MOLT_GDK(IPRv, MXv, false, true, 0); else MOLT_GDK(IPRv, MXv, false, false, 0); }     \
  } while (0)
#define MOLT_GDI(IPRv)                                                                               \
  do {                                                                                                 \
    if (mx == 1) MOLT_GD(IPRv, 1);                                                                     \
    else if (mx == 2) MOLT_GD(IPRv, 2);                                                                \
    else if (mx == 4) MOLT_GD(IPRv, 4);                                                                \
    else MOLT_GD((IPRv <= 2 ? IPRv : 2), 8);   /* eight rows: at most two pieces (see dot_m) */       \
  } while (0)
    switch (ipr) {
      case 1: MOLT_GDI(1); break;
      case 2: MOLT_GDI(2); break;
      case 3: MOLT_GDI(3); break;
      case 5: MOLT_GDI(5); break;
      default: MOLT_GDI(7); break;
    }
#undef MOLT_GDI
#undef MOLT_GD
#undef MOLT_GDS
#undef MOLT_GDK
    return check_launch(who);
  }
  // 2 <= M <= 16, K of 8 (or a multiple of 7 or 8) 512-element chunks:
  // streaming MFMA kernel over 16-row groups, one workgroup per CU, K split
  // over the waves (and, past 4096, over workgroups with fp32 partials).
  int gm_nw = 8;
  int gm_ks = gm_slices(M, w->cols, gm_nw);
  // K of 3, 4 or 6 chunks (1536, 2048, 3072: the hidden widths of the smaller
  // Qwen2.5 / Llama-3.2 models) with at least one 16-row group per CU: the
  // same kernel with 3, 4 or 6 waves owning a chunk each (the others only help
  // the reduction), so the code table is built once per CU instead of once per
  // 16 rows. Every LoRA rank chunk of 32 needs a wave of its own.
  if (gm_ks == 0 && M >= 2 && w->cols % 512 == 0 && ceil_div64(w->rows, 16) >= molt::device_cus()) {
    const int chunks = (int)(w->cols / 512);
    if ((chunks == 3 || chunks == 4 || chunks == 6) && r <= 32 * chunks) {
      gm_nw = chunks;
      gm_ks = 1;
    }
  }
  if (gm_ks > 0 && aligned(w->packed, 8) && aligned(x, 16) && ldx % 8 == 0) {
    const size_t need = molt_nf4_gemv_workspace(M, w->rows, w->cols);
    MOLT_REQUIRE(workspace_bytes >= need && (need == 0 || aligned(workspace, 16)), MOLT_EWORKSPACE,
                 "%s: workspace of %zu bytes (16-byte aligned) needed, got %zu", who, need, workspace_bytes);
    const int cus = molt::device_cus();
    const int64_t groups16 = ceil_div64(w->rows, 16);
    const int64_t wgs = std::max<int64_t>(1, std::min<int64_t>(groups16, cus / gm_ks));
    const int rounds = (int)ceil_div64(groups16, wgs);
    const bool q4u = nested && w->dq_block >= 4 && aligned(w->absmax_q, 4);
    float* part = gm_ks > 1 ? static_cast<float*>(workspace) : nullptr;
    const dim3 grid((unsigned)wgs, (unsigned)gm_ks);
    // LoRA B rows as 16-byte vectors where every 4-rank group is aligned
    const int lv = r == 0 ? 0 : (r % 4 == 0 && aligned(lora_b, 16) ? 1 : 2);
#define MOLT_GM3(SMv, NWv, LVv)                                                                        \
  do {                                                                                                  \
    if (rounds == 1)                                                                                    \
      hipLaunchKernelGGL((nf4_gemv_ms_kernel<SMv, NWv, LVv, true>), grid, dim3(GM_NT), 0, st, p, rounds, part);  \
    else                                                                                                \
      hipLaunchKernelGGL((nf4_gemv_ms_kernel<SMv, NWv, LVv, false>), grid, dim3(GM_NT), 0, st, p, rounds, part); \
  } while (0)
#define MOLT_GM(SMv, NWv) \
  do { if (lv == 0) MOLT_GM3(SMv, NWv, 0); else if (lv == 1) MOLT_GM3(SMv, NWv, 1); else MOLT_GM3(SMv, NWv, 2); } while (0)
#define MOLT_GMN(NWv) \
  do { if (!nested) MOLT_GM(0, NWv); else if (q4u) MOLT_GM(2, NWv); else MOLT_GM(1, NWv); } while (0)
    switch (gm_nw) {
      case 8: MOLT_GMN(8); break;
      case 7: MOLT_GMN(7); break;
      case 6: MOLT_GMN(6); break;
      case 4: MOLT_GMN(4); break;
      default: MOLT_GMN(3); break;
    }
#undef MOLT_GMN
#undef MOLT_GM
#undef MOLT_GM3
    if (gm_ks > 1) {
      const int64_t n = M * w->rows;
      hipLaunchKernelGGL(gm_reduce_kernel, dim3((unsigned)ceil_div64(n, 256)), dim3(256), 0, st, part, gm_ks,
                         (int)M, w->rows, y, ldy);
    }
    return check_launch(who);
  }
  const bool q4 = nested && (w->cols / 64) % 4 == 0 && w->dq_block >= 4 && aligned(w->absmax_q, 4);
  // narrow outputs split K over workgroups (fp32 partials summed in slice order)
  int vs = gv_slices(w->rows, w->cols);
  if (vs > 1) {
    const size_t need = (size_t)vs * (size_t)M * (size_t)w->rows * sizeof(float);
    if (!(workspace && aligned(workspace, 16) && workspace_bytes >= need)) vs = 1;   // a smaller workspace: unsplit
  }
  float* part = vs > 1 ? static_cast<float*>(workspace) : nullptr;
  const dim3 grid((unsigned)groups, (unsigned)vs);
  if (q4) hipLaunchKernelGGL((nf4_gemv_kernel<true>), grid, dim3(GV_NT), 0, st, p, part);
  else hipLaunchKernelGGL((nf4_gemv_kernel<false>), grid, dim3(GV_NT), 0, st, p, part);
  if (vs > 1) {
    const int rc = check_launch(who);
    if (rc) return rc;
    const int64_t n = M * w->rows;
    hipLaunchKernelGGL(gm_reduce_kernel, dim3((unsigned)ceil_div64(n, 256)), dim3(256), 0, st, part, vs, (int)M,
                       w->rows, y, ldy);
  }
  return check_launch(who);
}

// ---------------------------------------------------------------------------
// molt_nf4_gemv_noalloc: molt_nf4_gemv with its split-K partials in a static
// device array instead of a caller workspace, for callers that cannot allocate.
// ---------------------------------------------------------------------------
namespace {
constexpr size_t GEMV_SCRATCH_BYTES = size_t(8) << 20;   // 2 Mi fp32 partials
constexpr int GEMV_SCRATCH_DEVICES = 64;

// One copy per device, held until the process ends. Host code never uses this
// name as an address: it is the host-side handle of the symbol, and only the
// per-device address that hipGetSymbolAddress returns is passed to kernels.
static __device__ __align__(256) unsigned char scratch[GEMV_SCRATCH_BYTES];

std::mutex g_scratch_mu;
void* g_scratch_addr[GEMV_SCRATCH_DEVICES];
// Per device: an event recorded after the last call that used the scratch, and
// the stream that call ran on. A call on another stream waits on the event
// first, so calls from different streams are ordered instead of racing.
hipEvent_t g_scratch_done[GEMV_SCRATCH_DEVICES];
hipStream_t g_scratch_stream[GEMV_SCRATCH_DEVICES];
bool g_scratch_used[GEMV_SCRATCH_DEVICES];

// Set-up on the first call on a device (with it current): the address of
// `scratch` and the ordering event, both kept until the process ends. Returns
// the device index through `dev_out`. The caller holds g_scratch_mu.
int scratch_setup(int* dev_out, const char* who) {
  int dev = -1;
  const hipError_t de = hipGetDevice(&dev);
  MOLT_REQUIRE(de == hipSuccess && dev >= 0 && dev < GEMV_SCRATCH_DEVICES, MOLT_ELAUNCH,
               "%s: no current device (%s)", who, hipGetErrorString(de));
  if (g_scratch_addr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    MOLT_REQUIRE(e == hipSuccess && p != nullptr, MOLT_ELAUNCH, "%s: scratch symbol lookup failed on device %d: %s",
                 who, dev, hipGetErrorString(e));
    hipEvent_t ev = nullptr;
    const hipError_t ee = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    MOLT_REQUIRE(ee == hipSuccess, MOLT_ELAUNCH, "%s: scratch ordering event on device %d: %s", who, dev,
                 hipGetErrorString(ee));
    g_scratch_done[dev] = ev;
    g_scratch_addr[dev] = p;
  }
  *dev_out = dev;
  return MOLT_OK;
}

// True when `stream` is being captured into a graph. The legacy null stream
// cannot be captured, so it is not asked.
bool capturing(hipStream_t stream) {
  if (stream == nullptr) return false;
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(stream, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}
}  // namespace

extern "C" size_t molt_nf4_gemv_noalloc_limit(void) { return GEMV_SCRATCH_BYTES; }

extern "C" int molt_nf4_gemv_noalloc(const uint16_t* x, int64_t ldx, int64_t M, const molt_nf4_weight* w,
                                     const uint16_t* t, int64_t ldt, const float* lora_b, int32_t r, float scaling,
                                     uint16_t* y, int64_t ldy, void* stream) {
  const char* who = "molt_nf4_gemv_noalloc";
  MOLT_REQUIRE(w != nullptr, MOLT_EINVAL, "%s: null weight", who);
  MOLT_REQUIRE(M >= 1 && M <= 16 && w->rows > 0 && w->cols > 0, MOLT_EUNSUPPORTED, "%s: M=%lld outside 1..16 or empty weight",
               who, (long long)M);
  const size_t need = molt_nf4_gemv_workspace(M, w->rows, w->cols);
  MOLT_REQUIRE(need <= GEMV_SCRATCH_BYTES, MOLT_EUNSUPPORTED,
               "%s: M=%lld, %lld x %lld needs %zu bytes of split-K partials, more than the %zu-byte static scratch "
               "(use molt_nf4_gemv with a workspace)",
               who, (long long)M, (long long)w->rows, (long long)w->cols, need, GEMV_SCRATCH_BYTES);
  if (need == 0) return molt_nf4_gemv(x, ldx, M, w, t, ldt, lora_b, r, scaling, y, ldy, nullptr, 0, stream);
  // Wait, launch and record under one lock, so calls from several host threads
  // are ordered as they take it. Under graph capture the graph's own order
  // applies and the event is neither waited on nor recorded.
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  int dev = -1;
  const int rc = scratch_setup(&dev, who);
  if (rc != MOLT_OK) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool order = !capturing(s);
  if (order && g_scratch_used[dev] && g_scratch_stream[dev] != s) {
    const hipError_t e = hipStreamWaitEvent(s, g_scratch_done[dev], 0);
    MOLT_REQUIRE(e == hipSuccess, MOLT_ELAUNCH, "%s: wait for the previous scratch user: %s", who,
                 hipGetErrorString(e));
  }
  // Nothing in the scratch has to start at zero: every partial the reduction
  // reads is written earlier in the same call.
  const int lrc = molt_nf4_gemv(x, ldx, M, w, t, ldt, lora_b, r, scaling, y, ldy, g_scratch_addr[dev], need, stream);
  if (lrc != MOLT_OK || !order) return lrc;
  const hipError_t e = hipEventRecord(g_scratch_done[dev], s);
  MOLT_REQUIRE(e == hipSuccess, MOLT_ELAUNCH, "%s: record the scratch ordering event: %s", who, hipGetErrorString(e));
  g_scratch_stream[dev] = s;
  g_scratch_used[dev] = true;
  return MOLT_OK;
}
