// Rank-r LoRA kernels (gfx950): the low-rank projection T = z . bf16(W)^T and
// the adapter gradients dA = U^T X, dB = s dY^T T. Both stream one large
// [M, D] activation from HBM once; the rank-r side is small and L2-resident.
#include <stdlib.h>

#include <algorithm>

#include "mfma_core.h"

namespace molt {
namespace {

MOLT_DEV float silu_f32(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

// z transform: 0 plain, 1 SwiGLU replay bf16(bf16(silu(g)) u), 2 bf16(s z).
MOLT_DEV float ztrans(float a, float b, int mode, float s) {
  if (mode == 1) return round_bf16(silu_f32(a)) * b;
  if (mode == 2) return a * s;
  return a;
}

// Eight consecutive bf16 elements of one row of a [rows, C] operand (and of
// the up tensor for the SwiGLU replay), as loaded. With VEC (rows 16-byte
// aligned, C % 8 == 0) they are one 16-byte load from a clamped address, and
// the transform and the zero mask outside the matrix are applied only when
// the chunk is consumed, so the load stays in flight until then. Without VEC
// the elements are loaded one by one and transformed at once.
struct Chunk {
  u32x4_t a, b;
  bool ok;
};

template <bool VEC, bool REPLAY>
MOLT_DEV void chunk_load(Chunk& c, const uint16_t* __restrict__ z, const uint16_t* __restrict__ z2, int64_t ld,
                         int mode, float s, int64_t m, int64_t rows, int64_t col, int64_t C) {
  if (VEC) {
    c.ok = m < rows && col < C;
    const int64_t off = c.ok ? m * ld + col : 0;
    c.a = *reinterpret_cast<const u32x4_t*>(z + off);
    if (REPLAY) c.b = *reinterpret_cast<const u32x4_t*>(z2 + off);
    return;
  }
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float x = 0.0f;
    if (m < rows && col + e < C) {
      const float a = bf16_to_f32(z[m * ld + col + e]);
      const float b = mode == 1 ? bf16_to_f32(z2[m * ld + col + e]) : 0.0f;
      x = ztrans(a, b, mode, s);
    }
    v[e] = x;
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) c.a[e] = pack_bf16x2(v[2 * e], v[2 * e + 1]);
  c.ok = true;
}

template <bool VEC, bool REPLAY>
MOLT_DEV u32x4_t chunk_value(const Chunk& c, int mode, float s) {
  if (!VEC) return c.a;
  u32x4_t o = c.a;
  if (REPLAY || mode == 2) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = REPLAY ? ztrans(bf16_lo(c.a[e]), bf16_lo(c.b[e]), 1, s) : bf16_lo(c.a[e]) * s;
      const float hi = REPLAY ? ztrans(bf16_hi(c.a[e]), bf16_hi(c.b[e]), 1, s) : bf16_hi(c.a[e]) * s;
      o[e] = pack_bf16x2(lo, hi);
    }
  }
  const uint32_t keep = c.ok ? 0xffffffffu : 0u;
  return o & keep;
}

// ------------------------------------------------------------------------
// Projection out[M, R] = bf16(sum_d z(m, d) * bf16(W(q, d))).
//
// The adapter matrix is first packed to bf16 in MFMA fragment order:
// fragment (step, t, kk), lane l holds W(q = 32 t + l % 32, d) for the 8
// consecutive d = 64 step + 32 (l / 32) + 8 kk + e, so every fragment load is
// one coalesced 1 KB read (the packed matrix stays in L2). A workgroup owns
// 32 MT rows of z and all R outputs; each wave applies a W fragment to its MT
// 32-row z tiles. The 8 waves take every 8th 64-deep step, with the next
// step's z and W fragments in flight while the current step's MFMAs run, and
// their partial tiles are summed in wave order through LDS.
// ------------------------------------------------------------------------
constexpr int PJ_WAVES = 8, PJ_TQ_MAX = 4;

__global__ void lora_pack_kernel(const float* __restrict__ w, int layout, int R, int64_t D, int tq,
                                 int64_t steps, uint16_t* __restrict__ wp) {
  const int64_t total = steps * tq * 4 * 64;
  for (int64_t f = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; f < total;
       f += (int64_t)gridDim.x * blockDim.x) {
    const int lane = (int)(f & 63);
    const int64_t rest = f >> 6;
    const int kk = (int)(rest & 3);
    const int64_t st = rest >> 2;
    const int t = (int)(st % tq);
    const int64_t step = st / tq;
    const int q = 32 * t + (lane & 31);
    const int64_t d0 = 64 * step + 32 * (lane >> 5) + 8 * kk;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t d = d0 + e;
      v[e] = (q < R && d < D) ? (layout == 0 ? w[(int64_t)q * D + d] : w[d * R + q]) : 0.0f;
    }
    u32x4_t o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = pack_bf16x2(v[2 * e], v[2 * e + 1]);
    *reinterpret_cast<u32x4_t*>(wp + f * 8) = o;
  }
}

// Several adapters packed in one launch (molt_lora_pack_many): fragment f of
// adapter d is flat index first[d] + f, packed exactly as lora_pack_kernel
// does; rows q < split[d] come from w0[d], the rest from w1[d] (the gate and
// up A matrices stacked as one [2r, D] operand without a copy).
constexpr int kPackMany = 8;
struct PackMany {
  const float* w0[kPackMany];
  const float* w1[kPackMany];
  uint16_t* wp[kPackMany];
  int64_t D[kPackMany], steps[kPackMany];
  int64_t first[kPackMany + 1];
  int split[kPackMany], R[kPackMany], tq[kPackMany], layout[kPackMany];
  int n;
};

__global__ void lora_pack_many_kernel(const PackMany m) {
  const int64_t total = m.first[m.n];
  for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < total; g += (int64_t)gridDim.x * blockDim.x) {
    int d = 0;
#pragma unroll
    for (int k = 1; k < kPackMany; ++k) d += (k < m.n && g >= m.first[k]) ? 1 : 0;
    const int64_t f = g - m.first[d];
    const int lane = (int)(f & 63);
    const int64_t rest = f >> 6;
    const int kk = (int)(rest & 3);
    const int64_t st = rest >> 2;
    const int tq = m.tq[d];
    const int t = (int)(st % tq);
    const int64_t step = st / tq;
    const int q = 32 * t + (lane & 31);
    const int64_t D = m.D[d], d0 = 64 * step + 32 * (lane >> 5) + 8 * kk;
    const int R = m.R[d], split = m.split[d];
    const bool first_src = q < split;
    const float* w = first_src ? m.w0[d] : m.w1[d];
    const int qs = first_src ? q : q - split, Rs = first_src ? split : R - split;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t dd = d0 + e;
      v[e] = (q < R && dd < D) ? (m.layout[d] == 0 ? w[(int64_t)qs * D + dd] : w[dd * Rs + qs]) : 0.0f;
    }
    u32x4_t o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = pack_bf16x2(v[2 * e], v[2 * e + 1]);
    *reinterpret_cast<u32x4_t*>(m.wp[d] + f * 8) = o;
  }
}

struct ProjParams {
  const uint16_t* z; const uint16_t* z2; int64_t ldz; int mode; float zs;
  int64_t M, D; int R;
  const uint16_t* wp;
  uint16_t* out; int64_t ldo;
  float* part;          // K split: fp32 partials [ks][M][32 TQ]
  // a pair launch (lora_project_dma_kernel, gridDim.z == 2): the second
  // operand's z, packed adapter, scale, output and partials for blockIdx.z == 1
  const uint16_t* zb; const uint16_t* wpb; float zsb; uint16_t* outb; float* partb;
};

template <typename T>
MOLT_DEV T pick2(bool c, T a, T b) { return c ? a : b; }

template <int MT, bool VEC, bool REPLAY>
MOLT_DEV void proj_load_z(Chunk (&z)[MT][4], const ProjParams& p, int64_t s, int64_t m0, int lane) {
  const int h = lane >> 5;
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      chunk_load<VEC, REPLAY>(z[i][kk], p.z, p.z2, p.ldz, p.mode, p.zs, m0 + 32 * i + (lane & 31), p.M,
                              s * BK + 32 * h + 8 * kk, p.D);
}

template <int TQ>
MOLT_DEV void proj_load_w(u32x4_t (&w)[TQ][4], const ProjParams& p, int64_t s, int lane) {
#pragma unroll
  for (int t = 0; t < TQ; ++t)
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      w[t][kk] = *reinterpret_cast<const u32x4_t*>(p.wp + (((s * TQ + t) * 4 + kk) * 64 + lane) * 8);
}

template <int TQ, int MT, bool VEC, bool REPLAY>
MOLT_DEV void proj_mfma(const Chunk (&z)[MT][4], const u32x4_t (&w)[TQ][4], const ProjParams& p,
                        f32x16_t (&acc)[MT][TQ]) {
#pragma unroll
  for (int kk = 0; kk < 4; ++kk)
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const bf16x8_t zv = __builtin_bit_cast(bf16x8_t, chunk_value<VEC, REPLAY>(z[i][kk], p.mode, p.zs));
#pragma unroll
      for (int t = 0; t < TQ; ++t)
        acc[i][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, w[t][kk]), zv,
                                                            acc[i][t], 0, 0, 0);
    }
}

// With KS > 1 the 64-deep steps are split into KS contiguous ranges, one per
// workgroup of blockIdx.y, and each writes its fp32 partial tile; a second
// kernel sums the KS partials in range order and rounds to bf16 (more
// workgroups in flight for small M, same result on every run).
template <int TQ, int MT, bool VEC, bool REPLAY, int KS>
__global__ __launch_bounds__(64 * PJ_WAVES) void lora_project_kernel(const ProjParams p) {
  __shared__ f32x16_t red[PJ_WAVES - 1][64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t m0 = (int64_t)blockIdx.x * (32 * MT);
  const int64_t all_steps = ceil_div64(p.D, BK);
  const int64_t s_begin = KS > 1 ? all_steps * blockIdx.y / KS : 0;
  const int64_t steps = KS > 1 ? all_steps * (blockIdx.y + 1) / KS : all_steps;   // end of this range

  f32x16_t acc[MT][TQ];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int t = 0; t < TQ; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][t][e] = 0.0f;

  // Two z fragment sets alternate, so each step's activation loads (from HBM)
  // are issued a step ahead; the step's adapter fragments (L2 hits) are
  // issued just before them. Loads are never skipped (past the end they
  // repeat the last step), so the wait before each MFMA batch is a fixed count.
  if (s_begin + wave < steps) {
    Chunk za[MT][4], zb[MT][4];
    u32x4_t w[TQ][4];
    int64_t s = s_begin + wave;
    proj_load_z<MT, VEC, REPLAY>(za, p, s, m0, lane);
    for (;;) {
      proj_load_w<TQ>(w, p, s, lane);
      proj_load_z<MT, VEC, REPLAY>(zb, p, s + PJ_WAVES < steps ? s + PJ_WAVES : steps - 1, m0, lane);
      proj_mfma<TQ, MT, VEC, REPLAY>(za, w, p, acc);
      s += PJ_WAVES;
      if (s >= steps) break;
      proj_load_w<TQ>(w, p, s, lane);
      proj_load_z<MT, VEC, REPLAY>(za, p, s + PJ_WAVES < steps ? s + PJ_WAVES : steps - 1, m0, lane);
      proj_mfma<TQ, MT, VEC, REPLAY>(zb, w, p, acc);
      s += PJ_WAVES;
      if (s >= steps) break;
    }
  }

  // Partial tiles are summed in wave order, one (i, t) tile at a time.
  const int h = lane >> 5;
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int t = 0; t < TQ; ++t) {
      if (wave > 0) red[wave - 1][lane] = acc[i][t];
      __syncthreads();
      if (wave == 0) {
        f32x16_t v = acc[i][t];
#pragma unroll
        for (int w = 0; w < PJ_WAVES - 1; ++w) v += red[w][lane];
        // v is C[q][m]: column m = lane % 32, rows q = 32 t + 8 (e/4) + 4 h + e%4.
        const int64_t m = m0 + 32 * i + (lane & 31);
        if (m < p.M) {
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int q = 32 * t + 8 * (e >> 2) + 4 * h + (e & 3);
            if (KS > 1) p.part[((int64_t)blockIdx.y * p.M + m) * (32 * TQ) + q] = v[e];
            else if (q < p.R) p.out[m * p.ldo + q] = bf16_bits(v[e]);
          }
        }
      }
      __syncthreads();
    }
}

// DMA-staged variant (plain or pre-scaled z, rows 16-byte aligned, D % 64 ==
// 0): each wave streams its steps of z through a private pair of LDS buffers
// by buffer-load DMA. DMA instruction c of a step loads rows 8c .. 8c + 7 with
// 8 lanes per row, so every load covers whole 128-byte lines (the direct
// fragment loads touch 32 rows per instruction, 32 bytes of each line); the
// MFMA fragments are then read back with ds_read_b128. Chunk j of row r sits
// at position j ^ f(r), f(r) = (r ^ (r >> 3)) & 7 restricted as below, which
// keeps the 16-row fragment reads free of bank conflicts.
MOLT_DEV int pj_swz(int r) { return (r ^ ((r >> 3) & 3)) & 7; }

typedef __attribute__((address_space(3))) void* pj_lds_t;

MOLT_DEV __amdgpu_buffer_rsrc_t pj_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

MOLT_DEV void pj_dma16(__amdgpu_buffer_rsrc_t r, uint16_t* dst, uint32_t off, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (pj_lds_t)dst, 16, off, soff, 0, 0);
}

// Wait until at most N vector-memory ops are outstanding (vmcnt N, other
// counters untouched), with compiler barriers so no LDS read moves above the
// wait. gfx9 splits vmcnt over bits 3:0 and 15:14.
template <int N>
MOLT_DEV void pj_wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
  asm volatile("" ::: "memory");
}

// Workgroup barrier without __syncthreads()'s release fence, which would make
// every wave drain its DMA in flight (stages that are only read later); the
// caller waits (vmcnt) for the stage the other waves read next, and this
// wave's own LDS accesses are waited for here.
MOLT_DEV void pj_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// The adapter fragments of step s by buffer loads: the lane offset is fixed
// and the step's offset scalar, so a step needs no address registers (the
// compiler would otherwise reuse ones that a load in flight still writes).
template <int TQ>
MOLT_DEV void pj_load_w(u32x4_t (&w)[TQ][4], __amdgpu_buffer_rsrc_t wr, int64_t s, int lane) {
#pragma unroll
  for (int t = 0; t < TQ; ++t) {
    const uint32_t so = __builtin_amdgcn_readfirstlane((uint32_t)((s * TQ + t) * 4 * 64 * 16));
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) w[t][kk] = __builtin_amdgcn_raw_buffer_load_b128(wr, lane * 16 + kk * 1024, so, 0);
  }
}

template <int TQ, int MT, int KS>
__global__ __launch_bounds__(64 * PJ_WAVES) void lora_project_dma_kernel(const ProjParams p) {
  // operand blockIdx.z of a pair launch (kernel-argument values, selected in scalar registers)
  const bool second = blockIdx.z != 0;
  const uint16_t* const pz = pick2(second, p.zb, p.z);
  const uint16_t* const pwp = pick2(second, p.wpb, p.wp);
  const float pzs = pick2(second, p.zsb, p.zs);
  uint16_t* const pout = pick2(second, p.outb, p.out);
  float* const ppart = pick2(second, p.partb, p.part);
  // z buffers per wave: a ring of three (z two of the wave's steps ahead)
  // where the LDS allows it, else two (one step ahead). One array per ring
  // slot, selected statically: the compiler waits for every DMA that may
  // write the LDS a fragment read touches, and only distinct arrays tell it
  // that the DMA in flight does not.
  constexpr int NB = MT == 1 ? 3 : 2;
  constexpr int ZB = 32 * MT * BK;
  __shared__ f32x16_t red[PJ_WAVES - 1][64];
  __shared__ __attribute__((aligned(16))) uint16_t zs0[PJ_WAVES][ZB], zs1[PJ_WAVES][ZB];
  __shared__ __attribute__((aligned(16))) uint16_t zs2[NB == 3 ? PJ_WAVES : 1][NB == 3 ? ZB : 8];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5;
  const int64_t m0 = (int64_t)blockIdx.x * (32 * MT);
  const int64_t all_steps = p.D / BK;
  const int64_t s_begin = KS > 1 ? all_steps * blockIdx.y / KS : 0;
  const int64_t s_end = KS > 1 ? all_steps * (blockIdx.y + 1) / KS : all_steps;

  f32x16_t acc[MT][TQ];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int t = 0; t < TQ; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][t][e] = 0.0f;

  if (s_begin + wave < s_end) {
    const __amdgpu_buffer_rsrc_t zr = pj_rsrc(pz, ((p.M - 1) * p.ldz + p.D) * 2);
    const __amdgpu_buffer_rsrc_t wr = pj_rsrc(pwp, all_steps * TQ * 4 * 64 * 16);
    uint32_t zoff[4 * MT];
#pragma unroll
    for (int c = 0; c < 4 * MT; ++c) {
      const int r = 8 * c + (lane >> 3);
      const int64_t m = min(m0 + r, p.M - 1);
      zoff[c] = (uint32_t)((m * p.ldz + 8 * ((lane & 7) ^ pj_swz(r))) * 2);
    }
    int foff[MT][4];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int r = 32 * i + (lane & 31);
        foff[i][kk] = r * BK + (((4 * h + kk) ^ pj_swz(r)) << 3);
      }
    auto dma = [&](int64_t s, uint16_t* dst) {
#pragma unroll
      for (int c = 0; c < 4 * MT; ++c) pj_dma16(zr, dst + c * 512, zoff[c], (uint32_t)(s * BK * 2));
    };
    // The adapter fragments by register loads one step ahead (two register
    // sets, alternating; they come from L2). z by DMA NB - 1 steps ahead: with
    // three buffers a step issues the next step's adapter loads before the
    // z two steps on, so its wait (loads complete in issue order) leaves
    // both of those and the z issued a step earlier in flight.
    u32x4_t w0[TQ][4], w1[TQ][4];
    int64_t s = s_begin + wave;
    auto clamp = [&](int64_t t) { return t < s_end ? t : s_end - 1; };
    uint16_t* z0 = zs0[wave];
    uint16_t* z1 = zs1[wave];
    uint16_t* z2 = zs2[NB == 3 ? wave : 0];
    dma(s, z0);
    pj_load_w<TQ>(w0, wr, s, lane);
    if constexpr (NB == 3) dma(clamp(s + PJ_WAVES), z1);
    // step with z(s) in zc and the adapter in wc; zn receives the z load it issues
    auto step = [&](const u32x4_t (&wc)[TQ][4], u32x4_t (&wn)[TQ][4], const uint16_t* zc, uint16_t* zn) {
      const int64_t sn = clamp(s + PJ_WAVES);
      if constexpr (NB == 3) {
        pj_load_w<TQ>(wn, wr, sn, lane);
        dma(clamp(s + 2 * PJ_WAVES), zn);
        pj_wait_vm<8 * MT + 4 * TQ>();              // this step's z and adapter landed
      } else {
        dma(sn, zn);
        pj_load_w<TQ>(wn, wr, sn, lane);
        pj_wait_vm<4 * MT + 4 * TQ>();              // this step's z and adapter landed; the next step's may fly
      }
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          u32x4_t zv = *reinterpret_cast<const u32x4_t*>(zc + foff[i][kk]);
          if (p.mode == 2) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              zv[e] = pack_bf16x2(bf16_lo(zv[e]) * pzs, bf16_hi(zv[e]) * pzs);
          }
          const bf16x8_t zb = __builtin_bit_cast(bf16x8_t, zv);
#pragma unroll
          for (int t = 0; t < TQ; ++t)
            acc[i][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, wc[t][kk]), zb,
                                                                acc[i][t], 0, 0, 0);
        }
      s += PJ_WAVES;
      return s < s_end;
    };
    if constexpr (NB == 3) {
      // z of the wave's step j in buffer j % 3, the adapter in set j % 2: the pattern repeats every 6 steps
      while (step(w0, w1, z0, z2) && step(w1, w0, z1, z0) && step(w0, w1, z2, z1) && step(w1, w0, z0, z2) &&
             step(w0, w1, z1, z0) && step(w1, w0, z2, z1)) {
      }
    } else {
      while (step(w0, w1, z0, z1) && step(w1, w0, z1, z0)) {
      }
    }
    pj_wait_vm<0>();   // the last (repeated) loads before the kernel ends
  }

#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int t = 0; t < TQ; ++t) {
      if (wave > 0) red[wave - 1][lane] = acc[i][t];
      __syncthreads();
      if (wave == 0) {
        f32x16_t v = acc[i][t];
#pragma unroll
        for (int w2 = 0; w2 < PJ_WAVES - 1; ++w2) v += red[w2][lane];
        const int64_t m = m0 + 32 * i + (lane & 31);
        if (m < p.M) {
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int q = 32 * t + 8 * (e >> 2) + 4 * h + (e & 3);
            if (KS > 1) ppart[((int64_t)blockIdx.y * p.M + m) * (32 * TQ) + q] = v[e];
            else if (q < p.R) pout[m * p.ldo + q] = bf16_bits(v[e]);
          }
        }
      }
      __syncthreads();
    }
}

__global__ void proj_reduce_kernel(const float* __restrict__ part, int ks, int64_t M, int R, int RP,
                                   uint16_t* __restrict__ out, int64_t ldo) {
  const int64_t n = M * R;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = i / R;
    const int q = (int)(i - m * R);
    float v = part[m * RP + q];
    for (int k = 1; k < ks; ++k) v += part[((int64_t)k * M + m) * RP + q];
    out[m * ldo + q] = bf16_bits(v);
  }
}

// ------------------------------------------------------------------------
// Gradient partials part[s][p][q] = sum over the s-th slice of M of
// L(m, p) R(m, q). Both operands are loaded as 8 x 8 patches (8 rows of M,
// 16 bytes each) and transposed in registers (v_perm) so that M, the
// contraction index, is contiguous in LDS. One-deep register prefetch; the
// splits are summed in split order afterwards.
// ------------------------------------------------------------------------
constexpr int GR_P = 128, GR_Q = 64, GR_NT = 256;
constexpr int GR_WROWS = 64, GR_WCOLS = 32;   // waves 2 (p) x 2 (q)

// L operand modes: 0 plain, 1 SwiGLU replay from (gate, up), 2 the frozen
// RMSNorm output bf16(fp32(x) * inv[m] * (fp32(w) + offset)) replayed from
// the norm's input x, its per-row inv and its weight.
constexpr int L_PLAIN = 0, L_REPLAY = 1, L_NORM = 2;

struct GradParams {
  const uint16_t* l; const uint16_t* l2; int64_t ldl; int mode;
  const uint16_t* rm; int64_t ldr;
  int64_t M, P, Q;
  int64_t slice;
  float* part;          // split partials [S][P][Q] (layout 0) or [S][Q][P] (layout 1)
  int layout;
  const float* inv; const void* nw; int nw_f32; float noff;   // L_NORM only
};

struct Patch {
  Chunk v[8];
  float inv[8];   // L_NORM: inv of each patch row
};

// (fp32(w) + offset) of the 8 columns a thread stages; 1 past the matrix.
MOLT_DEV void norm_weights(const GradParams& p, int64_t col, float (&wo)[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int64_t c = col + e < p.P ? col + e : 0;
    const float w = p.nw_f32 ? reinterpret_cast<const float*>(p.nw)[c]
                             : bf16_to_f32(reinterpret_cast<const uint16_t*>(p.nw)[c]);
    wo[e] = __fadd_rn(w, p.noff);
  }
}

// The norm's bf16 output for one loaded chunk, with the products and their
// order of the RMSNorm forward kernel: bf16((x * inv) * (w + offset)).
MOLT_DEV u32x4_t norm_value(const Chunk& c, float inv, const float (&wo)[8]) {
  u32x4_t o;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    o[e] = pack_bf16x2(__fmul_rn(__fmul_rn(bf16_lo(c.a[e]), inv), wo[2 * e]),
                       __fmul_rn(__fmul_rn(bf16_hi(c.a[e]), inv), wo[2 * e + 1]));
  const uint32_t keep = c.ok ? 0xffffffffu : 0u;
  return o & keep;
}

// Which operand and patch a thread stages: waves 0-1 stage the 8 x 16 L
// patches of a 64 x 128 tile, wave 2 the 8 x 8 R patches of a 64 x 64 tile,
// wave 3 none. Within a patch group, mg (the 8-row group) varies fastest so
// the transposed 16-byte LDS stores of neighbouring lanes land in one row.
MOLT_DEV bool patch_role(int wave, int lane, bool& is_l, int& mg, int& cg) {
  mg = lane & 7;
  cg = (lane >> 3) + (wave == 1 ? 8 : 0);
  is_l = wave < 2;
  return wave < 3;
}

template <bool VEC, int LM>
MOLT_DEV void patch_load(Patch& pt, const GradParams& p, int wave, int lane, int64_t m0, int64_t mend,
                         int64_t p0, int64_t q0) {
  constexpr bool REPLAY = LM == L_REPLAY;
  bool is_l; int mg, cg;
  if (!patch_role(wave, lane, is_l, mg, cg)) return;
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int64_t m = m0 + 8 * mg + r;
    if (is_l) {
      chunk_load<VEC, REPLAY>(pt.v[r], p.l, p.l2, p.ldl, p.mode, 1.0f, m, mend, p0 + 8 * cg, p.P);
      if constexpr (LM == L_NORM) pt.inv[r] = p.inv[m < mend ? m : 0];
    } else {
      chunk_load<VEC, false>(pt.v[r], p.rm, nullptr, p.ldr, 0, 1.0f, m, mend, q0 + 8 * cg, p.Q);
    }
  }
}

template <bool VEC, int LM>
MOLT_DEV void patch_store(const Patch& pt, const GradParams& p, const float (&wo)[8], uint16_t* ls, uint16_t* rs,
                          int wave, int lane) {
  constexpr bool REPLAY = LM == L_REPLAY;
  bool is_l; int mg, cg;
  if (!patch_role(wave, lane, is_l, mg, cg)) return;
  u32x4_t v[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    if constexpr (LM == L_NORM)
      v[r] = is_l ? norm_value(pt.v[r], pt.inv[r], wo) : chunk_value<VEC, false>(pt.v[r], 0, 1.0f);
    else
      v[r] = is_l ? chunk_value<VEC, REPLAY>(pt.v[r], p.mode, 1.0f) : chunk_value<VEC, false>(pt.v[r], 0, 1.0f);
  }
  uint16_t* dst = is_l ? ls : rs;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
    u32x4_t o;
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = __builtin_amdgcn_perm(v[2 * k + 1][c >> 1], v[2 * k][c >> 1], sel);
    *reinterpret_cast<u32x4_t*>(dst + (8 * cg + c) * LDSW + 8 * mg) = o;
  }
}

// acc[i][0] is C[p][q]: column q = lane % 32, rows p = 8(e/4) + 4(lane/32) + e%4.
// The partial is stored in the output's layout, so that the split sum is
// element-wise; in layout 1 a lane's four consecutive p are one 16-byte store.
// isub < 0: the wave's two 32-row subtiles acc[0], acc[1]; isub = 0 or 1:
// only acc[0], which holds subtile isub (the narrow-Q wave layout).
MOLT_DEV void grad_store_partial(const GradParams& p, const f32x16_t (&acc)[2][1], int64_t p0, int64_t q0, int wp,
                                 int wq, int lane, int64_t slice, int isub = -1) {
  float* out = p.part + slice * p.P * p.Q;
  const int64_t q = q0 + wq * GR_WCOLS + (lane & 31);
  if (q >= p.Q) return;
  const bool v4 = p.P % 4 == 0 && ((uintptr_t)out & 15) == 0;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      if (isub >= 0 && i > 0) break;
      const int64_t pp = p0 + wp * GR_WROWS + (isub >= 0 ? isub : i) * 32 + 8 * g + 4 * (lane >> 5);
      if (p.layout == 0) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (pp + e < p.P) out[(pp + e) * p.Q + q] = acc[i][0][4 * g + e];
      } else if (v4 && pp < p.P) {
        const f32x4_t v = {acc[i][0][4 * g], acc[i][0][4 * g + 1], acc[i][0][4 * g + 2], acc[i][0][4 * g + 3]};
        *reinterpret_cast<f32x4_t*>(out + q * p.P + pp) = v;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (pp + e < p.P) out[q * p.P + pp + e] = acc[i][0][4 * g + e];
      }
    }
}

template <bool VEC, int LM>
__global__ __launch_bounds__(GR_NT) void lora_grad_kernel(const GradParams p) {
  // One LDS tile (27 KB: three workgroups per CU) where the registers allow
  // three; the SwiGLU- and RMSNorm-replay variants, held to two by their
  // registers, double-buffer instead and save a barrier per step.
  constexpr int NB = LM == L_PLAIN ? 1 : 2;
  __shared__ __attribute__((aligned(16))) uint16_t ls[NB][GR_P * LDSW];
  __shared__ __attribute__((aligned(16))) uint16_t rs[NB][GR_Q * LDSW];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wp = wave & 1, wq = wave >> 1;
  const int64_t p0 = (int64_t)blockIdx.x * GR_P;
  const int64_t q0 = (int64_t)blockIdx.y * GR_Q;
  const int64_t mbeg = (int64_t)blockIdx.z * p.slice;
  const int64_t mend = mbeg + p.slice < p.M ? mbeg + p.slice : p.M;
  const int steps = (int)ceil_div64(mend - mbeg, BK);

  float wo[8] = {};
  if constexpr (LM == L_NORM) {
    bool is_l; int mg, cg;
    if (patch_role(wave, lane, is_l, mg, cg) && is_l) norm_weights(p, p0 + 8 * cg, wo);
  }
  f32x16_t acc[2][1];
  zero_acc(acc);
  // a replayed operand's rank tile of at most 32 columns: four 32-row P
  // subtiles over the same columns (wave w: rows 32 w ..), no wave on
  // columns past Q; uniform (plain L keeps the 2 x 2 layout, whose registers
  // allow three workgroups per CU)
  const bool nq = LM != L_PLAIN && p.Q - q0 <= GR_WCOLS;
  f32x16_t (&acc0)[1][1] = *reinterpret_cast<f32x16_t(*)[1][1]>(&acc[0]);
  Patch pt;
  patch_load<VEC, LM>(pt, p, wave, lane, mbeg, mend, p0, q0);
  patch_store<VEC, LM>(pt, p, wo, ls[0], rs[0], wave, lane);
  __syncthreads();
  if constexpr (NB == 2) {
    for (int s = 0; s < steps; ++s) {
      const int cur = s & 1;
      if (s + 1 < steps) patch_load<VEC, LM>(pt, p, wave, lane, mbeg + (int64_t)(s + 1) * BK, mend, p0, q0);
      if (nq) mfma_step<1, 1>(ls[cur], rs[cur], 32 * wave, 0, acc0, lane);
      else mfma_step<2, 1>(ls[cur], rs[cur], wp * GR_WROWS, wq * GR_WCOLS, acc, lane);
      if (s + 1 < steps) patch_store<VEC, LM>(pt, p, wo, ls[cur ^ 1], rs[cur ^ 1], wave, lane);
      __syncthreads();
    }
  } else {
    for (int s = 0; s < steps; ++s) {
      if (s + 1 < steps) patch_load<VEC, LM>(pt, p, wave, lane, mbeg + (int64_t)(s + 1) * BK, mend, p0, q0);
      if (nq) mfma_step<1, 1>(ls[0], rs[0], 32 * wave, 0, acc0, lane);
      else mfma_step<2, 1>(ls[0], rs[0], wp * GR_WROWS, wq * GR_WCOLS, acc, lane);
      if (s + 1 >= steps) break;
      __syncthreads();                               // the single tile is consumed
      patch_store<VEC, LM>(pt, p, wo, ls[0], rs[0], wave, lane);
      __syncthreads();
    }
  }

  if (nq) grad_store_partial(p, acc, p0, q0, wave >> 1, 0, lane, blockIdx.z, wave & 1);
  else grad_store_partial(p, acc, p0, q0, wp, wq, lane, blockIdx.z);
}

// ------------------------------------------------------------------------
// DMA-staged gradient (plain L, 16-byte aligned rows, P and Q multiples of 8):
// the L and R tiles of a 64-row step arrive by buffer-load DMA in their
// natural row layout, in a ring of three stages (two steps ahead), and the
// MFMA fragments, which need M contiguous per lane, are gathered from LDS by
// 16-bit reads (eight per fragment, into the halves of four registers). In a
// row with bit 3 of its index set, 16-byte chunk j sits at position j ^ 4, so
// that the two lane halves of a fragment read (rows 8 apart) fall on
// different banks. Rows past M lie outside the buffer resource and read as
// zero; columns past P or Q only feed outputs that are not stored. Same tiles,
// slices and MFMA operands as lora_grad_kernel: the result is bitwise its.
// ------------------------------------------------------------------------
constexpr int GD_LT = BK * GR_P, GD_RT = BK * GR_Q;   // elements of one stage's L and R tile

MOLT_DEV bf16x8_t gd_frag(const uint16_t* __restrict__ s, int base, int stride) {
  typedef unsigned short us2_t __attribute__((ext_vector_type(2)));
  u32x4_t v;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    us2_t t;
    t.x = s[base + 2 * e * stride];
    t.y = s[base + (2 * e + 1) * stride];
    v[e] = __builtin_bit_cast(uint32_t, t);
  }
  return __builtin_bit_cast(bf16x8_t, v);
}

// One workgroup of the DMA-staged gradient: P tile bx, Q tile by, M slice bz.
// Stages of GS_BK = 32 rows: the three-stage ring takes 36 KB of LDS, so four
// workgroups (16 waves) share a CU and hide each other's fragment gathers.
constexpr int GS_BK = 32, GS_LT = GS_BK * GR_P, GS_RT = GS_BK * GR_Q;
MOLT_DEV void grad_dma_tile(const GradParams& p, int bx, int by, int bz) {
  __shared__ __attribute__((aligned(16))) uint16_t la[GS_LT], lb[GS_LT], lc[GS_LT];
  __shared__ __attribute__((aligned(16))) uint16_t ra[GS_RT], rb[GS_RT], rc[GS_RT];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wp = wave & 1, wq = wave >> 1, h = lane >> 5;
  const int64_t p0 = (int64_t)bx * GR_P;
  const int64_t q0 = (int64_t)by * GR_Q;
  const int64_t mbeg = (int64_t)bz * p.slice;
  const int64_t mend = mbeg + p.slice < p.M ? mbeg + p.slice : p.M;
  const int steps = (int)ceil_div64(mend - mbeg, GS_BK);
  const __amdgpu_buffer_rsrc_t lr = pj_rsrc(p.l, ((p.M - 1) * p.ldl + p.P) * 2);
  const __amdgpu_buffer_rsrc_t rr = pj_rsrc(p.rm, ((p.M - 1) * p.ldr + p.Q) * 2);
  // DMA instruction c of L covers rows 4c .. 4c + 3 (16 lanes per 256-byte
  // row), of R rows 8c .. 8c + 7 (8 lanes per 128-byte row); a wave issues
  // L instructions 2 wave, 2 wave + 1 and R instruction wave.
  uint32_t loff[2], roff;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int r = 4 * (2 * wave + j) + (lane >> 4);
    const int ch = (lane & 15) ^ (4 * ((r >> 3) & 1));
    loff[j] = (uint32_t)((r * p.ldl + p0 + 8 * ch) * 2);
  }
  {
    const int r = 8 * wave + (lane >> 3);
    const int ch = (lane & 7) ^ (4 * ((r >> 3) & 1));
    roff = (uint32_t)((r * p.ldr + q0 + 8 * ch) * 2);
  }
  auto dma = [&](int s, uint16_t* ld, uint16_t* rd) {
    s = s < steps ? s : steps - 1;   // past the end: the last stage again, never read
    const int64_t m = mbeg + (int64_t)s * GS_BK;
    const uint32_t ls = __builtin_amdgcn_readfirstlane((uint32_t)(m * p.ldl * 2));
    const uint32_t rs = __builtin_amdgcn_readfirstlane((uint32_t)(m * p.ldr * 2));
#pragma unroll
    for (int j = 0; j < 2; ++j) pj_dma16(lr, ld + (2 * wave + j) * 512, loff[j], ls);
    pj_dma16(rr, rd + wave * 512, roff, rs);
  };
  // Narrow Q tile (at most 32 columns, e.g. rank 16): the four waves take a
  // 32-row P subtile each (wave w: rows 32 w ..) over the same 32 columns,
  // instead of two waves per column half with one half past Q. Each output
  // sums the same MFMA products in the same order either way.
  const bool nq = p.Q - q0 <= GR_WCOLS;
  // fragment bases (row 8 h of the step; sub-step kk adds 16 rows, element e one row)
  int abase[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int pl = (nq ? 32 * wave : wp * GR_WROWS + 32 * i) + (lane & 31);
    abase[i] = 8 * h * GR_P + (((pl >> 3) ^ (4 * h)) << 3) + (pl & 7);
  }
  const int ql = (nq ? 0 : wq * GR_WCOLS) + (lane & 31);
  const int bbase = 8 * h * GR_Q + (((ql >> 3) ^ (4 * h)) << 3) + (ql & 7);

  f32x16_t acc[2][1];
  zero_acc(acc);
  dma(0, la, ra);
  dma(1, lb, rb);
  pj_wait_vm<3>();                   // stage 0 landed; stage 1 may fly
  pj_barrier();
  int s = 0;
  // step s: stage s from (lcur, rcur); the DMA of stage s + 2 goes to the
  // buffers stage s - 1 used, which every wave left at the last barrier
  auto step = [&](const uint16_t* lcur, const uint16_t* rcur, uint16_t* lnn, uint16_t* rnn) {
    dma(s + 2, lnn, rnn);
#pragma unroll
    for (int kk = 0; kk < GS_BK / 16; ++kk) {
      const bf16x8_t a0 = gd_frag(lcur, abase[0] + 16 * kk * GR_P, GR_P);
      const bf16x8_t b0 = gd_frag(rcur, bbase + 16 * kk * GR_Q, GR_Q);
      acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0, acc[0][0], 0, 0, 0);
      if (!nq) {                     // uniform per workgroup
        const bf16x8_t a1 = gd_frag(lcur, abase[1] + 16 * kk * GR_P, GR_P);
        acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b0, acc[1][0], 0, 0, 0);
      }
    }
    pj_wait_vm<3>();                 // stage s + 1 landed; stage s + 2 may fly
    pj_barrier();
    return ++s < steps;
  };
  // (two rounds of the ring per iteration: the compiler adds a wait for the
  // DMA in flight at the loop head, which this makes one step in six)
  while (step(la, ra, lc, rc) && step(lb, rb, la, ra) && step(lc, rc, lb, rb) && step(la, ra, lc, rc) &&
         step(lb, rb, la, ra) && step(lc, rc, lb, rb)) {
  }
  pj_wait_vm<0>();                   // the repeated stages past the end
  if (nq) grad_store_partial(p, acc, p0, q0, wave >> 1, 0, lane, bz, wave & 1);
  else grad_store_partial(p, acc, p0, q0, wp, wq, lane, bz);
}

__global__ __launch_bounds__(GR_NT, 4) void lora_grad_dma_kernel(const GradParams p) {
  grad_dma_tile(p, (int)blockIdx.x, (int)blockIdx.y, (int)blockIdx.z);
}

// Several DMA-staged gradients in one launch (molt_lora_grad_many): the
// workgroups of gradient d are the flat range [first[d], first[d + 1]),
// ordered as its own launch's grid (P tiles fastest, then Q tiles, then M
// slices), so each gradient's tiles, slices and partials are those of its
// own launch.
constexpr int kGradMany = 8;
struct GradMany {
  GradParams g[kGradMany];
  int first[kGradMany + 1];
  int gx[kGradMany], gy[kGradMany];
  int n;
};

__global__ __launch_bounds__(GR_NT, 4) void lora_grad_dma_many_kernel(const GradMany m) {
  const int b = (int)blockIdx.x;
  int d = 0;
#pragma unroll
  for (int i = 1; i < kGradMany; ++i) d += (i < m.n && b >= m.first[i]) ? 1 : 0;
  d = __builtin_amdgcn_readfirstlane(d);
  const int local = b - m.first[d], gx = m.gx[d], gy = m.gy[d];
  grad_dma_tile(m.g[d], local % gx, (local / gx) % gy, local / (gx * gy));
}

// SwiGLU-replay L = bf16(bf16(silu(g)) u) (ztrans mode 1, the forward's h)
// gathered from the g and u tiles: the fragment of gd_frag, formed per element.
MOLT_DEV bf16x8_t gd_frag_replay(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u, int base,
                                 int stride) {
  u32x4_t v;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int o0 = base + 2 * e * stride, o1 = o0 + stride;
    const float h0 = ztrans(bf16_to_f32(g[o0]), bf16_to_f32(u[o0]), 1, 1.0f);
    const float h1 = ztrans(bf16_to_f32(g[o1]), bf16_to_f32(u[o1]), 1, 1.0f);
    v[e] = pack_bf16x2(h0, h1);
  }
  return __builtin_bit_cast(bf16x8_t, v);
}

// The DMA-staged gradient with the SwiGLU-replayed L: g and u tiles arrive
// like the plain kernel's L tile (same slots and chunk order), in a ring of
// two stages (one step ahead: three stages of g, u and R would leave room for
// one workgroup per CU), and each fragment element is replayed as it is
// gathered. Same tiles, slices and MFMA operands as the other gradient
// kernels: bitwise the gradient of the materialised h.
// NQ: the narrow-Q wave layout of grad_dma_tile (Q <= 32, one column tile),
// which also forms each replayed h element once instead of twice.
template <bool NQ>
__global__ __launch_bounds__(GR_NT, 2) void lora_grad_dma_replay_kernel(const GradParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t ga[GD_LT], gb[GD_LT], ua[GD_LT], ub[GD_LT];
  __shared__ __attribute__((aligned(16))) uint16_t ra[GD_RT], rb[GD_RT];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wp = wave & 1, wq = wave >> 1, h = lane >> 5;
  const int64_t p0 = (int64_t)blockIdx.x * GR_P;
  const int64_t q0 = (int64_t)blockIdx.y * GR_Q;
  const int64_t mbeg = (int64_t)blockIdx.z * p.slice;
  const int64_t mend = mbeg + p.slice < p.M ? mbeg + p.slice : p.M;
  const int steps = (int)ceil_div64(mend - mbeg, BK);
  const int64_t lbytes = ((p.M - 1) * p.ldl + p.P) * 2;
  const __amdgpu_buffer_rsrc_t gr = pj_rsrc(p.l, lbytes), ur = pj_rsrc(p.l2, lbytes);
  const __amdgpu_buffer_rsrc_t rr = pj_rsrc(p.rm, ((p.M - 1) * p.ldr + p.Q) * 2);
  uint32_t loff[4], roff[2];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 4 * (4 * wave + j) + (lane >> 4);
    const int ch = (lane & 15) ^ (4 * ((r >> 3) & 1));
    loff[j] = (uint32_t)((r * p.ldl + p0 + 8 * ch) * 2);
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int r = 8 * (2 * wave + j) + (lane >> 3);
    const int ch = (lane & 7) ^ (4 * ((r >> 3) & 1));
    roff[j] = (uint32_t)((r * p.ldr + q0 + 8 * ch) * 2);
  }
  auto dma = [&](int s, uint16_t* gd, uint16_t* ud, uint16_t* rd) {
    s = s < steps ? s : steps - 1;   // past the end: the last stage again, never read
    const int64_t m = mbeg + (int64_t)s * BK;
    const uint32_t ls = __builtin_amdgcn_readfirstlane((uint32_t)(m * p.ldl * 2));
    const uint32_t rs = __builtin_amdgcn_readfirstlane((uint32_t)(m * p.ldr * 2));
#pragma unroll
    for (int j = 0; j < 4; ++j) pj_dma16(gr, gd + (4 * wave + j) * 512, loff[j], ls);
#pragma unroll
    for (int j = 0; j < 4; ++j) pj_dma16(ur, ud + (4 * wave + j) * 512, loff[j], ls);
#pragma unroll
    for (int j = 0; j < 2; ++j) pj_dma16(rr, rd + (2 * wave + j) * 512, roff[j], rs);
  };
  int abase[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int pl = (NQ ? 32 * wave : wp * GR_WROWS + 32 * i) + (lane & 31);
    abase[i] = 8 * h * GR_P + (((pl >> 3) ^ (4 * h)) << 3) + (pl & 7);
  }
  const int ql = (NQ ? 0 : wq * GR_WCOLS) + (lane & 31);
  const int bbase = 8 * h * GR_Q + (((ql >> 3) ^ (4 * h)) << 3) + (ql & 7);

  f32x16_t acc[2][1];
  zero_acc(acc);
  dma(0, ga, ua, ra);
  pj_wait_vm<0>();
  pj_barrier();
  int s = 0;
  // step s: stage s from the current buffers; stage s + 1 goes to the others,
  // which every wave left at the last barrier
  auto step = [&](const uint16_t* gc, const uint16_t* uc, const uint16_t* rc, uint16_t* gn, uint16_t* un,
                  uint16_t* rn) {
    dma(s + 1, gn, un, rn);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const bf16x8_t a0 = gd_frag_replay(gc, uc, abase[0] + 16 * kk * GR_P, GR_P);
      const bf16x8_t b0 = gd_frag(rc, bbase + 16 * kk * GR_Q, GR_Q);
      acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0, acc[0][0], 0, 0, 0);
      if constexpr (!NQ) {
        const bf16x8_t a1 = gd_frag_replay(gc, uc, abase[1] + 16 * kk * GR_P, GR_P);
        acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b0, acc[1][0], 0, 0, 0);
      }
    }
    pj_wait_vm<0>();                 // stage s + 1 landed
    pj_barrier();
    return ++s < steps;
  };
  while (step(ga, ua, ra, gb, ub, rb) && step(gb, ub, rb, ga, ua, ra)) {
  }
  if (NQ) grad_store_partial(p, acc, p0, q0, wave >> 1, 0, lane, blockIdx.z, wave & 1);
  else grad_store_partial(p, acc, p0, q0, wp, wq, lane, blockIdx.z);
}

__global__ void zero_fill_kernel(float* __restrict__ out, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    out[i] = 0.0f;
}

// Sum of the S split partials (stored in the output's layout) in split order,
// times scale: element-wise, four floats per thread with vec4 (n % 4 == 0,
// 16-byte aligned partials and output). The loads of up to 8 partials are
// issued before their in-order sum, so a thread waits once per 8 partials.
__global__ void lora_grad_reduce_kernel(const float* __restrict__ part, int S, int64_t n, float scale,
                                        float* __restrict__ out, int vec4) {
  if (vec4) {
    const int64_t n4 = n / 4;
    const f32x4_t* p4 = reinterpret_cast<const f32x4_t*>(part);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x) {
      f32x4_t s = {0.0f, 0.0f, 0.0f, 0.0f};
      int k = 0;
      for (; k + 8 <= S; k += 8) {
        f32x4_t v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = p4[(int64_t)(k + u) * n4 + i];
#pragma unroll
        for (int u = 0; u < 8; ++u) s += v[u];
      }
      for (; k < S; ++k) s += p4[(int64_t)k * n4 + i];
      reinterpret_cast<f32x4_t*>(out)[i] = s * scale;
    }
    return;
  }
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    float s = 0.0f;
    for (int k = 0; k < S; ++k) s += part[(int64_t)k * n + i];
    out[i] = s * scale;
  }
}

// The split sums of several gradients in one launch: items of gradient d
// (elements, or 4-element groups with vec4) are the flat range
// [first[d], first[d + 1]); each is summed as lora_grad_reduce_kernel does.
struct ReduceMany {
  const float* part[kGradMany];
  float* out[kGradMany];
  int64_t n[kGradMany];
  int64_t first[kGradMany + 1];
  float scale[kGradMany];
  int S[kGradMany], vec4[kGradMany];
  int cnt;
};

__global__ void lora_grad_reduce_many_kernel(const ReduceMany r) {
  const int64_t total = r.first[r.cnt];
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    int d = 0;
#pragma unroll
    for (int k = 1; k < kGradMany; ++k) d += (k < r.cnt && i >= r.first[k]) ? 1 : 0;
    const int64_t j = i - r.first[d];
    const float* part = r.part[d];
    const int S = r.S[d];
    if (r.vec4[d]) {
      const int64_t n4 = r.n[d] / 4;
      const f32x4_t* p4 = reinterpret_cast<const f32x4_t*>(part);
      f32x4_t s4 = {0.0f, 0.0f, 0.0f, 0.0f};
      int k = 0;
      for (; k + 8 <= S; k += 8) {
        f32x4_t v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = p4[(int64_t)(k + u) * n4 + j];
#pragma unroll
        for (int u = 0; u < 8; ++u) s4 += v[u];
      }
      for (; k < S; ++k) s4 += p4[(int64_t)k * n4 + j];
      reinterpret_cast<f32x4_t*>(r.out[d])[j] = s4 * r.scale[d];
    } else {
      float a = 0.0f;
      for (int k = 0; k < S; ++k) a += part[(int64_t)k * r.n[d] + j];
      r.out[d][j] = a * r.scale[d];
    }
  }
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// M slices of a gradient launch: as many as keep every workgroup resident at
// once (two per CU: the DMA kernel's LDS ring, the replay variants'
// registers), so no partial second round of workgroups trails the first
// (measured: 50 -> 46 us for the dB over dg at cfg4). The count must not depend on
// the L operand's mode: the slices fix the fp32 summation order, and the
// replayed and normalised operands must give bitwise the gradient of the
// materialised one.
int grad_splits(int64_t M, int64_t P, int64_t Q) {
  const int64_t tiles = ceil_div64(P, GR_P) * ceil_div64(Q, GR_Q);
  int64_t s = 2 * (int64_t)molt::device_cus() / tiles;
  const int64_t max_s = ceil_div64(M, 256);    // keep >= 256 rows per split
  if (s > max_s) s = max_s;
  if (s < 1) s = 1;
  if (s > 64) s = 64;
  return (int)s;
}

int64_t proj_tq(int r) { return (r + 31) / 32; }

}  // namespace
}  // namespace molt

using namespace molt;

// Row tiles per workgroup: two 32-row tiles halve the L2 reads of the packed
// adapter (ranks <= 64 only: larger accumulator sets would not fit in
// registers). K split: the steps are split two or four ways (at least 16
// steps per range) until there is a workgroup for every CU.
int proj_mt(int64_t M, int tq, bool vec, int z_mode) {
  return (vec && z_mode != 1 && M >= 256 * 64 && tq <= 2) ? 2 : 1;
}

int proj_ksplit(int64_t M, int64_t D, int mt, int operands = 1) {
  const int64_t tiles = operands * ceil_div64(M, 32 * mt), steps = ceil_div64(D, BK);
  int ks = 1;
  while (ks < 4 && tiles * ks < 256 && steps / (2 * ks) >= 16) ks *= 2;
  return ks;
}

size_t proj_packed_bytes(int64_t D, int32_t r) {
  return (size_t)ceil_div64(D, BK) * (size_t)proj_tq(r) * 4 * 64 * 8 * sizeof(uint16_t);
}

extern "C" size_t molt_lora_project_workspace(int64_t M, int64_t D, int32_t r) {
  if (D <= 0 || r <= 0 || M < 0) return 0;
  const int ks = proj_ksplit(M, D, proj_mt(M, (int)proj_tq(r), true, 0));
  const size_t part = ks > 1 ? (size_t)ks * (size_t)M * (size_t)(32 * proj_tq(r)) * sizeof(float) : 0;
  return proj_packed_bytes(D, r) + part;
}

static int launch_projection(const uint16_t* z, const uint16_t* z2, int64_t ldz, int32_t z_mode, float z_scale,
                             int64_t M, int64_t D, const uint16_t* wp, int32_t r, uint16_t* out, int64_t ldo,
                             void* part, hipStream_t st, const char* who);

extern "C" int molt_lora_project(const uint16_t* z, const uint16_t* z2, int64_t ldz, int32_t z_mode, float z_scale,
                                 int64_t M, int64_t D, const float* lora, int32_t lora_layout, int32_t r,
                                 uint16_t* out, int64_t ldo, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  const char* who = "molt_lora_project";
  MOLT_REQUIRE(z_mode >= 0 && z_mode <= 2, MOLT_EINVAL, "%s: bad z_mode %d", who, z_mode);
  MOLT_REQUIRE(lora_layout == 0 || lora_layout == 1, MOLT_EINVAL, "%s: bad lora_layout", who);
  MOLT_REQUIRE(M >= 0 && D > 0 && r > 0, MOLT_EINVAL, "%s: bad shape M=%lld D=%lld r=%d", who, (long long)M,
               (long long)D, r);
  MOLT_REQUIRE(r <= 32 * PJ_TQ_MAX, MOLT_EUNSUPPORTED, "%s: rank %d > %d", who, r, 32 * PJ_TQ_MAX);
  if (M == 0) return MOLT_OK;
  MOLT_REQUIRE(z && lora && out && ldz >= D && ldo >= r, MOLT_EINVAL, "%s: bad pointers/strides", who);
  MOLT_REQUIRE(z_mode != 1 || z2, MOLT_EINVAL, "%s: SwiGLU replay needs the up tensor", who);
  const size_t need = molt_lora_project_workspace(M, D, r);
  MOLT_REQUIRE(workspace && workspace_bytes >= need && aligned(workspace, 16), MOLT_EWORKSPACE,
               "%s: workspace %zu < %zu bytes (or not 16-byte aligned)", who, workspace_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  const int tq = (int)proj_tq(r);
  const int64_t steps = ceil_div64(D, BK);
  const int64_t frags = steps * tq * 4 * 64;
  unsigned pblocks = (unsigned)((frags + 255) / 256);
  if (pblocks > 4096) pblocks = 4096;
  uint16_t* wp = (uint16_t*)workspace;
  hipLaunchKernelGGL(lora_pack_kernel, dim3(pblocks), dim3(256), 0, st, lora, lora_layout, r, D, tq, steps, wp);
  int rc = check_launch(who);
  if (rc) return rc;
  return launch_projection(z, z2, ldz, z_mode, z_scale, M, D, wp, r, out, ldo,
                           (char*)workspace + proj_packed_bytes(D, r), st, who);
}

extern "C" size_t molt_lora_packed_bytes(int64_t D, int32_t r) {
  return D > 0 && r > 0 ? proj_packed_bytes(D, r) : 0;
}

extern "C" int molt_lora_pack_many(int32_t n, const molt_lora_pack_desc* d, void* stream) {
  const char* who = "molt_lora_pack_many";
  MOLT_REQUIRE(d && n >= 1 && n <= kPackMany, MOLT_EINVAL, "%s: 1..%d adapters", who, kPackMany);
  PackMany m{};
  int64_t total = 0;
  for (int i = 0; i < n; ++i) {
    const molt_lora_pack_desc& a = d[i];
    MOLT_REQUIRE(a.D > 0 && a.r > 0 && a.r <= 32 * PJ_TQ_MAX, MOLT_EINVAL, "%s: bad shape (adapter %d)", who, i);
    MOLT_REQUIRE(a.layout == 0 || a.layout == 1, MOLT_EINVAL, "%s: bad layout (adapter %d)", who, i);
    MOLT_REQUIRE(a.lora && a.packed && aligned(a.packed, 16), MOLT_EINVAL, "%s: null or unaligned (adapter %d)",
                 who, i);
    MOLT_REQUIRE(a.lora2 ? (a.split > 0 && a.split < a.r) : a.split == a.r, MOLT_EINVAL,
                 "%s: bad split (adapter %d)", who, i);
    m.w0[i] = a.lora; m.w1[i] = a.lora2 ? a.lora2 : a.lora; m.wp[i] = a.packed;
    m.D[i] = a.D; m.steps[i] = ceil_div64(a.D, BK); m.split[i] = a.split; m.R[i] = a.r;
    m.tq[i] = (int)proj_tq(a.r); m.layout[i] = a.layout;
    m.first[i] = total;
    total += m.steps[i] * m.tq[i] * 4 * 64;
  }
  m.first[n] = total;
  m.n = n;
  unsigned blocks = (unsigned)((total + 255) / 256);
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(lora_pack_many_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, m);
  return check_launch(who);
}

// ---------------------------------------------------------------------------
// Adapters of several projections that share one input, stacked for one
// projection node over their stacked weights: A_stack [lr, K] = [A_0; A_1; ..;
// zero rows] and B_blocks [N, lr] block-diagonal (rows of B_i in columns
// i r .. i r + r - 1, zeros elsewhere), both fp32. Four consecutive elements
// per thread: K and lr are multiples of 4, so the four never cross a row of
// A_stack nor a block of B_blocks.
constexpr int kStackMax = 8;
struct StackAdapters {
  const float* a[kStackMax];
  const float* b[kStackMax];
  int64_t n0[kStackMax + 1];                          // first row of each B block; n0[n] = N
  int n, r, lr;
  int64_t K;
  float* a_stack;
  float* b_blocks;
};

__global__ __launch_bounds__(256) void lora_stack_adapters_kernel(const StackAdapters p) {
  const int64_t na = (int64_t)p.lr * p.K, nb = p.n0[p.n] * p.lr;
  const int64_t e = 4 * ((int64_t)blockIdx.x * blockDim.x + threadIdx.x);
  if (e >= na + nb) return;
  f32x4_t v = {0.f, 0.f, 0.f, 0.f};
  if (e < na) {
    const int64_t j = e / p.K, k = e - j * p.K;
    const int i = (int)(j / p.r);
    if (i < p.n) {
      const float* src = p.a[i] + (j - (int64_t)i * p.r) * p.K + k;
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = src[q];
    }
    *reinterpret_cast<f32x4_t*>(p.a_stack + e) = v;
  } else {
    const int64_t f = e - na, row = f / p.lr;
    const int c = (int)(f - row * p.lr), i = c / p.r;
    if (i < p.n && row >= p.n0[i] && row < p.n0[i + 1]) {
      const float* src = p.b[i] + (row - p.n0[i]) * p.r + (c - i * p.r);
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = src[q];
    }
    *reinterpret_cast<f32x4_t*>(p.b_blocks + f) = v;
  }
}

extern "C" int molt_lora_stack_adapters(int32_t n, const float* const* a, const float* const* b,
                                        const int64_t* rows, int32_t r, int64_t K, int32_t lr, float* a_stack,
                                        float* b_blocks, void* stream) {
  const char* who = "molt_lora_stack_adapters";
  MOLT_REQUIRE(n >= 1 && n <= kStackMax && a && b && rows, MOLT_EINVAL, "%s: 1..%d adapters", who, kStackMax);
  MOLT_REQUIRE(r > 0 && r % 4 == 0 && lr % 4 == 0 && (int64_t)n * r <= lr && K > 0 && K % 4 == 0, MOLT_EINVAL,
               "%s: needs r and lr multiples of 4, n r <= lr and K a multiple of 4 (n=%d r=%d lr=%d K=%lld)", who,
               n, r, lr, (long long)K);
  MOLT_REQUIRE(a_stack && b_blocks && aligned(a_stack, 16) && aligned(b_blocks, 16), MOLT_EINVAL,
               "%s: outputs must be 16-byte aligned", who);
  StackAdapters p{};
  p.n = n; p.r = r; p.lr = lr; p.K = K; p.a_stack = a_stack; p.b_blocks = b_blocks;
  int64_t n0 = 0;
  for (int i = 0; i < n; ++i) {
    MOLT_REQUIRE(a[i] && b[i] && rows[i] > 0, MOLT_EINVAL, "%s: adapter %d missing or empty", who, i);
    p.a[i] = a[i]; p.b[i] = b[i]; p.n0[i] = n0;
    n0 += rows[i];
  }
  p.n0[n] = n0;
  const int64_t quads = ((int64_t)lr * K + n0 * lr) / 4;
  hipLaunchKernelGGL(lora_stack_adapters_kernel, dim3((unsigned)ceil_div64(quads, 256)), dim3(256), 0,
                     (hipStream_t)stream, p);
  return check_launch(who);
}

extern "C" size_t molt_lora_project_packed_workspace(int64_t M, int64_t D, int32_t r) {
  if (D <= 0 || r <= 0 || M < 0) return 0;
  return molt_lora_project_workspace(M, D, r) - proj_packed_bytes(D, r);
}

extern "C" int molt_lora_project_packed(const uint16_t* z, const uint16_t* z2, int64_t ldz, int32_t z_mode,
                                        float z_scale, int64_t M, int64_t D, const uint16_t* packed, int32_t r,
                                        uint16_t* out, int64_t ldo, void* workspace, size_t workspace_bytes,
                                        void* stream) {
  const char* who = "molt_lora_project_packed";
  MOLT_REQUIRE(z_mode >= 0 && z_mode <= 2, MOLT_EINVAL, "%s: bad z_mode %d", who, z_mode);
  MOLT_REQUIRE(M >= 0 && D > 0 && r > 0, MOLT_EINVAL, "%s: bad shape M=%lld D=%lld r=%d", who, (long long)M,
               (long long)D, r);
  MOLT_REQUIRE(r <= 32 * PJ_TQ_MAX, MOLT_EUNSUPPORTED, "%s: rank %d > %d", who, r, 32 * PJ_TQ_MAX);
  if (M == 0) return MOLT_OK;
  MOLT_REQUIRE(z && packed && aligned(packed, 16) && out && ldz >= D && ldo >= r, MOLT_EINVAL,
               "%s: bad pointers/strides", who);
  MOLT_REQUIRE(z_mode != 1 || z2, MOLT_EINVAL, "%s: SwiGLU replay needs the up tensor", who);
  const size_t need = molt_lora_project_packed_workspace(M, D, r);
  MOLT_REQUIRE(need == 0 || (workspace && workspace_bytes >= need && aligned(workspace, 16)), MOLT_EWORKSPACE,
               "%s: workspace %zu < %zu bytes (or not 16-byte aligned)", who, workspace_bytes, need);
  return launch_projection(z, z2, ldz, z_mode, z_scale, M, D, packed, r, out, ldo, workspace, (hipStream_t)stream,
                           who);
}

// Two projections of one shape over adapters already packed, as one launch
// of the DMA kernel with gridDim.z = 2 (blockIdx.z picks the operand): the
// split count counts both operands' row blocks, so a pair that fills the CUs
// together runs unsplit. Same tiles, split ranges and summation order per
// operand as its own launch with that split count. Returns MOLT_EUNSUPPORTED
// (nothing launched) where the DMA kernel does not apply.
static int launch_projection_pair(const uint16_t* z0, const uint16_t* z1, int64_t ldz, int32_t z_mode, float zs0,
                                  float zs1, int64_t M, int64_t D, const uint16_t* wp0, const uint16_t* wp1,
                                  int32_t r, uint16_t* out0, uint16_t* out1, int64_t ldo, void* part,
                                  hipStream_t st, const char* who) {
  const int tq = (int)proj_tq(r);
  const bool dma = z_mode != 1 && D % BK == 0 && ldz % 8 == 0 && aligned(z0, 16) && aligned(z1, 16) &&
                   molt::tuning_value(MOLT_TUNE_LORA_DMA) != 0 && ((M - 1) * ldz + D) * 2 < ((int64_t)1 << 31);
  if (!dma) return MOLT_EUNSUPPORTED;
  ProjParams p{};
  p.z = z0; p.ldz = ldz; p.mode = z_mode; p.zs = zs0;
  p.M = M; p.D = D; p.R = r; p.wp = wp0; p.out = out0; p.ldo = ldo;
  p.zb = z1; p.wpb = wp1; p.zsb = zs1; p.outb = out1;
  const int mt = proj_mt(M, tq, true, z_mode);
  const int ks = proj_ksplit(M, D, mt, 2);
  const size_t plane = (size_t)ks * (size_t)M * (size_t)(32 * tq);
  p.part = ks > 1 ? static_cast<float*>(part) : nullptr;
  p.partb = ks > 1 ? static_cast<float*>(part) + plane : nullptr;
  dim3 grid((unsigned)ceil_div64(M, 32 * mt), (unsigned)ks, 2u), block(64 * PJ_WAVES);
#define MOLT_PJD(TQ, MT)                                                                                       \
  do {                                                                                                         \
    if (ks == 4) hipLaunchKernelGGL((lora_project_dma_kernel<TQ, MT, 4>), grid, block, 0, st, p);               \
    else if (ks == 2) hipLaunchKernelGGL((lora_project_dma_kernel<TQ, MT, 2>), grid, block, 0, st, p);          \
    else hipLaunchKernelGGL((lora_project_dma_kernel<TQ, MT, 1>), grid, block, 0, st, p);                       \
  } while (0)
  switch (tq * 2 + mt - 1) {
    case 2: MOLT_PJD(1, 1); break;
    case 3: MOLT_PJD(1, 2); break;
    case 4: MOLT_PJD(2, 1); break;
    case 5: MOLT_PJD(2, 2); break;
    case 6: MOLT_PJD(3, 1); break;
    default: MOLT_PJD(4, 1); break;
  }
#undef MOLT_PJD
  if (ks > 1) {
    int rc = check_launch(who);
    if (rc) return rc;
    int64_t rb = ceil_div64(M * r, 256);
    if (rb > 4096) rb = 4096;
    hipLaunchKernelGGL(proj_reduce_kernel, dim3((unsigned)rb), dim3(256), 0, st, p.part, ks, M, r, 32 * tq, out0, ldo);
    rc = check_launch(who);
    if (rc) return rc;
    hipLaunchKernelGGL(proj_reduce_kernel, dim3((unsigned)rb), dim3(256), 0, st, p.partb, ks, M, r, 32 * tq, out1,
                       ldo);
  }
  return check_launch(who);
}

// Enough for the pair launch and for the two separate projections it falls
// back to (operands the DMA kernel does not take).
extern "C" size_t molt_lora_project_pair_packed_workspace(int64_t M, int64_t D, int32_t r) {
  if (D <= 0 || r <= 0 || M < 0) return 0;
  const int ks = proj_ksplit(M, D, proj_mt(M, (int)proj_tq(r), true, 0), 2);
  const size_t pair = ks > 1 ? 2 * (size_t)ks * (size_t)M * (size_t)(32 * proj_tq(r)) * sizeof(float) : 0;
  return std::max(pair, molt_lora_project_packed_workspace(M, D, r));
}

extern "C" int molt_lora_project_pair_packed(const uint16_t* z0, const uint16_t* z1, int64_t ldz, int32_t z_mode,
                                             float z_scale0, float z_scale1, int64_t M, int64_t D,
                                             const uint16_t* packed0, const uint16_t* packed1, int32_t r,
                                             uint16_t* out, int64_t ldo, void* workspace, size_t workspace_bytes,
                                             void* stream) {
  const char* who = "molt_lora_project_pair_packed";
  MOLT_REQUIRE(z_mode == 0 || z_mode == 2, MOLT_EINVAL, "%s: bad z_mode %d (0 or 2)", who, z_mode);
  MOLT_REQUIRE(M >= 0 && D > 0 && r > 0, MOLT_EINVAL, "%s: bad shape M=%lld D=%lld r=%d", who, (long long)M,
               (long long)D, r);
  MOLT_REQUIRE(r <= 32 * PJ_TQ_MAX, MOLT_EUNSUPPORTED, "%s: rank %d > %d", who, r, 32 * PJ_TQ_MAX);
  if (M == 0) return MOLT_OK;
  MOLT_REQUIRE(z0 && z1 && packed0 && packed1 && aligned(packed0, 16) && aligned(packed1, 16) && out && ldz >= D &&
               ldo >= 2 * r, MOLT_EINVAL, "%s: bad pointers/strides", who);
  hipStream_t st = (hipStream_t)stream;
  const size_t need = molt_lora_project_pair_packed_workspace(M, D, r);
  const bool room = need == 0 || (workspace && workspace_bytes >= need && aligned(workspace, 16));
  if (room) {
    const int rc = launch_projection_pair(z0, z1, ldz, z_mode, z_scale0, z_scale1, M, D, packed0, packed1, r, out,
                                          out + r, ldo, workspace, st, who);
    if (rc != MOLT_EUNSUPPORTED) return rc;
  }
  // operands the pair launch does not take: one projection each (their own
  // split counts), with the workspace their larger need asks for
  const size_t one = molt_lora_project_packed_workspace(M, D, r);
  MOLT_REQUIRE(one == 0 || (workspace && workspace_bytes >= one && aligned(workspace, 16)), MOLT_EWORKSPACE,
               "%s: workspace %zu < %zu bytes (or not 16-byte aligned)", who, workspace_bytes, one);
  int rc = launch_projection(z0, nullptr, ldz, z_mode, z_scale0, M, D, packed0, r, out, ldo, workspace, st, who);
  if (rc) return rc;
  return launch_projection(z1, nullptr, ldz, z_mode, z_scale1, M, D, packed1, r, out + r, ldo, workspace, st, who);
}

// The projection kernel(s) over an adapter already packed at wp (split
// partials, if any, at part); shared by molt_lora_project and
// molt_lora_project_packed.
static int launch_projection(const uint16_t* z, const uint16_t* z2, int64_t ldz, int32_t z_mode, float z_scale,
                             int64_t M, int64_t D, const uint16_t* wp, int32_t r, uint16_t* out, int64_t ldo,
                             void* part, hipStream_t st, const char* who) {
  int rc = MOLT_OK;
  const int tq = (int)proj_tq(r);
  ProjParams p{};
  p.z = z; p.z2 = z2; p.ldz = ldz; p.mode = z_mode; p.zs = z_scale;
  p.M = M; p.D = D; p.R = r; p.wp = wp; p.out = out; p.ldo = ldo;
  p.part = (float*)part;
  const bool vec = D % 8 == 0 && ldz % 8 == 0 && aligned(z, 16) && (z_mode != 1 || aligned(z2, 16));
  const int mt = proj_mt(M, tq, vec, z_mode);
  const int ks = vec ? proj_ksplit(M, D, mt) : 1;
  dim3 grid((unsigned)ceil_div64(M, 32 * mt), (unsigned)ks), block(64 * PJ_WAVES);
#define MOLT_PJK(TQ, MT, VEC, REPLAY, KS) \
  hipLaunchKernelGGL((lora_project_kernel<TQ, MT, VEC, REPLAY, KS>), grid, block, 0, st, p)
#define MOLT_PJ(TQ, MT, VEC, REPLAY)                        \
  do {                                                      \
    if (ks == 4) MOLT_PJK(TQ, MT, VEC, REPLAY, 4);          \
    else if (ks == 2) MOLT_PJK(TQ, MT, VEC, REPLAY, 2);     \
    else MOLT_PJK(TQ, MT, VEC, REPLAY, 1);                  \
  } while (0)
  // (the DMA kernel addresses z through a buffer resource: 32-bit byte offsets)
  const bool dma = vec && z_mode != 1 && D % BK == 0 && molt::tuning_value(MOLT_TUNE_LORA_DMA) != 0 &&
                   ((M - 1) * ldz + D) * 2 < ((int64_t)1 << 31);
#define MOLT_PJD(TQ, MT)                                                                                       \
  do {                                                                                                         \
    if (ks == 4) hipLaunchKernelGGL((lora_project_dma_kernel<TQ, MT, 4>), grid, block, 0, st, p);               \
    else if (ks == 2) hipLaunchKernelGGL((lora_project_dma_kernel<TQ, MT, 2>), grid, block, 0, st, p);          \
    else hipLaunchKernelGGL((lora_project_dma_kernel<TQ, MT, 1>), grid, block, 0, st, p);                       \
  } while (0)
  if (dma) {
    switch (tq * 2 + mt - 1) {
      case 2: MOLT_PJD(1, 1); break;
      case 3: MOLT_PJD(1, 2); break;
      case 4: MOLT_PJD(2, 1); break;
      case 5: MOLT_PJD(2, 2); break;
      case 6: MOLT_PJD(3, 1); break;
      default: MOLT_PJD(4, 1); break;
    }
  } else if (!vec) {
    switch (tq) {
      case 1: MOLT_PJ(1, 1, false, false); break;
      case 2: MOLT_PJ(2, 1, false, false); break;
      case 3: MOLT_PJ(3, 1, false, false); break;
      default: MOLT_PJ(4, 1, false, false); break;
    }
  } else if (z_mode == 1) {
    switch (tq) {
      case 1: MOLT_PJ(1, 1, true, true); break;
      case 2: MOLT_PJ(2, 1, true, true); break;
      case 3: MOLT_PJ(3, 1, true, true); break;
      default: MOLT_PJ(4, 1, true, true); break;
    }
  } else {
    switch (tq * 2 + mt - 1) {
      case 2: MOLT_PJ(1, 1, true, false); break;
      case 3: MOLT_PJ(1, 2, true, false); break;
      case 4: MOLT_PJ(2, 1, true, false); break;
      case 5: MOLT_PJ(2, 2, true, false); break;
      case 6: MOLT_PJ(3, 1, true, false); break;
      default: MOLT_PJ(4, 1, true, false); break;
    }
  }
#undef MOLT_PJ
#undef MOLT_PJK
#undef MOLT_PJD
  if (ks > 1) {
    rc = check_launch(who);
    if (rc) return rc;
    int64_t rb = ceil_div64(M * r, 256);
    if (rb > 4096) rb = 4096;
    hipLaunchKernelGGL(proj_reduce_kernel, dim3((unsigned)rb), dim3(256), 0, st, p.part, ks, M, r, 32 * tq, out, ldo);
  }
  return check_launch(who);
}

extern "C" size_t molt_lora_grad_workspace(int64_t M, int64_t P, int64_t Q) {
  if (M <= 0 || P <= 0 || Q <= 0) return 0;
  return (size_t)grad_splits(M, P, Q) * (size_t)P * (size_t)Q * sizeof(float);
}

// M slices of one gradient (the rows each takes); returns their count.
static int grad_slices(GradParams& p) {
  const int S = grad_splits(p.M, p.P, p.Q);
  p.slice = ceil_div64(ceil_div64(p.M, S), BK) * BK;
  return (int)ceil_div64(p.M, p.slice);
}

// The gradient kernel of one gradient (slices set by grad_slices, partials at
// p.part in p.layout), without the split sum.
static void grad_kernel_launch(const GradParams& p, bool vec, int lm, int S_eff, hipStream_t st) {
  const int64_t M = p.M, P = p.P, Q = p.Q;
  dim3 grid((unsigned)ceil_div64(P, GR_P), (unsigned)ceil_div64(Q, GR_Q), (unsigned)S_eff);
  // the DMA-staged kernel for plain aligned operands whose byte offsets fit the buffer resources
  const bool dma = vec && lm == L_PLAIN && molt::tuning_value(MOLT_TUNE_LORA_DMA) != 0 &&
                   ((M - 1) * p.ldl + P) * 2 < ((int64_t)1 << 31) && ((M - 1) * p.ldr + Q) * 2 < ((int64_t)1 << 31);
  const bool dma_replay = vec && lm == L_REPLAY && molt::tuning_value(MOLT_TUNE_LORA_DMA) != 0 &&
                          ((M - 1) * p.ldl + P) * 2 < ((int64_t)1 << 31) &&
                          ((M - 1) * p.ldr + Q) * 2 < ((int64_t)1 << 31);
  if (dma) hipLaunchKernelGGL(lora_grad_dma_kernel, grid, dim3(GR_NT), 0, st, p);
  else if (dma_replay && Q <= GR_WCOLS) hipLaunchKernelGGL(lora_grad_dma_replay_kernel<true>, grid, dim3(GR_NT), 0, st, p);
  else if (dma_replay) hipLaunchKernelGGL(lora_grad_dma_replay_kernel<false>, grid, dim3(GR_NT), 0, st, p);
  else if (!vec) hipLaunchKernelGGL((lora_grad_kernel<false, L_PLAIN>), grid, dim3(GR_NT), 0, st, p);
  else if (lm == L_REPLAY) hipLaunchKernelGGL((lora_grad_kernel<true, L_REPLAY>), grid, dim3(GR_NT), 0, st, p);
  else if (lm == L_NORM) hipLaunchKernelGGL((lora_grad_kernel<true, L_NORM>), grid, dim3(GR_NT), 0, st, p);
  else hipLaunchKernelGGL((lora_grad_kernel<true, L_PLAIN>), grid, dim3(GR_NT), 0, st, p);
}

// Split over M, launch the gradient kernel and sum the splits (shared by
// molt_lora_grad and molt_lora_grad_rmsnorm; p carries the operands).
static int launch_grad(GradParams& p, bool vec, int lm, float scale, float* out, int32_t out_layout,
                       void* workspace, size_t workspace_bytes, hipStream_t st, const char* who) {
  const int64_t P = p.P, Q = p.Q;
  const size_t need = (size_t)grad_splits(p.M, P, Q) * P * Q * sizeof(float);
  MOLT_REQUIRE(workspace && workspace_bytes >= need, MOLT_EWORKSPACE, "%s: workspace %zu < %zu bytes", who,
               workspace_bytes, need);
  p.part = (float*)workspace;
  p.layout = out_layout;
  const int S_eff = grad_slices(p);
  grad_kernel_launch(p, vec, lm, S_eff, st);
  int rc = check_launch(who);
  if (rc) return rc;
  const int64_t n = P * Q;
  const int vec4 = n % 4 == 0 && aligned(p.part, 16) && aligned(out, 16);
  const int64_t items = vec4 ? n / 4 : n;
  unsigned blocks = (unsigned)((items + 255) / 256);
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(lora_grad_reduce_kernel, dim3(blocks), dim3(256), 0, st, p.part, S_eff, n, scale, out, vec4);
  return check_launch(who);
}

// M == 0: the gradient is zero. A fill kernel rather than hipMemsetAsync, so
// that the call stays correct when a caller captures it into a HIP graph.
static int zero_grad(float* out, int64_t P, int64_t Q, hipStream_t st, const char* who) {
  const int64_t n = P * Q;
  const unsigned blocks = (unsigned)(n / 256 + 1 < 4096 ? n / 256 + 1 : 4096);
  hipLaunchKernelGGL(zero_fill_kernel, dim3(blocks), dim3(256), 0, st, out, n);
  return check_launch(who);
}

extern "C" int molt_lora_grad(const uint16_t* l, const uint16_t* l2, int64_t ldl, int32_t l_mode,
                              const uint16_t* rmat, int64_t ldr, int64_t M, int64_t P, int64_t Q, float scale,
                              float* out, int32_t out_layout, void* workspace, size_t workspace_bytes,
                              void* stream) {
  const char* who = "molt_lora_grad";
  MOLT_REQUIRE(l_mode == 0 || l_mode == 1, MOLT_EINVAL, "%s: bad l_mode", who);
  MOLT_REQUIRE(out_layout == 0 || out_layout == 1, MOLT_EINVAL, "%s: bad out_layout", who);
  MOLT_REQUIRE(M >= 0 && P > 0 && Q > 0, MOLT_EINVAL, "%s: bad shape", who);
  MOLT_REQUIRE(out && ldl >= P && ldr >= Q, MOLT_EINVAL, "%s: bad pointers/strides", who);
  hipStream_t st = (hipStream_t)stream;
  if (M == 0) return zero_grad(out, P, Q, st, who);
  MOLT_REQUIRE(l && rmat, MOLT_EINVAL, "%s: null operand", who);
  MOLT_REQUIRE(l_mode == 0 || l2, MOLT_EINVAL, "%s: SwiGLU replay needs the up tensor", who);
  GradParams p{};
  p.l = l; p.l2 = l2; p.ldl = ldl; p.mode = l_mode; p.rm = rmat; p.ldr = ldr;
  p.M = M; p.P = P; p.Q = Q;
  const bool vec = P % 8 == 0 && Q % 8 == 0 && ldl % 8 == 0 && ldr % 8 == 0 && aligned(l, 16) &&
                   aligned(rmat, 16) && (l_mode == 0 || aligned(l2, 16));
  return launch_grad(p, vec, l_mode, scale, out, out_layout, workspace, workspace_bytes, st, who);
}

// Several gradients and one launch that sums all their splits: each output
// is bitwise that of its own molt_lora_grad (l_mode 0, 1) or
// molt_lora_grad_rmsnorm (l_mode 2) call (same kernel, tiles, slices, partials
// and summation order). The gradients eligible for the DMA-staged plain
// kernel share one launch; each other one takes its own kernel launch.
static size_t grad_ws_bytes(int64_t M, int64_t P, int64_t Q) {
  return M > 0 ? ((size_t)grad_splits(M, P, Q) * (size_t)P * (size_t)Q * sizeof(float) + 255) / 256 * 256 : 0;
}

extern "C" size_t molt_lora_grad_many_workspace(int32_t n, const molt_lora_grad_desc* d) {
  if (n < 1 || n > kGradMany || !d) return 0;
  size_t b = 0;
  for (int i = 0; i < n; ++i)
    if (d[i].P > 0 && d[i].Q > 0) b += grad_ws_bytes(d[i].M, d[i].P, d[i].Q);
  return b;
}

extern "C" int molt_lora_grad_many(int32_t n, const molt_lora_grad_desc* d, void* workspace, size_t workspace_bytes,
                                   void* stream) {
  const char* who = "molt_lora_grad_many";
  MOLT_REQUIRE(d && n >= 1 && n <= kGradMany, MOLT_EINVAL, "%s: 1..%d gradients", who, kGradMany);
  hipStream_t st = (hipStream_t)stream;
  size_t off = 0;
  GradParams ps[kGradMany];
  bool vecs[kGradMany], batched[kGradMany];
  for (int i = 0; i < n; ++i) {
    const molt_lora_grad_desc& g = d[i];
    MOLT_REQUIRE(g.l_mode >= 0 && g.l_mode <= 2, MOLT_EINVAL, "%s: bad l_mode (gradient %d)", who, i);
    MOLT_REQUIRE(g.out_layout == 0 || g.out_layout == 1, MOLT_EINVAL, "%s: bad out_layout (gradient %d)", who, i);
    MOLT_REQUIRE(g.M >= 0 && g.P > 0 && g.Q > 0, MOLT_EINVAL, "%s: bad shape (gradient %d)", who, i);
    MOLT_REQUIRE(g.out && g.ldl >= g.P && g.ldr >= g.Q, MOLT_EINVAL, "%s: bad pointers/strides (gradient %d)", who, i);
    MOLT_REQUIRE(g.M == 0 || (g.l && g.rmat && (g.l_mode != 1 || g.l2)), MOLT_EINVAL,
                 "%s: null operand (gradient %d)", who, i);
    const bool vec = g.P % 8 == 0 && g.Q % 8 == 0 && g.ldl % 8 == 0 && g.ldr % 8 == 0 && aligned(g.l, 16) &&
                     aligned(g.rmat, 16) && (g.l_mode != 1 || aligned(g.l2, 16));
    if (g.l_mode == 2) {
      MOLT_REQUIRE(g.w_dtype == MOLT_DTYPE_BF16 || g.w_dtype == MOLT_DTYPE_F32, MOLT_EINVAL,
                   "%s: norm weight dtype must be bf16 or fp32 (gradient %d)", who, i);
      MOLT_REQUIRE(g.M == 0 || (g.inv_rms && g.norm_weight), MOLT_EINVAL, "%s: null norm operand (gradient %d)",
                   who, i);
      MOLT_REQUIRE(g.M == 0 || vec, MOLT_EUNSUPPORTED,
                   "%s: the RMSNorm replay needs 16-byte aligned rows and P, Q multiples of 8 (gradient %d)", who, i);
    }
    GradParams& p = ps[i];
    p = GradParams{};
    p.l = g.l; p.l2 = g.l_mode == 1 ? g.l2 : nullptr; p.ldl = g.ldl; p.mode = g.l_mode; p.rm = g.rmat; p.ldr = g.ldr;
    p.M = g.M; p.P = g.P; p.Q = g.Q; p.layout = g.out_layout;
    if (g.l_mode == 2) {
      p.inv = g.inv_rms; p.nw = g.norm_weight; p.nw_f32 = g.w_dtype == MOLT_DTYPE_F32; p.noff = g.norm_offset;
    }
    p.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + off);
    off += grad_ws_bytes(g.M, g.P, g.Q);
    vecs[i] = vec;
    // plain aligned operands whose byte offsets fit the buffer resources share the DMA launch
    batched[i] = g.M > 0 && vec && g.l_mode == 0 && molt::tuning_value(MOLT_TUNE_LORA_DMA) != 0 &&
                 ((g.M - 1) * g.ldl + g.P) * 2 < ((int64_t)1 << 31) &&
                 ((g.M - 1) * g.ldr + g.Q) * 2 < ((int64_t)1 << 31);
  }
  MOLT_REQUIRE(workspace ? workspace_bytes >= off && aligned(workspace, 256) : off == 0, MOLT_EWORKSPACE,
               "%s: workspace %zu < %zu bytes (or not 256-byte aligned)", who, workspace_bytes, off);
  GradMany gm{};
  ReduceMany rm{};
  int blocks = 0;
  int64_t items = 0;
  int rc;
  for (int i = 0; i < n; ++i) {
    GradParams& p = ps[i];
    if (p.M == 0) {   // nothing to sum: the gradient is zero
      rc = zero_grad(d[i].out, p.P, p.Q, st, who);
      if (rc) return rc;
      continue;
    }
    const int S_eff = grad_slices(p);
    if (batched[i]) {
      const int k = gm.n++;
      gm.g[k] = p;
      gm.gx[k] = (int)ceil_div64(p.P, GR_P);
      gm.gy[k] = (int)ceil_div64(p.Q, GR_Q);
      gm.first[k] = blocks;
      MOLT_REQUIRE((int64_t)blocks + (int64_t)gm.gx[k] * gm.gy[k] * S_eff < (1ll << 31), MOLT_EINVAL,
                   "%s: problem too large", who);
      blocks += gm.gx[k] * gm.gy[k] * S_eff;
    } else {
      grad_kernel_launch(p, vecs[i], p.mode, S_eff, st);
      rc = check_launch(who);
      if (rc) return rc;
    }
    const int k = rm.cnt++;
    const int64_t nel = p.P * p.Q;
    rm.part[k] = p.part; rm.out[k] = d[i].out; rm.n[k] = nel; rm.scale[k] = d[i].scale; rm.S[k] = S_eff;
    rm.vec4[k] = nel % 4 == 0 && aligned(p.part, 16) && aligned(d[i].out, 16);
    rm.first[k] = items;
    items += rm.vec4[k] ? nel / 4 : nel;
  }
  if (gm.n) {
    gm.first[gm.n] = blocks;
    hipLaunchKernelGGL(lora_grad_dma_many_kernel, dim3((unsigned)blocks), dim3(GR_NT), 0, st, gm);
    rc = check_launch(who);
    if (rc) return rc;
  }
  if (rm.cnt == 0) return MOLT_OK;
  rm.first[rm.cnt] = items;
  int64_t rb = ceil_div64(items, 256);
  if (rb > 4096) rb = 4096;
  hipLaunchKernelGGL(lora_grad_reduce_many_kernel, dim3((unsigned)rb), dim3(256), 0, st, rm);
  return check_launch(who);
}

extern "C" int molt_lora_grad_rmsnorm(const uint16_t* x, int64_t ldx, const float* inv_rms, const void* norm_weight,
                                      int32_t w_dtype, float offset, const uint16_t* rmat, int64_t ldr, int64_t M,
                                      int64_t P, int64_t Q, float scale, float* out, int32_t out_layout,
                                      void* workspace, size_t workspace_bytes, void* stream) {
  const char* who = "molt_lora_grad_rmsnorm";
  MOLT_REQUIRE(w_dtype == MOLT_DTYPE_BF16 || w_dtype == MOLT_DTYPE_F32, MOLT_EINVAL,
               "%s: norm weight dtype must be bf16 or fp32", who);
  MOLT_REQUIRE(out_layout == 0 || out_layout == 1, MOLT_EINVAL, "%s: bad out_layout", who);
  MOLT_REQUIRE(M >= 0 && P > 0 && Q > 0, MOLT_EINVAL, "%s: bad shape", who);
  MOLT_REQUIRE(out && ldx >= P && ldr >= Q, MOLT_EINVAL, "%s: bad pointers/strides", who);
  hipStream_t st = (hipStream_t)stream;
  if (M == 0) return zero_grad(out, P, Q, st, who);
  MOLT_REQUIRE(x && inv_rms && norm_weight && rmat, MOLT_EINVAL, "%s: null operand", who);
  MOLT_REQUIRE(P % 8 == 0 && Q % 8 == 0 && ldx % 8 == 0 && ldr % 8 == 0 && aligned(x, 16) && aligned(rmat, 16),
               MOLT_EUNSUPPORTED, "%s: needs 16-byte aligned rows and P, Q multiples of 8", who);
  GradParams p{};
  p.l = x; p.ldl = ldx; p.mode = L_NORM; p.rm = rmat; p.ldr = ldr;
  p.M = M; p.P = P; p.Q = Q;
  p.inv = inv_rms; p.nw = norm_weight; p.nw_f32 = w_dtype == MOLT_DTYPE_F32; p.noff = offset;
  return launch_grad(p, true, L_NORM, scale, out, out_layout, workspace, workspace_bytes, st, who);
}
