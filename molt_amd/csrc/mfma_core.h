// MFMA tile loop shared by the NF4 GEMM and the LoRA reduction kernels (gfx950).
//
// Operand staging convention: every kernel stages both operands of a
// contraction step into LDS as bf16 rows of BK contraction elements
// (row stride LDSW elements, padded by 16 B so 8 consecutive rows fall on
// distinct bank groups for ds_read_b128). The MFMA is v_mfma_f32_32x32x16_bf16:
// lane l supplies row (l % 32) and contraction elements [8*(l/32), +8) of
// each operand; the 32x32 fp32 result lives as 16 values per lane with
// column (l % 32) and rows 8*(i/4) + 4*(l/32) + (i%4), i = 0..15.
#pragma once

#include "common.h"

namespace molt {

constexpr int BK = 64;          // contraction elements per pipeline step
constexpr int LDSW = BK + 8;    // LDS row stride in bf16 elements (144 B)

// acc[i][j] += A_rows[arow0 + 32 i .. +32] x B_rows[brow0 + 32 j .. +32]^T over one BK step.
template <int TM, int TN>
MOLT_DEV void mfma_step(const uint16_t* __restrict__ As, const uint16_t* __restrict__ Bs,
                        int arow0, int brow0, f32x16_t (&acc)[TM][TN], int lane) {
  const int r = lane & 31;
  const int kq = (lane >> 5) * 8;
#pragma unroll
  for (int kk = 0; kk < BK; kk += 16) {
    bf16x8_t a[TM], b[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
      a[i] = *reinterpret_cast<const bf16x8_t*>(As + (arow0 + i * 32 + r) * LDSW + kk + kq);
#pragma unroll
    for (int j = 0; j < TN; ++j)
      b[j] = *reinterpret_cast<const bf16x8_t*>(Bs + (brow0 + j * 32 + r) * LDSW + kk + kq);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
  }
}

template <int TM, int TN>
MOLT_DEV void zero_acc(f32x16_t (&acc)[TM][TN]) {
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
}

// Byte -> (first, second) fp32 code pair. `order` 1 = element 2i in the high
// nibble (bitsandbytes), 0 = element 2i in the low nibble (MOLT NF4Tensor).
MOLT_DEV void build_pair_table(float2* tab, const float* __restrict__ code, int order) {
  for (int b = threadIdx.x; b < 256; b += blockDim.x) {
    const int hi = b >> 4, lo = b & 15;
    const int first = order ? hi : lo;
    const int second = order ? lo : hi;
    tab[b] = make_float2(code[first], code[second]);
  }
}

// Nibble of flat element f of a packed NF4 stream.
MOLT_DEV int nf4_nibble(const uint8_t* __restrict__ packed, int64_t f, int order) {
  const int byte = packed[f >> 1];
  const bool first = (f & 1) == 0;
  return (first == (order != 0)) ? (byte >> 4) : (byte & 15);
}

// XCD-aware tile id: the dispatcher places consecutive workgroups on XCD
// (b % 8); give each XCD a contiguous range of tiles so neighbouring tiles
// (which share operand rows) meet in the same L2.
MOLT_DEV int64_t xcd_tile(int64_t b, int64_t T) {
  const int64_t q = T / 8, rmd = T % 8;
  const int64_t xcd = b % 8, local = b / 8;
  return xcd < rmd ? xcd * (q + 1) + local : rmd * (q + 1) + (xcd - rmd) * q + local;
}

// Grouped ordering inside the XCD range: GM m-tiles advance fastest.
MOLT_DEV void grouped_tile(int64_t t, int64_t nt_m, int64_t nt_n, int GM, int64_t& tm, int64_t& tn) {
  const int64_t per_group = (int64_t)GM * nt_n;
  const int64_t group = t / per_group;
  const int64_t first_m = group * GM;
  const int64_t gsize = (nt_m - first_m) < GM ? (nt_m - first_m) : GM;
  const int64_t in_group = t % per_group;
  tm = first_m + in_group % gsize;
  tn = in_group / gsize;
}

}  // namespace molt
