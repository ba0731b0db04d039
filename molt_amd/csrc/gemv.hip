// Skinny-M (M <= 16) NF4 GEMV with the rank-r LoRA add-on (gfx950), HBM-bound.
//
// Y[m, n] = sum_b scale(n, b) * sum_{k in block b} X[m, k] * code[W(n, k)]
//           + sum_j T[m, j] * bf16(s * B[n, j])
//
// v_mfma_f32_16x16x32_bf16 with X as the 16-row operand (rows >= M are zero)
// and the NF4 codes as the 16-column operand. Lane group g = lane/16 owns the
// contiguous 16 elements [64b + 16g, +16) of block b (8 packed bytes, one
// 8-byte load per row), split over two 32-deep MFMAs, so each MFMA pair sums
// exactly one block and the block scale is applied once to its 16x16 result
// instead of to every weight. Codes come from a 256-entry LDS table of bf16
// code pairs indexed by the packed byte (the nibble order is folded into the
// table), so a byte costs one byte-select and one LDS read.
//
// A workgroup owns 16 rows and the whole of K: its 8 waves take contiguous
// eighths of K, keep 8 blocks of loads in flight each, and are summed in
// wave order through LDS. There is no cross-workgroup reduction, so no
// device-scope fence (an L2 write-back per workgroup) is ever needed.
#include "common.h"

namespace molt {
namespace {

constexpr int GV_WAVES = 8;
constexpr int GV_NT = 64 * GV_WAVES;
constexpr int GV_ROWS = 16;     // rows per workgroup (one MFMA column tile)
constexpr int GV_U = 8;         // blocks per wave kept in flight

typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));

struct GemvParams {
  const uint16_t* x; int64_t ldx; int M;
  const uint8_t* packed; int64_t N; int K;
  const float* scales;                                   // resolved, or null when nested
  const uint8_t* q; const float* absmax2; const float* code2; float offset; int dq_shift;
  const float* code; int order;
  const uint16_t* t; int64_t ldt; const float* lb; int r; float s;
  uint16_t* y; int64_t ldy;
};

MOLT_DEV float gv_scale(const GemvParams& p, const float* code2s, int64_t blk) {
#pragma clang fp contract(off)
  if (p.scales) return p.scales[blk];
  const float prod = code2s[p.q[blk]] * p.absmax2[blk >> p.dq_shift];
  return prod + p.offset;
}

__global__ __launch_bounds__(GV_NT) void nf4_gemv_kernel(const GemvParams p) {
  __shared__ uint32_t tab[256];
  __shared__ float code2s[256];
  __shared__ f32x4_t red[GV_WAVES - 1][64];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid < 256) {
    const int hi = tid >> 4, lo = tid & 15;
    tab[tid] = pack_bf16x2(p.code[p.order ? hi : lo], p.code[p.order ? lo : hi]);
    code2s[tid] = p.code2 ? p.code2[tid] : 0.0f;
  }
  __syncthreads();

  const int col = lane & 15, g = lane >> 4;
  const int64_t n = (int64_t)blockIdx.x * GV_ROWS + col;
  const bool rowok = n < p.N;
  const bool mrow = col < p.M;             // A-operand row m = lane % 16
  const int KB = p.K >> 6;
  const int b0 = wave * KB / GV_WAVES, b1 = (wave + 1) * KB / GV_WAVES;
  const uint8_t* wrow = p.packed + (rowok ? n : 0) * (int64_t)(p.K >> 1) + 8 * g;
  const uint16_t* xrow = p.x + (int64_t)col * p.ldx + 16 * g;
  const int64_t blk0 = (rowok ? n : 0) * (int64_t)KB;

  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int b = b0; b < b1; b += GV_U) {
    u32x2_t wq[GV_U];
    u32x4_t xa[GV_U], xb[GV_U];
    float sc[GV_U];
#pragma unroll
    for (int u = 0; u < GV_U; ++u) {
      const int bb = b + u;
      const bool ok = bb < b1;
      wq[u] = u32x2_t{0u, 0u};
      xa[u] = u32x4_t{0u, 0u, 0u, 0u};
      xb[u] = u32x4_t{0u, 0u, 0u, 0u};
      sc[u] = 0.0f;
      if (ok && rowok) {
        wq[u] = *reinterpret_cast<const u32x2_t*>(wrow + 32 * bb);
        sc[u] = gv_scale(p, code2s, blk0 + bb);
      }
      if (ok && mrow) {
        xa[u] = *reinterpret_cast<const u32x4_t*>(xrow + 64 * bb);
        xb[u] = *reinterpret_cast<const u32x4_t*>(xrow + 64 * bb + 8);
      }
    }
#pragma unroll
    for (int u = 0; u < GV_U; ++u) {
      u32x4_t w0, w1;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        w0[j] = tab[(wq[u][0] >> (8 * j)) & 0xffu];
        w1[j] = tab[(wq[u][1] >> (8 * j)) & 0xffu];
      }
      f32x4_t tmp = {0.f, 0.f, 0.f, 0.f};
      tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8v, xa[u]),
                                                    __builtin_bit_cast(bf16x8v, w0), tmp, 0, 0, 0);
      tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8v, xb[u]),
                                                    __builtin_bit_cast(bf16x8v, w1), tmp, 0, 0, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] += sc[u] * tmp[e];
    }
  }

  if (wave > 0) red[wave - 1][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < GV_WAVES - 1; ++w) acc += red[w][lane];

  // acc[e] is C[m][n] with m = 4 (lane / 16) + e.
  if (!rowok) return;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int m = 4 * g + e;
    if (m >= p.M) continue;
    float v = acc[e];
    for (int j = 0; j < p.r; ++j)
      v += bf16_to_f32(p.t[(int64_t)m * p.ldt + j]) * round_bf16(p.s * p.lb[n * p.r + j]);
    p.y[(int64_t)m * p.ldy + n] = bf16_bits(v);
  }
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

}  // namespace
}  // namespace molt

using namespace molt;

extern "C" size_t molt_nf4_gemv_workspace(int64_t M, int64_t N, int64_t K) {
  (void)M; (void)N; (void)K;
  return 0;   // the kernel needs no workspace; the argument is kept for callers
}

extern "C" int molt_nf4_gemv(const uint16_t* x, int64_t ldx, int64_t M, const molt_nf4_weight* w,
                             const uint16_t* t, int64_t ldt, const float* lora_b, int32_t r, float scaling,
                             uint16_t* y, int64_t ldy, void* workspace, size_t workspace_bytes,
                             void* stream) {
  (void)workspace; (void)workspace_bytes;
  const char* who = "molt_nf4_gemv";
  MOLT_REQUIRE(w && w->packed && w->code && x && y, MOLT_EINVAL, "%s: null argument", who);
  MOLT_REQUIRE(M >= 1 && M <= 16, MOLT_EUNSUPPORTED, "%s: M=%lld outside 1..16", who, (long long)M);
  MOLT_REQUIRE(w->block_size == 64 && w->cols % 64 == 0, MOLT_EUNSUPPORTED,
               "%s: needs block_size 64 and cols %% 64 == 0", who);
  MOLT_REQUIRE(w->cols < (1ll << 30), MOLT_EUNSUPPORTED, "%s: cols too large", who);
  MOLT_REQUIRE(w->rows > 0 && ldx >= w->cols && ldy >= w->rows, MOLT_EINVAL, "%s: bad shape/stride", who);
  MOLT_REQUIRE(ldx % 8 == 0 && aligned(x, 16) && aligned(w->packed, 8), MOLT_EINVAL,
               "%s: X rows must be 16-byte aligned and packed data 8-byte aligned", who);
  MOLT_REQUIRE(r >= 0 && (r == 0 || (t && lora_b && ldt >= r)), MOLT_EINVAL, "%s: bad LoRA operands", who);
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
  const int64_t grid = ceil_div64(p.N, GV_ROWS);
  MOLT_REQUIRE(grid < (1ll << 31), MOLT_EINVAL, "%s: problem too large", who);
  hipLaunchKernelGGL(nf4_gemv_kernel, dim3((unsigned)grid), dim3(GV_NT), 0, (hipStream_t)stream, p);
  return check_launch(who);
}
