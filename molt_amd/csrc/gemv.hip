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
// table). A workgroup (4 waves) owns 64 rows and one K-split; its waves
// interleave the split's blocks and are summed in wave order through LDS.
// K-splits meet in a caller workspace: the last workgroup of a row tile (an
// atomic counter) sums the split partials in split order, adds the LoRA term,
// rounds once to bf16 and resets the counter to zero.
#include "common.h"

namespace molt {
namespace {

constexpr int GV_NT = 256;
constexpr int GV_ROWS = 64;     // rows per workgroup (4 MFMA column tiles of 16)
constexpr int GV_WAVES = 4;

typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));

struct GemvParams {
  const uint16_t* x; int64_t ldx; int M;
  const uint8_t* packed; int64_t N, K;
  const float* scales;                                  // resolved, or null when nested
  const uint8_t* q; const float* absmax2; const float* code2; float offset; int dq;
  const float* code; int order;
  const uint16_t* t; int64_t ldt; const float* lb; int r; float s;
  uint16_t* y; int64_t ldy;
  int splits;
  unsigned* counters; float* partial;                  // [splits][M][N]
};

MOLT_DEV uint32_t lut4(const uint32_t* tab, uint32_t w, int j) {
  return tab[(w >> (8 * j)) & 0xffu];
}

MOLT_DEV float gv_scale(const GemvParams& p, const float* code2s, int64_t blk) {
  if (p.scales) return p.scales[blk];
  return __fadd_rn(__fmul_rn(code2s[p.q[blk]], p.absmax2[blk / p.dq]), p.offset);
}

__global__ __launch_bounds__(GV_NT) void nf4_gemv_kernel(const GemvParams p) {
  __shared__ uint32_t tab[256];
  __shared__ float code2s[256];
  __shared__ float red[GV_WAVES - 1][4][4][64];
  __shared__ float tile[16][GV_ROWS];
  __shared__ unsigned last_flag;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  {
    const int b = tid;  // 256 threads build the two 256-entry tables
    const int hi = b >> 4, lo = b & 15;
    const float first = p.code[p.order ? hi : lo];
    const float second = p.code[p.order ? lo : hi];
    tab[b] = pack_bf16x2(first, second);
    code2s[b] = p.code2 ? p.code2[b] : 0.0f;
  }
  __syncthreads();

  const int64_t ntile = blockIdx.x / p.splits;
  const int split = blockIdx.x % p.splits;
  const int64_t n0 = ntile * GV_ROWS;
  const int64_t KB = p.K / 64;
  const int64_t b_beg = split * KB / p.splits, b_end = (split + 1) * KB / p.splits;

  const int col = lane & 15, g = lane >> 4;
  const bool mrow = col < p.M;   // A-operand row m = lane % 16
  const uint16_t* xrow = p.x + (int64_t)col * p.ldx + 16 * g;

  f32x4_t acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  int64_t rowoff[4];
  bool rowok[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t n = n0 + 16 * i + col;
    rowok[i] = n < p.N;
    rowoff[i] = (rowok[i] ? n : 0) * (p.K / 2) + 8 * g;
  }

  for (int64_t b = b_beg + wave; b < b_end; b += GV_WAVES) {
    u32x4_t xa = {0u, 0u, 0u, 0u}, xb = {0u, 0u, 0u, 0u};
    if (mrow) {
      xa = *reinterpret_cast<const u32x4_t*>(xrow + 64 * b);
      xb = *reinterpret_cast<const u32x4_t*>(xrow + 64 * b + 8);
    }
    const bf16x8v xf0 = __builtin_bit_cast(bf16x8v, xa);
    const bf16x8v xf1 = __builtin_bit_cast(bf16x8v, xb);
    u32x2_t wq[4];
    float sc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      wq[i] = rowok[i] ? *reinterpret_cast<const u32x2_t*>(p.packed + rowoff[i] + 32 * b) : u32x2_t{0u, 0u};
      const int64_t n = n0 + 16 * i + col;
      sc[i] = rowok[i] ? gv_scale(p, code2s, n * KB + b) : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      u32x4_t w0, w1;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        w0[j] = lut4(tab, wq[i][0], j);
        w1[j] = lut4(tab, wq[i][1], j);
      }
      f32x4_t tmp = {0.f, 0.f, 0.f, 0.f};
      tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf0, __builtin_bit_cast(bf16x8v, w0), tmp, 0, 0, 0);
      tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf1, __builtin_bit_cast(bf16x8v, w1), tmp, 0, 0, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[i][e] += sc[i] * tmp[e];
    }
  }

  // Sum the four waves in wave order. acc[i][e] is C[m][n] with
  // n = n0 + 16 i + lane % 16 and m = 4 (lane / 16) + e.
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) red[wave - 1][i][e][lane] = acc[i][e];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int w = 0; w < GV_WAVES - 1; ++w)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[i][e] += red[w][i][e][lane];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) tile[4 * g + e][16 * i + col] = acc[i][e];
  }
  __syncthreads();

  // tile[m][c] holds this split's partial for row n0 + c.
  if (p.splits > 1) {
    for (int idx = tid; idx < 16 * GV_ROWS; idx += GV_NT) {
      const int m = idx / GV_ROWS, c = idx % GV_ROWS;
      const int64_t n = n0 + c;
      if (m < p.M && n < p.N) p.partial[((int64_t)split * p.M + m) * p.N + n] = tile[m][c];
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) last_flag = atomicAdd(&p.counters[ntile], 1u) == (unsigned)(p.splits - 1);
    __syncthreads();
    if (!last_flag) return;
    __threadfence();
  }

  for (int idx = tid; idx < 16 * GV_ROWS; idx += GV_NT) {
    const int m = idx / GV_ROWS, c = idx % GV_ROWS;
    const int64_t n = n0 + c;
    if (m >= p.M || n >= p.N) continue;
    float v;
    if (p.splits > 1) {
      v = 0.0f;
      for (int s = 0; s < p.splits; ++s) v += p.partial[((int64_t)s * p.M + m) * p.N + n];
    } else {
      v = tile[m][c];
    }
    for (int j = 0; j < p.r; ++j)
      v += bf16_to_f32(p.t[(int64_t)m * p.ldt + j]) * round_bf16(p.s * p.lb[n * p.r + j]);
    p.y[(int64_t)m * p.ldy + n] = bf16_bits(v);
  }
  if (p.splits > 1 && tid == 0) p.counters[ntile] = 0u;
}

int gemv_splits(int64_t N, int64_t K) {
  const int64_t tiles = ceil_div64(N, GV_ROWS);
  const int64_t kb = K / 64;
  int64_t s = (512 + tiles - 1) / tiles;        // ~512 workgroups (2 per CU)
  const int64_t max_s = kb / GV_WAVES > 0 ? kb / GV_WAVES : 1;   // >= 1 block per wave
  if (s > max_s) s = max_s;
  if (s > 64) s = 64;
  if (s < 1) s = 1;
  return (int)s;
}

size_t counter_bytes(int64_t N) { return (size_t)ceil_div64(ceil_div64(N, GV_ROWS) * 4, 256) * 256; }

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

}  // namespace
}  // namespace molt

using namespace molt;

extern "C" size_t molt_nf4_gemv_workspace(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  const int s = gemv_splits(N, K);
  if (s == 1) return 0;
  return counter_bytes(N) + (size_t)s * M * N * sizeof(float);
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
  MOLT_REQUIRE(w->rows > 0 && ldx >= w->cols && ldy >= w->rows, MOLT_EINVAL, "%s: bad shape/stride", who);
  MOLT_REQUIRE(ldx % 8 == 0 && aligned(x, 16) && aligned(w->packed, 8), MOLT_EINVAL,
               "%s: X rows must be 16-byte aligned and packed data 8-byte aligned", who);
  MOLT_REQUIRE(r >= 0 && (r == 0 || (t && lora_b && ldt >= r)), MOLT_EINVAL, "%s: bad LoRA operands", who);
  const bool nested = w->nested != 0;
  MOLT_REQUIRE(nested ? (w->absmax_q && w->absmax2 && w->code2 && w->dq_block > 0) : (w->scales != nullptr),
               MOLT_EINVAL, "%s: scale statistics missing", who);
  GemvParams p{};
  p.x = x; p.ldx = ldx; p.M = (int)M; p.packed = w->packed; p.N = w->rows; p.K = w->cols;
  p.scales = nested ? nullptr : w->scales;
  p.q = w->absmax_q; p.absmax2 = w->absmax2; p.code2 = nested ? w->code2 : nullptr; p.offset = w->offset;
  p.dq = w->dq_block > 0 ? w->dq_block : 1;
  p.code = w->code; p.order = w->nibble_order;
  p.t = t; p.ldt = ldt; p.lb = lora_b; p.r = r; p.s = scaling; p.y = y; p.ldy = ldy;
  p.splits = gemv_splits(p.N, p.K);
  if (p.splits > 1) {
    const size_t cb = counter_bytes(p.N);
    const size_t need = cb + (size_t)p.splits * M * p.N * sizeof(float);
    MOLT_REQUIRE(workspace && workspace_bytes >= need && aligned(workspace, 256), MOLT_EWORKSPACE,
                 "%s: workspace %zu < %zu bytes (or not 256-byte aligned)", who, workspace_bytes, need);
    p.counters = (unsigned*)workspace;
    p.partial = (float*)((char*)workspace + cb);
  }
  const int64_t grid = ceil_div64(p.N, GV_ROWS) * p.splits;
  MOLT_REQUIRE(grid < (1ll << 31), MOLT_EINVAL, "%s: problem too large", who);
  hipLaunchKernelGGL(nf4_gemv_kernel, dim3((unsigned)grid), dim3(GV_NT), 0, (hipStream_t)stream, p);
  return check_launch(who);
}
