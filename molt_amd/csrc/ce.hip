// Row-wise cross-entropy over a chunk of logits (gfx950): the fused reduction
// of the frozen-head loss (kernels/frozen_linear_cross_entropy.py:26-139).
//
// For row i with target y (valid when 0 <= y < V):
//   lse     = m + log(sum_j exp(l_j - m)),  m = max_j l_j       (fp32)
//   loss_i  = valid ? (lse - l_y) / total : 0
//   grad_ij = (exp(l_j - m) / d - [valid && j == y]) / total   (stored in the logits' dtype)
// Invalid targets give a zero loss and a softmax gradient, as the reference's
// fused kernel does (kernels/frozen_linear_cross_entropy.py:97-139). The exact
// entry point (molt_cross_entropy_rows_exact) follows F.cross_entropy's rule
// for ignored rows instead: zero loss and a zero gradient (the caller rejects
// targets that are neither valid nor ignored), and multiplies the gradient by
// an upstream scale read from device memory (kernels/partitioned_loss.py:56-98).
//
// One workgroup owns a row. Pass 1 keeps a per-thread online (max, sum) and
// combines them across the workgroup; pass 2 writes the gradient, in place
// when `grad` aliases the logits: every element is read by the thread that
// overwrites it, and the target logit is read in pass 1. bf16 rows of up to
// 163,840 logits (Qwen's 151,936-entry vocabulary is 297 KB) stay in
// registers between the passes (ce_reg_kernel); longer or fp32 rows are read
// twice (ce_kernel, the second read from the L2 / Infinity Cache). The
// exponentials use the hardware exp2 (__expf) and the two divisions of the
// gradient are multiplications by reciprocals taken once per row, as the
// reference's fused kernel computes them with the fast approximate forms
// (tl.exp, fp32 `/`); the loss keeps the accurate logf and division.
#include "common.h"

namespace molt {
namespace {

constexpr int CE_NT = 1024;   // 16 waves per row: enough loads in flight for one workgroup per CU

template <bool F32>
MOLT_DEV float ce_ld(const void* p, int64_t i) {
  if constexpr (F32) return reinterpret_cast<const float*>(p)[i];
  else return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
}

template <bool F32>
MOLT_DEV void ce_ld8(const void* p, int64_t i, float (&v)[8]) {
  if constexpr (F32) {
    const f32x4_t a = *reinterpret_cast<const f32x4_t*>(reinterpret_cast<const float*>(p) + i);
    const f32x4_t b = *reinterpret_cast<const f32x4_t*>(reinterpret_cast<const float*>(p) + i + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) { v[e] = a[e]; v[4 + e] = b[e]; }
  } else {
    const u32x4_t q = *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const uint16_t*>(p) + i);
#pragma unroll
    for (int e = 0; e < 4; ++e) { v[2 * e] = bf16_lo(q[e]); v[2 * e + 1] = bf16_hi(q[e]); }
  }
}

template <bool F32, bool NT = false>
MOLT_DEV void ce_st8(void* p, int64_t i, const float (&v)[8]) {
  if constexpr (F32) {
    f32x4_t a, b;
#pragma unroll
    for (int e = 0; e < 4; ++e) { a[e] = v[e]; b[e] = v[4 + e]; }
    *reinterpret_cast<f32x4_t*>(reinterpret_cast<float*>(p) + i) = a;
    *reinterpret_cast<f32x4_t*>(reinterpret_cast<float*>(p) + i + 4) = b;
  } else {
    u32x4_t q;
#pragma unroll
    for (int e = 0; e < 4; ++e) q[e] = pack_bf16x2(v[2 * e], v[2 * e + 1]);
    if constexpr (NT) __builtin_nontemporal_store(q, reinterpret_cast<u32x4_t*>(reinterpret_cast<uint16_t*>(p) + i));
    else *reinterpret_cast<u32x4_t*>(reinterpret_cast<uint16_t*>(p) + i) = q;
  }
}

template <bool F32>
MOLT_DEV void ce_st(void* p, int64_t i, float v) {
  if constexpr (F32) reinterpret_cast<float*>(p)[i] = v;
  else reinterpret_cast<uint16_t*>(p)[i] = bf16_bits(v);
}

// (m, d) online pair: d = sum exp(x - m); merging rescales the smaller max.
MOLT_DEV void ce_merge(float& m, float& d, float m2, float d2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;   // both empty
  d = (d > 0.0f ? d * __expf(m - mn) : 0.0f) + (d2 > 0.0f ? d2 * __expf(m2 - mn) : 0.0f);
  m = mn;
}

MOLT_DEV void ce_add(float& m, float& d, float x) {
  if (x > m) {
    d = (d > 0.0f ? d * __expf(m - x) : 0.0f) + 1.0f;
    m = x;
  } else {
    d += __expf(x - m);
  }
}

struct CeParams {
  const void* logits; int64_t ld;
  int64_t rows, V;
  const int64_t* targets;
  float total;
  float* loss;
  void* grad; int64_t ldg;
  const float* gscale;   // upstream gradient (exact rule), or null
  int zero_invalid;      // exact rule: rows without a valid target get a zero gradient
};

// Gradient of one element from its fp32 softmax-minus-target term: / total,
// then (EXACT) the upstream scale; zero on ignored rows under the exact rule
// (also for a NaN upstream scale, as F.cross_entropy leaves ignored rows
// untouched). The rule is a template parameter, so the fused rule's loop
// carries no per-element select or scale.
template <bool EXACT>
MOLT_DEV float ce_grad(float diff, float inv_total, bool zero_row, float gs) {
  float g = diff * inv_total;
  if constexpr (EXACT) {
    g *= gs;
    return zero_row ? 0.0f : g;
  } else {
    return g;
  }
}

template <bool F32, bool VEC, bool GRAD, bool EXACT>
__global__ __launch_bounds__(CE_NT) void ce_kernel(const CeParams p) {
  __shared__ float red_m[CE_NT / 64], red_d[CE_NT / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = blockIdx.x;
  const void* lrow = F32 ? (const void*)(reinterpret_cast<const float*>(p.logits) + row * p.ld)
                         : (const void*)(reinterpret_cast<const uint16_t*>(p.logits) + row * p.ld);
  const int64_t y = p.targets[row];
  const bool valid = y >= 0 && y < p.V;
  const float ly = valid ? ce_ld<F32>(lrow, y) : 0.0f;

  float m = -INFINITY, d = 0.0f;
  if constexpr (VEC) {
    for (int64_t i = 8 * (int64_t)tid; i < p.V; i += 8 * CE_NT) {
      float v[8];
      ce_ld8<F32>(lrow, i, v);
      float bm = v[0];
#pragma unroll
      for (int e = 1; e < 8; ++e) bm = fmaxf(bm, v[e]);
      float bs = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) bs += __expf(v[e] - bm);
      ce_merge(m, d, bm, bs);
    }
  } else {
    for (int64_t i = tid; i < p.V; i += CE_NT) ce_add(m, d, ce_ld<F32>(lrow, i));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float m2 = __shfl_xor(m, o, 64), d2 = __shfl_xor(d, o, 64);
    ce_merge(m, d, m2, d2);
  }
  if (lane == 0) { red_m[wave] = m; red_d[wave] = d; }
  __syncthreads();
  m = red_m[0];
  d = red_d[0];
#pragma unroll
  for (int w = 1; w < CE_NT / 64; ++w) ce_merge(m, d, red_m[w], red_d[w]);

  if (tid == 0) p.loss[row] = valid ? (m + logf(d) - ly) / p.total : 0.0f;
  if constexpr (GRAD) {
    void* grow = F32 ? (void*)(reinterpret_cast<float*>(p.grad) + row * p.ldg)
                     : (void*)(reinterpret_cast<uint16_t*>(p.grad) + row * p.ldg);
    const float inv_d = 1.0f / d, inv_total = 1.0f / p.total;
    const bool zero_row = EXACT && p.zero_invalid && !valid;
    const float gs = EXACT && p.gscale ? *p.gscale : 1.0f;
    if constexpr (VEC) {
      for (int64_t i = 8 * (int64_t)tid; i < p.V; i += 8 * CE_NT) {
        float v[8];
        ce_ld8<F32>(lrow, i, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float t = (valid && i + e == y) ? 1.0f : 0.0f;
          v[e] = ce_grad<EXACT>(__expf(v[e] - m) * inv_d - t, inv_total, zero_row, gs);
        }
        ce_st8<F32>(grow, i, v);
      }
    } else {
      for (int64_t i = tid; i < p.V; i += CE_NT) {
        const float t = (valid && i == y) ? 1.0f : 0.0f;
        ce_st<F32>(grow, i, ce_grad<EXACT>(__expf(ce_ld<F32>(lrow, i) - m) * inv_d - t, inv_total, zero_row, gs));
      }
    }
  }
}

// bf16 rows of at most 8 * CE_NT * CH elements, read once: every thread loads
// its CH chunks of 8 logits (chunk c at element 8 (tid + c CE_NT), the chunks
// the two-pass loop above visits, in the same order) into registers, all
// loads issued at once; pass 1 and pass 2 then run from registers, so the
// row is read from memory once instead of twice, and with the same
// arithmetic in the same order the results equal the two-pass kernel's bit
// for bit. Chunks past the row re-load the last chunk and are skipped.
template <int CH, bool GRAD, bool EXACT>
__global__ __launch_bounds__(CE_NT) void ce_reg_kernel(const CeParams p) {
  __shared__ float red_m[CE_NT / 64], red_d[CE_NT / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = blockIdx.x;
  const uint16_t* lrow = reinterpret_cast<const uint16_t*>(p.logits) + row * p.ld;
  const int64_t y = p.targets[row];
  const bool valid = y >= 0 && y < p.V;
  const float ly = bf16_to_f32(lrow[valid ? y : 0]);

  u32x4_t q[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int64_t i = 8 * ((int64_t)tid + (int64_t)c * CE_NT);
    q[c] = *reinterpret_cast<const u32x4_t*>(lrow + (i < p.V ? i : p.V - 8));
  }
  float m = -INFINITY, d = 0.0f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int64_t i = 8 * ((int64_t)tid + (int64_t)c * CE_NT);
    if (i >= p.V) continue;
    float v[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) { v[2 * e] = bf16_lo(q[c][e]); v[2 * e + 1] = bf16_hi(q[c][e]); }
    float bm = v[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) bm = fmaxf(bm, v[e]);
    float bs = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) bs += __expf(v[e] - bm);
    ce_merge(m, d, bm, bs);
    __builtin_amdgcn_sched_barrier(0);   // one chunk at a time: the row already fills the registers
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float m2 = __shfl_xor(m, o, 64), d2 = __shfl_xor(d, o, 64);
    ce_merge(m, d, m2, d2);
  }
  if (lane == 0) { red_m[wave] = m; red_d[wave] = d; }
  __syncthreads();
  m = red_m[0];
  d = red_d[0];
#pragma unroll
  for (int w = 1; w < CE_NT / 64; ++w) ce_merge(m, d, red_m[w], red_d[w]);

  if (tid == 0) p.loss[row] = valid ? (m + logf(d) - ly) / p.total : 0.0f;
  if constexpr (GRAD) {
    uint16_t* grow = reinterpret_cast<uint16_t*>(p.grad) + row * p.ldg;
    const float inv_d = 1.0f / d, inv_total = 1.0f / p.total;
    const bool zero_row = EXACT && p.zero_invalid && !valid;
    const float gs = EXACT && p.gscale ? *p.gscale : 1.0f;
    // keep only the packed row alive across the reduction (unpacked, pass 1's
    // fp32 copies would double its registers)
#pragma unroll
    for (int c = 0; c < CH; ++c) asm volatile("" : "+v"(q[c]));
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int64_t i = 8 * ((int64_t)tid + (int64_t)c * CE_NT);
      if (i >= p.V) continue;
      float v[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) { v[2 * e] = bf16_lo(q[c][e]); v[2 * e + 1] = bf16_hi(q[c][e]); }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float t = (valid && i + e == y) ? 1.0f : 0.0f;
        v[e] = ce_grad<EXACT>(__expf(v[e] - m) * inv_d - t, inv_total, zero_row, gs);
      }
      ce_st8<false, true>(grow, i, v);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

bool ce_a16(const void* q) { return ((uintptr_t)q & 15) == 0; }

}  // namespace
}  // namespace molt

using namespace molt;

namespace {

int ce_rows(const char* who, const void* logits, int32_t dtype, int64_t ld, int64_t rows, int64_t vocab,
            const int64_t* targets, float total, const float* grad_scale, int zero_invalid, float* loss, void* grad,
            int64_t ldg, void* stream) {
  MOLT_REQUIRE(dtype == MOLT_DTYPE_BF16 || dtype == MOLT_DTYPE_F32, MOLT_EINVAL, "%s: dtype must be bf16 or fp32",
               who);
  MOLT_REQUIRE(rows >= 0 && vocab > 0 && ld >= vocab && (!grad || ldg >= vocab), MOLT_EINVAL,
               "%s: bad shape (rows=%lld vocab=%lld)", who, (long long)rows, (long long)vocab);
  MOLT_REQUIRE(total > 0.0f, MOLT_EINVAL, "%s: total token count must be positive", who);
  if (rows == 0) return MOLT_OK;
  MOLT_REQUIRE(logits && targets && loss, MOLT_EINVAL, "%s: null pointer", who);
  MOLT_REQUIRE(rows < (1ll << 31), MOLT_EINVAL, "%s: too many rows", who);
  const bool f32 = dtype == MOLT_DTYPE_F32;
  const int es = f32 ? 4 : 2;
  const bool vec = vocab % 8 == 0 && ce_a16(logits) && (ld * es) % 16 == 0 &&
                   (!grad || (ce_a16(grad) && (ldg * es) % 16 == 0));
  CeParams p{logits, ld, rows, vocab, targets, total, loss, grad, ldg, grad_scale, zero_invalid};
  const dim3 grid((unsigned)rows), block(CE_NT);
  hipStream_t st = (hipStream_t)stream;
  const bool exact = grad_scale != nullptr || zero_invalid != 0;
  // bf16 rows up to 8 * CE_NT * 20 = 163,840 logits: one read, from registers
  const int64_t chunks = ceil_div64(vocab, 8 * CE_NT);
  if (!f32 && vec && chunks <= 20) {
#define MOLT_CE_REG(CH)                                                                    \
  do {                                                                                     \
    if (grad && exact) hipLaunchKernelGGL((ce_reg_kernel<CH, true, true>), grid, block, 0, st, p); \
    else if (grad) hipLaunchKernelGGL((ce_reg_kernel<CH, true, false>), grid, block, 0, st, p);    \
    else hipLaunchKernelGGL((ce_reg_kernel<CH, false, false>), grid, block, 0, st, p);             \
  } while (0)
    if (chunks <= 4) MOLT_CE_REG(4);
    else if (chunks <= 8) MOLT_CE_REG(8);
    else if (chunks <= 12) MOLT_CE_REG(12);
    else if (chunks <= 16) MOLT_CE_REG(16);
    else if (chunks <= 19) MOLT_CE_REG(19);   // Qwen's 151,936-entry vocabulary
    else MOLT_CE_REG(20);
#undef MOLT_CE_REG
    return check_launch(who);
  }
#define MOLT_CE_LAUNCH(F, V, G)                                                              \
  do {                                                                                       \
    if (G && exact) hipLaunchKernelGGL((ce_kernel<F, V, G, true>), grid, block, 0, st, p);   \
    else hipLaunchKernelGGL((ce_kernel<F, V, G, false>), grid, block, 0, st, p);             \
  } while (0)
  if (grad) {
    if (f32) { if (vec) MOLT_CE_LAUNCH(true, true, true); else MOLT_CE_LAUNCH(true, false, true); }
    else { if (vec) MOLT_CE_LAUNCH(false, true, true); else MOLT_CE_LAUNCH(false, false, true); }
  } else {
    if (f32) { if (vec) MOLT_CE_LAUNCH(true, true, false); else MOLT_CE_LAUNCH(true, false, false); }
    else { if (vec) MOLT_CE_LAUNCH(false, true, false); else MOLT_CE_LAUNCH(false, false, false); }
  }
#undef MOLT_CE_LAUNCH
  return check_launch(who);
}

}  // namespace

extern "C" int molt_cross_entropy_rows(const void* logits, int32_t dtype, int64_t ld, int64_t rows, int64_t vocab,
                                       const int64_t* targets, float total, float* loss, void* grad, int64_t ldg,
                                       void* stream) {
  return ce_rows("molt_cross_entropy_rows", logits, dtype, ld, rows, vocab, targets, total, nullptr, 0, loss, grad,
                 ldg, stream);
}

extern "C" int molt_cross_entropy_rows_exact(const void* logits, int32_t dtype, int64_t ld, int64_t rows,
                                             int64_t vocab, const int64_t* targets, float total,
                                             const float* grad_scale, float* loss, void* grad, int64_t ldg,
                                             void* stream) {
  return ce_rows("molt_cross_entropy_rows_exact", logits, dtype, ld, rows, vocab, targets, total, grad_scale, 1, loss,
                 grad, ldg, stream);
}
