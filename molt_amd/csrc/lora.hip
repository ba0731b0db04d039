// Rank-r LoRA kernels (gfx950): the low-rank projection T = z . bf16(A)^T and
// the adapter gradients dA = U^T X, dB = s dY^T T.
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

// ------------------------------------------------------------------------
// Projection out[M, R] = bf16(sum_d z(m, d) * bf16(W(q, d))).
// Workgroup = 4 waves over one 32-row slab of z and 64 outputs q; wave w
// takes every 4th 64-wide contraction step and the four partial tiles are
// summed in wave order through LDS (deterministic). Operands go straight
// from global memory to MFMA registers: lane half h covers contraction
// [d0 + 32h, +32), split across the four 16-deep MFMA sub-steps.
// ------------------------------------------------------------------------
constexpr int PJ_M = 32, PJ_Q = 64, PJ_WAVES = 4;

struct ProjParams {
  const uint16_t* z; const uint16_t* z2; int64_t ldz; int mode; float zs;
  int64_t M, D;
  const float* w; int layout; int R;     // layout 0: W(q,d) = w[q*D + d]; 1: w[d*R + q]
  uint16_t* out; int64_t ldo;
  int vec;                               // z rows 16-byte loadable
};

MOLT_DEV bf16x8_t load_z8(const ProjParams& p, int64_t m, int64_t d) {
  float v[8];
  if (m < p.M && p.vec && d + 8 <= p.D) {
    const u32x4_t a = *reinterpret_cast<const u32x4_t*>(p.z + m * p.ldz + d);
    u32x4_t b = {0u, 0u, 0u, 0u};
    if (p.mode == 1) b = *reinterpret_cast<const u32x4_t*>(p.z2 + m * p.ldz + d);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = ztrans(bf16_lo(a[e]), bf16_lo(b[e]), p.mode, p.zs);
      v[2 * e + 1] = ztrans(bf16_hi(a[e]), bf16_hi(b[e]), p.mode, p.zs);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float x = 0.0f;
      if (m < p.M && d + e < p.D) {
        const float a = bf16_to_f32(p.z[m * p.ldz + d + e]);
        const float b = p.mode == 1 ? bf16_to_f32(p.z2[m * p.ldz + d + e]) : 0.0f;
        x = ztrans(a, b, p.mode, p.zs);
      }
      v[e] = x;
    }
  }
  u32x4_t o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = pack_bf16x2(v[2 * e], v[2 * e + 1]);
  return __builtin_bit_cast(bf16x8_t, o);
}

MOLT_DEV bf16x8_t load_w8(const ProjParams& p, int64_t q, int64_t d) {
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float x = 0.0f;
    if (q < p.R && d + e < p.D) x = p.layout == 0 ? p.w[q * p.D + d + e] : p.w[(d + e) * p.R + q];
    v[e] = x;
  }
  u32x4_t o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = pack_bf16x2(v[2 * e], v[2 * e + 1]);
  return __builtin_bit_cast(bf16x8_t, o);
}

__global__ __launch_bounds__(64 * PJ_WAVES) void lora_project_kernel(const ProjParams p) {
  __shared__ float red[PJ_WAVES - 1][2][16][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t m0 = (int64_t)blockIdx.x * PJ_M;
  const int64_t q0 = (int64_t)blockIdx.y * PJ_Q;
  const int r = lane & 31, h = lane >> 5;
  const int64_t steps = ceil_div64(p.D, BK);

  f32x16_t acc[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[t][e] = 0.0f;

  for (int64_t s = wave; s < steps; s += PJ_WAVES) {
    const int64_t d0 = s * BK + 32 * h;
    bf16x8_t zf[4], wf[2][4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      zf[kk] = load_z8(p, m0 + r, d0 + 8 * kk);
#pragma unroll
      for (int t = 0; t < 2; ++t) wf[t][kk] = load_w8(p, q0 + t * 32 + r, d0 + 8 * kk);
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int t = 0; t < 2; ++t)
        acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[t][kk], zf[kk], acc[t], 0, 0, 0);
  }

  if (wave > 0) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) red[wave - 1][t][e][lane] = acc[t][e];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < PJ_WAVES - 1; ++w)
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[t][e] += red[w][t][e][lane];

  // acc[t] is C[q][m]: column m = lane % 32, rows q = 8(e/4) + 4h + e%4.
  const int64_t m = m0 + r;
  if (m >= p.M) return;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int64_t q = q0 + t * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
      if (q < p.R) p.out[m * p.ldo + q] = bf16_bits(acc[t][e]);
    }
}

// ------------------------------------------------------------------------
// Gradient partials: part[s][p][q] = sum over the s-th slice of M of
// L(m, p) * R(m, q). Both operands are staged into LDS transposed (the
// contraction index m contiguous) from 8-row x 4-column register patches.
// ------------------------------------------------------------------------
constexpr int GR_P = 128, GR_Q = 64;
constexpr int GR_NT = 256;
constexpr int GR_WROWS = 64, GR_WCOLS = 32;   // waves 2 (p) x 2 (q)

struct GradParams {
  const uint16_t* l; const uint16_t* l2; int64_t ldl; int mode;
  const uint16_t* rm; int64_t ldr;
  int64_t M, P, Q;
  int64_t slice;             // rows of M per split (multiple of BK)
  float* part;               // [S][P][Q]
  int vec;                   // 8-byte patch loads allowed
};

MOLT_DEV void load_patch4(const uint16_t* __restrict__ src, const uint16_t* __restrict__ src2,
                          int mode, int64_t ld, int64_t m, int64_t c, int64_t M, int64_t C,
                          bool vec, float* v) {
  if (m < M && vec && c + 4 <= C) {
    const u32x2_t a = *reinterpret_cast<const u32x2_t*>(src + m * ld + c);
    float x[4] = {bf16_lo(a[0]), bf16_hi(a[0]), bf16_lo(a[1]), bf16_hi(a[1])};
    if (mode == 1) {
      const u32x2_t b = *reinterpret_cast<const u32x2_t*>(src2 + m * ld + c);
      float y[4] = {bf16_lo(b[0]), bf16_hi(b[0]), bf16_lo(b[1]), bf16_hi(b[1])};
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = round_bf16(round_bf16(silu_f32(x[e])) * y[e]);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = x[e];
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float x = 0.0f;
      if (m < M && c + e < C) {
        x = bf16_to_f32(src[m * ld + c + e]);
        if (mode == 1) x = round_bf16(round_bf16(silu_f32(x)) * bf16_to_f32(src2[m * ld + c + e]));
      }
      v[e] = x;
    }
  }
}

// Stage a (8*8 rows of M) x (4*CGS columns) tile transposed into LDS rows.
template <int CGS>
MOLT_DEV void stage_t(uint16_t* dst, const uint16_t* src, const uint16_t* src2, int mode, int64_t ld,
                      int64_t m0, int64_t c0, int64_t M, int64_t mend, int64_t C, bool vec, int tid) {
  if (tid >= CGS * 8) return;
  const int cg = tid % CGS, rg = tid / CGS;
  float v[8][4];
#pragma unroll
  for (int rr = 0; rr < 8; ++rr) {
    const int64_t m = m0 + 8 * rg + rr;
    load_patch4(src, src2, mode, ld, m, c0 + 4 * cg, m < mend ? M : 0, C, vec, v[rr]);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    u32x4_t o;
    o[0] = pack_bf16x2(v[0][j], v[1][j]);
    o[1] = pack_bf16x2(v[2][j], v[3][j]);
    o[2] = pack_bf16x2(v[4][j], v[5][j]);
    o[3] = pack_bf16x2(v[6][j], v[7][j]);
    *reinterpret_cast<u32x4_t*>(dst + (4 * cg + j) * LDSW + 8 * rg) = o;
  }
}

__global__ __launch_bounds__(GR_NT) void lora_grad_kernel(const GradParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t ls[GR_P * LDSW];
  __shared__ __attribute__((aligned(16))) uint16_t rs[GR_Q * LDSW];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wp = wave & 1, wq = wave >> 1;
  const int64_t p0 = (int64_t)blockIdx.x * GR_P;
  const int64_t q0 = (int64_t)blockIdx.y * GR_Q;
  const int64_t mbeg = (int64_t)blockIdx.z * p.slice;
  int64_t mend = mbeg + p.slice;
  if (mend > p.M) mend = p.M;
  const bool vec = p.vec != 0;

  f32x16_t acc[2][1];
  zero_acc(acc);
  for (int64_t m0 = mbeg; m0 < mend; m0 += BK) {
    stage_t<GR_P / 4>(ls, p.l, p.l2, p.mode, p.ldl, m0, p0, p.M, mend, p.P, vec, tid);
    stage_t<GR_Q / 4>(rs, p.rm, nullptr, 0, p.ldr, m0, q0, p.M, mend, p.Q, vec, tid);
    __syncthreads();
    mfma_step<2, 1>(ls, rs, wp * GR_WROWS, wq * GR_WCOLS, acc, lane);
    __syncthreads();
  }

  // acc[i][0] is C[p][q]: column q = lane % 32, rows p = 8(e/4) + 4(lane/32) + e%4.
  float* out = p.part + (int64_t)blockIdx.z * p.P * p.Q;
  const int64_t q = q0 + wq * GR_WCOLS + (lane & 31);
  if (q >= p.Q) return;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int64_t pp = p0 + wp * GR_WROWS + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
      if (pp < p.P) out[pp * p.Q + q] = acc[i][0][e];
    }
}

__global__ void lora_grad_reduce_kernel(const float* __restrict__ part, int S, int64_t P, int64_t Q,
                                        float scale, float* __restrict__ out, int layout) {
  const int64_t n = P * Q;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    float s = 0.0f;
    for (int k = 0; k < S; ++k) s += part[(int64_t)k * n + i];
    const int64_t pp = i / Q, q = i % Q;
    out[layout == 0 ? i : q * P + pp] = s * scale;
  }
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

int grad_splits(int64_t M, int64_t P, int64_t Q) {
  const int64_t tiles = ceil_div64(P, GR_P) * ceil_div64(Q, GR_Q);
  int64_t s = (1024 + tiles - 1) / tiles;      // aim for ~1024 workgroups
  const int64_t max_s = ceil_div64(M, 256);    // keep >= 256 rows per split
  if (s > max_s) s = max_s;
  if (s < 1) s = 1;
  if (s > 64) s = 64;
  return (int)s;
}

}  // namespace
}  // namespace molt

using namespace molt;

extern "C" int molt_lora_project(const uint16_t* z, const uint16_t* z2, int64_t ldz, int32_t z_mode,
                                 float z_scale, int64_t M, int64_t D, const float* lora,
                                 int32_t lora_layout, int32_t r, uint16_t* out, int64_t ldo,
                                 void* stream) {
  const char* who = "molt_lora_project";
  MOLT_REQUIRE(z_mode >= 0 && z_mode <= 2, MOLT_EINVAL, "%s: bad z_mode %d", who, z_mode);
  MOLT_REQUIRE(lora_layout == 0 || lora_layout == 1, MOLT_EINVAL, "%s: bad lora_layout", who);
  MOLT_REQUIRE(M >= 0 && D > 0 && r > 0 && r <= 1024, MOLT_EINVAL, "%s: bad shape M=%lld D=%lld r=%d", who,
               (long long)M, (long long)D, r);
  MOLT_REQUIRE(z && lora && out && ldz >= D && ldo >= r, MOLT_EINVAL, "%s: bad pointers/strides", who);
  MOLT_REQUIRE(z_mode != 1 || z2, MOLT_EINVAL, "%s: SwiGLU replay needs the up tensor", who);
  if (M == 0) return MOLT_OK;
  ProjParams p{};
  p.z = z; p.z2 = z2; p.ldz = ldz; p.mode = z_mode; p.zs = z_scale;
  p.M = M; p.D = D; p.w = lora; p.layout = lora_layout; p.R = r; p.out = out; p.ldo = ldo;
  p.vec = ldz % 8 == 0 && aligned(z, 16) && (z_mode != 1 || aligned(z2, 16));
  dim3 grid((unsigned)ceil_div64(M, PJ_M), (unsigned)ceil_div64(r, PJ_Q));
  hipLaunchKernelGGL(lora_project_kernel, grid, dim3(64 * PJ_WAVES), 0, (hipStream_t)stream, p);
  return check_launch(who);
}

extern "C" size_t molt_lora_grad_workspace(int64_t M, int64_t P, int64_t Q) {
  if (M <= 0 || P <= 0 || Q <= 0) return 0;
  return (size_t)grad_splits(M, P, Q) * (size_t)P * (size_t)Q * sizeof(float);
}

extern "C" int molt_lora_grad(const uint16_t* l, const uint16_t* l2, int64_t ldl, int32_t l_mode,
                              const uint16_t* rmat, int64_t ldr, int64_t M, int64_t P, int64_t Q,
                              float scale, float* out, int32_t out_layout, void* workspace,
                              size_t workspace_bytes, void* stream) {
  const char* who = "molt_lora_grad";
  MOLT_REQUIRE(l_mode == 0 || l_mode == 1, MOLT_EINVAL, "%s: bad l_mode", who);
  MOLT_REQUIRE(out_layout == 0 || out_layout == 1, MOLT_EINVAL, "%s: bad out_layout", who);
  MOLT_REQUIRE(M >= 0 && P > 0 && Q > 0, MOLT_EINVAL, "%s: bad shape", who);
  MOLT_REQUIRE(l && rmat && out && ldl >= P && ldr >= Q, MOLT_EINVAL, "%s: bad pointers/strides", who);
  MOLT_REQUIRE(l_mode == 0 || l2, MOLT_EINVAL, "%s: SwiGLU replay needs the up tensor", who);
  hipStream_t st = (hipStream_t)stream;
  if (M == 0) {
    MOLT_REQUIRE(hipMemsetAsync(out, 0, (size_t)P * Q * sizeof(float), st) == hipSuccess, MOLT_ELAUNCH,
                 "%s: memset failed", who);
    return MOLT_OK;
  }
  const int S = grad_splits(M, P, Q);
  const size_t need = (size_t)S * P * Q * sizeof(float);
  MOLT_REQUIRE(workspace && workspace_bytes >= need, MOLT_EWORKSPACE, "%s: workspace %zu < %zu bytes", who,
               workspace_bytes, need);
  GradParams p{};
  p.l = l; p.l2 = l2; p.ldl = ldl; p.mode = l_mode; p.rm = rmat; p.ldr = ldr;
  p.M = M; p.P = P; p.Q = Q;
  p.slice = ceil_div64(ceil_div64(M, S), BK) * BK;
  p.part = (float*)workspace;
  p.vec = ldl % 4 == 0 && ldr % 4 == 0 && aligned(l, 8) && aligned(rmat, 8) && (l_mode == 0 || aligned(l2, 8));
  const int S_eff = (int)ceil_div64(M, p.slice);
  dim3 grid((unsigned)ceil_div64(P, GR_P), (unsigned)ceil_div64(Q, GR_Q), (unsigned)S_eff);
  hipLaunchKernelGGL(lora_grad_kernel, grid, dim3(GR_NT), 0, st, p);
  int rc = check_launch(who);
  if (rc) return rc;
  const int64_t n = P * Q;
  unsigned blocks = (unsigned)((n + 255) / 256);
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(lora_grad_reduce_kernel, dim3(blocks), dim3(256), 0, st, p.part, S_eff, P, Q, scale,
                     out, out_layout);
  return check_launch(who);
}
