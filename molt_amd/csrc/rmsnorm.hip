// Frozen RMSNorm (gfx950): the forward of _FrozenRMSNormFunction and of the
// gated MLP's norm-replay recipe, and the frozen-weight backward.
//
//   forward  (kernels/frozen_rmsnorm.py:10-23, methods/gated_replay.py:22-30):
//     inv  = rsqrt(sum(fp32(x)^2) * (1 / H) + eps)
//     out  = bf16( fp32(x) * inv * (fp32(w) + offset) )
//   backward (kernels/frozen_rmsnorm.py:25-37):
//     n    = fp32(x) * inv,  g = fp32(dy) * (fp32(w) + offset)
//     dx   = inv * (g - n * (sum(g * n) * (1 / H))), stored in x's dtype
//
// One wave owns a row; the row's sums are wave reductions, so no LDS and no
// barrier. HBM-bound. Vector path (H <= 8192, H % 8 == 0, every row start
// 16-byte aligned): the row is read once into registers, 8 consecutive
// elements per lane and access (16 B of bf16, 32 B of fp32). Otherwise one
// element per lane and access, and the later passes re-read the row from the
// L1/L2 (4 rows per workgroup).
#include "common.h"

namespace molt {
namespace {

constexpr int RN_NT = 256;
constexpr int RN_ROWS = RN_NT / 64;

struct RmsParams {
  const void* x;
  const uint16_t* dy;
  const void* w;
  void* out;        // forward: bf16 out; backward: dx in x's dtype
  float* inv_rms;   // forward only, may be null
  int64_t ldx, lddy, ldo, M, H;
  float eps, offset;
};

template <bool F32>
MOLT_DEV float ld1(const void* p, int64_t i) {
  if constexpr (F32) return reinterpret_cast<const float*>(p)[i];
  else return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
}

template <bool F32>
MOLT_DEV void ld8(const void* p, int64_t i, float (&v)[8]) {
  if constexpr (F32) {
    const f32x4_t a = *reinterpret_cast<const f32x4_t*>(reinterpret_cast<const float*>(p) + i);
    const f32x4_t b = *reinterpret_cast<const f32x4_t*>(reinterpret_cast<const float*>(p) + i + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) { v[e] = a[e]; v[4 + e] = b[e]; }
  } else {
    const u32x4_t q = *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const uint16_t*>(p) + i);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t d = q[e];
      v[2 * e] = bf16_lo(d);
      v[2 * e + 1] = bf16_hi(d);
    }
  }
}

// 8 consecutive elements as loaded (bf16: one 16-byte word, 4 registers;
// fp32: two, 8 registers), converted to fp32 where used.
template <bool F32>
struct Raw8;
template <>
struct Raw8<false> {
  u32x4_t q;
  MOLT_DEV void load(const void* p, int64_t i) { q = *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const uint16_t*>(p) + i); }
  MOLT_DEV void zero() { q = u32x4_t{0, 0, 0, 0}; }
  MOLT_DEV float operator[](int e) const {
    const uint32_t d = q[e >> 1];
    return (e & 1) ? bf16_hi(d) : bf16_lo(d);
  }
};
template <>
struct Raw8<true> {
  f32x4_t a, b;
  MOLT_DEV void load(const void* p, int64_t i) {
    a = *reinterpret_cast<const f32x4_t*>(reinterpret_cast<const float*>(p) + i);
    b = *reinterpret_cast<const f32x4_t*>(reinterpret_cast<const float*>(p) + i + 4);
  }
  MOLT_DEV void zero() { a = b = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}; }
  MOLT_DEV float operator[](int e) const { return e < 4 ? a[e] : b[e - 4]; }
};

// NT: non-temporal bf16 stores (whole 16-byte runs of consecutive lanes);
// faster for the forward's output, slower for the backward's dx.
template <bool F32, bool NT = false>
MOLT_DEV void st8(void* p, int64_t i, const float (&v)[8]) {
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
MOLT_DEV void st1(void* p, int64_t i, float v) {
  if constexpr (F32) reinterpret_cast<float*>(p)[i] = v;
  else reinterpret_cast<uint16_t*>(p)[i] = bf16_bits(v);
}

MOLT_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// sum over the row of fp32(x)^2 (each square rounded to fp32, then summed),
// one element per lane and access
template <bool XF32>
MOLT_DEV float row_sumsq(const void* xr, int64_t H, int lane) {
  float s = 0.0f;
  for (int64_t i = lane; i < H; i += 64) {
    const float v = ld1<XF32>(xr, i);
    s += __fmul_rn(v, v);
  }
  return wave_sum(s);
}

template <bool XF32>
MOLT_DEV const void* row_ptr(const void* base, int64_t row, int64_t ld) {
  return XF32 ? (const void*)(reinterpret_cast<const float*>(base) + row * ld)
              : (const void*)(reinterpret_cast<const uint16_t*>(base) + row * ld);
}

// NV > 0: the row stays in registers, NV chunks of 8 elements per lane (chunk
// c of lane l = elements 8 l + 512 c .. +7, masked past H; H <= 512 NV). All of
// a row's loads are issued before the reduction. NV == 0: one element per
// lane and access, the row re-read from the cache for each pass.
template <bool XF32, bool WF32, int NV>
__global__ __launch_bounds__(RN_NT) void rmsnorm_fwd_kernel(const RmsParams p) {
  const int lane = threadIdx.x & 63;
  const float inv_h = 1.0f / (float)p.H;
  for (int64_t row = (int64_t)blockIdx.x * RN_ROWS + (threadIdx.x >> 6); row < p.M;
       row += (int64_t)gridDim.x * RN_ROWS) {
    const void* xr = row_ptr<XF32>(p.x, row, p.ldx);
    uint16_t* orow = reinterpret_cast<uint16_t*>(p.out) + row * p.ldo;
    if constexpr (NV > 0) {
      Raw8<XF32> xv[NV];
      float s = 0.0f;
#pragma unroll
      for (int c = 0; c < NV; ++c) {
        const int64_t i = 8 * lane + 512 * c;
        if (i < p.H) xv[c].load(xr, i);
        else xv[c].zero();
      }
#pragma unroll
      for (int c = 0; c < NV; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) s += __fmul_rn(xv[c][e], xv[c][e]);
      const float inv = rsqrtf(wave_sum(s) * inv_h + p.eps);
      if (p.inv_rms && lane == 0) p.inv_rms[row] = inv;
      if (!p.out) continue;   // inv only
#pragma unroll
      for (int c = 0; c < NV; ++c) {
        const int64_t i = 8 * lane + 512 * c;
        if (i < p.H) {
          float w[8], o8[8];
          ld8<WF32>(p.w, i, w);
#pragma unroll
          for (int e = 0; e < 8; ++e) o8[e] = __fmul_rn(__fmul_rn(xv[c][e], inv), __fadd_rn(w[e], p.offset));
          st8<false, true>(orow, i, o8);
        }
      }
    } else {
      const float inv = rsqrtf(row_sumsq<XF32>(xr, p.H, lane) * inv_h + p.eps);
      if (p.inv_rms && lane == 0) p.inv_rms[row] = inv;
      if (!p.out) continue;
      for (int64_t i = lane; i < p.H; i += 64) {
        const float v = __fmul_rn(__fmul_rn(ld1<XF32>(xr, i), inv), __fadd_rn(ld1<WF32>(p.w, i), p.offset));
        orow[i] = bf16_bits(v);
      }
    }
  }
}

template <bool XF32, bool WF32, int NV>
__global__ __launch_bounds__(RN_NT) void rmsnorm_bwd_kernel(const RmsParams p) {
  const int lane = threadIdx.x & 63;
  const float inv_h = 1.0f / (float)p.H;
  for (int64_t row = (int64_t)blockIdx.x * RN_ROWS + (threadIdx.x >> 6); row < p.M;
       row += (int64_t)gridDim.x * RN_ROWS) {
    const void* xr = row_ptr<XF32>(p.x, row, p.ldx);
    const uint16_t* dyr = p.dy + row * p.lddy;
    void* dxr = XF32 ? (void*)(reinterpret_cast<float*>(p.out) + row * p.ldo)
                     : (void*)(reinterpret_cast<uint16_t*>(p.out) + row * p.ldo);
    if constexpr (NV > 0) {
      Raw8<XF32> xv[NV];
      Raw8<false> dv[NV];
      Raw8<WF32> wv[NV];
      float s = 0.0f;
#pragma unroll
      for (int c = 0; c < NV; ++c) {
        const int64_t i = 8 * lane + 512 * c;
        if (i < p.H) {
          xv[c].load(xr, i);
          dv[c].load(dyr, i);
        } else {
          xv[c].zero();
          dv[c].zero();
        }
      }
#pragma unroll
      for (int c = 0; c < NV; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) s += __fmul_rn(xv[c][e], xv[c][e]);
      const float inv = rsqrtf(wave_sum(s) * inv_h + p.eps);
      // g = dy * (w + offset), n = x * inv; correction = mean(g * n)
      float cs = 0.0f;
#pragma unroll
      for (int c = 0; c < NV; ++c) {
        const int64_t i = 8 * lane + 512 * c;
        if (i < p.H) wv[c].load(p.w, i);
        else wv[c].zero();
#pragma unroll
        for (int e = 0; e < 8; ++e)
          cs += __fmul_rn(__fmul_rn(dv[c][e], __fadd_rn(wv[c][e], p.offset)), __fmul_rn(xv[c][e], inv));
      }
      const float corr = wave_sum(cs) * inv_h;
#pragma unroll
      for (int c = 0; c < NV; ++c) {
        const int64_t i = 8 * lane + 512 * c;
        if (i < p.H) {
          float o8[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float g = __fmul_rn(dv[c][e], __fadd_rn(wv[c][e], p.offset));
            o8[e] = __fmul_rn(inv, __fsub_rn(g, __fmul_rn(__fmul_rn(xv[c][e], inv), corr)));
          }
          st8<XF32>(dxr, i, o8);
        }
      }
    } else {
      const float inv = rsqrtf(row_sumsq<XF32>(xr, p.H, lane) * inv_h + p.eps);
      float c = 0.0f;
      for (int64_t i = lane; i < p.H; i += 64) {
        const float g = __fmul_rn(bf16_to_f32(dyr[i]), __fadd_rn(ld1<WF32>(p.w, i), p.offset));
        c += __fmul_rn(g, __fmul_rn(ld1<XF32>(xr, i), inv));
      }
      const float corr = wave_sum(c) * inv_h;
      for (int64_t i = lane; i < p.H; i += 64) {
        const float g = __fmul_rn(bf16_to_f32(dyr[i]), __fadd_rn(ld1<WF32>(p.w, i), p.offset));
        const float n = __fmul_rn(ld1<XF32>(xr, i), inv);
        st1<XF32>(dxr, i, __fmul_rn(inv, __fsub_rn(g, __fmul_rn(n, corr))));
      }
    }
  }
}

unsigned rn_grid(int64_t M) {
  int64_t g = (M + RN_ROWS - 1) / RN_ROWS;
  if (g > 65536) g = 65536;
  return (unsigned)(g < 1 ? 1 : g);
}

// Chunks of 8 per lane for a register-resident row: the smallest power of two
// with 512 NV >= H, or 0 (one element per access) when H > 512 max_nv or the
// rows are not 16-byte aligned.
int pick_nv(int64_t H, bool aligned, int max_nv = 16) {
  if (!aligned || H % 8 != 0 || H > 512 * max_nv) return 0;
  int nv = 1;
  while (512 * nv < H) nv *= 2;
  return nv;
}

#define MOLT_RN_KERNEL_NV(KERNEL, XF, WF, nv, grid, st, prm)                                       \
  do {                                                                                             \
    switch (nv) {                                                                                  \
      case 1: hipLaunchKernelGGL((KERNEL<XF, WF, 1>), grid, dim3(RN_NT), 0, st, prm); break;         \
      case 2: hipLaunchKernelGGL((KERNEL<XF, WF, 2>), grid, dim3(RN_NT), 0, st, prm); break;         \
      case 4: hipLaunchKernelGGL((KERNEL<XF, WF, 4>), grid, dim3(RN_NT), 0, st, prm); break;         \
      case 8: hipLaunchKernelGGL((KERNEL<XF, WF, 8>), grid, dim3(RN_NT), 0, st, prm); break;         \
      case 16: hipLaunchKernelGGL((KERNEL<XF, WF, 16>), grid, dim3(RN_NT), 0, st, prm); break;       \
      default: hipLaunchKernelGGL((KERNEL<XF, WF, 0>), grid, dim3(RN_NT), 0, st, prm); break;        \
    }                                                                                              \
  } while (0)

#define MOLT_RN_LAUNCH(KERNEL, xf, wf, nv, grid, st, prm)                                          \
  do {                                                                                             \
    if (xf && wf) MOLT_RN_KERNEL_NV(KERNEL, true, true, nv, grid, st, prm);                         \
    else if (xf) MOLT_RN_KERNEL_NV(KERNEL, true, false, nv, grid, st, prm);                         \
    else if (wf) MOLT_RN_KERNEL_NV(KERNEL, false, true, nv, grid, st, prm);                         \
    else MOLT_RN_KERNEL_NV(KERNEL, false, false, nv, grid, st, prm);                                \
  } while (0)

bool a16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

// Row starts are 16-byte aligned for every row when the base is and the row
// stride is a multiple of 16 bytes.
bool vec_ok(const void* base, int64_t ld, int esize) { return a16(base) && (ld * esize) % 16 == 0; }

int check_dtype(int32_t d, const char* who, const char* what) {
  MOLT_REQUIRE(d == MOLT_DTYPE_BF16 || d == MOLT_DTYPE_F32, MOLT_EINVAL, "%s: %s dtype must be bf16 or fp32", who,
               what);
  return MOLT_OK;
}

}  // namespace
}  // namespace molt

using namespace molt;

extern "C" int molt_rmsnorm_forward(const void* x, int32_t x_dtype, int64_t ldx, int64_t M, int64_t H,
                                    const void* weight, int32_t w_dtype, float eps, float offset, uint16_t* out,
                                    int64_t ldo, float* inv_rms, void* stream) {
  const char* who = "molt_rmsnorm_forward";
  if (int e = check_dtype(x_dtype, who, "x")) return e;
  if (int e = check_dtype(w_dtype, who, "weight")) return e;
  MOLT_REQUIRE(M >= 0 && H > 0 && ldx >= H && ldo >= H, MOLT_EINVAL, "%s: bad shape (M=%lld H=%lld ldx=%lld ldo=%lld)",
               who, (long long)M, (long long)H, (long long)ldx, (long long)ldo);
  if (M == 0) return MOLT_OK;
  MOLT_REQUIRE(x && weight && (out || inv_rms), MOLT_EINVAL, "%s: null pointer", who);
  const bool xf = x_dtype == MOLT_DTYPE_F32, wf = w_dtype == MOLT_DTYPE_F32;
  // Without out (inv only) the kernel choice is that of a call whose out rows
  // are 16-byte aligned, so inv is bitwise that of such a call.
  const int nv = pick_nv(H, vec_ok(x, ldx, xf ? 4 : 2) && a16(weight) && (!out || vec_ok(out, ldo, 2)));
  RmsParams p{x, nullptr, weight, out, inv_rms, ldx, 0, ldo, M, H, eps, offset};
  MOLT_RN_LAUNCH(rmsnorm_fwd_kernel, xf, wf, nv, dim3(rn_grid(M)), (hipStream_t)stream, p);
  return check_launch(who);
}

extern "C" int molt_rmsnorm_backward(const uint16_t* dy, int64_t lddy, const void* x, int32_t x_dtype, int64_t ldx,
                                     int64_t M, int64_t H, const void* weight, int32_t w_dtype, float eps,
                                     float offset, void* dx, int64_t lddx, void* stream) {
  const char* who = "molt_rmsnorm_backward";
  if (int e = check_dtype(x_dtype, who, "x")) return e;
  if (int e = check_dtype(w_dtype, who, "weight")) return e;
  MOLT_REQUIRE(M >= 0 && H > 0 && ldx >= H && lddy >= H && lddx >= H, MOLT_EINVAL,
               "%s: bad shape (M=%lld H=%lld)", who, (long long)M, (long long)H);
  if (M == 0) return MOLT_OK;
  MOLT_REQUIRE(dy && x && weight && dx, MOLT_EINVAL, "%s: null pointer", who);
  const bool xf = x_dtype == MOLT_DTYPE_F32, wf = w_dtype == MOLT_DTYPE_F32;
  const int xs = xf ? 4 : 2;
  // an fp32 row of 8192 would not fit in registers beside dY and the weight
  const int nv = pick_nv(H, vec_ok(x, ldx, xs) && vec_ok(dy, lddy, 2) && a16(weight) && vec_ok(dx, lddx, xs),
                         xf ? 8 : 16);
  RmsParams p{x, dy, weight, dx, nullptr, ldx, lddy, lddx, M, H, eps, offset};
  MOLT_RN_LAUNCH(rmsnorm_bwd_kernel, xf, wf, nv, dim3(rn_grid(M)), (hipStream_t)stream, p);
  return check_launch(who);
}
