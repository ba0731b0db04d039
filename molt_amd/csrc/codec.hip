// NF4 codec kernels (gfx950): dequantise, resolve nested scales, quantise,
// double-quantise. Every arithmetic step is a single IEEE fp32 operation in a
// fixed order, which makes the results bit-exact against the CPU restatement.
// `fp contract(off)` keeps a multiply and the following add from being fused
// into one FMA; it applies to the raw operators written here (it does not
// reach the operators inside HIP's __fmul_rn/__fadd_rn, so those are not used).
#include "common.h"

namespace molt {
namespace {

constexpr int CODEC_NT = 256;

struct ScaleSrc {
  const float* scales;
  const uint8_t* q; const float* absmax2; const float* code2; float offset; int dq_block;
  int nested;
  int dq_shift;    // log2(dq_block) when it is a power of two, else -1
};

// scale = fp32(fp32(code2[q] * absmax2[b / dq]) + offset), or the fp32 scale itself.
MOLT_DEV float block_scale(const ScaleSrc& s, int64_t b) {
#pragma clang fp contract(off)
  if (!s.nested) return s.scales[b];
  const float prod = s.code2[s.q[b]] * s.absmax2[b / s.dq_block];
  return prod + s.offset;
}

// ---------------------------------------------------------------- dequantise
// Work unit: 4 packed bytes = 8 elements, one 16-byte bf16 (32-byte fp32)
// output chunk. Unit u of a pass goes to lane u % 64 of the wave, so each
// load instruction reads 256 contiguous bytes and each store instruction
// writes 1 KB (2 KB fp32) contiguous. A thread takes DQ_UPT units per pass,
// all loads (packed bytes, then block statistics) issued before any use;
// loads past the last whole unit re-read it. The unit that holds the end of
// an element count not divisible by 8 is decoded element by element.
// Byte -> code pair from a 256-entry LDS table, times the block scale,
// rounded once to the output dtype.
constexpr int DQ_UPT = 4;

template <int OUT_F32>
MOLT_DEV void dq_store(void* out, int64_t e0, const float (&v)[8]) {
  if (OUT_F32) {
    float* o = reinterpret_cast<float*>(out) + e0;
    *reinterpret_cast<f32x4_t*>(o) = f32x4_t{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4_t*>(o + 4) = f32x4_t{v[4], v[5], v[6], v[7]};
  } else {
    u32x4_t w;
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = pack_bf16x2(v[2 * j], v[2 * j + 1]);
    __builtin_nontemporal_store(w, reinterpret_cast<u32x4_t*>(reinterpret_cast<uint16_t*>(out) + e0));
  }
}

// BLK8 with a power-of-two block (blk_shift >= 0): the 8-element unit u lies
// in block (8 u) >> blk_shift, the nested statistics' code table sits in LDS
// and every statistics load of the pass is issued before the first is used
// (no 64-bit division, no dependent global load per unit).
template <int OUT_F32, bool BLK8>
__global__ __launch_bounds__(CODEC_NT) void dequant_kernel(const uint8_t* __restrict__ packed,
                                                           ScaleSrc ss, const float* __restrict__ code,
                                                           int order, int64_t n, int block, int blk_shift,
                                                           void* __restrict__ out) {
  static_assert(CODEC_NT == 256, "one table entry per thread");
  __shared__ float2 tab[256];
  __shared__ float c2s[256];
  {
    const int b = threadIdx.x;
    const int hi = b >> 4, lo = b & 15;
    tab[b] = make_float2(code[order ? hi : lo], code[order ? lo : hi]);
    c2s[b] = ss.nested ? ss.code2[b] : 0.0f;
  }
  __syncthreads();
  const bool fast = BLK8 && blk_shift >= 0 && (!ss.nested || ss.dq_shift >= 0);
  const int64_t whole = n / 8;                 // units with 8 elements
  const int64_t units = (n + 7) / 8;
  const int64_t step = (int64_t)gridDim.x * CODEC_NT * DQ_UPT;
  for (int64_t base = (int64_t)blockIdx.x * CODEC_NT * DQ_UPT; base < units; base += step) {
    uint32_t q[DQ_UPT];
    float sc[DQ_UPT];
    if (whole > 0) {
#pragma unroll
      for (int i = 0; i < DQ_UPT; ++i) {
        const int64_t u = base + i * CODEC_NT + threadIdx.x;
        q[i] = *reinterpret_cast<const uint32_t*>(packed + 4 * (u < whole ? u : whole - 1));
      }
      if (BLK8 && fast) {
        int64_t blk[DQ_UPT];
#pragma unroll
        for (int i = 0; i < DQ_UPT; ++i) {
          const int64_t u = base + i * CODEC_NT + threadIdx.x;
          blk[i] = (8 * (u < whole ? u : whole - 1)) >> blk_shift;
        }
        if (ss.nested) {
          uint32_t qb[DQ_UPT];
          float a2[DQ_UPT];
#pragma unroll
          for (int i = 0; i < DQ_UPT; ++i) {
            qb[i] = ss.q[blk[i]];
            a2[i] = ss.absmax2[blk[i] >> ss.dq_shift];
          }
#pragma unroll
          for (int i = 0; i < DQ_UPT; ++i) {
#pragma clang fp contract(off)
            const float prod = c2s[qb[i]] * a2[i];   // block_scale's order: fp32(code2[q] * absmax2) + offset
            sc[i] = prod + ss.offset;
          }
        } else {
#pragma unroll
          for (int i = 0; i < DQ_UPT; ++i) sc[i] = ss.scales[blk[i]];
        }
      } else if (BLK8) {
#pragma unroll
        for (int i = 0; i < DQ_UPT; ++i) {
          const int64_t u = base + i * CODEC_NT + threadIdx.x;
          sc[i] = block_scale(ss, 8 * (u < whole ? u : whole - 1) / block);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < DQ_UPT; ++i) {
      const int64_t u = base + i * CODEC_NT + threadIdx.x;
      const int64_t e0 = 8 * u;
      float v[8];
      if (u < whole) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float2 p = tab[(q[i] >> (8 * j)) & 0xffu];
          if (BLK8) {
            v[2 * j] = p.x * sc[i];
            v[2 * j + 1] = p.y * sc[i];
          } else {
            v[2 * j] = p.x * block_scale(ss, (e0 + 2 * j) / block);
            v[2 * j + 1] = p.y * block_scale(ss, (e0 + 2 * j + 1) / block);
          }
        }
        dq_store<OUT_F32>(out, e0, v);
      } else if (u < units) {
        // the last, partial unit: its bytes and elements one by one
        for (int k = 0; e0 + k < n; ++k) {
          const int byte = packed[(e0 + k) >> 1];
          const float2 p = tab[byte];
          const float c = ((e0 + k) & 1) ? p.y : p.x;
          const float vk = c * block_scale(ss, (e0 + k) / block);
          if (OUT_F32) reinterpret_cast<float*>(out)[e0 + k] = vk;
          else reinterpret_cast<uint16_t*>(out)[e0 + k] = bf16_bits(vk);
        }
      }
    }
  }
}

__global__ void resolve_kernel(ScaleSrc ss, int64_t nblocks, float* __restrict__ out) {
  for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < nblocks;
       b += (int64_t)gridDim.x * blockDim.x)
    out[b] = block_scale(ss, b);
}

// ------------------------------------------------------------------ quantise
// One wave per block: absmax by wave reduction (max is order independent),
// then each element's code is the first index of the minimum |x/absmax - code|
// (the running minimum's strict `<` keeps the first index on ties).
MOLT_DEV float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

template <int IN_BF16>
__global__ __launch_bounds__(CODEC_NT) void quantize_kernel(const void* __restrict__ x, int64_t n,
                                                            int block, int order,
                                                            const float* __restrict__ code,
                                                            uint8_t* __restrict__ packed,
                                                            float* __restrict__ absmax,
                                                            int64_t nblocks) {
  __shared__ float cb[16];
  if (threadIdx.x < 16) cb[threadIdx.x] = code[threadIdx.x];
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int64_t waves = (int64_t)gridDim.x * (CODEC_NT / 64);
  auto load = [&](int64_t i) -> float {
    if (i >= n) return 0.0f;
    if (IN_BF16) return bf16_to_f32(reinterpret_cast<const uint16_t*>(x)[i]);
    return reinterpret_cast<const float*>(x)[i];
  };
  auto nearest = [&](float nv) -> uint32_t {
    float best = fabsf(nv - cb[0]);
    uint32_t bi = 0;
#pragma unroll
    for (int c = 1; c < 16; ++c) {
      const float d = fabsf(nv - cb[c]);
      if (d < best) { best = d; bi = (uint32_t)c; }
    }
    return bi;
  };
  if (block == 64) {
    // one element per lane, loaded once; QB blocks per pass with every load
    // issued before the first is used; the odd lane's code joins its even
    // neighbour's by a lane shift and the even lanes store the bytes
    constexpr int QB = 4;
    for (int64_t b0 = (int64_t)blockIdx.x * (CODEC_NT / 64) + (threadIdx.x >> 6); b0 < nblocks; b0 += QB * waves) {
      float v[QB];
#pragma unroll
      for (int k = 0; k < QB; ++k) {
        const int64_t b = b0 + k * waves;
        v[k] = b < nblocks ? load(b * 64 + lane) : 0.0f;
      }
#pragma unroll
      for (int k = 0; k < QB; ++k) {
        const int64_t b = b0 + k * waves;
        if (b >= nblocks) break;   // uniform across the wave
        const float am = fmaxf(wave_max(fmaxf(0.0f, fabsf(v[k]))), 1.17549435e-38f);
        if (lane == 0) absmax[b] = am;
        const uint32_t bi = nearest(v[k] / am);
        const uint32_t odd = (uint32_t)__shfl_down((int)bi, 1, 64);
        if ((lane & 1) == 0)
          packed[b * 32 + (lane >> 1)] = (uint8_t)(order ? ((bi << 4) | odd) : (bi | (odd << 4)));
      }
    }
    return;
  }
  for (int64_t b = (int64_t)blockIdx.x * (CODEC_NT / 64) + (threadIdx.x >> 6); b < nblocks; b += waves) {
    const int64_t base = b * block;
    float m = 0.0f;
    for (int i = lane; i < block; i += 64) m = fmaxf(m, fabsf(load(base + i)));
    m = wave_max(m);
    const float am = fmaxf(m, 1.17549435e-38f);
    if (lane == 0) absmax[b] = am;
    // pairs: lane handles elements (2j, 2j+1) of the block
    for (int j = lane; j < block / 2; j += 64) {
      uint32_t idx[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) idx[t] = nearest(load(base + 2 * j + t) / am);
      packed[(base >> 1) + j] = (uint8_t)(order ? ((idx[0] << 4) | idx[1]) : (idx[0] | (idx[1] << 4)));
    }
  }
}

// ------------------------------------------------------------ double quantise
// offset = fp32(S / n) with S the fp64 sum in a fixed tree: each workgroup
// sums a chunk of 4096 values (thread t adds values 16t..16t+15 left to right,
// then a halving tree over the 256 threads); chunk sums are added left to right.
constexpr int DQ_CHUNK = 4096;

__global__ __launch_bounds__(CODEC_NT) void dq_chunk_sum_kernel(const float* __restrict__ a, int64_t n,
                                                                double* __restrict__ partial) {
  __shared__ double red[CODEC_NT];
  const int64_t base = (int64_t)blockIdx.x * DQ_CHUNK + threadIdx.x * 16;
  double s = 0.0;
  for (int i = 0; i < 16; ++i) {
    const int64_t k = base + i;
    s += k < n ? (double)a[k] : 0.0;
  }
  red[threadIdx.x] = s;
  __syncthreads();
  for (int stride = CODEC_NT / 2; stride >= 1; stride >>= 1) {
    if (threadIdx.x < stride) red[threadIdx.x] += red[threadIdx.x + stride];
    __syncthreads();
  }
  if (threadIdx.x == 0) partial[blockIdx.x] = red[0];
}

// One wave: the chunk sums are fetched 64 at a time into LDS (so the loads
// overlap), then lane 0 adds them left to right, the order the sum is defined by.
__global__ void dq_offset_kernel(const double* __restrict__ partial, int64_t chunks, int64_t n,
                                 float* __restrict__ offset) {
  __shared__ double stage[64];
  const int lane = threadIdx.x;
  double s = 0.0;
  for (int64_t base = 0; base < chunks; base += 64) {
    const int64_t i = base + lane;
    stage[lane] = i < chunks ? partial[i] : 0.0;
    __syncthreads();
    if (lane == 0) {
      const int64_t cnt = chunks - base < 64 ? chunks - base : 64;
      for (int64_t k = 0; k < cnt; ++k) s += stage[k];
    }
    __syncthreads();
  }
  if (lane == 0) *offset = (float)(s / (double)n);
}

// One workgroup per dq block (<= 256 values): absmax2 over |absmax - offset|,
// then the first index of the nearest code2 entry for each value.
__global__ __launch_bounds__(CODEC_NT) void dq_quant_kernel(const float* __restrict__ a, int64_t n, int dq,
                                                            const float* __restrict__ code2,
                                                            const float* __restrict__ offset,
                                                            uint8_t* __restrict__ q,
                                                            float* __restrict__ absmax2) {
  __shared__ float cb[256];
  __shared__ float wmax[CODEC_NT / 64];
  cb[threadIdx.x] = code2[threadIdx.x];
  const float off = *offset;
  const int64_t b = blockIdx.x;
  float mx = 0.0f;
  for (int i = threadIdx.x; i < dq; i += CODEC_NT) {
    const int64_t k = b * dq + i;
    if (k < n) mx = fmaxf(mx, fabsf(a[k] - off));
  }
  mx = wave_max(mx);
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = mx;
  __syncthreads();
  float am = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  am = fmaxf(am, 1.17549435e-38f);
  if (threadIdx.x == 0) absmax2[b] = am;
  for (int i = threadIdx.x; i < dq; i += CODEC_NT) {
    const int64_t k = b * dq + i;
    if (k >= n) continue;
    const float nv = (a[k] - off) / am;
    float best = fabsf(nv - cb[0]);
    int bi = 0;
    for (int c = 1; c < 256; ++c) {
      const float d = fabsf(nv - cb[c]);
      if (d < best) { best = d; bi = c; }
    }
    q[k] = (uint8_t)bi;
  }
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// log2(v) for a power of two, else -1.
int pow2_shift(int64_t v) {
  if (v <= 0 || (v & (v - 1)) != 0) return -1;
  int s = 0;
  while ((int64_t{1} << s) < v) ++s;
  return s;
}

int make_scale_src(const molt_nf4_weight* w, ScaleSrc& s, const char* who) {
  s = ScaleSrc{};
  s.nested = w->nested != 0;
  if (s.nested) {
    MOLT_REQUIRE(w->absmax_q && w->absmax2 && w->code2 && w->dq_block > 0, MOLT_EINVAL,
                 "%s: nested statistics incomplete", who);
    s.q = w->absmax_q; s.absmax2 = w->absmax2; s.code2 = w->code2; s.offset = w->offset;
    s.dq_block = w->dq_block;
    s.dq_shift = pow2_shift(w->dq_block);
  } else {
    MOLT_REQUIRE(w->scales, MOLT_EINVAL, "%s: scales missing", who);
    s.scales = w->scales;
  }
  return MOLT_OK;
}

unsigned grid_for(int64_t items, int64_t per_block) {
  int64_t g = (items + per_block - 1) / per_block;
  if (g > 8192) g = 8192;
  if (g < 1) g = 1;
  return (unsigned)g;
}

}  // namespace
}  // namespace molt

using namespace molt;

extern "C" int molt_nf4_dequantize(const molt_nf4_weight* w, void* out, int32_t out_dtype, void* stream) {
  const char* who = "molt_nf4_dequantize";
  MOLT_REQUIRE(w && w->packed && w->code && out, MOLT_EINVAL, "%s: null argument", who);
  MOLT_REQUIRE(out_dtype == MOLT_DTYPE_BF16 || out_dtype == MOLT_DTYPE_F32, MOLT_EINVAL, "%s: bad dtype", who);
  MOLT_REQUIRE(w->rows >= 0 && w->cols >= 0 && w->block_size > 0, MOLT_EINVAL, "%s: bad shape", who);
  MOLT_REQUIRE(w->nibble_order == 0 || w->nibble_order == 1, MOLT_EINVAL, "%s: bad nibble order", who);
  ScaleSrc ss;
  int rc = make_scale_src(w, ss, who);
  if (rc) return rc;
  const int64_t n = w->rows * w->cols;
  if (n == 0) return MOLT_OK;
  MOLT_REQUIRE(aligned(w->packed, 16), MOLT_EINVAL, "%s: packed data must be 16-byte aligned", who);
  MOLT_REQUIRE(aligned(out, 16), MOLT_EINVAL, "%s: output must be 16-byte aligned", who);
  const bool blk8 = w->block_size % 8 == 0;
  const unsigned grid = grid_for(ceil_div64((n + 7) / 8, DQ_UPT), CODEC_NT);
  hipStream_t st = (hipStream_t)stream;
#define MOLT_DQ(F32, B32)                                                                        \
  hipLaunchKernelGGL((dequant_kernel<F32, B32>), dim3(grid), dim3(CODEC_NT), 0, st, w->packed, ss, \
                     w->code, w->nibble_order, n, w->block_size, pow2_shift(w->block_size), out)
  if (out_dtype == MOLT_DTYPE_F32) {
    if (blk8) MOLT_DQ(1, true); else MOLT_DQ(1, false);
  } else {
    if (blk8) MOLT_DQ(0, true); else MOLT_DQ(0, false);
  }
#undef MOLT_DQ
  return check_launch(who);
}

extern "C" int molt_nf4_resolve_scales(const molt_nf4_weight* w, float* out, void* stream) {
  const char* who = "molt_nf4_resolve_scales";
  MOLT_REQUIRE(w && out && w->block_size > 0, MOLT_EINVAL, "%s: null argument", who);
  ScaleSrc ss;
  int rc = make_scale_src(w, ss, who);
  if (rc) return rc;
  const int64_t nblocks = ceil_div64(w->rows * w->cols, w->block_size);
  if (nblocks == 0) return MOLT_OK;
  hipLaunchKernelGGL(resolve_kernel, dim3(grid_for(nblocks, 256)), dim3(256), 0, (hipStream_t)stream, ss,
                     nblocks, out);
  return check_launch(who);
}

extern "C" int molt_nf4_quantize(const void* x, int32_t x_dtype, int64_t n, int32_t block_size,
                                 int32_t nibble_order, const float* code, uint8_t* packed, float* absmax,
                                 void* stream) {
  const char* who = "molt_nf4_quantize";
  MOLT_REQUIRE(x && code && packed && absmax, MOLT_EINVAL, "%s: null argument", who);
  MOLT_REQUIRE(n > 0 && block_size >= 16 && block_size % 2 == 0, MOLT_EINVAL,
               "%s: invalid tensor or NF4 block size", who);
  MOLT_REQUIRE(x_dtype == MOLT_DTYPE_BF16 || x_dtype == MOLT_DTYPE_F32, MOLT_EINVAL, "%s: bad dtype", who);
  MOLT_REQUIRE(nibble_order == 0 || nibble_order == 1, MOLT_EINVAL, "%s: bad nibble order", who);
  const int64_t nblocks = ceil_div64(n, block_size);
  const unsigned grid = grid_for(nblocks, CODEC_NT / 64);
  hipStream_t st = (hipStream_t)stream;
  if (x_dtype == MOLT_DTYPE_BF16)
    hipLaunchKernelGGL((quantize_kernel<1>), dim3(grid), dim3(CODEC_NT), 0, st, x, n, block_size, nibble_order,
                       code, packed, absmax, nblocks);
  else
    hipLaunchKernelGGL((quantize_kernel<0>), dim3(grid), dim3(CODEC_NT), 0, st, x, n, block_size, nibble_order,
                       code, packed, absmax, nblocks);
  return check_launch(who);
}

extern "C" size_t molt_nf4_double_quantize_workspace(int64_t n) {
  if (n <= 0) return 0;
  return (size_t)ceil_div64(n, DQ_CHUNK) * sizeof(double);
}

extern "C" int molt_nf4_double_quantize(const float* absmax, int64_t n, int32_t dq_block, const float* code2,
                                        uint8_t* q, float* absmax2, float* offset_out, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  const char* who = "molt_nf4_double_quantize";
  MOLT_REQUIRE(absmax && code2 && q && absmax2 && offset_out, MOLT_EINVAL, "%s: null argument", who);
  MOLT_REQUIRE(n > 0 && dq_block > 0 && dq_block <= 4096, MOLT_EINVAL, "%s: bad shape", who);
  const int64_t chunks = ceil_div64(n, DQ_CHUNK);
  MOLT_REQUIRE(workspace && workspace_bytes >= (size_t)chunks * sizeof(double), MOLT_EWORKSPACE,
               "%s: workspace too small", who);
  MOLT_REQUIRE(aligned(workspace, 8), MOLT_EINVAL, "%s: workspace must be 8-byte aligned", who);
  hipStream_t st = (hipStream_t)stream;
  double* partial = (double*)workspace;
  hipLaunchKernelGGL(dq_chunk_sum_kernel, dim3((unsigned)chunks), dim3(CODEC_NT), 0, st, absmax, n, partial);
  int rc = check_launch(who);
  if (rc) return rc;
  hipLaunchKernelGGL(dq_offset_kernel, dim3(1), dim3(64), 0, st, partial, chunks, n, offset_out);
  rc = check_launch(who);
  if (rc) return rc;
  const int64_t nb = ceil_div64(n, dq_block);
  MOLT_REQUIRE(nb < (1ll << 31), MOLT_EINVAL, "%s: too many blocks", who);
  hipLaunchKernelGGL(dq_quant_kernel, dim3((unsigned)nb), dim3(CODEC_NT), 0, st, absmax, n, dq_block, code2,
                     offset_out, q, absmax2);
  return check_launch(who);
}
