// Standalone SwiGLU elementwise kernels (gfx950), the fused_silu_multiply op
// (kernels/gated_activation.py:29-51): fp32 math, stored in the input dtype.
#include "common.h"

namespace molt {
namespace {

constexpr int SW_NT = 256;

MOLT_DEV float sigm(float g) { return 1.0f / (1.0f + __expf(-g)); }

template <bool BF16>
MOLT_DEV float ld(const void* p, int64_t i) {
  if (BF16) return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
  return reinterpret_cast<const float*>(p)[i];
}

template <bool BF16>
MOLT_DEV void st(void* p, int64_t i, float v) {
  if (BF16) reinterpret_cast<uint16_t*>(p)[i] = bf16_bits(v);
  else reinterpret_cast<float*>(p)[i] = v;
}

template <bool BF16, bool ROUND_SILU>
__global__ __launch_bounds__(SW_NT) void silu_mul_fwd_kernel(const void* __restrict__ g, const void* __restrict__ u,
                                                             void* __restrict__ h, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * SW_NT + threadIdx.x; i < n; i += (int64_t)gridDim.x * SW_NT) {
    const float gv = ld<BF16>(g, i), uv = ld<BF16>(u, i);
    const float sv = gv * sigm(gv);
    st<BF16>(h, i, (ROUND_SILU ? round_bf16(sv) : sv) * uv);
  }
}

template <bool BF16>
__global__ __launch_bounds__(SW_NT) void silu_mul_bwd_kernel(const void* __restrict__ dh, const void* __restrict__ g,
                                                             const void* __restrict__ u, void* __restrict__ dg,
                                                             void* __restrict__ du, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * SW_NT + threadIdx.x; i < n; i += (int64_t)gridDim.x * SW_NT) {
    const float d = ld<BF16>(dh, i), gv = ld<BF16>(g, i), uv = ld<BF16>(u, i);
    const float sg = sigm(gv);
    st<BF16>(dg, i, d * uv * (sg * (1.0f + gv * (1.0f - sg))));
    st<BF16>(du, i, d * (gv * sg));
  }
}

unsigned sw_grid(int64_t n) {
  int64_t g = (n + SW_NT - 1) / SW_NT;
  if (g > 16384) g = 16384;
  return (unsigned)(g < 1 ? 1 : g);
}

}  // namespace
}  // namespace molt

using namespace molt;

extern "C" int molt_silu_mul_forward(const void* gate, const void* up, void* out, int64_t n, int32_t dtype,
                                     int32_t round_silu, void* stream) {
  const char* who = "molt_silu_mul_forward";
  MOLT_REQUIRE(n >= 0 && (n == 0 || (gate && up && out)), MOLT_EINVAL, "%s: bad arguments", who);
  MOLT_REQUIRE(dtype == MOLT_DTYPE_BF16 || dtype == MOLT_DTYPE_F32, MOLT_EINVAL, "%s: bad dtype", who);
  if (n == 0) return MOLT_OK;
  MOLT_REQUIRE(round_silu == 0 || dtype == MOLT_DTYPE_BF16, MOLT_EINVAL, "%s: round_silu needs bf16", who);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == MOLT_DTYPE_BF16 && round_silu)
    hipLaunchKernelGGL((silu_mul_fwd_kernel<true, true>), dim3(sw_grid(n)), dim3(SW_NT), 0, st, gate, up, out, n);
  else if (dtype == MOLT_DTYPE_BF16)
    hipLaunchKernelGGL((silu_mul_fwd_kernel<true, false>), dim3(sw_grid(n)), dim3(SW_NT), 0, st, gate, up, out, n);
  else
    hipLaunchKernelGGL((silu_mul_fwd_kernel<false, false>), dim3(sw_grid(n)), dim3(SW_NT), 0, st, gate, up, out, n);
  return check_launch(who);
}

extern "C" int molt_silu_mul_backward(const void* grad, const void* gate, const void* up, void* dgate, void* dup,
                                      int64_t n, int32_t dtype, void* stream) {
  const char* who = "molt_silu_mul_backward";
  MOLT_REQUIRE(n >= 0 && (n == 0 || (grad && gate && up && dgate && dup)), MOLT_EINVAL, "%s: bad arguments", who);
  MOLT_REQUIRE(dtype == MOLT_DTYPE_BF16 || dtype == MOLT_DTYPE_F32, MOLT_EINVAL, "%s: bad dtype", who);
  if (n == 0) return MOLT_OK;
  if (dtype == MOLT_DTYPE_BF16)
    hipLaunchKernelGGL((silu_mul_bwd_kernel<true>), dim3(sw_grid(n)), dim3(SW_NT), 0, (hipStream_t)stream, grad, gate,
                       up, dgate, dup, n);
  else
    hipLaunchKernelGGL((silu_mul_bwd_kernel<false>), dim3(sw_grid(n)), dim3(SW_NT), 0, (hipStream_t)stream, grad,
                       gate, up, dgate, dup, n);
  return check_launch(who);
}
