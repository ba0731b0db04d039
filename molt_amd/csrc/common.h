// Shared device/host helpers for the MI355X (gfx950) NF4 QLoRA kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/molt_amd.h"

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

#define MOLT_DEV __device__ __forceinline__

// ---------------------------------------------------------------------------
// bf16 conversion. fp32 -> bf16 is round-to-nearest-even (v_cvt_pk_bf16_f32),
// the same rounding torch applies in `.to(torch.bfloat16)`.
// ---------------------------------------------------------------------------
MOLT_DEV uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  f32x2_t v = {lo, hi};
  bf16x2_t r = __builtin_convertvector(v, bf16x2_t);
  return __builtin_bit_cast(uint32_t, r);
}

MOLT_DEV uint16_t bf16_bits(float x) {
  return __builtin_bit_cast(uint16_t, (__bf16)x);
}

MOLT_DEV float bf16_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
MOLT_DEV float bf16_hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }
MOLT_DEV float bf16_to_f32(uint16_t b) { return __builtin_bit_cast(float, ((uint32_t)b) << 16); }
MOLT_DEV float round_bf16(float x) { return bf16_to_f32(bf16_bits(x)); }

MOLT_DEV float fast_sigmoid(float x) { return 1.0f / (1.0f + __expf(-x)); }

// ---------------------------------------------------------------------------
// Host-side status plumbing (thread-local last error, see molt_amd_last_error).
// ---------------------------------------------------------------------------
namespace molt {
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
int64_t tuning_value(int32_t key);   // a MOLT_TUNE_* setting (molt_amd_set_tuning)
int device_cus();                    // compute units of the current device, cached per device
// Events registered by molt_amd_time_next_gemm for this thread (null if none);
// taking them clears the registration.
void take_gemm_events(void** start, void** end);
// deq(W)^T copies handed from a forward GEMM to the input gradient of the same
// weights (bf16 [K, N], row stride N, one per weight): `out` asks a forward to
// write them, `written` (host memory) tells whether it did, `in` gives them to
// an input-gradient GEMM, which then does not stage the weights itself.
// `required`: the input gradient must read `in` (the weight descriptor then
// only carries the shape and format); a plan that would not is refused before
// any launch.
struct WtHandoff {
  uint16_t* out[2];
  int32_t* written;
  const uint16_t* in[2];
  int32_t required;
};
}  // namespace molt

#define MOLT_REQUIRE(cond, code, ...)              \
  do {                                             \
    if (!(cond)) return molt::set_error((code), __VA_ARGS__); \
  } while (0)

__host__ __device__ inline int64_t ceil_div64(int64_t a, int64_t b) { return (a + b - 1) / b; }
