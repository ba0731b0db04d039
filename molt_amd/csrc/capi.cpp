// C ABI glue: thread-local error reporting and the NF4+LoRA GEMM entry points
// declared in include/molt_amd.h (the kernels live in nf4_gemm.hip).
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include <atomic>

#include "../../include/molt_amd.h"
#include "common.h"

namespace molt {

static thread_local char g_last_error[512] = "";
static thread_local void* g_gemm_events[2] = {nullptr, nullptr};

void take_gemm_events(void** start, void** end) {
  *start = g_gemm_events[0];
  *end = g_gemm_events[1];
  g_gemm_events[0] = g_gemm_events[1] = nullptr;
}

// A GEMM entry point that returns before reaching its implementation still
// consumes the events armed for it.
static int drop_gemm_events(int rc) {
  g_gemm_events[0] = g_gemm_events[1] = nullptr;
  return rc;
}

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(MOLT_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return MOLT_OK;
}

// Kernel-choice settings: initialised from the environment once (a function-
// local static, so the first use from any thread reads it exactly once), then
// changed only through molt_amd_set_tuning. Entry points read them with one
// relaxed atomic load per call.
namespace {
struct Tuning {
  std::atomic<int64_t> v[6];
  Tuning() {
    const char* e = getenv("MOLT_AMD_BIG_TILE_MIN");
    v[MOLT_TUNE_BIG_TILE_MIN].store(e ? atoll(e) : 256);
    e = getenv("MOLT_AMD_GEMV_DOT_M");
    const int64_t m = e ? atoll(e) : -1;
    v[MOLT_TUNE_GEMV_DOT_M].store(m < -1 ? -1 : (m > 8 ? 8 : m));
    v[MOLT_TUNE_LORA_DMA].store(getenv("MOLT_AMD_PJ_NODMA") ? 0 : 1);
    v[MOLT_TUNE_SPLIT_K].store(getenv("MOLT_AMD_NO_SPLIT_K") ? 0 : 1);
    e = getenv("MOLT_AMD_SPLIT_MIN_STEPS");
    const int64_t ms = e ? atoll(e) : 8;
    v[MOLT_TUNE_SPLIT_MIN_STEPS].store(ms < 2 ? 2 : ms);
    e = getenv("MOLT_AMD_STAGE_MIN_MTILES");
    const int64_t st = e ? atoll(e) : 16;
    v[MOLT_TUNE_STAGE_MIN_MTILES].store(st < 0 ? 0 : st);
  }
};
Tuning& tuning() {
  static Tuning t;
  return t;
}
bool tuning_ok(int32_t key, int64_t value) {
  switch (key) {
    case MOLT_TUNE_BIG_TILE_MIN: return value >= 0;
    case MOLT_TUNE_GEMV_DOT_M: return value >= -1 && value <= 8;
    case MOLT_TUNE_LORA_DMA: return value == 0 || value == 1;
    case MOLT_TUNE_SPLIT_K: return value == 0 || value == 1;
    case MOLT_TUNE_SPLIT_MIN_STEPS: return value >= 2 && value <= 4096;
    case MOLT_TUNE_STAGE_MIN_MTILES: return value >= 0;
    default: return false;
  }
}
}  // namespace

int64_t tuning_value(int32_t key) { return tuning().v[key].load(std::memory_order_relaxed); }

int device_cus() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

}  // namespace molt

extern "C" int molt_nf4_lora_forward_impl(const uint16_t* x, int64_t ldx, int64_t M, const molt_nf4_weight* w0,
                                          const molt_nf4_weight* w1, const uint16_t* t, int64_t ldt, int lr,
                                          const float* b0, const float* b1, int64_t ldb, int r, float s0, float s1,
                                          uint16_t* y0, uint16_t* y1, uint16_t* y2, int64_t ldy,
                                          const molt::WtHandoff* wt, void* workspace, size_t workspace_bytes,
                                          hipStream_t stream);
extern "C" int molt_nf4_lora_backward_impl(const uint16_t* dy0, const uint16_t* dy1, int64_t lddy, int64_t M,
                                           const molt_nf4_weight* w0, const molt_nf4_weight* w1,
                                           const uint16_t* u0, const uint16_t* u1, int64_t ldu, const float* a0,
                                           const float* a1, int64_t lda, int r, float lora_scale, uint16_t* dx,
                                           int64_t lddx, const uint16_t* gate, const uint16_t* up, uint16_t* dg, uint16_t* du,
                                           int64_t ldg, const molt::WtHandoff* wt, void* workspace,
                                           size_t workspace_bytes, hipStream_t stream);

extern "C" int molt_nf4_stacked_forward_impl(const uint16_t* x, int64_t ldx, int64_t M, int32_t nw,
                                             const molt_nf4_weight* w, const uint16_t* t, int64_t ldt, int32_t lr,
                                             const float* b, int64_t ldb, float s, uint16_t* y, int64_t ldy,
                                             uint16_t* wt_out, int32_t* wt_written, void* workspace,
                                             size_t workspace_bytes, hipStream_t stream);

extern "C" {

const char* molt_amd_last_error(void) { return molt::g_last_error; }

const char* molt_amd_version(void) { return "molt_amd 0.3.0 gfx950"; }

int molt_amd_set_tuning(int32_t key, int64_t value) {
  if (!molt::tuning_ok(key, value))
    return molt::set_error(MOLT_EINVAL, "molt_amd_set_tuning: key %d does not accept %lld", key, (long long)value);
  molt::tuning().v[key].store(value, std::memory_order_relaxed);
  return MOLT_OK;
}

int64_t molt_amd_get_tuning(int32_t key) {
  return key >= 0 && key <= MOLT_TUNE_STAGE_MIN_MTILES ? molt::tuning_value(key) : -2;
}

int molt_amd_time_next_gemm(void* start_event, void* end_event) {
  molt::g_gemm_events[0] = start_event;
  molt::g_gemm_events[1] = end_event;
  return MOLT_OK;
}

int molt_nf4_lora_forward(const uint16_t* x, int64_t ldx, int64_t M, const molt_nf4_weight* w,
                          const uint16_t* t, int64_t ldt, const float* lora_b, int32_t r, float scaling,
                          uint16_t* y, int64_t ldy, void* workspace, size_t workspace_bytes, void* stream) {
  if (!w)
    return molt::drop_gemm_events(molt::set_error(MOLT_EINVAL, "molt_nf4_lora_forward: null weight"));
  return molt_nf4_lora_forward_impl(x, ldx, M, w, nullptr, t, ldt, r, lora_b, nullptr, r, r, scaling, scaling,
                                    y, nullptr, nullptr, ldy, nullptr, workspace, workspace_bytes,
                                    (hipStream_t)stream);
}

int molt_nf4_gateup_forward(const uint16_t* x, int64_t ldx, int64_t M, const molt_nf4_weight* wg,
                            const molt_nf4_weight* wu, const uint16_t* t, int64_t ldt, const float* bg,
                            const float* bu, int32_t r, float sg, float su, uint16_t* gate, uint16_t* up,
                            uint16_t* h, int64_t ldo, void* workspace, size_t workspace_bytes, void* stream) {
  if (!wg || !wu)
    return molt::drop_gemm_events(molt::set_error(MOLT_EINVAL, "molt_nf4_gateup_forward: null weight"));
  return molt_nf4_lora_forward_impl(x, ldx, M, wg, wu, t, ldt, 2 * r, bg, bu, r, r, sg, su, gate, up, h, ldo,
                                    nullptr, workspace, workspace_bytes, (hipStream_t)stream);
}

int molt_nf4_lora_backward_input(const uint16_t* dy, int64_t lddy, int64_t M, const molt_nf4_weight* w,
                                 const uint16_t* u, int64_t ldu, const float* lora_a, int32_t r, float lora_scale,
                                 uint16_t* dx, int64_t lddx, void* workspace, size_t workspace_bytes, void* stream) {
  if (!w)
    return molt::drop_gemm_events(molt::set_error(MOLT_EINVAL, "molt_nf4_lora_backward_input: null weight"));
  return molt_nf4_lora_backward_impl(dy, nullptr, lddy, M, w, nullptr, u, nullptr, ldu, lora_a, nullptr, w->cols,
                                     r, lora_scale, dx, lddx, nullptr, nullptr, nullptr, nullptr, 0, nullptr,
                                     workspace, workspace_bytes, (hipStream_t)stream);
}

int molt_nf4_lora_backward_input_pair(const uint16_t* dy0, const uint16_t* dy1, int64_t lddy, int64_t M,
                                      const molt_nf4_weight* w0, const molt_nf4_weight* w1, const uint16_t* u0,
                                      const uint16_t* u1, int64_t ldu, const float* a0, const float* a1,
                                      int32_t r, uint16_t* dx, int64_t lddx, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  if (!w0 || !w1)
    return molt::drop_gemm_events(molt::set_error(MOLT_EINVAL, "molt_nf4_lora_backward_input_pair: null weight"));
  return molt_nf4_lora_backward_impl(dy0, dy1, lddy, M, w0, w1, u0, u1, ldu, a0, a1, w0->cols, r, 1.0f, dx, lddx,
                                     nullptr, nullptr, nullptr, nullptr, 0, nullptr, workspace, workspace_bytes,
                                     (hipStream_t)stream);
}

int molt_nf4_swiglu_backward(const uint16_t* dy, int64_t lddy, int64_t M, const molt_nf4_weight* wd,
                             const uint16_t* u, int64_t ldu, const float* lora_a, int32_t r, const uint16_t* gate,
                             const uint16_t* up, int64_t ldg, uint16_t* dgate, uint16_t* dup, void* workspace,
                             size_t workspace_bytes, void* stream) {
  if (!wd)
    return molt::drop_gemm_events(molt::set_error(MOLT_EINVAL, "molt_nf4_swiglu_backward: null weight"));
  if (M == 0) return molt::drop_gemm_events(MOLT_OK);   // an empty token batch: the outputs are empty too
  if (!dgate)
    return molt::drop_gemm_events(molt::set_error(MOLT_EINVAL, "molt_nf4_swiglu_backward: null dgate"));
  return molt_nf4_lora_backward_impl(dy, nullptr, lddy, M, wd, nullptr, u, nullptr, ldu, lora_a, nullptr, wd->cols,
                                     r, 1.0f, nullptr, 0, gate, up, dgate, dup, ldg, nullptr, workspace,
                                     workspace_bytes, (hipStream_t)stream);
}

int molt_nf4_lora_forward_keep_wt(const uint16_t* x, int64_t ldx, int64_t M, const molt_nf4_weight* w,
                                  const uint16_t* t, int64_t ldt, const float* lora_b, int32_t r, float scaling,
                                  uint16_t* y, int64_t ldy, uint16_t* wt, int32_t* wt_written, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  if (wt_written) *wt_written = 0;
  if (!w)
    return molt::drop_gemm_events(molt::set_error(MOLT_EINVAL, "molt_nf4_lora_forward_keep_wt: null weight"));
  const molt::WtHandoff h{{wt, wt}, wt_written, {nullptr, nullptr}};
  return molt_nf4_lora_forward_impl(x, ldx, M, w, nullptr, t, ldt, r, lora_b, nullptr, r, r, scaling, scaling,
                                    y, nullptr, nullptr, ldy, &h, workspace, workspace_bytes, (hipStream_t)stream);
}

int molt_nf4_gateup_forward_keep_wt(const uint16_t* x, int64_t ldx, int64_t M, const molt_nf4_weight* wg,
                                    const molt_nf4_weight* wu, const uint16_t* t, int64_t ldt, const float* bg,
                                    const float* bu, int32_t r, float sg, float su, uint16_t* gate, uint16_t* up,
                                    uint16_t* h, int64_t ldo, uint16_t* wgt, uint16_t* wut, int32_t* wt_written,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  if (wt_written) *wt_written = 0;
  if (!wg || !wu)
    return molt::drop_gemm_events(molt::set_error(MOLT_EINVAL, "molt_nf4_gateup_forward_keep_wt: null weight"));
  const molt::WtHandoff ho{{wgt, wut}, wt_written, {nullptr, nullptr}};
  return molt_nf4_lora_forward_impl(x, ldx, M, wg, wu, t, ldt, 2 * r, bg, bu, r, r, sg, su, gate, up, h, ldo,
                                    &ho, workspace, workspace_bytes, (hipStream_t)stream);
}

int molt_nf4_lora_backward_input_wt(const uint16_t* dy, int64_t lddy, int64_t M, const molt_nf4_weight* w,
                                    const uint16_t* wt, const uint16_t* u, int64_t ldu, const float* lora_a,
                                    int32_t r, float lora_scale, uint16_t* dx, int64_t lddx, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  if (!w)
    return molt::drop_gemm_events(molt::set_error(MOLT_EINVAL, "molt_nf4_lora_backward_input_wt: null weight"));
  const molt::WtHandoff h{{nullptr, nullptr}, nullptr, {wt, wt}};
  return molt_nf4_lora_backward_impl(dy, nullptr, lddy, M, w, nullptr, u, nullptr, ldu, lora_a, nullptr, w->cols,
                                     r, lora_scale, dx, lddx, nullptr, nullptr, nullptr, nullptr, 0, &h,
                                     workspace, workspace_bytes, (hipStream_t)stream);
}

int molt_nf4_lora_backward_input_pair_wt(const uint16_t* dy0, const uint16_t* dy1, int64_t lddy, int64_t M,
                                         const molt_nf4_weight* w0, const molt_nf4_weight* w1, const uint16_t* wt0,
                                         const uint16_t* wt1, const uint16_t* u0, const uint16_t* u1, int64_t ldu,
                                         const float* a0, const float* a1, int32_t r, uint16_t* dx, int64_t lddx,
                                         void* workspace, size_t workspace_bytes, void* stream) {
  if (!w0 || !w1)
    return molt::drop_gemm_events(
        molt::set_error(MOLT_EINVAL, "molt_nf4_lora_backward_input_pair_wt: null weight"));
  const molt::WtHandoff h{{nullptr, nullptr}, nullptr, {wt0, wt1}};
  return molt_nf4_lora_backward_impl(dy0, dy1, lddy, M, w0, w1, u0, u1, ldu, a0, a1, w0->cols, r, 1.0f, dx, lddx,
                                     nullptr, nullptr, nullptr, nullptr, 0, &h, workspace, workspace_bytes,
                                     (hipStream_t)stream);
}

int molt_nf4_swiglu_backward_wt(const uint16_t* dy, int64_t lddy, int64_t M, const molt_nf4_weight* wd,
                                const uint16_t* wdt, const uint16_t* u, int64_t ldu, const float* lora_a, int32_t r,
                                const uint16_t* gate, const uint16_t* up, int64_t ldg, uint16_t* dgate,
                                uint16_t* dup, void* workspace, size_t workspace_bytes, void* stream) {
  if (!wd)
    return molt::drop_gemm_events(molt::set_error(MOLT_EINVAL, "molt_nf4_swiglu_backward_wt: null weight"));
  if (M == 0) return molt::drop_gemm_events(MOLT_OK);
  if (!dgate)
    return molt::drop_gemm_events(molt::set_error(MOLT_EINVAL, "molt_nf4_swiglu_backward_wt: null dgate"));
  const molt::WtHandoff h{{nullptr, nullptr}, nullptr, {wdt, wdt}};
  return molt_nf4_lora_backward_impl(dy, nullptr, lddy, M, wd, nullptr, u, nullptr, ldu, lora_a, nullptr, wd->cols,
                                     r, 1.0f, nullptr, 0, gate, up, dgate, dup, ldg, &h, workspace,
                                     workspace_bytes, (hipStream_t)stream);
}

int molt_nf4_stacked_forward(const uint16_t* x, int64_t ldx, int64_t M, int32_t nw, const molt_nf4_weight* w,
                             const uint16_t* t, int64_t ldt, int32_t lr, const float* b_blocks, int64_t ldb,
                             float scaling, uint16_t* y, int64_t ldy, uint16_t* wt, int32_t* wt_written,
                             void* workspace, size_t workspace_bytes, void* stream) {
  return molt_nf4_stacked_forward_impl(x, ldx, M, nw, w, t, ldt, lr, b_blocks, ldb, scaling, y, ldy, wt, wt_written,
                                       workspace, workspace_bytes, (hipStream_t)stream);
}

int molt_nf4_stacked_backward_input(const uint16_t* dy, int64_t lddy, int64_t M, int32_t nw,
                                    const molt_nf4_weight* w, const uint16_t* wt, const uint16_t* u, int64_t ldu,
                                    const float* a_stack, int32_t r, float lora_scale, uint16_t* dx, int64_t lddx,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  const char* who = "molt_nf4_stacked_backward_input";
  if (!w || nw < 1 || nw > 8)
    return molt::drop_gemm_events(molt::set_error(MOLT_EINVAL, "%s: 1..8 weights", who));
  if (!wt)
    return molt::drop_gemm_events(
        molt::set_error(MOLT_EINVAL, "%s: the forward's transposed weight is required", who));
  // the stack's shape and format in one descriptor: the GEMM reads wt, not the packed data
  molt_nf4_weight stack = w[0];
  stack.rows = 0;
  for (int i = 0; i < nw; ++i) {
    if (w[i].cols != w[0].cols || w[i].block_size != w[0].block_size || w[i].nibble_order != w[0].nibble_order ||
        w[i].code != w[0].code)
      return molt::drop_gemm_events(molt::set_error(
          MOLT_EINVAL, "%s: stacked weights must share columns, block size, nibble order and code table", who));
    stack.rows += w[i].rows;
  }
  const molt::WtHandoff h{{nullptr, nullptr}, nullptr, {wt, wt}, 1};
  return molt_nf4_lora_backward_impl(dy, nullptr, lddy, M, &stack, nullptr, u, nullptr, ldu, a_stack, nullptr,
                                     stack.cols, r, lora_scale, dx, lddx, nullptr, nullptr, nullptr, nullptr, 0, &h,
                                     workspace, workspace_bytes, (hipStream_t)stream);
}

}  // extern "C"
