/*
 * molt_amd.h - C ABI of the MI355X (gfx950) NF4 QLoRA hot-path library
 * (libmolt_amd.so).
 *
 * The reference (PraveenNimilka/MOLT) is Python; its hot path reaches GPU
 * code through bitsandbytes, cuBLAS (torch.nn.functional.linear under bf16
 * autocast) and two Triton kernels. Each entry point below replaces one of
 * those calls and cites it (paths relative to the reference's src/molt_stream/).
 *
 * Conventions
 *  - Plain device pointers, element counts, strides (in elements) and scalars.
 *    bf16 tensors are passed as uint16_t bit patterns.
 *  - Every entry point launches asynchronously on `stream` (a hipStream_t;
 *    NULL = the legacy default stream), never synchronises and never
 *    allocates: any workspace is passed in by the caller.
 *  - Return 0 on success or a MOLT_E* code; molt_amd_last_error() then holds a
 *    thread-local message. The only state kept between calls is the set of
 *    kernel-choice settings (molt_amd_set_tuning) and per-device constants.
 *  - NF4 weights: `rows x cols` row-major elements, two 4-bit codes per byte,
 *    `nibble_order` 1 = element 2i in the high nibble (bitsandbytes,
 *    methods/nf4_backward.py:97-98), 0 = element 2i in the low nibble
 *    (streaming/nf4.py:62). Blocks of `block_size` consecutive flat elements
 *    share one absmax. Dequantised value = bf16_rne(fp32(code[nibble] * scale)).
 */
#ifndef MOLT_AMD_H
#define MOLT_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOLT_OK 0
#define MOLT_EINVAL 1        /* bad shape, stride, pointer or argument */
#define MOLT_EUNSUPPORTED 2  /* valid request this library does not implement */
#define MOLT_ELAUNCH 3       /* the HIP runtime refused a launch */
#define MOLT_EWORKSPACE 4    /* caller workspace too small */

#define MOLT_DTYPE_BF16 0
#define MOLT_DTYPE_F32 1

/* A quantised NF4 matrix. Either `scales` (one fp32 per block) is set, or the
 * nested statistics (`absmax_q`, `absmax2`, `code2`, `offset`) are, with
 * scale = fp32(fp32(code2[absmax_q[b]] * absmax2[b / dq_block]) + offset)
 * (methods/nf4_backward.py:145-164). */
typedef struct molt_nf4_weight {
  const uint8_t* packed;
  const float* scales;
  const uint8_t* absmax_q;
  const float* absmax2;
  const float* code2;
  const float* code;       /* 16 fp32 NF4 levels (quant_state.code) */
  float offset;
  int32_t nested;
  int32_t block_size;
  int32_t dq_block;        /* nested block of absmax values (256) */
  int32_t nibble_order;
  int64_t rows;            /* N = out_features */
  int64_t cols;            /* K = in_features  */
} molt_nf4_weight;

/* ------------------------------------------------------------------------ */
/* Library                                                                   */
/* ------------------------------------------------------------------------ */
const char* molt_amd_last_error(void);
const char* molt_amd_version(void);

/* Kernel-choice settings. Each starts from its environment variable, read once
 * when the library first needs it, and can be changed at run time; the value in
 * force when an entry point is called applies to that call. No counterpart in
 * the reference (its kernel choices are Triton autotuning and fixed
 * geometries); used by tests and benchmarks to pin a kernel path.
 *   MOLT_TUNE_BIG_TILE_MIN  (MOLT_AMD_BIG_TILE_MIN, default 256): fewest
 *       256 x 256 output tiles for which the GEMMs use the large-tile kernels.
 *   MOLT_TUNE_GEMV_DOT_M    (MOLT_AMD_GEMV_DOT_M, default -1 = per-shape rule,
 *       else 0..8): largest token count for the streaming dot-product GEMV
 *       (5..8 tokens only where K <= 4096).
 *   MOLT_TUNE_LORA_DMA      (0 when MOLT_AMD_PJ_NODMA is set, else 1): LDS DMA
 *       staging in the LoRA projection and in the (plain-operand) LoRA
 *       gradient; 0 selects the register-staged kernels (same results).
 *   MOLT_TUNE_SPLIT_K       (0 when MOLT_AMD_NO_SPLIT_K is set, else 1): split
 *       the contraction of a long-K GEMM with few output tiles over
 *       workgroups (needs the caller's workspace, see below).
 *   MOLT_TUNE_SPLIT_MIN_STEPS (MOLT_AMD_SPLIT_MIN_STEPS, default 8, 2..4096):
 *       fewest 64-deep contraction steps per split range of a 256 x 256 tile;
 *       a 128 x 128 tile, a quarter of the work per step, takes a quarter.
 *   MOLT_TUNE_STAGE_MIN_MTILES (MOLT_AMD_STAGE_MIN_MTILES, default 16, 0 = never):
 *       fewest 256-row blocks of X (dY) for which the 256 x 256 kernels read
 *       the weight as a bf16 copy that one pass dequantises into the caller's
 *       workspace (transposed for the input gradient), instead of dequantising
 *       every weight tile again in each row block (see the workspace queries).
 * molt_amd_set_tuning returns MOLT_EINVAL for an unknown key or a value out of
 * range; molt_amd_get_tuning returns -2 for an unknown key. */
#define MOLT_TUNE_BIG_TILE_MIN 0
#define MOLT_TUNE_GEMV_DOT_M 1
#define MOLT_TUNE_LORA_DMA 2
#define MOLT_TUNE_SPLIT_K 3
#define MOLT_TUNE_SPLIT_MIN_STEPS 4
#define MOLT_TUNE_STAGE_MIN_MTILES 5
int molt_amd_set_tuning(int32_t key, int64_t value);
int64_t molt_amd_get_tuning(int32_t key);

/* Kernel timing: record the HIP events start_event and end_event (hipEvent_t)
 * on the call's stream immediately before and after the GEMM kernel launched
 * by the next NF4 GEMM entry point this thread calls (molt_nf4_lora_forward,
 * molt_nf4_gateup_forward, molt_nf4_lora_backward_input(_pair),
 * molt_nf4_swiglu_backward): not around its weight staging or split-K sum, so
 * hipEventElapsedTime gives that kernel's duration. No counterpart in the
 * reference; used by the benchmark. */
int molt_amd_time_next_gemm(void* start_event, void* end_event);

/* ------------------------------------------------------------------------ */
/* NF4 codec                                                                 */
/* ------------------------------------------------------------------------ */

/* Dense decode of an NF4 matrix to bf16 or fp32 (`out` holds rows*cols).
 * Replaces bitsandbytes.functional.dequantize_4bit at methods/nf4_lora.py:97-98,
 * methods/gated_replay.py:244, methods/nf4_layer_cache.py:51-53, and
 * NF4DevicePayload.dequantize at streaming/nf4.py:29-35. */
int molt_nf4_dequantize(const molt_nf4_weight* w, void* out, int32_t out_dtype, void* stream);

/* Nested absmax -> fp32 scale per block (`out` holds ceil(rows*cols/block_size)).
 * Replaces resolved_nf4_scales at methods/nf4_backward.py:145-164. */
int molt_nf4_resolve_scales(const molt_nf4_weight* w, float* out, void* stream);

/* Blockwise NF4 quantisation: fp32 absmax per block (clamped to FLT_MIN),
 * code = first index of the nearest code to fp32(x / absmax); zero padding to a
 * whole block. `packed` holds ceil(padded/2) bytes, `absmax` ceil(n/block) floats.
 * Replaces NF4Tensor.quantize (streaming/nf4.py:46-68) and the NF4 part of
 * bitsandbytes.functional.quantize_4bit (training/qlora.py:332-337). */
int molt_nf4_quantize(const void* x, int32_t x_dtype, int64_t n, int32_t block_size,
                      int32_t nibble_order, const float* code, uint8_t* packed,
                      float* absmax, void* stream);

/* Double quantisation of block absmax values (compress_statistics=True):
 * offset = fp32(fp64 sum / n); q = first index of the nearest code2 value to
 * fp32((absmax - offset) / absmax2[j]), absmax2[j] = max |absmax - offset| over
 * each `dq_block` values. `offset_out` is one device float. Needs
 * molt_nf4_double_quantize_workspace() bytes of workspace.
 * Replaces the nested statistics of bitsandbytes quantize_4bit (training/qlora.py:332-337). */
size_t molt_nf4_double_quantize_workspace(int64_t n);
int molt_nf4_double_quantize(const float* absmax, int64_t n, int32_t dq_block,
                             const float* code2, uint8_t* q, float* absmax2,
                             float* offset_out, void* workspace, size_t workspace_bytes,
                             void* stream);

/* ------------------------------------------------------------------------ */
/* NF4 + LoRA linear                                                         */
/* ------------------------------------------------------------------------ */

/* Low-rank projection out[M, r] = bf16( sum_d z(m, d) * bf16(lora[q, d]) ), r <= 128.
 *  z_mode 0: z = Z (bf16 [M, D], row stride ldz);
 *  z_mode 1: z = bf16(bf16(silu(Z)) * Z2) (SwiGLU replay; Z = gate, Z2 = up);
 *  z_mode 2: z = bf16(Z * z_scale)     (scale-before-matmul, methods/nf4_lora.py:87-90).
 *  lora_layout 0: lora is [r, D] (LoRA A); 1: lora is [D, r] (LoRA B).
 * Replaces the rank-r GEMMs F.linear(x, lora_a) (methods/nf4_lora.py:49) and
 * scaled_grad @ lora_b (methods/nf4_lora.py:89-90). The adapter is first
 * converted to bf16 into the caller's workspace (16-byte aligned, at least
 * molt_lora_project_workspace(M, D, r) bytes), which also holds the fp32
 * partials when the contraction is split over workgroups (small M); concurrent
 * calls need separate workspaces. */
size_t molt_lora_project_workspace(int64_t M, int64_t D, int32_t r);
int molt_lora_project(const uint16_t* z, const uint16_t* z2, int64_t ldz, int32_t z_mode,
                      float z_scale, int64_t M, int64_t D, const float* lora,
                      int32_t lora_layout, int32_t r, uint16_t* out, int64_t ldo,
                      void* workspace, size_t workspace_bytes, void* stream);

/* The projection's adapter operand prepared ahead, for callers that project
 * with the same adapter more than once or prepare several adapters at once
 * (no counterpart in the reference, which casts each adapter under autocast
 * per matmul). molt_lora_pack_many converts 1..8 fp32 adapters to the
 * projection's bf16 fragment order in one launch: rows q < split from lora,
 * the rest from lora2 (two stacked matrices of one layout without a copy;
 * lora2 NULL and split = r for one). Each packed operand takes
 * molt_lora_packed_bytes(D, r) bytes (16-byte aligned). molt_lora_project_packed
 * is molt_lora_project over such an operand: no pack launch, and a workspace
 * of molt_lora_project_packed_workspace(M, D, r) bytes (the split partials;
 * often 0). Outputs are bitwise those of molt_lora_project on the same
 * adapter. */
typedef struct molt_lora_pack_desc {
  const float* lora;
  const float* lora2;
  int32_t split;
  int32_t layout;
  int32_t r;
  int64_t D;
  uint16_t* packed;
} molt_lora_pack_desc;
size_t molt_lora_packed_bytes(int64_t D, int32_t r);
int molt_lora_pack_many(int32_t n, const molt_lora_pack_desc* d, void* stream);
size_t molt_lora_project_packed_workspace(int64_t M, int64_t D, int32_t r);
int molt_lora_project_packed(const uint16_t* z, const uint16_t* z2, int64_t ldz, int32_t z_mode,
                             float z_scale, int64_t M, int64_t D, const uint16_t* packed, int32_t r,
                             uint16_t* out, int64_t ldo, void* workspace, size_t workspace_bytes,
                             void* stream);

/* Two packed projections of one shape as one launch: out[:, :r] from (z0,
 * z_scale0, packed0) and out[:, r:2r] from (z1, z_scale1, packed1), z_mode 0
 * or 2 (ldo >= 2r). The split over the contraction counts both operands'
 * row blocks, so a pair that fills the CUs together runs unsplit; each half
 * is the projection of its own operand (fp32 sums in the order of its own
 * launch at that split count). Operands the single launch does not take
 * (unaligned rows, D not a multiple of 64) run as two projections. Workspace:
 * molt_lora_project_pair_packed_workspace(M, D, r) bytes (often 0). No
 * counterpart in the reference, which projects the gate and up gradients
 * separately (methods/nf4_lora.py:89-90 per projection); used for
 * U_g = bf16(s_g dg) bf16(B_g) and U_u of the fused gated MLP's backward. */
size_t molt_lora_project_pair_packed_workspace(int64_t M, int64_t D, int32_t r);
int molt_lora_project_pair_packed(const uint16_t* z0, const uint16_t* z1, int64_t ldz, int32_t z_mode,
                                  float z_scale0, float z_scale1, int64_t M, int64_t D,
                                  const uint16_t* packed0, const uint16_t* packed1, int32_t r,
                                  uint16_t* out, int64_t ldo, void* workspace, size_t workspace_bytes,
                                  void* stream);

/* Y[M, N] = bf16( X . deq(W)^T + T . bf16(s * B)^T ), fp32 accumulation, with
 * X bf16 [M, K], T bf16 [M, r] = molt_lora_project(X, lora_a) and B fp32 [N, r]
 * (row stride r). `w->scales` must be resolved fp32 scales. r = 0 skips LoRA.
 * Workspace (256-byte aligned, molt_nf4_lora_forward_workspace(M, N, K, r) bytes):
 * for many token rows the bf16 weight, written once by the dequant and read by
 * the GEMM (MOLT_TUNE_STAGE_MIN_MTILES), and for r % 64 == 0 the bf16(s B)
 * rows its LoRA steps then stream the same way; and, when the output has too few
 * 256 x 256 tiles to fill the GPU and K is long, the fp32 partials of a
 * contraction split over workgroups, summed in split order (deterministic).
 * The results do not depend on the workspace; a NULL or smaller workspace runs
 * without staging and without the split. Concurrent calls need separate
 * workspaces.
 * Replaces bnb.matmul_4bit + the LoRA epilogue at methods/nf4_lora.py:43-50 and
 * methods/gated_replay.py:211-224. */
size_t molt_nf4_lora_forward_workspace(int64_t M, int64_t N, int64_t K, int32_t r);
int molt_nf4_lora_forward(const uint16_t* x, int64_t ldx, int64_t M, const molt_nf4_weight* w,
                          const uint16_t* t, int64_t ldt, const float* lora_b, int32_t r,
                          float scaling, uint16_t* y, int64_t ldy, void* workspace,
                          size_t workspace_bytes, void* stream);

/* Gate and up projections of a gated MLP in one launch, sharing X:
 *   gate = bf16(X . deq(Wg)^T + T[:, :r] . bf16(sg Bg)^T)
 *   up   = bf16(X . deq(Wu)^T + T[:, r:] . bf16(su Bu)^T)
 *   h    = bf16(bf16(silu(gate)) * up)
 * with T bf16 [M, 2r] = [X . Ag^T | X . Au^T]. A workgroup owns gate and up of
 * the same intermediate columns, so h is formed in registers from the two
 * accumulators. Outputs are bf16 [M, I] with row stride ldo. Workspace: the
 * two staged bf16 weights, molt_nf4_gateup_forward_workspace(M, I, K, r) bytes
 * (see molt_nf4_lora_forward; NULL runs unstaged).
 * Replaces the gate_proj/up_proj calls and `F.silu(gate) * up` of
 * methods/gated_replay.py:78-94,290-291 (and benchmarks/qualified_path_measure.py:404-432). */
size_t molt_nf4_gateup_forward_workspace(int64_t M, int64_t N, int64_t K, int32_t r);
int molt_nf4_gateup_forward(const uint16_t* x, int64_t ldx, int64_t M, const molt_nf4_weight* wg,
                            const molt_nf4_weight* wu, const uint16_t* t, int64_t ldt,
                            const float* bg, const float* bu, int32_t r, float sg, float su,
                            uint16_t* gate, uint16_t* up, uint16_t* h, int64_t ldo, void* workspace,
                            size_t workspace_bytes, void* stream);

/* dX[M, K] = bf16( dY . deq(W) + U . bf16(lora_scale * A) ), U bf16 [M, r] (for
 * the scheduled backward U = molt_lora_project(dY, lora_b, z_mode 2, s) and
 * lora_scale = 1), A fp32 [r, K] (row stride K). r = 0 skips LoRA.
 * Workspace as in molt_nf4_lora_forward, molt_nf4_lora_backward_workspace(M, N,
 * K, 1) bytes (N = w->rows, K = w->cols): the staged weight is deq(W)^T
 * [K, N] in bf16, then the split partials.
 * Replaces the dX half of _ScheduledNF4LoRA.backward (methods/nf4_lora.py:86-101)
 * and packed_nf4_backward_input / packed_nf4_lora_backward_input
 * (methods/nf4_backward.py:167-284). */
size_t molt_nf4_lora_backward_workspace(int64_t M, int64_t N, int64_t K, int32_t segments);
int molt_nf4_lora_backward_input(const uint16_t* dy, int64_t lddy, int64_t M,
                                 const molt_nf4_weight* w, const uint16_t* u, int64_t ldu,
                                 const float* lora_a, int32_t r, float lora_scale, uint16_t* dx,
                                 int64_t lddx, void* workspace, size_t workspace_bytes, void* stream);

/* dX = dY0 . deq(W0) + dY1 . deq(W1) + U0 . bf16(A0) + U1 . bf16(A1): the input
 * gradient of the gate and up projections of a gated MLP in one contraction
 * (methods/gated_replay.py:167-186). Workspace: molt_nf4_lora_backward_workspace(M,
 * N, K, 2) bytes (see molt_nf4_lora_backward_input). */
int molt_nf4_lora_backward_input_pair(const uint16_t* dy0, const uint16_t* dy1, int64_t lddy,
                                      int64_t M, const molt_nf4_weight* w0,
                                      const molt_nf4_weight* w1, const uint16_t* u0,
                                      const uint16_t* u1, int64_t ldu, const float* a0,
                                      const float* a1, int32_t r, uint16_t* dx, int64_t lddx,
                                      void* workspace, size_t workspace_bytes, void* stream);

/* SwiGLU backward fused into the down projection's input gradient
 * (methods/gated_replay.py:376-387; kernels/gated_activation.py:44-51):
 * dh = bf16(dY . deq(Wd) + U . bf16(Ad)); dg = bf16(bf16(dh * up) * silu'(gate)),
 * du = bf16(dh * bf16(silu(gate))). gate, up, dg, du are bf16 [M, I] with row
 * stride ldg; dh is never stored. Workspace: the staged deq(Wd)^T,
 * molt_nf4_lora_backward_workspace(M, H, I, 1) bytes (NULL runs unstaged). */
int molt_nf4_swiglu_backward(const uint16_t* dy, int64_t lddy, int64_t M,
                             const molt_nf4_weight* wd, const uint16_t* u, int64_t ldu,
                             const float* lora_a, int32_t r, const uint16_t* gate,
                             const uint16_t* up, int64_t ldg, uint16_t* dgate, uint16_t* dup,
                             void* workspace, size_t workspace_bytes, void* stream);

/* Weight transposes handed from the forward to the input gradient (no
 * counterpart in the reference, whose backward re-dequantises the NF4 weight
 * for dX, methods/nf4_backward.py:167-284; methods/gated_replay.py:376-387).
 * For many token rows both GEMMs of a weight stage it in bf16, the input
 * gradient transposed. A *_keep_wt forward also writes deq(W)^T, bf16 [K, N]
 * with row stride N (16-byte aligned, N * K elements per weight), from the W
 * tiles its own staged GEMM already holds: a tile of each contraction step is
 * written by one row block, so the copy costs the GEMM little. It sets
 * *wt_written to 1 when it did (its plan staged the weights, N % 8 == 0), else
 * 0, and its outputs are those of the plain entry point. A *_wt input gradient
 * given that copy (the same weight; NULL = none) reads it instead of
 * dequantising and transposing the weight itself, with a workspace of
 * molt_nf4_lora_backward_workspace_wt(M, N, K, segments) bytes; its results
 * are bitwise those of the plain entry point. molt_nf4_keeps_wt(M, N, K,
 * weights) is 1 when a forward and input gradient over M rows both stage
 * (for 16-byte aligned operands): then keeping the copy (N * K * 2 bytes per
 * weight, held from the forward to the backward) replaces the backward's
 * staging pass. */
int32_t molt_nf4_keeps_wt(int64_t M, int64_t N, int64_t K, int32_t weights);
int molt_nf4_lora_forward_keep_wt(const uint16_t* x, int64_t ldx, int64_t M, const molt_nf4_weight* w,
                                  const uint16_t* t, int64_t ldt, const float* lora_b, int32_t r,
                                  float scaling, uint16_t* y, int64_t ldy, uint16_t* wt,
                                  int32_t* wt_written, void* workspace, size_t workspace_bytes,
                                  void* stream);
int molt_nf4_gateup_forward_keep_wt(const uint16_t* x, int64_t ldx, int64_t M, const molt_nf4_weight* wg,
                                    const molt_nf4_weight* wu, const uint16_t* t, int64_t ldt,
                                    const float* bg, const float* bu, int32_t r, float sg, float su,
                                    uint16_t* gate, uint16_t* up, uint16_t* h, int64_t ldo,
                                    uint16_t* wgt, uint16_t* wut, int32_t* wt_written, void* workspace,
                                    size_t workspace_bytes, void* stream);
size_t molt_nf4_lora_backward_workspace_wt(int64_t M, int64_t N, int64_t K, int32_t segments);
int molt_nf4_lora_backward_input_wt(const uint16_t* dy, int64_t lddy, int64_t M,
                                    const molt_nf4_weight* w, const uint16_t* wt, const uint16_t* u,
                                    int64_t ldu, const float* lora_a, int32_t r, float lora_scale,
                                    uint16_t* dx, int64_t lddx, void* workspace, size_t workspace_bytes,
                                    void* stream);
int molt_nf4_lora_backward_input_pair_wt(const uint16_t* dy0, const uint16_t* dy1, int64_t lddy,
                                         int64_t M, const molt_nf4_weight* w0,
                                         const molt_nf4_weight* w1, const uint16_t* wt0,
                                         const uint16_t* wt1, const uint16_t* u0, const uint16_t* u1,
                                         int64_t ldu, const float* a0, const float* a1, int32_t r,
                                         uint16_t* dx, int64_t lddx, void* workspace,
                                         size_t workspace_bytes, void* stream);
int molt_nf4_swiglu_backward_wt(const uint16_t* dy, int64_t lddy, int64_t M,
                                const molt_nf4_weight* wd, const uint16_t* wdt, const uint16_t* u,
                                int64_t ldu, const float* lora_a, int32_t r, const uint16_t* gate,
                                const uint16_t* up, int64_t ldg, uint16_t* dgate, uint16_t* dup,
                                void* workspace, size_t workspace_bytes, void* stream);

/* Several NF4-LoRA projections that share one input as one node: their
 * weights stacked along the output rows, W = [W_0; W_1; ..] (1..8 weights of
 * the same columns, block size, nibble order and code table; N = sum of their
 * rows), e.g. a decoder layer's q, k and v projections. No counterpart in the
 * reference, which runs each projection as its own node
 * (methods/nf4_lora.py:12-113 per projection); each output column is the
 * product that projection's own node computes (its LoRA term through its own
 * adapter), with fp32 sums in another order.
 *  molt_lora_stack_adapters: A_stack fp32 [lr, K] = [A_0; A_1; ..; zero rows]
 *   and B_blocks fp32 [N, lr], block-diagonal (B_i [rows_i, r] in columns
 *   i r .. i r + r - 1 of its rows, zeros elsewhere); r and lr multiples of
 *   4, n r <= lr; one launch.
 *  molt_nf4_stacked_forward: Y[M, N] = bf16(X deq(W)^T + T bf16(s B_blocks)^T)
 *   with T = molt_lora_project(X, A_stack) [M, lr], lr 0 or a multiple of 64;
 *   it dequantises each weight into its rows of the staged copy and runs one
 *   GEMM. Workspace: molt_nf4_lora_forward_workspace(M, N, K, lr). With wt
 *   (bf16 [K, N], 16-byte aligned) it also writes deq(W)^T for the input
 *   gradient (*wt_written = 1). Only the staged plan applies
 *   (molt_nf4_keeps_wt(M, N, K, 1) = 1 for 16-byte aligned operands); other
 *   shapes are refused with MOLT_EUNSUPPORTED before any launch.
 *  molt_nf4_stacked_backward_input: dX = dY deq(W) + U bf16(lora_scale A_stack)
 *   from that deq(W)^T (required), dY bf16 [M, N]; workspace
 *   molt_nf4_lora_backward_workspace_wt(M, N, K, 1); refused like the forward
 *   where the plan would not read wt. */
int molt_lora_stack_adapters(int32_t n, const float* const* a, const float* const* b, const int64_t* rows,
                             int32_t r, int64_t K, int32_t lr, float* a_stack, float* b_blocks, void* stream);
int molt_nf4_stacked_forward(const uint16_t* x, int64_t ldx, int64_t M, int32_t nw, const molt_nf4_weight* w,
                             const uint16_t* t, int64_t ldt, int32_t lr, const float* b_blocks, int64_t ldb,
                             float scaling, uint16_t* y, int64_t ldy, uint16_t* wt, int32_t* wt_written,
                             void* workspace, size_t workspace_bytes, void* stream);
int molt_nf4_stacked_backward_input(const uint16_t* dy, int64_t lddy, int64_t M, int32_t nw,
                                    const molt_nf4_weight* w, const uint16_t* wt, const uint16_t* u, int64_t ldu,
                                    const float* a_stack, int32_t r, float lora_scale, uint16_t* dx, int64_t lddx,
                                    void* workspace, size_t workspace_bytes, void* stream);

/* LoRA weight gradient out = scale * L^T . R over M rows, fp32:
 *  L bf16 [M, P] (l_mode 0) or SwiGLU replay of (L, L2) (l_mode 1); R bf16 [M, Q].
 *  out_layout 0: out[P, Q] (dB = s dY^T T, methods/nf4_lora.py:102);
 *  out_layout 1: out[Q, P] (dA = U^T X, methods/nf4_lora.py:103).
 * Deterministic: a fixed split of M, partials summed in split order. */
size_t molt_lora_grad_workspace(int64_t M, int64_t P, int64_t Q);
int molt_lora_grad(const uint16_t* l, const uint16_t* l2, int64_t ldl, int32_t l_mode,
                   const uint16_t* rmat, int64_t ldr, int64_t M, int64_t P, int64_t Q,
                   float scale, float* out, int32_t out_layout, void* workspace,
                   size_t workspace_bytes, void* stream);

/* Several LoRA weight gradients with one launch that sums all their splits (a
 * molt_lora_grad call takes two launches per gradient). Each descriptor holds
 * the arguments of one molt_lora_grad call (l_mode 0 or 1), or of one
 * molt_lora_grad_rmsnorm call (l_mode 2: l = x, inv_rms, norm_weight of
 * w_dtype and norm_offset; l2 unused), and its output is bitwise what that
 * call gives: same tiles, M slices, partials and summation order. The
 * gradients with plain operands (l_mode 0), 16-byte aligned rows and P and Q
 * multiples of 8 share one launch; each other gradient takes a launch of its
 * own; then one launch sums every split. 1..8 descriptors. Workspace
 * (256-byte aligned): molt_lora_grad_many_workspace(n, d) bytes. No
 * counterpart in the reference, which computes each adapter gradient as its
 * own matmul (methods/nf4_lora.py:102-103, methods/gated_replay.py:392-405);
 * the gated-MLP backward runs all its adapter gradients, and a scheduled
 * projection its two, as one call. */
typedef struct molt_lora_grad_desc {
  const uint16_t* l;
  const uint16_t* l2;
  int64_t ldl;
  int32_t l_mode;
  const uint16_t* rmat;
  int64_t ldr;
  int64_t M, P, Q;
  float scale;
  float* out;
  int32_t out_layout;
  /* l_mode 2 only */
  const float* inv_rms;
  const void* norm_weight;
  int32_t w_dtype;
  float norm_offset;
} molt_lora_grad_desc;
size_t molt_lora_grad_many_workspace(int32_t n, const molt_lora_grad_desc* d);
int molt_lora_grad_many(int32_t n, const molt_lora_grad_desc* d, void* workspace, size_t workspace_bytes,
                        void* stream);

/* molt_lora_grad with the frozen RMSNorm's output as L, formed as it is
 * staged: L(m, p) = bf16(fp32(x(m, p)) * inv_rms[m] * (fp32(w[p]) + offset)),
 * the products and roundings of molt_rmsnorm_forward, so the result is
 * bitwise that of molt_lora_grad over the materialised norm output when
 * inv_rms comes from molt_rmsnorm_forward on the same x and weight. x bf16
 * [M, P] (row stride ldx), inv_rms fp32 [M], w bf16 or fp32 [P] (w_dtype).
 * Same workspace as molt_lora_grad (molt_lora_grad_workspace(M, P, Q)).
 * Requires 16-byte aligned rows of x and rmat and P, Q multiples of 8, else
 * MOLT_EUNSUPPORTED. Replaces the replay of the normalised input for the
 * gate/up adapters' dA in _ResidualRecipeGatedNF4LoRA.backward
 * (methods/gated_replay.py:146-151,167-184), which the reference
 * materialises (_RMSNormReplayRecipe.materialize, :22-30). */
int molt_lora_grad_rmsnorm(const uint16_t* x, int64_t ldx, const float* inv_rms,
                           const void* norm_weight, int32_t w_dtype, float offset,
                           const uint16_t* rmat, int64_t ldr, int64_t M, int64_t P, int64_t Q,
                           float scale, float* out, int32_t out_layout, void* workspace,
                           size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Skinny-M NF4 GEMV (M <= 16)                                               */
/* ------------------------------------------------------------------------ */

/* Y[M, N] = bf16( X . (code[W] * scale)^T + T . bf16(s * B)^T ) for M <= 16,
 * reading the nested statistics (or fp32 scales) directly; the block scale is
 * applied once per 64-element block sum, so each weight enters as its NF4 code
 * rounded to bf16 times the fp32 scale. T bf16 [M, r] from molt_lora_project,
 * B fp32 [N, r] (row stride r); r = 0 skips LoRA. Requires cols % 64 == 0,
 * block_size == 64 and a power-of-two dq_block. molt_nf4_gemv_workspace()
 * returns the workspace size: fp32 partials (slices x M x N) when the kernel
 * for 2 <= M <= 16 splits K over workgroups (K = 14336: four slices), else 0.
 * Concurrent calls need separate workspaces.
 * Replaces the bnb.matmul_4bit decode path (training/qlora.py:1332-1358). */
size_t molt_nf4_gemv_workspace(int64_t M, int64_t N, int64_t K);
int molt_nf4_gemv(const uint16_t* x, int64_t ldx, int64_t M, const molt_nf4_weight* w,
                  const uint16_t* t, int64_t ldt, const float* lora_b, int32_t r,
                  float scaling, uint16_t* y, int64_t ldy, void* workspace,
                  size_t workspace_bytes, void* stream);

/* molt_nf4_gemv without a workspace argument and without any allocation. No
 * counterpart in the reference: it is for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). The split-K partials live in a static device array of
 * molt_nf4_gemv_noalloc_limit() bytes (8 MiB) per GPU, held until the process
 * ends; a shape needing more (molt_nf4_gemv_workspace above the limit) returns
 * MOLT_EUNSUPPORTED before any launch. Every call on one GPU shares that GPU's
 * array. Calls from different streams or host threads are ordered: each waits
 * on an event the previous call recorded on its own stream. Calls made during a
 * graph capture are not ordered that way (no wait, no record); replays of such a
 * graph that overlap other calls on the same GPU race. Same results as
 * molt_nf4_gemv, bit for bit. */
size_t molt_nf4_gemv_noalloc_limit(void);
int molt_nf4_gemv_noalloc(const uint16_t* x, int64_t ldx, int64_t M, const molt_nf4_weight* w,
                          const uint16_t* t, int64_t ldt, const float* lora_b, int32_t r,
                          float scaling, uint16_t* y, int64_t ldy, void* stream);

/* ------------------------------------------------------------------------ */
/* SwiGLU elementwise                                                        */
/* ------------------------------------------------------------------------ */

/* h = g * sigmoid(g) * u in fp32, stored in the input dtype
 * (kernels/gated_activation.py:29-36). With round_silu = 1 (bf16 only) silu(g)
 * is rounded to bf16 before the product, as `F.silu(gate) * up` under bf16
 * autocast does (methods/gated_replay.py:291). dtype: MOLT_DTYPE_BF16 or _F32. */
int molt_silu_mul_forward(const void* gate, const void* up, void* out, int64_t n,
                          int32_t dtype, int32_t round_silu, void* stream);

/* dg = dh*u*sig*(1 + g*(1 - sig)), du = dh*g*sig in fp32
 * (kernels/gated_activation.py:38-51). */
int molt_silu_mul_backward(const void* grad, const void* gate, const void* up, void* dgate,
                           void* dup, int64_t n, int32_t dtype, void* stream);

/* ------------------------------------------------------------------------ */
/* Frozen RMSNorm (forward, norm replay, backward)                           */
/* ------------------------------------------------------------------------ */

/* Row-wise over H: inv = rsqrt(sum(fp32(x)^2) * (1/H) + eps),
 * out = bf16(fp32(fp32(x) * inv) * (fp32(w) + offset)). x is bf16 or fp32
 * (x_dtype) with row stride ldx, weight bf16 or fp32 [H], out bf16 with row
 * stride ldo. inv_rms (fp32 [M], may be NULL) receives inv of every row.
 * out may be NULL when inv_rms is not: then only inv is computed, bitwise as
 * by a call whose out rows are 16-byte aligned (the norm-replay gradient,
 * molt_lora_grad_rmsnorm, uses it).
 * Replaces _FrozenRMSNormFunction.forward (kernels/frozen_rmsnorm.py:10-23) and
 * _RMSNormReplayRecipe.materialize (methods/gated_replay.py:22-30). */
int molt_rmsnorm_forward(const void* x, int32_t x_dtype, int64_t ldx, int64_t M, int64_t H,
                         const void* weight, int32_t w_dtype, float eps, float offset,
                         uint16_t* out, int64_t ldo, float* inv_rms, void* stream);

/* Frozen-weight backward: n = fp32(x) * inv, g = fp32(dy) * (fp32(w) + offset),
 * dx = inv * (g - n * sum(g * n) * (1/H)), stored in x's dtype with row stride
 * lddx; inv is recomputed from x. dy is bf16.
 * Replaces _FrozenRMSNormFunction.backward (kernels/frozen_rmsnorm.py:25-37). */
int molt_rmsnorm_backward(const uint16_t* dy, int64_t lddy, const void* x, int32_t x_dtype,
                          int64_t ldx, int64_t M, int64_t H, const void* weight,
                          int32_t w_dtype, float eps, float offset, void* dx, int64_t lddx,
                          void* stream);

/* ------------------------------------------------------------------------ */
/* Frozen-head cross-entropy                                                 */
/* ------------------------------------------------------------------------ */

/* Row-wise cross-entropy of a chunk of logits (bf16 or fp32 [rows, vocab],
 * row stride ld) against int64 targets, reduced in fp32 with an online
 * log-sum-exp: loss[i] = (lse_i - l[i, y_i]) / total for 0 <= y_i < vocab, else
 * 0. With grad non-NULL also grad[i, j] = (softmax_ij - [j == y_i]) / total in
 * the logits' dtype (row stride ldg); grad may alias the logits (in place).
 * Replaces the fused Triton reductions of the frozen LM head
 * (kernels/frozen_linear_cross_entropy.py:26-139, kernels/split_frozen_loss.py:56-89). */
int molt_cross_entropy_rows(const void* logits, int32_t dtype, int64_t ld, int64_t rows, int64_t vocab,
                            const int64_t* targets, float total, float* loss, void* grad, int64_t ldg,
                            void* stream);

/* The same rows under F.cross_entropy's rule for the exact chunked loss
 * (kernels/partitioned_loss.py:18-103, which sums F.cross_entropy over chunks
 * and divides by the token count): a row whose target lies outside [0, vocab)
 * (the ignored index -100; the caller rejects any other) gets a zero loss and a
 * zero gradient, and the gradient is multiplied by *grad_scale (device fp32
 * scalar, the upstream gradient; NULL for 1), so no host read of it is needed:
 * grad[i, j] = (softmax_ij - [j == y_i]) / total * (*grad_scale). */
int molt_cross_entropy_rows_exact(const void* logits, int32_t dtype, int64_t ld, int64_t rows, int64_t vocab,
                                  const int64_t* targets, float total, const float* grad_scale, float* loss,
                                  void* grad, int64_t ldg, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOLT_AMD_H */
