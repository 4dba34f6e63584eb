/*
 * hk.h — C ABI of libhk.so, the MI355X (gfx950) BF16 transformer kernel path.
 *
 * Every entry point here replaces one host entry point of the reference
 * (shuqi2077/rust-ascend). Citations are path:line relative to the reference
 * repository root. The ABI uses plain pointers, sizes and a contiguous tensor
 * descriptor; it exposes no C++ or torch types, so a Rust `extern "C"` shim, a
 * ctypes binding or a C program can call it directly.
 *
 * Conventions shared by every op (mirroring rust-ascend-driver/src/tensor/runtime/mod.rs:147-435):
 *   - Tensors are contiguous, row-major, device-resident. The caller owns all
 *     memory; no entry point frees caller memory. Outputs are written into
 *     caller storage ("_into" style; the reference's allocating forms map to
 *     hk_alloc + the op).
 *   - Every shape/dtype/domain check runs before any device work; a failed check
 *     returns HK_INVALID_ARGUMENT and touches nothing.
 *   - Outputs must not overlap any input or each other ([ptr, ptr+bytes) ranges),
 *     as rust-ascend-driver/src/tensor/deepgemm/mod.rs:99-100,117-119 require.
 *   - By default each call synchronizes its stream before returning, as every
 *     reference launch does (deepgemm/mod.rs:134-145). hk_set_async(ctx,1)
 *     leaves work queued on the context's stream until hk_sync().
 *   - A failed launch or synchronization poisons the context: later calls return
 *     HK_POISONED (deepgemm/mod.rs:39,143; common_ir/mod.rs:75,120).
 *   - There is no CPU fallback (deepgemm/mod.rs:1-3, README.md:44).
 *   - The message of the last failure on the calling thread is hk_last_error().
 */
#ifndef HK_H
#define HK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes; reference: CannError, rust-ascend-driver/src/lib.rs:18-78. */
typedef enum hk_status {
    HK_OK = 0,
    HK_INVALID_ARGUMENT = 1,   /* CannError::InvalidTensor */
    HK_HIP_ERROR = 2,          /* CannError::Status (runtime call failed) */
    HK_COMPLETION_ERROR = 3,   /* CannError::Completion (launch or sync failed) */
    HK_POISONED = 4,           /* provider poisoned by an earlier completion failure */
    HK_NOT_INITIALIZED = 5,    /* "runtime is not initialized" (runtime/matrix.rs:41) */
    HK_LOAD_ERROR = 6,         /* CannError::Library / Symbol (no gfx950 device, no code object) */
} hk_status;

/* Element types; the codes are the reference's DType codes,
 * rust-ascend-driver/src/tensor/layout.rs:5-17. */
typedef enum hk_dtype {
    HK_F32 = 0,
    HK_F16 = 1,
    HK_I32 = 3,   /* embedding IDs only */
    HK_I64 = 9,   /* embedding IDs only */
    HK_BOOL = 12, /* one byte, nonzero = true: module attention masks only */
    HK_BF16 = 27,
} hk_dtype;

/* Reference: deepgemm::Transpose, rust-ascend-driver/src/tensor/deepgemm/plan.rs:7. */
typedef enum hk_transpose { HK_NO = 0, HK_YES = 1 } hk_transpose;

/* Reference: RotaryLayout, rust-ascend-compiler/src/ascend/rotary_programs.rs:5-6. */
typedef enum hk_rotary_layout { HK_ROTARY_INTERLEAVED = 0, HK_ROTARY_SPLIT_HALF = 1 } hk_rotary_layout;

#define HK_MAX_RANK 8

/* Contiguous tensor; reference: TensorBuffer {handle, shape, strides, dtype}
 * restricted to contiguous strides (runtime/mod.rs:907-925). */
typedef struct hk_tensor {
    void* data;
    int32_t dtype;            /* hk_dtype */
    int32_t rank;             /* 0..HK_MAX_RANK */
    int64_t shape[HK_MAX_RANK];
} hk_tensor;

/* Launch and module counters; reference: KernelStats{modules_loaded, launches,
 * synchronizations}, deepgemm/mod.rs:15-16,142 and common_ir/mod.rs:11-12,119. */
typedef struct hk_stats {
    uint64_t modules_loaded;
    uint64_t launches;
    uint64_t synchronizations;
} hk_stats;

/* Host-only result of a GEMM contract check; reference: GemmSpec,
 * deepgemm/plan.rs:31-86. kind: 0 dense, 1 batched, 2 M-grouped. */
typedef struct hk_gemm_plan {
    int32_t kind;
    int32_t out_rank;
    int64_t batch, m, n, k;
    int64_t out_shape[3];
    char key[32];             /* "bf16_<kind>_<ta><tb>_<out>", plan.rs:84-86 */
} hk_gemm_plan;

typedef struct hk_context hk_context;

/* ---------------------------------------------------------------- runtime */

/* Reference: AscendRuntime::initialize_exclusive, runtime/mod.rs:424-435 and
 * Worker::start (runtime/worker.rs:34-90). Binds `device`, checks that it is a
 * gfx950 part, and creates the context. Only one context per process; a second
 * call returns HK_INVALID_ARGUMENT ("already initialized", mod.rs:427-433). */
hk_status hk_init(int32_t device, hk_context** out);
/* Releases the context (the reference keeps its worker for the process lifetime;
 * this exists for tests). */
hk_status hk_shutdown(hk_context* ctx);
/* Use `stream` (a hipStream_t; NULL = the null stream) for later launches. */
hk_status hk_set_stream(hk_context* ctx, void* stream);
void* hk_get_stream(hk_context* ctx);
/* 0 (default): synchronize after every op, like the reference. 1: leave queued. */
hk_status hk_set_async(hk_context* ctx, int32_t async_mode);
/* Reference: CannSession::synchronize / ComputeClient::flush. */
hk_status hk_sync(hk_context* ctx);
hk_status hk_get_stats(hk_context* ctx, hk_stats* out);
/* The context's workspace: device scratch that ops allocate on first need, grow when a
 * larger call needs more, and keep for later calls (the stored-dS attention backward holds
 * B*Hq*ceil(N/32)*ceil(M/64)*4 KiB, 4 GiB at B4 S4096 Hq32, within HK_ATTN_DS_BUDGET;
 * a backward whose dS buffer cannot be allocated falls back to the recompute form). No
 * reference counterpart: the reference allocates per call (runtime/matrix.rs:33-44).
 * hk_workspace_size reports its size in bytes; hk_trim_workspace frees it, after the queued
 * work, when it holds more than keep_bytes (0: always). */
hk_status hk_workspace_size(hk_context* ctx, uint64_t* bytes);
hk_status hk_trim_workspace(hk_context* ctx, uint64_t keep_bytes);
/* Thread-local message of the last failure; reference: Display for CannError. */
const char* hk_last_error(void);
/* Number of the library's ABI (bumped on incompatible change). */
int32_t hk_abi_version(void);

/* Device memory; reference: ComputeStorage alloc/dealloc with 32-B alignment
 * (runtime/mod.rs:486-517), create_from_slice / read_one. */
hk_status hk_alloc(hk_context* ctx, size_t bytes, void** out);
hk_status hk_free(hk_context* ctx, void* ptr);
hk_status hk_upload(hk_context* ctx, void* dst, const void* src, size_t bytes);
hk_status hk_download(hk_context* ctx, void* dst, const void* src, size_t bytes);

/* ---------------------------------------------------------------- GEMM */

/* Host-only contract check, no device access. Reference: GemmSpec::new,
 * deepgemm/plan.rs:49-80: BF16 A/B, BF16 or F32 output, rank 2 or equal-batch
 * rank 3 (batch 1..4096, no broadcast), M/N/K positive multiples of 16 and at
 * most INT32_MAX. */
hk_status hk_gemm_plan_check(const hk_tensor* a, const hk_tensor* b, int32_t ta, int32_t tb,
                             int32_t out_dtype, hk_gemm_plan* plan);

/* out = op(A) @ op(B), FP32 accumulation, BF16 (RNE) or F32 out.
 * Reference: AscendRuntime::gemm_into, runtime/mod.rs:350-354 (matrix.rs:54-59);
 * AscendRuntime::gemm (mod.rs:344-348) is hk_alloc + this call. */
hk_status hk_gemm_into(hk_context* ctx, const hk_tensor* a, const hk_tensor* b,
                       int32_t ta, int32_t tb, hk_tensor* out);

/* Linear backward for Y = X W^T: dX = dY W (BF16), dW = dY^T X (F32).
 * Reference: AscendRuntime::linear_nt_backward, runtime/mod.rs:357-362 (matrix.rs:60-74). */
hk_status hk_linear_nt_backward(hk_context* ctx, const hk_tensor* x, const hk_tensor* w,
                                const hk_tensor* dy, hk_tensor* dx, hk_tensor* dw);

/* M-grouped (mixture-of-experts) NT GEMM: out[i,:] = A[i,:] W[g]^T for the rows i of group g,
 * A [M,K] BF16, W [G,N,K] BF16, out [M,N] BF16 or F32. Groups are "aligned physical" row
 * ranges: ends[g] is the row after group g, nondecreasing multiples of 256, ends[G-1] = M;
 * a repeated end is an empty expert (no rows).
 *
 * Host-only check of the ends. Reference: GroupEnds::new, deepgemm/plan.rs:16-26 (1..=4096
 * groups, nondecreasing multiples of 256, not all empty). */
hk_status hk_group_ends_check(const int32_t* ends, int32_t count);
/* Opaque, immutable device copy of checked group ends, uploaded once and reused by every
 * grouped call. Reference: DeepGemm::upload_group_ends / DeviceGroupEnds, deepgemm/mod.rs:61-67. */
typedef struct hk_group_ends hk_group_ends;
hk_status hk_group_ends_upload(hk_context* ctx, const int32_t* ends, int32_t count, hk_group_ends** out);
/* Frees the device copy after the context's queued work has completed. */
hk_status hk_group_ends_free(hk_context* ctx, hk_group_ends* ends);
/* Host-only contract check (plan->kind 2, key "bf16_mgrouped_nt_<out>"). Reference:
 * GemmSpec::grouped_nt, deepgemm/plan.rs:61-67, then GemmSpec::checked (:68-80). */
hk_status hk_gemm_grouped_plan_check(const hk_tensor* a, const hk_tensor* weights, const int32_t* ends,
                                     int32_t count, int32_t out_dtype, hk_gemm_plan* plan);
/* Reference: DeepGemm::grouped_nt_into, deepgemm/mod.rs:74-78 (grouped_nt, :68-73, is
 * hk_alloc + this call). */
hk_status hk_gemm_grouped_nt_into(hk_context* ctx, const hk_tensor* a, const hk_tensor* weights,
                                  const hk_group_ends* ends, hk_tensor* out);

/* Generic floating matmul with the inputs' dtype out (aclnnMatmul KEEP_DTYPE): F32, F16 or BF16
 * A [..., M, K] and B [..., K, N], rank 2..6 each, batch dims broadcast numpy-style, any M/N/K
 * (K = 0 gives zeros), FP32 products and sums, the output rounded to the dtype (RNE).
 * Host-only output layout. Reference: generic_matrix::output_layout (runtime/generic_matrix.rs:4-15,
 * tensor/layout.rs:106-142). */
hk_status hk_matmul_layout(const hk_tensor* a, const hk_tensor* b, hk_tensor* out);
/* out = A @ B into a caller-allocated contiguous output of that layout. Reference:
 * AscendRuntime::tensor_matmul (runtime/mod.rs:156-158; generic_matrix.rs:17-54, worker.rs:128-162),
 * the op behind RudaAscend::float_matmul (src/backend.rs:692-703). */
hk_status hk_tensor_matmul(hk_context* ctx, const hk_tensor* a, const hk_tensor* b, hk_tensor* out);
/* Gradients of hk_tensor_matmul: dA = dY B^T and dB = A^T dY, each summed (FP32, in batch order)
 * over the batch dims its operand broadcasts along, in A's and B's dtype and shape. The rule is the
 * autodiff of float_matmul (src/backend.rs:692-703) in the reference's tensor library. */
hk_status hk_tensor_matmul_backward(hk_context* ctx, const hk_tensor* a, const hk_tensor* b, const hk_tensor* dy,
                                    hk_tensor* da, hk_tensor* db);

/* ------------------------------------------------ module attention (the backend's fallback) */

/* RudaAscend's ModuleOps::attention (src/backend.rs:1323-1333) composes the backend's own ops
 * (ruda_tensor's attention_fallback): scores = Q (K^T) * scale, softcap, + bias, -inf where masked,
 * softmax over the keys, then P V. With hk_tensor_matmul and hk_softmax these are the remaining
 * pieces; rust_ascend_hip.nn.module_attention is the composition.
 *
 * y = x with its last two dims swapped, materialized (float_swap_dims + contiguous,
 * src/backend.rs:133-140,641): F32, F16 or BF16, rank >= 2. */
hk_status hk_swap_last_dims(hk_context* ctx, const hk_tensor* x, hk_tensor* y);
/* out = masked ? -inf : softcap(s * scale) + bias over F32 scores s [B, H, Sq, Sk]; softcap(x) =
 * c tanh(x / c) when softcap = c > 0 (0: none); bias (nullable) F32 and mask (nullable, HK_BOOL,
 * nonzero = masked) rank 4 with each dim equal to the scores' or 1 (broadcast); causal masks the keys
 * k > q (the top-left-aligned rule of a lower-triangular mask). */
hk_status hk_attention_scores(hk_context* ctx, const hk_tensor* s, float scale, float softcap, const hk_tensor* bias,
                              const hk_tensor* mask, int32_t causal, hk_tensor* out);
/* ds = d out / d s (zero where masked) and, when dbias is given (shaped like the bias), the bias
 * gradient summed over its broadcast dims in a fixed order. */
hk_status hk_attention_scores_backward(hk_context* ctx, const hk_tensor* s, const hk_tensor* dout, float scale,
                                       float softcap, const hk_tensor* mask, int32_t causal, hk_tensor* ds,
                                       hk_tensor* dbias);

/* ------------------------------------------------ GEMM device programs (code object) */

/* The reference's launch ABI for its 18 BF16 GEMM device programs
 * (rust-ascend-kernels/src/ascend.rs:88-114, deepgemm/native.rs:80-93):
 *   ruda_rust_bf16_{dense,batched}_{n,t}{n,t}_{bf16,f32}, ruda_rust_bf16_mgrouped_nt_{bf16,f32}
 *   (hk_gm a, hk_gm b, hk_gm d, uint32_t m, uint32_t n, uint32_t k, int32_t* grouped_layout,
 *    uint32_t num_groups, hk_epilogue epilogue)
 * D = op(A) op(B), FP32 accumulation, BF16 (RNE) or F32 out; "t" in the name means A stored
 * [K,M] (first letter) or B stored [N,K] (second letter). The programs ship ahead of time as one
 * gfx950 code object, rust-ascend_amd/lib/hk_programs.hsaco (the reference's per-key checked
 * artifacts, deepgemm/artifact.rs:6-27). The argument structs are the reference's, field for
 * field (GmPtr / Epilogue, native.rs:80-86; sizes 24 and 32 bytes, native.rs:96). */
typedef struct hk_gm {
    uint64_t addr;          /* device address of the operand */
    uint64_t stride_outer;  /* elements per row: the operand's last physical dimension */
    uint64_t stride_batch;  /* elements per batch: m*k, n*k, m*n for batched programs, else 0 */
} hk_gm;
typedef struct hk_epilogue {
    float alpha;  /* 1 */
    uint32_t pad0;
    uint64_t sfd;
    uint64_t stride;
    uint32_t n;   /* N */
    uint32_t pad1;
} hk_epilogue;
typedef struct hk_module hk_module;
typedef struct hk_function hk_function;

/* Loads a code object image (an unbundled little-endian ELF64 gfx950 object of at most 128 MiB;
 * the bytes are copied). Reference: Kernel::load's aclrtBinaryLoadFromData (native.rs:46-52),
 * after artifact::read's size and ELF checks (artifact.rs:18-22). Counts in modules_loaded. */
hk_status hk_module_load_data(hk_context* ctx, const void* image, size_t bytes, hk_module** out);
/* Entry point `name` of a loaded module (one of the 18 names above; a repeated lookup returns the
 * same handle, valid until the module is unloaded). Reference: aclrtBinaryGetFunction,
 * native.rs:53-63. */
hk_status hk_module_get_function(hk_context* ctx, hk_module* module, const char* name, hk_function** out);
/* Launches a device program on the context's stream with `args`, the nine argument pointers in
 * parameter order (&a, &b, &d, &m, &n, &k, &grouped_layout, &num_groups, &epilogue), then
 * synchronizes unless async mode is on. block_dim is the reference's core count (it passes 32);
 * any positive value is accepted, the grid being one 256-thread workgroup per 256x256 output
 * tile. Before the launch every argument is checked against the reference's contract
 * (GemmSpec::checked, plan.rs:68-80; the packing of execute_addresses, mod.rs:122-132): M/N/K
 * positive multiples of 16; packed row-major strides; num_groups 0 (dense), 1..=4096 (batched)
 * or the group count with grouped_layout from hk_group_ends_data and M its last end
 * (M-grouped); epilogue {1, 0, 0, 0, N, 0}; 16-byte aligned operands, each inside one device
 * allocation; the output overlapping no input. The 256x256 kernel's 32-bit offsets add one
 * limit: M*K and N*K (K rounded up to 64) below 2^30 elements. Reference:
 * aclrtLaunchKernelWithArgsArray (native.rs:11), as DeepGemm::execute_addresses calls it
 * (mod.rs:122-145). */
hk_status hk_launch_kernel_with_args(hk_context* ctx, const hk_function* fn, uint32_t block_dim, void** args);
/* Unloads a module after the context's queued work completes; its function handles end with it.
 * A poisoned context keeps the code loaded (HK_POISONED). Reference: Drop for Kernel,
 * native.rs:66-76. */
hk_status hk_module_unload(hk_context* ctx, hk_module* module);
/* The device copy of uploaded group ends: the grouped_layout argument of the M-grouped
 * programs. Reference: DeviceGroupEnds' device tensor (deepgemm/mod.rs:63-67,101). */
hk_status hk_group_ends_data(hk_context* ctx, const hk_group_ends* ends, const int32_t** out);

/* FP32-storage, BF16-compute GEMM: rounds A and B to BF16 into a_bf16/b_bf16
 * (the saved snapshots), then out(F32) = op(A) @ op(B).
 * Reference: AscendRuntime::gemm_bf16_fp32, runtime/mod.rs:388-392 (matrix.rs:84-93). */
hk_status hk_gemm_bf16_fp32(hk_context* ctx, const hk_tensor* a, const hk_tensor* b,
                            int32_t ta, int32_t tb, hk_tensor* out,
                            hk_tensor* a_bf16, hk_tensor* b_bf16);
/* FP32 gradients in the original physical layouts from saved BF16 A/B and F32 dY
 * (rounded to BF16 on device). Reference: AscendRuntime::gemm_bf16_fp32_backward,
 * runtime/mod.rs:395-399 (matrix.rs:95-121). */
hk_status hk_gemm_bf16_fp32_backward(hk_context* ctx, const hk_tensor* a_bf16,
                                     const hk_tensor* b_bf16, const hk_tensor* dy,
                                     int32_t ta, int32_t tb, hk_tensor* da, hk_tensor* db);
/* Y(F32) = bf16(X) bf16(W)^T with rank-2 F32 X/W. Reference:
 * AscendRuntime::linear_bf16_fp32, runtime/mod.rs:364-370 (matrix.rs:129-133). */
hk_status hk_linear_bf16_fp32(hk_context* ctx, const hk_tensor* x, const hk_tensor* w,
                              hk_tensor* y, hk_tensor* x_bf16, hk_tensor* w_bf16);
/* Reference: AscendRuntime::linear_bf16_fp32_backward, runtime/mod.rs:372-377. */
hk_status hk_linear_bf16_fp32_backward(hk_context* ctx, const hk_tensor* x_bf16,
                                       const hk_tensor* w_bf16, const hk_tensor* dy,
                                       hk_tensor* dx, hk_tensor* dw);

/* Padded BF16-compute GEMM for any positive M/N/K (no multiple-of-16 rule): the matrix axes of
 * F32 A and B are rounded to BF16 and zero-padded up to multiples of 16 into a_pad/b_pad (the
 * saved snapshots, "native" shapes), the native GEMM runs with F32 output, and the result is
 * cropped to out's logical shape ([M,N] or [batch,M,N]). Rank 2 or equal-batch rank 3, all four
 * transposes. Reference: AscendRuntime::gemm_padded_bf16_fp32, runtime/mod.rs:186-190
 * (padded_matrix.rs:39-46, PaddedGemmSpec::new in deepgemm/padded.rs:13-36). */
hk_status hk_gemm_padded_bf16_fp32(hk_context* ctx, const hk_tensor* a, const hk_tensor* b,
                                   int32_t ta, int32_t tb, hk_tensor* out,
                                   hk_tensor* a_pad, hk_tensor* b_pad);
/* F32 gradients cropped to the original physical input shapes, which da/db carry, from the
 * saved padded snapshots and the logical F32 dY. Reference:
 * AscendRuntime::gemm_padded_bf16_fp32_backward, runtime/mod.rs:191-195 (padded_matrix.rs:47-63,
 * PaddedGemmSpec::backward_specs, deepgemm/padded.rs:39-50). */
hk_status hk_gemm_padded_bf16_fp32_backward(hk_context* ctx, const hk_tensor* a_pad,
                                            const hk_tensor* b_pad, const hk_tensor* dy,
                                            int32_t ta, int32_t tb, hk_tensor* da, hk_tensor* db);
/* Y[M,N] (F32) = bf16(X[M,K]) W[N,K]^T with a fixed BF16 weight. w_pad (BF16, both axes rounded
 * up to 16) receives the zero-padded weight the backward uses; it may be NULL when W's axes are
 * already multiples of 16 (W itself is then the saved weight, as the reference reuses the aligned
 * handle). Reference: AscendRuntime::linear_frozen_padded_bf16_fp32, runtime/mod.rs:196-200
 * (padded_matrix.rs:64-76). */
hk_status hk_linear_frozen_padded_bf16_fp32(hk_context* ctx, const hk_tensor* x, const hk_tensor* w,
                                            hk_tensor* y, hk_tensor* w_pad);
/* dX[M,K] (F32) from the saved padded weight and the logical F32 dY[M,N]. Reference:
 * AscendRuntime::linear_frozen_padded_bf16_fp32_backward, runtime/mod.rs:201-204
 * (padded_matrix.rs:77-87). */
hk_status hk_linear_frozen_padded_bf16_fp32_backward(hk_context* ctx, const hk_tensor* w_pad,
                                                     const hk_tensor* dy, hk_tensor* dx);

/* Y[M,N] (F32) = bf16(X[M,K]) W[N,K]^T for a fixed BF16 weight used in place (no cast or copy of
 * W); M/N/K positive multiples of 16. Reference: AscendRuntime::linear_frozen_bf16_fp32,
 * runtime/mod.rs:379-382 (matrix.rs:147-159). */
hk_status hk_linear_frozen_bf16_fp32(hk_context* ctx, const hk_tensor* x, const hk_tensor* w, hk_tensor* y);
/* dX[M,K] (F32) = bf16(dY[M,N]) W[N,K]; the weight receives no gradient. dX carries the input's
 * shape. Reference: AscendRuntime::linear_frozen_bf16_fp32_backward, runtime/mod.rs:383-386
 * (matrix.rs:160-172). */
hk_status hk_linear_frozen_bf16_fp32_backward(hk_context* ctx, const hk_tensor* w, const hk_tensor* dy,
                                              hk_tensor* dx);

/* Elementwise F32 <-> BF16 conversion (RNE, NaN kept quiet, Inf kept).
 * Reference: AscendRuntime::cast_into, runtime/mod.rs:276-279 (conversion.rs:21-62). */
hk_status hk_cast_into(hk_context* ctx, const hk_tensor* in, hk_tensor* out);

/* ---------------------------------------------------------------- RMSNorm */

/* y = x * rstd * w, rstd = 1/sqrt(mean(x^2) + eps) per row of the last axis.
 * x: F32 or BF16 [..., W]; w: F32 [W] (or x's dtype); y: x's dtype; rstd: F32 [rows].
 * Any positive W; empty batches are allowed. eps must be finite and positive in F32.
 * Reference: AscendRuntime::rms_norm, runtime/mod.rs:402-408 (normalization.rs:153-166,
 * row_programs.rs:144-151) and, for BF16 x with F32 rstd, CannSession::rms_norm
 * (tensor/ops.rs:347-385). */
hk_status hk_rms_norm(hk_context* ctx, const hk_tensor* x, const hk_tensor* w, double eps,
                      hk_tensor* y, hk_tensor* rstd);
/* dx (x's dtype) and dw (F32 [W], summed over all rows; zeros for an empty batch),
 * from the saved rstd (eps is not recomputed).
 * Reference: AscendRuntime::rms_norm_backward, runtime/mod.rs:410-415
 * (normalization.rs:168-186, row_programs.rs:200-217) and CannSession::rms_norm_backward
 * (tensor/backward.rs:127-148). */
hk_status hk_rms_norm_backward(hk_context* ctx, const hk_tensor* x, const hk_tensor* w,
                               const hk_tensor* dy, const hk_tensor* rstd,
                               hk_tensor* dx, hk_tensor* dw);
/* hk_rms_norm_backward with the residual branch's gradient added: dx = residual + the backward's dx,
 * the dx as stored (BF16: rounded) plus the residual in F32, stored again; dw as
 * hk_rms_norm_backward. Bit-identical to hk_rms_norm_backward followed by hk_bias_add(dx, no bias,
 * residual): the reference's rms_norm backward (row_programs.rs:200-217, normalization.rs:168-186)
 * and residual add (src/nn/affine.rs:14-25) of a pre-norm block's input, in one pass. residual:
 * dX's dtype and shape, not overlapping dX. */
hk_status hk_rms_norm_backward_residual(hk_context* ctx, const hk_tensor* x, const hk_tensor* w, const hk_tensor* dy,
                                        const hk_tensor* rstd, const hk_tensor* residual, hk_tensor* dx,
                                        hk_tensor* dw);
/* hk_rms_norm_backward without any allocation: no counterpart in the reference. For callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). Same arguments, checks and results as hk_rms_norm_backward (the same
 * kernels); its dgamma partials live in a fixed 8 MiB device array of the library (one per GPU,
 * held until the process ends) instead of the context workspace. Shapes whose partials exceed
 * it (widths above 4096 with many rows) are invalid arguments. Calls that overlap on one GPU
 * share the array and race. */
hk_status hk_rms_norm_backward_noalloc(hk_context* ctx, const hk_tensor* x, const hk_tensor* w,
                                       const hk_tensor* dy, const hk_tensor* rstd,
                                       hk_tensor* dx, hk_tensor* dw);

/* ---------------------------------------------------------------- softmax rows */

/* Softmax (logarithmic = 0) or log-softmax (logarithmic = 1) over the last axis of a
 * contiguous F32 tensor of any positive last-axis width; y has x's shape. Reference:
 * AscendRuntime::softmax / log_softmax, runtime/mod.rs:322-330 (runtime/rows.rs:50-62,
 * wide_rows.rs:162-210; arithmetic row_programs.rs:135-143). */
hk_status hk_softmax(hk_context* ctx, const hk_tensor* x, int32_t logarithmic, hk_tensor* y);
/* Backward from the saved output y: dx = y (dy - sum(y dy)) for softmax,
 * dx = dy - exp(y) sum(dy) for log-softmax. Reference: AscendRuntime::softmax_backward /
 * log_softmax_backward, runtime/mod.rs:332-341 (rows.rs:64-79, wide_rows.rs:212-232;
 * row_programs.rs:152-163). */
hk_status hk_softmax_backward(hk_context* ctx, const hk_tensor* y, const hk_tensor* dy, int32_t logarithmic,
                              hk_tensor* dx);

/* ---------------------------------------------------------------- SwiGLU gate */

/* y = SiLU(gate) * up = gate * sigmoid(gate) * up, element-wise over contiguous tensors of one
 * shape, F32 (the reference's dtype) or BF16 storage with F32 arithmetic; at most 2^32-1
 * elements. Reference: AscendRuntime::silu_mul, runtime/mod.rs:282-285 (elementwise.rs:13-19;
 * arithmetic rust-ascend-compiler/src/ascend/programs.rs:41). */
hk_status hk_silu_mul(hk_context* ctx, const hk_tensor* gate, const hk_tensor* up, hk_tensor* y);
/* dgate = dy * up * s (1 + gate (1 - s)), dup = dy * gate * s with s = sigmoid(gate).
 * Reference: AscendRuntime::silu_mul_backward, runtime/mod.rs:287-290 (elementwise.rs:21-30;
 * programs.rs:43). */
hk_status hk_silu_mul_backward(hk_context* ctx, const hk_tensor* gate, const hk_tensor* up, const hk_tensor* dy,
                               hk_tensor* dgate, hk_tensor* dup);

/* ---------------------------------------------------------------- bias and residual add */

/* y = (x + residual) + bias[c] over the last axis c, in that F32 order; residual may be NULL
 * (y = x + bias). X rank 1..8 with a positive last axis and at most 2^32-1 elements; X, residual
 * and Y F32 (the reference's dtype) or BF16 storage with F32 arithmetic; bias F32 [width];
 * residual exactly X's shape. Beyond the reference, bias may be NULL when a residual is given
 * (y = x + residual: the decoder layer's bias-free residual adds). Reference: AscendRuntime::bias_add, runtime/mod.rs:177-181
 * (runtime/affine.rs:10-22; nn::bias_add / residual_bias_add, src/nn/affine.rs:14-25). */
hk_status hk_bias_add(hk_context* ctx, const hk_tensor* x, const hk_tensor* bias, const hk_tensor* residual,
                      hk_tensor* y);
/* dbias [width] F32 = dY summed over every leading axis, pairwise in the reference's order (row i
 * plus row i + floor(r/2) per level, odd last row carried), so bit-identical to it; zeros when
 * there are no rows. Reference: AscendRuntime::bias_add_backward, runtime/mod.rs:182-185
 * (runtime/affine.rs:23-26, normalization.rs:95-114). */
hk_status hk_bias_add_backward(hk_context* ctx, const hk_tensor* dy, hk_tensor* dbias);

/* ---------------------------------------------------------------- decoder-layer relayouts */

/* These have no counterpart in the reference, whose composed layers keep one tensor per
 * projection; they serve a decoder layer built on one fused QKV projection. BF16, 16-byte aligned
 * tensors, D % 16 == 0.
 * qkv [B, S, (Hq + 2 Hkv) D] (per token: Q heads, K heads, V heads) -> q [B, Hq, S, D],
 * k, v [B, Hkv, S, D], with RoPE applied to Q and K in the same pass (the rotation of hk_rotary,
 * same layout codes, F32 tables cos/sin [S, D/2] indexed by the position s; bit-identical to
 * hk_rotary_prefix on [1,1,S,D/2] tables) and V copied bit-exactly. */
hk_status hk_qkv_rope_split(hk_context* ctx, const hk_tensor* qkv, const hk_tensor* cos, const hk_tensor* sin,
                            int32_t layout, hk_tensor* q, hk_tensor* k, hk_tensor* v);
/* The transpose: dQ, dK (rotated back) and dV -> dqkv [B, S, (Hq + 2 Hkv) D]. */
hk_status hk_qkv_rope_merge(hk_context* ctx, const hk_tensor* dq, const hk_tensor* dk, const hk_tensor* dv,
                            const hk_tensor* cos, const hk_tensor* sin, int32_t layout, hk_tensor* dqkv);
/* The fused QKV projection with RoPE in the GEMM's epilogue: x [B*S, H] (or [B, S, H]) times
 * W [(Hq + 2 Hkv) D, H]^T (BF16, FP32 accumulation), each 128-wide head of the product written
 * straight to its plane q [B, Hq, S, D] or k, v [B, Hkv, S, D], Q and K rotated on the way (tables
 * cos/sin [S, D/2] F32 indexed by s, either layout). D = 128 and H % 8 == 0. Bit-identical to
 * hk_gemm_into (NT, BF16 output) followed by hk_qkv_rope_split: each value is rounded to BF16 before
 * its rotation, as the product's storage rounds it there. It composes the reference's linear NT
 * (runtime/matrix.rs:47-74) and rotary_prefix (rotary_programs.rs:47-97, 101-156) on the rows of
 * the fused projection, in one launch. */
hk_status hk_qkv_projection_rope(hk_context* ctx, const hk_tensor* x, const hk_tensor* w, const hk_tensor* cos,
                                 const hk_tensor* sin, int32_t layout, hk_tensor* q, hk_tensor* k, hk_tensor* v);
/* y [M, N] = residual + x [M, K] W [N, K]^T (BF16, FP32 accumulation): the product is rounded to BF16
 * and the residual added in F32 and rounded, in the GEMM's epilogue. Bit-identical to hk_gemm_into
 * (NT, BF16 output) followed by hk_bias_add(product, no bias, residual); the reference's linear
 * (runtime/matrix.rs:47-74) and residual add (src/nn/affine.rs:14-25) in one launch. N % 16 == 0,
 * K % 8 == 0. */
hk_status hk_linear_residual(hk_context* ctx, const hk_tensor* x, const hk_tensor* w, const hk_tensor* residual,
                             hk_tensor* y);
/* SwiGLU's two projections as one GEMM: x [T, H] times W_gu [2F, H]^T, whose rows interleave the gate
 * and up weights in blocks of 16 (row 32 b + r is gate row 16 b + r for r < 16, up row 16 b + r - 16
 * otherwise), writes gate and up [T, F] (BF16) and act = SiLU(gate) * up [T, F] from the BF16 values
 * in the epilogue. Bit-identical to the two projections (hk_gemm_into, NT) and hk_silu_mul; the
 * reference's swiglu_bf16_fp32 (src/nn/feed_forward.rs:24-42, MapProgram::SiluMul,
 * rust-ascend-compiler/src/ascend/programs.rs:21-46) in one launch. F % 16 == 0, H % 8 == 0. */
hk_status hk_swiglu_projection(hk_context* ctx, const hk_tensor* x, const hk_tensor* w_gu, hk_tensor* gate,
                               hk_tensor* up, hk_tensor* act);
/* The SwiGLU backward fused into the down projection's input gradient: dM = dY [T, H] Wd [H, F]
 * (rounded to BF16 as hk_linear_nt_backward stores it) and hk_silu_mul_backward(gate, up, dM) in the
 * epilogue, written as dgu [T, 2F] interleaved like W_gu's rows, so that dX = dgu W_gu and
 * dW_gu = dgu^T X are single GEMMs (hk_linear_nt_backward(x, w_gu, dgu)). */
hk_status hk_swiglu_projection_backward(hk_context* ctx, const hk_tensor* dy, const hk_tensor* wd,
                                        const hk_tensor* gate, const hk_tensor* up, hk_tensor* dgu);
/* x [B, H, S, D] -> y [B, S, H D] (attention output into token rows), and the reverse; D % 8 == 0. */
hk_status hk_heads_to_rows(hk_context* ctx, const hk_tensor* x, hk_tensor* y);
hk_status hk_rows_to_heads(hk_context* ctx, const hk_tensor* x, hk_tensor* y);

/* ---------------------------------------------------------------- embedding */

/* No padding row (the SDK's unsigned sentinel, rust-ascend-driver/src/tensor/embedding.rs:14-15). */
#define HK_NO_PADDING UINT64_MAX

/* out [ids..., H] = weight[ids, :] for an F32/F16/BF16 table weight [V, H] and INT32/INT64 IDs of
 * rank 1..7 with values in [0, V); out has the table's dtype. An ID outside [0, V) writes a zero
 * row and, in synchronous mode, returns HK_INVALID_ARGUMENT after the call (asynchronous mode does
 * not check). Reference: AscendRuntime::embedding, runtime/mod.rs:237-241 (runtime/indexing.rs:33-37,
 * embedding.rs:21-34,46-60). */
hk_status hk_embedding(hk_context* ctx, const hk_tensor* weight, const hk_tensor* ids, hk_tensor* out);
/* dweight [num_weights, H] = sum of grad[t, :] over the positions t of each ID, in increasing
 * position order with F32 accumulation (deterministic); the padding row (padding_idx, or
 * HK_NO_PADDING) stays zero; with scale_grad_by_freq = 1 each row is divided by its ID count.
 * grad [ids..., H] F32/F16/BF16, dweight in grad's dtype. Reference: AscendRuntime::embedding_backward,
 * runtime/mod.rs:252-256 (runtime/indexing.rs:60-64, embedding.rs:35-44,60-79). */
hk_status hk_embedding_backward(hk_context* ctx, const hk_tensor* grad, const hk_tensor* ids, uint64_t num_weights,
                                uint64_t padding_idx, int32_t scale_grad_by_freq, hk_tensor* dweight);

/* ---------------------------------------------------------------- NLLLoss */

/* Reference: LossReduction {None=0, Mean=1, Sum=2}, rust-ascend-driver/src/tensor/loss.rs:3-6. */
typedef enum hk_loss_reduction { HK_LOSS_NONE = 0, HK_LOSS_MEAN = 1, HK_LOSS_SUM = 2 } hk_loss_reduction;

/* NLLLoss over log-probabilities input [N,C] (F32/F16/BF16) with INT32/INT64 labels target [N]
 * and class weights weight [C] (input's dtype). Row loss l_n = -weight[t_n] input[n,t_n]; a row
 * whose label equals ignore_index contributes nothing (pass NllLossOptions::ignore(): the ignore
 * label, or -1 when none is set, loss.rs:10-12). out: [N] (None) or [1] = sum (Sum) or sum / W
 * (Mean); total_weight [1] = W, the summed weight of the non-ignored labels (Sum, Mean; 0 for None).
 * A label outside [0, C) that is not ignore_index contributes nothing and, in synchronous mode,
 * returns HK_INVALID_ARGUMENT after the call. Sums over rows are deterministic.
 * Reference: AscendRuntime::nll_loss, runtime/mod.rs:227-228 (runtime/loss.rs:15-20,
 * CannSession::nll_loss, tensor/loss.rs:31-46, aclnnNLLLoss). */
hk_status hk_nll_loss(hk_context* ctx, const hk_tensor* input, const hk_tensor* target,
                      const hk_tensor* weight, int32_t reduction, int64_t ignore_index,
                      hk_tensor* out, hk_tensor* total_weight);
/* Dense dinput [N,C]: -weight[t_n] g_n at (n, t_n), zero elsewhere, g_n = grad[n] (None),
 * grad[0] (Sum) or grad[0] / total_weight (Mean). Reference: AscendRuntime::nll_loss_backward,
 * runtime/mod.rs:233-236 (tensor/loss.rs:47-60, aclnnNLLLossBackward). */
hk_status hk_nll_loss_backward(hk_context* ctx, const hk_tensor* grad, const hk_tensor* input,
                               const hk_tensor* target, const hk_tensor* weight,
                               const hk_tensor* total_weight, int32_t reduction,
                               int64_t ignore_index, hk_tensor* dinput);

/* ---------------------------------------------------------------- composed-attention shims */

/* The fused attention entry points apply the mask and the KV-head mapping themselves; these
 * three serve callers of the reference's composed attention. All F32, contiguous. */

/* out [B, Q, K] F32: -inf where key_start + k > query_start + q, else +0. Q, K > 0; the
 * absolute positions must not overflow u64 and B*Q*K must fit u32 (CausalMaskSpec::elements,
 * mask_programs.rs:7-19). Reference: AscendRuntime::causal_mask, runtime/mod.rs:205-206
 * (mask_programs.rs:20-40). */
hk_status hk_causal_mask(hk_context* ctx, uint64_t query_start, uint64_t key_start, hk_tensor* out);
/* x [B, Hkv, N, D] -> y [B, Hq, N, D] with kv_head = q_head / (Hq/Hkv); Hq % Hkv == 0 and both
 * element counts fit u32 (RepeatKvSpec::elements, heads_programs.rs:5-18). Reference:
 * AscendRuntime::repeat_kv_heads, runtime/mod.rs:208-209 (runtime/heads.rs:21-28). */
hk_status hk_repeat_kv_heads(hk_context* ctx, const hk_tensor* x, hk_tensor* y);
/* dy [B, Hq, N, D] -> dx [B, Hkv, N, D]: the replicas' sum, added in the reference's pairwise
 * level order. Reference: AscendRuntime::repeat_kv_heads_backward, runtime/mod.rs:210-213
 * (runtime/heads.rs:29-51). */
hk_status hk_repeat_kv_heads_backward(hk_context* ctx, const hk_tensor* dy, hk_tensor* dx);

/* ---------------------------------------------------------------- RoPE */

/* Full last-axis rotation with same-row F32 tables (table shape = input shape with
 * the last axis halved). x/y: F32 or BF16. Reference: AscendRuntime::rotary,
 * runtime/mod.rs:257-261 (runtime/rotary.rs:15-29, rotary_programs.rs:47-97). */
hk_status hk_rotary(hk_context* ctx, const hk_tensor* x, const hk_tensor* cos_t,
                    const hk_tensor* sin_t, int32_t layout, hk_tensor* y);
/* Transpose Jacobian. Reference: AscendRuntime::rotary_backward, runtime/mod.rs:264-268. */
hk_status hk_rotary_backward(hk_context* ctx, const hk_tensor* dy, const hk_tensor* cos_t,
                             const hk_tensor* sin_t, int32_t layout, hk_tensor* dx);
/* Rotate the first `width` values of the last axis; the tail is copied bit-exactly;
 * table leading axes are 1 or equal to the input's, last axis width/2.
 * Reference: AscendRuntime::rotary_prefix(_backward), runtime/mod.rs:214-221
 * (rotary_programs.rs:7-23,101-156). */
hk_status hk_rotary_prefix(hk_context* ctx, const hk_tensor* x, const hk_tensor* cos_t,
                           const hk_tensor* sin_t, int32_t width, int32_t layout, hk_tensor* y);
hk_status hk_rotary_prefix_backward(hk_context* ctx, const hk_tensor* dy, const hk_tensor* cos_t,
                                    const hk_tensor* sin_t, int32_t width, int32_t layout,
                                    hk_tensor* dx);

/* ---------------------------------------------------------------- attention */

/* Fused causal/non-causal grouped-query attention forward (FlashAttention-style,
 * online softmax, nothing materialized).
 *   q [B,Hq,M,D], k/v [B,Hkv,N,D] all BF16, or all F32 (the reference's FP32 surface: rounded
 *   to BF16 in the workspace first, as its matmul_bf16_fp32 rounds GEMM operands);
 *   o [B,Hq,M,D] BF16 or F32; lse [B,Hq,M] F32
 *   (natural-log logsumexp of the scaled, masked scores, saved for backward).
 *   Hq % Hkv == 0 and query head h reads KV head h / (Hq/Hkv) (heads_programs.rs:5-60).
 *   Causal: key j is excluded when key_start + j > query_start + i (mask_programs.rs:5-40).
 *   D in {16, 32, 64, 128}; the value width equals D.
 * Replaces the composed chain of src/nn/attention.rs:10-80 (causal_mask,
 * repeat_kv_heads, BF16 GEMMs, softmax) with one kernel; GEMM operands are BF16
 * and P is rounded to BF16 before P.V, as matmul_bf16_fp32 does. */
hk_status hk_attention_forward(hk_context* ctx, const hk_tensor* q, const hk_tensor* k,
                               const hk_tensor* v, float scale, int32_t causal,
                               uint64_t query_start, uint64_t key_start,
                               hk_tensor* o, hk_tensor* lse);
/* Materialized attention with an optional additive mask, the reference's composed path:
 * scaled_dot_product_attention_bf16_fp32 (rank 3: Q[B,M,D], K[B,N,D], V[B,N,Dv], mask F32 [B,M,N])
 * and grouped_query_attention_bf16_fp32 (rank 4: Q[B,Hq,M,D], K[B,Hkv,N,D], V[B,Hkv,N,Dv], mask F32
 * [B,Hq,M,N]), src/nn/attention.rs:10-67. O = bf16(softmax(bf16(Q) bf16(K)^T * scale + mask))
 * bf16(V), scores and softmax F32, O [.., M, Dv] F32 (or BF16). Q/K/V are F32 as in the reference
 * (BF16 also accepted); mask may be NULL. validate_dimensions' rules apply (src/nn/attention.rs:
 * 95-104): B*Hq in 1..4096, M/D/Dv positive multiples of 16, N a positive multiple of 32, a finite
 * scale, B*Hq*M*N within u32. Rows whose mask excludes every key give NaN, as the reference's
 * softmax does. */
hk_status hk_attention_masked_forward(hk_context* ctx, const hk_tensor* q, const hk_tensor* k,
                                      const hk_tensor* v, float scale, const hk_tensor* mask,
                                      hk_tensor* o);
/* Backward of hk_attention_masked_forward (the reference's autodiff chain: matmul_bf16_fp32 and
 * SoftmaxBackward, src/nn.rs:234-278,375-453): P is recomputed from Q, K and the mask; dP =
 * bf16(dO) bf16(V)^T, dS = P * (dP - rowsum(P * dP)), dMask = dS (F32, shaped like the mask;
 * NULL when not wanted), dQ = bf16(scale dS) bf16(K), dK = bf16(scale dS)^T bf16(Q) summed over
 * each KV head's query heads, dV = bf16(P)^T bf16(dO). dO F32 (or BF16); dq/dk/dv F32 or BF16. */
hk_status hk_attention_masked_backward(hk_context* ctx, const hk_tensor* q, const hk_tensor* k,
                                       const hk_tensor* v, const hk_tensor* mask,
                                       const hk_tensor* dout, float scale, hk_tensor* dq,
                                       hk_tensor* dk, hk_tensor* dv, hk_tensor* dmask);
/* Backward of hk_attention_forward from saved o and lse: dq [B,Hq,M,D],
 * dk/dv [B,Hkv,N,D] (F32 or BF16). Q/K/V, O and dO may each be F32 (F32 inputs are rounded to
 * BF16 first; an F32 O enters the row term rowsum(dO * O) unrounded). dK/dV sum over the query heads of each group in a
 * fixed order (no atomics), the deterministic analogue of repeat_kv_heads_backward
 * (runtime/heads.rs:29-51). dS enters its two GEMMs rounded to BF16, as in the reference's
 * MatmulBf16Fp32Backward chain (examples/grouped_attention_tensor.rs:30-40), which rounds scale*dS;
 * here dS is rounded before the scale, which multiplies dQ and dK once (equal within BF16
 * rounding). The context's workspace grows to B*Hq*ceil(N/32)*ceil(M/64)*4 KiB for the stored dS
 * (4 GiB at B4, Hq32, S4096) unless that exceeds the environment's HK_ATTN_DS_BUDGET bytes (default
 * 8 GiB), in which case dQ recomputes S and dP instead. */
hk_status hk_attention_backward(hk_context* ctx, const hk_tensor* q, const hk_tensor* k,
                                const hk_tensor* v, const hk_tensor* o, const hk_tensor* lse,
                                const hk_tensor* dout, float scale, int32_t causal,
                                uint64_t query_start, uint64_t key_start,
                                hk_tensor* dq, hk_tensor* dk, hk_tensor* dv);
/* hk_attention_backward for a decoder layer whose Q, K and V come from one fused projection with
 * RoPE (hk_qkv_projection_rope): dQ, dK and dV are written straight into the projection's gradient
 * rows dqkv [B, S, (Hq + 2 Hkv) D] (BF16), dQ and dK rotated back by RoPE's transpose (tables
 * cos/sin [S, D/2] F32, either layout), instead of into planes. D = 64 or 128 and M = N = S.
 * Bit-identical to hk_attention_backward with BF16 gradients followed by hk_qkv_rope_merge: each
 * gradient is rounded to BF16 before its rotation, as the planes would store it. No reference
 * counterpart as one call: it composes the attention backward (src/nn/attention.rs:69-80) with
 * rotary_prefix_backward (rotary_programs.rs:47-97) on the fused projection's rows. */
hk_status hk_attention_backward_qkv_rows(hk_context* ctx, const hk_tensor* q, const hk_tensor* k, const hk_tensor* v,
                                         const hk_tensor* o, const hk_tensor* lse, const hk_tensor* dout, float scale,
                                         int32_t causal, uint64_t query_start, uint64_t key_start, const hk_tensor* cos,
                                         const hk_tensor* sin, int32_t layout, hk_tensor* dqkv);

#ifdef __cplusplus
}
#endif

#endif /* HK_H */
