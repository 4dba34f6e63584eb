// hk_kernels.hpp — host-side launchers of the gfx950 kernels (internal to libhk.so).
// Each launcher enqueues work on `s` and returns hipGetLastError(); shapes were
// validated by the C-ABI layer (hk_driver.cpp) before any launcher is called.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hk {

// ---- RMSNorm (hk_rmsnorm.hip)
// The row-split kernels' exchange check: a wave whose bounded wait (spin_limit polls) for a
// partner's post runs out writes `seq` into *flag; the launchers set `used` when they launch a
// kernel that may write it, so the caller knows to read the word back.
struct RowCheck {
    int* flag;
    int seq;
    int spin_limit;
    int used;
};
// Bytes of workspace the backward needs for its FP64 dγ partial rows on the path these
// operands take.
size_t rms_backward_workspace_bytes(int64_t rows, int64_t width, const void* x, const void* w, const void* dy,
                                    const void* dx);
hipError_t rms_norm_forward(int dtype_bf16, const void* x, const float* w, void* y, float* rstd,
                            int64_t rows, int64_t width, float eps, RowCheck& rc, hipStream_t s);
// res (nullable, like dx): dx = res + the backward's dx as stored, added in F32 and stored again.
hipError_t rms_norm_backward(int dtype_bf16, const void* x, const float* w, const void* dy,
                             const float* rstd, const void* res, void* dx, float* dw, float* workspace, int64_t rows,
                             int64_t width, RowCheck& rc, hipStream_t s);

// ---- RoPE and casts (hk_rope.hip)
// Table row of input row r: sum over leading axes a of coord_a(r) * tstride[a]
// (tstride 0 on broadcast axes); same_row means table row == input row.
struct RopeMap {
    int32_t same_row;
    int32_t nlead;
    int64_t shape[7];
    int64_t tstride[7];
};
hipError_t rope_apply(int dtype_bf16, const void* x, const float* cos_t, const float* sin_t, void* y,
                      int64_t rows, int64_t width, int64_t p, int layout, int backward,
                      const RopeMap& map, hipStream_t s);
hipError_t cast_apply(int to_bf16, const void* in, void* out, int64_t n, hipStream_t s);

// ---- GEMM (hk_gemm.hip)
// C[g] = op(A[g]) op(B[g]) for g < batch; A, B BF16; C BF16 or F32. ta/tb as in the
// reference (0 = row-major [M,K] / [K,N]; 1 = [K,M] / [N,K]). Operands that are not
// K-contiguous are first transposed into `workspace` (gemm_workspace_bytes).
size_t gemm_workspace_bytes(int64_t batch, int64_t m, int64_t n, int64_t k, int ta, int tb);

// Generic floating matmul (hk_matmul.hip). MatmulBatch: the output's batch dims (innermost last,
// at most 4) and one operand's element stride along each (0 where the operand broadcasts).
struct MatmulBatch {
    int dims = 0;
    int64_t count = 1;  // product of shape
    int64_t shape[4] = {1, 1, 1, 1};
    int64_t stride[4] = {0, 0, 0, 0};
};
struct MatmulSpec {
    int dtype = 0;  // element type code of A, B and the output (F32 0, F16 1, BF16 27)
    int64_t m = 0, n = 0, k = 0;
    MatmulBatch batch, a_batch, b_batch;  // output batch shape; A's and B's strides over it
};
size_t matmul_workspace_bytes(const MatmulSpec& s);
hipError_t matmul(const MatmulSpec& s, const void* a, const void* b, void* out, void* workspace, int num_cus,
                  hipStream_t st);
// Module attention's score transform (hk_attention_module.hip) over F32 scores [B, H, Sq, Sk]:
// masked ? -inf : softcap(s * scale) + bias; masked = (causal and key > query) or mask != 0.
struct AttnScoreSpec {
    int64_t shape[4] = {0, 0, 0, 0};
    int64_t bias_stride[4] = {0, 0, 0, 0};  // element strides (0 along a broadcast dim)
    int64_t mask_stride[4] = {0, 0, 0, 0};
    float scale = 1.0f;
    float softcap = 0.0f;  // 0: none
    int causal = 0;
};
hipError_t attention_scores(const AttnScoreSpec& sp, const float* s, float* out, const float* bias,
                            const uint8_t* mask, hipStream_t st);
// ds and, when dbias is given, the bias gradient summed to bias_shape (4 dims; needs a workspace of
// B*H*Sq*Sk floats).
hipError_t attention_scores_backward(const AttnScoreSpec& sp, const float* s, const float* dout, float* ds,
                                     const uint8_t* mask, float* dbias, const int64_t* bias_shape, float* workspace,
                                     hipStream_t st);
hipError_t swap_last_dims(int elem_bytes, const void* x, void* y, int64_t G, int64_t R, int64_t C, hipStream_t st);
size_t matmul_backward_workspace_bytes(const MatmulSpec& s);
// dA = dY B^T summed over A's broadcast batches, dB = A^T dY summed over B's, each in the dtype.
hipError_t matmul_backward(const MatmulSpec& s, const void* a, const void* b, const void* dy, void* da, void* db,
                           void* workspace, int num_cus, hipStream_t st);
hipError_t gemm_bf16(const void* a, const void* b, void* c, int out_bf16, int64_t batch, int64_t m,
                     int64_t n, int64_t k, int ta, int tb, void* workspace, int num_cus, hipStream_t s);
// M-grouped NT GEMM: C[i, :] = A[i, :] W[g(i)]^T with A [m, k], W [groups, n, k], C [m, n];
// g(i) = block_group[i / 256] (group ends are multiples of 256). No workspace.
hipError_t gemm_bf16_grouped_nt(const void* a, const void* w, void* c, int out_bf16, int64_t m, int64_t n,
                                int64_t k, const int32_t* block_group, int num_cus, hipStream_t s);

// The decoder layer's fused QKV projection with RoPE: x [T, H] times W [(Hq + 2 Hkv) 128, H]^T into
// q [B, Hq, seq, 128], k, v [B, Hkv, seq, 128] (T = B seq), Q and K rotated with tables
// [seq, 64]; bit-identical to gemm_bf16 (NT, BF16 out) followed by qkv_rope (split).
bool qkv_rope_applies(int64_t tokens, int64_t hidden, int64_t width);
hipError_t gemm_qkv_rope(const void* x, const void* w, int64_t tokens, int64_t hidden, int64_t seq, int64_t hq,
                         int64_t hkv, const float* cos_t, const float* sin_t, int layout, void* q, void* k, void* v,
                         hipStream_t s);
// The other fused-epilogue GEMMs of a decoder layer (BF16, 256x256 tiles at any M and N; they apply
// when K % 8 == 0 and M K, N K stay below 2^30 elements, K rounded up to 64):
bool epi_applies(int64_t m, int64_t n, int64_t k);
// y [m, n] = res + x [m, k] W [n, k]^T (the product rounded to BF16 before the add)
hipError_t gemm_residual(const void* x, const void* w, const void* res, void* y, int64_t m, int64_t n, int64_t k,
                         hipStream_t s);
// gate, up, act [m, f]: x [m, k] W_gu [2f, k]^T with W_gu's rows interleaving gate and up in blocks of
// 16 (row 32 b + r: gate row 16 b + r for r < 16, else up row 16 b + r - 16); act = SiLU(gate) up
hipError_t gemm_swiglu(const void* x, const void* w_gu, void* gate, void* up, void* act, int64_t m, int64_t f,
                       int64_t k, hipStream_t s);
// dgu [m, 2f] (interleaved as W_gu's rows) = the SwiGLU gradients of gate and up for
// dM = dY [m, k] Wd [k, f] (Wd stored [k, f])
hipError_t gemm_swiglu_backward(const void* dy, const void* wd, const void* gate, const void* up, void* dgu, int64_t m,
                                int64_t f, int64_t k, hipStream_t s);

// ---- NLLLoss (hk_loss.hip)
// dtype 0 F32, 1 F16, 2 BF16 (input, weight, out, total, grad, dinput); id_bytes 4 or 8;
// reduction 0 None, 1 Mean, 2 Sum. The forward writes *bad = 1 if a label outside [0, classes)
// that is not `ignore` occurs.
size_t nll_loss_workspace_bytes(int64_t rows);  // the label flag and the per-row terms
hipError_t nll_loss(int dtype, int id_bytes, const void* input, const void* target, const void* weight, void* out,
                    void* total, int64_t rows, int64_t classes, int reduction, int64_t ignore, void* workspace, hipStream_t s);
hipError_t nll_loss_backward(int dtype, int id_bytes, const void* grad, const void* target, const void* weight,
                             const void* total, void* dinput, int64_t rows, int64_t classes, int reduction,
                             int64_t ignore, hipStream_t s);

// ---- matrix tails (hk_pad.hip)
// dst [batch, R, C] BF16 = src [batch, rows, cols] (F32 rounded to BF16 with RNE, or BF16 copied)
// zero-padded (rows <= R, cols <= C, C even).
hipError_t pad_bf16(int src_bf16, const void* src, void* dst, int64_t batch, int64_t rows, int64_t cols, int64_t R,
                    int64_t C, hipStream_t s);
// dst [batch, rows, cols] = the leading window of src [batch, R, C] (F32).
hipError_t crop_f32(const float* src, float* dst, int64_t batch, int64_t rows, int64_t cols, int64_t R, int64_t C,
                    hipStream_t s);

// ---- element-wise (hk_elementwise.hip)
// SwiGLU gate, element-wise over n values of F32 or BF16 storage.
hipError_t silu_mul(int dtype_bf16, const void* gate, const void* up, void* y, int64_t n, hipStream_t s);
// Composed attention helpers: scores = scores * scale (+ mask), in place; out = bf16(scale * x).
hipError_t scale_mask(float* scores, const float* mask, float scale, int64_t n, hipStream_t s);
hipError_t scale_to_bf16(const float* x, float scale, void* out, int64_t n, hipStream_t s);
hipError_t silu_mul_backward(int dtype_bf16, const void* gate, const void* up, const void* dy, void* dgate,
                             void* dup, int64_t n, hipStream_t s);
// y = (x + residual) + bias[i % width] over n values (residual may be null); x/residual/y F32 or
// BF16 storage, bias F32.
hipError_t bias_add(int dtype_bf16, const void* x, const float* bias, const void* residual, void* y, int64_t n,
                    int64_t width, hipStream_t s);
// out[width] = pairwise column sum of dy[rows, width] (F32) in the order of repeated halving.
size_t column_sum_workspace_bytes(int64_t rows, int64_t width);
hipError_t column_sum(const float* dy, float* out, int64_t rows, int64_t width, void* workspace, hipStream_t s);

// ---- embedding (hk_embedding.hip)
// Lookup of `tokens` rows of `row_bytes` bytes from a [vocab, .] table by INT32/INT64 IDs
// (id_bytes 4 or 8); the workspace's first int becomes nonzero if an ID lies outside [0, vocab).
size_t embedding_workspace_bytes(int64_t tokens, int64_t vocab, bool backward);
// An index outside [0, vocab) writes `seq` to *flag (and zeros to its row); *flag is not cleared
// first, so a caller gives every call its own seq and compares afterwards.
hipError_t embedding(const void* table, int id_bytes, const void* ids, void* out, int64_t tokens, int64_t vocab,
                     int64_t row_bytes, int* flag, int seq, hipStream_t s);
// Dense gradient dw[vocab, width] from grad[tokens, width]; dtype is the hk_dtype code of grad/dw
// (F32, F16 or BF16); padding == UINT64_MAX means no padding row.
hipError_t embedding_backward(int dtype, const void* grad, int id_bytes, const void* ids, void* dw, int64_t tokens,
                              int64_t vocab, int64_t width, uint64_t padding, int scale, void* workspace,
                              hipStream_t s);
// Kernel launches one embedding_backward call enqueues (for the context's launch counter).
int embedding_backward_launches(int64_t tokens, int64_t vocab, int64_t width);

// Row softmax / log-softmax over the last axis of contiguous F32 [rows, width] (hk_softmax.hip).
hipError_t softmax_forward(const float* x, float* y, int64_t rows, int64_t width, int logarithmic, hipStream_t s);
hipError_t softmax_backward(const float* y, const float* dy, float* dx, int64_t rows, int64_t width, int logarithmic,
                            hipStream_t s);

// Composed-attention compatibility kernels (hk_heads.hip); F32, contiguous.
hipError_t causal_mask(float* out, int64_t batch, int64_t queries, int64_t keys, uint64_t query_start,
                       uint64_t key_start, hipStream_t s);
hipError_t repeat_kv_heads(const float* x, float* y, int64_t batch, int64_t kv_heads, int64_t query_heads,
                           int64_t plane, hipStream_t s);
size_t repeat_kv_backward_workspace_bytes(int64_t batch, int64_t kv_heads, int64_t query_heads, int64_t plane);
hipError_t repeat_kv_heads_backward(const float* dy, float* dx, int64_t batch, int64_t kv_heads,
                                    int64_t query_heads, int64_t plane, void* workspace, hipStream_t s);

// ---- decoder-layer relayouts (hk_layout.hip); BF16, D % 16 == 0, 16-byte aligned bases.
// merge = false: rows [B,S,(Hq+2Hkv)D] -> q [B,Hq,S,D], k/v [B,Hkv,S,D], RoPE on q/k;
// merge = true: the transpose (dq, dk, dv -> rows) with the backward rotation.
hipError_t qkv_rope(bool merge, int layout, void* rows, void* q, void* k, void* v, const float* cos_t,
                    const float* sin_t, int64_t batch, int64_t seq, int64_t hq, int64_t hkv, int64_t d, hipStream_t s);
// to_rows: x [B,H,S,D] -> y [B,S,H*D]; otherwise the reverse (D % 8 == 0).
hipError_t heads_rows(bool to_rows, const void* x, void* y, int64_t batch, int64_t heads, int64_t seq, int64_t d,
                      hipStream_t s);

// ---- attention (hk_attention.hip)
struct AttnShape {
    int64_t batch, heads, kv_heads, m, n, d;
    float scale;
    int32_t causal;
    uint64_t query_start, key_start;
    int32_t o_f32 = 0;  // O (forward output, backward input) is F32 instead of BF16
    int32_t store_ds = 0;  // backward: dS stored for the dQ kernel (set by attention_bwd_plan)
    int32_t dkv_splits = 1;  // backward: workgroups per dK/dV key block (set by attention_bwd_plan)
};
// Chooses the backward's dQ form (store_ds) and dK/dV split (dkv_splits) for the shape on num_cus
// CUs; the workspace size and the backward call then follow that choice.
void attention_bwd_plan(AttnShape& sh, int num_cus);
size_t attention_bwd_workspace_bytes(const AttnShape& sh);
// Whether the fused kernels can take the shape: one head of Q/K/V (M*D and N*D BF16 elements)
// within 32-bit buffer offsets, and every launch's work items within a dispatch's 32-bit count.
bool attention_shape_fits(const AttnShape& sh);
hipError_t attention_forward(const AttnShape& sh, const void* q, const void* k, const void* v, void* o,
                             float* lse, hipStream_t s);
// The backward's rows output (D = 64 or 128, M = N = S): dQ, dK, dV written as BF16 token rows
// [B, S, row_w] of a fused QKV projection's gradient, dQ and dK rotated back by RoPE (tables
// [S, D/2]); dq/dk/dv are then not written.
struct AttnRowsOut {
    void* rows;
    int64_t row_w;
    const float* cos;
    const float* sin;
    int layout;
};
hipError_t attention_backward(const AttnShape& sh, const void* q, const void* k, const void* v,
                              const void* o, const float* lse, const void* dout, void* dq, int dq_bf16,
                              void* dk, void* dv, int dkv_bf16, const AttnRowsOut* rows, void* workspace,
                              hipStream_t s);

}  // namespace hk
