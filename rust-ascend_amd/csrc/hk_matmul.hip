// hk_matmul.hip — the generic floating matmul (F32, F16, BF16 with the input's own dtype out,
// FP32 accumulation), batch dimensions broadcast, any positive M/N/K, for gfx950.
//
// Semantics (reference: AscendRuntime::tensor_matmul, rust-ascend-driver/src/tensor/runtime/
// mod.rs:156-158 -> generic_matrix::matmul (generic_matrix.rs:17-54) -> worker.rs:128-162, which
// runs aclnnMatmul with cubeMathType 0 = KEEP_DTYPE): out[b..., i, j] = sum_k A[b_a..., i, k] *
// B[b_b..., k, j], A [..., M, K] and B [..., K, N] row-major, batch dims broadcast numpy-style
// (layout.rs:106-142), FP32 products and sums, the output rounded to the inputs' dtype (RNE).
//
// Design: the operands are first gathered into packed, zero-padded NT operands in the workspace,
// A' [G, Mp, Kp] and B' [G, Np, Kp] (B transposed on the way), one slice per output batch with the
// broadcast applied by the gather's batch strides (0 along a broadcast dim). Padding with zeros
// adds nothing to the sums. The product runs on MFMA tiles without any bounds logic: BF16 on the
// library's BF16 GEMM (hk_gemm.hip), F32 and F16 on the 64x64-tile kernels below, into C'
// [G, Mp, Np], from which the [G, M, N] output is cropped. This path serves the generic backend
// op (float_matmul); the transformer's own GEMMs use hk_gemm.hip directly.
#include "hk_common.hpp"
#include "hk_kernels.hpp"

#include <algorithm>

namespace hk {

namespace {

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

constexpr int kMT = 64;  // output tile edge of both kernels
constexpr int kThreads = 256;

// dst[g][r][c] = src[batch g][r][c] (or, transposed, src[batch g][c][r]) for r < rows, c < cols,
// zero elsewhere; dst is [G, R, C]. The source offset of batch g is sum_d idx_d(g) * stride_d over
// the output batch dims (innermost last), a zero stride broadcasting that dim.
template <typename T>
__global__ void __launch_bounds__(256)
gather_pad(const T* __restrict__ src, T* __restrict__ dst, MatmulBatch mb, int64_t rows, int64_t cols,
           int64_t ld, int transpose, int64_t R, int64_t C) {
    const int64_t plane = R * C, total = plane * mb.count;
    for (int64_t i = flat_begin(256); i < total; i += flat_stride(256)) {
        const int64_t g = i / plane, rc = i - g * plane;
        const int64_t r = rc / C, c = rc - r * C;
        T v = T(0);
        if (r < rows && c < cols) {
            int64_t off = 0, rest = g;
            for (int d = mb.dims - 1; d >= 0; --d) {
                const int64_t idx = rest % mb.shape[d];
                rest /= mb.shape[d];
                off += idx * mb.stride[d];
            }
            v = transpose ? src[off + c * ld + r] : src[off + r * ld + c];
        }
        dst[i] = v;
    }
}

// dst[g][r][c] = src[g][r][c] for r < rows, c < cols; src is [G, R, C], dst [G, rows, cols].
template <typename T>
__global__ void __launch_bounds__(256)
crop(const T* __restrict__ src, T* __restrict__ dst, int64_t G, int64_t rows, int64_t cols, int64_t R, int64_t C) {
    const int64_t plane = rows * cols, total = plane * G;
    for (int64_t i = flat_begin(256); i < total; i += flat_stride(256)) {
        const int64_t g = i / plane, rc = i - g * plane;
        const int64_t r = rc / cols, c = rc - r * cols;
        dst[i] = src[(g * R + r) * C + c];
    }
}

__global__ void __launch_bounds__(256) zero_u8(unsigned char* p, int64_t n) {
    for (int64_t i = flat_begin(256); i < n; i += flat_stride(256)) p[i] = 0;
}

// Epilogue of a 64x64 tile computed as four 32x32 MFMA blocks, B as the MFMA's first operand:
// lane l holds C[m = tm*64 + 32 wm + l%32][n = tn*64 + 32 wn + 8 grp + 4 (l/32) + 0..3] in
// acc[4 grp .. 4 grp + 3].
template <typename T>
__device__ __forceinline__ void store_tile64(T* C, int64_t ldc, int m0, int n0, int lane, const f32x16_t& acc) {
    const int m = m0 + (lane & 31);
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
        const int n = n0 + grp * 8 + (lane >> 5) * 4;
        T* p = C + m * ldc + n;
#pragma unroll
        for (int e = 0; e < 4; ++e) p[e] = static_cast<T>(acc[grp * 4 + e]);
    }
}

// F32: C'[g] = A'[g] B'[g]^T with v_mfma_f32_32x32x2_f32. 64x64 tile per workgroup, four waves
// (2x2) of 32x32, K steps of 32 through LDS (rows padded to 36 floats: the 32 lanes of a
// half-wave read 32 rows at a 144-byte stride, each 8-lane group over distinct banks), the next
// step prefetched into registers. An MFMA takes one k pair per lane half: lane l contributes
// k = 8s + 4(l/32) + u to MFMA (s, u) for A and B alike, so the 16 MFMAs of a step cover its 32 k.
constexpr int kF32K = 32, kF32Ld = kF32K + 4;
__global__ void __launch_bounds__(kThreads)
matmul_f32_nt(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int tiles_n,
              int64_t Mp, int64_t Np, int64_t Kp) {
    __shared__ __attribute__((aligned(16))) float la[2][kMT * kF32Ld];
    __shared__ __attribute__((aligned(16))) float lb[2][kMT * kF32Ld];
    const int tm = blockIdx.x / tiles_n, tn = blockIdx.x - (blockIdx.x / tiles_n) * tiles_n;
    const int64_t g = blockIdx.z;
    A += (g * Mp + tm * kMT) * Kp;
    B += (g * Np + tn * kMT) * Kp;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1, lr = lane & 31, h = lane >> 5;
    const int row = t >> 3, col = (t & 7) * 4;
    f32x4_t ra[2], rb[2];
    auto load = [&](int kt) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            ra[i] = *reinterpret_cast<const f32x4_t*>(A + (row + 32 * i) * Kp + kt * kF32K + col);
            rb[i] = *reinterpret_cast<const f32x4_t*>(B + (row + 32 * i) * Kp + kt * kF32K + col);
        }
    };
    auto stash = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            *reinterpret_cast<f32x4_t*>(&la[buf][(row + 32 * i) * kF32Ld + col]) = ra[i];
            *reinterpret_cast<f32x4_t*>(&lb[buf][(row + 32 * i) * kF32Ld + col]) = rb[i];
        }
    };
    f32x16_t acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
    const int nk = static_cast<int>(Kp / kF32K);
    load(0);
    stash(0);
    if (nk > 1) load(1);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
#pragma unroll
        for (int s = 0; s < kF32K / 8; ++s) {
            const f32x4_t fa = *reinterpret_cast<const f32x4_t*>(&la[cur][(wm * 32 + lr) * kF32Ld + 8 * s + 4 * h]);
            const f32x4_t fb = *reinterpret_cast<const f32x4_t*>(&lb[cur][(wn * 32 + lr) * kF32Ld + 8 * s + 4 * h]);
#pragma unroll
            for (int u = 0; u < 4; ++u) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(fb[u], fa[u], acc, 0, 0, 0);
        }
        if (kt + 1 < nk) {
            stash(cur ^ 1);
            if (kt + 2 < nk) load(kt + 2);
        }
        __syncthreads();
    }
    store_tile64(C + g * Mp * Np, Np, tm * kMT + wm * 32, tn * kMT + wn * 32, lane, acc);
}

// F16: the same tile with v_mfma_f32_32x32x16_f16, K steps of 64 halves (LDS rows padded to 72
// halves = 144 bytes); lane l contributes k = 16s + 8(l/32) + 0..7 to MFMA s.
constexpr int kF16K = 64, kF16Ld = kF16K + 8;
template <typename TO>
__global__ void __launch_bounds__(kThreads)
matmul_f16_nt(const _Float16* __restrict__ A, const _Float16* __restrict__ B, TO* __restrict__ C, int tiles_n,
              int64_t Mp, int64_t Np, int64_t Kp) {
    __shared__ __attribute__((aligned(16))) _Float16 la[2][kMT * kF16Ld];
    __shared__ __attribute__((aligned(16))) _Float16 lb[2][kMT * kF16Ld];
    const int tm = blockIdx.x / tiles_n, tn = blockIdx.x - (blockIdx.x / tiles_n) * tiles_n;
    const int64_t g = blockIdx.z;
    A += (g * Mp + tm * kMT) * Kp;
    B += (g * Np + tn * kMT) * Kp;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1, lr = lane & 31, h = lane >> 5;
    const int row = t >> 3, col = (t & 7) * 8;
    f16x8_t ra[2], rb[2];
    auto load = [&](int kt) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            ra[i] = *reinterpret_cast<const f16x8_t*>(A + (row + 32 * i) * Kp + kt * kF16K + col);
            rb[i] = *reinterpret_cast<const f16x8_t*>(B + (row + 32 * i) * Kp + kt * kF16K + col);
        }
    };
    auto stash = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            *reinterpret_cast<f16x8_t*>(&la[buf][(row + 32 * i) * kF16Ld + col]) = ra[i];
            *reinterpret_cast<f16x8_t*>(&lb[buf][(row + 32 * i) * kF16Ld + col]) = rb[i];
        }
    };
    f32x16_t acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
    const int nk = static_cast<int>(Kp / kF16K);
    load(0);
    stash(0);
    if (nk > 1) load(1);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
#pragma unroll
        for (int s = 0; s < kF16K / 16; ++s) {
            const f16x8_t fa = *reinterpret_cast<const f16x8_t*>(&la[cur][(wm * 32 + lr) * kF16Ld + 16 * s + 8 * h]);
            const f16x8_t fb = *reinterpret_cast<const f16x8_t*>(&lb[cur][(wn * 32 + lr) * kF16Ld + 16 * s + 8 * h]);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb, fa, acc, 0, 0, 0);
        }
        if (kt + 1 < nk) {
            stash(cur ^ 1);
            if (kt + 2 < nk) load(kt + 2);
        }
        __syncthreads();
    }
    store_tile64(C + g * Mp * Np, Np, tm * kMT + wm * 32, tn * kMT + wn * 32, lane, acc);
}

template <typename T> __device__ __forceinline__ T to_elem(float x);
template <> __device__ __forceinline__ float to_elem<float>(float x) { return x; }
template <> __device__ __forceinline__ _Float16 to_elem<_Float16>(float x) { return static_cast<_Float16>(x); }
template <> __device__ __forceinline__ uint16_t to_elem<uint16_t>(float x) { return f32_to_bf16(x); }  // BF16 RNE

// out[go][r][c] = sum over the output batches g that broadcast onto batch go of src[g][r][c], in
// increasing g, for r < rows, c < cols; src is [G, R, C] F32 (G = the output batch count), out
// [count of the operand's batch, rows, cols]. op_shape is the operand's batch shape aligned to the
// output's (1 along a dim it broadcasts), so with no broadcast dim this is a crop and a conversion.
template <typename T>
__global__ void __launch_bounds__(256)
reduce_batches(const float* __restrict__ src, T* __restrict__ out, MatmulBatch ob, MatmulBatch op, int64_t rows,
               int64_t cols, int64_t R, int64_t C) {
    const int64_t plane = rows * cols, total = plane * op.count;
    int64_t ostride[4], reps = 1, st = 1;
    for (int d = ob.dims - 1; d >= 0; --d) {
        ostride[d] = st;
        st *= ob.shape[d];
        if (op.shape[d] == 1) reps *= ob.shape[d];
    }
    for (int64_t i = flat_begin(256); i < total; i += flat_stride(256)) {
        const int64_t go = i / plane, rc = i - go * plane;
        const int64_t r = rc / cols, c = rc - r * cols;
        int64_t base = 0, rest = go;
        for (int d = ob.dims - 1; d >= 0; --d) {
            const int64_t idx = rest % op.shape[d];
            rest /= op.shape[d];
            base += idx * ostride[d];
        }
        float sum = 0.0f;
        for (int64_t rep = 0; rep < reps; ++rep) {  // the broadcast dims' indices, lexicographic
            int64_t g = base, q = rep;
            for (int d = ob.dims - 1; d >= 0; --d)
                if (op.shape[d] == 1) {
                    g += (q % ob.shape[d]) * ostride[d];
                    q /= ob.shape[d];
                }
            sum += src[(g * R + r) * C + c];
        }
        out[i] = to_elem<T>(sum);
    }
}

int64_t round_up(int64_t x, int64_t q) { return (x + q - 1) / q * q; }

// Padded extents of an NT product X [rows, K] Y [cols, K]^T: whole kernel tiles and K steps.
struct Padded {
    int64_t M, N, K;
};
Padded padded(int dtype, int64_t m, int64_t n, int64_t k) {
    const int64_t kq = dtype == 0 ? kF32K : dtype == 1 ? kF16K : 16;
    const int64_t mq = dtype == 27 ? 16 : kMT;
    return {round_up(m, mq), round_up(n, mq), round_up(k, kq)};
}

size_t round256(size_t x) { return (x + 255) & ~size_t(255); }

// One gathered operand: the [rows, cols] matrices of src (row stride ld, or transposed: element
// (r, c) at c * ld + r) over the output batches, strides in b.
struct Gather {
    const void* src;
    MatmulBatch b;
    int64_t rows, cols, ld;
    int transpose;
};

template <typename T>
void gather(const Gather& x, void* dst, int64_t R, int64_t C, hipStream_t st) {
    hipLaunchKernelGGL((gather_pad<T>), dim3(flat_blocks(x.b.count * R * C, 256)), dim3(256), 0, st,
                       static_cast<const T*>(x.src), static_cast<T*>(dst), x.b, x.rows, x.cols, x.ld, x.transpose, R,
                       C);
}

size_t product_bytes(int dtype, int64_t G, const Padded& p, bool out_f32) {
    const size_t es = dtype == 0 ? 4 : 2, eo = out_f32 ? 4 : es;
    return round256(G * p.M * p.K * es) + round256(G * p.N * p.K * es) + round256(G * p.M * p.N * eo);
}

// C'[g] = X[g] Y[g]^T for the output batches g, X [rows M, K] and Y [cols N, K] gathered into the
// workspace, zero-padded to p; C' [G, p.M, p.N] in F32 (out_f32) or the dtype, at *c (the
// workspace's third piece).
hipError_t product(int dtype, int64_t G, const Gather& x, const Gather& y, const Padded& p, bool out_f32,
                   void* workspace, void** c, int num_cus, hipStream_t st) {
    const size_t es = dtype == 0 ? 4 : 2;
    char* ws = static_cast<char*>(workspace);
    void* xp = ws;
    void* yp = ws + round256(G * p.M * p.K * es);
    void* cp = static_cast<char*>(yp) + round256(G * p.N * p.K * es);
    *c = cp;
    if (dtype == 0) {
        gather<float>(x, xp, p.M, p.K, st);
        gather<float>(y, yp, p.N, p.K, st);
    } else {
        gather<uint16_t>(x, xp, p.M, p.K, st);  // F16 and BF16 move as 16-bit words
        gather<uint16_t>(y, yp, p.N, p.K, st);
    }
    const size_t eo = out_f32 ? 4 : es;
    const int tiles_n = static_cast<int>(p.N / kMT);
    for (int64_t g0 = 0; g0 < G; g0 += 4096) {  // at most 4096 batches per launch
        const int64_t gc = G - g0 < 4096 ? G - g0 : 4096;
        const char* xg = static_cast<const char*>(xp) + g0 * p.M * p.K * es;
        const char* yg = static_cast<const char*>(yp) + g0 * p.N * p.K * es;
        char* cg = static_cast<char*>(cp) + g0 * p.M * p.N * eo;
        const dim3 grid(static_cast<unsigned>((p.M / kMT) * tiles_n), 1, static_cast<unsigned>(gc));
        if (dtype == 0) {
            hipLaunchKernelGGL(matmul_f32_nt, grid, dim3(kThreads), 0, st, reinterpret_cast<const float*>(xg),
                               reinterpret_cast<const float*>(yg), reinterpret_cast<float*>(cg), tiles_n, p.M, p.N, p.K);
        } else if (dtype == 1) {
            if (out_f32)
                hipLaunchKernelGGL((matmul_f16_nt<float>), grid, dim3(kThreads), 0, st,
                                   reinterpret_cast<const _Float16*>(xg), reinterpret_cast<const _Float16*>(yg),
                                   reinterpret_cast<float*>(cg), tiles_n, p.M, p.N, p.K);
            else
                hipLaunchKernelGGL((matmul_f16_nt<_Float16>), grid, dim3(kThreads), 0, st,
                                   reinterpret_cast<const _Float16*>(xg), reinterpret_cast<const _Float16*>(yg),
                                   reinterpret_cast<_Float16*>(cg), tiles_n, p.M, p.N, p.K);
        } else {
            // NT operands need no transposition, so the GEMM takes no workspace
            hipError_t e = gemm_bf16(xg, yg, cg, out_f32 ? 0 : 1, gc, p.M, p.N, p.K, 0, 1, nullptr, num_cus, st);
            if (e != hipSuccess) return e;
        }
    }
    return hipGetLastError();
}

MatmulBatch packed_batch(const MatmulBatch& shape, int64_t plane) {  // a contiguous [G, ...] operand
    MatmulBatch b = shape;
    int64_t st = plane;
    for (int d = shape.dims - 1; d >= 0; --d) {
        b.stride[d] = st;
        st *= shape.shape[d];
    }
    return b;
}

MatmulBatch operand_shape(const MatmulBatch& out, const MatmulBatch& op) {  // 1 along broadcast dims
    MatmulBatch b = out;
    for (int d = 0; d < out.dims; ++d) b.shape[d] = op.stride[d] == 0 ? 1 : out.shape[d];
    b.count = 1;
    for (int d = 0; d < out.dims; ++d) b.count *= b.shape[d];
    return b;
}

hipError_t zero_fill(void* p, int64_t bytes, hipStream_t st) {
    if (bytes <= 0) return hipSuccess;
    hipLaunchKernelGGL(zero_u8, dim3(flat_blocks(bytes, 256)), dim3(256), 0, st, static_cast<unsigned char*>(p), bytes);
    return hipGetLastError();
}

template <typename T>
void reduce(const float* c, void* out, const MatmulBatch& ob, const MatmulBatch& op, int64_t rows, int64_t cols,
            int64_t R, int64_t C, hipStream_t st) {
    hipLaunchKernelGGL((reduce_batches<T>), dim3(flat_blocks(op.count * rows * cols, 256)), dim3(256), 0, st, c,
                       static_cast<T*>(out), ob, op, rows, cols, R, C);
}

void reduce_any(int dtype, const float* c, void* out, const MatmulBatch& ob, const MatmulBatch& op, int64_t rows,
                int64_t cols, int64_t R, int64_t C, hipStream_t st) {
    if (dtype == 0) reduce<float>(c, out, ob, op, rows, cols, R, C, st);
    else if (dtype == 1) reduce<_Float16>(c, out, ob, op, rows, cols, R, C, st);
    else reduce<uint16_t>(c, out, ob, op, rows, cols, R, C, st);
}

}  // namespace

size_t matmul_workspace_bytes(const MatmulSpec& s) {
    return product_bytes(s.dtype, s.batch.count, padded(s.dtype, s.m, s.n, s.k), false);
}

size_t matmul_backward_workspace_bytes(const MatmulSpec& s) {
    const Padded pa = padded(s.dtype, s.m, s.k, s.n), pb = padded(s.dtype, s.k, s.n, s.m);
    return std::max(product_bytes(s.dtype, s.batch.count, pa, true), product_bytes(s.dtype, s.batch.count, pb, true));
}

hipError_t matmul(const MatmulSpec& s, const void* a, const void* b, void* out, void* workspace, int num_cus,
                  hipStream_t st) {
    const int64_t G = s.batch.count;
    const size_t es = s.dtype == 0 ? 4 : 2;
    if (G * s.m * s.n == 0) return hipSuccess;
    if (s.k == 0) return zero_fill(out, G * s.m * s.n * static_cast<int64_t>(es), st);  // an empty contraction
    const Padded p = padded(s.dtype, s.m, s.n, s.k);
    const Gather x{a, s.a_batch, s.m, s.k, s.k, 0}, y{b, s.b_batch, s.n, s.k, s.n, 1};
    void* c = nullptr;
    hipError_t e = product(s.dtype, G, x, y, p, false, workspace, &c, num_cus, st);
    if (e != hipSuccess) return e;
    if (s.dtype == 0)
        hipLaunchKernelGGL((crop<float>), dim3(flat_blocks(G * s.m * s.n, 256)), dim3(256), 0, st,
                           static_cast<const float*>(c), static_cast<float*>(out), G, s.m, s.n, p.M, p.N);
    else
        hipLaunchKernelGGL((crop<uint16_t>), dim3(flat_blocks(G * s.m * s.n, 256)), dim3(256), 0, st,
                           static_cast<const uint16_t*>(c), static_cast<uint16_t*>(out), G, s.m, s.n, p.M, p.N);
    return hipGetLastError();
}

hipError_t matmul_backward(const MatmulSpec& s, const void* a, const void* b, const void* dy, void* da, void* db,
                           void* workspace, int num_cus, hipStream_t st) {
    const int64_t G = s.batch.count;
    const size_t es = s.dtype == 0 ? 4 : 2;
    const MatmulBatch oa = operand_shape(s.batch, s.a_batch), obb = operand_shape(s.batch, s.b_batch);
    const MatmulBatch dyb = packed_batch(s.batch, s.m * s.n);
    hipError_t e;
    if (G * s.m * s.n == 0) {  // no output elements: both gradients are zero
        if ((e = zero_fill(da, oa.count * s.m * s.k * static_cast<int64_t>(es), st)) != hipSuccess) return e;
        return zero_fill(db, obb.count * s.k * s.n * static_cast<int64_t>(es), st);
    }
    if (s.k == 0) return hipSuccess;  // dA [.., M, 0] and dB [.., 0, N] hold nothing
    void* c = nullptr;
    // dA[g] = dY[g] B[g]^T: X = dY [M, N], Y = B as [K, N]; then summed over A's broadcast batches
    {
        const Padded p = padded(s.dtype, s.m, s.k, s.n);
        const Gather x{dy, dyb, s.m, s.n, s.n, 0}, y{b, s.b_batch, s.k, s.n, s.n, 0};
        if ((e = product(s.dtype, G, x, y, p, true, workspace, &c, num_cus, st)) != hipSuccess) return e;
        reduce_any(s.dtype, static_cast<const float*>(c), da, s.batch, oa, s.m, s.k, p.M, p.N, st);
    }
    // dB[g] = A[g]^T dY[g]: X = A^T [K, M], Y = dY^T [N, M]; then summed over B's broadcast batches
    {
        const Padded p = padded(s.dtype, s.k, s.n, s.m);
        const Gather x{a, s.a_batch, s.k, s.m, s.k, 1}, y{dy, dyb, s.n, s.m, s.n, 1};
        if ((e = product(s.dtype, G, x, y, p, true, workspace, &c, num_cus, st)) != hipSuccess) return e;
        reduce_any(s.dtype, static_cast<const float*>(c), db, s.batch, obb, s.k, s.n, p.M, p.N, st);
    }
    return hipGetLastError();
}

}  // namespace hk
