// hk_elementwise.hip — element-wise kernels for gfx950: the SwiGLU gate SiLU(gate) * up and its
// backward, the last-axis bias add with an optional residual, and the bias gradient's column sum.
//
// SwiGLU semantics (reference rust-ascend-compiler/src/ascend/programs.rs:21-46, MapProgram::SiluMul
// and SiluMulBackward, driven by rust-ascend-driver/src/tensor/runtime/elementwise.rs:13-30), in
// the reference's order of operations:
//   s = 1 / (1 + exp(-x));  h = x * s;  y = h * up
//   ds = s * (1 + x * (1 - s));  dgate = (dy * up) * ds;  dup = dy * h
// over contiguous tensors of one shape, F32 (the reference's dtype) or BF16 storage with F32
// arithmetic.
//
// Bias add (reference src/nn/affine.rs:17-25, runtime/affine.rs:10-22): y = (x + residual) + b[c]
// in that F32 order. Its backward sums dY over rows in the reference's pairwise order
// (runtime/normalization.rs:95-114): each level adds row i and row i + floor(r/2) and carries an
// odd last row, so dbias is bit-identical to the reference's.
//
// Layout: element-wise over n elements, HBM-bound (forward SwiGLU 3 values per element, backward
// 5, bias add 2 or 3). Each thread handles one 16-byte chunk per tensor (4 F32 or 8 BF16 values)
// with vector loads; a ragged tail and tensors not 16-byte aligned take the element path.
#include "hk_common.hpp"
#include "hk_kernels.hpp"

namespace hk {

namespace {

constexpr int kEwThreads = 256;

template <typename T>
__global__ void __launch_bounds__(kEwThreads)
silu_mul_kernel(const T* __restrict__ g, const T* __restrict__ u, T* __restrict__ y, int64_t n, bool vec) {
    constexpr int P = Chunk<T>::kPer;
    for (int64_t i0 = flat_begin(kEwThreads) * P; i0 < n; i0 += flat_stride(kEwThreads) * P) {
        if (vec && i0 + P <= n) {
            float gv[P], uv[P], o[P];
            Chunk<T>::load(g + i0, gv);
            Chunk<T>::load(u + i0, uv);
#pragma unroll
            for (int e = 0; e < P; ++e) o[e] = silu_mul1(gv[e], uv[e]);
            Chunk<T>::store(y + i0, o);
        } else {
            for (int64_t i = i0; i < n && i < i0 + P; ++i)
                Elem<T>::store(y, i, silu_mul1(Elem<T>::load(g, i), Elem<T>::load(u, i)));
        }
    }
}

template <typename T>
__global__ void __launch_bounds__(kEwThreads)
silu_mul_bwd_kernel(const T* __restrict__ g, const T* __restrict__ u, const T* __restrict__ dy,
                    T* __restrict__ dg, T* __restrict__ du, int64_t n, bool vec) {
    constexpr int P = Chunk<T>::kPer;
    for (int64_t i0 = flat_begin(kEwThreads) * P; i0 < n; i0 += flat_stride(kEwThreads) * P) {
        if (vec && i0 + P <= n) {
            float gv[P], uv[P], dv[P], og[P], ou[P];
            Chunk<T>::load(g + i0, gv);
            Chunk<T>::load(u + i0, uv);
            Chunk<T>::load(dy + i0, dv);
#pragma unroll
            for (int e = 0; e < P; ++e) silu_mul_bwd1(gv[e], uv[e], dv[e], og[e], ou[e]);
            Chunk<T>::store(dg + i0, og);
            Chunk<T>::store(du + i0, ou);
        } else {
            for (int64_t i = i0; i < n && i < i0 + P; ++i) {
                float a, b;
                silu_mul_bwd1(Elem<T>::load(g, i), Elem<T>::load(u, i), Elem<T>::load(dy, i), a, b);
                Elem<T>::store(dg, i, a);
                Elem<T>::store(du, i, b);
            }
        }
    }
}

// y = (x + r) + b[i % width] (b may be null: y = x + r); with vec, width % P == 0 so a chunk
// never crosses a row and its bias slice b[c .. c+P) is 16-byte aligned.
template <typename T, bool RES>
__global__ void __launch_bounds__(kEwThreads)
bias_add_kernel(const T* __restrict__ x, const float* __restrict__ b, const T* __restrict__ r, T* __restrict__ y,
                int64_t n, int64_t width, bool vec) {
    constexpr int P = Chunk<T>::kPer;
    for (int64_t i0 = flat_begin(kEwThreads) * P; i0 < n; i0 += flat_stride(kEwThreads) * P) {
        if (vec && i0 + P <= n) {
            float xv[P], rv[P], bv[P], o[P];
            Chunk<T>::load(x + i0, xv);
            if (RES) Chunk<T>::load(r + i0, rv);
            if (b) {
                const float* bp = b + i0 % width;
#pragma unroll
                for (int q = 0; q < P / 4; ++q) {
                    const f32x4_t w = *reinterpret_cast<const f32x4_t*>(bp + 4 * q);
#pragma unroll
                    for (int e = 0; e < 4; ++e) bv[4 * q + e] = w[e];
                }
            }
#pragma unroll
            for (int e = 0; e < P; ++e) {
                const float sum = RES ? xv[e] + rv[e] : xv[e];
                o[e] = b ? sum + bv[e] : sum;
            }
            Chunk<T>::store(y + i0, o);
        } else {
            for (int64_t i = i0; i < n && i < i0 + P; ++i) {
                const float s = RES ? Elem<T>::load(x, i) + Elem<T>::load(r, i) : Elem<T>::load(x, i);
                Elem<T>::store(y, i, b ? s + b[i % width] : s);
            }
        }
    }
}

// Value of row i after D pairwise levels over a [rows, width] buffer: level l has
// ceil(rows / 2^l) rows; below floor(r/2) a row is the sum of rows i and i + floor(r/2) of the level
// before, and an odd level's last row is carried.
template <int D>
__device__ __forceinline__ float fold_eval(const float* __restrict__ v, int64_t rows, int64_t width, int64_t i,
                                           int64_t c) {
    if constexpr (D == 0) {
        return v[i * width + c];
    } else {
        const int64_t r = (rows + (int64_t(1) << (D - 1)) - 1) >> (D - 1);
        const int64_t p = r >> 1;
        if (i < p) return fold_eval<D - 1>(v, rows, width, i, c) + fold_eval<D - 1>(v, rows, width, i + p, c);
        return fold_eval<D - 1>(v, rows, width, r - 1, c);
    }
}

template <int D>
__global__ void __launch_bounds__(kEwThreads)
fold_rows_kernel(const float* __restrict__ v, float* __restrict__ out, int64_t rows, int64_t width) {
    const int64_t out_rows = (rows + (int64_t(1) << D) - 1) >> D;
    for (int64_t idx = flat_begin(kEwThreads); idx < out_rows * width; idx += flat_stride(kEwThreads))
        out[idx] = fold_eval<D>(v, rows, width, idx / width, idx % width);
}

__global__ void __launch_bounds__(kEwThreads) zero_f32_kernel(float* __restrict__ p, int64_t n) {
    for (int64_t i = flat_begin(kEwThreads); i < n; i += flat_stride(kEwThreads)) p[i] = 0.0f;
}

unsigned blocks_for(int64_t work) { return flat_blocks(work, kEwThreads); }

template <typename T>
unsigned grid_for(int64_t n) {
    constexpr int P = Chunk<T>::kPer;
    return blocks_for((n + P - 1) / P);
}

constexpr int kFoldLevels = 5;  // pairwise levels per launch (32 rows read per output)

// Attention scores of the composed (materialized) path, in place: s = s * scale, then + mask
// when a mask is given (two F32 roundings, the reference's `scores * scale + mask` of
// src/nn/attention.rs:25-26).
__global__ void __launch_bounds__(kEwThreads)
scale_mask_kernel(float* __restrict__ s, const float* __restrict__ mask, float scale, int64_t n) {
    for (int64_t i = flat_begin(kEwThreads); i < n; i += flat_stride(kEwThreads)) {
        const float v = s[i] * scale;
        s[i] = mask ? v + mask[i] : v;
    }
}

// out = bf16(scale * x): the gradient of `scores * scale` rounded to BF16 as the score GEMM's
// backward rounds its upstream gradient (matmul_bf16_fp32's backward).
__global__ void __launch_bounds__(kEwThreads)
scale_to_bf16_kernel(const float* __restrict__ x, float scale, uint16_t* __restrict__ out, int64_t n) {
    for (int64_t i = flat_begin(kEwThreads); i < n; i += flat_stride(kEwThreads)) out[i] = f32_to_bf16(x[i] * scale);
}

}  // namespace

hipError_t scale_mask(float* scores, const float* mask, float scale, int64_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(scale_mask_kernel, dim3(blocks_for(n)), dim3(kEwThreads), 0, s, scores, mask, scale, n);
    return hipGetLastError();
}

hipError_t scale_to_bf16(const float* x, float scale, void* out, int64_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(scale_to_bf16_kernel, dim3(blocks_for(n)), dim3(kEwThreads), 0, s, x, scale,
                       static_cast<uint16_t*>(out), n);
    return hipGetLastError();
}

hipError_t silu_mul(int dtype_bf16, const void* gate, const void* up, void* y, int64_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const bool vec = aligned16({gate, up, y});  // otherwise every thread takes the element path
    if (dtype_bf16)
        hipLaunchKernelGGL(silu_mul_kernel<uint16_t>, dim3(grid_for<uint16_t>(n)), dim3(kEwThreads), 0, s,
                           static_cast<const uint16_t*>(gate), static_cast<const uint16_t*>(up),
                           static_cast<uint16_t*>(y), n, vec);
    else
        hipLaunchKernelGGL(silu_mul_kernel<float>, dim3(grid_for<float>(n)), dim3(kEwThreads), 0, s,
                           static_cast<const float*>(gate), static_cast<const float*>(up), static_cast<float*>(y),
                           n, vec);
    return hipGetLastError();
}

hipError_t silu_mul_backward(int dtype_bf16, const void* gate, const void* up, const void* dy, void* dgate,
                             void* dup, int64_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const bool vec = aligned16({gate, up, dy, dgate, dup});
    if (dtype_bf16)
        hipLaunchKernelGGL(silu_mul_bwd_kernel<uint16_t>, dim3(grid_for<uint16_t>(n)), dim3(kEwThreads), 0, s,
                           static_cast<const uint16_t*>(gate), static_cast<const uint16_t*>(up),
                           static_cast<const uint16_t*>(dy), static_cast<uint16_t*>(dgate),
                           static_cast<uint16_t*>(dup), n, vec);
    else
        hipLaunchKernelGGL(silu_mul_bwd_kernel<float>, dim3(grid_for<float>(n)), dim3(kEwThreads), 0, s,
                           static_cast<const float*>(gate), static_cast<const float*>(up),
                           static_cast<const float*>(dy), static_cast<float*>(dgate), static_cast<float*>(dup), n,
                           vec);
    return hipGetLastError();
}

template <typename T>
static hipError_t bias_add_t(const T* x, const float* b, const T* r, T* y, int64_t n, int64_t width, hipStream_t s) {
    constexpr int P = Chunk<T>::kPer;
    const bool vec = width % P == 0 && aligned16({x, b, r, y});
    if (r)
        hipLaunchKernelGGL((bias_add_kernel<T, true>), dim3(grid_for<T>(n)), dim3(kEwThreads), 0, s, x, b, r, y, n,
                           width, vec);
    else
        hipLaunchKernelGGL((bias_add_kernel<T, false>), dim3(grid_for<T>(n)), dim3(kEwThreads), 0, s, x, b, r, y, n,
                           width, vec);
    return hipGetLastError();
}

hipError_t bias_add(int dtype_bf16, const void* x, const float* bias, const void* residual, void* y, int64_t n,
                    int64_t width, hipStream_t s) {
    if (n == 0) return hipSuccess;
    if (dtype_bf16)
        return bias_add_t(static_cast<const uint16_t*>(x), bias, static_cast<const uint16_t*>(residual),
                          static_cast<uint16_t*>(y), n, width, s);
    return bias_add_t(static_cast<const float*>(x), bias, static_cast<const float*>(residual), static_cast<float*>(y),
                      n, width, s);
}

size_t column_sum_workspace_bytes(int64_t rows, int64_t width) {
    if (rows <= (int64_t(1) << kFoldLevels)) return 0;  // one launch writes the result directly
    const int64_t first = (rows + (int64_t(1) << kFoldLevels) - 1) >> kFoldLevels;
    return 2 * static_cast<size_t>(first * width) * sizeof(float);
}

hipError_t column_sum(const float* dy, float* out, int64_t rows, int64_t width, void* workspace, hipStream_t s) {
    if (width == 0) return hipSuccess;
    if (rows == 0) {
        hipLaunchKernelGGL(zero_f32_kernel, dim3(blocks_for(width)), dim3(kEwThreads), 0, s, out, width);
        return hipGetLastError();
    }
    float* buf[2] = {static_cast<float*>(workspace), nullptr};
    if (workspace) buf[1] = buf[0] + ((rows + (int64_t(1) << kFoldLevels) - 1) >> kFoldLevels) * width;
    const float* value = dy;
    int level = 0;
    do {
        int remaining = 0;  // pairwise levels left: ceil(log2(rows)), at least one launch for rows == 1
        while ((int64_t(1) << remaining) < rows) ++remaining;
        const int d = remaining < 1 ? 1 : (remaining < kFoldLevels ? remaining : kFoldLevels);
        const int64_t next_rows = (rows + (int64_t(1) << d) - 1) >> d;
        float* next = next_rows == 1 ? out : buf[level & 1];
        const unsigned grid = blocks_for(next_rows * width);
        switch (d) {
            case 1: hipLaunchKernelGGL(fold_rows_kernel<1>, dim3(grid), dim3(kEwThreads), 0, s, value, next, rows, width); break;
            case 2: hipLaunchKernelGGL(fold_rows_kernel<2>, dim3(grid), dim3(kEwThreads), 0, s, value, next, rows, width); break;
            case 3: hipLaunchKernelGGL(fold_rows_kernel<3>, dim3(grid), dim3(kEwThreads), 0, s, value, next, rows, width); break;
            case 4: hipLaunchKernelGGL(fold_rows_kernel<4>, dim3(grid), dim3(kEwThreads), 0, s, value, next, rows, width); break;
            default: hipLaunchKernelGGL(fold_rows_kernel<kFoldLevels>, dim3(grid), dim3(kEwThreads), 0, s, value, next, rows, width); break;
        }
        value = next;
        rows = next_rows;
        ++level;
    } while (rows > 1);
    return hipGetLastError();
}

}  // namespace hk
