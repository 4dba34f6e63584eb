// hk_softmax.hip — row softmax / log-softmax, forward and backward, for gfx950.
//
// Semantics (reference rust-ascend-compiler/src/ascend/row_programs.rs:135-143 and :152-163,
// driven by rust-ascend-driver/src/tensor/runtime/rows.rs:50-79 and wide_rows.rs:162-232):
//   softmax      m = max_j x_j;  e_j = exp(x_j - m);  s = sum_j e_j;  y_j = e_j / s
//   log_softmax  y_j = (x_j - m) - log(s)
//   backward     softmax:      dot = sum_j y_j dy_j;  dx_j = y_j (dy_j - dot)
//                log_softmax:  dot = sum_j dy_j;      dx_j = dy_j - exp(y_j) dot
// over the last axis of a contiguous FP32 tensor (any positive width; the reference runs
// widths of 32..4096 in multiples of 32 as one row program and tiles the others).
//
// Layout: x/y/dy/dx [rows, W] row-major F32. HBM-bound: the forward moves 8 bytes per element,
// the backward 12.
//
// Fast path (W % 4 == 0, W <= 4096, 16-byte aligned): one wavefront owns one row; lane l holds
// the float4 chunks l, l+64, ... of the row in registers, so the row is read once, and row
// maxima and sums are butterfly reductions across the wave. Wide path (W % 4 == 0,
// 4096 < W <= 32768, aligned; vocabulary-sized rows): one 1024-thread workgroup owns one row,
// thread t holding the float4 chunks t, t+1024, ... in registers, so the row is again read once
// (non-temporal: these working sets exceed the on-package cache), with wave then workgroup
// reductions. General path: one workgroup per row, the row re-read from cache for each pass,
// reductions through LDS.
#include "hk_common.hpp"
#include "hk_kernels.hpp"

#include <initializer_list>

namespace hk {

namespace {

constexpr int kFastThreads = 256;  // 4 rows per workgroup on the fast path
constexpr int kRowThreads = 256;   // one row per workgroup on the general path
constexpr int kWideThreads = 1024; // one row per workgroup on the wide path
constexpr int kWideMaxWidth = kWideThreads * 4 * 8;  // 8 float4 chunks per thread

template <int MAXJ>
__device__ __forceinline__ void load_row4(const float* rowp, int lane, int chunks, f32x4_t (&v)[MAXJ]) {
#pragma unroll
    for (int j = 0; j < MAXJ; ++j) {
        const int c = lane + 64 * j;
        v[j] = c < chunks ? *reinterpret_cast<const f32x4_t*>(rowp + 4 * c) : f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
}

template <int MAXJ, bool LOG>
__global__ void __launch_bounds__(kFastThreads)
softmax_fwd_fast(const float* __restrict__ x, float* __restrict__ y, int64_t rows, int width) {
    const int lane = threadIdx.x & 63;
    for (int64_t row = static_cast<int64_t>(blockIdx.x) * (kFastThreads / 64) + (threadIdx.x >> 6); row < rows;
         row += static_cast<int64_t>(gridDim.x) * (kFastThreads / 64)) {
        const int chunks = width >> 2;
        f32x4_t v[MAXJ];
        load_row4<MAXJ>(x + row * width, lane, chunks, v);
        float m = -INFINITY;
#pragma unroll
        for (int j = 0; j < MAXJ; ++j)
            if (lane + 64 * j < chunks)
#pragma unroll
                for (int e = 0; e < 4; ++e) m = fmaxf(m, v[j][e]);
        m = wave_max(m);
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < MAXJ; ++j)
            if (lane + 64 * j < chunks)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float ex = expf(v[j][e] - m);
                    s += ex;
                    if (!LOG) v[j][e] = ex;
                }
        s = wave_sum(s);
        float* yr = y + row * width;
        if (LOG) {
            const float ls = logf(s);
#pragma unroll
            for (int j = 0; j < MAXJ; ++j) {
                const int c = lane + 64 * j;
                if (c < chunks) {
                    f32x4_t o;
#pragma unroll
                    for (int e = 0; e < 4; ++e) o[e] = (v[j][e] - m) - ls;
                    *reinterpret_cast<f32x4_t*>(yr + 4 * c) = o;
                }
            }
        } else {
            const float inv = 1.0f / s;
#pragma unroll
            for (int j = 0; j < MAXJ; ++j) {
                const int c = lane + 64 * j;
                if (c < chunks) {
                    f32x4_t o;
#pragma unroll
                    for (int e = 0; e < 4; ++e) o[e] = v[j][e] * inv;
                    *reinterpret_cast<f32x4_t*>(yr + 4 * c) = o;
                }
            }
        }
    }
}

template <int MAXJ, bool LOG>
__global__ void __launch_bounds__(kFastThreads)
softmax_bwd_fast(const float* __restrict__ y, const float* __restrict__ dy, float* __restrict__ dx,
                 int64_t rows, int width) {
    const int lane = threadIdx.x & 63;
    for (int64_t row = static_cast<int64_t>(blockIdx.x) * (kFastThreads / 64) + (threadIdx.x >> 6); row < rows;
         row += static_cast<int64_t>(gridDim.x) * (kFastThreads / 64)) {
        const int chunks = width >> 2;
        f32x4_t yv[MAXJ], gv[MAXJ];
        load_row4<MAXJ>(y + row * width, lane, chunks, yv);
        load_row4<MAXJ>(dy + row * width, lane, chunks, gv);
        float dot = 0.0f;
#pragma unroll
        for (int j = 0; j < MAXJ; ++j)
            if (lane + 64 * j < chunks)
#pragma unroll
                for (int e = 0; e < 4; ++e) dot += LOG ? gv[j][e] : yv[j][e] * gv[j][e];
        dot = wave_sum(dot);
        float* dr = dx + row * width;
#pragma unroll
        for (int j = 0; j < MAXJ; ++j) {
            const int c = lane + 64 * j;
            if (c < chunks) {
                f32x4_t o;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    o[e] = LOG ? gv[j][e] - expf(yv[j][e]) * dot : yv[j][e] * (gv[j][e] - dot);
                *reinterpret_cast<f32x4_t*>(dr + 4 * c) = o;
            }
        }
    }
}

// Workgroup-wide reduction through LDS (wave results combined in wave order).
template <bool MAX, int NT = kRowThreads>
__device__ __forceinline__ float block_reduce(float v, float* scratch) {
    v = MAX ? wave_max(v) : wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float r = scratch[0];
#pragma unroll
    for (int i = 1; i < NT / 64; ++i) r = MAX ? fmaxf(r, scratch[i]) : r + scratch[i];
    __syncthreads();  // scratch is reused by the next reduction
    return r;
}

// chunks past the row's end read as `pad`
template <int MAXJ>
__device__ __forceinline__ void load_row_wide(const float* rowp, int chunks, f32x4_t (&v)[MAXJ], float pad = 0.0f) {
#pragma unroll
    for (int j = 0; j < MAXJ; ++j) {
        const int c = threadIdx.x + kWideThreads * j;
        v[j] = c < chunks ? stream_load(reinterpret_cast<const f32x4_t*>(rowp) + c) : f32x4_t{pad, pad, pad, pad};
    }
}

// At most 64 VGPRs (8 waves per SIMD), so two rows' workgroups share a CU and one streams
// while the other waits in its reductions.
template <int MAXJ, bool LOG>
__global__ void __launch_bounds__(kWideThreads) __attribute__((amdgpu_waves_per_eu(8)))
softmax_fwd_wide(const float* __restrict__ x, float* __restrict__ y, int64_t rows, int width) {
    __shared__ float scratch[kWideThreads / 64];
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {  // uniform per workgroup
        const int chunks = width >> 2;
        // chunks past the end hold -inf: they leave the maximum alone and add exp(-inf) = 0
        f32x4_t v[MAXJ];
        load_row_wide<MAXJ>(x + row * width, chunks, v, -INFINITY);
        float m = -INFINITY;
#pragma unroll
        for (int j = 0; j < MAXJ; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) m = fmaxf(m, v[j][e]);
        m = block_reduce<true, kWideThreads>(m, scratch);
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < MAXJ; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float ex = expf(v[j][e] - m);
                s += ex;
                if (!LOG) v[j][e] = ex;
            }
        s = block_reduce<false, kWideThreads>(s, scratch);
        f32x4_t* yr = reinterpret_cast<f32x4_t*>(y + row * width);
        const float ls = LOG ? logf(s) : 0.0f, inv = LOG ? 0.0f : 1.0f / s;
#pragma unroll
        for (int j = 0; j < MAXJ; ++j) {
            const int c = threadIdx.x + kWideThreads * j;
            if (c < chunks) {
                f32x4_t o;
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = LOG ? (v[j][e] - m) - ls : v[j][e] * inv;
                stream_store(o, yr + c);
            }
        }
    }
}

template <int MAXJ, bool LOG>
__global__ void __launch_bounds__(kWideThreads)
softmax_bwd_wide(const float* __restrict__ y, const float* __restrict__ dy, float* __restrict__ dx, int64_t rows, int width) {
    __shared__ float scratch[kWideThreads / 64];
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {  // uniform per workgroup
        const int chunks = width >> 2;
        f32x4_t yv[MAXJ], gv[MAXJ];
        load_row_wide<MAXJ>(y + row * width, chunks, yv);
        load_row_wide<MAXJ>(dy + row * width, chunks, gv);
        float dot = 0.0f;
#pragma unroll
        for (int j = 0; j < MAXJ; ++j)
            if (static_cast<int>(threadIdx.x) + kWideThreads * j < chunks)
#pragma unroll
                for (int e = 0; e < 4; ++e) dot += LOG ? gv[j][e] : yv[j][e] * gv[j][e];
        dot = block_reduce<false, kWideThreads>(dot, scratch);
        f32x4_t* dr = reinterpret_cast<f32x4_t*>(dx + row * width);
#pragma unroll
        for (int j = 0; j < MAXJ; ++j) {
            const int c = threadIdx.x + kWideThreads * j;
            if (c < chunks) {
                f32x4_t o;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    o[e] = LOG ? gv[j][e] - expf(yv[j][e]) * dot : yv[j][e] * (gv[j][e] - dot);
                stream_store(o, dr + c);
            }
        }
    }
}

template <bool LOG>
__global__ void __launch_bounds__(kRowThreads)
softmax_fwd_general(const float* __restrict__ x, float* __restrict__ y, int64_t rows, int64_t width) {
    __shared__ float scratch[kRowThreads / 64];
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {  // uniform per workgroup
        const float* xr = x + row * width;
        float* yr = y + row * width;
        float m = -INFINITY;
        for (int64_t c = threadIdx.x; c < width; c += kRowThreads) m = fmaxf(m, xr[c]);
        m = block_reduce<true>(m, scratch);
        float s = 0.0f;
        for (int64_t c = threadIdx.x; c < width; c += kRowThreads) s += expf(xr[c] - m);
        s = block_reduce<false>(s, scratch);
        if (LOG) {
            const float ls = logf(s);
            for (int64_t c = threadIdx.x; c < width; c += kRowThreads) yr[c] = (xr[c] - m) - ls;
        } else {
            const float inv = 1.0f / s;
            for (int64_t c = threadIdx.x; c < width; c += kRowThreads) yr[c] = expf(xr[c] - m) * inv;
        }
    }
}

template <bool LOG>
__global__ void __launch_bounds__(kRowThreads)
softmax_bwd_general(const float* __restrict__ y, const float* __restrict__ dy, float* __restrict__ dx,
                    int64_t rows, int64_t width) {
    __shared__ float scratch[kRowThreads / 64];
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {  // uniform per workgroup
        const float* yr = y + row * width;
        const float* gr = dy + row * width;
        float* dr = dx + row * width;
        float dot = 0.0f;
        for (int64_t c = threadIdx.x; c < width; c += kRowThreads) dot += LOG ? gr[c] : yr[c] * gr[c];
        dot = block_reduce<false>(dot, scratch);
        for (int64_t c = threadIdx.x; c < width; c += kRowThreads)
            dr[c] = LOG ? gr[c] - expf(yr[c]) * dot : yr[c] * (gr[c] - dot);
    }
}

bool aligned16(std::initializer_list<const void*> ptrs) {
    for (const void* p : ptrs)
        if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return false;
    return true;
}

bool fast_softmax(int64_t width, std::initializer_list<const void*> ptrs) {
    return width % 4 == 0 && width <= 4096 && aligned16(ptrs);
}

bool wide_softmax(int64_t width, std::initializer_list<const void*> ptrs) {
    return width % 4 == 0 && width > 4096 && width <= kWideMaxWidth && aligned16(ptrs);
}

// float4 chunks per thread of the wide path: 2, 4 or 8
int wide_per_thread(int64_t width) {
    const int64_t per = (width / 4 + kWideThreads - 1) / kWideThreads;
    return per <= 2 ? 2 : (per <= 4 ? 4 : 8);
}

template <bool LOG>
void launch_fwd(const float* x, float* y, int64_t rows, int64_t width, hipStream_t s) {
    if (fast_softmax(width, {x, y})) {
        const dim3 grid(flat_blocks(rows, 4));
        const int per_lane = static_cast<int>((width / 4 + 63) / 64);
        const int w = static_cast<int>(width);
        if (per_lane <= 1) hipLaunchKernelGGL((softmax_fwd_fast<1, LOG>), grid, dim3(kFastThreads), 0, s, x, y, rows, w);
        else if (per_lane <= 2) hipLaunchKernelGGL((softmax_fwd_fast<2, LOG>), grid, dim3(kFastThreads), 0, s, x, y, rows, w);
        else if (per_lane <= 4) hipLaunchKernelGGL((softmax_fwd_fast<4, LOG>), grid, dim3(kFastThreads), 0, s, x, y, rows, w);
        else if (per_lane <= 8) hipLaunchKernelGGL((softmax_fwd_fast<8, LOG>), grid, dim3(kFastThreads), 0, s, x, y, rows, w);
        else hipLaunchKernelGGL((softmax_fwd_fast<16, LOG>), grid, dim3(kFastThreads), 0, s, x, y, rows, w);
    } else if (wide_softmax(width, {x, y})) {
        const dim3 grid(flat_blocks(rows, 1));
        const int w = static_cast<int>(width);
        switch (wide_per_thread(width)) {
            case 2: hipLaunchKernelGGL((softmax_fwd_wide<2, LOG>), grid, dim3(kWideThreads), 0, s, x, y, rows, w); break;
            case 4: hipLaunchKernelGGL((softmax_fwd_wide<4, LOG>), grid, dim3(kWideThreads), 0, s, x, y, rows, w); break;
            default: hipLaunchKernelGGL((softmax_fwd_wide<8, LOG>), grid, dim3(kWideThreads), 0, s, x, y, rows, w); break;
        }
    } else {
        hipLaunchKernelGGL((softmax_fwd_general<LOG>), dim3(flat_blocks(rows, 1)), dim3(kRowThreads), 0, s, x, y,
                           rows, width);
    }
}

template <bool LOG>
void launch_bwd(const float* y, const float* dy, float* dx, int64_t rows, int64_t width, hipStream_t s) {
    if (fast_softmax(width, {y, dy, dx})) {
        const dim3 grid(flat_blocks(rows, 4));
        const int per_lane = static_cast<int>((width / 4 + 63) / 64);
        const int w = static_cast<int>(width);
        if (per_lane <= 1) hipLaunchKernelGGL((softmax_bwd_fast<1, LOG>), grid, dim3(kFastThreads), 0, s, y, dy, dx, rows, w);
        else if (per_lane <= 2) hipLaunchKernelGGL((softmax_bwd_fast<2, LOG>), grid, dim3(kFastThreads), 0, s, y, dy, dx, rows, w);
        else if (per_lane <= 4) hipLaunchKernelGGL((softmax_bwd_fast<4, LOG>), grid, dim3(kFastThreads), 0, s, y, dy, dx, rows, w);
        else if (per_lane <= 8) hipLaunchKernelGGL((softmax_bwd_fast<8, LOG>), grid, dim3(kFastThreads), 0, s, y, dy, dx, rows, w);
        else hipLaunchKernelGGL((softmax_bwd_fast<16, LOG>), grid, dim3(kFastThreads), 0, s, y, dy, dx, rows, w);
    } else if (wide_softmax(width, {y, dy, dx})) {
        const dim3 grid(flat_blocks(rows, 1));
        const int w = static_cast<int>(width);
        switch (wide_per_thread(width)) {
            case 2: hipLaunchKernelGGL((softmax_bwd_wide<2, LOG>), grid, dim3(kWideThreads), 0, s, y, dy, dx, rows, w); break;
            case 4: hipLaunchKernelGGL((softmax_bwd_wide<4, LOG>), grid, dim3(kWideThreads), 0, s, y, dy, dx, rows, w); break;
            default: hipLaunchKernelGGL((softmax_bwd_wide<8, LOG>), grid, dim3(kWideThreads), 0, s, y, dy, dx, rows, w); break;
        }
    } else {
        hipLaunchKernelGGL((softmax_bwd_general<LOG>), dim3(flat_blocks(rows, 1)), dim3(kRowThreads), 0, s, y, dy,
                           dx, rows, width);
    }
}

}  // namespace

hipError_t softmax_forward(const float* x, float* y, int64_t rows, int64_t width, int logarithmic, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    if (logarithmic) launch_fwd<true>(x, y, rows, width, s);
    else launch_fwd<false>(x, y, rows, width, s);
    return hipGetLastError();
}

hipError_t softmax_backward(const float* y, const float* dy, float* dx, int64_t rows, int64_t width, int logarithmic,
                            hipStream_t s) {
    if (rows == 0) return hipSuccess;
    if (logarithmic) launch_bwd<true>(y, dy, dx, rows, width, s);
    else launch_bwd<false>(y, dy, dx, rows, width, s);
    return hipGetLastError();
}

}  // namespace hk
