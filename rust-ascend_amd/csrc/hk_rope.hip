// hk_rope.hip — table-driven rotary position encoding (RoPE) and F32<->BF16 casts.
//
// RoPE semantics (reference rust-ascend-compiler/src/ascend/rotary_programs.rs:47-156):
// the pair (a, b) is (2p, 2p+1) for Interleaved or (p, p+P/2) for SplitHalf;
//   forward   y_a = x_a*c - x_b*s,  y_b = x_b*c + x_a*s
//   backward  y_a = x_a*c + x_b*s,  y_b = x_b*c - x_a*s   (the transpose Jacobian)
// with c, s = cos/sin[table_row, p]. Columns >= P (prefix form) are copied bit-exactly.
// Table rows broadcast singleton leading axes (rotary_programs.rs:125-139); the full
// form uses same-row tables (table row = input row).
//
// Memory-bound: each thread owns V consecutive pairs of one row (V = 8: 16-byte BF16
// loads/stores for both halves in SplitHalf, one 32-byte span for Interleaved) and
// reads V cos and V sin values (F32).
#include "hk_common.hpp"
#include "hk_kernels.hpp"

namespace hk {

namespace {

template <typename T, int V>
__device__ __forceinline__ void load_v(const T* p, float (&v)[V]) {
    if constexpr (V == 8) {
        load8(p, v);
    } else {
#pragma unroll
        for (int i = 0; i < V; ++i) v[i] = Elem<T>::load(p, i);
    }
}
template <typename T, int V>
__device__ __forceinline__ void store_v(T* p, const float (&v)[V]) {
    if constexpr (V == 8) {
        store8(p, v);
    } else {
#pragma unroll
        for (int i = 0; i < V; ++i) Elem<T>::store(p, i, v[i]);
    }
}

__device__ __forceinline__ int64_t table_row(int64_t row, const RopeMap& map) {
    if (map.same_row) return row;
    int64_t rem = row, t = 0;
    for (int a = map.nlead - 1; a >= 0; --a) {
        const int64_t coord = rem % map.shape[a];
        rem /= map.shape[a];
        t += coord * map.tstride[a];
    }
    return t;
}

// One thread's V pairs p0 .. p0+V-1 of one row: xr, yr at the row's first element, t the offset
// of the pairs' first angle in the tables.
template <typename T, int V, int LAYOUT, bool BWD>
__device__ __forceinline__ void rope_chunk(const T* __restrict__ xr, T* __restrict__ yr, const float* __restrict__ cos_t,
                                           const float* __restrict__ sin_t, int64_t t, int64_t p0, int64_t half) {
        float c[V], s[V], a[V], b[V];
#pragma unroll
        for (int i = 0; i < V; ++i) {
            c[i] = cos_t[t + i];
            s[i] = sin_t[t + i];
        }
        if constexpr (LAYOUT == 1) {
            load_v<T, V>(xr + p0, a);
            load_v<T, V>(xr + half + p0, b);
        } else {
            float ab[2 * V];
            if constexpr (V == 8) {
                float lo[8], hi[8];
                load8(xr + 2 * p0, lo);
                load8(xr + 2 * p0 + 8, hi);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    ab[i] = lo[i];
                    ab[8 + i] = hi[i];
                }
            } else {
#pragma unroll
                for (int i = 0; i < 2 * V; ++i) ab[i] = Elem<T>::load(xr, 2 * p0 + i);
            }
#pragma unroll
            for (int i = 0; i < V; ++i) {
                a[i] = ab[2 * i];
                b[i] = ab[2 * i + 1];
            }
        }
        float ya[V], yb[V];
#pragma unroll
        for (int i = 0; i < V; ++i) rope_rotate<BWD>(a[i], b[i], c[i], s[i], ya[i], yb[i]);
        if constexpr (LAYOUT == 1) {
            store_v<T, V>(yr + p0, ya);
            store_v<T, V>(yr + half + p0, yb);
        } else {
            if constexpr (V == 8) {
                float lo[8], hi[8];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    lo[2 * i] = ya[i];
                    lo[2 * i + 1] = yb[i];
                    hi[2 * i] = ya[4 + i];
                    hi[2 * i + 1] = yb[4 + i];
                }
                store8(yr + 2 * p0, lo);
                store8(yr + 2 * p0 + 8, hi);
            } else {
#pragma unroll
                for (int i = 0; i < V; ++i) {
                    Elem<T>::store(yr, 2 * (p0 + i), ya[i]);
                    Elem<T>::store(yr, 2 * (p0 + i) + 1, yb[i]);
                }
            }
        }
}

// Any table map: work item idx is pair chunk idx % (half / V) of row idx / (half / V).
template <typename T, int V, int LAYOUT, bool BWD>
__global__ void __launch_bounds__(256)
rope_pairs(const T* __restrict__ x, const float* __restrict__ cos_t, const float* __restrict__ sin_t,
           T* __restrict__ y, int64_t rows, int64_t width, int64_t half, RopeMap map) {
    const int64_t per_row = half / V;
    for (int64_t idx = flat_begin(256); idx < rows * per_row; idx += flat_stride(256)) {
        const int64_t row = idx / per_row;
        const int64_t p0 = (idx - row * per_row) * V;
        rope_chunk<T, V, LAYOUT, BWD>(x + row * width, y + row * width, cos_t, sin_t, table_row(row, map) * half + p0,
                                      p0, half);
    }
}

// The common table maps without a division per work item: the table row is the input row
// (period 0) or the input row modulo `period` (tables broadcast over the leading axes outside a
// contiguous innermost run, e.g. [1, 1, S, P/2] for [B, H, S, P] inputs). 2^tpr_shift threads per
// row (half / 8, a power of two dividing 256), each the same 8 pairs of every row it visits; the
// table row advances with the row by a step taken modulo the period once. Same arithmetic per
// pair as rope_pairs, so the results are bit-identical.
template <typename T, int LAYOUT, bool BWD>
__global__ void __launch_bounds__(256)
rope_rows(const T* __restrict__ x, const float* __restrict__ cos_t, const float* __restrict__ sin_t,
          T* __restrict__ y, int rows, int width, int half, int tpr_shift, int period) {
    const int rb = 256 >> tpr_shift;  // rows per workgroup pass
    const int p0 = (static_cast<int>(threadIdx.x) & ((1 << tpr_shift) - 1)) * 8;
    const int step = static_cast<int>(gridDim.x) * rb;
    int row = static_cast<int>(blockIdx.x) * rb + (static_cast<int>(threadIdx.x) >> tpr_shift);
    int t = period ? row % period : row;
    const int tstep = period ? step % period : step;
    for (; row < rows; row += step) {
        const int64_t off = static_cast<int64_t>(row) * width;
        rope_chunk<T, 8, LAYOUT, BWD>(x + off, y + off, cos_t, sin_t, static_cast<int64_t>(t) * half + p0, p0, half);
        t += tstep;
        if (period && t >= period) t -= period;
    }
}

// 0: the table row is the input row; P > 0: the input row modulo P; -1: a general map.
int64_t table_period(const RopeMap& map) {
    if (map.same_row) return 0;
    int64_t acc = 1;
    int a = map.nlead - 1;
    for (; a >= 0; --a) {  // the innermost axes whose table strides are their row-major strides
        if (map.shape[a] == 1) continue;
        if (map.tstride[a] != acc) break;
        acc *= map.shape[a];
    }
    for (; a >= 0; --a)  // every other axis broadcast
        if (map.shape[a] != 1 && map.tstride[a] != 0) return -1;
    return acc;
}

// Columns [p, width) of every row, copied as raw bits.
template <typename T>
__global__ void __launch_bounds__(256)
copy_tail(const T* __restrict__ x, T* __restrict__ y, int64_t rows, int64_t width, int64_t p) {
    const int64_t tail = width - p;
    for (int64_t idx = flat_begin(256); idx < rows * tail; idx += flat_stride(256)) {
        const int64_t row = idx / tail;
        const int64_t col = p + (idx - row * tail);
        y[row * width + col] = x[row * width + col];
    }
}

template <typename T, int V, int LAYOUT>
void launch_pairs(bool bwd, const void* x, const float* c, const float* s, void* y, int64_t rows,
                  int64_t width, int64_t half, const RopeMap& map, hipStream_t st) {
    const int64_t n = rows * (half / V);
    const dim3 grid(flat_blocks(n, 256));
    if constexpr (V == 8) {
        const int64_t tpr = half / 8, period = table_period(map);
        if (period >= 0 && tpr >= 1 && tpr <= 256 && (tpr & (tpr - 1)) == 0 && rows * width < (int64_t{1} << 31)) {
            const int shift = __builtin_ctzll(static_cast<unsigned long long>(tpr));
            if (bwd)
                hipLaunchKernelGGL((rope_rows<T, LAYOUT, true>), grid, dim3(256), 0, st, static_cast<const T*>(x), c, s,
                                   static_cast<T*>(y), (int)rows, (int)width, (int)half, shift, (int)period);
            else
                hipLaunchKernelGGL((rope_rows<T, LAYOUT, false>), grid, dim3(256), 0, st, static_cast<const T*>(x), c,
                                   s, static_cast<T*>(y), (int)rows, (int)width, (int)half, shift, (int)period);
            return;
        }
    }
    if (bwd)
        hipLaunchKernelGGL((rope_pairs<T, V, LAYOUT, true>), grid, dim3(256), 0, st, static_cast<const T*>(x), c,
                           s, static_cast<T*>(y), rows, width, half, map);
    else
        hipLaunchKernelGGL((rope_pairs<T, V, LAYOUT, false>), grid, dim3(256), 0, st, static_cast<const T*>(x), c,
                           s, static_cast<T*>(y), rows, width, half, map);
}

template <typename T>
hipError_t rope_t(const void* x, const float* c, const float* s, void* y, int64_t rows, int64_t width,
                  int64_t p, int layout, bool bwd, const RopeMap& map, hipStream_t st) {
    const int64_t half = p / 2;
    if (rows == 0) return hipSuccess;
    // 8 pairs per thread when every row's pair spans are 16-byte aligned (the tables are
    // F32 with 8*4 = 32-byte spans, aligned when half % 8 == 0).
    const bool vec = (half % 8 == 0) && (width % 8 == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0) &&
                     (reinterpret_cast<uintptr_t>(y) % 16 == 0);
    if (layout == 0) {
        if (vec) launch_pairs<T, 8, 0>(bwd, x, c, s, y, rows, width, half, map, st);
        else launch_pairs<T, 1, 0>(bwd, x, c, s, y, rows, width, half, map, st);
    } else {
        if (vec) launch_pairs<T, 8, 1>(bwd, x, c, s, y, rows, width, half, map, st);
        else launch_pairs<T, 1, 1>(bwd, x, c, s, y, rows, width, half, map, st);
    }
    if (p < width) {
        const int64_t n = rows * (width - p);
        hipLaunchKernelGGL((copy_tail<T>), dim3(flat_blocks(n, 256)), dim3(256), 0, st,
                           static_cast<const T*>(x), static_cast<T*>(y), rows, width, p);
    }
    return hipGetLastError();
}

// Each work item converts 8 consecutive elements (grid-stride); `vec` (16-byte aligned bases) selects
// the vector loads/stores, otherwise element accesses.
__global__ void __launch_bounds__(256)
cast_f32_to_bf16(const float* __restrict__ in, uint16_t* __restrict__ out, int64_t n, int vec) {
    for (int64_t i = flat_begin(256) * 8; i < n; i += flat_stride(256) * 8) {
        if (vec && i + 8 <= n) {
            float v[8];
            load8(in + i, v);
            store8(out + i, v);
        } else {
            for (int64_t j = i; j < n && j < i + 8; ++j) out[j] = f32_to_bf16(in[j]);
        }
    }
}

__global__ void __launch_bounds__(256)
cast_bf16_to_f32(const uint16_t* __restrict__ in, float* __restrict__ out, int64_t n, int vec) {
    for (int64_t i = flat_begin(256) * 8; i < n; i += flat_stride(256) * 8) {
        if (vec && i + 8 <= n) {
            float v[8];
            load8(in + i, v);
            store8(out + i, v);
        } else {
            for (int64_t j = i; j < n && j < i + 8; ++j) out[j] = bf16_to_f32(in[j]);
        }
    }
}

}  // namespace

hipError_t rope_apply(int dtype_bf16, const void* x, const float* cos_t, const float* sin_t, void* y,
                      int64_t rows, int64_t width, int64_t p, int layout, int backward,
                      const RopeMap& map, hipStream_t s) {
    return dtype_bf16 ? rope_t<uint16_t>(x, cos_t, sin_t, y, rows, width, p, layout, backward != 0, map, s)
                      : rope_t<float>(x, cos_t, sin_t, y, rows, width, p, layout, backward != 0, map, s);
}

hipError_t cast_apply(int to_bf16, const void* in, void* out, int64_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const int64_t threads = (n + 7) / 8;
    const dim3 grid(flat_blocks(threads, 256));
    const int vec = (reinterpret_cast<uintptr_t>(in) % 16 == 0) && (reinterpret_cast<uintptr_t>(out) % 16 == 0);
    if (to_bf16)
        hipLaunchKernelGGL(cast_f32_to_bf16, grid, dim3(256), 0, s, static_cast<const float*>(in),
                           static_cast<uint16_t*>(out), n, vec);
    else
        hipLaunchKernelGGL(cast_bf16_to_f32, grid, dim3(256), 0, s, static_cast<const uint16_t*>(in),
                           static_cast<float*>(out), n, vec);
    return hipGetLastError();
}

}  // namespace hk
