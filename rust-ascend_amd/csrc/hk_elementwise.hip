// hk_elementwise.hip — the SwiGLU gate: SiLU(gate) * up and its backward, for gfx950.
//
// Semantics (reference rust-ascend-compiler/src/ascend/programs.rs:21-46, MapProgram::SiluMul and
// SiluMulBackward, driven by rust-ascend-driver/src/tensor/runtime/elementwise.rs:13-30), in the
// reference's order of operations:
//   s = 1 / (1 + exp(-x));  h = x * s;  y = h * up
//   ds = s * (1 + x * (1 - s));  dgate = (dy * up) * ds;  dup = dy * h
// over contiguous tensors of one shape, F32 (the reference's dtype) or BF16 storage with F32
// arithmetic.
//
// Layout: element-wise over n elements. HBM-bound: the forward moves 3 values per element, the
// backward 5. Each thread handles one 16-byte chunk per tensor (4 F32 or 8 BF16 values) with
// vector loads; a ragged tail (n not a multiple of the chunk) and tensors not 16-byte aligned are
// handled element by element.
#include "hk_common.hpp"
#include "hk_kernels.hpp"

#include <initializer_list>

namespace hk {

namespace {

constexpr int kEwThreads = 256;

__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

__device__ __forceinline__ float silu_mul1(float g, float u) {
    const float s = sigmoid(g);
    return (g * s) * u;
}

__device__ __forceinline__ void silu_mul_bwd1(float g, float u, float dy, float& dg, float& du) {
    const float s = sigmoid(g);
    const float h = g * s;
    const float ds = s * (1.0f + g * (1.0f - s));
    dg = (dy * u) * ds;
    du = dy * h;
}

// Chunks of 16 bytes: kPer values of T.
template <typename T> struct Chunk;
template <> struct Chunk<float> {
    static constexpr int kPer = 4;
    __device__ static void load(const float* p, float (&v)[4]) {
        const f32x4_t w = *reinterpret_cast<const f32x4_t*>(p);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = w[i];
    }
    __device__ static void store(float* p, const float (&v)[4]) {
        *reinterpret_cast<f32x4_t*>(p) = f32x4_t{v[0], v[1], v[2], v[3]};
    }
};
template <> struct Chunk<uint16_t> {
    static constexpr int kPer = 8;
    __device__ static void load(const uint16_t* p, float (&v)[8]) { load8(p, v); }
    __device__ static void store(uint16_t* p, const float (&v)[8]) { store8(p, v); }
};

template <typename T>
__global__ void __launch_bounds__(kEwThreads)
silu_mul_kernel(const T* __restrict__ g, const T* __restrict__ u, T* __restrict__ y, int64_t n, bool vec) {
    constexpr int P = Chunk<T>::kPer;
    const int64_t c = static_cast<int64_t>(blockIdx.x) * kEwThreads + threadIdx.x;
    const int64_t i0 = c * P;
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

template <typename T>
__global__ void __launch_bounds__(kEwThreads)
silu_mul_bwd_kernel(const T* __restrict__ g, const T* __restrict__ u, const T* __restrict__ dy,
                    T* __restrict__ dg, T* __restrict__ du, int64_t n, bool vec) {
    constexpr int P = Chunk<T>::kPer;
    const int64_t c = static_cast<int64_t>(blockIdx.x) * kEwThreads + threadIdx.x;
    const int64_t i0 = c * P;
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

template <typename T>
unsigned grid_for(int64_t n) {
    constexpr int P = Chunk<T>::kPer;
    const int64_t chunks = (n + P - 1) / P;
    return static_cast<unsigned>((chunks + kEwThreads - 1) / kEwThreads);
}

bool aligned16(std::initializer_list<const void*> ptrs) {
    for (const void* p : ptrs)
        if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return false;
    return true;
}

}  // namespace

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

}  // namespace hk
