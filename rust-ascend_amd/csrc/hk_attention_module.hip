// hk_attention_module.hip — the pieces of the backend's module-level attention that are not
// matmuls or softmax, for gfx950: the score transform and its gradient, the reduction of a
// broadcast bias gradient, and the materialized swap of the last two dims.
//
// Reference: RudaAscend's ModuleOps::attention (src/backend.rs:1323-1333) calls
// ruda_tensor::ops::attention::attention_fallback (the RUDA tensor library, git rev
// 126b1c78267267eb467c43e597f59f40f3d7c4f6, not vendored), which composes the backend's own float
// ops: scores = Q K^T * scale (K^T a swapped view materialized, src/backend.rs:133-140), an optional
// softcap s -> c tanh(s / c), an additive bias, -inf where the causal rule or the boolean mask
// (true = masked) excludes a key, softmax over the keys, then P V. The matmuls and the softmax run
// on hk_matmul.hip and hk_softmax.hip; this file transforms the F32 scores [B, H, Sq, Sk] in one
// pass (mask and bias broadcast over any of their dims of size 1).
#include "hk_common.hpp"
#include "hk_kernels.hpp"

namespace hk {

namespace {

struct ScoreDims {
    int64_t shape[4];        // B, H, Sq, Sk
    int64_t bias_stride[4];  // element strides of the bias over the four dims (0 = broadcast)
    int64_t mask_stride[4];
};

__device__ __forceinline__ void coords(const ScoreDims& d, int64_t i, int64_t (&c)[4]) {
    for (int k = 3; k >= 0; --k) {
        c[k] = i % d.shape[k];
        i /= d.shape[k];
    }
}

__device__ __forceinline__ int64_t offset(const int64_t (&c)[4], const int64_t (&st)[4]) {
    return c[0] * st[0] + c[1] * st[1] + c[2] * st[2] + c[3] * st[3];
}

// out = masked ? -inf : softcap(s * scale) + bias, softcap(x) = c tanh(x / c) when c > 0.
__global__ void __launch_bounds__(256)
scores_forward(const float* __restrict__ s, float* __restrict__ out, ScoreDims d, float scale, float softcap,
               const float* __restrict__ bias, const uint8_t* __restrict__ mask, int causal) {
    const int64_t n = d.shape[0] * d.shape[1] * d.shape[2] * d.shape[3];
    for (int64_t i = flat_begin(256); i < n; i += flat_stride(256)) {
        int64_t c[4];
        coords(d, i, c);
        const bool masked = (causal && c[3] > c[2]) || (mask && mask[offset(c, d.mask_stride)] != 0);
        float x = s[i] * scale;
        if (softcap > 0.0f) x = softcap * tanhf(x / softcap);
        if (bias) x += bias[offset(c, d.bias_stride)];
        out[i] = masked ? -__builtin_inff() : x;
    }
}

// ds = masked ? 0 : dout * scale * (1 - tanh^2(s * scale / c)) (the softcap's derivative, 1 without
// one); dbias_full (when given) = masked ? 0 : dout, over the full [B, H, Sq, Sk].
__global__ void __launch_bounds__(256)
scores_backward(const float* __restrict__ s, const float* __restrict__ dout, float* __restrict__ ds,
                float* __restrict__ dbias_full, ScoreDims d, float scale, float softcap, const uint8_t* __restrict__ mask,
                int causal) {
    const int64_t n = d.shape[0] * d.shape[1] * d.shape[2] * d.shape[3];
    for (int64_t i = flat_begin(256); i < n; i += flat_stride(256)) {
        int64_t c[4];
        coords(d, i, c);
        const bool masked = (causal && c[3] > c[2]) || (mask && mask[offset(c, d.mask_stride)] != 0);
        const float g = masked ? 0.0f : dout[i];
        float dx = g * scale;
        if (softcap > 0.0f) {
            const float t = tanhf(s[i] * scale / softcap);
            dx = g * (1.0f - t * t) * scale;
        }
        ds[i] = dx;
        if (dbias_full) dbias_full[i] = g;
    }
}

// out[j] = sum of full[i] over the elements i of the [B, H, Sq, Sk] grid that the bias element j
// broadcasts onto, in increasing i (fixed order); out_shape is the bias shape aligned to four dims.
__global__ void __launch_bounds__(256)
sum_to_shape(const float* __restrict__ full, float* __restrict__ out, ScoreDims d, ScoreDims o) {
    const int64_t n = o.shape[0] * o.shape[1] * o.shape[2] * o.shape[3];
    int64_t fstride[4], reps = 1;
    fstride[3] = 1;
    for (int k = 2; k >= 0; --k) fstride[k] = fstride[k + 1] * d.shape[k + 1];
    for (int k = 0; k < 4; ++k)
        if (o.shape[k] == 1) reps *= d.shape[k];
    for (int64_t j = flat_begin(256); j < n; j += flat_stride(256)) {
        int64_t c[4];
        coords(o, j, c);
        const int64_t base = offset(c, fstride);
        float sum = 0.0f;
        for (int64_t r = 0; r < reps; ++r) {
            int64_t i = base, q = r;
            for (int k = 3; k >= 0; --k)
                if (o.shape[k] == 1) {
                    i += (q % d.shape[k]) * fstride[k];
                    q /= d.shape[k];
                }
            sum += full[i];
        }
        out[j] = sum;
    }
}

// y[g][c][r] = x[g][r][c] for [G, R, C] x: 64x64 tiles through LDS (rows padded by one element),
// coalesced on both sides. T is the element's storage type (F32, or a 16-bit F16/BF16 word).
template <typename T>
__global__ void __launch_bounds__(256)
swap_last(const T* __restrict__ x, T* __restrict__ y, int64_t R, int64_t C, int64_t tiles_c) {
    __shared__ T tile[64][65];
    const int64_t g = blockIdx.z;
    const int64_t r0 = (blockIdx.x / tiles_c) * 64, c0 = (blockIdx.x % tiles_c) * 64;
    const T* src = x + g * R * C;
    T* dst = y + g * R * C;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int i = ty; i < 64; i += 4) {
        const int64_t r = r0 + i, c = c0 + tx;
        if (r < R && c < C) tile[i][tx] = src[r * C + c];
    }
    __syncthreads();
    for (int i = ty; i < 64; i += 4) {
        const int64_t c = c0 + i, r = r0 + tx;
        if (r < R && c < C) dst[c * R + r] = tile[tx][i];
    }
}

ScoreDims dims_of(const AttnScoreSpec& sp) {
    ScoreDims d{};
    for (int k = 0; k < 4; ++k) {
        d.shape[k] = sp.shape[k];
        d.bias_stride[k] = sp.bias_stride[k];
        d.mask_stride[k] = sp.mask_stride[k];
    }
    return d;
}

}  // namespace

hipError_t attention_scores(const AttnScoreSpec& sp, const float* s, float* out, const float* bias,
                            const uint8_t* mask, hipStream_t st) {
    const int64_t n = sp.shape[0] * sp.shape[1] * sp.shape[2] * sp.shape[3];
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(scores_forward, dim3(flat_blocks(n, 256)), dim3(256), 0, st, s, out, dims_of(sp), sp.scale,
                       sp.softcap, bias, mask, sp.causal);
    return hipGetLastError();
}

hipError_t attention_scores_backward(const AttnScoreSpec& sp, const float* s, const float* dout, float* ds,
                                     const uint8_t* mask, float* dbias, const int64_t* bias_shape, float* workspace,
                                     hipStream_t st) {
    const int64_t n = sp.shape[0] * sp.shape[1] * sp.shape[2] * sp.shape[3];
    if (n == 0) return hipSuccess;
    const ScoreDims d = dims_of(sp);
    hipLaunchKernelGGL(scores_backward, dim3(flat_blocks(n, 256)), dim3(256), 0, st, s, dout, ds,
                       dbias ? workspace : nullptr, d, sp.scale, sp.softcap, mask, sp.causal);
    if (dbias) {
        ScoreDims o{};
        int64_t m = 1;
        for (int k = 0; k < 4; ++k) {
            o.shape[k] = bias_shape[k];
            m *= bias_shape[k];
        }
        hipLaunchKernelGGL(sum_to_shape, dim3(flat_blocks(m, 256)), dim3(256), 0, st, workspace, dbias, d, o);
    }
    return hipGetLastError();
}

hipError_t swap_last_dims(int elem_bytes, const void* x, void* y, int64_t G, int64_t R, int64_t C, hipStream_t st) {
    if (G * R * C == 0) return hipSuccess;
    const int64_t tiles_r = (R + 63) / 64, tiles_c = (C + 63) / 64;
    for (int64_t g0 = 0; g0 < G; g0 += 65535) {
        const int64_t gc = G - g0 < 65535 ? G - g0 : 65535;
        const dim3 grid(static_cast<unsigned>(tiles_r * tiles_c), 1, static_cast<unsigned>(gc));
        if (elem_bytes == 4)
            hipLaunchKernelGGL((swap_last<float>), grid, dim3(256), 0, st, static_cast<const float*>(x) + g0 * R * C,
                               static_cast<float*>(y) + g0 * R * C, R, C, tiles_c);
        else
            hipLaunchKernelGGL((swap_last<uint16_t>), grid, dim3(256), 0, st,
                               static_cast<const uint16_t*>(x) + g0 * R * C, static_cast<uint16_t*>(y) + g0 * R * C, R,
                               C, tiles_c);
    }
    return hipGetLastError();
}

}  // namespace hk
