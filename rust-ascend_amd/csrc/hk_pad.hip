// hk_pad.hip — zero padding and cropping of matrix tails for the padded BF16-compute GEMM.
//
// Reference (paths relative to the shuqi2077/rust-ascend root): runtime/padded_matrix.rs:6-43
// pads each matrix axis of a rank-2/3 tensor up to a multiple of 16 with zeros ("prefix
// resize", positive end padding), rounding F32 to BF16 first (conversion::cast, RNE), runs the
// native GEMM on the padded operands with F32 output, and crops the F32 result back to its
// logical shape (negative end padding: retained values are copied bit for bit).
//
// Layout: [batch, rows, cols] row-major on both sides. pad_bf16 writes the whole padded
// [batch, R, C] destination (zeros outside the source), so no separate clearing pass is needed;
// crop_f32 reads only the retained [batch, rows, cols] window. Both are HBM-bound: one work item per
// destination element pair (BF16) or element (F32) in a grid-stride walk, coalesced along the
// last axis.
#include "hk_common.hpp"
#include "hk_kernels.hpp"

namespace hk {

namespace {

constexpr int kPadThreads = 256;

// dst[b, r, c] = bf16(src[b, r, c]) inside the source, 0 outside; two BF16 per thread.
template <typename T>
__global__ void __launch_bounds__(kPadThreads)
pad_bf16_kernel(const T* __restrict__ src, uint16_t* __restrict__ dst, int64_t rows, int64_t cols, int64_t R,
                int64_t C, int64_t total_pairs) {
    for (int64_t pair = flat_begin(kPadThreads); pair < total_pairs; pair += flat_stride(kPadThreads)) {
        const int64_t i = 2 * pair;  // C is even (a multiple of 16), so a pair never crosses a row
        const int64_t c = i % C, rb = i / C;
        const int64_t r = rb % R, b = rb / R;
        uint16_t v[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int64_t cc = c + e;
            if (r < rows && cc < cols) {
                const int64_t s = (b * rows + r) * cols + cc;
                if constexpr (sizeof(T) == 4) v[e] = f32_to_bf16(src[s]);
                else v[e] = src[s];
            } else {
                v[e] = 0;
            }
        }
        *reinterpret_cast<uint32_t*>(dst + i) = static_cast<uint32_t>(v[0]) | (static_cast<uint32_t>(v[1]) << 16);
    }
}

// dst[b, r, c] = src[b, r, c] for the retained window of a [batch, R, C] F32 source.
__global__ void __launch_bounds__(kPadThreads)
crop_f32_kernel(const float* __restrict__ src, float* __restrict__ dst, int64_t rows, int64_t cols, int64_t R,
                int64_t C, int64_t total) {
    for (int64_t i = flat_begin(kPadThreads); i < total; i += flat_stride(kPadThreads)) {
        const int64_t c = i % cols, rb = i / cols;
        const int64_t r = rb % rows, b = rb / rows;
        dst[i] = src[(b * R + r) * C + c];
    }
}

unsigned blocks_for(int64_t work) { return flat_blocks(work, kPadThreads); }

}  // namespace

hipError_t pad_bf16(int src_bf16, const void* src, void* dst, int64_t batch, int64_t rows, int64_t cols, int64_t R,
                    int64_t C, hipStream_t s) {
    const int64_t pairs = batch * R * C / 2;
    if (pairs == 0) return hipSuccess;
    if (src_bf16)
        hipLaunchKernelGGL(pad_bf16_kernel<uint16_t>, dim3(blocks_for(pairs)), dim3(kPadThreads), 0, s,
                           static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst), rows, cols, R, C, pairs);
    else
        hipLaunchKernelGGL(pad_bf16_kernel<float>, dim3(blocks_for(pairs)), dim3(kPadThreads), 0, s,
                           static_cast<const float*>(src), static_cast<uint16_t*>(dst), rows, cols, R, C, pairs);
    return hipGetLastError();
}

hipError_t crop_f32(const float* src, float* dst, int64_t batch, int64_t rows, int64_t cols, int64_t R, int64_t C,
                    hipStream_t s) {
    const int64_t total = batch * rows * cols;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(crop_f32_kernel, dim3(blocks_for(total)), dim3(kPadThreads), 0, s, src, dst, rows, cols, R, C,
                       total);
    return hipGetLastError();
}

}  // namespace hk
