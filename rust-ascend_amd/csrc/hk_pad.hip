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
// crop_f32 reads only the retained [batch, rows, cols] window. Both are HBM-bound. Rows of at least
// 512 (pad) or 256 (crop) columns with 16-byte aligned destinations go through the row kernels
// (a workgroup per row at a time, 16-byte chunks per thread); the rest through element kernels (one
// work item per destination element pair or element in a grid-stride walk).
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

// pad_bf16_kernel's result, row by row: destination row rb of [batch, R, C] (its batch and row
// from one division per row), thread j its 8 columns 8j .. 8j+7 as one 16-byte store. Where all 8
// exist in the source and vec_src (the source rows are 16-byte aligned), one 16-byte (BF16) or two
// (F32) loads; else per element, zero outside the source. BF16 is copied bit for bit, F32 rounded
// as pad_bf16_kernel rounds it.
template <typename T>
__global__ void __launch_bounds__(kPadThreads)
pad_rows_kernel(const T* __restrict__ src, uint16_t* __restrict__ dst, int64_t rows, int64_t cols, int64_t R,
                int64_t C, int64_t nrows, int vec_src) {
    const int64_t chunks = C / 8;  // C is a multiple of 16
    for (int64_t rb = blockIdx.x; rb < nrows; rb += gridDim.x) {
        const int64_t b = rb / R, r = rb - b * R;
        const T* srow = src + (b * rows + r) * cols;  // read only for r < rows
        uint16_t* drow = dst + rb * C;
        for (int64_t j = threadIdx.x; j < chunks; j += kPadThreads) {
            const int64_t c0 = 8 * j;
            u32x4_t w;
            if (vec_src && r < rows && c0 + 8 <= cols) {
                if constexpr (sizeof(T) == 2) {
                    w = *reinterpret_cast<const u32x4_t*>(srow + c0);
                } else {
                    float v[8];
                    load8(srow + c0, v);
#pragma unroll
                    for (int i = 0; i < 4; ++i) w[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
                }
            } else {
                uint16_t h[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    h[e] = 0;
                    if (r < rows && c0 + e < cols) {
                        if constexpr (sizeof(T) == 4) h[e] = f32_to_bf16(srow[c0 + e]);
                        else h[e] = srow[c0 + e];
                    }
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) w[i] = static_cast<uint32_t>(h[2 * i]) | (static_cast<uint32_t>(h[2 * i + 1]) << 16);
            }
            *reinterpret_cast<u32x4_t*>(drow + c0) = w;
        }
    }
}

// crop_f32_kernel's result, row by row: destination row rb of [batch, rows, cols] copied from its
// source row of [batch, R, C] as 16-byte chunks (vec: cols % 4 == 0 and both bases 16-byte
// aligned), else per element.
__global__ void __launch_bounds__(kPadThreads)
crop_rows_kernel(const float* __restrict__ src, float* __restrict__ dst, int64_t rows, int64_t cols, int64_t R,
                 int64_t C, int64_t nrows, int vec) {
    for (int64_t rb = blockIdx.x; rb < nrows; rb += gridDim.x) {
        const int64_t b = rb / rows, r = rb - b * rows;
        const float* srow = src + (b * R + r) * C;
        float* drow = dst + rb * cols;
        if (vec) {
            for (int64_t j = threadIdx.x; j < cols / 4; j += kPadThreads)
                *reinterpret_cast<f32x4_t*>(drow + 4 * j) = *reinterpret_cast<const f32x4_t*>(srow + 4 * j);
        } else {
            for (int64_t c = threadIdx.x; c < cols; c += kPadThreads) drow[c] = srow[c];
        }
    }
}

unsigned blocks_for(int64_t work) { return flat_blocks(work, kPadThreads); }
bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace

hipError_t pad_bf16(int src_bf16, const void* src, void* dst, int64_t batch, int64_t rows, int64_t cols, int64_t R,
                    int64_t C, hipStream_t s) {
    const int64_t pairs = batch * R * C / 2;
    if (pairs == 0) return hipSuccess;
    if (C >= 512 && aligned16(dst)) {
        const int64_t nrows = batch * R;
        const int vec = aligned16(src) && cols % (src_bf16 ? 8 : 4) == 0;
        const dim3 grid(static_cast<unsigned>(nrows < kMaxFlatBlocks ? nrows : kMaxFlatBlocks));
        if (src_bf16)
            hipLaunchKernelGGL(pad_rows_kernel<uint16_t>, grid, dim3(kPadThreads), 0, s, static_cast<const uint16_t*>(src),
                               static_cast<uint16_t*>(dst), rows, cols, R, C, nrows, vec);
        else
            hipLaunchKernelGGL(pad_rows_kernel<float>, grid, dim3(kPadThreads), 0, s, static_cast<const float*>(src),
                               static_cast<uint16_t*>(dst), rows, cols, R, C, nrows, vec);
        return hipGetLastError();
    }
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
    if (cols >= 256) {
        const int64_t nrows = batch * rows;
        const int vec = cols % 4 == 0 && aligned16(src) && aligned16(dst);
        const dim3 grid(static_cast<unsigned>(nrows < kMaxFlatBlocks ? nrows : kMaxFlatBlocks));
        hipLaunchKernelGGL(crop_rows_kernel, grid, dim3(kPadThreads), 0, s, src, dst, rows, cols, R, C, nrows, vec);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(crop_f32_kernel, dim3(blocks_for(total)), dim3(kPadThreads), 0, s, src, dst, rows, cols, R, C,
                       total);
    return hipGetLastError();
}

}  // namespace hk
