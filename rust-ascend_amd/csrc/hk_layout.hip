// hk_layout.hip — the decoder layer's relayouts between token rows and attention head planes,
// for gfx950.
//
// The fused QKV projection writes token rows qkv [B, S, (Hq + 2 Hkv) D] (Q heads, then K heads,
// then V heads, each D wide). Attention reads head planes q [B, Hq, S, D], k, v [B, Hkv, S, D].
// qkv_rope_split moves the rows into the planes and applies RoPE to Q and K in the same pass
// (the rotation of hk_rotary: pairs (p, p + D/2) for SplitHalf or (2p, 2p + 1) for Interleaved,
// angles from F32 tables cos/sin [S, D/2] indexed by the position s); V is copied bit-exactly.
// qkv_rope_merge is its transpose for the gradients (the rotation's transpose on dQ and dK).
// heads_to_rows / rows_to_heads convert [B, H, S, D] <-> [B, S, H D] (the attention output into
// the output projection's rows and back for its gradient).
//
// All four are HBM-bound copies: 2 bytes read and written per element (plus the tables, which
// stay in cache). Each thread owns 8 pairs (16 BF16 values, two 16-byte accesses) of one
// (token, head) row; D % 16 == 0.
#include "hk_common.hpp"
#include "hk_kernels.hpp"

namespace hk {

namespace {

constexpr int kLayoutThreads = 256;

// 8 pairs (a_i, b_i) of one head row at pair index p0: SplitHalf a at p0.., b at D/2 + p0..;
// Interleaved (a, b) interleaved over 16 values at 2 p0.
template <int LAYOUT>
__device__ __forceinline__ void load_pairs(const uint16_t* row, int64_t half, int64_t p0, float (&a)[8],
                                           float (&b)[8]) {
    if constexpr (LAYOUT == 1) {
        load8(row + p0, a);
        load8(row + half + p0, b);
    } else {
        float lo[8], hi[8];
        load8(row + 2 * p0, lo);
        load8(row + 2 * p0 + 8, hi);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            a[i] = lo[2 * i];
            b[i] = lo[2 * i + 1];
            a[4 + i] = hi[2 * i];
            b[4 + i] = hi[2 * i + 1];
        }
    }
}
template <int LAYOUT>
__device__ __forceinline__ void store_pairs(uint16_t* row, int64_t half, int64_t p0, const float (&a)[8],
                                            const float (&b)[8]) {
    if constexpr (LAYOUT == 1) {
        store8(row + p0, a);
        store8(row + half + p0, b);
    } else {
        float lo[8], hi[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            lo[2 * i] = a[i];
            lo[2 * i + 1] = b[i];
            hi[2 * i] = a[4 + i];
            hi[2 * i + 1] = b[4 + i];
        }
        store8(row + 2 * p0, lo);
        store8(row + 2 * p0 + 8, hi);
    }
}

// The 16 values of a chunk as raw bits (V heads: no rotation, bit-exact copy).
template <int LAYOUT>
__device__ __forceinline__ void copy_pairs(const uint16_t* src, uint16_t* dst, int64_t half, int64_t p0) {
    if constexpr (LAYOUT == 1) {
        *reinterpret_cast<u32x4_t*>(dst + p0) = *reinterpret_cast<const u32x4_t*>(src + p0);
        *reinterpret_cast<u32x4_t*>(dst + half + p0) = *reinterpret_cast<const u32x4_t*>(src + half + p0);
    } else {
        *reinterpret_cast<u32x4_t*>(dst + 2 * p0) = *reinterpret_cast<const u32x4_t*>(src + 2 * p0);
        *reinterpret_cast<u32x4_t*>(dst + 2 * p0 + 8) = *reinterpret_cast<const u32x4_t*>(src + 2 * p0 + 8);
    }
}

// MERGE = false: qkv rows -> (q, k, v) planes with the forward rotation on Q and K.
// MERGE = true: (dq, dk, dv) planes -> dqkv rows with the backward rotation on dQ and dK.
template <int LAYOUT, bool MERGE>
__global__ void __launch_bounds__(kLayoutThreads)
qkv_rope_kernel(uint16_t* __restrict__ rows, uint16_t* __restrict__ q, uint16_t* __restrict__ k,
                uint16_t* __restrict__ v, const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                int64_t seq, int64_t hq, int64_t hkv, int64_t d, int64_t total) {
    for (int64_t idx = flat_begin(kLayoutThreads); idx < total; idx += flat_stride(kLayoutThreads)) {
        const int64_t half = d / 2, chunks = half / 8, heads = hq + 2 * hkv;
        const int64_t chunk = idx % chunks;
        const int64_t head_row = idx / chunks;
        const int64_t h = head_row % heads, t = head_row / heads;
        const int64_t b = t / seq, s = t - b * seq;
        const int64_t p0 = chunk * 8;
        uint16_t* row = rows + t * heads * d + h * d;
        uint16_t* plane;
        if (h < hq) plane = q + ((b * hq + h) * seq + s) * d;
        else if (h < hq + hkv) plane = k + ((b * hkv + (h - hq)) * seq + s) * d;
        else plane = v + ((b * hkv + (h - hq - hkv)) * seq + s) * d;
        if (h >= hq + hkv) {
            if (MERGE) copy_pairs<LAYOUT>(plane, row, half, p0);
            else copy_pairs<LAYOUT>(row, plane, half, p0);
            return;
        }
        float c[8], sn[8], a[8], bb[8], ya[8], yb[8];
        const float* ct = cos_t + s * half + p0;
        const float* st = sin_t + s * half + p0;
        load8(ct, c);
        load8(st, sn);
        load_pairs<LAYOUT>(MERGE ? plane : row, half, p0, a, bb);
#pragma unroll
        for (int i = 0; i < 8; ++i) rope_rotate<MERGE>(a[i], bb[i], c[i], sn[i], ya[i], yb[i]);
        store_pairs<LAYOUT>(MERGE ? row : plane, half, p0, ya, yb);
    }
}

// TO_ROWS: x [B, H, S, D] -> y [B, S, H D]; otherwise the reverse. 8 elements per thread.
template <bool TO_ROWS>
__global__ void __launch_bounds__(kLayoutThreads)
heads_rows_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ y, int64_t heads, int64_t seq, int64_t d,
                  int64_t total) {
    for (int64_t idx = flat_begin(kLayoutThreads); idx < total; idx += flat_stride(kLayoutThreads)) {
        const int64_t chunks = d / 8;
        const int64_t c = idx % chunks;
        // idx enumerates the row layout [B, S, H, D/8] so the row-side accesses are contiguous
        const int64_t h = (idx / chunks) % heads;
        const int64_t t = idx / (chunks * heads);  // b * seq + s
        const int64_t b = t / seq, s = t - b * seq;
        const int64_t row_off = (t * heads + h) * d + c * 8;
        const int64_t plane_off = ((b * heads + h) * seq + s) * d + c * 8;
        const int64_t from = TO_ROWS ? plane_off : row_off, to = TO_ROWS ? row_off : plane_off;
        *reinterpret_cast<u32x4_t*>(y + to) = *reinterpret_cast<const u32x4_t*>(x + from);
    }
}

unsigned blocks_of(int64_t work) { return flat_blocks(work, kLayoutThreads); }

}  // namespace

hipError_t qkv_rope(bool merge, int layout, void* rows, void* q, void* k, void* v, const float* cos_t,
                    const float* sin_t, int64_t batch, int64_t seq, int64_t hq, int64_t hkv, int64_t d, hipStream_t s) {
    const int64_t total = batch * seq * (hq + 2 * hkv) * (d / 16);
    if (total == 0) return hipSuccess;
    auto* r = static_cast<uint16_t*>(rows);
    auto* qp = static_cast<uint16_t*>(q);
    auto* kp = static_cast<uint16_t*>(k);
    auto* vp = static_cast<uint16_t*>(v);
    const dim3 grid(blocks_of(total)), block(kLayoutThreads);
    if (layout == 1) {
        if (merge) hipLaunchKernelGGL((qkv_rope_kernel<1, true>), grid, block, 0, s, r, qp, kp, vp, cos_t, sin_t, seq, hq, hkv, d, total);
        else hipLaunchKernelGGL((qkv_rope_kernel<1, false>), grid, block, 0, s, r, qp, kp, vp, cos_t, sin_t, seq, hq, hkv, d, total);
    } else {
        if (merge) hipLaunchKernelGGL((qkv_rope_kernel<0, true>), grid, block, 0, s, r, qp, kp, vp, cos_t, sin_t, seq, hq, hkv, d, total);
        else hipLaunchKernelGGL((qkv_rope_kernel<0, false>), grid, block, 0, s, r, qp, kp, vp, cos_t, sin_t, seq, hq, hkv, d, total);
    }
    return hipGetLastError();
}

hipError_t heads_rows(bool to_rows, const void* x, void* y, int64_t batch, int64_t heads, int64_t seq, int64_t d,
                      hipStream_t s) {
    const int64_t total = batch * heads * seq * (d / 8);
    if (total == 0) return hipSuccess;
    if (to_rows)
        hipLaunchKernelGGL(heads_rows_kernel<true>, dim3(blocks_of(total)), dim3(kLayoutThreads), 0, s,
                           static_cast<const uint16_t*>(x), static_cast<uint16_t*>(y), heads, seq, d, total);
    else
        hipLaunchKernelGGL(heads_rows_kernel<false>, dim3(blocks_of(total)), dim3(kLayoutThreads), 0, s,
                           static_cast<const uint16_t*>(x), static_cast<uint16_t*>(y), heads, seq, d, total);
    return hipGetLastError();
}

}  // namespace hk
