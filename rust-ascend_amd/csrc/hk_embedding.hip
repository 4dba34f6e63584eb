// hk_embedding.hip — embedding lookup and its dense weight gradient for gfx950.
//
// Semantics (reference rust-ascend-driver/src/tensor/embedding.rs:21-79, the ACLNN
// aclnnEmbedding / aclnnEmbeddingDenseBackward pair behind AscendRuntime::embedding and
// embedding_backward, runtime/mod.rs:237-256, runtime/indexing.rs:33-64; autodiff in
// src/nn/embedding.rs):
//   forward   out[t, :] = weight[ids[t], :]  (padding does not change the lookup)
//   backward  dW[v, :] = sum over t with ids[t] == v of grad[t, :], except the padding row, which
//             stays zero; with scale_grad_by_freq each row is divided by its ID count.
// IDs are INT32 or INT64 and must lie in [0, V). An ID outside that range never addresses
// memory: its lookup row is written as zeros, its gradient is dropped, and a device flag reports
// it to the host (which turns it into an invalid-argument error after the call completes).
//
// Layout: the lookup copies rows with 16-byte (or the widest aligned) units, one wavefront per
// token. The gradient is deterministic: a stable radix sort of (ID, position) pairs groups the
// positions of each ID in increasing order, and one workgroup per table row sums its gradient rows
// in that order in F32 (no floating-point atomics), writing every row of dW (zeros where no ID
// falls). Work: the lookup moves 2 * H * sizeof(T) bytes per token; the gradient reads
// H * sizeof(T) per token and writes V * H * sizeof(T).
#include "hk_common.hpp"
#include "hk_kernels.hpp"

#include <hipcub/hipcub.hpp>

namespace hk {

namespace {

constexpr int kEmbThreads = 256;
constexpr int kTokensPerBlock = kEmbThreads / kWave;

template <typename Idx, typename U>
__global__ void __launch_bounds__(kEmbThreads)
embedding_gather_kernel(const U* __restrict__ table, const Idx* __restrict__ ids, U* __restrict__ out, int64_t tokens,
                        int64_t vocab, int64_t units, int* __restrict__ flag, int seq) {
    const int lane = threadIdx.x % kWave;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * kTokensPerBlock + threadIdx.x / kWave; t < tokens;
         t += static_cast<int64_t>(gridDim.x) * kTokensPerBlock) {
        const int64_t id = static_cast<int64_t>(ids[t]);
        const bool valid = id >= 0 && id < vocab;
        U* dst = out + t * units;
        if (valid) {
            const U* src = table + id * units;
            for (int64_t u = lane; u < units; u += kWave) dst[u] = src[u];
        } else {
            for (int64_t u = lane; u < units; u += kWave) dst[u] = U{};
            if (lane == 0) *flag = seq;
        }
    }
}

// Sort keys (ID, or V for an invalid ID), the positions 0..N-1, and per-key counts.
template <typename Idx>
__global__ void __launch_bounds__(kEmbThreads)
embedding_keys_kernel(const Idx* __restrict__ ids, int64_t tokens, int64_t vocab, uint32_t* __restrict__ keys,
                      uint32_t* __restrict__ pos, uint32_t* __restrict__ counts, int* __restrict__ flag) {
    for (int64_t t = flat_begin(kEmbThreads); t < tokens; t += flat_stride(kEmbThreads)) {
        const int64_t id = static_cast<int64_t>(ids[t]);
        const bool valid = id >= 0 && id < vocab;
        const uint32_t key = static_cast<uint32_t>(valid ? id : vocab);
        keys[t] = key;
        pos[t] = static_cast<uint32_t>(t);
        atomicAdd(counts + key, 1u);
        if (!valid) *flag = 1;
    }
}

__global__ void __launch_bounds__(kEmbThreads)
clear_counts_kernel(uint32_t* __restrict__ counts, int64_t n, int* __restrict__ flag) {
    for (int64_t i = flat_begin(kEmbThreads); i < n; i += flat_stride(kEmbThreads)) counts[i] = 0;
    if (flat_begin(kEmbThreads) == 0) *flag = 0;
}


// One workgroup per table row v: the positions of ID v are sorted[offsets[v] .. + counts[v]).
template <typename T>
__global__ void __launch_bounds__(kEmbThreads)
embedding_dense_grad_kernel(const T* __restrict__ grad, const uint32_t* __restrict__ sorted_pos,
                            const uint32_t* __restrict__ counts, const uint32_t* __restrict__ offsets,
                            T* __restrict__ dw, int64_t width, uint64_t padding, int scale, bool vec) {
    constexpr int P = Chunk<T>::kPer;
    const int64_t v = blockIdx.x;
    const uint32_t cnt = (static_cast<uint64_t>(v) == padding) ? 0u : counts[v];
    const uint32_t off = offsets[v];
    const float divisor = static_cast<float>(counts[v]);
    T* row = dw + v * width;
    if (vec) {
        for (int64_t c = static_cast<int64_t>(threadIdx.x) * P; c < width; c += kEmbThreads * P) {
            float acc[P];
#pragma unroll
            for (int e = 0; e < P; ++e) acc[e] = 0.0f;
            for (uint32_t j = 0; j < cnt; ++j) {
                float g[P];
                Chunk<T>::load(grad + static_cast<int64_t>(sorted_pos[off + j]) * width + c, g);
#pragma unroll
                for (int e = 0; e < P; ++e) acc[e] += g[e];
            }
            if (scale && cnt) {
#pragma unroll
                for (int e = 0; e < P; ++e) acc[e] = acc[e] / divisor;
            }
            Chunk<T>::store(row + c, acc);
        }
    } else {
        for (int64_t c = threadIdx.x; c < width; c += kEmbThreads) {
            float acc = 0.0f;
            for (uint32_t j = 0; j < cnt; ++j)
                acc += Elem<T>::load(grad, static_cast<int64_t>(sorted_pos[off + j]) * width + c);
            if (scale && cnt) acc = acc / divisor;
            Elem<T>::store(row, c, acc);
        }
    }
}

// Workspace carve-up (256-byte aligned pieces).
struct EmbWs {
    int* flag;
    uint32_t *keys, *pos, *keys_sorted, *pos_sorted, *counts, *offsets;
    void* cub;
    size_t cub_bytes;
};

size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

int key_bits(int64_t vocab) {  // bits holding keys 0..vocab (vocab itself marks invalid IDs)
    int b = 1;
    while (b < 32 && (int64_t(1) << b) <= vocab) ++b;
    return b;
}

size_t cub_bytes_for(int64_t tokens, int64_t vocab) {
    size_t sort_bytes = 0, scan_bytes = 0;
    (void)hipcub::DeviceRadixSort::SortPairs(nullptr, sort_bytes, static_cast<const uint32_t*>(nullptr),
                                             static_cast<uint32_t*>(nullptr), static_cast<const uint32_t*>(nullptr),
                                             static_cast<uint32_t*>(nullptr), static_cast<int>(tokens), 0,
                                             key_bits(vocab));
    (void)hipcub::DeviceScan::ExclusiveSum(nullptr, scan_bytes, static_cast<const uint32_t*>(nullptr),
                                           static_cast<uint32_t*>(nullptr), static_cast<int>(vocab + 1));
    return sort_bytes > scan_bytes ? sort_bytes : scan_bytes;
}

EmbWs carve(void* base, int64_t tokens, int64_t vocab) {
    EmbWs w{};
    char* p = static_cast<char*>(base);
    w.flag = reinterpret_cast<int*>(p);
    p += 256;
    const size_t tok = align256(static_cast<size_t>(tokens) * 4), voc = align256(static_cast<size_t>(vocab + 1) * 4);
    w.keys = reinterpret_cast<uint32_t*>(p); p += tok;
    w.pos = reinterpret_cast<uint32_t*>(p); p += tok;
    w.keys_sorted = reinterpret_cast<uint32_t*>(p); p += tok;
    w.pos_sorted = reinterpret_cast<uint32_t*>(p); p += tok;
    w.counts = reinterpret_cast<uint32_t*>(p); p += voc;
    w.offsets = reinterpret_cast<uint32_t*>(p); p += voc;
    w.cub = p;
    w.cub_bytes = cub_bytes_for(tokens, vocab);
    return w;
}

template <typename Idx, typename U>
void launch_gather(const void* table, const void* ids, void* out, int64_t tokens, int64_t vocab, int64_t row_bytes,
                   int* flag, int seq, hipStream_t s) {
    const unsigned grid = flat_blocks(tokens, kTokensPerBlock);
    hipLaunchKernelGGL((embedding_gather_kernel<Idx, U>), dim3(grid), dim3(kEmbThreads), 0, s,
                       static_cast<const U*>(table), static_cast<const Idx*>(ids), static_cast<U*>(out), tokens,
                       vocab, row_bytes / static_cast<int64_t>(sizeof(U)), flag, seq);
}

template <typename Idx>
void gather_by_unit(const void* table, const void* ids, void* out, int64_t tokens, int64_t vocab, int64_t row_bytes,
                    int* flag, int seq, hipStream_t s) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(table) | reinterpret_cast<uintptr_t>(out) |
                        static_cast<uintptr_t>(row_bytes);
    if (a % 16 == 0) launch_gather<Idx, u32x4_t>(table, ids, out, tokens, vocab, row_bytes, flag, seq, s);
    else if (a % 8 == 0) launch_gather<Idx, u32x2_t>(table, ids, out, tokens, vocab, row_bytes, flag, seq, s);
    else if (a % 4 == 0) launch_gather<Idx, uint32_t>(table, ids, out, tokens, vocab, row_bytes, flag, seq, s);
    else launch_gather<Idx, uint16_t>(table, ids, out, tokens, vocab, row_bytes, flag, seq, s);
}

template <typename T>
void launch_dense_grad(const void* grad, const EmbWs& w, void* dw, int64_t vocab, int64_t width, uint64_t padding,
                       int scale, hipStream_t s) {
    const bool vec = width % Chunk<T>::kPer == 0 && aligned16({grad, dw});
    hipLaunchKernelGGL(embedding_dense_grad_kernel<T>, dim3(static_cast<unsigned>(vocab)), dim3(kEmbThreads), 0, s,
                       static_cast<const T*>(grad), w.pos_sorted, w.counts, w.offsets, static_cast<T*>(dw), width,
                       padding, scale, vec);
}

}  // namespace

size_t embedding_workspace_bytes(int64_t tokens, int64_t vocab, bool backward) {
    if (!backward) return 256;
    return 256 + 4 * align256(static_cast<size_t>(tokens) * 4) + 2 * align256(static_cast<size_t>(vocab + 1) * 4) +
           align256(cub_bytes_for(tokens, vocab));
}

hipError_t embedding(const void* table, int id_bytes, const void* ids, void* out, int64_t tokens, int64_t vocab,
                     int64_t row_bytes, int* flag, int seq, hipStream_t s) {
    if (tokens > 0 && row_bytes > 0) {
        if (id_bytes == 8) gather_by_unit<int64_t>(table, ids, out, tokens, vocab, row_bytes, flag, seq, s);
        else gather_by_unit<int32_t>(table, ids, out, tokens, vocab, row_bytes, flag, seq, s);
    }
    return hipGetLastError();
}

hipError_t embedding_backward(int dtype, const void* grad, int id_bytes, const void* ids, void* dw, int64_t tokens,
                              int64_t vocab, int64_t width, uint64_t padding, int scale, void* workspace,
                              hipStream_t s) {
    EmbWs w = carve(workspace, tokens, vocab);
    const unsigned cgrid = flat_blocks(vocab + 1, kEmbThreads);
    hipLaunchKernelGGL(clear_counts_kernel, dim3(cgrid), dim3(kEmbThreads), 0, s, w.counts, vocab + 1, w.flag);
    if (tokens > 0) {
        const unsigned tgrid = flat_blocks(tokens, kEmbThreads);
        if (id_bytes == 8)
            hipLaunchKernelGGL(embedding_keys_kernel<int64_t>, dim3(tgrid), dim3(kEmbThreads), 0, s,
                               static_cast<const int64_t*>(ids), tokens, vocab, w.keys, w.pos, w.counts, w.flag);
        else
            hipLaunchKernelGGL(embedding_keys_kernel<int32_t>, dim3(tgrid), dim3(kEmbThreads), 0, s,
                               static_cast<const int32_t*>(ids), tokens, vocab, w.keys, w.pos, w.counts, w.flag);
        size_t cb = w.cub_bytes;
        hipError_t e = hipcub::DeviceRadixSort::SortPairs(w.cub, cb, w.keys, w.keys_sorted, w.pos, w.pos_sorted,
                                                          static_cast<int>(tokens), 0, key_bits(vocab), s);
        if (e != hipSuccess) return e;
    }
    size_t cb = w.cub_bytes;
    hipError_t e = hipcub::DeviceScan::ExclusiveSum(w.cub, cb, w.counts, w.offsets, static_cast<int>(vocab + 1), s);
    if (e != hipSuccess) return e;
    if (vocab > 0 && width > 0) {
        if (dtype == 1) launch_dense_grad<_Float16>(grad, w, dw, vocab, width, padding, scale, s);
        else if (dtype == 27) launch_dense_grad<uint16_t>(grad, w, dw, vocab, width, padding, scale, s);
        else launch_dense_grad<float>(grad, w, dw, vocab, width, padding, scale, s);
    }
    return hipGetLastError();
}

}  // namespace hk
