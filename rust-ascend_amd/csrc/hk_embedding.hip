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
// token. The gradient is deterministic: a stable least-significant-digit radix sort of
// (ID, position) pairs, 8-bit digits, groups the positions of each ID in increasing order, and one
// workgroup per table row sums its gradient rows in that order in F32 (no floating-point
// atomics), writing every row of dW (zeros where no ID falls). Each sort pass is three launches:
// per-tile digit histograms (4096 positions per workgroup, LDS counters), an exclusive scan of
// the histograms in digit-major order (the output slot of each digit's first element in each
// tile), and a scatter that places every element at its digit's slot plus its rank among the
// tile's earlier elements with the same digit (ballots within a wavefront, LDS counts across
// wavefronts and rounds), so equal digits keep their position order. The row offsets of dW come
// from per-ID counts (integer atomics) and the same scan. Up to 8192 positions and 65535 table rows
// (the decoder layer's 4096 x 32000) the whole grouping runs in one 1024-thread workgroup instead:
// the same digit passes and ballot ranks over keys held in LDS, each ID's range then read off the
// sorted keys. Work: the lookup moves
// 2 * H * sizeof(T) bytes per token; the gradient reads H * sizeof(T) per token and writes
// V * H * sizeof(T); the sort moves 16 bytes per token and pass.
#include "hk_common.hpp"
#include "hk_kernels.hpp"

#include <algorithm>
#include <utility>

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


// ---- grouping by ID: exclusive scan and a stable radix sort, hand-written for wave64

constexpr int kScanThreads = 1024;
constexpr int kScanItems = 4;
constexpr int kScanTile = kScanThreads * kScanItems;  // elements per workgroup

// out[i] = sum of in[j] for j < i within each tile of kScanTile elements (in may equal out); the
// tile's total goes to tile_sums[blockIdx.x] when tile_sums is not null.
__global__ void __launch_bounds__(kScanThreads)
scan_tiles_kernel(const uint32_t* in, uint32_t* out, int64_t n, uint32_t* __restrict__ tile_sums) {
    __shared__ uint32_t wave_total[kScanThreads / kWave];
    const int t = threadIdx.x, lane = t % kWave, w = t / kWave;
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile + static_cast<int64_t>(t) * kScanItems;
    uint32_t v[kScanItems], ex[kScanItems];
    uint32_t sum = 0;
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        v[j] = base + j < n ? in[base + j] : 0u;
        ex[j] = sum;
        sum += v[j];
    }
    uint32_t incl = sum;  // inclusive scan of the threads' sums within the wavefront
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const uint32_t y = __shfl_up(incl, off, kWave);
        if (lane >= off) incl += y;
    }
    if (lane == kWave - 1) wave_total[w] = incl;
    __syncthreads();
    uint32_t before = incl - sum;
    for (int ww = 0; ww < w; ++ww) before += wave_total[ww];
#pragma unroll
    for (int j = 0; j < kScanItems; ++j)
        if (base + j < n) out[base + j] = before + ex[j];
    if (tile_sums != nullptr && t == kScanThreads - 1) tile_sums[blockIdx.x] = before + sum;
}

// Adds the scanned tile totals: out[i] += tile_base[i / kScanTile].
__global__ void __launch_bounds__(kScanThreads)
scan_add_kernel(uint32_t* __restrict__ out, int64_t n, const uint32_t* __restrict__ tile_base) {
    const uint32_t add = tile_base[blockIdx.x];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile;
    for (int j = threadIdx.x; j < kScanTile; j += kScanThreads)
        if (base + j < n) out[base + j] += add;
}

size_t scan_scratch_elems(int64_t n) {  // tile totals of every level, 64-entry aligned
    size_t total = 0;
    for (int64_t m = (n + kScanTile - 1) / kScanTile; m > 1; m = (m + kScanTile - 1) / kScanTile)
        total += static_cast<size_t>((m + 63) / 64 * 64);
    return total;
}

// Exclusive scan of n (< 2^31) counts whose total fits 32 bits.
void scan_exclusive(const uint32_t* in, uint32_t* out, int64_t n, uint32_t* scratch, hipStream_t s) {
    if (n <= 0) return;
    const int64_t tiles = (n + kScanTile - 1) / kScanTile;
    if (tiles == 1) {
        hipLaunchKernelGGL(scan_tiles_kernel, dim3(1), dim3(kScanThreads), 0, s, in, out, n, nullptr);
        return;
    }
    uint32_t* sums = scratch;
    hipLaunchKernelGGL(scan_tiles_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kScanThreads), 0, s, in, out, n,
                       sums);
    scan_exclusive(sums, sums, tiles, scratch + (tiles + 63) / 64 * 64, s);
    hipLaunchKernelGGL(scan_add_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kScanThreads), 0, s, out, n, sums);
}

constexpr int kSortThreads = 256;
constexpr int kSortWaves = kSortThreads / kWave;
constexpr int kSortRounds = 16;
constexpr int kSortTile = kSortThreads * kSortRounds;  // positions per workgroup
constexpr int kDigits = 256;

// hist[d * tiles + b] = how many keys of tile b have digit d ((key >> shift) & 255).
__global__ void __launch_bounds__(kSortThreads)
digit_hist_kernel(const uint32_t* __restrict__ keys, int64_t n, int shift, uint32_t* __restrict__ hist, int tiles) {
    __shared__ uint32_t h[kDigits];
    h[threadIdx.x] = 0;
    __syncthreads();
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kSortTile;
    for (int r = 0; r < kSortRounds; ++r) {
        const int64_t i = base + r * kSortThreads + threadIdx.x;
        if (i < n) atomicAdd(&h[(keys[i] >> shift) & 255u], 1u);
    }
    __syncthreads();
    hist[static_cast<int64_t>(threadIdx.x) * tiles + blockIdx.x] = h[threadIdx.x];
}

// Stable scatter of one pass: element i of tile b (positions in order, 256 per round) goes to
// slot[d][b] + (elements of tile b before i with digit d). Within a round, a wavefront ranks its
// lanes by eight ballots (the lanes sharing the digit, counted below the lane); the wavefronts
// before it and the rounds before this one are added through LDS counts.
__global__ void __launch_bounds__(kSortThreads)
digit_scatter_kernel(const uint32_t* __restrict__ keys, const uint32_t* __restrict__ vals, int64_t n, int shift,
                     const uint32_t* __restrict__ slot, int tiles, uint32_t* __restrict__ keys_out,
                     uint32_t* __restrict__ vals_out) {
    __shared__ uint32_t next[kDigits];                 // this tile's next free slot of each digit
    __shared__ uint32_t wave_count[kSortWaves][kDigits];
    const int t = threadIdx.x, lane = t % kWave, w = t / kWave;
    next[t] = slot[static_cast<int64_t>(t) * tiles + blockIdx.x];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kSortTile;
    for (int r = 0; r < kSortRounds; ++r) {
#pragma unroll
        for (int ww = 0; ww < kSortWaves; ++ww) wave_count[ww][t] = 0;
        __syncthreads();
        const int64_t i = base + r * kSortThreads + t;
        const bool active = i < n;
        const uint32_t key = active ? keys[i] : 0u;
        const uint32_t d = (key >> shift) & 255u;
        uint64_t peers = __ballot(active);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const bool bit = (d >> b) & 1u;
            const uint64_t set = __ballot(bit);
            peers &= bit ? set : ~set;
        }
        const uint64_t below = peers & ((uint64_t{1} << lane) - 1);
        if (active && below == 0) wave_count[w][d] = static_cast<uint32_t>(__popcll(peers));
        __syncthreads();
        if (active) {
            uint32_t at = next[d] + static_cast<uint32_t>(__popcll(below));
            for (int ww = 0; ww < w; ++ww) at += wave_count[ww][d];
            keys_out[at] = key;
            vals_out[at] = vals[i];
        }
        __syncthreads();
        uint32_t add = 0;
#pragma unroll
        for (int ww = 0; ww < kSortWaves; ++ww) add += wave_count[ww][t];
        next[t] += add;  // read by the next round after its first barrier
    }
}

// The whole sort in one workgroup for up to kSmallSort positions (C5: 4096): keys and positions
// stay in LDS through every 8-bit pass, so a pass is a histogram, a 256-entry scan and a stable
// scatter separated by barriers instead of three launches with global round trips. The scatter
// takes the positions in rounds of 1024 in order, each wavefront ranking its lanes by ballots as
// digit_scatter_kernel does, so the order is that of the multi-workgroup sort.
constexpr int kSmallSortThreads = 1024;
constexpr int kSmallSortWaves = kSmallSortThreads / kWave;
constexpr int kSmallSort = 8192;
struct SmallSortLds {
    uint32_t kb[2][kSmallSort];
    uint32_t pb[2][kSmallSort];
    uint32_t base[kDigits];
    uint32_t wave_count[kSmallSortWaves][kDigits];
};

// Sorts the n pairs in L.kb[0] / L.pb[0] (filled by the caller before a barrier); returns the
// buffer index holding the result. Every thread of the workgroup calls it.
__device__ int lds_radix_sort(SmallSortLds& L, int n, int bits) {
    const int t = threadIdx.x, lane = t % kWave, w = t / kWave;
    for (int i = t; i < kSmallSortWaves * kDigits; i += kSmallSortThreads) (&L.wave_count[0][0])[i] = 0;
    int src = 0;
    for (int shift = 0; shift < bits; shift += 8, src ^= 1) {
        if (t < kDigits) L.base[t] = 0;
        __syncthreads();
        for (int i = t; i < n; i += kSmallSortThreads) atomicAdd(&L.base[(L.kb[src][i] >> shift) & 255u], 1u);
        __syncthreads();
        if (t < kWave) {  // exclusive scan of the 256 digit counts by the first wavefront
            uint32_t c[4], sum = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                c[j] = L.base[4 * t + j];
                sum += c[j];
            }
            uint32_t incl = sum;
#pragma unroll
            for (int off = 1; off < kWave; off <<= 1) {
                const uint32_t y = __shfl_up(incl, off, kWave);
                if (lane >= off) incl += y;
            }
            uint32_t run = incl - sum;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                L.base[4 * t + j] = run;
                run += c[j];
            }
        }
        __syncthreads();
        for (int r0 = 0; r0 < n; r0 += kSmallSortThreads) {
            const int i = r0 + t;
            const bool active = i < n;
            const uint32_t key = active ? L.kb[src][i] : 0u;
            const uint32_t d = (key >> shift) & 255u;
            uint64_t peers = __ballot(active);
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                const bool bit = (d >> b) & 1u;
                const uint64_t set = __ballot(bit);
                peers &= bit ? set : ~set;
            }
            const uint64_t below = peers & ((uint64_t{1} << lane) - 1);
            if (active && below == 0) L.wave_count[w][d] = static_cast<uint32_t>(__popcll(peers));
            __syncthreads();
            if (active) {
                uint32_t at = L.base[d] + static_cast<uint32_t>(__popcll(below));
                for (int ww = 0; ww < w; ++ww) at += L.wave_count[ww][d];
                L.kb[src ^ 1][at] = key;
                L.pb[src ^ 1][at] = L.pb[src][i];
            }
            __syncthreads();
            if (t < kDigits) {
                uint32_t add = 0;
#pragma unroll
                for (int ww = 0; ww < kSmallSortWaves; ++ww) {
                    add += L.wave_count[ww][t];
                    L.wave_count[ww][t] = 0;
                }
                L.base[t] += add;
            }
            __syncthreads();
        }
    }
    return src;
}

__global__ void __launch_bounds__(kSmallSortThreads)
small_sort_kernel(const uint32_t* __restrict__ keys_in, const uint32_t* __restrict__ pos_in, int n, int bits,
                  uint32_t* __restrict__ keys_out, uint32_t* __restrict__ pos_out) {
    __shared__ SmallSortLds L;
    const int t = threadIdx.x;
    for (int i = t; i < n; i += kSmallSortThreads) {
        L.kb[0][i] = keys_in[i];
        L.pb[0][i] = pos_in[i];
    }
    const int src = lds_radix_sort(L, n, bits);
    for (int i = t; i < n; i += kSmallSortThreads) {
        keys_out[i] = L.kb[src][i];
        pos_out[i] = L.pb[src][i];
    }
}

// The whole grouping for up to kSmallSort positions and tables of up to kSmallVocab rows in one
// workgroup (C5: 4096 positions, 32000 rows): the check word and the V + 1 counts cleared, the
// keys (ID, or V for an invalid ID) and positions built in LDS, sorted there, and each ID's
// range read off the sorted keys (offsets[k] = its first slot, counts[k] = its run length; the
// counts of IDs that do not occur stay 0) -- one launch for what the general path does in six
// (clear, keys, sort passes, a multi-tile scan of the counts).
constexpr int64_t kSmallVocab = 1 << 16;
template <typename Idx>
__global__ void __launch_bounds__(kSmallSortThreads)
small_grouping_kernel(const Idx* __restrict__ ids, int n, int64_t vocab, int bits, uint32_t* __restrict__ counts,
                      uint32_t* __restrict__ offsets, uint32_t* __restrict__ pos_out, int* __restrict__ flag) {
    __shared__ SmallSortLds L;
    const int t = threadIdx.x;
    for (int64_t i = t; i <= vocab; i += kSmallSortThreads) counts[i] = 0;
    if (t == 0) *flag = 0;
    __syncthreads();  // the clears come before any count or check-word write below
    for (int i = t; i < n; i += kSmallSortThreads) {
        const int64_t id = static_cast<int64_t>(ids[i]);
        const bool valid = id >= 0 && id < vocab;
        L.kb[0][i] = static_cast<uint32_t>(valid ? id : vocab);
        L.pb[0][i] = static_cast<uint32_t>(i);
        if (!valid) *flag = 1;
    }
    const int src = lds_radix_sort(L, n, bits);
    // runs of equal keys: the last position of a run finds the run's first by a binary search of the
    // sorted keys (in LDS) and writes both
    const uint32_t* keys = L.kb[src];
    for (int i = t; i < n; i += kSmallSortThreads) {
        const uint32_t k = keys[i];
        pos_out[i] = L.pb[src][i];
        if (i == n - 1 || keys[i + 1] != k) {
            int lo = 0, hi = i;  // first index in [0, i] holding k
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                if (keys[mid] < k) lo = mid + 1;
                else hi = mid;
            }
            offsets[k] = static_cast<uint32_t>(lo);
            counts[k] = static_cast<uint32_t>(i + 1 - lo);
        }
    }
}

// One workgroup per table row v: the positions of ID v are sorted[offsets[v] .. + counts[v]),
// summed in that order (offsets[v] is read only where counts[v] > 0: the one-workgroup grouping
// leaves the offsets of absent IDs unwritten).
template <typename T>
__global__ void __launch_bounds__(kEmbThreads)
embedding_dense_grad_kernel(const T* __restrict__ grad, const uint32_t* __restrict__ sorted_pos,
                            const uint32_t* __restrict__ counts, const uint32_t* __restrict__ offsets,
                            T* __restrict__ dw, int64_t width, uint64_t padding, int scale, bool vec) {
    constexpr int P = Chunk<T>::kPer;
    const int64_t v = blockIdx.x;
    const uint32_t cnt = (static_cast<uint64_t>(v) == padding) ? 0u : counts[v];
    const uint32_t off = cnt ? offsets[v] : 0u;
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
    uint32_t *keys, *pos, *keys_alt, *pos_alt, *counts, *offsets, *hist, *scan;
};

size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

int key_bits(int64_t vocab) {  // bits holding keys 0..vocab (vocab itself marks invalid IDs)
    int b = 1;
    while (b < 32 && (int64_t(1) << b) <= vocab) ++b;
    return b;
}

int64_t sort_tiles(int64_t tokens) { return (tokens + kSortTile - 1) / kSortTile; }

size_t scan_bytes_for(int64_t tokens, int64_t vocab) {
    const int64_t hist = kDigits * std::max<int64_t>(sort_tiles(tokens), 1);
    return align256(4 * std::max(scan_scratch_elems(hist), scan_scratch_elems(vocab + 1)) + 256);
}

EmbWs carve(void* base, int64_t tokens, int64_t vocab) {
    EmbWs w{};
    char* p = static_cast<char*>(base);
    w.flag = reinterpret_cast<int*>(p);
    p += 256;
    const size_t tok = align256(static_cast<size_t>(tokens) * 4), voc = align256(static_cast<size_t>(vocab + 1) * 4);
    w.keys = reinterpret_cast<uint32_t*>(p); p += tok;
    w.pos = reinterpret_cast<uint32_t*>(p); p += tok;
    w.keys_alt = reinterpret_cast<uint32_t*>(p); p += tok;
    w.pos_alt = reinterpret_cast<uint32_t*>(p); p += tok;
    w.counts = reinterpret_cast<uint32_t*>(p); p += voc;
    w.offsets = reinterpret_cast<uint32_t*>(p); p += voc;
    w.hist = reinterpret_cast<uint32_t*>(p); p += align256(static_cast<size_t>(kDigits * sort_tiles(tokens)) * 4);
    w.scan = reinterpret_cast<uint32_t*>(p);
    return w;
}

// Stable sort of (keys, pos) by the low `bits` bits of the keys, 8 bits per pass (in one workgroup
// up to kSmallSort positions); returns the buffers that hold the result (the input pair or the
// alternate pair).
void sort_pairs(EmbWs& w, int64_t tokens, int bits, hipStream_t s, uint32_t** keys_out, uint32_t** pos_out) {
    uint32_t *k0 = w.keys, *p0 = w.pos, *k1 = w.keys_alt, *p1 = w.pos_alt;
    if (tokens <= kSmallSort) {
        hipLaunchKernelGGL(small_sort_kernel, dim3(1), dim3(kSmallSortThreads), 0, s, k0, p0, static_cast<int>(tokens),
                           bits, k1, p1);
        *keys_out = k1;
        *pos_out = p1;
        return;
    }
    const int64_t tiles = sort_tiles(tokens);
    for (int shift = 0; shift < bits; shift += 8) {
        hipLaunchKernelGGL(digit_hist_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kSortThreads), 0, s, k0, tokens,
                           shift, w.hist, static_cast<int>(tiles));
        scan_exclusive(w.hist, w.hist, kDigits * tiles, w.scan, s);
        hipLaunchKernelGGL(digit_scatter_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kSortThreads), 0, s, k0, p0,
                           tokens, shift, w.hist, static_cast<int>(tiles), k1, p1);
        std::swap(k0, k1);
        std::swap(p0, p1);
    }
    *keys_out = k0;
    *pos_out = p0;
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
void launch_dense_grad(const void* grad, const EmbWs& w, const uint32_t* pos_sorted, void* dw, int64_t vocab,
                       int64_t width, uint64_t padding, int scale, hipStream_t s) {
    const bool vec = width % Chunk<T>::kPer == 0 && aligned16({grad, dw});
    hipLaunchKernelGGL(embedding_dense_grad_kernel<T>, dim3(static_cast<unsigned>(vocab)), dim3(kEmbThreads), 0, s,
                       static_cast<const T*>(grad), pos_sorted, w.counts, w.offsets, static_cast<T*>(dw), width,
                       padding, scale, vec);
}

}  // namespace

size_t embedding_workspace_bytes(int64_t tokens, int64_t vocab, bool backward) {
    if (!backward) return 256;
    return 256 + 4 * align256(static_cast<size_t>(tokens) * 4) + 2 * align256(static_cast<size_t>(vocab + 1) * 4) +
           align256(static_cast<size_t>(kDigits * sort_tiles(tokens)) * 4) + scan_bytes_for(tokens, vocab);
}

hipError_t embedding(const void* table, int id_bytes, const void* ids, void* out, int64_t tokens, int64_t vocab,
                     int64_t row_bytes, int* flag, int seq, hipStream_t s) {
    if (tokens > 0 && row_bytes > 0) {
        if (id_bytes == 8) gather_by_unit<int64_t>(table, ids, out, tokens, vocab, row_bytes, flag, seq, s);
        else gather_by_unit<int32_t>(table, ids, out, tokens, vocab, row_bytes, flag, seq, s);
    }
    return hipGetLastError();
}

namespace {

bool small_grouping(int64_t tokens, int64_t vocab) {
    return tokens > 0 && tokens <= kSmallSort && vocab < kSmallVocab;
}

int scan_launches(int64_t n) {
    if (n <= 0) return 0;
    const int64_t tiles = (n + kScanTile - 1) / kScanTile;
    return tiles == 1 ? 1 : 2 + scan_launches(tiles);
}

}  // namespace

int embedding_backward_launches(int64_t tokens, int64_t vocab, int64_t width) {
    const int dense = vocab > 0 && width > 0 ? 1 : 0;
    if (small_grouping(tokens, vocab)) return 1 + dense;
    int n = 1 + scan_launches(vocab + 1) + dense;  // clear, count scan, dense rows
    if (tokens > 0) {
        n += 1;  // keys
        if (tokens <= kSmallSort) n += 1;
        else n += (key_bits(vocab) + 7) / 8 * (2 + scan_launches(kDigits * sort_tiles(tokens)));
    }
    return n;
}

hipError_t embedding_backward(int dtype, const void* grad, int id_bytes, const void* ids, void* dw, int64_t tokens,
                              int64_t vocab, int64_t width, uint64_t padding, int scale, void* workspace,
                              hipStream_t s) {
    EmbWs w = carve(workspace, tokens, vocab);
    if (small_grouping(tokens, vocab)) {
        if (id_bytes == 8)
            hipLaunchKernelGGL(small_grouping_kernel<int64_t>, dim3(1), dim3(kSmallSortThreads), 0, s,
                               static_cast<const int64_t*>(ids), static_cast<int>(tokens), vocab, key_bits(vocab),
                               w.counts, w.offsets, w.pos_alt, w.flag);
        else
            hipLaunchKernelGGL(small_grouping_kernel<int32_t>, dim3(1), dim3(kSmallSortThreads), 0, s,
                               static_cast<const int32_t*>(ids), static_cast<int>(tokens), vocab, key_bits(vocab),
                               w.counts, w.offsets, w.pos_alt, w.flag);
        if (vocab > 0 && width > 0) {
            if (dtype == 1) launch_dense_grad<_Float16>(grad, w, w.pos_alt, dw, vocab, width, padding, scale, s);
            else if (dtype == 27) launch_dense_grad<uint16_t>(grad, w, w.pos_alt, dw, vocab, width, padding, scale, s);
            else launch_dense_grad<float>(grad, w, w.pos_alt, dw, vocab, width, padding, scale, s);
        }
        return hipGetLastError();
    }
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
    }
    uint32_t *keys_sorted = w.keys, *pos_sorted = w.pos;
    if (tokens > 0) sort_pairs(w, tokens, key_bits(vocab), s, &keys_sorted, &pos_sorted);
    scan_exclusive(w.counts, w.offsets, vocab + 1, w.scan, s);
    if (vocab > 0 && width > 0) {
        if (dtype == 1) launch_dense_grad<_Float16>(grad, w, pos_sorted, dw, vocab, width, padding, scale, s);
        else if (dtype == 27) launch_dense_grad<uint16_t>(grad, w, pos_sorted, dw, vocab, width, padding, scale, s);
        else launch_dense_grad<float>(grad, w, pos_sorted, dw, vocab, width, padding, scale, s);
    }
    return hipGetLastError();
}

}  // namespace hk
