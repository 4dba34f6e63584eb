// hk_rmsnorm.hip — RMSNorm forward and backward for gfx950.
//
// Semantics (reference, paths relative to the shuqi2077/rust-ascend root):
//   forward  rust-ascend-compiler/src/ascend/row_programs.rs:144-151
//            rstd = 1/sqrt(sum(x^2)/W + eps); y = (x*rstd)*w
//   backward row_programs.rs:208-217 (input) and :200-207 (weight contributions)
//            g = dy*w; mean = sum(g*x)/W; dx = (g - x*(mean*rstd^2))*rstd
//            dw[c] = sum_rows (x*rstd)*dy, the column sum of normalization.rs:95-114
//
// Layout: x/y/dy/dx are [rows, W] row-major in F32 or BF16; w is F32 [W]; rstd is F32
// [rows]; dw is F32 [W]. HBM-bound: per row the forward moves W*(2 sizeof(T)) bytes
// and the backward W*(3 sizeof(T)) bytes.
//
// Forward fast path (W % 8 == 0, W <= 4096): one wavefront owns one row; lane l owns the
// 8-element chunks l, l+64, l+128, ... (16-byte loads for BF16, fully coalesced), so a row is
// MAXJ chunks per lane held in registers; the row sum is a butterfly across the wave.
// Split path (W % 8 == 0, W <= 16384: the backward at every such width, the forward above 4096):
// a row spread over several waves of a workgroup that exchange their part sums through LDS (see
// rms_fwd_split / rms_bwd_split). The backward writes one FP64 dw partial row per workgroup and a
// second kernel sums the partials in a fixed order: deterministic, no atomics.
//
// General path (any positive W): the same math with one element per lane-step and the
// row re-read from cache for the second pass; dw comes from a column-parallel kernel.
#include "hk_common.hpp"
#include "hk_kernels.hpp"

#include <algorithm>
#include <initializer_list>

namespace hk {

namespace {

constexpr int kRowsThreads = 256;  // 4 waves per workgroup (forward)

// Eight elements kept in their storage form between the two passes over a row
// (4 VGPRs for BF16, 8 for F32) and widened to float on use.
template <typename T> struct Raw8;
template <> struct Raw8<uint16_t> {
    u32x4_t w;
    __device__ __forceinline__ void load(const uint16_t* p) { w = stream_load(reinterpret_cast<const u32x4_t*>(p)); }
    // Opaque to the optimizer: the widening below is recomputed after this point instead
    // of being kept live (as 8 extra VGPRs per chunk) across the row reduction.
    __device__ __forceinline__ void pin() { asm volatile("" : "+v"(w)); }
    __device__ __forceinline__ void get(float (&v)[8]) const {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = bf16lo(w[i]);
            v[2 * i + 1] = bf16hi(w[i]);
        }
    }
};
template <> struct Raw8<float> {
    f32x4_t a, b;
    __device__ __forceinline__ void load(const float* p) {
        a = stream_load(reinterpret_cast<const f32x4_t*>(p));
        b = stream_load(reinterpret_cast<const f32x4_t*>(p + 4));
    }
    __device__ __forceinline__ void pin() {}
    __device__ __forceinline__ void get(float (&v)[8]) const {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = a[i];
            v[4 + i] = b[i];
        }
    }
};

// One wavefront per row and one row per wavefront (no grid-stride loop): the row is held
// in its storage form (32 VGPRs for a 4096-wide BF16 row), so the kernel runs at high
// occupancy and every wave has its whole row of loads in flight at once. The workgroup
// stages w in LDS with loads issued together with the rows', so a row costs one memory
// round trip, not two (x, then w after the reduction).
template <typename T, int MAXJ, bool FULL>
__global__ void __launch_bounds__(kRowsThreads)
rms_fwd_fast(const T* __restrict__ x, const float* __restrict__ w, T* __restrict__ y,
             float* __restrict__ rstd, int64_t rows, int width, float eps) {
    extern __shared__ float w_lds[];
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const bool active = row < rows;
    const int chunks = width >> 3;
    const T* xr = x + row * width;
    Raw8<T> xs[MAXJ];
    if (active) {
#pragma unroll
        for (int j = 0; j < MAXJ; ++j) {
            const int c = lane + 64 * j;
            if (FULL || c < chunks) xs[j].load(xr + 8 * c);
        }
    }
    for (int c = threadIdx.x; c < chunks; c += kRowsThreads) {
        float wv[8];
        load8(w + 8 * c, wv);
        store8(w_lds + 8 * c, wv);
    }
    __syncthreads();
    if (!active) return;
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < MAXJ; ++j) {
        const int c = lane + 64 * j;
        if (FULL || c < chunks) {
            float v[8];
            xs[j].get(v);
#pragma unroll
            for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
        }
    }
    ss = wave_sum(ss);
    const float r = 1.0f / sqrtf(ss * (1.0f / static_cast<float>(width)) + eps);
    T* yr = y + row * width;
#pragma unroll
    for (int j = 0; j < MAXJ; ++j) {
        const int c = lane + 64 * j;
        if (FULL || c < chunks) {
            float v[8], wv[8], o[8];
            xs[j].pin();
            xs[j].get(v);
            load8(w_lds + 8 * c, wv);
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = (v[e] * r) * wv[e];
            store8_stream(yr + 8 * c, o);
        }
    }
    if (lane == 0) rstd[row] = r;
}

// Row-split kernels (W % 8 == 0, W <= 16384). A row of `chunks` = W/8 eight-element chunks is
// spread over QN waves ("parts"), each holding CPL chunks per lane: lane l of part q owns the
// chunks 64 CPL q + l + 64 j (j < CPL) that lie below `chunks` (all of them when FULL). A
// workgroup holds G row groups of QN waves (QN G <= 16, one workgroup per CU, so up to four waves
// per SIMD); the waves of a row group walk the same rows in a grid-stride loop. The row's sum (of
// squares in the forward, of dy*w*x in the backward) is the sum of the parts' sums, exchanged
// through LDS without a barrier: each wave posts its part's sum, tagged with the row's sequence
// number, as one 64-bit LDS word into one of two slots, and reads the QN posts of the row once
// their tags match. Every wave adds the QN posts in part order, so all of them compute the same
// row statistic. A wave posts row k+2 into the slot of row k only after it has read every post of
// row k+1, each made after its author had read row k's posts, so no post is overwritten before it
// is read; all waves of a workgroup are resident together and every wave posts before it waits,
// so every wait ends (the spin is also bounded).
// Why split rows: a row per wave needs the whole row in flight and, in the backward, all of the
// row's FP64 dγ sums (64 per lane at W = 4096: ~230 registers, one wave per SIMD), and four waves
// per SIMD stream faster than one wave with two to four rows in flight. C2 (16384 x 4096 BF16)
// backward: 71-72 us against 74-76 us for the row-per-wave kernel on the same box; W = 8192 BF16
// ran at 1.7 TB/s (backward) and 2.9 TB/s (forward) on the column-parallel path before.
constexpr int kSplitThreads = 1024;
constexpr int kSplitMaxWaves = 16;
constexpr int kSplitMaxChunks = 2048;  // W <= 16384
constexpr int kPostBytes = 2 * kSplitMaxWaves * 8;  // [G][2][QN] 64-bit posts, G * QN <= 16

struct SplitShape {
    int chunks;  // W / 8
    int qn;      // waves per row
    int groups;  // row groups per workgroup
    int cpl;     // chunks per lane per wave
    bool full;   // every lane owns CPL chunks
};

// Two chunks per lane for rows of at least 256 chunks (W >= 2048), else one, and enough waves to
// cover the row; W = 2048 keeps one chunk per lane over four waves, the split measured there.
SplitShape split_shape(int64_t width) {
    SplitShape sh;
    sh.chunks = static_cast<int>(width / 8);
    sh.cpl = sh.chunks >= 256 && width != 2048 ? 2 : 1;
    const int per_wave = 64 * sh.cpl;
    sh.qn = (sh.chunks + per_wave - 1) / per_wave;
    sh.groups = kSplitMaxWaves / sh.qn;
    sh.full = sh.chunks == sh.qn * per_wave;
    return sh;
}

// Failure report of the exchange: a wave whose wait for a partner's post runs out of spins goes
// on with the stale post (wrong results, no hang) and writes the call's sequence number into the
// check word, which the host reads after a synchronous call.
struct SplitCheck {
    int* flag;
    int seq;
    int spin_limit;
};

// Sum over the QN parts of row sequence k of group g (every wave of the group calls it with its
// own part's value).
__device__ __forceinline__ float split_row_sum(uint64_t* post, int g, int qn, int q, int64_t k, int lane, float part,
                                               const SplitCheck& chk) {
    const uint32_t tag = static_cast<uint32_t>(k) + 1;
    uint64_t* slots = post + (2 * g + static_cast<int>(k & 1)) * qn;
    // single 64-bit LDS accesses (tag and value together); the atomics keep the compiler from
    // caching or reordering them
    if (lane == 0)
        __hip_atomic_store(&slots[q], (static_cast<uint64_t>(tag) << 32) | __float_as_uint(part), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_WORKGROUP);
    float total = 0.0f;
    bool stale = false;
    for (int p = 0; p < qn; ++p) {
        uint64_t val;
        int spins = 0;
        do {
            val = __hip_atomic_load(&slots[p], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        } while (static_cast<uint32_t>(val >> 32) != tag && ++spins < chk.spin_limit);
        stale |= static_cast<uint32_t>(val >> 32) != tag;
        const float v = __uint_as_float(static_cast<uint32_t>(val));
        total = p == 0 ? v : total + v;
    }
    if (stale && lane == 0) *chk.flag = chk.seq;
    return total;
}

// LDS: the posts, then w [W] F32, then (backward with G > 1) the FP64 group-combine row [W].
__host__ __device__ constexpr size_t split_lds_bytes(int chunks, int groups, bool bwd) {
    return kPostBytes + static_cast<size_t>(chunks) * 8 * 4 + (bwd && groups > 1 ? static_cast<size_t>(chunks) * 8 * 8 : 0);
}

template <typename T, int CPL, bool FULL>
__global__ void __launch_bounds__(kSplitThreads)
rms_fwd_split(const T* __restrict__ x, const float* __restrict__ w, T* __restrict__ y, float* __restrict__ rstd,
              int64_t rows, int chunks, int qn, int groups, float eps, SplitCheck chk) {
    extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
    uint64_t* post = reinterpret_cast<uint64_t*>(lds_raw);
    float* w_lds = reinterpret_cast<float*>(lds_raw + kPostBytes);
    const int W = 8 * chunks;
    const int lane = threadIdx.x & 63;
    const int v = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = v / qn, q = v - g * qn;
    if (threadIdx.x < kPostBytes / 8) post[threadIdx.x] = 0;
    for (int c = threadIdx.x; c < W; c += blockDim.x) w_lds[c] = w[c];
    __syncthreads();
    const float inv_w = 1.0f / static_cast<float>(W);
    const int64_t stride = static_cast<int64_t>(gridDim.x) * groups;
    const int64_t first = static_cast<int64_t>(blockIdx.x) * groups + g;
    const int64_t n = first < rows ? (rows - 1 - first) / stride + 1 : 0;
    const int cbase = 64 * CPL * q + lane;
    for (int64_t k = 0; k < n; ++k) {
        const int64_t row = first + k * stride;
        const T* xr = x + row * W;
        Raw8<T> xs[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j)
            if (FULL || cbase + 64 * j < chunks) xs[j].load(xr + 8 * (cbase + 64 * j));
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            if (FULL || cbase + 64 * j < chunks) {
                float xv[8];
                xs[j].get(xv);
#pragma unroll
                for (int e = 0; e < 8; ++e) ss += xv[e] * xv[e];
            }
        }
        ss = wave_sum(ss);
        const float total = split_row_sum(post, g, qn, q, k, lane, ss, chk);
        const float r = 1.0f / sqrtf(total * inv_w + eps);
        T* yr = y + row * W;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = cbase + 64 * j;
            if (FULL || c < chunks) {
                float xv[8], wv[8], o[8];
                xs[j].pin();
                xs[j].get(xv);
                load8(w_lds + 8 * c, wv);
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e] = (xv[e] * r) * wv[e];
                store8_stream(yr + 8 * c, o);
            }
        }
        if (lane == 0 && q == 0) rstd[row] = r;
    }
}

// v as a store of type T keeps it (BF16: rounded to nearest even; F32: v itself) plus r: the
// empty asm makes v a finished value, so the product that formed it is not contracted into the
// add (the unfused composition stores v, then adds).
template <typename T>
__device__ __forceinline__ float add_stored(float v, float r) {
    float s;
    if constexpr (sizeof(T) == 2) s = round_bf16(v);
    else s = v;
    asm volatile("" : "+v"(s));
    return s + r;
}

// RES: dx = res + (the row's dx as stored), added in F32 and stored again -- the backward followed
// by a residual add of the stored dx, in one pass (a decoder layer's residual branch gradient).
template <typename T, int CPL, bool FULL, bool RES>
__global__ void __launch_bounds__(kSplitThreads)
rms_bwd_split(const T* __restrict__ x, const float* __restrict__ w, const T* __restrict__ dy,
              const float* __restrict__ rstd, const T* __restrict__ res, T* __restrict__ dx,
              double* __restrict__ partial, int64_t rows, int chunks, int qn, int groups, SplitCheck chk) {
    extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
    uint64_t* post = reinterpret_cast<uint64_t*>(lds_raw);
    float* w_lds = reinterpret_cast<float*>(lds_raw + kPostBytes);
    const int W = 8 * chunks;
    double* p_lds = reinterpret_cast<double*>(lds_raw + kPostBytes + static_cast<size_t>(W) * 4);
    const int lane = threadIdx.x & 63;
    const int v = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = v / qn, q = v - g * qn;
    if (threadIdx.x < kPostBytes / 8) post[threadIdx.x] = 0;
    for (int c = threadIdx.x; c < W; c += blockDim.x) w_lds[c] = w[c];
    double acc[CPL][8];
#pragma unroll
    for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[j][e] = 0.0;
    __syncthreads();
    const float inv_w = 1.0f / static_cast<float>(W);
    const int64_t stride = static_cast<int64_t>(gridDim.x) * groups;
    const int64_t first = static_cast<int64_t>(blockIdx.x) * groups + g;
    const int64_t n = first < rows ? (rows - 1 - first) / stride + 1 : 0;
    const int cbase = 64 * CPL * q + lane;
    for (int64_t k = 0; k < n; ++k) {
        const int64_t row = first + k * stride;
        const float r = rstd[row];
        const T* xr = x + row * W;
        const T* gr = dy + row * W;
        Raw8<T> xs[CPL], gs[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = cbase + 64 * j;
            if (FULL || c < chunks) {
                xs[j].load(xr + 8 * c);
                gs[j].load(gr + 8 * c);
            }
        }
        const double rd = r;
        float dot = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = cbase + 64 * j;
            if (FULL || c < chunks) {
                float xv[8], gv[8], wv[8];
                xs[j].get(xv);
                gs[j].get(gv);
                load8(w_lds + 8 * c, wv);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    dot += (gv[e] * wv[e]) * xv[e];
                    // dγ sums in FP64: x * dy is exact in FP32 for BF16 storage and in FP64 for
                    // F32, so each term x*dy*rstd is formed exactly in the fused multiply-add and
                    // the sums carry only FP64 rounding (FP32 sums put C2's error at 0.8-1.6e-4 of
                    // |dγ| + 1e-3 rms(dγ), against 3.9e-5 now, the part due to rstd being F32).
                    if constexpr (sizeof(T) == 2)
                        acc[j][e] = __builtin_fma(static_cast<double>(xv[e] * gv[e]), rd, acc[j][e]);
                    else
                        acc[j][e] = __builtin_fma(static_cast<double>(xv[e]) * gv[e], rd, acc[j][e]);
                }
            }
        }
        dot = wave_sum(dot);
        Raw8<T> rs[RES ? CPL : 1];
        if constexpr (RES) {  // issued before the exchange wait, used at the stores
#pragma unroll
            for (int j = 0; j < CPL; ++j)
                if (FULL || cbase + 64 * j < chunks) rs[j].load(res + row * W + 8 * (cbase + 64 * j));
        }
        const float total = split_row_sum(post, g, qn, q, k, lane, dot, chk);
        const float corr = (total * inv_w) * (r * r);
        T* dr = dx + row * W;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = cbase + 64 * j;
            if (FULL || c < chunks) {
                float xv[8], gv[8], wv[8], o[8];
                xs[j].pin();
                gs[j].pin();
                xs[j].get(xv);
                gs[j].get(gv);
                load8(w_lds + 8 * c, wv);
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e] = (gv[e] * wv[e] - xv[e] * corr) * r;
                if constexpr (RES) {
                    float rv[8];
                    rs[j].get(rv);
#pragma unroll
                    for (int e = 0; e < 8; ++e) o[e] = add_stored<T>(o[e], rv[e]);
                }
                store8_stream(dr + 8 * c, o);
            }
        }
    }
    // The workgroup's FP64 partial row: the row groups' sums combined in group order through LDS
    // (one group: each wave writes its own columns).
    double* out = partial + static_cast<int64_t>(blockIdx.x) * W;
    if (groups == 1) {
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = cbase + 64 * j;
            if (FULL || c < chunks)
#pragma unroll
                for (int e = 0; e < 8; ++e) out[8 * c + e] = acc[j][e];
        }
        return;
    }
    for (int src = 0; src < groups; ++src) {
        if (g == src) {
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const int c = cbase + 64 * j;
                if (FULL || c < chunks)
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        double* p = &p_lds[8 * c + e];
                        *p = (src == 0) ? acc[j][e] : (*p + acc[j][e]);
                    }
            }
        }
        __syncthreads();
    }
    for (int c = threadIdx.x; c < W; c += blockDim.x) out[c] = p_lds[c];
}

// dw[c] = sum over p of the FP64 partial[p][c] for parts <= 256 and width % 8 == 0 (the fast and
// split backward kernels): workgroup b covers columns 8b .. 8b+7; thread (slice, pair) loads the
// 16-byte column pair of partial rows slice, slice + 64, slice + 128, slice + 192 at once and adds
// them in that order, then the 64 slice sums are combined by a pairwise tree in LDS. The order is
// sum_partials' (below) for these shapes, so the result is bit-identical to it; C2: 3.1-3.9 us
// against 3.8-4.8 us.
typedef double f64x2_t __attribute__((ext_vector_type(2)));
__global__ void __launch_bounds__(256)
sum_partials8(const double* __restrict__ partial, int parts, int width, float* __restrict__ dw) {
    __shared__ f64x2_t red[64][4];
    const int pr = threadIdx.x & 3, slice = threadIdx.x >> 2;
    const int col0 = blockIdx.x * 8 + pr * 2;
    f64x2_t a[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int p = slice + 64 * k;
        a[k] = p < parts ? *reinterpret_cast<const f64x2_t*>(partial + static_cast<int64_t>(p) * width + col0)
                         : f64x2_t{0.0, 0.0};
    }
    f64x2_t s = {0.0, 0.0};
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (slice + 64 * k < parts) s += a[k];
    red[slice][pr] = s;
    __syncthreads();
    for (int half = 32; half >= 1; half >>= 1) {
        if (slice < half) red[slice][pr] += red[slice + half][pr];
        __syncthreads();
    }
    if (slice == 0) {
        dw[col0] = static_cast<float>(red[0][pr][0]);
        dw[col0 + 1] = static_cast<float>(red[0][pr][1]);
    }
}

// dw[c] = sum over p of the FP64 partial[p][c]. A workgroup covers 16 columns: thread t takes the
// four columns 4 (t % 4) .. +3 of its slice of partial rows, p = t/4, t/4 + 64, ... (one row each
// for 64 partials, four for C2's 256), so every load of the kernel is issued at once; the 64 slice
// sums of each column are then combined in LDS by a fixed pairwise tree. The order is fixed for
// given (parts, width) and the sums are kept in double, so this stage adds no rounding beyond the
// final conversion to F32. On C2 (256 partials x 4096) it takes 4.2 us, as the former 64-column
// workgroups did while leaving 3/4 of the CUs idle: the time is mostly the launch itself.
constexpr int kSumSlices = 64;
__global__ void __launch_bounds__(256)
sum_partials(const double* __restrict__ partial, int parts, int width, float* __restrict__ dw) {
    __shared__ double red[kSumSlices][16];
    const int quad = threadIdx.x & 3, slice = threadIdx.x >> 2;
    const int groups = (width + 15) / 16;
    for (int grp = blockIdx.x; grp < groups; grp += gridDim.x) {  // uniform per workgroup
        const int col0 = grp * 16 + quad * 4;
        double s[4] = {0.0, 0.0, 0.0, 0.0};
        for (int p = slice; p < parts; p += kSumSlices)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (col0 + e < width) s[e] += partial[static_cast<int64_t>(p) * width + col0 + e];
#pragma unroll
        for (int e = 0; e < 4; ++e) red[slice][quad * 4 + e] = s[e];
        __syncthreads();
        for (int half = kSumSlices / 2; half >= 1; half >>= 1) {
            if (slice < half)
#pragma unroll
                for (int e = 0; e < 4; ++e) red[slice][quad * 4 + e] += red[slice + half][quad * 4 + e];
            __syncthreads();
        }
        if (slice == 0)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (col0 + e < width) dw[col0 + e] = static_cast<float>(red[0][quad * 4 + e]);
        __syncthreads();  // red is rewritten by the next group
    }
}

template <typename T>
__global__ void __launch_bounds__(kRowsThreads)
rms_fwd_general(const T* __restrict__ x, const float* __restrict__ w, T* __restrict__ y,
                float* __restrict__ rstd, int64_t rows, int64_t width, float eps) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int waves_per_block = blockDim.x >> 6;
    for (int64_t row = static_cast<int64_t>(blockIdx.x) * waves_per_block + wave; row < rows;
         row += static_cast<int64_t>(gridDim.x) * waves_per_block) {
        const T* xr = x + row * width;
        float ss = 0.0f;
        for (int64_t c = lane; c < width; c += 64) {
            const float v = Elem<T>::load(xr, c);
            ss += v * v;
        }
        ss = wave_sum(ss);
        const float r = 1.0f / sqrtf(ss / static_cast<float>(width) + eps);
        T* yr = y + row * width;
        for (int64_t c = lane; c < width; c += 64) Elem<T>::store(yr, c, (Elem<T>::load(xr, c) * r) * w[c]);
        if (lane == 0) rstd[row] = r;
    }
}

template <typename T>
__global__ void __launch_bounds__(kRowsThreads)
rms_bwd_dx_general(const T* __restrict__ x, const float* __restrict__ w, const T* __restrict__ dy,
                   const float* __restrict__ rstd, const T* __restrict__ res, T* __restrict__ dx, int64_t rows,
                   int64_t width) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int waves_per_block = blockDim.x >> 6;
    for (int64_t row = static_cast<int64_t>(blockIdx.x) * waves_per_block + wave; row < rows;
         row += static_cast<int64_t>(gridDim.x) * waves_per_block) {
        const T* xr = x + row * width;
        const T* gr = dy + row * width;
        const float r = rstd[row];
        float dot = 0.0f;
        for (int64_t c = lane; c < width; c += 64)
            dot += (Elem<T>::load(gr, c) * w[c]) * Elem<T>::load(xr, c);
        dot = wave_sum(dot);
        const float corr = (dot / static_cast<float>(width)) * (r * r);
        T* dr = dx + row * width;
        for (int64_t c = lane; c < width; c += 64) {
            const float v = (Elem<T>::load(gr, c) * w[c] - Elem<T>::load(xr, c) * corr) * r;
            Elem<T>::store(dr, c, res ? add_stored<T>(v, Elem<T>::load(res + row * width, c)) : v);
        }
    }
}

// partial[chunk][c] = sum over the chunk's rows of x*dy*rstd, rows ascending, in FP64 (each term
// exact, as in the fast kernel).
template <typename T>
__global__ void __launch_bounds__(256)
rms_bwd_dw_general(const T* __restrict__ x, const T* __restrict__ dy, const float* __restrict__ rstd,
                   double* __restrict__ partial, int64_t rows, int64_t width, int64_t rows_per_chunk) {
    const int64_t col = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t chunk = blockIdx.y;
    if (col >= width) return;
    const int64_t r0 = chunk * rows_per_chunk;
    const int64_t r1 = (r0 + rows_per_chunk < rows) ? r0 + rows_per_chunk : rows;
    double s = 0.0;
    for (int64_t r = r0; r < r1; ++r)
        s = __builtin_fma(static_cast<double>(Elem<T>::load(x, r * width + col)) * Elem<T>::load(dy, r * width + col),
                          static_cast<double>(rstd[r]), s);
    partial[chunk * width + col] = s;
}

__global__ void __launch_bounds__(256) fill_zero_f32(float* p, int64_t n) {
    for (int64_t i = flat_begin(256); i < n; i += flat_stride(256)) p[i] = 0.0f;
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

bool fast_rows(int64_t width, std::initializer_list<const void*> ptrs) {
    if (width % 8 != 0 || width > 4096) return false;
    for (const void* p : ptrs)
        if (!aligned16(p)) return false;
    return true;
}

int grid_for_rows(int64_t rows, int waves_per_block, int cap) {
    int64_t g = (rows + waves_per_block - 1) / waves_per_block;
    if (g > cap) g = cap;
    return g < 1 ? 1 : static_cast<int>(g);
}

template <typename T, int MAXJ>
void launch_fwd_fast(const void* x, const float* w, void* y, float* rstd, int64_t rows, int width,
                     float eps, hipStream_t s) {
    // One row per wave. Launches take at most 2^22 rows each (2^20 workgroups), so a launch's
    // work items stay within a dispatch's 32-bit count; C2's 16384 rows are one launch.
    constexpr int64_t kRowsPerLaunch = int64_t{1} << 22;
    auto kernel = width == 512 * MAXJ ? rms_fwd_fast<T, MAXJ, true> : rms_fwd_fast<T, MAXJ, false>;
    for (int64_t r0 = 0; r0 < rows; r0 += kRowsPerLaunch) {
        const int64_t n = rows - r0 < kRowsPerLaunch ? rows - r0 : kRowsPerLaunch;
        const int64_t grid = (n + kRowsThreads / 64 - 1) / (kRowsThreads / 64);
        hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(grid)), dim3(kRowsThreads),
                           static_cast<size_t>(width) * sizeof(float), s, static_cast<const T*>(x) + r0 * width, w,
                           static_cast<T*>(y) + r0 * width, rstd + r0, n, width, eps);
    }
}

bool split_rows(int64_t width, std::initializer_list<const void*> ptrs) {
    if (width % 8 != 0 || width / 8 > kSplitMaxChunks) return false;
    for (const void* p : ptrs)
        if (!aligned16(p)) return false;
    return true;
}

// One round of workgroups: at most 256 (one per CU), each covering `groups` rows at a time.
int split_grid(int64_t rows, int groups) { return grid_for_rows(rows, groups, 256); }

template <typename T, int CPL>
void launch_split(bool bwd, const SplitShape& sh, int grid, const void* x, const float* w, const void* dy,
                  const float* rstd_in, const void* res, void* out, float* rstd_out, double* partial, int64_t rows,
                  float eps, const SplitCheck& chk, hipStream_t s) {
    const dim3 block(64 * sh.qn * sh.groups);
    const size_t lds = split_lds_bytes(sh.chunks, sh.groups, bwd);
    if (bwd) {
        auto kernel = res ? (sh.full ? rms_bwd_split<T, CPL, true, true> : rms_bwd_split<T, CPL, false, true>)
                          : (sh.full ? rms_bwd_split<T, CPL, true, false> : rms_bwd_split<T, CPL, false, false>);
        hipLaunchKernelGGL(kernel, dim3(grid), block, lds, s, static_cast<const T*>(x), w, static_cast<const T*>(dy),
                           rstd_in, static_cast<const T*>(res), static_cast<T*>(out), partial, rows, sh.chunks, sh.qn,
                           sh.groups, chk);
    } else {
        auto kernel = sh.full ? rms_fwd_split<T, CPL, true> : rms_fwd_split<T, CPL, false>;
        hipLaunchKernelGGL(kernel, dim3(grid), block, lds, s, static_cast<const T*>(x), w, static_cast<T*>(out),
                           rstd_out, rows, sh.chunks, sh.qn, sh.groups, eps, chk);
    }
}

template <typename T>
void run_split(bool bwd, int64_t width, const void* x, const float* w, const void* dy, const float* rstd_in,
               const void* res, void* out, float* rstd_out, double* partial, int* parts, int64_t rows, float eps,
               RowCheck& rc, hipStream_t s) {
    const SplitShape sh = split_shape(width);
    const int grid = split_grid(rows, sh.groups);
    if (parts) *parts = grid;
    const SplitCheck chk{rc.flag, rc.seq, rc.spin_limit > 0 ? rc.spin_limit : 1};
    rc.used = 1;
    if (sh.cpl == 2)
        launch_split<T, 2>(bwd, sh, grid, x, w, dy, rstd_in, res, out, rstd_out, partial, rows, eps, chk, s);
    else
        launch_split<T, 1>(bwd, sh, grid, x, w, dy, rstd_in, res, out, rstd_out, partial, rows, eps, chk, s);
}

int parts_general(int64_t rows) {
    int64_t parts = (rows + 63) / 64;  // at most 64 rows per column chunk
    if (parts > 512) parts = 512;
    return parts < 1 ? 1 : static_cast<int>(parts);
}

template <typename T>
hipError_t rms_forward_t(const void* x, const float* w, void* y, float* rstd, int64_t rows,
                         int64_t width, float eps, RowCheck& rc, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    if (fast_rows(width, {x, w, y})) {
        const int chunks_per_lane = static_cast<int>((width / 8 + 63) / 64);
        if (chunks_per_lane <= 1) launch_fwd_fast<T, 1>(x, w, y, rstd, rows, (int)width, eps, s);
        else if (chunks_per_lane <= 2) launch_fwd_fast<T, 2>(x, w, y, rstd, rows, (int)width, eps, s);
        else if (chunks_per_lane <= 4) launch_fwd_fast<T, 4>(x, w, y, rstd, rows, (int)width, eps, s);
        else launch_fwd_fast<T, 8>(x, w, y, rstd, rows, (int)width, eps, s);
    } else if (split_rows(width, {x, w, y})) {  // 4096 < W <= 16384
        run_split<T>(false, width, x, w, nullptr, nullptr, nullptr, y, rstd, nullptr, nullptr, rows, eps, rc, s);
    } else {
        const int grid = grid_for_rows(rows, kRowsThreads / 64, 4096);
        hipLaunchKernelGGL((rms_fwd_general<T>), dim3(grid), dim3(kRowsThreads), 0, s,
                           static_cast<const T*>(x), w, static_cast<T*>(y), rstd, rows, width, eps);
    }
    return hipGetLastError();
}

template <typename T>
hipError_t rms_backward_t(const void* x, const float* w, const void* dy, const float* rstd, const void* res, void* dx,
                          float* dw, void* ws, int64_t rows, int64_t width, RowCheck& rc, hipStream_t s) {
    double* workspace = static_cast<double*>(ws);  // the FP64 dγ partials
    if (rows == 0) {
        hipLaunchKernelGGL(fill_zero_f32, dim3(flat_blocks(width, 256)), dim3(256), 0, s, dw, width);
        return hipGetLastError();
    }
    if (split_rows(width, {x, w, dy, dx})) {
        int parts = 0;  // one FP64 partial row per workgroup, at most 256
        run_split<T>(true, width, x, w, dy, rstd, res, dx, nullptr, workspace, &parts, rows, 0.0f, rc, s);
        hipLaunchKernelGGL(sum_partials8, dim3(static_cast<unsigned>(width / 8)), dim3(256), 0, s, workspace, parts,
                           (int)width, dw);
    } else {
        const int grid = grid_for_rows(rows, kRowsThreads / 64, 4096);
        hipLaunchKernelGGL((rms_bwd_dx_general<T>), dim3(grid), dim3(kRowsThreads), 0, s,
                           static_cast<const T*>(x), w, static_cast<const T*>(dy), rstd, static_cast<const T*>(res),
                           static_cast<T*>(dx), rows, width);
        const int parts = parts_general(rows);
        const int64_t per = (rows + parts - 1) / parts;
        hipLaunchKernelGGL((rms_bwd_dw_general<T>), dim3((width + 255) / 256, parts), dim3(256), 0, s,
                           static_cast<const T*>(x), static_cast<const T*>(dy), rstd, workspace, rows,
                           width, per);
        hipLaunchKernelGGL(sum_partials, dim3(flat_blocks((width + 15) / 16, 1)), dim3(256), 0, s, workspace, parts, (int)width, dw);
    }
    return hipGetLastError();
}

}  // namespace

// FP64 dγ partial rows of the backward's path for these operands: one per workgroup of the
// row-split kernels (at most 256), else parts_general's column-chunk count (at most 512).
size_t rms_backward_workspace_bytes(int64_t rows, int64_t width, const void* x, const void* w, const void* dy,
                                    const void* dx) {
    if (rows == 0) return 0;
    const int parts = split_rows(width, {x, w, dy, dx}) ? split_grid(rows, split_shape(width).groups)
                                                        : parts_general(rows);
    return static_cast<size_t>(parts) * static_cast<size_t>(width) * sizeof(double);
}

hipError_t rms_norm_forward(int dtype_bf16, const void* x, const float* w, void* y, float* rstd,
                            int64_t rows, int64_t width, float eps, RowCheck& rc, hipStream_t s) {
    return dtype_bf16 ? rms_forward_t<uint16_t>(x, w, y, rstd, rows, width, eps, rc, s)
                      : rms_forward_t<float>(x, w, y, rstd, rows, width, eps, rc, s);
}

hipError_t rms_norm_backward(int dtype_bf16, const void* x, const float* w, const void* dy,
                             const float* rstd, const void* res, void* dx, float* dw, float* workspace, int64_t rows,
                             int64_t width, RowCheck& rc, hipStream_t s) {
    return dtype_bf16 ? rms_backward_t<uint16_t>(x, w, dy, rstd, res, dx, dw, workspace, rows, width, rc, s)
                      : rms_backward_t<float>(x, w, dy, rstd, res, dx, dw, workspace, rows, width, rc, s);
}

}  // namespace hk
