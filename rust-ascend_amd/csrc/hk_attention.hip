// hk_attention.hip — fused causal / grouped-query attention (forward and backward) for gfx950.
//
// Semantics (reference src/nn/attention.rs:10-80, examples/grouped_attention_tensor.rs:14-44):
//   S = scale * Q K^T (+ causal mask: key_start + j > query_start + i is excluded),
//   P = softmax(S) per query row, O = P V, with query head h reading KV head h / (Hq/Hkv)
//   (heads_programs.rs:5-60). GEMM operands are BF16 and accumulate in FP32; P is rounded to
//   BF16 before P.V (matmul_bf16_fp32 rounds its inputs), softmax statistics are FP32.
//   Backward: dV = P^T dO, dP = dO V^T, dS = P (dP - rowsum(dO o O)), dQ = scale dS K,
//   dK = scale dS^T Q; dS is scaled and rounded to BF16 before its two GEMMs, as the
//   reference's MatmulBf16Fp32Backward chain rounds it.
//   Rows that see no key produce O = 0, lse = -inf and zero gradients (the composed reference
//   would produce NaN from softmax over an all -inf row).
//
// Layout: Q/O/dO [B,Hq,M,D], K/V [B,Hkv,N,D] BF16 row-major; lse and the backward's row
// statistics F32 [B,Hq,M]. Nothing of size M x N is ever materialized.
//
// Forward kernel (FlashAttention-2 style, MI355X-first):
//   * one workgroup = 4 wavefronts = 128 query rows of one (batch, head); K/V tiles of 64 keys
//     are double-buffered in LDS (rows XOR-swizzled in 16-byte chunks) and prefetched from HBM
//     into registers one tile ahead;
//   * each wave computes S^T = K Q^T (Q held in registers as the B operand; v_mfma_f32_32x32x16_bf16
//     for D <= 32, 16x16x32 in the ping-pong kernel for D = 64 / 128), so every lane owns query
//     columns: the row max/sum need one or two lane exchanges instead of a 32-lane reduction;
//   * the FP32 accumulators of S^T, converted to BF16, are directly the B operand of
//     O^T = V^T P^T (the key order inside each MFMA k-group is matched on the V side);
//     V^T comes straight from the row-major V tile through ds_read_b64_tr_b16 (the gfx950
//     transposing LDS read), so V is never transposed in memory;
//   * online softmax in base 2 (scale*log2(e) folded into one multiply, v_exp_f32);
//   * causal: tiles past the diagonal are never loaded, waves skip tiles that are fully masked
//     for their 32 rows, and blocks are issued heaviest-first within each (batch, head).
#include <type_traits>

#include "hk_common.hpp"

#include <cstdlib>
#include "hk_kernels.hpp"

namespace hk {

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kBlockM = 128;  // query rows per forward workgroup (4 waves x 32)
constexpr int kBlockN = 64;   // keys per K/V tile
constexpr int kThreads = 256;
constexpr int kXcds = 8;     // accelerator complex dies; workgroups are dispatched round-robin over them


// 16-byte chunk swizzle of a tile row (XOR applied to the chunk index). gfx950's LDS has 64
// banks: one clock serves 16 lanes of a 16-byte read or 32 lanes of an 8-byte read, i.e. one
// 256-byte bank line. The MFMA operand reads put 16 consecutive rows at the same chunk in those
// 16 lanes, and the transposing reads put 4 consecutive rows (from a multiple of 4) x 4
// consecutive chunks (from a multiple of 4) in 32 lanes; the XOR gives both patterns 16
// distinct 16-byte bank groups. Row-contiguous tile writes stay conflict-free.
template <int D>
__device__ __forceinline__ int tile_swz(int row) {
    constexpr int chunks = D / 8;
    static_assert(chunks == 4 || chunks == 8 || chunks == 16, "tile widths of 32, 64 or 128 elements");
    if constexpr (chunks == 16) {  // 256-byte rows: one row per bank line
        return ((row & 3) << 2) | ((row >> 2) & 3);
    } else if constexpr (chunks == 8) {  // 128-byte rows: two rows per bank line
        const int u = row >> 1;
        return ((u & 1) << 2) | ((u >> 1) & 3);
    } else {  // 64-byte rows: four rows per bank line
        return (row >> 2) & 3;
    }
}

template <int D>
__device__ __forceinline__ int tile_off(int row, int col) {  // element offset in a [rows][D] tile
    return row * D + ((((col >> 3) ^ tile_swz<D>(row))) << 3) + (col & 7);
}

// 16 bytes at (row, 8*chunk) of a swizzled tile.
template <int D>
__device__ __forceinline__ bf16x8_t tile_read16(const uint16_t* t, int row, int chunk) {
    return *reinterpret_cast<const bf16x8_t*>(t + tile_off<D>(row, chunk * 8));
}

// MFMA 32x32x16 operand "rows i = this lane's l%32, k = 8 consecutive tile rows" read from a
// row-major [k][i] tile: two transposing reads of 4 rows each. kbase0/kbase1 are the tile rows
// of the two 4-row halves for this lane's k-group; ibase is the first of the 32 columns.
template <int D>
__device__ __forceinline__ bf16x8_t tile_read_tr(const uint16_t* t, int lane, int kbase0, int kbase1, int ibase) {
    const int g = (lane >> 4) & 1;     // which 16 columns of the 32
    const int i = lane & 15;           // lane within its 16-lane group
    const int col = ibase + 16 * g + 4 * (i & 3);
    const int r = i >> 2;
    const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_v4i16_t*)(t + tile_off<D>(kbase0 + r, col)));
    const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_v4i16_t*)(t + tile_off<D>(kbase1 + r, col)));
    typedef short v8i16_t __attribute__((ext_vector_type(8)));
    v8i16_t v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(bf16x8_t, v);
}

__device__ __forceinline__ bf16x8_t pack_bf16x8(const f32x16_t& a, int base) {
    u32x4_t w = {pack_bf16x2(a[base + 0], a[base + 1]), pack_bf16x2(a[base + 2], a[base + 3]),
                 pack_bf16x2(a[base + 4], a[base + 5]), pack_bf16x2(a[base + 6], a[base + 7])};
    return __builtin_bit_cast(bf16x8_t, w);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Loop-invariant operands loaded from global memory before a tile loop are passed through an
// empty asm: the one wait for their loads then happens here, before the loop. Otherwise the
// compiler's wait-count insertion cannot prove them complete inside the loop, and because
// loads complete in order, its wait for them also waits for the K/V prefetch loads issued one
// iteration earlier, exposing a full HBM round trip per tile.
template <int N>
__device__ __forceinline__ void settle(bf16x8_t (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) asm volatile("" : "+v"(v[i]));
}
__device__ __forceinline__ void settle(float& v) { asm volatile("" : "+v"(v)); }

// Workgroups are dispatched round-robin over the 8 XCDs, each with its own L2. Renumbering
// blockIdx so that each XCD runs one contiguous range of a logical order lets a kernel place
// the workgroups that share operands on the same XCD.
__device__ __forceinline__ int xcd_logical() {
    const int nwg = static_cast<int>(gridDim.x), id = static_cast<int>(blockIdx.x);
    const int xcd = id % kXcds, per_xcd = nwg / kXcds, extra = nwg % kXcds;
    return xcd * per_xcd + (xcd < extra ? xcd : extra) + id / kXcds;
}

struct FwdArgs {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    void* o;     // BF16, or F32 when o_f32 (the reference's FP32 output surface)
    int o_f32;
    float* lse;
    int64_t heads, kv_heads, m, n;
    int64_t diag;  // key j is visible to query i iff j <= i + diag (causal only)
    float scale_log2;
    int causal;
    int mblocks;
};

// Four consecutive output elements of O at element offset `off` (a multiple of 4): packed BF16
// (RNE), or F32 when the caller asked for the FP32 output.
__device__ __forceinline__ void store_o4(const FwdArgs& a, int64_t off, float x0, float x1, float x2, float x3) {
    if (a.o_f32) {
        *reinterpret_cast<f32x4_t*>(static_cast<float*>(a.o) + off) = f32x4_t{x0, x1, x2, x3};
    } else {
        const u32x2_t w = {pack_bf16x2(x0, x1), pack_bf16x2(x2, x3)};
        *reinterpret_cast<u32x2_t*>(static_cast<uint16_t*>(a.o) + off) = w;
    }
}

// Tile rows [row0, row0+64) of a [N, D] matrix -> registers (rows >= n clamp to n-1), laid
// out in LDS as [64][DP] with DP = max(D, 32); columns >= D are zero.
template <int D, int DP, int THREADS = kThreads>
struct TileLoader {
    static constexpr int kChunks = DP / 8;                          // 16-byte chunks per LDS row
    static constexpr int kPerThread = kBlockN * kChunks / THREADS;
    static_assert(kPerThread >= 1 && kBlockN * kChunks % THREADS == 0, "tile must split over the threads");
    u32x4_t r[kPerThread];
    __device__ __forceinline__ void load(const uint16_t* base, int64_t row0, int64_t n, int t) {
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            const int idx = t + i * THREADS;
            const int row = idx / kChunks, chunk = idx % kChunks;
            int64_t gr = row0 + row;
            gr = gr < n ? gr : n - 1;
            r[i] = (chunk * 8 < D) ? *reinterpret_cast<const u32x4_t*>(base + gr * D + chunk * 8) : u32x4_t{0, 0, 0, 0};
        }
    }
    __device__ __forceinline__ void store(uint16_t* tile, int t) const {
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            const int idx = t + i * THREADS;
            const int row = idx / kChunks, chunk = idx % kChunks;
            *reinterpret_cast<u32x4_t*>(tile + tile_off<DP>(row, chunk * 8)) = r[i];
        }
    }
};

// S^T = K Q^T for one 64-key tile and this wave's 32 queries (keys in rows, one query per lane).
template <int DP, int KS>
__device__ __forceinline__ void tile_scores(const uint16_t* Kt, const bf16x8_t (&qf)[KS], int lq, int lg,
                                            f32x16_t (&s)[2]) {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int v = 0; v < 16; ++v) s[tt][v] = 0.0f;
    // the two 32-key halves alternate so that consecutive MFMAs never depend on each other
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
            s[tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tile_read16<DP>(Kt, 32 * tt + lq, 2 * ks + lg), qf[ks],
                                                            s[tt], 0, 0, 0);
}

// Online-softmax update of one tile's raw scores (masked, when MASK, to the keys visible to
// this lane's query), then O^T += V^T P^T. c = |scale|*log2(e) > 0 (a negative scale is folded
// into Q), so the scaled row max is c times the raw max and p = 2^(c*s - m) is one FMA + exp2.
//
// The running max m is allowed to lag the true max by up to kStaleMax (base-2 units): O, l and
// m are only rescaled when some row of the wave sees its max grow by more than that, so most
// tiles skip the 64-register rescale of O. Then p <= 2^kStaleMax, well inside BF16/F32 range,
// and O / l and lse = m + log2(l) are the same quantities as with an exact running max.
constexpr float kStaleMax = 8.0f;

// Softmax part: updates m, l (and rescales O when needed) and leaves P in BF16 as the B
// operands of the four 16-key MFMA steps of P.V.
template <int DT>
__device__ __forceinline__ void tile_softmax(f32x16_t (&s)[2], int lane, float c, bool mask, int64_t kv0,
                                             int64_t key_limit, float& m_run, float& l_run, f32x16_t (&o)[DT],
                                             bf16x8_t (&pb)[4]) {
    const int lg = lane >> 5;
    // key kv0 + 32*tt + 8*(v/4) + 4*lg + v%4 is visible iff it is <= key_limit, i.e. iff
    // 32*tt + 8*(v/4) + v%4 <= rel (a compile-time constant against one register)
    if (mask) {
        int64_t rel64 = key_limit - kv0 - 4 * lg;
        rel64 = rel64 < -1 ? -1 : (rel64 > kBlockN ? kBlockN : rel64);
        int rel = static_cast<int>(rel64);
        asm volatile("" : "+v"(rel));  // keep the compares 32-bit
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int v = 0; v < 16; ++v)
                s[tt][v] = 32 * tt + (v >> 2) * 8 + (v & 3) <= rel ? s[tt][v] : -INFINITY;
    }
    float mt = -INFINITY;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int v = 0; v < 16; ++v) mt = fmaxf(mt, s[tt][v]);
    mt = pair32_max(mt) * c;
    if (__any(mt > m_run + kStaleMax)) {
        const float m_new = fmaxf(m_run, mt);
        const float alpha = m_new == -INFINITY ? 1.0f : fast_exp2(m_run - m_new);
        m_run = m_new;
        l_run *= alpha;
#pragma unroll
        for (int i = 0; i < DT; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) o[i][v] *= alpha;
    }
    const float neg_m = m_run == -INFINITY ? 0.0f : -m_run;
    float ls = 0.0f;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const float p = fast_exp2(__builtin_fmaf(s[tt][v], c, neg_m));
            s[tt][v] = p;
            ls += p;
        }
    l_run += ls;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) pb[ks] = pack_bf16x8(s[ks >> 1], 8 * (ks & 1));
}

// O^T += V^T P^T over one 64-key tile (V^T through transposing reads of the row-major V tile).
template <int DP, int DT>
__device__ __forceinline__ void tile_pv(const bf16x8_t (&pb)[4], const uint16_t* Vt, int lane, f32x16_t (&o)[DT]) {
    const int lg = lane >> 5;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        const int kb0 = 16 * ks + 4 * lg;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
            o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tile_read_tr<DP>(Vt, lane, kb0, kb0 + 8, 32 * dt), pb[ks],
                                                            o[dt], 0, 0, 0);
    }
}

template <int DP, int DT>
__device__ __forceinline__ void tile_update(f32x16_t (&s)[2], const uint16_t* Vt, int lane, float c, bool mask,
                                            int64_t kv0, int64_t key_limit, float& m_run, float& l_run,
                                            f32x16_t (&o)[DT]) {
    bf16x8_t pb[4];
    tile_softmax<DT>(s, lane, c, mask, kv0, key_limit, m_run, l_run, o, pb);
    tile_pv<DP, DT>(pb, Vt, lane, o);
}

// D is the head dim in memory; the kernel works on DP = max(D, 32) (zero-padded columns).
// Used for D <= 32; wider heads use the ping-pong kernel below. Tile j is read from LDS buffer
// j&1 while tile j+1 waits in registers and is stored into the other buffer at the end of the
// iteration. Tiles fully visible to every row of the workgroup run without mask arithmetic.
template <int D>
__global__ void __launch_bounds__(kThreads, 2)
attn_fwd(FwdArgs a) {
    constexpr int DP = D < 32 ? 32 : D;
    constexpr int KS = DP / 16;  // MFMA k-steps over the head dim
    constexpr int DT = DP / 32;  // 32-wide output tiles over the head dim
    __shared__ __attribute__((aligned(16))) uint16_t lds[2][2][kBlockN * DP];  // [buf][K,V]

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int lq = lane & 31, lg = lane >> 5;
    // logical order: KV head group, query block heaviest first, query head in the group -- the
    // workgroups resident on one XCD share one K/V head, which stays in that XCD's L2
    const int logical = xcd_logical();
    const int group_heads = static_cast<int>(a.heads / a.kv_heads);
    const int per_group = a.mblocks * group_heads;
    const int grp = logical / per_group, in_grp = logical % per_group;
    const int mb = a.mblocks - 1 - in_grp / group_heads;  // heaviest causal blocks first
    const int64_t b = grp / a.kv_heads, kvh = grp % a.kv_heads;
    const int64_t h = kvh * group_heads + in_grp % group_heads;
    const int64_t bh = b * a.heads + h;
    const uint16_t* Q = a.q + (bh * a.m) * D;
    const uint16_t* K = a.k + ((b * a.kv_heads + kvh) * a.n) * D;
    const uint16_t* V = a.v + ((b * a.kv_heads + kvh) * a.n) * D;
    const int64_t q0 = static_cast<int64_t>(mb) * kBlockM;
    const int64_t my_q = q0 + wave * 32 + lq;

    // keys this workgroup needs: [0, kv_end); tiles [0, nfull) are visible to all its rows
    int64_t kv_end = a.n, full_end = a.n;
    if (a.causal) {
        const int64_t last = q0 + kBlockM - 1 + a.diag;  // last key visible to the block's last row
        kv_end = last + 1 < kv_end ? last + 1 : kv_end;
        const int64_t first = q0 + a.diag + 1;            // keys [0, first) are visible to its first row
        full_end = first < full_end ? first : full_end;
    }
    const int ntiles = kv_end > 0 ? static_cast<int>((kv_end + kBlockN - 1) / kBlockN) : 0;
    int nfull = full_end > 0 ? static_cast<int>(full_end / kBlockN) : 0;
    nfull = nfull < ntiles ? nfull : ntiles;
    // the last key this lane's query may see (causal and bounds)
    int64_t key_limit = a.n - 1;
    if (a.causal) key_limit = my_q + a.diag < key_limit ? my_q + a.diag : key_limit;

    // Q of this lane's query as the B operand: d = 16*s + 8*lg .. +7
    bf16x8_t qf[KS];
    {
        const int64_t qr = my_q < a.m ? my_q : a.m - 1;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const int d0 = 16 * s + 8 * lg;
            qf[s] = d0 < D ? *reinterpret_cast<const bf16x8_t*>(Q + qr * D + d0)
                           : __builtin_bit_cast(bf16x8_t, u32x4_t{0, 0, 0, 0});
        }
    }
    // c = |scale| log2(e); a negative scale flips the sign of Q instead
    float c = a.scale_log2;
    if (c < 0.0f) {
        c = -c;
#pragma unroll
        for (int s = 0; s < KS; ++s)
            qf[s] = __builtin_bit_cast(bf16x8_t, __builtin_bit_cast(u32x4_t, qf[s]) ^ 0x80008000u);
    }
    settle(qf);

    f32x16_t o[DT];
#pragma unroll
    for (int i = 0; i < DT; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[i][v] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;

    TileLoader<D, DP> lk, lv;
    if (ntiles > 0) {
        lk.load(K, 0, a.n, t);
        lv.load(V, 0, a.n, t);
        lk.store(lds[0][0], t);
        lv.store(lds[0][1], t);
        if (ntiles > 1) {
            lk.load(K, kBlockN, a.n, t);
            lv.load(V, kBlockN, a.n, t);
        }
    }
    __syncthreads();

    // Tile j is read from buffer j&1 while tile j+1 waits in registers (stored into the other
    // buffer at the end of the iteration) and tile j+2 is being fetched.
    const int64_t q0w = q0 + wave * 32;
    for (int j = 0; j < ntiles; ++j) {
        const int cur = j & 1;
        const int64_t kv0 = static_cast<int64_t>(j) * kBlockN;
        // this wave's rows see no key of this tile -> skip (still takes part in the barriers)
        const bool skip = a.causal && (kv0 > q0w + 31 + a.diag);
        if (!skip) {
            f32x16_t s[2];
            tile_scores<DP, KS>(lds[cur][0], qf, lq, lg, s);
            tile_update<DP, DT>(s, lds[cur][1], lane, c, j >= nfull, kv0, key_limit, m_run, l_run, o);
        }
        if (j + 1 < ntiles) {
            lk.store(lds[cur ^ 1][0], t);
            lv.store(lds[cur ^ 1][1], t);
            if (j + 2 < ntiles) {
                lk.load(K, kv0 + 2 * kBlockN, a.n, t);
                lv.load(V, kv0 + 2 * kBlockN, a.n, t);
            }
        }
        __syncthreads();
    }

    // epilogue: O[q][d] = O^T / l ; lse = (m + log2 l) ln 2
    const float l_tot = pair32_sum(l_run);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    if (my_q < a.m) {
        const int64_t obase = (bh * a.m + my_q) * D;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = 32 * dt + 8 * g + 4 * lg;
                if (d >= D) continue;
                store_o4(a, obase + d, o[dt][4 * g] * inv, o[dt][4 * g + 1] * inv, o[dt][4 * g + 2] * inv,
                         o[dt][4 * g + 3] * inv);
            }
        if (lg == 0)
            a.lse[bh * a.m + my_q] = l_tot > 0.0f ? (m_run + log2f(l_tot)) * kLn2 : -INFINITY;
    }
}

// Ping-pong forward kernel for D = 64 / 128: 8 wavefronts = 256 query rows per workgroup,
// two waves per SIMD (waves w and w+4). Each wave alternates an MFMA phase (P.V of the previous
// tile and S = K Q^T of the current one, 64 16x16x32 MFMAs at D = 128) with a softmax phase (VALU and v_exp_f32),
// and the second group of four waves runs one phase behind the first: at every barrier the two
// waves on a SIMD swap roles, so the matrix core is fed by one while the other computes the
// exponentials, instead of both waiting on their own softmax. The MFMA phase raises the wave's
// issue priority so its next MFMA is issued as soon as the matrix core frees up.
//
// Half-step h (barrier-separated): tiles K_t and V_{t-1} (t = h/2) are in LDS; the group lagging
// by g half-steps does its phase s = h - g: even s -> MFMA phase of tile s/2, odd s -> softmax
// of tile (s-1)/2. K_{t+1} and V_t are fetched straight into LDS (into the buffers read two
// half-steps earlier) from the even half-step on, and waited for before the barrier that ends
// the odd one. The K/V tile is shared by all 8 waves: half the global->LDS traffic per query
// of the 4-wave kernel.
// The ping-pong kernel keeps its K and V tiles in padded rows instead of XOR-swizzled ones, so
// that every operand read is one base register plus an immediate offset (the swizzle's
// lane-dependent XOR would need a register per read pattern, and with Q, O, S and P resident
// those spill). The pads are chosen for gfx950's 64 banks (256-byte bank line):
//   K rows of D+8 elements: the 16 rows of an operand read (16 lanes, 16 bytes each) start
//     16 bytes apart modulo 256 -> 16 distinct bank groups;
//   V rows of D+16 elements (kV16Stride below).
template <int D> constexpr int kKStride = D + 8;

template <int STRIDE>
__device__ __forceinline__ bf16x8_t pad_read16(const uint16_t* t, int row, int chunk) {
    return *reinterpret_cast<const bf16x8_t*>(t + row * STRIDE + chunk * 8);
}

constexpr int kPPWaves = 8;
constexpr int kPPThreads = kPPWaves * 64;
constexpr int kPPBlockM = kPPWaves * 32;

// Rows [row0, row0 + 64) of one K or V head into a padded [64][STRIDE] LDS tile through the
// global->LDS path (no staging registers, no LDS write instructions). The tile is a run of
// 64 * STRIDE / 8 16-byte positions; wave instruction q fills positions 64q .. 64q+63, so lane
// l fetches the chunk that belongs at position 64q + l (pad positions fetch a chunk of their
// row again). Rows past n repeat row n-1 (finite values for the masked keys). The caller waits
// (vmcnt) before the barrier that publishes the tile.
template <int D, int STRIDE>
struct PadTileDma {
    static constexpr int kPerRow = STRIDE / 8;  // 16-byte positions per row, pad included
    static constexpr int kInstr = kPerRow;      // 64 rows * kPerRow positions / 64 lanes
    // Instruction q (< kInstr) of the tile. row0 and n fit in 32 bits: the launcher keeps
    // n * D * 2 below 2^31.
    __device__ __forceinline__ static void issue_one(i32x4_t rsrc, uint16_t* tile, int row0, int n, int q, int lane) {
        // recompute the lane's position here rather than keep it in a register across the loop
        asm volatile("" : "+v"(lane));
        const int pos = 64 * q + lane;
        const int row = pos / kPerRow, c = pos % kPerRow;
        const int chunk = c < D / 8 ? c : 0;
        const int gr = min(row0 + row, n - 1);
        load_lds16(rsrc, lds_address(tile + 8 * 64 * q), (gr * D + chunk * 8) * 2, 0);
    }
    // Lane byte offset of instruction q within a tile whose rows are all below n: the load is
    // then rsrc + lane_offset(q) + row0 * D * 2 (uniform), with nothing to compute per load.
    __device__ __forceinline__ static int lane_offset(int q, int lane) {
        const int pos = 64 * q + lane;
        const int row = pos / kPerRow, c = pos % kPerRow;
        const int chunk = c < D / 8 ? c : 0;
        return (row * D + chunk * 8) * 2;
    }
    // The whole tile from the 8 waves of the workgroup.
    __device__ __forceinline__ static void issue(i32x4_t rsrc, uint16_t* tile, int row0, int n, int wave,
                                                 int lane) {
#pragma unroll
        for (int i = 0; i < (kInstr + kPPWaves - 1) / kPPWaves; ++i) {
            const int q = wave + kPPWaves * i;
            if (q < kInstr) issue_one(rsrc, tile, row0, n, q, lane);
        }
    }
};

// The ping-pong kernel's tiles are v_mfma_f32_16x16x32_bf16 ones. Each wave's 32 queries are two
// 16-query blocks qb and a 64-key tile four 16-key blocks kb:
//   S^T = K Q^T: s[qb][kb] (lane l: query 16 qb + l % 16, keys 16 kb + 4 (l / 16) + 0..3), the A
//     operand K rows 16 kb + l % 16 at head dims 32 ks + 8 (l / 16) from LDS, the B operand Q from
//     registers; every K operand read feeds the MFMAs of both query blocks;
//   O^T += V^T P^T: o[db][qb] (lane l: query 16 qb + l % 16, head dims 16 db + 4 (l / 16) + 0..3)
//     over two 32-key steps ps. The lane's P values of step ps are keys 32 ps + 4 g + 0..3 and
//     32 ps + 16 + 4 g + 0..3 (g = l / 16), used as its 8 k values in that order; the V^T operand
//     follows the same key order: two transposing reads of 4 key rows each (v16_read_tr). Every V
//     operand read also feeds both query blocks.
// Against the same kernel with 32x32x16 tiles (one 32-query block per wave, the lane's query
// l % 32) this moves a quarter of the accumulator registers per MFMA and half the register bytes
// per multiply-accumulate; measured on one box at C4 0.636-0.640 ms against 0.649-0.650 ms. A
// query's row max and sum span the four lanes l % 16 + 16 g (two lane swaps).

// V tile rows of D + 16 elements (288 bytes for D = 128): the 8 rows x 32 bytes a transposing
// read touches per 32 lanes (rows 32 ps + 4 g + r, g < 2, r < 4, at 16 db .. 16 db + 15) start
// 32 bytes apart modulo 256, so they fall on 8 distinct 32-byte bank groups.
template <int D> constexpr int kV16Stride = D + 16;

// 16x16x32 A operand V^T of head dims 16 db .. 16 db + 15 and key step ps (see above).
template <int STRIDE>
__device__ __forceinline__ bf16x8_t v16_read_tr(const uint16_t* t, int lane, int ps, int db) {
    const int i = lane & 15, g = lane >> 4;
    const int col = 16 * db + 4 * (i & 3);
    const int r = i >> 2;
    const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(t + (32 * ps + 4 * g + r) * STRIDE + col));
    const v4i16_t hi =
        __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(t + (32 * ps + 16 + 4 * g + r) * STRIDE + col));
    typedef short v8i16_t __attribute__((ext_vector_type(8)));
    v8i16_t v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(bf16x8_t, v);
}

// Max / sum over the four lanes l % 16 + 16 g that share a query (two swap steps; partners compute
// the same value in the same order).
__device__ __forceinline__ float quad_max(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return pair32_max(fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1])));
}
__device__ __forceinline__ float quad_sum(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return pair32_sum(__uint_as_float(r[0]) + __uint_as_float(r[1]));
}

// Online-softmax update of one tile for the 16x16 layout (tile_softmax's rules: base 2, the
// running max lagging by at most kStaleMax, masked keys -inf), leaving P as the B operands
// pb[ps][qb] of the two 32-key steps.
template <int DB>
__device__ __forceinline__ void tile_softmax16(f32x4_t (&s)[2][4], int lane, float c, bool mask, int64_t kv0,
                                               const int64_t (&key_limit)[2], float (&m_run)[2], float (&l_run)[2],
                                               f32x4_t (&o)[DB][2], bf16x8_t (&pb)[2][2]) {
    const int g = lane >> 4;
    if (mask) {
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
            // key kv0 + 16 kb + 4 g + e is visible iff 16 kb + e <= rel
            int64_t rel64 = key_limit[qb] - kv0 - 4 * g;
            rel64 = rel64 < -1 ? -1 : (rel64 > kBlockN ? kBlockN : rel64);
            int rel = static_cast<int>(rel64);
            asm volatile("" : "+v"(rel));
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                for (int e = 0; e < 4; ++e) s[qb][kb][e] = 16 * kb + e <= rel ? s[qb][kb][e] : -INFINITY;
        }
    }
    float mt[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        float x = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int e = 0; e < 4; ++e) x = fmaxf(x, s[qb][kb][e]);
        mt[qb] = quad_max(x) * c;
    }
    if (__any(mt[0] > m_run[0] + kStaleMax || mt[1] > m_run[1] + kStaleMax)) {
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
            const float m_new = fmaxf(m_run[qb], mt[qb]);
            const float alpha = m_new == -INFINITY ? 1.0f : fast_exp2(m_run[qb] - m_new);
            m_run[qb] = m_new;
            l_run[qb] *= alpha;
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int e = 0; e < 4; ++e) o[db][qb][e] *= alpha;
        }
    }
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        const float neg_m = m_run[qb] == -INFINITY ? 0.0f : -m_run[qb];
        float ls = 0.0f;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float p = fast_exp2(__builtin_fmaf(s[qb][kb][e], c, neg_m));
                s[qb][kb][e] = p;
                ls += p;
            }
        l_run[qb] += ls;
    }
#pragma unroll
    for (int ps = 0; ps < 2; ++ps)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
            const f32x4_t& a = s[qb][2 * ps];
            const f32x4_t& b = s[qb][2 * ps + 1];
            const u32x4_t w = {pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3]), pack_bf16x2(b[0], b[1]),
                               pack_bf16x2(b[2], b[3])};
            pb[ps][qb] = __builtin_bit_cast(bf16x8_t, w);
        }
}

// MFMA phase of the ping-pong kernel: O^T += V^T P^T of tile j-1 (2 DB operand reads, 4 DB MFMAs),
// then S^T = K Q^T of tile j (4 KS reads, 8 KS MFMAs), as one software pipeline: the LDS operand of
// read i + kAhead is fetched while the MFMAs of read i run, through a ring of kAhead + 1 registers.
// The fences keep the compiler from regrouping the reads in front of their MFMAs (which serializes
// every MFMA behind a full LDS round trip); the empty asm makes the wait for each operand land
// right before its MFMAs.
constexpr int kAhead = 6;

template <int D>
__device__ __forceinline__ void mfma_phase16(const uint16_t* Vt, const uint16_t* Kt, const bf16x8_t (&pb)[2][2],
                                             const bf16x8_t (&qf)[2][D / 32], int lane, f32x4_t (&o)[D / 16][2],
                                             f32x4_t (&s)[2][4]) {
    constexpr int DB = D / 16, KS = D / 32;
    constexpr int NPV = 2 * DB;  // (ps, db), ps-major
    constexpr int NQK = 4 * KS;  // (ks, kb), ks-major
    constexpr int N = NPV + NQK;
    constexpr int R = kAhead + 1;
    const int l16 = lane & 15, g = lane >> 4;
    auto fetch = [&](int i) -> bf16x8_t {
        if (i < NPV) return v16_read_tr<kV16Stride<D>>(Vt, lane, i / DB, i % DB);
        const int q = i - NPV, ks = q >> 2, kb = q & 3;
        return pad_read16<kKStride<D>>(Kt, 16 * kb + l16, 4 * ks + g);
    };
    bf16x8_t ring[R];
#pragma unroll
    for (int i = 0; i < kAhead && i < N; ++i) ring[i % R] = fetch(i);
#pragma unroll
    for (int i = 0; i < N; ++i) {
        if (i + kAhead < N) ring[(i + kAhead) % R] = fetch(i + kAhead);
        __builtin_amdgcn_sched_barrier(0);
        bf16x8_t x = ring[i % R];
        asm volatile("" : "+v"(x));
        if (i < NPV) {
            const int ps = i / DB, db = i % DB;
#pragma unroll
            for (int qb = 0; qb < 2; ++qb)
                o[db][qb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x, pb[ps][qb], o[db][qb], 0, 0, 0);
        } else {
            const int q = i - NPV, ks = q >> 2, kb = q & 3;
            const f32x4_t zero = {};
#pragma unroll
            for (int qb = 0; qb < 2; ++qb)
                s[qb][kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x, qf[qb][ks], ks == 0 ? zero : s[qb][kb], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

template <int D>
__global__ void __launch_bounds__(kPPThreads, 1)
attn_fwd_pp16(FwdArgs a) {
    static_assert(D == 64 || D == 128, "ping-pong kernel is for D = 64 or 128");
    constexpr int KS = D / 32;  // 32-wide head-dim steps of S^T
    constexpr int DB = D / 16;  // 16-wide head-dim blocks of O^T
    __shared__ __attribute__((aligned(16))) uint16_t kbuf[2][kBlockN * kKStride<D>];
    __shared__ __attribute__((aligned(16))) uint16_t vbuf[2][kBlockN * kV16Stride<D>];
    using KDma = PadTileDma<D, kKStride<D>>;
    using VDma = PadTileDma<D, kV16Stride<D>>;

    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int l16 = lane & 15, g = lane >> 4;
    const int group = wave >> 2;  // 0: leads, 1: one half-step behind
    const int logical = xcd_logical();
    const int group_heads = static_cast<int>(a.heads / a.kv_heads);
    const int per_group = a.mblocks * group_heads;
    const int grp = logical / per_group, in_grp = logical % per_group;
    const int mb = a.mblocks - 1 - in_grp / group_heads;
    const int64_t b = grp / a.kv_heads, kvh = grp % a.kv_heads;
    const int64_t h = kvh * group_heads + in_grp % group_heads;
    const int64_t bh = b * a.heads + h;
    const uint16_t* Q = a.q + (bh * a.m) * D;
    const uint16_t* K = a.k + ((b * a.kv_heads + kvh) * a.n) * D;
    const uint16_t* V = a.v + ((b * a.kv_heads + kvh) * a.n) * D;
    const int64_t q0 = static_cast<int64_t>(mb) * kPPBlockM;
    const int64_t q0w = q0 + wave * 32;
    const int64_t my_q[2] = {q0w + l16, q0w + 16 + l16};

    int64_t kv_end = a.n, full_end = a.n;
    if (a.causal) {
        const int64_t last = q0 + kPPBlockM - 1 + a.diag;
        kv_end = last + 1 < kv_end ? last + 1 : kv_end;
        const int64_t first = q0 + a.diag + 1;
        full_end = first < full_end ? first : full_end;
    }
    const int ntiles = kv_end > 0 ? static_cast<int>((kv_end + kBlockN - 1) / kBlockN) : 0;
    int nfull = full_end > 0 ? static_cast<int>(full_end / kBlockN) : 0;
    nfull = nfull < ntiles ? nfull : ntiles;
    int64_t key_limit[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        key_limit[qb] = a.n - 1;
        if (a.causal) key_limit[qb] = my_q[qb] + a.diag < key_limit[qb] ? my_q[qb] + a.diag : key_limit[qb];
    }
    auto skip = [&](int j) { return a.causal && static_cast<int64_t>(j) * kBlockN > q0w + 31 + a.diag; };

    bf16x8_t qf[2][KS];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        const int64_t qr = my_q[qb] < a.m ? my_q[qb] : a.m - 1;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) qf[qb][ks] = *reinterpret_cast<const bf16x8_t*>(Q + qr * D + 32 * ks + 8 * g);
    }
    float c = a.scale_log2;
    if (c < 0.0f) {
        c = -c;
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                qf[qb][ks] = __builtin_bit_cast(bf16x8_t, __builtin_bit_cast(u32x4_t, qf[qb][ks]) ^ 0x80008000u);
    }
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) settle(qf[qb]);

    f32x4_t o[DB][2];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) o[db][qb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.0f, 0.0f};
    f32x4_t s[2][4];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) s[qb][kb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    bf16x8_t pb[2][2];
#pragma unroll
    for (int ps = 0; ps < 2; ++ps)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) pb[ps][qb] = __builtin_bit_cast(bf16x8_t, u32x4_t{0, 0, 0, 0});

    const i32x4_t rk = buffer_resource(K, static_cast<int>(a.n * D * 2));
    const i32x4_t rv = buffer_resource(V, static_cast<int>(a.n * D * 2));
    const int n32 = static_cast<int>(a.n);
    if (ntiles > 0) KDma::issue(rk, kbuf[0], 0, n32, wave, lane);
    for (int i = t; i < kBlockN * kV16Stride<D> / 8; i += kPPThreads)
        *reinterpret_cast<u32x4_t*>(vbuf[1] + 8 * i) = u32x4_t{0, 0, 0, 0};
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();

    constexpr int kKInstr = KDma::kInstr, kVInstr = VDma::kInstr;
    constexpr int kLoadsPerWave = (kKInstr + kVInstr + 3) / 4;
    int loff[kLoadsPerWave];
#pragma unroll
    for (int d = 0; d < kLoadsPerWave; ++d) {
        const int q = (wave & 3) + 4 * d;
        loff[d] = q < kKInstr ? KDma::lane_offset(q, lane)
                              : (q < kKInstr + kVInstr ? VDma::lane_offset(q - kKInstr, lane) : 0);
    }
    auto landed = [&]() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); };
    auto softmax = [&](int j) {
        if (!skip(j)) {
            tile_softmax16<DB>(s, lane, c, j >= nfull, static_cast<int64_t>(j) * kBlockN, key_limit, m_run, l_run, o,
                               pb);
        } else {
#pragma unroll
            for (int ps = 0; ps < 2; ++ps)
#pragma unroll
                for (int qb = 0; qb < 2; ++qb) pb[ps][qb] = __builtin_bit_cast(bf16x8_t, u32x4_t{0, 0, 0, 0});
        }
    };
    auto tile_loads = [&](int j) {
        const bool k_next = j + 1 < ntiles, v_cur = j < ntiles;
        uint16_t* kdst = kbuf[(j + 1) & 1];
        uint16_t* vdst = vbuf[j & 1];
        const bool k_whole = (j + 2) * kBlockN <= n32, v_whole = (j + 1) * kBlockN <= n32;
        if (k_next && k_whole && v_cur && v_whole) {
#pragma unroll
            for (int d = 0; d < kLoadsPerWave; ++d) {
                const int q = (wave & 3) + 4 * d;
                if (q < kKInstr)
                    load_lds16(rk, lds_address(kdst + 8 * 64 * q), loff[d], (j + 1) * kBlockN * D * 2);
                else if (q < kKInstr + kVInstr)
                    load_lds16(rv, lds_address(vdst + 8 * 64 * (q - kKInstr)), loff[d], j * kBlockN * D * 2);
            }
            return;
        }
#pragma unroll
        for (int d = 0; d < kLoadsPerWave; ++d) {
            const int q = (wave & 3) + 4 * d;
            if (q < kKInstr) {
                if (k_next && k_whole)
                    load_lds16(rk, lds_address(kdst + 8 * 64 * q), loff[d], (j + 1) * kBlockN * D * 2);
                else if (k_next)
                    KDma::issue_one(rk, kdst, (j + 1) * kBlockN, n32, q, lane);
            } else if (q < kKInstr + kVInstr) {
                const int qv = q - kKInstr;
                if (v_cur && v_whole)
                    load_lds16(rv, lds_address(vdst + 8 * 64 * qv), loff[d], j * kBlockN * D * 2);
                else if (v_cur)
                    VDma::issue_one(rv, vdst, j * kBlockN, n32, qv, lane);
            }
        }
    };
    auto mfma_step = [&](int j) {
        const bool pv = j >= 1 && !skip(j - 1), qk = j < ntiles && !skip(j);
        if (pv || qk) mfma_phase16<D>(vbuf[(j - 1) & 1], kbuf[j & 1], pb, qf, lane, o, s);
    };
    if (group == 0) {
        for (int j = 0; j <= ntiles; ++j) {
            __builtin_amdgcn_s_setprio(1);
            mfma_step(j);
            __builtin_amdgcn_s_setprio(0);
            lds_barrier();
            if (j < ntiles) softmax(j);
            lds_barrier();
        }
    } else {
        tile_loads(0);
        lds_barrier();
        for (int j = 0; j <= ntiles; ++j) {
            __builtin_amdgcn_s_setprio(1);
            mfma_step(j);
            __builtin_amdgcn_s_setprio(0);
            landed();
            lds_barrier();
            if (j < ntiles) {
                tile_loads(j + 1);
                softmax(j);
                lds_barrier();
            }
        }
        landed();
    }

#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        const float l_tot = quad_sum(l_run[qb]);
        const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
        if (my_q[qb] < a.m) {
            const int64_t obase = (bh * a.m + my_q[qb]) * D;
#pragma unroll
            for (int db = 0; db < DB; ++db)
                store_o4(a, obase + 16 * db + 4 * g, o[db][qb][0] * inv, o[db][qb][1] * inv, o[db][qb][2] * inv,
                         o[db][qb][3] * inv);
            if (g == 0)
                a.lse[bh * a.m + my_q[qb]] = l_tot > 0.0f ? (m_run[qb] + log2f(l_tot)) * kLn2 : -INFINITY;
        }
    }
}

int64_t clamp_diag(const AttnShape& sh) {
    // visible iff key_start + j <= query_start + i  <=>  j <= i + (query_start - key_start)
    if (!sh.causal) return 0;
    const uint64_t qs = sh.query_start, ks = sh.key_start;
    if (qs >= ks) {
        const uint64_t d = qs - ks;
        return d > static_cast<uint64_t>(sh.n) ? sh.n : static_cast<int64_t>(d);
    }
    const uint64_t d = ks - qs;
    const uint64_t cap = static_cast<uint64_t>(sh.m + sh.n + 1);
    return -static_cast<int64_t>(d > cap ? cap : d);
}

template <int D>
hipError_t launch_fwd(const AttnShape& sh, const void* q, const void* k, const void* v, void* o, float* lse,
                      hipStream_t s) {
    FwdArgs a;
    a.q = static_cast<const uint16_t*>(q);
    a.k = static_cast<const uint16_t*>(k);
    a.v = static_cast<const uint16_t*>(v);
    a.o = o;
    a.o_f32 = sh.o_f32;
    a.lse = lse;
    a.heads = sh.heads;
    a.kv_heads = sh.kv_heads;
    a.m = sh.m;
    a.n = sh.n;
    a.diag = clamp_diag(sh);
    a.scale_log2 = sh.scale * kLog2e;
    a.causal = sh.causal;
    if constexpr (D >= 64) {
        a.mblocks = static_cast<int>((sh.m + kPPBlockM - 1) / kPPBlockM);
        const dim3 grid(static_cast<unsigned>(sh.batch * sh.heads * a.mblocks));
        hipLaunchKernelGGL((attn_fwd_pp16<D>), grid, dim3(kPPThreads), 0, s, a);
    } else {
        a.mblocks = static_cast<int>((sh.m + kBlockM - 1) / kBlockM);
        const dim3 grid(static_cast<unsigned>(sh.batch * sh.heads * a.mblocks));
        hipLaunchKernelGGL((attn_fwd<D>), grid, dim3(kThreads), 0, s, a);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------- backward
//
// Pre-pass: rowstat[bh, i] = sum_d dO[i, d] * O[i, d] (F32). With O = P V this equals
// sum_j P_ij dP_ij, the softmax-backward row term of row_programs.rs:152-163. It also writes
// lse2 = lse * log2(e), the form in which the gradient kernels use the row's log-sum-exp.
// O is BF16, or F32 (the FP32 output surface: the row term then carries no rounding of O).
template <int D, typename TO>
__global__ void __launch_bounds__(256)
attn_bwd_rowstat(const TO* __restrict__ o, const uint16_t* __restrict__ dout, const float* __restrict__ lse,
                 float* __restrict__ stat, float* __restrict__ lse2, int64_t rows) {
    constexpr int kLanesPerRow = D / 8;  // each lane reads 8 elements
    constexpr int kRowsPerBlock = 256 / kLanesPerRow;
    const int part = static_cast<int>(threadIdx.x % kLanesPerRow);
    // grid-stride over rows; the kLanesPerRow lanes of a row (the shuffle's segment) share its trip count
    for (int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / kLanesPerRow; row < rows;
         row += static_cast<int64_t>(gridDim.x) * kRowsPerBlock) {
        float s = 0.0f;
        float a[8], b[8];
        load8(o + row * D + part * 8, a);
        load8(dout + row * D + part * 8, b);
#pragma unroll
        for (int e = 0; e < 8; ++e) s += a[e] * b[e];
#pragma unroll
        for (int off = kLanesPerRow / 2; off >= 1; off >>= 1) s += __shfl_xor(s, off, kLanesPerRow);
        if (part == 0) {
            stat[row] = s;
            lse2[row] = lse[row] * kLog2e;
        }
    }
}

struct BwdArgs {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const uint16_t* dout;
    const float* lse2;  // lse * log2(e), per row
    const float* stat;
    void* dq;
    void* dk;
    void* dv;
    int64_t heads, kv_heads, m, n;
    int64_t diag;
    float scale, scale_log2;
    int causal;
    int dq_bf16, dkv_bf16;
    int blocks;  // key blocks (dK/dV kernel) or query blocks (dQ kernel) per head
    // dS (BF16, unscaled) in 4 KB blocks of 32 keys x 64 queries, block (bh, key/32, query/64)
    // at ((bh * nsq + query/64) * nkb + key/32) * 4096 bytes (a 64-query row of blocks is
    // contiguous, in the order the dQ kernel reads it): written by the dK/dV kernel when set,
    // read by attn_bwd_dq_ds. Blocks whose pairs no query sees are left unwritten.
    uint16_t* ds;
    int64_t nkb, nsq;  // ceil(N / 32), ceil(M / 64)
    // Rows output (a decoder layer's fused QKV gradient; M = N = S, D = 64 or 128): when rows is
    // set, dQ, dK and dV go to BF16 token rows rows[(b S + s) row_w + col + d] instead of dq, dk
    // and dv, col being the head's column in the fused projection (h D for Q, (Hq + kvh) D for K,
    // (Hq + Hkv + kvh) D for V), with dQ and dK rotated back by RoPE's transpose (F32 tables
    // rope_cos/rope_sin [S, D/2] indexed by s; layout 1 split-half, 0 interleaved).
    uint16_t* rows;
    int64_t row_w;
    const float* rope_cos;
    const float* rope_sin;
    int rope_layout;
    // dK/dV split (splits > 1): each head's query steps of a key block are divided into `splits`
    // contiguous ranges, one workgroup each, which write their F32 dK (scaled) and dV sums to
    // partial[((split * 2 + kv) * B Hkv + bkv) * n + key][d] (kv 0: dK, 1: dV); attn_bwd_dkdv_reduce
    // adds them in split order and stores the result as the unsplit kernel would.
    int splits;
    float* partial;
};

// Layout inside a dS block: four 1 KB chunks c = 2 qt + h, each holding 64 lanes x 16 bytes as
// the dK/dV kernel's wave has them (pack_bf16x8 of its dS accumulators): lane L (key L % 32,
// k-group L / 32) holds queries 32 qt + 16 h + 8 (e / 4) + 4 (L / 32) + e % 4, e = 0..7, of its
// key. Lane L's 16 bytes sit at slot L ^ 4 (L / 32) ^ 8 (c % 2) of the chunk, so that the dQ
// kernel's transposing reads (32 lanes: four keys x two k-groups x two chunks, 8 bytes each)
// fall on 32 distinct 8-byte bank slots.
__device__ __forceinline__ int ds_slot(int lane, int c) { return lane ^ ((lane >> 5) << 2) ^ ((c & 1) << 3); }

// A [64][DP] tile (tile_off<DP> swizzle) of rows row0 .. row0+63 of a row-major [*, D] BF16
// matrix, filled through the global->LDS path: DP / 8 instructions of 1 KB, instruction q
// covering tile rows (512 / DP) * q onwards. Lane l lands at tile position 512 q + 8 l and so
// fetches the global chunk the swizzle puts there. The row offset is part of the per-lane
// offset, which the hardware checks against the buffer size: rows past the end read as zero
// (as do, for D < DP, the pad chunks, given an offset past any buffer). Wave w issues the
// instructions q = w, w + 4, ..., which all see the same swizzle, so one lane offset serves.
template <int D, int DP>
struct SwzTileDma {
    static constexpr int kInstr = DP / 8;
    static constexpr int kPerWave = kInstr / 4;
    static constexpr int kRowsPerInstr = 512 / DP;
    __device__ __forceinline__ static int lane_offset(int wave, int lane) {
        constexpr int kLanesPerRow = DP / 8;
        const int r_in = lane / kLanesPerRow, pchunk = lane % kLanesPerRow;
        const int c = pchunk ^ tile_swz<DP>(kRowsPerInstr * wave + r_in);
        return c * 8 < D ? (r_in * D + c * 8) * 2 : 0x7fff0000;
    }
    __device__ __forceinline__ static void issue(i32x4_t rsrc, uint32_t tile_lds, int row0, int voff, int wave) {
#pragma unroll
        for (int i = 0; i < kPerWave; ++i) {
            const int q = wave + 4 * i;
            load_lds16(rsrc, tile_lds + 1024 * q, voff + (row0 + kRowsPerInstr * q) * D * 2, 0);
        }
    }
};

// One lane's MFMA operand of 8 head-dim values of row `row` (d = 16*s + 8*lg .. +7).
template <int D, int KS>
__device__ __forceinline__ void load_row_operand(const uint16_t* base, int64_t row, int lg, bf16x8_t (&f)[KS]) {
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        const int d0 = 16 * s + 8 * lg;
        f[s] = d0 < D ? *reinterpret_cast<const bf16x8_t*>(base + row * D + d0)
                      : __builtin_bit_cast(bf16x8_t, u32x4_t{0, 0, 0, 0});
    }
}

template <int D>
__device__ __forceinline__ void store_row4(void* base, bool bf16_out, int64_t row, int d, const float (&v)[4]) {
    if (d >= D) return;
    if (bf16_out) {
        u32x2_t w = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        *reinterpret_cast<u32x2_t*>(static_cast<uint16_t*>(base) + row * D + d) = w;
    } else {
        f32x4_t w = {v[0], v[1], v[2], v[3]};
        *reinterpret_cast<f32x4_t*>(static_cast<float*>(base) + row * D + d) = w;
    }
}

// One lane's gradient row in the rows output: head dims 32 dt + 8 g4 + 4 lg + e of row s of batch b,
// at column col of the token row. Each value is rounded to BF16 first (the planes' storage in the
// unfused composition), then rotated back in F32 by rope_rotate and rounded again: the result is
// bit-identical to writing the BF16 planes and running qkv_rope_merge on them. Split-half pairs
// (d, d + D/2) sit in fragments dt and dt + DT/2 of the lane, interleaved ones next to each other.
template <int D, int DT>
__device__ __forceinline__ void store_grad_row(const BwdArgs& a, int64_t b, int64_t s, int64_t col, bool rotate,
                                               int lg, const f32x16_t (&g)[DT]) {
    static_assert(D == 32 * DT && DT % 2 == 0, "rows output for D = 64 or 128");
    uint16_t* row = a.rows + (b * a.m + s) * a.row_w + col;
    const float* ct = a.rope_cos + s * (D / 2);
    const float* st = a.rope_sin + s * (D / 2);
    if (!rotate) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int d = 32 * dt + 8 * g4 + 4 * lg;
                *reinterpret_cast<u32x2_t*>(row + d) =
                    u32x2_t{pack_bf16x2(g[dt][4 * g4], g[dt][4 * g4 + 1]), pack_bf16x2(g[dt][4 * g4 + 2], g[dt][4 * g4 + 3])};
            }
    } else if (a.rope_layout == 1) {
#pragma unroll
        for (int dt = 0; dt < DT / 2; ++dt)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int d = 32 * dt + 8 * g4 + 4 * lg;
                const f32x4_t c = *reinterpret_cast<const f32x4_t*>(ct + d);
                const f32x4_t sn = *reinterpret_cast<const f32x4_t*>(st + d);
                float ya[4], yb[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    rope_rotate<true>(round_bf16(g[dt][4 * g4 + e]), round_bf16(g[dt + DT / 2][4 * g4 + e]), c[e], sn[e],
                                      ya[e], yb[e]);
                *reinterpret_cast<u32x2_t*>(row + d) = u32x2_t{pack_bf16x2(ya[0], ya[1]), pack_bf16x2(ya[2], ya[3])};
                *reinterpret_cast<u32x2_t*>(row + d + D / 2) =
                    u32x2_t{pack_bf16x2(yb[0], yb[1]), pack_bf16x2(yb[2], yb[3])};
            }
    } else {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int d = 32 * dt + 8 * g4 + 4 * lg;  // pairs (d, d + 1), (d + 2, d + 3)
                const f32x2_t c = *reinterpret_cast<const f32x2_t*>(ct + d / 2);
                const f32x2_t sn = *reinterpret_cast<const f32x2_t*>(st + d / 2);
                float y[4];
                rope_rotate<true>(round_bf16(g[dt][4 * g4]), round_bf16(g[dt][4 * g4 + 1]), c[0], sn[0], y[0], y[1]);
                rope_rotate<true>(round_bf16(g[dt][4 * g4 + 2]), round_bf16(g[dt][4 * g4 + 3]), c[1], sn[1], y[2], y[3]);
                *reinterpret_cast<u32x2_t*>(row + d) = u32x2_t{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
            }
    }
}

// N MFMAs, MFMA i taking the LDS operand fetch(i): the operand of MFMA i + kAhead is read while
// MFMA i runs, through a ring of kAhead + 1 registers, so no MFMA waits on an LDS round trip
// (left to itself, with the registers of these kernels in use, the compiler reads each
// operand into one register right before its MFMA). The fences and the empty asm are those of
// mfma_phase16.
template <int N, class Fetch, class Mma>
__device__ __forceinline__ void mfma_ring(Fetch&& fetch, Mma&& mma) {
    constexpr int R = kAhead + 1;
    bf16x8_t ring[R];
#pragma unroll
    for (int i = 0; i < kAhead && i < N; ++i) ring[i % R] = fetch(i);
#pragma unroll
    for (int i = 0; i < N; ++i) {
        if (i + kAhead < N) ring[(i + kAhead) % R] = fetch(i + kAhead);
        __builtin_amdgcn_sched_barrier(0);
        bf16x8_t x = ring[i % R];
        asm volatile("" : "+v"(x));
        mma(i, x);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// mfma_ring with between(i) after MFMA i: VALU work that does not depend on these MFMAs, issued
// while the matrix core runs them (one wave per SIMD: nothing else would fill the VALU).
template <int N, class Fetch, class Mma, class Between>
__device__ __forceinline__ void mfma_ring_x(Fetch&& fetch, Mma&& mma, Between&& between) {
    constexpr int R = kAhead + 1;
    bf16x8_t ring[R];
#pragma unroll
    for (int i = 0; i < kAhead && i < N; ++i) ring[i % R] = fetch(i);
#pragma unroll
    for (int i = 0; i < N; ++i) {
        if (i + kAhead < N) ring[(i + kAhead) % R] = fetch(i + kAhead);
        __builtin_amdgcn_sched_barrier(0);
        bf16x8_t x = ring[i % R];
        asm volatile("" : "+v"(x));
        mma(i, x);
        __builtin_amdgcn_sched_barrier(0);
        between(i);
        __builtin_amdgcn_sched_barrier(0);
    }
}

__device__ __forceinline__ uint32_t lds_address_f(const float* p) {
    return lds_address(reinterpret_cast<const uint16_t*>(p));
}

constexpr int kQStep = 64;    // queries per step of the dK/dV kernel
constexpr int kKBlock = 128;  // keys per dK/dV workgroup (4 waves x 32)

// dK (scaled here: the kernel leaves the softmax scale out of dS) and dV of key my_key of (b, kvh)
// from a lane's accumulators (head dims 32 dt + 8 g4 + 4 lg + e in acc[dt][4 g4 + e]): BF16/F32
// planes, or the rows output with RoPE's transpose on dK.
template <int D, int DT>
__device__ __forceinline__ void dkdv_store(const BwdArgs& a, int64_t b, int64_t kvh, int bkv, int64_t my_key, int lg,
                                           f32x16_t (&dk)[DT], f32x16_t (&dv)[DT]) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int v = 0; v < 16; ++v) dk[dt][v] *= a.scale;
    if constexpr (D >= 64) {
        if (a.rows != nullptr) {
            if (my_key < a.n) {
                store_grad_row<D, DT>(a, b, my_key, (a.heads + kvh) * D, true, lg, dk);
                store_grad_row<D, DT>(a, b, my_key, (a.heads + a.kv_heads + kvh) * D, false, lg, dv);
            }
            return;
        }
    }
    if (my_key < a.n) {
        const int64_t row = static_cast<int64_t>(bkv) * a.n + my_key;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int d = 32 * dt + 8 * g4 + 4 * lg;
                const float kv4[4] = {dk[dt][4 * g4], dk[dt][4 * g4 + 1], dk[dt][4 * g4 + 2], dk[dt][4 * g4 + 3]};
                const float vv4[4] = {dv[dt][4 * g4], dv[dt][4 * g4 + 1], dv[dt][4 * g4 + 2], dv[dt][4 * g4 + 3]};
                store_row4<D>(a.dk, a.dkv_bf16, row, d, kv4);
                store_row4<D>(a.dv, a.dkv_bf16, row, d, vv4);
            }
    }
}

// dK and dV of 128 keys of one (batch, KV head): loop over the group's query heads (in head
// order) and over 64-query steps, accumulating in registers; no atomics.
//   S = Q K^T and dP = dO V^T are computed with the queries as rows and this wave's 32 keys
//   as columns, so the accumulators (keys in lanes) are directly the B operands of
//   dV^T += dO^T P and dK^T += Q^T dS, whose A operands (dO^T, Q^T) come from the row-major
//   Q and dO tiles through transposing LDS reads.
//   The Q/dO tiles and the rows' statistics of step it+1 are fetched straight into LDS (no
//   staging registers) while step it is computed, and waited for before the barrier that ends
//   step it.
//   Split (a.splits > 1, for grids too small or too uneven to keep every CU busy: causal key
//   blocks near the start see every query, those near the end few of them): each head's query
//   steps of the key block are divided among a.splits workgroups (contiguous ranges), whose F32
//   partial sums attn_bwd_dkdv_reduce adds.
template <int D, bool SPLIT>
__global__ void __launch_bounds__(kThreads, 1)
attn_bwd_dkdv(BwdArgs a) {
    constexpr int DP = D < 32 ? 32 : D;
    constexpr int KS = DP / 16;
    constexpr int DT = DP / 32;
    using TDma = SwzTileDma<D, DP>;
    __shared__ __attribute__((aligned(1024))) uint16_t tiles[2][2][kQStep * DP];  // [buf][Q, dO]
    __shared__ __attribute__((aligned(256))) float stats[2][2][kQStep];          // [buf][lse*log2e, rowstat]

    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int lq = lane & 31, lg = lane >> 5;
    // logical order: (batch, KV head), key block heaviest first -- the workgroups resident on
    // one XCD read the same Q / dO heads
    const int logical = xcd_logical();
    const int splits = SPLIT ? a.splits : 1;
    const int bkv = logical / (a.blocks * splits);  // b * kv_heads + kvh
    const int nb = logical % (a.blocks * splits) / splits;
    const int split = SPLIT ? logical % splits : 0;
    const int64_t b = bkv / a.kv_heads;
    const int64_t group = a.heads / a.kv_heads;
    const int64_t kvh = bkv % a.kv_heads;
    const int64_t n0 = static_cast<int64_t>(nb) * kKBlock;
    const int64_t n0w = n0 + wave * 32;
    const int64_t my_key = n0w + lq;
    const uint16_t* K = a.k + (static_cast<int64_t>(bkv) * a.n) * D;
    const uint16_t* V = a.v + (static_cast<int64_t>(bkv) * a.n) * D;

    bf16x8_t kf[KS], vf[KS];
    {
        const int64_t kr = my_key < a.n ? my_key : a.n - 1;
        load_row_operand<D, KS>(K, kr, lg, kf);
        load_row_operand<D, KS>(V, kr, lg, vf);
    }
    settle(kf);
    settle(vf);
    f32x16_t dk[DT], dv[DT];
#pragma unroll
    for (int i = 0; i < DT; ++i) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            dk[i][v] = 0.0f;
            dv[i][v] = 0.0f;
        }
        asm volatile("" : "+a"(dk[i]));  // the accumulators live in the AGPR file
        asm volatile("" : "+a"(dv[i]));
    }

    // query steps that can see a key of this block: causal -> from the block's first key on
    int64_t qfirst = 0;
    if (a.causal) {
        qfirst = n0 - a.diag;
        qfirst = qfirst < 0 ? 0 : qfirst;
    }
    int step0 = static_cast<int>(qfirst / kQStep);
    int nsteps_head = qfirst < a.m ? static_cast<int>((a.m + kQStep - 1) / kQStep) - step0 : 0;
    if constexpr (SPLIT) {  // this split's share of each head's query steps
        const int chunk = (nsteps_head + splits - 1) / splits;
        const int s0 = min(split * chunk, nsteps_head), s1 = min(s0 + chunk, nsteps_head);
        step0 += s0;
        nsteps_head = s1 - s0;
    }
    const int total = nsteps_head * static_cast<int>(group);

    const int tile_voff = TDma::lane_offset(wave, lane);
    const int m32 = static_cast<int>(a.m);  // the launcher keeps m * D * 2 below 2^31
    // Loads of step it into buffer buf: this wave's share of the Q and dO tiles; waves 0 and 1
    // also fetch the 64 rows' lse*log2(e) and row statistic (rows past m read as zero).
    auto issue_step = [&](int it, int buf) {
        const int64_t bh = b * a.heads + kvh * group + it / nsteps_head;
        const int q0 = (step0 + it % nsteps_head) * kQStep;
        const i32x4_t rq = buffer_resource(a.q + bh * a.m * D, m32 * D * 2);
        const i32x4_t ro = buffer_resource(a.dout + bh * a.m * D, m32 * D * 2);
        TDma::issue(rq, lds_address(tiles[buf][0]), q0, tile_voff, wave);
        TDma::issue(ro, lds_address(tiles[buf][1]), q0, tile_voff, wave);
        if (wave < 2) {
            const float* src = (wave == 0 ? a.lse2 : a.stat) + bh * a.m;
            load_lds4(buffer_resource(src, m32 * 4), lds_address_f(stats[buf][wave]), (q0 + lane) * 4, 0);
        }
    };
    auto landed = [&]() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); };
    if (total > 0) issue_step(0, 0);
    landed();
    lds_barrier();

    for (int it = 0; it < total; ++it) {
        const int cur = it & 1;
        // buffer cur^1 was last read in step it-1, which the previous barrier closed
        if (it + 1 < total) issue_step(it + 1, cur ^ 1);
        const int64_t q0 = static_cast<int64_t>(step0 + it % nsteps_head) * kQStep;
        const uint16_t* Qt = tiles[cur][0];
        const uint16_t* Ot = tiles[cur][1];
        const bool skip = a.causal && (n0w > q0 + kQStep - 1 + a.diag);
        const int64_t bh_cur = b * a.heads + kvh * group + it / nsteps_head;
        const bool stores = a.ds && n0w < a.n;  // this wave's dS block exists
        // Steps whose 64 queries all see this wave's 32 keys (the common case) run a copy of the
        // step without the mask arithmetic; the others test one 32-bit offset per element:
        // query q0 + qq sees my_key iff qq + rel >= 0 (causal), qq < qlim and my_key < n.
        const bool full = (!a.causal || q0 + a.diag >= n0w + 31) && q0 + kQStep <= a.m && n0w + 32 <= a.n;
        auto step = [&](auto full_c) __attribute__((always_inline)) {
            constexpr bool FULL = decltype(full_c)::value;
            // Query tile qt of S (even i) and dP (odd i): MFMA i = 2 ks + which. The P / dS
            // arithmetic of tile 0 runs between the MFMAs of tile 1, that of tile 1 between the
            // dV / dK MFMAs of k-slices 0-1 (which use only tile 0): one wave per SIMD, so the
            // exponentials would otherwise leave the matrix core idle.
            f32x16_t s[2], dp[2];
            const f32x16_t zero = {};
            auto sdp = [&](int qt) {
                return [&, qt](int i) {
                    const int ks = i >> 1;
                    return tile_read16<DP>((i & 1) ? Ot : Qt, 32 * qt + lq, 2 * ks + lg);
                };
            };
            auto sdp_mma = [&](int qt) {
                return [&, qt](int i, bf16x8_t x) {
                    const int ks = i >> 1;
                    if (i & 1) dp[qt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, vf[ks], ks == 0 ? zero : dp[qt], 0, 0, 0);
                    else s[qt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, kf[ks], ks == 0 ? zero : s[qt], 0, 0, 0);
                };
            };
            // P and dS / scale (the scale is applied to dK once, at the end); lane holds key
            // my_key, queries q0 + 32*qt + 8*(v/4) + 4*lg + v%4.
            int64_t rel64 = q0 + a.diag - my_key;
            rel64 = rel64 < -(int64_t{1} << 30) ? -(int64_t{1} << 30) : (rel64 > (int64_t{1} << 30) ? (int64_t{1} << 30) : rel64);
            const int rel = a.causal ? static_cast<int>(rel64) : (1 << 30);
            const int qlim = static_cast<int>(a.m - q0 < kQStep ? a.m - q0 : kQStep);
            const bool key_ok = my_key < a.n;
            // score v of tile qt; the statistics of its 4 rows come in as one 16-byte read each
            f32x4_t l4, d4;
            auto pds = [&](int qt, int v) __attribute__((always_inline)) {
                const int qi = 32 * qt + 8 * (v >> 2) + 4 * lg + (v & 3);
                if ((v & 3) == 0) {
                    l4 = *reinterpret_cast<const f32x4_t*>(&stats[cur][0][qi]);
                    d4 = *reinterpret_cast<const f32x4_t*>(&stats[cur][1][qi]);
                }
                const float l = l4[v & 3], d = d4[v & 3];
                float p = fast_exp2(__builtin_fmaf(s[qt][v], a.scale_log2, -l));
                if constexpr (!FULL) p = key_ok && qi < qlim && qi + rel >= 0 ? p : 0.0f;
                s[qt][v] = p;
                dp[qt][v] = p * (dp[qt][v] - d);
            };
            // dV^T += dO^T P ; dK^T += Q^T dS  (k = 64 queries in 4 steps of 16), k-slices
            // 2h, 2h+1: MFMA i = 2 (DT kk + dt) + which, which 0: dV, 1: dK
            bf16x8_t pb[4], sb[4];
            auto dkv = [&](int h) {
                return [&, h](int i) {
                    const int ks = 2 * h + i / (2 * DT), dt = (i >> 1) % DT;
                    const int kb0 = 16 * ks + 4 * lg;
                    return tile_read_tr<DP>((i & 1) ? Qt : Ot, lane, kb0, kb0 + 8, 32 * dt);
                };
            };
            auto dkv_mma = [&](int h) {
                return [&, h](int i, bf16x8_t x) {
                    const int ks = 2 * h + i / (2 * DT), dt = (i >> 1) % DT;
                    if (i & 1) dk[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, sb[ks], dk[dt], 0, 0, 0);
                    else dv[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, pb[ks], dv[dt], 0, 0, 0);
                };
            };
            // dS of query tile qt (BF16, unscaled: the B operand of dK) into its block for the dQ
            // kernel: chunks 2 qt and 2 qt + 1, 1 KB each, two 16-byte stores per lane. Pairs past
            // N or M hold zeros (P is zero there), so the whole block is written. Non-temporal
            // stores: 2 GB of dS at C4 would otherwise push the shared Q / dO tiles out of L2.
            auto store_ds = [&](int qt) __attribute__((always_inline)) {
                char* blk = reinterpret_cast<char*>(a.ds) + ((bh_cur * a.nsq + q0 / kQStep) * a.nkb + n0w / 32) * 4096;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int c = 2 * qt + h;
                    stream_store(__builtin_bit_cast(u32x4_t, sb[c]), reinterpret_cast<u32x4_t*>(blk + c * 1024 + ds_slot(lane, c) * 16));
                }
            };
            // the 16 scores of a tile spread evenly over the ring's MFMAs (16 of them for D = 128)
            static_assert(16 % (2 * KS) == 0 && 16 % (4 * DT) == 0, "scores per MFMA");
            mfma_ring<2 * KS>(sdp(0), sdp_mma(0));
            mfma_ring_x<2 * KS>(sdp(1), sdp_mma(1), [&](int i) {
#pragma unroll
                for (int v = i * 16 / (2 * KS); v < (i + 1) * 16 / (2 * KS); ++v) pds(0, v);
            });
            pb[0] = pack_bf16x8(s[0], 0);
            pb[1] = pack_bf16x8(s[0], 8);
            sb[0] = pack_bf16x8(dp[0], 0);
            sb[1] = pack_bf16x8(dp[0], 8);
            mfma_ring_x<4 * DT>(dkv(0), dkv_mma(0), [&](int i) {
#pragma unroll
                for (int v = i * 16 / (4 * DT); v < (i + 1) * 16 / (4 * DT); ++v) pds(1, v);
            });
            pb[2] = pack_bf16x8(s[1], 0);
            pb[3] = pack_bf16x8(s[1], 8);
            sb[2] = pack_bf16x8(dp[1], 0);
            sb[3] = pack_bf16x8(dp[1], 8);
            mfma_ring<4 * DT>(dkv(1), dkv_mma(1));
            if (stores) {
                // after the step's last MFMA and the wait for step it+1's loads: the stores go into
                // an empty memory queue instead of stalling behind those loads mid-step
                landed();
                store_ds(0);
                store_ds(1);
            }
        };
        if (!skip) {
            if (full) step(std::integral_constant<bool, true>{});
            else step(std::integral_constant<bool, false>{});
        }
        // a step that stored dS has waited for its loads before the stores, which complete
        // within the next step (whose own wait covers them)
        if (!stores || skip) landed();
        lds_barrier();
    }

    if constexpr (SPLIT) {
        // this split's sums (dK scaled) as F32 planes: the store path of the unsplit kernel, with
        // the partial planes as its dK and dV
        BwdArgs pa = a;
        const int64_t nkv = a.n * (static_cast<int64_t>(gridDim.x) / (a.blocks * splits));
        pa.dk = a.partial + static_cast<int64_t>(split) * 2 * nkv * D;
        pa.dv = a.partial + (static_cast<int64_t>(split) * 2 + 1) * nkv * D;
        pa.dkv_bf16 = 0;
        pa.rows = nullptr;
        dkdv_store<D, DT>(pa, b, kvh, bkv, my_key, lg, dk, dv);
    } else {
        dkdv_store<D, DT>(a, b, kvh, bkv, my_key, lg, dk, dv);
    }
}

// The splits' F32 partial dK (scaled) and dV of 128 keys of one (batch, KV head), added in split
// order and stored by dkdv_store (BF16/F32 planes or rows output; scale 1, the partials carry it)
// in the dK/dV kernel's lane layout: the result is what that kernel stores unsplit, up to the
// order of the F32 additions.
template <int D>
__global__ void __launch_bounds__(kThreads)
attn_bwd_dkdv_reduce(BwdArgs a) {
    constexpr int DP = D < 32 ? 32 : D;
    constexpr int DT = DP / 32;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lq = lane & 31, lg = lane >> 5;
    const int bkv = blockIdx.x / a.blocks, nb = blockIdx.x % a.blocks;
    const int64_t b = bkv / a.kv_heads, kvh = bkv % a.kv_heads;
    const int64_t my_key = static_cast<int64_t>(nb) * kKBlock + wave * 32 + lq;
    if (my_key >= a.n) return;
    const int64_t nkv = a.n * static_cast<int64_t>(gridDim.x / a.blocks);
    f32x16_t dk[DT], dv[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int v = 0; v < 16; ++v) dk[dt][v] = dv[dt][v] = 0.0f;
    for (int sp = 0; sp < a.splits; ++sp) {
        const float* pk = a.partial + ((static_cast<int64_t>(sp) * 2) * nkv + static_cast<int64_t>(bkv) * a.n + my_key) * D;
        const float* pv = pk + nkv * D;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int d = 32 * dt + 8 * g4 + 4 * lg;
                if (d >= D) continue;
                const f32x4_t k4 = *reinterpret_cast<const f32x4_t*>(pk + d);
                const f32x4_t v4 = *reinterpret_cast<const f32x4_t*>(pv + d);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    dk[dt][4 * g4 + e] += k4[e];
                    dv[dt][4 * g4 + e] += v4[e];
                }
            }
    }
    BwdArgs ra = a;
    ra.scale = 1.0f;
    dkdv_store<D, DT>(ra, b, kvh, bkv, my_key, lg, dk, dv);
}

// dQ of 128 queries of one (batch, head), looping over 64-key tiles up to the diagonal:
// S^T = K Q^T and dP^T = V dO^T with keys as rows (each lane owns one query, so the softmax
// row statistics are per-lane scalars), dS^T is the B operand of dQ^T += K^T dS^T with K^T
// read from the row-major K tile through transposing LDS reads. The K/V tiles of step j+1 are
// fetched straight into LDS while step j is computed.
template <int D>
__global__ void __launch_bounds__(kThreads, 1)
attn_bwd_dq(BwdArgs a) {
    constexpr int DP = D < 32 ? 32 : D;
    constexpr int KS = DP / 16;
    constexpr int DT = DP / 32;
    using TDma = SwzTileDma<D, DP>;
    __shared__ __attribute__((aligned(1024))) uint16_t lds[2][2][kBlockN * DP];  // [buf][K, V]

    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int lq = lane & 31, lg = lane >> 5;
    // same logical order as the forward kernel: KV head group, query block heaviest first,
    // query head in the group
    const int logical = xcd_logical();
    const int group_heads = static_cast<int>(a.heads / a.kv_heads);
    const int per_group = a.blocks * group_heads;
    const int grp = logical / per_group, in_grp = logical % per_group;
    const int mb = a.blocks - 1 - in_grp / group_heads;
    const int64_t b = grp / a.kv_heads, kvh = grp % a.kv_heads;
    const int64_t h = kvh * group_heads + in_grp % group_heads;
    const int64_t bh = b * a.heads + h;
    const uint16_t* K = a.k + ((b * a.kv_heads + kvh) * a.n) * D;
    const uint16_t* V = a.v + ((b * a.kv_heads + kvh) * a.n) * D;
    const int64_t q0 = static_cast<int64_t>(mb) * kBlockM;
    const int64_t q0w = q0 + wave * 32;
    const int64_t my_q = q0w + lq;
    const int64_t qr = my_q < a.m ? my_q : a.m - 1;

    bf16x8_t qf[KS], of[KS];
    load_row_operand<D, KS>(a.q + static_cast<int64_t>(bh) * a.m * D, qr, lg, qf);
    load_row_operand<D, KS>(a.dout + static_cast<int64_t>(bh) * a.m * D, qr, lg, of);
    float lse2 = a.lse2[static_cast<int64_t>(bh) * a.m + qr];
    float rstat = a.stat[static_cast<int64_t>(bh) * a.m + qr];
    settle(qf);
    settle(of);
    settle(lse2);
    settle(rstat);

    f32x16_t dq[DT];
#pragma unroll
    for (int i = 0; i < DT; ++i) {
#pragma unroll
        for (int v = 0; v < 16; ++v) dq[i][v] = 0.0f;
        asm volatile("" : "+a"(dq[i]));
    }

    int64_t kv_end = a.n;
    if (a.causal) {
        const int64_t last = q0 + kBlockM - 1 + a.diag;
        kv_end = last + 1 < kv_end ? last + 1 : kv_end;
    }
    const int ntiles = kv_end > 0 ? static_cast<int>((kv_end + kBlockN - 1) / kBlockN) : 0;

    const int tile_voff = TDma::lane_offset(wave, lane);
    const int n32 = static_cast<int>(a.n);  // the launcher keeps n * D * 2 below 2^31
    const i32x4_t rk = buffer_resource(K, n32 * D * 2);
    const i32x4_t rv = buffer_resource(V, n32 * D * 2);
    auto issue_tile = [&](int j, int buf) {
        TDma::issue(rk, lds_address(lds[buf][0]), j * kBlockN, tile_voff, wave);
        TDma::issue(rv, lds_address(lds[buf][1]), j * kBlockN, tile_voff, wave);
    };
    auto landed = [&]() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); };
    if (ntiles > 0) issue_tile(0, 0);
    landed();
    lds_barrier();

    for (int j = 0; j < ntiles; ++j) {
        const int cur = j & 1;
        if (j + 1 < ntiles) issue_tile(j + 1, cur ^ 1);
        const int64_t kv0 = static_cast<int64_t>(j) * kBlockN;
        const uint16_t* Kt = lds[cur][0];
        const uint16_t* Vt = lds[cur][1];
        const bool skip = a.causal && (kv0 > q0w + 31 + a.diag);
        // Tiles whose 64 keys all lie at or below every query of this wave run a copy of the
        // step without the mask arithmetic; the others compare one 32-bit offset per element
        // (key offset <= rel, < klim).
        const bool full = (!a.causal || kv0 + kBlockN - 1 <= q0w + a.diag) && q0w + 32 <= a.m &&
                          kv0 + kBlockN <= a.n;
        auto step = [&](auto full_c) __attribute__((always_inline)) {
            constexpr bool FULL = decltype(full_c)::value;
            // S^T (even i) and dP^T (odd i) of key tile tt: MFMA i = 2 ks + which. The P / dS
            // arithmetic of key tile 0 runs between the MFMAs of key tile 1, that of key tile 1
            // between the dQ MFMAs of k-slices 0-1 (which use only key tile 0): one wave per SIMD,
            // so the exponentials would otherwise leave the matrix core idle.
            f32x16_t s[2], dp[2];
            const f32x16_t zero = {};
            auto sdp = [&](int tt) {
                return [&, tt](int i) { return tile_read16<DP>((i & 1) ? Vt : Kt, 32 * tt + lq, 2 * (i >> 1) + lg); };
            };
            auto sdp_mma = [&](int tt) {
                return [&, tt](int i, bf16x8_t x) {
                    const int ks = i >> 1;
                    if (i & 1) dp[tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, of[ks], ks == 0 ? zero : dp[tt], 0, 0, 0);
                    else s[tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, qf[ks], ks == 0 ? zero : s[tt], 0, 0, 0);
                };
            };
            // Lane holds query my_q, keys kv0 + 32*tt + 8*(v/4) + 4*lg + v%4; dS / scale (the scale
            // is applied to dQ once, at the end).
            int64_t rel64 = my_q + a.diag - kv0;
            rel64 = rel64 < -(int64_t{1} << 30) ? -(int64_t{1} << 30) : (rel64 > (int64_t{1} << 30) ? (int64_t{1} << 30) : rel64);
            const int rel = (a.causal ? static_cast<int>(rel64) : (1 << 30)) - 4 * lg;
            const int klim = static_cast<int>(a.n - kv0 < kBlockN ? a.n - kv0 : kBlockN) - 4 * lg;
            const bool q_ok = my_q < a.m;
            auto pds = [&](int tt, int v) __attribute__((always_inline)) {
                float p = fast_exp2(__builtin_fmaf(s[tt][v], a.scale_log2, -lse2));
                if constexpr (!FULL) {
                    const int kk = 32 * tt + (v >> 2) * 8 + (v & 3);
                    p = q_ok && kk <= rel && kk < klim ? p : 0.0f;
                }
                dp[tt][v] = p * (dp[tt][v] - rstat);
            };
            // dQ^T += K^T dS^T over k-slices 2h, 2h+1 (keys 32h .. 32h+31): MFMA i = DT kk + dt
            bf16x8_t sb[4];
            auto dqf = [&](int h) {
                return [&, h](int i) {
                    const int kb0 = 16 * (2 * h + i / DT) + 4 * lg;
                    return tile_read_tr<DP>(Kt, lane, kb0, kb0 + 8, 32 * (i % DT));
                };
            };
            auto dq_mma = [&](int h) {
                return [&, h](int i, bf16x8_t x) {
                    const int dt = i % DT;
                    dq[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, sb[2 * h + i / DT], dq[dt], 0, 0, 0);
                };
            };
            static_assert(16 % (2 * KS) == 0 && 16 % (2 * DT) == 0, "scores per MFMA");
            mfma_ring<2 * KS>(sdp(0), sdp_mma(0));
            mfma_ring_x<2 * KS>(sdp(1), sdp_mma(1), [&](int i) {
#pragma unroll
                for (int v = i * 16 / (2 * KS); v < (i + 1) * 16 / (2 * KS); ++v) pds(0, v);
            });
            sb[0] = pack_bf16x8(dp[0], 0);
            sb[1] = pack_bf16x8(dp[0], 8);
            mfma_ring_x<2 * DT>(dqf(0), dq_mma(0), [&](int i) {
#pragma unroll
                for (int v = i * 16 / (2 * DT); v < (i + 1) * 16 / (2 * DT); ++v) pds(1, v);
            });
            sb[2] = pack_bf16x8(dp[1], 0);
            sb[3] = pack_bf16x8(dp[1], 8);
            mfma_ring<2 * DT>(dqf(1), dq_mma(1));
        };
        if (!skip) {
            if (full) step(std::integral_constant<bool, true>{});
            else step(std::integral_constant<bool, false>{});
        }
        landed();
        lds_barrier();
    }

#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int v = 0; v < 16; ++v) dq[dt][v] *= a.scale;
    if constexpr (D >= 64) {
        if (a.rows != nullptr) {
            if (my_q < a.m) store_grad_row<D, DT>(a, b, my_q, h * D, true, lg, dq);
            return;
        }
    }
    if (my_q < a.m) {
        const int64_t row = static_cast<int64_t>(bh) * a.m + my_q;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const float v4[4] = {dq[dt][4 * g4], dq[dt][4 * g4 + 1], dq[dt][4 * g4 + 2], dq[dt][4 * g4 + 3]};
                store_row4<D>(a.dq, a.dq_bf16, row, 32 * dt + 8 * g4 + 4 * lg, v4);
            }
    }
}

// dQ of 128 queries of one (batch, head) from the dS blocks that attn_bwd_dkdv stored: one
// GEMM, dQ^T += K^T dS^T over 64-key tiles up to the diagonal, with no S or dP recomputed. A
// tile's dS is four blocks (two of 32 keys x two of 64 queries, 16 KB) copied verbatim into LDS;
// the B operand (this lane's query, 8 keys) comes from them through transposing reads (each lane
// reads 4 consecutive queries of one key, 8 contiguous bytes of a block), and K^T from the
// row-major K tile as in attn_bwd_dq, with the same key order inside each MFMA k-group on both
// sides. The dS blocks go straight into LDS two tiles ahead (three buffers), the K tile one
// tile ahead (two), and two workgroups share a CU. Blocks that no query sees may never have been written: on tiles that hold such pairs
// the operand is masked (the causal test of attn_bwd_dkdv), so stale memory never reaches an
// MFMA; blocks past this head's read as zero. Queries past M feed only dQ^T columns that are not
// stored. Keys past N in a block that exists (the next query row's first blocks) are masked too.
template <int D>
__global__ void __launch_bounds__(kThreads, 2)
attn_bwd_dq_ds(BwdArgs a) {
    constexpr int DP = D < 32 ? 32 : D;
    constexpr int DT = DP / 32;
    using TDma = SwzTileDma<D, DP>;
    // dS (from HBM) runs two tiles ahead through three buffers, K (from L2) one tile ahead
    // through two: 80 KB at D = 128, two workgroups per CU
    __shared__ __attribute__((aligned(1024))) uint16_t k_lds[2][kBlockN * DP];
    __shared__ __attribute__((aligned(1024))) uint16_t ds_lds[3][4 * 2048];  // 4 blocks of 4 KB
    constexpr int kDsInstr = 4;  // global->LDS instructions per wave per dS tile

    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int lq = lane & 31, lg = lane >> 5;
    // the order of attn_bwd_dq: KV head group, query block heaviest first, query head in the group
    const int logical = xcd_logical();
    const int group_heads = static_cast<int>(a.heads / a.kv_heads);
    const int per_group = a.blocks * group_heads;
    const int grp = logical / per_group, in_grp = logical % per_group;
    const int mb = a.blocks - 1 - in_grp / group_heads;
    const int64_t b = grp / a.kv_heads, kvh = grp % a.kv_heads;
    const int64_t h = kvh * group_heads + in_grp % group_heads;
    const int64_t bh = b * a.heads + h;
    const uint16_t* K = a.k + ((b * a.kv_heads + kvh) * a.n) * D;
    const int64_t q0 = static_cast<int64_t>(mb) * kBlockM;
    const int64_t q0w = q0 + wave * 32;
    const int64_t my_q = q0w + lq;

    f32x16_t dq[DT];
#pragma unroll
    for (int i = 0; i < DT; ++i) {
#pragma unroll
        for (int v = 0; v < 16; ++v) dq[i][v] = 0.0f;
        asm volatile("" : "+a"(dq[i]));
    }

    int64_t kv_end = a.n;
    if (a.causal) {
        const int64_t last = q0 + kBlockM - 1 + a.diag;
        kv_end = last + 1 < kv_end ? last + 1 : kv_end;
    }
    const int ntiles = kv_end > 0 ? static_cast<int>((kv_end + kBlockN - 1) / kBlockN) : 0;

    const int tile_voff = TDma::lane_offset(wave, lane);
    const int n32 = static_cast<int>(a.n);  // the launcher keeps n * D * 2 below 2^31
    const int nkb = static_cast<int>(a.nkb);
    const i32x4_t rk = buffer_resource(K, n32 * D * 2);
    // this head's blocks (the launcher keeps nkb * nsq * 4096 below 2^31)
    const i32x4_t rds = buffer_resource(reinterpret_cast<const char*>(a.ds) + bh * a.nkb * a.nsq * 4096,
                                        static_cast<int>(a.nkb * a.nsq * 4096));
    // DMA instruction q = wave + 4 i of the 16: block q / 4 = 2 (key half) + query half, chunk q % 4
    auto issue_k = [&](int j, int buf) { TDma::issue(rk, lds_address(k_lds[buf]), j * kBlockN, tile_voff, wave); };
    auto issue_ds = [&](int j, int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q = wave + 4 * i, blk = q >> 2;
            const int src = ((2 * mb + (blk & 1)) * nkb + 2 * j + (blk >> 1)) * 4096 + (q & 3) * 1024;
            load_lds16_nt(rds, lds_address(ds_lds[buf]) + 1024 * q, src + 16 * lane, 0);
        }
    };
    // B operand reads: lane (lg, g = lane/16 % 2, i = lane % 16) reads key kbase + i/4 of its
    // transposing group, queries 32 wave + 16 g + 4 (i % 4) .. +3: block (key / 32, wave / 2),
    // chunk 2 (wave % 2) + g, k-group lane (key % 32) + 32 (i % 2), element 4 ((i % 4) / 2).
    const int tg = (lane >> 4) & 1, ti = lane & 15;
    const int chunk = 2 * (wave & 1) + tg;
    auto ds_read = [&](const uint16_t* St, int kbase) __attribute__((always_inline)) {
        const int kk = kbase + (ti >> 2);
        const int L = (kk & 31) + 32 * (ti & 1);
        const int byte = (2 * (kk >> 5) + (wave >> 1)) * 4096 + chunk * 1024 + ds_slot(L, chunk) * 16 + 8 * ((ti & 3) >> 1);
        return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(reinterpret_cast<const char*>(St) + byte));
    };
    // Loads complete in issue order: when the last loads issued are dS tile t's, vmcnt(kDsInstr)
    // means everything issued before them has landed.
    auto landed = [&]() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); };
    auto landed_but_ds = [&]() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kDsInstr) : "memory"); };
    if (ntiles > 0) {
        issue_k(0, 0);
        issue_ds(0, 0);
    }
    if (ntiles > 1) {
        issue_ds(1, 1);
        landed_but_ds();
    } else {
        landed();
    }
    lds_barrier();

    int cur = 0;  // dS buffer of tile j (j % 3); K's is j % 2
    for (int j = 0; j < ntiles; ++j) {
        // K buffer (j+1) % 2 and dS buffer (j+2) % 3 were last read in step j-1, which the
        // previous barrier closed
        if (j + 1 < ntiles) issue_k(j + 1, (j + 1) & 1);
        if (j + 2 < ntiles) issue_ds(j + 2, cur == 0 ? 2 : cur - 1);
        const int64_t kv0 = static_cast<int64_t>(j) * kBlockN;
        const uint16_t* Kt = k_lds[j & 1];
        const uint16_t* St = ds_lds[cur];
        const bool skip = a.causal && (kv0 > q0w + 31 + a.diag);
        // every key of the tile visible to every query of the wave, and below N
        const bool full = (!a.causal || kv0 + kBlockN - 1 <= q0w + a.diag) && kv0 + kBlockN <= a.n;
        if (!skip) {
            int64_t rel64 = my_q + a.diag - kv0;
            rel64 = rel64 < -(int64_t{1} << 30) ? -(int64_t{1} << 30) : (rel64 > (int64_t{1} << 30) ? (int64_t{1} << 30) : rel64);
            const int rel = a.causal ? static_cast<int>(rel64) : (1 << 30);
            const int klim = static_cast<int>(a.n - kv0 < kBlockN ? a.n - kv0 : kBlockN);
            // B operands of the four 16-key slices: keys 16 ks + 4 lg + {0..3, 8..11}
            bf16x8_t sb[4];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const int kb0 = 16 * ks + 4 * lg;
                const v4i16_t lo = ds_read(St, kb0), hi = ds_read(St, kb0 + 8);
                typedef short v8i16_t __attribute__((ext_vector_type(8)));
                v8i16_t e = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                if (!full) {
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const int kk = kb0 + (u < 4 ? u : u + 4);
                        e[u] = kk <= rel && kk < klim ? e[u] : static_cast<short>(0);
                    }
                }
                sb[ks] = __builtin_bit_cast(bf16x8_t, e);
            }
            mfma_ring<4 * DT>(
                [&](int i) {
                    const int kb0 = 16 * (i / DT) + 4 * lg;
                    return tile_read_tr<DP>(Kt, lane, kb0, kb0 + 8, 32 * (i % DT));
                },
                [&](int i, bf16x8_t x) {
                    const int dt = i % DT;
                    dq[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, sb[i / DT], dq[dt], 0, 0, 0);
                });
        }
        // K and dS of tile j+1 must have landed; dS tile j+2's loads may stay in flight
        if (j + 2 < ntiles) landed_but_ds();
        else landed();
        lds_barrier();
        cur = cur == 2 ? 0 : cur + 1;
    }

#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int v = 0; v < 16; ++v) dq[dt][v] *= a.scale;
    if constexpr (D >= 64) {
        if (a.rows != nullptr) {
            if (my_q < a.m) store_grad_row<D, DT>(a, b, my_q, h * D, true, lg, dq);
            return;
        }
    }
    if (my_q < a.m) {
        const int64_t row = static_cast<int64_t>(bh) * a.m + my_q;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const float v4[4] = {dq[dt][4 * g4], dq[dt][4 * g4 + 1], dq[dt][4 * g4 + 2], dq[dt][4 * g4 + 3]};
                store_row4<D>(a.dq, a.dq_bf16, row, 32 * dt + 8 * g4 + 4 * lg, v4);
            }
    }
}

// The stored-dS backward (attn_bwd_dkdv writing dS blocks, attn_bwd_dq_ds reading them) applies
// when a head's blocks have 32-bit byte offsets and all of them fit the dS budget: 8 GiB, or the
// byte count in the environment variable HK_ATTN_DS_BUDGET (read on every call; 0 turns the path
// off). Otherwise attn_bwd_dq recomputes S and dP, with no workspace beyond the row statistics.
int64_t ds_budget() {
    const char* env = std::getenv("HK_ATTN_DS_BUDGET");
    if (env == nullptr || *env == '\0') return int64_t{8} << 30;
    char* end = nullptr;
    const long long v = std::strtoll(env, &end, 10);
    return end != nullptr && *end == '\0' && v >= 0 ? static_cast<int64_t>(v) : int64_t{8} << 30;
}
int64_t ds_head_bytes(const AttnShape& sh) { return ((sh.n + 31) / 32) * ((sh.m + kQStep - 1) / kQStep) * 4096; }
bool bwd_stores_ds(const AttnShape& sh) {
    // the dQ kernel's block offsets reach one query row of blocks past the last
    const int64_t reach = ds_head_bytes(sh) + ((sh.n + 31) / 32 + 2) * 4096;
    return reach < (int64_t{1} << 31) && sh.batch * sh.heads * ds_head_bytes(sh) <= ds_budget();
}
size_t ds_bytes(const AttnShape& sh) {
    return sh.store_ds ? static_cast<size_t>(sh.batch * sh.heads * ds_head_bytes(sh)) : 0;
}
size_t stat_bytes(const AttnShape& sh) {  // row statistic and lse2, rounded to 256 bytes
    return (2 * static_cast<size_t>(sh.batch * sh.heads * sh.m) * sizeof(float) + 255) & ~size_t(255);
}

// Workgroups per dK/dV key block: causal key blocks near the start of the sequence see every
// query and those near its end few of them, so a grid of one round of workgroups (C5: 256 key
// blocks on 256 CUs) takes as long as its heaviest block, ~1.9x the average at C5. Splitting
// every block's steps s ways (s = 2 or 4) lets the dispatcher fill the CUs evenly: s is the
// smallest whose heaviest share is at most the average work per CU, i.e. ratio = heaviest block x
// CUs / all blocks' work <= s (1 when the ratio is at most 1: C4's four rounds already balance).
// The environment variable HK_ATTN_DKV_SPLITS (1, 2 or 4) overrides the choice.
int dkv_splits_for(const AttnShape& sh, int num_cus) {
    if (const char* env = std::getenv("HK_ATTN_DKV_SPLITS")) {
        const int v = std::atoi(env);
        if (v == 1 || v == 2 || v == 4) return v;
    }
    const int64_t blocks = (sh.n + kKBlock - 1) / kKBlock, qsteps = (sh.m + kQStep - 1) / kQStep;
    const int64_t group = sh.heads / sh.kv_heads, diag = clamp_diag(sh);
    int64_t heaviest = 0, work = 0;
    for (int64_t nb = 0; nb < blocks; ++nb) {
        const int64_t qfirst = sh.causal ? std::max<int64_t>(nb * kKBlock - diag, 0) : 0;
        const int64_t steps = qfirst < sh.m ? (qsteps - qfirst / kQStep) * group : 0;
        heaviest = std::max(heaviest, steps);
        work += steps;
    }
    work *= sh.batch * sh.kv_heads;
    if (work == 0) return 1;
    const double ratio = static_cast<double>(heaviest) * num_cus / static_cast<double>(work);
    return ratio <= 1.0 ? 1 : (ratio <= 2.0 ? 2 : 4);
}
size_t partial_bytes(const AttnShape& sh) {  // the split's F32 dK and dV partial sums
    return sh.dkv_splits > 1 ? static_cast<size_t>(sh.dkv_splits) * 2 * sh.batch * sh.kv_heads * sh.n * sh.d * 4 : 0;
}

template <int D>
hipError_t launch_bwd(const AttnShape& sh, const void* q, const void* k, const void* v, const void* o,
                      const float* lse, const void* dout, void* dq, int dq_bf16, void* dk, void* dv, int dkv_bf16,
                      const AttnRowsOut* rows_out, float* stat, uint16_t* ds, float* partial, hipStream_t s) {
    const int64_t rows = sh.batch * sh.heads * sh.m;
    constexpr int lanes = D / 8;
    const int64_t threads = rows * lanes;
    float* lse2 = stat + rows;
    if (sh.o_f32)
        hipLaunchKernelGGL((attn_bwd_rowstat<D, float>), dim3(flat_blocks(threads, 256)), dim3(256), 0, s,
                           static_cast<const float*>(o), static_cast<const uint16_t*>(dout), lse, stat, lse2, rows);
    else
        hipLaunchKernelGGL((attn_bwd_rowstat<D, uint16_t>), dim3(flat_blocks(threads, 256)), dim3(256), 0, s,
                           static_cast<const uint16_t*>(o), static_cast<const uint16_t*>(dout), lse, stat, lse2, rows);
    BwdArgs a;
    a.q = static_cast<const uint16_t*>(q);
    a.k = static_cast<const uint16_t*>(k);
    a.v = static_cast<const uint16_t*>(v);
    a.dout = static_cast<const uint16_t*>(dout);
    a.lse2 = lse2;
    a.stat = stat;
    a.dq = dq;
    a.dk = dk;
    a.dv = dv;
    a.heads = sh.heads;
    a.kv_heads = sh.kv_heads;
    a.m = sh.m;
    a.n = sh.n;
    a.diag = clamp_diag(sh);
    a.scale = sh.scale;
    a.scale_log2 = sh.scale * kLog2e;
    a.causal = sh.causal;
    a.dq_bf16 = dq_bf16;
    a.dkv_bf16 = dkv_bf16;
    a.blocks = static_cast<int>((sh.n + kKBlock - 1) / kKBlock);
    a.ds = ds;
    a.nkb = (sh.n + 31) / 32;
    a.nsq = (sh.m + kQStep - 1) / kQStep;
    a.rows = rows_out ? static_cast<uint16_t*>(rows_out->rows) : nullptr;
    a.row_w = rows_out ? rows_out->row_w : 0;
    a.rope_cos = rows_out ? rows_out->cos : nullptr;
    a.rope_sin = rows_out ? rows_out->sin : nullptr;
    a.rope_layout = rows_out ? rows_out->layout : 0;
    a.splits = sh.dkv_splits;
    a.partial = partial;
    const dim3 dkdv_grid(static_cast<unsigned>(sh.batch * sh.kv_heads * a.blocks * a.splits));
    if (a.splits > 1) {
        hipLaunchKernelGGL((attn_bwd_dkdv<D, true>), dkdv_grid, dim3(kThreads), 0, s, a);
        hipLaunchKernelGGL((attn_bwd_dkdv_reduce<D>), dim3(static_cast<unsigned>(sh.batch * sh.kv_heads * a.blocks)),
                           dim3(kThreads), 0, s, a);
    } else {
        hipLaunchKernelGGL((attn_bwd_dkdv<D, false>), dkdv_grid, dim3(kThreads), 0, s, a);
    }
    a.blocks = static_cast<int>((sh.m + kBlockM - 1) / kBlockM);
    if (ds)
        hipLaunchKernelGGL((attn_bwd_dq_ds<D>), dim3(static_cast<unsigned>(sh.batch * sh.heads * a.blocks)),
                           dim3(kThreads), 0, s, a);
    else
        hipLaunchKernelGGL((attn_bwd_dq<D>), dim3(static_cast<unsigned>(sh.batch * sh.heads * a.blocks)),
                           dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace

bool attention_shape_fits(const AttnShape& sh) {
    constexpr int64_t kOffsetLimit = int64_t{1} << 31, kItemLimit = int64_t{1} << 32;
    if (sh.m * sh.d * 2 >= kOffsetLimit || sh.n * sh.d * 2 >= kOffsetLimit) return false;
    const bool pp = sh.d >= 64;
    const int64_t fwd_rows = pp ? kPPBlockM : kBlockM, fwd_threads = pp ? kPPThreads : kThreads;
    const int64_t fwd = sh.batch * sh.heads * ((sh.m + fwd_rows - 1) / fwd_rows) * fwd_threads;
    const int64_t dkdv = sh.batch * sh.kv_heads * ((sh.n + kKBlock - 1) / kKBlock) * kThreads;
    const int64_t dq = sh.batch * sh.heads * ((sh.m + kBlockM - 1) / kBlockM) * kThreads;
    return fwd < kItemLimit && dkdv < kItemLimit && dq < kItemLimit;
}

void attention_bwd_plan(AttnShape& sh, int num_cus) {
    sh.store_ds = bwd_stores_ds(sh) ? 1 : 0;
    sh.dkv_splits = dkv_splits_for(sh, num_cus);
}

size_t attention_bwd_workspace_bytes(const AttnShape& sh) {
    return stat_bytes(sh) + ((ds_bytes(sh) + 255) & ~size_t(255)) + partial_bytes(sh);
}

hipError_t attention_forward(const AttnShape& sh, const void* q, const void* k, const void* v, void* o, float* lse,
                             hipStream_t s) {
    switch (sh.d) {
        case 16: return launch_fwd<16>(sh, q, k, v, o, lse, s);
        case 32: return launch_fwd<32>(sh, q, k, v, o, lse, s);
        case 64: return launch_fwd<64>(sh, q, k, v, o, lse, s);
        case 128: return launch_fwd<128>(sh, q, k, v, o, lse, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t attention_backward(const AttnShape& sh, const void* q, const void* k, const void* v, const void* o,
                              const float* lse, const void* dout, void* dq, int dq_bf16, void* dk, void* dv,
                              int dkv_bf16, const AttnRowsOut* rows, void* workspace, hipStream_t s) {
    float* stat = static_cast<float*>(workspace);
    char* after_stat = static_cast<char*>(workspace) + stat_bytes(sh);
    uint16_t* ds = sh.store_ds ? reinterpret_cast<uint16_t*>(after_stat) : nullptr;
    float* partial = sh.dkv_splits > 1 ? reinterpret_cast<float*>(after_stat + ((ds_bytes(sh) + 255) & ~size_t(255)))
                                       : nullptr;
    if (rows && sh.d != 64 && sh.d != 128) return hipErrorInvalidValue;
    switch (sh.d) {
        case 16: return launch_bwd<16>(sh, q, k, v, o, lse, dout, dq, dq_bf16, dk, dv, dkv_bf16, nullptr, stat, ds, partial, s);
        case 32: return launch_bwd<32>(sh, q, k, v, o, lse, dout, dq, dq_bf16, dk, dv, dkv_bf16, nullptr, stat, ds, partial, s);
        case 64: return launch_bwd<64>(sh, q, k, v, o, lse, dout, dq, dq_bf16, dk, dv, dkv_bf16, rows, stat, ds, partial, s);
        case 128: return launch_bwd<128>(sh, q, k, v, o, lse, dout, dq, dq_bf16, dk, dv, dkv_bf16, rows, stat, ds, partial, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace hk
