// hk_gemm_device.hpp — device code of the 256x256-tile BF16 GEMM (gfx950), shared by libhk.so
// (hk_gemm.hip) and the ahead-of-time code object of device programs (hk_programs.hip).
//
// Semantics (reference rust-ascend-kernels/src/kernel.rs:5-76, ascend.rs:22-68):
//   C[g, i, j] = sum_k A'[g, i, k] * B'[g, k, j]  with FP32 accumulation, C stored as BF16
//   (RNE) or F32; A' is A ([M,K]) or A^T (A stored [K,M]); B' is B ([K,N]) or B^T (B [N,K]).
#pragma once

#include "hk_common.hpp"

namespace hk {

namespace {

struct GemmArgs {
    const uint16_t* a;  // [batch][m][k]
    const uint16_t* b;  // [batch][n][k], or [groups][n][k] for the M-grouped form
    void* c;            // [batch][m][n]
    int m, n, k;
    int tiles_m, tiles_n;
    // M-grouped form (batch 1): block_group[r / 256] is the weight slice of rows r of A and C.
    // Group ends are multiples of 256, so an output tile (256, 128 or 64 rows) has one group.
    const int32_t* block_group;
    // 4-wave kernel tile order: 0 = bands of 4 M-tile rows per XCD, else bands of this many
    // N-tile columns.
    int band_n;
};

// The decoder layer's fused QKV projection: the product's columns are Hq + 2 Hkv heads of 128
// (Q heads, then K, then V) and its rows are tokens b * seq + s. Instead of the [T, W] rows, each
// head's 128 columns go to its plane q [B, Hq, seq, 128] or k, v [B, Hkv, seq, 128], Q and K
// rotated on the way (RoPE with F32 tables [seq, 64] indexed by s).
struct QkvRopeOut {
    uint16_t* q;
    uint16_t* k;
    uint16_t* v;
    const float* cos;
    const float* sin;
    int seq, hq, hkv;
    int layout;  // 1: split-half pairs (d, d + 64); 0: interleaved pairs (2p, 2p + 1)
};
// Epilogues of the tile kernel: the plain store, or one of the decoder layer's fusions.
constexpr int kEpiPlain = 0;
constexpr int kEpiQkvRope = 1;   // the QKV projection into rotated head planes (QkvRopeOut)
constexpr int kEpiResidual = 2;  // C = bf16(bf16(acc) + res): a projection plus its residual
constexpr int kEpiSwiglu = 3;    // gate and up in one product -> gate, up, SiLU(gate) * up
constexpr int kEpiSwigluBwd = 4; // dM = dY Wd -> the SwiGLU gradients of gate and up
// The gate/up product's B rows (and the columns of the SwiGLU gradient) interleave gate and up in
// blocks of 16: row 32 b + r is gate row 16 b + r for r < 16 and up row 16 b + r - 16 otherwise,
// so a wave's fragments 2q and 2q + 1 hold the gate and up values of the same 16 columns.
struct GemmEpiArgs : GemmArgs {
    QkvRopeOut qkv;
    const uint16_t* res;  // kEpiResidual: [M, N] like C
    uint16_t* gate;       // kEpiSwiglu: written, kEpiSwigluBwd: read; [M, F] with F = N / 2 (fwd), N (bwd)
    uint16_t* up;
    uint16_t* act;        // kEpiSwiglu: SiLU(gate) * up [M, F]
    uint16_t* dgu;        // kEpiSwigluBwd: [M, 2F], the interleaved gradient of the gate/up product
};

// B operand of the tile whose first output row is row0 in batch g.
// (The tile kernel below is a template over its argument type: other callers give it their own
// argument struct and weight_slice overload.)
__device__ __forceinline__ const uint16_t* weight_slice(const GemmArgs& p, int row0, int64_t g) {
    const int64_t slice = p.block_group ? static_cast<int64_t>(p.block_group[row0 >> 8]) : g;
    return p.b + slice * static_cast<int64_t>(p.n) * p.k;
}


// The compiler may not move instructions across this point.
__device__ __forceinline__ void phase_fence() { __builtin_amdgcn_sched_barrier(0); }


// Workgroup barrier after which the loads of the step before the last N outstanding ones
// (per wave, in issue order) have landed in LDS and every LDS read issued before it has
// completed. A plain barrier without the memory fence of __syncthreads, whose release
// semantics would wait for every outstanding load, including the prefetches meant to stay in
// flight. The empty asm statements keep the compiler from moving memory accesses across it.
// gfx9 s_waitcnt encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8.
template <int N>
__device__ __forceinline__ void stage_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (0 << 8));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// 256x256-tile stages: 64 k deep, two 64 KB LDS slots (A half, then B half).
constexpr int kPPTile = 256;
constexpr int kPK = 64;  // K per stage

__device__ __forceinline__ int swz64(int row, int chunk) {  // element offset in a [rows][64] stage
    return row * kPK + ((chunk ^ ((row >> 1) & 7)) << 3);
}


// 256x256 output tiles with four wavefronts, one per SIMD, each owning a 128x128 block of 8x8
// v_mfma_f32_16x16x32_bf16 tiles (4 accumulators per lane each: the whole AGPR file). Measured
// against an 8-wave "ping-pong" design (two groups of four waves alternating MFMA turns and
// memory turns, 32x32x16 MFMAs) at 8192^3 on N(0,1) data, this runs ~15% faster:
//   * one wave per SIMD interleaves its own memory instructions between its MFMAs, and a 128x128
//     block reads 0.5 KB of LDS operands per 32x32x16-equivalent MFMA instead of 0.75 KB;
//   * the 16x16x32 shape moves fewer register-file bytes per multiply-accumulate than 32x32x16
//     (4 accumulator registers per lane per MFMA instead of 16), and this part is power-limited:
//     the clock it sustains depends on the work per flop;
//   * tiles travel straight from global memory into LDS (buffer_load ... lds; no staging
//     registers, no LDS write instructions). K stages of 64 in two 64 KB slots, 128-byte
//     swizzled rows (full 128-byte lines per global request). A stage is two k-slices of 32 (64 MFMAs each) with one
//     barrier between them; all of stage s+2 is fetched during slice 1 of stage s into the slot
//     that barrier has just freed, so every load has one to two slices to land before the
//     barrier that needs it (issuing the same loads half a stage later cost ~10%);
//   * within a slice, a fragment read for the next slice follows every fourth MFMA and a load
//     follows every fourth MFMA two later, so no gap between MFMAs holds more than one memory
//     instruction (bunching them cost 3-8%);
//   * bands of 4 M-tiles per XCD for square tile grids (8 measured 2% slower at 8192^3, 16 8%), of
//     8 N-tiles otherwise (see launch_pp);
//   * an MN-major operand (the backward's dY W and dY^T X) is read in place: its half of a stage
//     is 64 k-rows of 256 columns (512-byte rows, 64-byte blocks XORed with k-row % 4) filled by
//     the same 1 KB global->LDS loads (two k-rows each), and each fragment is two
//     ds_read_b64_tr_b16 transposing reads, which hand every lane the 8 consecutive k of its
//     column that the K-major 16-byte read gives. The four 16-lane groups read the same 16
//     columns at k-rows 8 apart, so two groups share banks (a 2-way conflict: ~128 LDS cycles
//     per 1024-cycle slice). 8192^3 NN/TN/TT: 1.48-1.51 PFLOP/s, against 1.30 for the 8-wave
//     ping-pong design with register-staged loads and transposing reads that this replaced.
constexpr int kW4Threads = 256;

// Byte offset past any operand's buffer range: a buffer load at it reads zero. The range check
// compares the unsigned 32-bit offset with the resource's byte count, which pp_applies keeps
// below 2^31 (m * k * 2 <= m * k64 * 2 < 2^31), so 2^31 is out of range for every operand.
constexpr int kOutOfRange = static_cast<int>(0x80000000u);

// KTAIL: K % 64 != 0 (K % 8 == 0), so the last stage is partial. Its K-major 16-byte chunks past
// K take an out-of-range offset and read as zero; the k-rows of an MN-major operand past K lie
// past the end of that operand's range already. Zeros add nothing to the accumulators, so the
// result equals that of K zero-padded to a multiple of 64.
// One 256 x (32 NJ) output tile per workgroup: tile blockIdx.x of batch blockIdx.z, the grid being
// tiles_m * tiles_n x 1 x batch (the libhk.so kernel and the device-program entry points both
// call it; kW4Threads threads, one workgroup per CU). NJ = 8 gives the square 256x256 tile; the
// launcher takes NJ = 6 (192-wide tiles, each wave 128 x 96) when that saves a whole round of
// workgroups (a 1.5-round grid of square tiles as 2 rounds of narrow ones). The B stage keeps its
// 256 rows or columns; an MN-major B is staged 256 columns wide as for NJ = 8 (the columns past the
// tile feed nothing).
// Epilogue of the fused QKV projection (NJ = 8): a wave's 128 output columns are exactly one head
// and a lane holds columns 16 j + 4 lg .. +3 of row 16 i + l16 in acc[i][j], so both members of
// every rotation pair are in the lane (split-half: fragments j and j + 4; interleaved: neighbours
// within a fragment). Each value is first rounded to BF16 -- the product's storage in the
// unfused composition -- then rotated in F32 by rope_rotate and rounded again, so the planes are
// bit-identical to the GEMM's BF16 rows followed by qkv_rope_split. The cos/sin values of a row
// are fetched four rows ahead of its stores (a load issued after a store waits for it: vmcnt
// counts both in order).
struct RopeRowIn {  // the lane's 16 angles of one row: split-half c[j] = angles 16 j + 4 lg .. +3,
    f32x4_t c[4];   // interleaved c[q] = angles 16 q + 2 lg, +1 (fragment 2q) and 16 q + 8 + 2 lg, +1
    f32x4_t s[4];   // (fragment 2q + 1)
};

template <class Args>
__device__ __forceinline__ void store_qkv_rope(const Args& p, f32x4_t (&acc)[8][8], int tm, int tn, int wm, int wn,
                                               int l16, int lg) {
    const QkvRopeOut& o = p.qkv;
    const int n0 = tn * kPPTile + 128 * wn;
    if (n0 >= p.n) return;
    const int head = n0 >> 7;
    uint16_t* plane;
    int hx, hh;
    if (head < o.hq) {
        plane = o.q, hx = o.hq, hh = head;
    } else if (head < o.hq + o.hkv) {
        plane = o.k, hx = o.hkv, hh = head - o.hq;
    } else {
        plane = o.v, hx = o.hkv, hh = head - o.hq - o.hkv;
    }
    const bool rotate = head < o.hq + o.hkv;
    const int m0 = tm * kPPTile + 128 * wm + l16;
    constexpr int kAhead = 4;
    RopeRowIn in[kAhead];
    auto load_row = [&](RopeRowIn& r, int i) __attribute__((always_inline)) {
        const int s = min(m0 + 16 * i, p.m - 1) % o.seq;  // issued for every row (no load under a branch)
        const float* ct = o.cos + static_cast<int64_t>(s) * 64;
        const float* st = o.sin + static_cast<int64_t>(s) * 64;
        if (o.layout == 1) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                r.c[j] = *reinterpret_cast<const f32x4_t*>(ct + 16 * j + 4 * lg);
                r.s[j] = *reinterpret_cast<const f32x4_t*>(st + 16 * j + 4 * lg);
            }
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const f32x2_t c0 = *reinterpret_cast<const f32x2_t*>(ct + 16 * q + 2 * lg);
                const f32x2_t c1 = *reinterpret_cast<const f32x2_t*>(ct + 16 * q + 8 + 2 * lg);
                const f32x2_t s0 = *reinterpret_cast<const f32x2_t*>(st + 16 * q + 2 * lg);
                const f32x2_t s1 = *reinterpret_cast<const f32x2_t*>(st + 16 * q + 8 + 2 * lg);
                r.c[q] = f32x4_t{c0[0], c0[1], c1[0], c1[1]};
                r.s[q] = f32x4_t{s0[0], s0[1], s1[0], s1[1]};
            }
        }
    };
#pragma unroll
    for (int i = 0; i < kAhead; ++i) load_row(in[i], i);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int m = m0 + 16 * i;
        if (m < p.m) {
            const int b = m / o.seq, s = m - b * o.seq;
            uint16_t* row = plane + (static_cast<int64_t>(b) * hx + hh) * o.seq * 128 + static_cast<int64_t>(s) * 128;
            const RopeRowIn& r = in[i % kAhead];
            if (!rotate) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const u32x2_t w = {pack_bf16x2(acc[i][j][0], acc[i][j][1]), pack_bf16x2(acc[i][j][2], acc[i][j][3])};
                    *reinterpret_cast<u32x2_t*>(row + 16 * j + 4 * lg) = w;
                }
            } else if (o.layout == 1) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int d = 16 * j + 4 * lg;
                    float ya[4], yb[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        rope_rotate<false>(round_bf16(acc[i][j][e]), round_bf16(acc[i][j + 4][e]), r.c[j][e], r.s[j][e],
                                           ya[e], yb[e]);
                    *reinterpret_cast<u32x2_t*>(row + d) = u32x2_t{pack_bf16x2(ya[0], ya[1]), pack_bf16x2(ya[2], ya[3])};
                    *reinterpret_cast<u32x2_t*>(row + d + 64) = u32x2_t{pack_bf16x2(yb[0], yb[1]), pack_bf16x2(yb[2], yb[3])};
                }
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int d = 16 * j + 4 * lg;  // pairs (d, d + 1) and (d + 2, d + 3): angles d/2, d/2 + 1
                    const int h = 2 * (j & 1);
                    const float c0 = r.c[j >> 1][h], c1 = r.c[j >> 1][h + 1];
                    const float s0 = r.s[j >> 1][h], s1 = r.s[j >> 1][h + 1];
                    float y[4];
                    rope_rotate<false>(round_bf16(acc[i][j][0]), round_bf16(acc[i][j][1]), c0, s0, y[0], y[1]);
                    rope_rotate<false>(round_bf16(acc[i][j][2]), round_bf16(acc[i][j][3]), c1, s1, y[2], y[3]);
                    *reinterpret_cast<u32x2_t*>(row + d) = u32x2_t{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
                }
            }
        }
        if (i + kAhead < 8) load_row(in[i % kAhead], i + kAhead);
    }
}

// The element-wise fused epilogues (NJ fragments of 16 columns per wave): row m, the wave's first
// column n0; each lane holds columns n0 + 16 j + 4 lg .. +3. Every value is rounded to BF16 where the
// unfused composition stores it, so the results are bit-identical to the GEMM followed by the
// element-wise kernel.
// What an epilogue reads for one of a lane's rows: the residual (kEpiResidual) or the saved gate
// and up values (kEpiSwigluBwd), 4 columns of each fragment. The tile loop fetches these rows
// several ahead of its stores: vmcnt counts loads and stores together and in order, so a load
// issued after a store is waited on only once that store has completed too, and fetching each row
// just before storing it would serialize one store and one load round trip per fragment.
template <int EPI, int NJ>
struct EpiRowIn {
    u32x2_t a[NJ];
    u32x2_t b[EPI == kEpiSwigluBwd ? NJ : 1];
};
template <int EPI>
constexpr bool epi_reads() {
    return EPI == kEpiResidual || EPI == kEpiSwigluBwd;
}
template <int EPI>
constexpr int epi_rows_ahead() {  // 16 VGPRs per residual row, 32 per gate/up row (8 residual rows spill)
    return EPI == kEpiResidual ? 4 : 4;
}

// Issued for every row and fragment, also past the output's last row or column (clamped to the
// last one: the value feeds no store), so no load sits under a branch.
template <int EPI, int NJ, class Args>
__device__ __forceinline__ void load_fused_row(const Args& p, EpiRowIn<EPI, NJ>& in, int64_t g, int m, int n0,
                                               int lg) {
    const int mc = min(m, p.m - 1);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int n = min(n0 + 16 * j + 4 * lg, p.n - 4);
        if constexpr (EPI == kEpiResidual) {
            in.a[j] = *reinterpret_cast<const u32x2_t*>(p.res + (g * p.m + mc) * static_cast<int64_t>(p.n) + n);
        } else {
            static_assert(EPI == kEpiSwigluBwd, "epilogue inputs");
            const int64_t off = static_cast<int64_t>(mc) * p.n + n;
            in.a[j] = *reinterpret_cast<const u32x2_t*>(p.gate + off);
            in.b[j] = *reinterpret_cast<const u32x2_t*>(p.up + off);
        }
    }
}

template <int EPI, int NJ, class Args>
__device__ __forceinline__ void store_fused_row(const Args& p, const f32x4_t (&acc)[NJ], const EpiRowIn<EPI, NJ>& in,
                                                int64_t g, int m, int n0, int lg) {
    if constexpr (EPI == kEpiResidual) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int n = n0 + 16 * j + 4 * lg;
            if (n >= p.n) continue;
            const int64_t off = (g * p.m + m) * static_cast<int64_t>(p.n) + n;
            const u32x2_t r = in.a[j];
            const float y0 = round_bf16(acc[j][0]) + bf16lo(r[0]), y1 = round_bf16(acc[j][1]) + bf16hi(r[0]);
            const float y2 = round_bf16(acc[j][2]) + bf16lo(r[1]), y3 = round_bf16(acc[j][3]) + bf16hi(r[1]);
            *reinterpret_cast<u32x2_t*>(static_cast<uint16_t*>(p.c) + off) = u32x2_t{pack_bf16x2(y0, y1), pack_bf16x2(y2, y3)};
        }
    } else if constexpr (EPI == kEpiSwiglu) {
        static_assert(NJ % 2 == 0, "gate/up fragment pairs");
        const int f_cols = p.n / 2;
#pragma unroll
        for (int q = 0; q < NJ / 2; ++q) {
            if (n0 + 32 * q >= p.n) continue;
            const int f = n0 / 2 + 16 * q + 4 * lg;
            float gv[4], uv[4], y[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                gv[e] = round_bf16(acc[2 * q][e]);
                uv[e] = round_bf16(acc[2 * q + 1][e]);
                y[e] = silu_mul1(gv[e], uv[e]);
            }
            const int64_t off = static_cast<int64_t>(m) * f_cols + f;
            *reinterpret_cast<u32x2_t*>(p.gate + off) = u32x2_t{pack_bf16x2(gv[0], gv[1]), pack_bf16x2(gv[2], gv[3])};
            *reinterpret_cast<u32x2_t*>(p.up + off) = u32x2_t{pack_bf16x2(uv[0], uv[1]), pack_bf16x2(uv[2], uv[3])};
            *reinterpret_cast<u32x2_t*>(p.act + off) = u32x2_t{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
        }
    } else {
        static_assert(EPI == kEpiSwigluBwd, "fused epilogue");
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int f = n0 + 16 * j + 4 * lg;
            if (f >= p.n) continue;
            const u32x2_t gw = in.a[j], uw = in.b[j];
            const float gv[4] = {bf16lo(gw[0]), bf16hi(gw[0]), bf16lo(gw[1]), bf16hi(gw[1])};
            const float uv[4] = {bf16lo(uw[0]), bf16hi(uw[0]), bf16lo(uw[1]), bf16hi(uw[1])};
            float dg[4], du[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) silu_mul_bwd1(gv[e], uv[e], round_bf16(acc[j][e]), dg[e], du[e]);
            uint16_t* row = p.dgu + static_cast<int64_t>(m) * (2 * p.n) + 32 * (f >> 4) + (f & 15);
            *reinterpret_cast<u32x2_t*>(row) = u32x2_t{pack_bf16x2(dg[0], dg[1]), pack_bf16x2(dg[2], dg[3])};
            *reinterpret_cast<u32x2_t*>(row + 16) = u32x2_t{pack_bf16x2(du[0], du[1]), pack_bf16x2(du[2], du[3])};
        }
    }
}

// WIDE: operands past 32-bit byte offsets (M*K or N*K >= 2^30 elements). Each buffer resource then
// starts at the tile: a K-major operand at the tile's first row (its 256 rows span 256 K 2 < 2^31
// bytes for K < 2^22), an MN-major one at the tile's first column of the stage's first k-row, rebuilt
// per stage (64 k-rows of M or N columns: 128 M < 2^31 bytes for M < 2^24). Each resource's byte
// count ends where the operand ends or, further from the end, past everything its loads can reach,
// so rows past M or N and k-rows past K read as zero exactly as in the 32-bit form.
template <bool OUT_BF16, bool A_MN, bool B_MN, bool KTAIL, class Args, int NJ = 8, int EPI = kEpiPlain,
          bool WIDE = false>
__device__ __forceinline__ void gemm_m16_tile(Args p) {
    static_assert(NJ >= 1 && NJ <= 8, "B fragments per wave");
    constexpr int kTileN = 32 * NJ;  // output columns per tile
    constexpr int kWaveN = 16 * NJ;  // output columns per wave
    constexpr int kLoadsA = 8, kLoadsB = B_MN ? 8 : NJ;  // 1 KB global->LDS loads per wave per stage
    constexpr int kLoads = kLoadsA + kLoadsB;
    constexpr int kReads = 8 + NJ;  // fragment reads per wave per k-slice
    constexpr int kMfma = 8 * NJ;   // MFMAs per wave per k-slice
    constexpr int kStage = 2 * kPPTile * kPK;
    __shared__ __attribute__((aligned(1024))) uint16_t slot0[kStage];
    __shared__ __attribute__((aligned(1024))) uint16_t slot1[kStage];

    const int tiles = p.tiles_m * p.tiles_n;
    int bid = blockIdx.x;
    if ((tiles & 7) == 0) bid = (bid & 7) * (tiles >> 3) + (bid >> 3);
    int tm, tn;
    if (p.band_n == 0) {
        constexpr int GROUP = 4;
        const int per_group = GROUP * p.tiles_n;
        const int first_m = (bid / per_group) * GROUP;
        const int gsize = min(p.tiles_m - first_m, GROUP);
        tm = first_m + (bid % per_group) % gsize;
        tn = (bid % per_group) / gsize;
    } else {
        const int per_group = p.band_n * p.tiles_m;
        const int first_n = (bid / per_group) * p.band_n;
        const int gsize = min(p.tiles_n - first_n, p.band_n);
        tn = first_n + (bid % per_group) % gsize;
        tm = (bid % per_group) / gsize;
    }
    const int64_t g = blockIdx.z;
    const uint16_t* A = p.a + g * static_cast<int64_t>(p.m) * p.k;
    const uint16_t* B = weight_slice(p, tm * kPPTile, g);

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int l16 = lane & 15, lg = lane >> 4;  // 16x16x32 operand: row l16, k chunk lg of the slice

    const int r_in = lane >> 3;
    const int src_chunk = (lane & 7) ^ ((4 * (wave & 1) + (r_in >> 1)) & 7);
    const int voff = (r_in * p.k + src_chunk * 8) * 2;
    // 32-bit form: one resource per operand slice, the tile's rows or columns in the offsets.
    // WIDE: K-major resources start at the tile's first row (tile_a_row, tile_b_row); MN-major ones
    // are built per stage by mn_resource below.
    const int tile_a_row = WIDE && !A_MN ? tm * kPPTile : 0, tile_b_row = WIDE && !B_MN ? tn * kTileN : 0;
    auto kmajor_bytes = [&](int rows, int row0) __attribute__((always_inline)) {
        if constexpr (!WIDE) return rows * p.k * 2;
        return min(rows - row0, kPPTile) * p.k * 2;
    };
    const i32x4_t ra4 = buffer_resource(A + static_cast<int64_t>(tile_a_row) * p.k, kmajor_bytes(p.m, tile_a_row));
    const i32x4_t rb4 = buffer_resource(B + static_cast<int64_t>(tile_b_row) * p.k, kmajor_bytes(p.n, tile_b_row));
    // WIDE MN-major operand X stored [K, cols]: the stage's 64 k-rows from column col0 on.
    auto mn_resource = [&](const uint16_t* X, int cols, int col0, int kt) __attribute__((always_inline)) {
        const int64_t first = static_cast<int64_t>(kt) * kPK * cols + col0;
        const int64_t left = (static_cast<int64_t>(p.k) * cols - first) * 2;
        const int64_t reach = static_cast<int64_t>(kPK) * cols * 2 + 2 * kPPTile;
        return buffer_resource(X + first, static_cast<int>(left < reach ? left : reach));
    };
    // MN-major operand (A stored [K,M] or B stored [K,N]): its half of a stage is 64 k-rows x 256
    // columns, 512-byte rows whose 64-byte blocks are XORed with k-row % 4. Load d of a wave fills
    // k-rows 2(wave + 4d) + {0, 1}; lane l takes position l % 32 of k-row l / 32, which holds the
    // global chunk the swizzle puts there (k-row % 4 is the same for every d). The k-row and column
    // are in the range-checked offset (K * M * 2 < 2^31): columns past M (N) in the last k-row read
    // as zero, elsewhere they feed only outputs that are not stored.
    const int mn_row0 = 2 * wave + (lane >> 5), mn_pos = lane & 31;
    const int mn_c = (((mn_pos >> 2) ^ (mn_row0 & 3)) << 2) | (mn_pos & 3);
    const int mn_voff_a = (mn_row0 * p.m + (WIDE ? 0 : tm * kPPTile) + mn_c * 8) * 2;
    const int mn_voff_b = (mn_row0 * p.n + (WIDE ? 0 : tn * kTileN) + mn_c * 8) * 2;
    const uint32_t lds0 = lds_address(slot0), lds1 = lds_address(slot1);
    // K-major load: the stage offset moves into the lane's offset, which the range check sees
    auto kmajor = [&](const i32x4_t& r, uint32_t dst, int row_off, int kt) __attribute__((always_inline)) {
        if constexpr (KTAIL)
            load_lds16(r, dst, kt * kPK + src_chunk * 8 < p.k ? row_off + kt * kPK * 2 : kOutOfRange, 0);
        else
            load_lds16(r, dst, row_off, kt * kPK * 2);
    };
    auto dload = [&](uint32_t lds_slot, int kt, int d) __attribute__((always_inline)) {
        const int blk = wave + 4 * d;
        const uint32_t dst = lds_slot + (wave * 8 * kPK + d * 4 * 8 * kPK) * 2;
        if (d < 8) {
            if constexpr (A_MN && WIDE) load_lds16(mn_resource(A, p.m, tm * kPPTile, kt), dst, mn_voff_a + 8 * d * p.m * 2, 0);
            else if constexpr (A_MN) load_lds16(ra4, dst, mn_voff_a + (kt * kPK + 8 * d) * p.m * 2, 0);
            else kmajor(ra4, dst, voff + (tm * kPPTile - tile_a_row + 8 * blk) * p.k * 2, kt);
        } else {
            if constexpr (B_MN && WIDE) load_lds16(mn_resource(B, p.n, tn * kTileN, kt), dst, mn_voff_b + 8 * (d - 8) * p.n * 2, 0);
            else if constexpr (B_MN) load_lds16(rb4, dst, mn_voff_b + (kt * kPK + 8 * (d - 8)) * p.n * 2, 0);
            else kmajor(rb4, dst, voff + (tn * kTileN - tile_b_row + 8 * (blk - 32)) * p.k * 2, kt);
        }
    };

    const int a_row = 128 * wm + l16, b_row = kPPTile + kWaveN * wn + l16;
    // Transposing read of an MN-major 16x16x32 operand: columns col0 .. col0+15 (col0 % 16 == 0),
    // k-rows k0 .. k0+7 with k0 = 32 ks + 8 lg (each 16-lane group its own k0; k0 % 4 == 0, so the
    // k-row's XOR term is i/4). Lane i of a group reads 4 columns of k-row k0 + i/4 (then k0 + 4 +
    // i/4), and the hardware hands lane i the 4 k values of column col0 + i.
    const int tr_i = lane & 15;
    const int tr_lane = (tr_i >> 2) * kPPTile + 4 * (tr_i & 3);
    auto read_tr = [&](const uint16_t* stage, int k0, int col0) __attribute__((always_inline)) {
        const uint16_t* at = stage + k0 * kPPTile + tr_lane + ((((col0 >> 5) ^ (tr_i >> 2)) << 5) | (col0 & 31));
        const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(at));
        const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(at + 4 * kPPTile));
        typedef short v8i16_t __attribute__((ext_vector_type(8)));
        const v8i16_t v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        return __builtin_bit_cast(bf16x8_t, v);
    };
    bf16x8_t fa[2][8], fb[2][NJ];
    auto read1 = [&](const uint16_t* slot, int ks, int buf, int f) __attribute__((always_inline)) {
        const int c = 4 * ks + lg;
        if (f < 8) {
            if constexpr (A_MN) fa[buf][f] = read_tr(slot, 8 * c, 128 * wm + 16 * f);
            else fa[buf][f] = *reinterpret_cast<const bf16x8_t*>(slot + swz64(a_row + 16 * f, c));
        } else {
            if constexpr (B_MN) fb[buf][f - 8] = read_tr(slot + kPPTile * kPK, 8 * c, kWaveN * wn + 16 * (f - 8));
            else fb[buf][f - 8] = *reinterpret_cast<const bf16x8_t*>(slot + swz64(b_row + 16 * (f - 8), c));
        }
    };

    f32x4_t acc[8][NJ];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) asm volatile("" : "+a"(acc[i][j]));

    const int nk = KTAIL ? (p.k + kPK - 1) / kPK : p.k / kPK;
    // kMfma MFMAs on buffer `cur`, with the kReads fragment reads of slice `next_ks` (from
    // `next_slot` into the other buffer) and the loads d0 .. d1-1 spread evenly between them: read t
    // follows MFMA ceil(t kMfma / kReads), load t MFMA floor((t + 1/2) kMfma / kLoads), so for NJ = 8
    // a read follows every fourth MFMA and a load two MFMAs later.
    auto slice = [&](int cur, const uint16_t* next_slot, int next_ks, uint32_t load_slot, int d0, int d1,
                     int kt) __attribute__((always_inline)) {
        const int nxt = cur ^ 1;
#pragma unroll
        for (int e = 0; e < kMfma; ++e) {
            const int i = e / NJ, j = e % NJ;
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[cur][j], fa[cur][i], acc[i][j], 0, 0, 0);
            phase_fence();
            // At most one read and one load per MFMA (kReads, kLoads <= kMfma): read t = floor(e kReads /
            // kMfma) goes here when ceil(t kMfma / kReads) == e, load t = ceil((2 e kLoads - kMfma) /
            // (2 kMfma)) when floor((2t + 1) kMfma / (2 kLoads)) == e.
            const int tr = e * kReads / kMfma;
            if ((tr * kMfma + kReads - 1) / kReads == e) read1(next_slot, next_ks, nxt, tr);
            const int tl = (2 * e * kLoads - kMfma + 2 * kMfma - 1) / (2 * kMfma);  // ceil, numerator >= -kMfma
            if (tl < kLoads && ((2 * tl + 1) * kMfma) / (2 * kLoads) == e && d0 + tl < d1) dload(load_slot, kt, d0 + tl);
            phase_fence();
        }
    };

    // Prologue: stage 0 into slot 0, stage 1 into slot 1, slice 0's fragments.
#pragma unroll
    for (int d = 0; d < kLoads; ++d) dload(lds0, 0, d);
    stage_barrier<0>();
#pragma unroll
    for (int d = 0; d < kLoads; ++d) dload(lds1, nk > 1 ? 1 : 0, d);
#pragma unroll
    for (int f = 0; f < kReads; ++f) read1(slot0, 0, 0, f);

    auto stage = [&](const uint16_t* R, const uint16_t* W, uint32_t Rl, int s) __attribute__((always_inline)) {
        const int ahead = s + 2 < nk ? s + 2 : nk - 1;
        slice(0, R, 1, Rl, 0, 0, ahead);      // reads only
        stage_barrier<0>();                   // stage s+1 complete in W; every read of R done
        slice(1, W, 0, Rl, 0, kLoads, ahead);  // + all of stage s+2 into the freed R
    };
    int s = 0;
    do {
        stage(slot0, slot1, lds0, s);
        if (s + 1 < nk) stage(slot1, slot0, lds1, s + 1);
        s += 2;
    } while (s < nk);
    stage_barrier<0>();  // no load may still be writing LDS at exit

    if constexpr (EPI == kEpiQkvRope) {
        static_assert(NJ == 8 && OUT_BF16, "the fused QKV epilogue needs 128-column wave blocks");
        store_qkv_rope(p, acc, tm, tn, wm, wn, l16, lg);
        return;
    } else if constexpr (EPI != kEpiPlain) {
        const int m0 = tm * kPPTile + 128 * wm + l16, n0 = tn * kTileN + kWaveN * wn;
        constexpr int kAhead = epi_reads<EPI>() ? epi_rows_ahead<EPI>() : 1;
        EpiRowIn<EPI, NJ> in[kAhead];
        if constexpr (epi_reads<EPI>()) {
#pragma unroll
            for (int i = 0; i < kAhead; ++i) load_fused_row<EPI, NJ>(p, in[i], g, m0 + 16 * i, n0, lg);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (m0 + 16 * i < p.m) store_fused_row<EPI, NJ>(p, acc[i], in[i % kAhead], g, m0 + 16 * i, n0, lg);
            if constexpr (epi_reads<EPI>()) {
                if (i + kAhead < 8) load_fused_row<EPI, NJ>(p, in[i % kAhead], g, m0 + 16 * (i + kAhead), n0, lg);
            }
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int m = tm * kPPTile + 128 * wm + 16 * i + l16;
        if (m >= p.m) continue;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int n = tn * kTileN + kWaveN * wn + 16 * j + 4 * lg;
            if (n >= p.n) continue;
            const int64_t off = (g * p.m + m) * static_cast<int64_t>(p.n) + n;
            if constexpr (OUT_BF16) {
                u32x2_t w = {pack_bf16x2(acc[i][j][0], acc[i][j][1]), pack_bf16x2(acc[i][j][2], acc[i][j][3])};
                *reinterpret_cast<u32x2_t*>(static_cast<uint16_t*>(p.c) + off) = w;
            } else {
                *reinterpret_cast<f32x4_t*>(static_cast<float*>(p.c) + off) = acc[i][j];
            }
        }
    }
}

template <bool OUT_BF16, bool A_MN, bool B_MN, bool KTAIL = false, int NJ = 8>
__global__ void __launch_bounds__(kW4Threads, 1)
gemm_nt_m16_kernel(GemmArgs p) {
    gemm_m16_tile<OUT_BF16, A_MN, B_MN, KTAIL, GemmArgs, NJ>(p);
}

// The fused-epilogue GEMMs (256x256 tiles, A K-major, B K-major or, for the SwiGLU backward's
// dY Wd, MN-major).
template <int EPI, bool B_MN, bool KTAIL>
__global__ void __launch_bounds__(kW4Threads, 1)
gemm_epi_kernel(GemmEpiArgs p) {
    gemm_m16_tile<true, false, B_MN, KTAIL, GemmEpiArgs, 8, EPI>(p);
}

}  // namespace

}  // namespace hk
