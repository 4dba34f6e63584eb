// hk_gemm.hip — BF16 GEMM with FP32 accumulation for gfx950 (MI355X).
//
// Semantics (reference rust-ascend-kernels/src/kernel.rs:5-76, ascend.rs:22-68):
//   C[g, i, j] = sum_k A'[g, i, k] * B'[g, k, j]  with FP32 accumulation,
//   C stored as BF16 (round to nearest even) or F32. A' is A ([M,K]) or A^T (A stored
//   [K,M]); B' is B ([K,N]) or B^T (B stored [N,K]). Batched operands are contiguous
//   [G, ...] with strides M*K, N*K, M*N (ascend.rs:88-114).
//
// Design (MI355X-first, not a translation of the reference's 64x64 Ascend tiles):
//   * Large problems (at least one 256x256 tile per CU, K % 64 == 0), every transpose read in
//     place -> gemm_nt_m16_kernel: four wavefronts of 128x128 with 16x16x32 MFMAs and
//     global->LDS loads; a K-contiguous operand (A [M,K], B [N,K]) is staged in 128-byte k-rows
//     and read with 16-byte LDS reads, an MN-contiguous one (A stored [K,M] or B stored [K,N]) in
//     512-byte rows of 256 columns and read with transposing LDS reads.
//   * Smaller problems: MN-contiguous operands are first transposed into the workspace by an
//     HBM-bound kernel, then a workgroup of 4 wavefronts (2x2) computes a BMxBN output tile (256, 128 or 64
//     when a larger grid would not fill the 256 CUs). Each wave owns a (BM/2)x(BN/2) block of
//     32x32 MFMA tiles, v_mfma_f32_32x32x16_bf16, accumulators in the AGPR half of the
//     register file.
//   * K loop in steps of BK = 64: A and B slices are prefetched from HBM into registers one
//     step ahead, written to a double-buffered LDS tile (rows of 64 BF16 = 128 B, 16-byte
//     chunks XOR-swizzled by row%8 so both the row-contiguous writes and the 32-row
//     fragment reads are bank-conflict-free), one barrier per step.
//   * MFMA operand order is swapped (B tile as the MFMA "A" operand) so each lane ends with
//     4 consecutive output columns per register group: 8-byte BF16 / 16-byte F32 stores.
//   * Tile order: blocks are remapped so each of the 8 XCDs (blockIdx % 8) receives a
//     contiguous range of tiles, then grouped in 8-tile-row bands, so tiles that share A/B
//     slices run on the same XCD's L2.
#include "hk_common.hpp"
#include "hk_gemm_device.hpp"
#include "hk_kernels.hpp"

namespace hk {

namespace {

constexpr int kBK = 64;
constexpr int kThreads = 256;

__device__ __forceinline__ int swz(int row, int chunk) { return row * kBK + ((chunk ^ (row & 7)) << 3); }

template <int BM, int BN, bool OUT_BF16>
__global__ void __launch_bounds__(kThreads)
gemm_nt_kernel(GemmArgs p) {
    constexpr int TI = BM / 64;          // 32x32 tiles per wave along M
    constexpr int TJ = BN / 64;          // along N
    constexpr int A_LOADS = BM * 8 / kThreads;  // 16-byte chunks per thread per K step
    constexpr int B_LOADS = BN * 8 / kThreads;
    __shared__ __attribute__((aligned(16))) uint16_t lds[2][(BM + BN) * kBK];

    // ---- tile coordinates: XCD-contiguous ranges, then 8-row grouped order
    const int tiles = p.tiles_m * p.tiles_n;
    int bid = blockIdx.x;
    if ((tiles & 7) == 0) bid = (bid & 7) * (tiles >> 3) + (bid >> 3);
    constexpr int GROUP = 8;
    const int per_group = GROUP * p.tiles_n;
    const int first_m = (bid / per_group) * GROUP;
    const int gsize = min(p.tiles_m - first_m, GROUP);
    const int tm = first_m + (bid % per_group) % gsize;
    const int tn = (bid % per_group) / gsize;
    const int64_t g = blockIdx.z;

    const uint16_t* A = p.a + g * static_cast<int64_t>(p.m) * p.k;
    const uint16_t* B = weight_slice(p, tm * BM, g);

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, lk = lane >> 5;

    // ---- global -> register prefetch assignment
    const int lcol = t & 7;   // 16-byte chunk within the 64-wide K slice
    const int lrow = t >> 3;  // 0..31, plus 32*i
    const uint16_t* a_src[A_LOADS];
    const uint16_t* b_src[B_LOADS];
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
        int r = tm * BM + lrow + 32 * i;
        r = r < p.m ? r : p.m - 1;  // rows past M read a valid row; their outputs are not stored
        a_src[i] = A + static_cast<int64_t>(r) * p.k + lcol * 8;
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
        int r = tn * BN + lrow + 32 * i;
        r = r < p.n ? r : p.n - 1;
        b_src[i] = B + static_cast<int64_t>(r) * p.k + lcol * 8;
    }
    u32x4_t ra[A_LOADS], rb[B_LOADS];
    auto load_global = [&](int kt) {
        const int kk = kt * kBK + lcol * 8;
        const bool in = kk < p.k;  // K % 16 == 0: a 16-byte chunk is wholly in or out
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i)
            ra[i] = in ? *reinterpret_cast<const u32x4_t*>(a_src[i] + kt * kBK) : u32x4_t{0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i)
            rb[i] = in ? *reinterpret_cast<const u32x4_t*>(b_src[i] + kt * kBK) : u32x4_t{0, 0, 0, 0};
    };
    auto store_lds = [&](int buf) {
        uint16_t* la = lds[buf];
        uint16_t* lb = lds[buf] + BM * kBK;
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i)
            *reinterpret_cast<u32x4_t*>(la + swz(lrow + 32 * i, lcol)) = ra[i];
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i)
            *reinterpret_cast<u32x4_t*>(lb + swz(lrow + 32 * i, lcol)) = rb[i];
    };

    f32x16_t acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    const int nk = (p.k + kBK - 1) / kBK;
    load_global(0);
    store_lds(0);
    if (nk > 1) load_global(1);
    __syncthreads();

    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        const uint16_t* la = lds[cur];
        const uint16_t* lb = lds[cur] + BM * kBK;
#pragma unroll
        for (int ks = 0; ks < kBK / 16; ++ks) {
            const int chunk = ks * 2 + lk;
            bf16x8_t af[TI], bfr[TJ];
#pragma unroll
            for (int i = 0; i < TI; ++i)
                af[i] = *reinterpret_cast<const bf16x8_t*>(la + swz(wm * (BM / 2) + i * 32 + lr, chunk));
#pragma unroll
            for (int j = 0; j < TJ; ++j)
                bfr[j] = *reinterpret_cast<const bf16x8_t*>(lb + swz(wn * (BN / 2) + j * 32 + lr, chunk));
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j], af[i], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) {
            store_lds(cur ^ 1);
            if (kt + 2 < nk) load_global(kt + 2);
        }
        __syncthreads();
    }

    // ---- epilogue: lane holds C[m = .. + lr][n = .. + 8*grp + 4*lk + 0..3]
#pragma unroll
    for (int i = 0; i < TI; ++i) {
        const int m = tm * BM + wm * (BM / 2) + i * 32 + lr;
        if (m >= p.m) continue;
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
#pragma unroll
            for (int grp = 0; grp < 4; ++grp) {
                const int n = tn * BN + wn * (BN / 2) + j * 32 + grp * 8 + lk * 4;
                if (n >= p.n) continue;
                const int64_t off = (g * p.m + m) * static_cast<int64_t>(p.n) + n;
                if constexpr (OUT_BF16) {
                    u32x2_t w = {pack_bf16x2(acc[i][j][grp * 4 + 0], acc[i][j][grp * 4 + 1]),
                                 pack_bf16x2(acc[i][j][grp * 4 + 2], acc[i][j][grp * 4 + 3])};
                    *reinterpret_cast<u32x2_t*>(static_cast<uint16_t*>(p.c) + off) = w;
                } else {
                    f32x4_t w = {acc[i][j][grp * 4 + 0], acc[i][j][grp * 4 + 1], acc[i][j][grp * 4 + 2],
                                 acc[i][j][grp * 4 + 3]};
                    *reinterpret_cast<f32x4_t*>(static_cast<float*>(p.c) + off) = w;
                }
            }
        }
    }
}

// Same GEMM for K % 32 == 0, with the operand slices moved by the global->LDS path
// (buffer_load ... lds) instead of through registers:
//   * K steps of 32 rotate through four LDS stages, so the loads of step kt+3 are in flight
//     while step kt is multiplied (no staging registers, no ds_write instructions);
//   * the stages are four separately declared arrays and the K loop is unrolled by four, so
//     every access names its stage statically: the compiler can then tell the loads into one
//     stage from the fragment reads of another and does not make the reads wait for them;
//   * a stage row is 32 BF16 = 64 B = 4 chunks of 16 B; the chunk index is XORed with
//     (row/4)%4. gfx950's LDS serves a 16-byte read for 16 lanes per clock (64 banks), and
//     a fragment read has 16 consecutive rows at the same chunk in those lanes: four rows share
//     each 256-byte bank line, and the XOR moves the four to distinct chunks, so the 16 reads
//     hit 16 distinct bank groups (measured: 2x the throughput of a (row/2)%4 swizzle). Each
//     wave load instruction fills 1 KB of consecutive LDS (16 rows), so lane l fetches the
//     global chunk the swizzle places at its position (row l/4, chunk (l%4) ^ ((l/16) % 4));
//   * each step is two 16-wide k slices ("phases"); a phase issues the next slice's fragment
//     reads, then the current slice's MFMAs, and the compiler may not reorder across phases.
constexpr int kSBK = 32;       // K per stage (four stages)
__device__ __forceinline__ int swz32(int row, int chunk) {  // element offset in a [rows][32] stage
    return row * kSBK + ((chunk ^ ((row >> 2) & 3)) << 3);
}

// This wave's MFMA operands for one 16-wide k slice of a stage.
template <int BM, int BN>
struct Frags {
    bf16x8_t a[BM / 64];
    bf16x8_t b[BN / 64];
};

template <int BM, int BN>
__device__ __forceinline__ void read_frags(const uint16_t* stage, int ks, int wm, int wn, int lr, int lk,
                                           Frags<BM, BN>& f) {
    const int c = ks * 2 + lk;
    const uint16_t* lb = stage + BM * kSBK;
#pragma unroll
    for (int i = 0; i < BM / 64; ++i)
        f.a[i] = *reinterpret_cast<const bf16x8_t*>(stage + swz32(wm * (BM / 2) + i * 32 + lr, c));
#pragma unroll
    for (int j = 0; j < BN / 64; ++j)
        f.b[j] = *reinterpret_cast<const bf16x8_t*>(lb + swz32(wn * (BN / 2) + j * 32 + lr, c));
}

// The empty asm pins the fragments to VGPRs (the accumulators fill the AGPR file; left to
// itself the register allocator may park fragments there and spill accumulators).
template <int BM, int BN>
__device__ __forceinline__ void mma_frags(Frags<BM, BN>& f, f32x16_t (&acc)[BM / 64][BN / 64]) {
#pragma unroll
    for (int i = 0; i < BM / 64; ++i) asm volatile("" : "+v"(f.a[i]));
#pragma unroll
    for (int j = 0; j < BN / 64; ++j) asm volatile("" : "+v"(f.b[j]));
#pragma unroll
    for (int i = 0; i < BM / 64; ++i)
#pragma unroll
        for (int j = 0; j < BN / 64; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.b[j], f.a[i], acc[i][j], 0, 0, 0);
}

// Fragment r of a slice: r < TI is A fragment r, otherwise B fragment r - TI.
template <int BM, int BN>
__device__ __forceinline__ void read_frag(const uint16_t* stage, int ks, int r, int wm, int wn, int lr, int lk,
                                          Frags<BM, BN>& f) {
    constexpr int TI = BM / 64;
    const int c = ks * 2 + lk;
    if (r < TI)
        f.a[r] = *reinterpret_cast<const bf16x8_t*>(stage + swz32(wm * (BM / 2) + r * 32 + lr, c));
    else
        f.b[r - TI] =
            *reinterpret_cast<const bf16x8_t*>(stage + BM * kSBK + swz32(wn * (BN / 2) + (r - TI) * 32 + lr, c));
}

// One phase: the MFMAs of the current slice (fragments in cur) with, spread between them
// in this order, the reads of the next slice's fragments (read(r), r < TI + TJ, one after
// each of the first MFMAs, so they complete well before the next phase needs them) and P
// global->LDS loads (load(d)). Spreading matters because issue is in order: a burst of LDS or
// memory instructions that the memory pipelines accept slowly would hold back the MFMAs
// behind it. The compiler may not reorder across the fences.
template <int BM, int BN, int P, class Read, class Load>
__device__ __forceinline__ void mma_phase(Frags<BM, BN>& cur, f32x16_t (&acc)[BM / 64][BN / 64], Read&& read,
                                          Load&& load) {
    constexpr int TI = BM / 64, TJ = BN / 64, NM = TI * TJ, NR = TI + TJ;
#pragma unroll
    for (int i = 0; i < TI; ++i) asm volatile("" : "+v"(cur.a[i]));
#pragma unroll
    for (int j = 0; j < TJ; ++j) asm volatile("" : "+v"(cur.b[j]));
    phase_fence();
#pragma unroll
    for (int mi = 0; mi < NM; ++mi) {
        const int i = mi / TJ, j = mi % TJ;
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cur.b[j], cur.a[i], acc[i][j], 0, 0, 0);
        phase_fence();
        // reads: r in [mi*NR/NM', ...) over the first NM' = max(NM/2, 1) MFMAs
        constexpr int NMR = NM / 2 > 0 ? NM / 2 : 1;
#pragma unroll
        for (int r = mi * NR / NMR; r < (mi + 1) * NR / NMR && r < NR; ++r) read(r);
#pragma unroll
        for (int d = mi * P / NM; d < (mi + 1) * P / NM; ++d) load(d);
        phase_fence();
    }
}

// mma_frags with the P global->LDS instructions of one step spread between the MFMAs, so
// the wave issues them while the matrix core is busy instead of stalling on a burst of
// vector memory issue. load(d) issues instruction d.
template <int BM, int BN, int P, class Load>
__device__ __forceinline__ void mma_frags_loads(Frags<BM, BN>& f, f32x16_t (&acc)[BM / 64][BN / 64], Load&& load) {
    constexpr int TI = BM / 64, TJ = BN / 64, NM = TI * TJ;
#pragma unroll
    for (int i = 0; i < TI; ++i) asm volatile("" : "+v"(f.a[i]));
#pragma unroll
    for (int j = 0; j < TJ; ++j) asm volatile("" : "+v"(f.b[j]));
#pragma unroll
    for (int mi = 0; mi < NM; ++mi) {
        const int i = mi / TJ, j = mi % TJ;
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.b[j], f.a[i], acc[i][j], 0, 0, 0);
        // loads [mi*P/NM, (mi+1)*P/NM) follow MFMA mi
#pragma unroll
        for (int d = mi * P / NM; d < (mi + 1) * P / NM; ++d) {
            phase_fence();
            load(d);
            phase_fence();
        }
    }
}


template <int BM, int BN, bool OUT_BF16>
__device__ __forceinline__ void store_tile(const GemmArgs& p, const f32x16_t (&acc)[BM / 64][BN / 64], int tm,
                                           int tn, int64_t g, int wm, int wn, int lr, int lk) {
#pragma unroll
    for (int i = 0; i < BM / 64; ++i) {
        const int m = tm * BM + wm * (BM / 2) + i * 32 + lr;
        if (m >= p.m) continue;
#pragma unroll
        for (int j = 0; j < BN / 64; ++j) {
#pragma unroll
            for (int grp = 0; grp < 4; ++grp) {
                const int n = tn * BN + wn * (BN / 2) + j * 32 + grp * 8 + lk * 4;
                if (n >= p.n) continue;
                const int64_t off = (g * p.m + m) * static_cast<int64_t>(p.n) + n;
                if constexpr (OUT_BF16) {
                    u32x2_t w = {pack_bf16x2(acc[i][j][grp * 4 + 0], acc[i][j][grp * 4 + 1]),
                                 pack_bf16x2(acc[i][j][grp * 4 + 2], acc[i][j][grp * 4 + 3])};
                    *reinterpret_cast<u32x2_t*>(static_cast<uint16_t*>(p.c) + off) = w;
                } else {
                    f32x4_t w = {acc[i][j][grp * 4 + 0], acc[i][j][grp * 4 + 1], acc[i][j][grp * 4 + 2],
                                 acc[i][j][grp * 4 + 3]};
                    *reinterpret_cast<f32x4_t*>(static_cast<float*>(p.c) + off) = w;
                }
            }
        }
    }
}

// NS LDS stages in a ring: step kt reads stage kt % NS while the loads of steps kt+1 .. kt+NS-1 are
// in flight. A grid of at most one 64x64 tile per CU (C1's 128 tiles, 1024^3's 256) is bound by
// that pipeline's depth: each tile walks K in 32-deep steps, each waiting for its loads, so it
// keeps 8 stages (7 steps in flight, 64 KB of LDS); measured back to back on MI355X that takes
// 512x1024x1024 from 6.03 to 5.80 us and 1024^3 from 6.44 to 6.15 us. Fuller grids keep 4 (with
// 8, 512x4096x4096's 512 tiles went from 32.2 to 32.8 us).
template <int BM, int BN, bool OUT_BF16, int NS>
__global__ void __launch_bounds__(kThreads, (BM >= 256 ? 1 : 2))
gemm_nt_dma_kernel(GemmArgs p) {
    constexpr int TI = BM / 64;
    constexpr int TJ = BN / 64;
    constexpr int kStage = (BM + BN) * kSBK;        // elements per stage
    constexpr int kPerWave = (BM + BN) / 16 / 4;    // 1 KB (16-row) load instructions per wave per step
    static_assert(NS >= 4, "the barrier's wait count assumes NS - 3 whole steps in flight");
    __shared__ __attribute__((aligned(1024))) uint16_t stages[NS][kStage];

    const int tiles = p.tiles_m * p.tiles_n;
    int bid = blockIdx.x;
    if ((tiles & 7) == 0) bid = (bid & 7) * (tiles >> 3) + (bid >> 3);
    constexpr int GROUP = 8;
    const int per_group = GROUP * p.tiles_n;
    const int first_m = (bid / per_group) * GROUP;
    const int gsize = min(p.tiles_m - first_m, GROUP);
    const int tm = first_m + (bid % per_group) % gsize;
    const int tn = (bid % per_group) / gsize;
    const int64_t g = blockIdx.z;
    const uint16_t* A = p.a + g * static_cast<int64_t>(p.m) * p.k;
    const uint16_t* B = weight_slice(p, tm * BM, g);

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, lk = lane >> 5;

    // Loads go through buffer resources over this batch's A and B. The row offset is part of
    // the per-lane (VGPR) offset, which the hardware checks against the buffer's size, so rows
    // past M (N) read as zero instead of reading past the matrix (the scalar offset, which
    // carries only the K position, is not range-checked); they only feed outputs that are not
    // stored.
    const i32x4_t ra = buffer_resource(A, p.m * p.k * 2);
    const i32x4_t rb = buffer_resource(B, p.n * p.k * 2);
    // instruction i of this wave fills stage rows 16*(wave + 4*i) .. +15
    const int r_in = lane >> 2;
    const int voff = ((16 * wave + r_in) * p.k + ((lane & 3) ^ ((r_in >> 2) & 3)) * 8) * 2;
    auto fetch_one = [&](uint16_t* stage, int kt, int i) {
        const uint32_t dst = lds_address(stage + (16 * wave + 64 * i) * kSBK);
        if (i < BM / 64)
            load_lds16(ra, dst, voff + (tm * BM + 64 * i) * p.k * 2, kt * kSBK * 2);
        else
            load_lds16(rb, dst, voff + (tn * BN + 64 * (i - BM / 64)) * p.k * 2, kt * kSBK * 2);
    };
    auto fetch = [&](uint16_t* stage, int kt) {
#pragma unroll
        for (int i = 0; i < kPerWave; ++i) fetch_one(stage, kt, i);
    };

    f32x16_t acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    // Step kt multiplies stage X; its first fragments arrive in fa. Its two phases also issue
    // the loads of step kt+NS-1 into stage Z, freed by the barrier of step kt-1. Between them the
    // workgroup waits for step kt+1 to land in stage Y (the loads of steps kt+2 .. kt+NS-2 and the
    // first half of step kt+NS-1 stay in flight) and meets at the barrier, and Y's first fragments
    // are read while X's last MFMAs run. Every step issues its loads, so the wait counts are the
    // same for all steps: past the last step the loads repeat step nk-1 into stages that are no
    // longer read.
    const int nk = p.k / kSBK;
    const int last = nk - 1;
    Frags<BM, BN> fa, fb;
    auto step = [&](const uint16_t* X, const uint16_t* Y, uint16_t* Z, int kt) {
        const int ahead = kt + NS - 1 < nk ? kt + NS - 1 : last;
        // the loads of step kt+NS-1 are split over both phases (stage Z stays free until that
        // step reads it); at the barrier the second half is still in flight
        constexpr int P0 = (kPerWave + 1) / 2, P1 = kPerWave - P0;
        mma_phase<BM, BN, P0>(
            fa, acc, [&](int r) { read_frag<BM, BN>(X, 1, r, wm, wn, lr, lk, fb); },
            [&](int d) { fetch_one(Z, ahead, d); });
        if (kt + 1 < nk) stage_barrier<(NS - 3) * kPerWave + P0>();
        // after the last step these reads fetch fragments that are never used
        mma_phase<BM, BN, P1>(
            fb, acc, [&](int r) { read_frag<BM, BN>(Y, 0, r, wm, wn, lr, lk, fa); },
            [&](int d) { fetch_one(Z, ahead, P0 + d); });
    };

#pragma unroll
    for (int u = 0; u < NS - 1; ++u) fetch(stages[u], nk > u ? u : last);
    stage_barrier<(NS - 2) * kPerWave>();
    read_frags<BM, BN>(stages[0], 0, wm, wn, lr, lk, fa);
    int kt = 0;
    do {  // nk >= 1: the accumulators never bypass the MFMAs on their way to the epilogue
#pragma unroll
        for (int u = 0; u < NS; ++u)
            if (u == 0 || kt + u < nk) step(stages[u], stages[(u + 1) % NS], stages[(u + NS - 1) % NS], kt + u);
        kt += NS;
    } while (kt < nk);
    // the trailing loads must land before the workgroup ends and its LDS is handed on
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    store_tile<BM, BN, OUT_BF16>(p, acc, tm, tn, g, wm, wn, lr, lk);
}

// out[g][c][r] = in[g][r][c] for BF16, 64x64 tiles through LDS (padded rows).
__global__ void __launch_bounds__(256)
transpose_bf16(const uint16_t* __restrict__ in, uint16_t* __restrict__ out, int64_t rows, int64_t cols) {
    __shared__ uint16_t tile[64][66];
    const int64_t g = blockIdx.z;
    const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 64, c0 = static_cast<int64_t>(blockIdx.x) * 64;
    const uint16_t* src = in + g * rows * cols;
    uint16_t* dst = out + g * rows * cols;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int i = ty; i < 64; i += 4) {
        const int64_t r = r0 + i, c = c0 + tx;
        if (r < rows && c < cols) tile[i][tx] = src[r * cols + c];
    }
    __syncthreads();
    for (int i = ty; i < 64; i += 4) {
        const int64_t c = c0 + i, r = r0 + tx;
        if (r < rows && c < cols) dst[c * rows + r] = tile[tx][i];
    }
}

// The 256x256-tile 4-wave kernel (every transpose) applies when there are enough tiles to fill
// the GPU, K % 8 == 0 (a partial last stage takes the KTAIL variant) and 32-bit byte offsets
// up to the end of the last (zero-padded) stage.
bool pp_applies(int64_t batch, int64_t m, int64_t n, int64_t k, int num_cus) {
    const int64_t tiles = ((m + kPPTile - 1) / kPPTile) * ((n + kPPTile - 1) / kPPTile) * batch;
    const int64_t k64 = (k + kPK - 1) / kPK * kPK;
    return tiles >= num_cus && k > 0 && k % 8 == 0 && m * k64 * 2 < (int64_t{1} << 31) &&
           n * k64 * 2 < (int64_t{1} << 31);
}

// Output tile width: 256 (NJ = 8) or 192 (NJ = 6) for a grid of `batch` x M/256 x N/(32 NJ) tiles
// on num_cus CUs, whichever takes fewer rounds of workgroups times the time of one tile. Measured
// on MI355X with each width forced: a part-empty last round costs nearly a full one, and a narrow
// tile takes ~1.1-1.15x the square tile's time per flop, so a round costs 80 (square) or 69
// (192-wide): narrow tiles are taken only when they save a whole round. C3's shapes fill whole
// rounds of square tiles and stay square; C5's 4096 x 6144 QKV projection (384 square tiles, 1.5
// rounds) runs 512 narrow tiles in 2 rounds (alone 168 -> 151 us; 180 -> 175 us inside the layer).
// 224-wide tiles (NJ = 7) for the 896-tile 4096 x 14336 outputs gained 1-4% alone and nothing
// inside the layer, so they are not built.
int pick_tile_nj(int64_t batch, int64_t m, int64_t n, int num_cus) {
    const int64_t tiles_m = (m + kPPTile - 1) / kPPTile;
    auto cost = [&](int nj, int per_round) {
        const int64_t tiles = tiles_m * ((n + 32 * nj - 1) / (32 * nj)) * batch;
        return (tiles + num_cus - 1) / num_cus * per_round;
    };
    return cost(6, 69) < cost(8, 80) ? 6 : 8;
}

template <bool OUT_BF16, int NJ>
void launch_pp_nj(const GemmArgs& p, const dim3& grid, bool a_mn, bool b_mn, hipStream_t s) {
    if (a_mn && b_mn) hipLaunchKernelGGL((gemm_nt_m16_kernel<OUT_BF16, true, true, false, NJ>), grid, dim3(kW4Threads), 0, s, p);
    else if (a_mn) hipLaunchKernelGGL((gemm_nt_m16_kernel<OUT_BF16, true, false, false, NJ>), grid, dim3(kW4Threads), 0, s, p);
    else if (b_mn) hipLaunchKernelGGL((gemm_nt_m16_kernel<OUT_BF16, false, true, false, NJ>), grid, dim3(kW4Threads), 0, s, p);
    else hipLaunchKernelGGL((gemm_nt_m16_kernel<OUT_BF16, false, false, false, NJ>), grid, dim3(kW4Threads), 0, s, p);
}

template <bool OUT_BF16>
void launch_pp(const GemmArgs& a, int64_t batch, bool a_mn, bool b_mn, int num_cus, hipStream_t s) {
    GemmArgs p = a;
    // narrower tiles only for whole K stages (the KTAIL variants stay square)
    const int nj = p.k % kPK == 0 ? pick_tile_nj(batch, p.m, p.n, num_cus) : 8;
    p.tiles_m = (p.m + kPPTile - 1) / kPPTile;
    p.tiles_n = (p.n + 32 * nj - 1) / (32 * nj);
    const dim3 grid(static_cast<unsigned>(p.tiles_m * p.tiles_n), 1, static_cast<unsigned>(batch));
    // Square tile grids run bands of 4 M-tile rows per XCD; other grids bands of 8 N-tile
    // columns, so an XCD's L2 holds a narrow slice of B (Llama projections 8192x4096->14336
    // and 8192x14336->4096: 1.40 -> 1.49 and 1.38 -> 1.47 PFLOP/s; 8192^3 keeps 1.54 with
    // M bands vs 1.50 with N bands).
    p.band_n = p.tiles_m == p.tiles_n ? 0 : 8;
    if (p.k % kPK != 0) {
        if (a_mn && b_mn) hipLaunchKernelGGL((gemm_nt_m16_kernel<OUT_BF16, true, true, true>), grid, dim3(kW4Threads), 0, s, p);
        else if (a_mn) hipLaunchKernelGGL((gemm_nt_m16_kernel<OUT_BF16, true, false, true>), grid, dim3(kW4Threads), 0, s, p);
        else if (b_mn) hipLaunchKernelGGL((gemm_nt_m16_kernel<OUT_BF16, false, true, true>), grid, dim3(kW4Threads), 0, s, p);
        else hipLaunchKernelGGL((gemm_nt_m16_kernel<OUT_BF16, false, false, true>), grid, dim3(kW4Threads), 0, s, p);
        return;
    }
    if (nj == 6) launch_pp_nj<OUT_BF16, 6>(p, grid, a_mn, b_mn, s);
    else launch_pp_nj<OUT_BF16, 8>(p, grid, a_mn, b_mn, s);
}

template <int BM, int BN>
void launch_nt(const GemmArgs& a, int64_t batch, bool out_bf16, int num_cus, hipStream_t s) {
    GemmArgs p = a;
    p.tiles_m = (p.m + BM - 1) / BM;
    p.tiles_n = (p.n + BN - 1) / BN;
    const dim3 grid(static_cast<unsigned>(p.tiles_m * p.tiles_n), 1, static_cast<unsigned>(batch));
    // the global->LDS kernel needs whole K steps and 32-bit byte offsets into A and B
    const bool whole_steps = p.k % kSBK == 0 && p.k > 0 && static_cast<int64_t>(p.m) * p.k * 2 < (int64_t{1} << 31) &&
                             static_cast<int64_t>(p.n) * p.k * 2 < (int64_t{1} << 31);
    if (whole_steps && p.k % kPK == 0 && BM == kPPTile && BN == kPPTile) {
        if (out_bf16) launch_pp<true>(p, batch, false, false, num_cus, s);
        else launch_pp<false>(p, batch, false, false, num_cus, s);
    } else if (whole_steps && BM == 64 && grid.x * grid.z <= static_cast<unsigned>(num_cus)) {
        if constexpr (BM == 64) {
            if (out_bf16) hipLaunchKernelGGL((gemm_nt_dma_kernel<BM, BN, true, 8>), grid, dim3(kThreads), 0, s, p);
            else hipLaunchKernelGGL((gemm_nt_dma_kernel<BM, BN, false, 8>), grid, dim3(kThreads), 0, s, p);
        }
    } else if (whole_steps && out_bf16)
        hipLaunchKernelGGL((gemm_nt_dma_kernel<BM, BN, true, 4>), grid, dim3(kThreads), 0, s, p);
    else if (whole_steps)
        hipLaunchKernelGGL((gemm_nt_dma_kernel<BM, BN, false, 4>), grid, dim3(kThreads), 0, s, p);
    else if (out_bf16)
        hipLaunchKernelGGL((gemm_nt_kernel<BM, BN, true>), grid, dim3(kThreads), 0, s, p);
    else
        hipLaunchKernelGGL((gemm_nt_kernel<BM, BN, false>), grid, dim3(kThreads), 0, s, p);
}

// Output tile of 256, 128 or 64: the largest whose grid still fills the CUs.
void launch_nt_sized(const GemmArgs& p, int64_t batch, bool out_bf16, int num_cus, hipStream_t s) {
    const int64_t m = p.m, n = p.n;
    const int64_t t256 = ((m + 255) / 256) * ((n + 255) / 256) * batch;
    const int64_t t128 = ((m + 127) / 128) * ((n + 127) / 128) * batch;
    if (t256 >= num_cus) launch_nt<256, 256>(p, batch, out_bf16, num_cus, s);
    else if (t128 >= num_cus) launch_nt<128, 128>(p, batch, out_bf16, num_cus, s);
    else launch_nt<64, 64>(p, batch, out_bf16, num_cus, s);
}

size_t round256(size_t x) { return (x + 255) & ~size_t(255); }

}  // namespace

size_t gemm_workspace_bytes(int64_t batch, int64_t m, int64_t n, int64_t k, int ta, int tb) {
    size_t bytes = 0;
    if (ta) bytes += round256(static_cast<size_t>(batch * m * k) * 2);
    if (!tb) bytes += round256(static_cast<size_t>(batch * n * k) * 2);
    return bytes;
}

hipError_t gemm_bf16(const void* a, const void* b, void* c, int out_bf16, int64_t batch, int64_t m, int64_t n,
                     int64_t k, int ta, int tb, void* workspace, int num_cus, hipStream_t s) {
    const uint16_t* ak = static_cast<const uint16_t*>(a);
    const uint16_t* bk = static_cast<const uint16_t*>(b);
    if (pp_applies(batch, m, n, k, num_cus)) {  // MN-major operands are read in place
        GemmArgs p{};
        p.a = ak;
        p.b = bk;
        p.c = c;
        p.m = static_cast<int>(m);
        p.n = static_cast<int>(n);
        p.k = static_cast<int>(k);
        if (out_bf16) launch_pp<true>(p, batch, ta != 0, tb == 0, num_cus, s);
        else launch_pp<false>(p, batch, ta != 0, tb == 0, num_cus, s);
        return hipGetLastError();
    }
    char* ws = static_cast<char*>(workspace);
    if (ta) {  // A stored [K,M] -> [M,K]
        uint16_t* t = reinterpret_cast<uint16_t*>(ws);
        hipLaunchKernelGGL(transpose_bf16, dim3((unsigned)((m + 63) / 64), (unsigned)((k + 63) / 64), (unsigned)batch),
                           dim3(256), 0, s, ak, t, k, m);
        ak = t;
        ws += round256(static_cast<size_t>(batch * m * k) * 2);
    }
    if (!tb) {  // B stored [K,N] -> [N,K]
        uint16_t* t = reinterpret_cast<uint16_t*>(ws);
        hipLaunchKernelGGL(transpose_bf16, dim3((unsigned)((n + 63) / 64), (unsigned)((k + 63) / 64), (unsigned)batch),
                           dim3(256), 0, s, bk, t, k, n);
        bk = t;
    }
    GemmArgs p{};
    p.a = ak;
    p.b = bk;
    p.c = c;
    p.m = static_cast<int>(m);
    p.n = static_cast<int>(n);
    p.k = static_cast<int>(k);
    launch_nt_sized(p, batch, out_bf16, num_cus, s);
    return hipGetLastError();
}

bool epi_applies(int64_t m, int64_t n, int64_t k) {
    const int64_t k64 = (k + kPK - 1) / kPK * kPK;
    return m > 0 && n > 0 && k > 0 && k % 8 == 0 && m * k64 * 2 < (int64_t{1} << 31) &&
           n * k64 * 2 < (int64_t{1} << 31);
}

bool qkv_rope_applies(int64_t tokens, int64_t hidden, int64_t width) {
    return width % 128 == 0 && epi_applies(tokens, width, hidden);
}

namespace {
// A fused-epilogue GEMM over p.m x p.n outputs (256x256 tiles, bands of 8 N-tiles per XCD unless
// the tile grid is square, as launch_pp chooses).
template <int EPI, bool B_MN>
hipError_t launch_epi(GemmEpiArgs p, hipStream_t s) {
    p.tiles_m = (p.m + kPPTile - 1) / kPPTile;
    p.tiles_n = (p.n + kPPTile - 1) / kPPTile;
    p.band_n = p.tiles_m == p.tiles_n ? 0 : 8;
    const dim3 grid(static_cast<unsigned>(p.tiles_m * p.tiles_n));
    if (p.k % kPK != 0) hipLaunchKernelGGL((gemm_epi_kernel<EPI, B_MN, true>), grid, dim3(kW4Threads), 0, s, p);
    else hipLaunchKernelGGL((gemm_epi_kernel<EPI, B_MN, false>), grid, dim3(kW4Threads), 0, s, p);
    return hipGetLastError();
}

GemmEpiArgs epi_args(const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t k) {
    GemmEpiArgs p{};
    p.a = static_cast<const uint16_t*>(a);
    p.b = static_cast<const uint16_t*>(b);
    p.c = c;
    p.m = static_cast<int>(m);
    p.n = static_cast<int>(n);
    p.k = static_cast<int>(k);
    return p;
}
}  // namespace

hipError_t gemm_qkv_rope(const void* x, const void* w, int64_t tokens, int64_t hidden, int64_t seq, int64_t hq,
                         int64_t hkv, const float* cos_t, const float* sin_t, int layout, void* q, void* k, void* v,
                         hipStream_t s) {
    GemmEpiArgs p = epi_args(x, w, nullptr, tokens, (hq + 2 * hkv) * 128, hidden);
    p.qkv = QkvRopeOut{static_cast<uint16_t*>(q), static_cast<uint16_t*>(k), static_cast<uint16_t*>(v), cos_t, sin_t,
                       static_cast<int>(seq), static_cast<int>(hq), static_cast<int>(hkv), layout};
    return launch_epi<kEpiQkvRope, false>(p, s);
}

hipError_t gemm_residual(const void* x, const void* w, const void* res, void* y, int64_t m, int64_t n, int64_t k,
                         hipStream_t s) {
    GemmEpiArgs p = epi_args(x, w, y, m, n, k);
    p.res = static_cast<const uint16_t*>(res);
    return launch_epi<kEpiResidual, false>(p, s);
}

hipError_t gemm_swiglu(const void* x, const void* w_gu, void* gate, void* up, void* act, int64_t m, int64_t f,
                       int64_t k, hipStream_t s) {
    GemmEpiArgs p = epi_args(x, w_gu, nullptr, m, 2 * f, k);
    p.gate = static_cast<uint16_t*>(gate);
    p.up = static_cast<uint16_t*>(up);
    p.act = static_cast<uint16_t*>(act);
    return launch_epi<kEpiSwiglu, false>(p, s);
}

hipError_t gemm_swiglu_backward(const void* dy, const void* wd, const void* gate, const void* up, void* dgu, int64_t m,
                                int64_t f, int64_t k, hipStream_t s) {
    GemmEpiArgs p = epi_args(dy, wd, nullptr, m, f, k);
    p.gate = const_cast<uint16_t*>(static_cast<const uint16_t*>(gate));
    p.up = const_cast<uint16_t*>(static_cast<const uint16_t*>(up));
    p.dgu = static_cast<uint16_t*>(dgu);
    return launch_epi<kEpiSwigluBwd, true>(p, s);
}

hipError_t gemm_bf16_grouped_nt(const void* a, const void* w, void* c, int out_bf16, int64_t m, int64_t n, int64_t k,
                                const int32_t* block_group, int num_cus, hipStream_t s) {
    GemmArgs p{};
    p.a = static_cast<const uint16_t*>(a);
    p.b = static_cast<const uint16_t*>(w);
    p.c = c;
    p.m = static_cast<int>(m);
    p.n = static_cast<int>(n);
    p.k = static_cast<int>(k);
    p.block_group = block_group;
    if (pp_applies(1, m, n, k, num_cus)) {
        if (out_bf16) launch_pp<true>(p, 1, false, false, num_cus, s);
        else launch_pp<false>(p, 1, false, false, num_cus, s);
    } else {
        launch_nt_sized(p, 1, out_bf16, num_cus, s);
    }
    return hipGetLastError();
}

}  // namespace hk
