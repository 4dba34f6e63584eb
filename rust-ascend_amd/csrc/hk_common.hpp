// hk_common.hpp — device helpers shared by the gfx950 kernels of libhk.so.
//
// BF16 values live in memory as raw uint16_t (the top half of an IEEE float32).
// Conversions use the gfx950 hardware converter (v_cvt_pk_bf16_f32, round to
// nearest even), the rounding the reference's host checks apply
// (rust-ascend-kernels/src/tests.rs:7-11).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <initializer_list>

namespace hk {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Two floats -> one dword holding two BF16 (lo = a, hi = b), RNE.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    f32x2_t v = {a, b};
    bf16x2_t h = __builtin_convertvector(v, bf16x2_t);
    return __builtin_bit_cast(uint32_t, h);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float a) {
    return static_cast<uint16_t>(pack_bf16x2(a, 0.0f) & 0xffffu);
}
// a rounded to BF16 (RNE) and widened back: the value a BF16 store and reload would give.
__device__ __forceinline__ float round_bf16(float a) { return bf16lo(pack_bf16x2(a, 0.0f)); }

// Element loaders/storers used by kernels templated on the storage type.
template <typename T> struct Elem;
template <> struct Elem<float> {
    static __device__ __forceinline__ float load(const float* p, int64_t i) { return p[i]; }
    static __device__ __forceinline__ void store(float* p, int64_t i, float v) { p[i] = v; }
};
template <> struct Elem<uint16_t> {
    static __device__ __forceinline__ float load(const uint16_t* p, int64_t i) { return bf16_to_f32(p[i]); }
    static __device__ __forceinline__ void store(uint16_t* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }
};

// Eight consecutive elements as floats: one 16-byte load for BF16, two for F32.
__device__ __forceinline__ void load8(const uint16_t* p, float (&v)[8]) {
    u32x4_t w = *reinterpret_cast<const u32x4_t*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = bf16lo(w[i]);
        v[2 * i + 1] = bf16hi(w[i]);
    }
}
__device__ __forceinline__ void load8(const float* p, float (&v)[8]) {
    f32x4_t a = *reinterpret_cast<const f32x4_t*>(p);
    f32x4_t b = *reinterpret_cast<const f32x4_t*>(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[i] = a[i];
        v[4 + i] = b[i];
    }
}
__device__ __forceinline__ void store8(uint16_t* p, const float (&v)[8]) {
    u32x4_t w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
    *reinterpret_cast<u32x4_t*>(p) = w;
}
__device__ __forceinline__ void store8(float* p, const float (&v)[8]) {
    f32x4_t a = {v[0], v[1], v[2], v[3]};
    f32x4_t b = {v[4], v[5], v[6], v[7]};
    *reinterpret_cast<f32x4_t*>(p) = a;
    *reinterpret_cast<f32x4_t*>(p + 4) = b;
}

// Streaming (non-temporal) 16-byte accesses for rows that are read or written once: the nt bit
// marks the lines as streaming in L2 and in the on-package cache. Measured on MI355X over 1 GiB
// buffers: copy 6.4 TB/s with nt loads and stores vs 5.5-5.7 TB/s without; two reads + one
// write 6.4 vs 5.5-5.7 TB/s; read-only 7.1 vs 6.3 TB/s. Used where a kernel's working set is
// larger than the 256 MB on-package cache; a kernel whose input may still sit in that cache
// (RoPE over a 134 MB Q measured 6.25 TB/s cached vs 5.06 TB/s streaming) keeps plain accesses.
template <class V>
__device__ __forceinline__ V stream_load(const V* p) { return __builtin_nontemporal_load(p); }
template <class V>
__device__ __forceinline__ void stream_store(const V& v, V* p) { __builtin_nontemporal_store(v, p); }

__device__ __forceinline__ void load8_stream(const uint16_t* p, float (&v)[8]) {
    const u32x4_t w = stream_load(reinterpret_cast<const u32x4_t*>(p));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = bf16lo(w[i]);
        v[2 * i + 1] = bf16hi(w[i]);
    }
}
__device__ __forceinline__ void load8_stream(const float* p, float (&v)[8]) {
    const f32x4_t a = stream_load(reinterpret_cast<const f32x4_t*>(p));
    const f32x4_t b = stream_load(reinterpret_cast<const f32x4_t*>(p + 4));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[i] = a[i];
        v[4 + i] = b[i];
    }
}
__device__ __forceinline__ void store8_stream(uint16_t* p, const float (&v)[8]) {
    u32x4_t w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
    stream_store(w, reinterpret_cast<u32x4_t*>(p));
}
__device__ __forceinline__ void store8_stream(float* p, const float (&v)[8]) {
    stream_store(f32x4_t{v[0], v[1], v[2], v[3]}, reinterpret_cast<f32x4_t*>(p));
    stream_store(f32x4_t{v[4], v[5], v[6], v[7]}, reinterpret_cast<f32x4_t*>(p + 4));
}

// IEEE half storage (F16), converted with the hardware round-to-nearest-even converter.
template <> struct Elem<_Float16> {
    static __device__ __forceinline__ float load(const _Float16* p, int64_t i) { return static_cast<float>(p[i]); }
    static __device__ __forceinline__ void store(_Float16* p, int64_t i, float v) { p[i] = static_cast<_Float16>(v); }
};

// 16-byte chunks of kPer consecutive elements as floats (one streaming vector load/store per
// chunk: element-wise tensors are read or written once).
template <typename T> struct Chunk;
template <> struct Chunk<float> {
    static constexpr int kPer = 4;
    __device__ static void load(const float* p, float (&v)[4]) {
        const f32x4_t w = stream_load(reinterpret_cast<const f32x4_t*>(p));
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = w[i];
    }
    __device__ static void store(float* p, const float (&v)[4]) {
        stream_store(f32x4_t{v[0], v[1], v[2], v[3]}, reinterpret_cast<f32x4_t*>(p));
    }
};
template <> struct Chunk<uint16_t> {
    static constexpr int kPer = 8;
    __device__ static void load(const uint16_t* p, float (&v)[8]) { load8_stream(p, v); }
    __device__ static void store(uint16_t* p, const float (&v)[8]) { store8_stream(p, v); }
};
template <> struct Chunk<_Float16> {
    static constexpr int kPer = 8;
    typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
    __device__ static void load(const _Float16* p, float (&v)[8]) {
        const h8_t w = *reinterpret_cast<const h8_t*>(p);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = static_cast<float>(w[i]);
    }
    __device__ static void store(_Float16* p, const float (&v)[8]) {
        h8_t w;
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = static_cast<_Float16>(v[i]);
        *reinterpret_cast<h8_t*>(p) = w;
    }
};

// RoPE rotation of the pair (a, b) by (c, s) = (cos, sin) of its angle, in the reference's
// expression order (rust-ascend-compiler/src/ascend/rotary_programs.rs:47-156): forward
// y_a = a c - b s, y_b = b c + a s; backward (the transpose Jacobian) y_a = a c + b s,
// y_b = b c - a s. Every kernel that rotates calls this, so fused and standalone RoPE agree bit
// for bit; the products are rounded before the sum (no contraction into fused multiply-adds,
// which the compiler could otherwise choose differently in different kernels), as the
// reference's separate vector multiply and add do.
template <bool BWD>
__device__ __forceinline__ void rope_rotate(float a, float b, float c, float s, float& ya, float& yb) {
#pragma clang fp contract(off)
    if constexpr (!BWD) {
        ya = a * c - b * s;
        yb = b * c + a * s;
    } else {
        ya = a * c + b * s;
        yb = b * c - a * s;
    }
}

// SwiGLU gate in the reference's order of operations (rust-ascend-compiler/src/ascend/programs.rs:
// 21-46): s = 1 / (1 + exp(-g)), y = (g s) u; backward ds = s (1 + g (1 - s)), dgate = (dy u) ds,
// dup = dy (g s). Shared by the element-wise kernels and the GEMM epilogues that fuse them, with
// no contraction into fused multiply-adds, so both give the same bits.
// The sigmoid takes the hardware's exp2 and reciprocal (v_exp_f32, v_rcp_f32, each within 1 ulp)
// on -g log2(e): relative error ~1e-6 at |g| = 12 (the rounding of g log2(e) scaled by |g|), far
// inside the reference's |a-b| <= 2e-5 + 1e-4|b|, in 4 instructions where expf and an IEEE
// division take ~25 -- in a GEMM epilogue, which overlaps nothing, that is ~10% of the SwiGLU
// backward's time. exp2 of a large argument is +inf, whose reciprocal is 0 (s = 0); of a very
// negative one 0 (s = 1).
__device__ __forceinline__ float sigmoid1(float g) {
#pragma clang fp contract(off)
    const float e = __builtin_amdgcn_exp2f(g * -1.44269504088896340736f);
    return __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ float silu_mul1(float g, float u) {
#pragma clang fp contract(off)
    const float s = sigmoid1(g);
    return (g * s) * u;
}

__device__ __forceinline__ void silu_mul_bwd1(float g, float u, float dy, float& dg, float& du) {
#pragma clang fp contract(off)
    const float s = sigmoid1(g);
    const float h = g * s;
    const float ds = s * (1.0f + g * (1.0f - s));
    dg = (dy * u) * ds;
    du = dy * h;
}

// max / sum of x over lanes l and l ^ 32, on every lane: v_permlane32_swap exchanges the wave's two
// 32-lane halves in the VALU (a few cycles) where __shfl_xor(x, 32) takes a ds_bpermute (~75 cycles
// of LDS latency). The swap returns {lanes 0-31 of x twice, lanes 32-63 of x twice}, so lane l sees
// x[l % 32] and x[l % 32 + 32]; both operations are symmetric, so every lane gets the same value
// __shfl_xor would give it.
__device__ __forceinline__ float pair32_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair32_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// LDS vector types for the transposing reads (ds_read_b64_tr_b16).
typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16_t lds_v4i16_t;

// Every pointer 16-byte aligned (the vector chunk paths need it).
__host__ __forceinline__ bool aligned16(std::initializer_list<const void*> ptrs) {
    for (const void* p : ptrs)
        if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return false;
    return true;
}

// Flat (one work item per element or chunk) launches. A dispatch's work-item count is a 32-bit
// quantity, so these grids are capped at 2^20 workgroups (2^28 work items at 256 threads, which
// still fills 256 CUs many times over) and the kernels walk their index space with a grid stride.
constexpr int64_t kMaxFlatBlocks = int64_t{1} << 20;
__host__ __forceinline__ unsigned flat_blocks(int64_t work, int threads) {
    const int64_t b = (work + threads - 1) / threads;
    return static_cast<unsigned>(b < kMaxFlatBlocks ? b : kMaxFlatBlocks);
}
__device__ __forceinline__ int64_t flat_begin(int threads) {
    return static_cast<int64_t>(blockIdx.x) * threads + threadIdx.x;
}
__device__ __forceinline__ int64_t flat_stride(int threads) { return static_cast<int64_t>(gridDim.x) * threads; }

// x of lane l ^ 7 (ctrl 0x141, DPP row_half_mirror), l ^ 15 (0x140, row_mirror), l ^ 1 (0xB1,
// quad_perm [1,0,3,2]) or l ^ 2 (0x4E, quad_perm [2,3,0,1]): VALU lane moves within 16-lane rows.
template <int CTRL>
__device__ __forceinline__ float lane_dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Sum / max over the 64 lanes of a wavefront; every lane receives the same value. A butterfly over
// the lane masks 32, 16 (the half swaps of v_permlane32_swap / v_permlane16_swap), 7, 15, 1, 2 (DPP
// moves): six steps, each adding lane l's value and lane l ^ mask's in a commutative operation, so
// partners compute the same value, and the masks span all 64 lanes, so every lane ends with the
// total of one fixed association (deterministic). No LDS traffic: the ds_bpermute that __shfl_xor
// compiles to costs ~75 cycles of latency per step, on the row's dependency chain in the row kernels.
__device__ __forceinline__ float wave_sum(float v) {
    v = pair32_sum(v);
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    v += lane_dpp<0x141>(v);
    v += lane_dpp<0x140>(v);
    v += lane_dpp<0xB1>(v);
    v += lane_dpp<0x4E>(v);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
    v = pair32_max(v);
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    v = fmaxf(v, lane_dpp<0x141>(v));
    v = fmaxf(v, lane_dpp<0x140>(v));
    v = fmaxf(v, lane_dpp<0xB1>(v));
    v = fmaxf(v, lane_dpp<0x4E>(v));
    return v;
}

// ---- global->LDS loads (buffer_load ... lds)

typedef int i32x4_t __attribute__((ext_vector_type(4)));

// Buffer resource word 3 for gfx9-family raw buffer loads (32-bit data format).
constexpr int kBufferConfig = 0x00020000;

// Raw buffer resource over `bytes` bytes at `base` (wave-uniform).
__device__ __forceinline__ i32x4_t buffer_resource(const void* base, int bytes) {
    const uint64_t addr = reinterpret_cast<uint64_t>(base);
    return i32x4_t{__builtin_amdgcn_readfirstlane(static_cast<int>(addr)),
                   __builtin_amdgcn_readfirstlane(static_cast<int>(addr >> 32)),
                   __builtin_amdgcn_readfirstlane(bytes), kBufferConfig};
}

// LDS byte address of a __shared__ element (wave-uniform pointer).
__device__ __forceinline__ uint32_t lds_address(const uint16_t* p) {
    const auto* l = (const __attribute__((address_space(3))) uint16_t*)(p);
    return __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(l)));
}

// One wave instruction of the global->LDS path: 16 bytes per lane from rsrc + voff + soff
// into LDS at lds + 16 * lane. Issued as inline assembly so that the compiler's wait-count
// insertion does not track it: a kernel using it waits for these loads itself (s_waitcnt
// vmcnt before the barrier that publishes the tile), at the distance its buffering allows,
// instead of before every later LDS read. M0 holds the LDS address; the kernels that use this
// keep no other value in M0.
__device__ __forceinline__ void load_lds16(i32x4_t rsrc, uint32_t lds, int voff, int soff) {
    asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %0, %2, %3 offen lds"
                 :
                 : "v"(voff), "s"(lds), "s"(rsrc), "s"(soff)
                 : "memory");
}

// load_lds16 for data read once: the non-temporal hint lets the line leave the caches first.
__device__ __forceinline__ void load_lds16_nt(i32x4_t rsrc, uint32_t lds, int voff, int soff) {
    asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %0, %2, %3 offen nt lds"
                 :
                 : "v"(voff), "s"(lds), "s"(rsrc), "s"(soff)
                 : "memory");
}

// The 4-byte form: lane l's dword lands at lds + 4 * l (one instruction moves 256 bytes).
__device__ __forceinline__ void load_lds4(i32x4_t rsrc, uint32_t lds, int voff, int soff) {
    asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dword %0, %2, %3 offen lds"
                 :
                 : "v"(voff), "s"(lds), "s"(rsrc), "s"(soff)
                 : "memory");
}

// Workgroup barrier for kernels whose global->LDS loads must stay in flight across it: every
// LDS access this wave issued before it has completed (lgkmcnt 0), but outstanding vector
// memory operations are not waited for (the release fence of __syncthreads would wait for
// them too). The empty asm statements keep the compiler from moving memory accesses across.
// gfx9 s_waitcnt encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // vmcnt 63 (no wait), expcnt 7 (no wait), lgkmcnt 0
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

}  // namespace hk
