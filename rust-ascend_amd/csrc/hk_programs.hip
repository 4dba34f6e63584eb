// hk_programs.hip — the GEMM device programs of the reference's launch ABI, built ahead of time
// into a gfx950 code object (rust-ascend_amd/lib/hk_programs.hsaco) that the driver loads with
// hipModuleLoad and launches with hipModuleLaunchKernel (hk_module_load / hk_module_launch_gemm).
//
// Reference: rust-ascend-kernels/src/ascend.rs:88-114 (entry signature and the RudaGm /
// RudaEpilogue structs), config.rs:14-40 (the 18 programs and their names), deepgemm/native.rs:
// 80-93 and deepgemm/mod.rs:122-145 (the nine-argument launch). Each entry point
//   ruda_rust_bf16_{dense,batched}_{n,t}{n,t}_{bf16,f32}, ruda_rust_bf16_mgrouped_nt_{bf16,f32}
// takes (RudaGm a, RudaGm b, RudaGm d, u32 m, u32 n, u32 k, i32* grouped_layout, u32 num_groups,
// RudaEpilogue epilogue) and computes D = op(A) op(B) (alpha 1, FP32 accumulation) with the
// 256x256-tile kernel of libhk.so (hk_gemm_device.hpp): one output tile per workgroup, grid
// tiles_m * tiles_n x 1 x batches, 256 threads. num_groups is the batch count of the batched
// programs and the group count of the M-grouped ones, whose grouped_layout holds the ascending,
// 256-aligned group row ends (repeated ends are empty groups). The driver checks every argument
// against the reference's contract before a launch (packed strides, alpha 1, M/N/K multiples of
// 16, operand offsets within the 32-bit or the wide form's reach), so the programs trust them.
#include "hk_common.hpp"
#include "hk_gemm_device.hpp"

namespace hk {

namespace {

// ascend.rs:90-91 (sizes checked by the reference at native.rs:96)
struct RudaGm {
    uint64_t addr;
    uint64_t stride_outer;
    uint64_t stride_batch;
};
struct RudaEpilogue {
    float alpha;
    uint32_t pad0;
    uint64_t sfd;
    uint64_t stride;
    uint32_t n;
    uint32_t pad1;
};
static_assert(sizeof(RudaGm) == 24, "RudaGm layout");
static_assert(sizeof(RudaEpilogue) == 32, "RudaEpilogue layout");

// The tile kernel's arguments plus the reference's group-end table of the M-grouped programs.
struct ProgramArgs : GemmArgs {
    const int32_t* group_ends;
    int num_groups;
};

// B slice of the tile whose first row is row0: the batch's, or the group's whose row range
// [ends[s-1], ends[s]) holds row0 (empty groups, with repeated ends, are passed over).
__device__ __forceinline__ const uint16_t* weight_slice(const ProgramArgs& p, int row0, int64_t g) {
    int64_t slice = g;
    if (p.group_ends) {
        int s = 0;
        while (s + 1 < p.num_groups && p.group_ends[s] <= row0) ++s;
        slice = s;
    }
    return p.b + slice * static_cast<int64_t>(p.n) * p.k;
}

// ta / tb are the reference's transposes: A stored [K,M] (ta) is the MN-major A operand of the
// tile kernel; B stored [K,N] (not tb) is its MN-major B operand. The tile kernel's partial last
// K stage handles K % 64 != 0 and reads whole stages exactly as the full-stage variant when
// K % 64 == 0, so one variant serves every K.
template <bool OUT_BF16, bool TA, bool TB, bool WIDE>
__device__ __forceinline__ void run_program(const RudaGm& a, const RudaGm& b, const RudaGm& d, uint32_t m, uint32_t n,
                                            uint32_t k, const int32_t* grouped_layout, uint32_t num_groups) {
    ProgramArgs p{};
    p.a = reinterpret_cast<const uint16_t*>(a.addr);
    p.b = reinterpret_cast<const uint16_t*>(b.addr);
    p.c = reinterpret_cast<void*>(d.addr);
    p.m = static_cast<int>(m);
    p.n = static_cast<int>(n);
    p.k = static_cast<int>(k);
    p.tiles_m = static_cast<int>((m + kPPTile - 1) / kPPTile);
    p.tiles_n = static_cast<int>((n + kPPTile - 1) / kPPTile);
    p.block_group = nullptr;
    p.band_n = p.tiles_m == p.tiles_n ? 0 : 8;  // libhk.so's tile order for the shape
    p.group_ends = grouped_layout;
    p.num_groups = static_cast<int>(num_groups);
    gemm_m16_tile<OUT_BF16, TA, !TB, true, ProgramArgs, 8, kEpiPlain, WIDE>(p);
}

}  // namespace

}  // namespace hk

// Each program NAME has a companion NAME_wide, the same program for operand slices past 32-bit
// byte offsets (M*K or N*K >= 2^30 elements); the driver launches it in NAME's place for those
// shapes. It is not one of the reference's names and callers never ask for it.
#define HK_PROGRAM_ENTRY(SYMBOL, OUT_BF16, TA, TB, WIDE)                                                        \
    extern "C" __global__ void __launch_bounds__(hk::kW4Threads, 1)                                            \
        SYMBOL(hk::RudaGm gm_a, hk::RudaGm gm_b, hk::RudaGm gm_d, uint32_t shape_m, uint32_t shape_n,           \
               uint32_t shape_k, int32_t* grouped_layout, uint32_t num_groups, hk::RudaEpilogue epilogue) {       \
        (void)epilogue;                                                                                        \
        hk::run_program<OUT_BF16, TA, TB, WIDE>(gm_a, gm_b, gm_d, shape_m, shape_n, shape_k, grouped_layout,   \
                                                num_groups);                                                   \
    }
#define HK_PROGRAM(NAME, OUT_BF16, TA, TB)               \
    HK_PROGRAM_ENTRY(NAME, OUT_BF16, TA, TB, false)      \
    HK_PROGRAM_ENTRY(NAME##_wide, OUT_BF16, TA, TB, true)

HK_PROGRAM(ruda_rust_bf16_dense_nn_bf16, true, false, false)
HK_PROGRAM(ruda_rust_bf16_dense_nn_f32, false, false, false)
HK_PROGRAM(ruda_rust_bf16_dense_nt_bf16, true, false, true)
HK_PROGRAM(ruda_rust_bf16_dense_nt_f32, false, false, true)
HK_PROGRAM(ruda_rust_bf16_dense_tn_bf16, true, true, false)
HK_PROGRAM(ruda_rust_bf16_dense_tn_f32, false, true, false)
HK_PROGRAM(ruda_rust_bf16_dense_tt_bf16, true, true, true)
HK_PROGRAM(ruda_rust_bf16_dense_tt_f32, false, true, true)
HK_PROGRAM(ruda_rust_bf16_batched_nn_bf16, true, false, false)
HK_PROGRAM(ruda_rust_bf16_batched_nn_f32, false, false, false)
HK_PROGRAM(ruda_rust_bf16_batched_nt_bf16, true, false, true)
HK_PROGRAM(ruda_rust_bf16_batched_nt_f32, false, false, true)
HK_PROGRAM(ruda_rust_bf16_batched_tn_bf16, true, true, false)
HK_PROGRAM(ruda_rust_bf16_batched_tn_f32, false, true, false)
HK_PROGRAM(ruda_rust_bf16_batched_tt_bf16, true, true, true)
HK_PROGRAM(ruda_rust_bf16_batched_tt_f32, false, true, true)
HK_PROGRAM(ruda_rust_bf16_mgrouped_nt_bf16, true, false, true)
HK_PROGRAM(ruda_rust_bf16_mgrouped_nt_f32, false, false, true)
