// hk_heads.hip — the composed-attention compatibility kernels: causal mask, grouped-query KV
// head repetition and its backward, for gfx950.
//
// The fused attention kernels need none of these (they apply the mask and the KV-head mapping
// in place); they exist for callers of the reference's composed attention.
//
// Semantics:
//   causal mask   out[b,q,k] = -inf if key_start + k > query_start + q, else +0
//                 (reference rust-ascend-compiler/src/ascend/mask_programs.rs:5-40)
//   repeat        Y[b,h,n,d] = X[b, h / (Hq/Hkv), n, d]   (heads_programs.rs:42-55)
//   backward      dX[b,j] = sum over the group's Hq/Hkv replicas of dY, added as the reference's
//                 pairwise tree: each level adds neighbouring groups (2i, 2i+1) and carries an
//                 odd last group through, until one group is left (runtime/heads.rs:29-51,
//                 heads_programs.rs:56-86), so the sums round exactly as the reference's do.
// All F32, contiguous. HBM-bound element-wise kernels.
#include "hk_common.hpp"
#include "hk_kernels.hpp"

namespace hk {

namespace {

constexpr int kThreads = 256;

__global__ void __launch_bounds__(kThreads)
causal_mask_kernel(float* __restrict__ out, int64_t total, int64_t queries, int64_t keys, uint64_t query_start,
                   uint64_t key_start) {
    for (int64_t i = flat_begin(kThreads); i < total; i += flat_stride(kThreads)) {
        const int64_t k = i % keys, q = (i / keys) % queries;
        out[i] = key_start + static_cast<uint64_t>(k) > query_start + static_cast<uint64_t>(q) ? -INFINITY : 0.0f;
    }
}

// Y[(b, h), c] = X[(b, h / group), c] over the columns c of one (n, d) plane; with Hq = Hkv * group the
// flattened head index (b * Hq + h) / group is b * Hkv + h / group.
__global__ void __launch_bounds__(kThreads)
repeat_kv_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t total, int64_t plane, int64_t group) {
    for (int64_t i = flat_begin(kThreads); i < total; i += flat_stride(kThreads)) {
        const int64_t head = i / plane;  // flattened (b, h)
        y[i] = x[(head / group) * plane + i % plane];
    }
}

// One tree level over [rows, groups, width]: next[r, i] = value[r, 2i] + value[r, 2i+1]
// (i < groups/2); an odd last group is carried through.
__global__ void __launch_bounds__(kThreads)
pair_level_kernel(const float* __restrict__ value, float* __restrict__ next, int64_t rows, int64_t groups,
                  int64_t width) {
    const int64_t next_groups = (groups + 1) / 2;
    const int64_t total = rows * next_groups * width;
    for (int64_t i = flat_begin(kThreads); i < total; i += flat_stride(kThreads)) {
        const int64_t c = i % width, g = (i / width) % next_groups, r = i / (width * next_groups);
        const float* src = value + (r * groups + 2 * g) * width + c;
        next[i] = 2 * g + 1 < groups ? src[0] + src[width] : src[0];
    }
}

unsigned blocks(int64_t n) { return flat_blocks(n, kThreads); }

}  // namespace

hipError_t causal_mask(float* out, int64_t batch, int64_t queries, int64_t keys, uint64_t query_start,
                       uint64_t key_start, hipStream_t s) {
    const int64_t total = batch * queries * keys;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(causal_mask_kernel, dim3(blocks(total)), dim3(kThreads), 0, s, out, total, queries, keys,
                       query_start, key_start);
    return hipGetLastError();
}

hipError_t repeat_kv_heads(const float* x, float* y, int64_t batch, int64_t kv_heads, int64_t query_heads,
                           int64_t plane, hipStream_t s) {
    const int64_t total = batch * query_heads * plane;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(repeat_kv_kernel, dim3(blocks(total)), dim3(kThreads), 0, s, x, y, total, plane,
                       query_heads / kv_heads);
    return hipGetLastError();
}

size_t repeat_kv_backward_workspace_bytes(int64_t batch, int64_t kv_heads, int64_t query_heads, int64_t plane) {
    const int64_t group = query_heads / kv_heads;
    if (group <= 2) return 0;  // a single level writes dX directly
    // two ping-pong buffers, each the size of the first level's output
    return 2 * static_cast<size_t>(batch * kv_heads * ((group + 1) / 2) * plane) * sizeof(float);
}

hipError_t repeat_kv_heads_backward(const float* dy, float* dx, int64_t batch, int64_t kv_heads,
                                    int64_t query_heads, int64_t plane, void* workspace, hipStream_t s) {
    const int64_t rows = batch * kv_heads;
    int64_t groups = query_heads / kv_heads;
    if (rows * plane == 0) return hipSuccess;
    if (groups == 1) return hipMemcpyAsync(dx, dy, static_cast<size_t>(rows * plane) * sizeof(float),
                                           hipMemcpyDeviceToDevice, s);
    float* buf[2] = {static_cast<float*>(workspace), nullptr};
    if (workspace) buf[1] = buf[0] + rows * ((groups + 1) / 2) * plane;
    const float* value = dy;
    int level = 0;
    while (groups > 1) {
        const int64_t next_groups = (groups + 1) / 2;
        float* next = next_groups == 1 ? dx : buf[level & 1];
        hipLaunchKernelGGL(pair_level_kernel, dim3(blocks(rows * next_groups * plane)), dim3(kThreads), 0, s, value,
                           next, rows, groups, plane);
        value = next;
        groups = next_groups;
        ++level;
    }
    return hipGetLastError();
}

}  // namespace hk
