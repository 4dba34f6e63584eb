// hk_loss.hip — NLLLoss forward and backward over log-probabilities for gfx950.
//
// Semantics (reference: CannSession::nll_loss / nll_loss_backward, rust-ascend-driver/src/tensor/
// loss.rs:31-70, over the closed aclnnNLLLoss / aclnnNLLLossBackward; the expectations of
// examples/cross_entropy_tensor.rs:38-52): input [N, C] log-probabilities, target [N] class
// labels, weight [C]. A row whose label equals ignore_index (-1 when the caller sets none,
// NllLossOptions::ignore, loss.rs:10-12) contributes nothing.
//   row loss  l_n = -weight[t_n] * input[n, t_n]         (0 for an ignored row)
//   None -> out[n] = l_n;  Sum -> out[0] = sum_n l_n;  Mean -> out[0] = sum_n l_n / W
//   total_weight[0] = W = sum over non-ignored rows of weight[t_n] (for Sum and Mean)
//   backward: dinput[n, c] = -weight[t_n] * g_n * [c == t_n], g_n = grad[n] (None), grad[0]
//   (Sum) or grad[0] / W (Mean).
// Arithmetic is F32 per element; the forward's sums over rows are kept in double and reduced in
// a fixed order (deterministic). A label outside [0, C) that is not ignore_index raises a flag the
// host checks (the row then contributes nothing).
//
// Layout: the forward computes every row's term in parallel into a workspace, then one workgroup
// sums the terms in a fixed order (N is a token count; the loss is tiny next to the logits it
// follows); the backward writes the dense [N, C] gradient, one element per
// thread, coalesced along C (HBM-bound: sizeof(T) bytes written per element).
#include "hk_common.hpp"
#include "hk_kernels.hpp"

namespace hk {

namespace {

constexpr int kNllThreads = 1024;
constexpr int kNllBwdThreads = 256;

// Per-row terms, one row per thread over every CU: v_n = -weight[t_n] input[n, t_n] and the
// row's counted weight (0 for an ignored or out-of-range label), both exact in F32; out[n] = v_n
// for reduction None. The gathers of input[n, t_n] land on a different 128 KB row each (C = 32000
// F32): spread over the chip they cost ~5 us at 8192 rows, against ~34 us walked by one workgroup.
template <typename T, typename I>
__global__ void __launch_bounds__(kNllBwdThreads)
nll_rows_kernel(const T* __restrict__ input, const I* __restrict__ target, const T* __restrict__ weight,
                T* __restrict__ out, float* __restrict__ row_v, float* __restrict__ row_w, int64_t rows,
                int64_t classes, int reduction, int64_t ignore) {
    for (int64_t r = flat_begin(kNllBwdThreads); r < rows; r += flat_stride(kNllBwdThreads)) {
        const int64_t t = static_cast<int64_t>(target[r]);
        float v = 0.0f, wc = 0.0f;
        if (t != ignore && t >= 0 && t < classes) {
            const float wt = Elem<T>::load(weight, t);
            v = -(wt * Elem<T>::load(input, r * classes + t));
            wc = wt;
        }
        if (reduction == 0) Elem<T>::store(out, r, v);
        row_v[r] = v;
        row_w[r] = wc;
    }
}

// The sums over rows, by one workgroup in a fixed order: thread x adds rows x, x + 1024, ... in
// double, then the 1024 partial sums are combined by pairwise halving. The label check (a label
// outside [0, C) that is not ignore_index) raises the flag the host reads.
template <typename I>
__global__ void __launch_bounds__(kNllThreads)
nll_reduce_kernel(const I* __restrict__ target, const float* __restrict__ row_v, const float* __restrict__ row_w,
                  void* __restrict__ out, void* __restrict__ total, int out_dtype, int64_t rows, int64_t classes,
                  int reduction, int64_t ignore, int* __restrict__ bad) {
    __shared__ double sl[kNllThreads], sw[kNllThreads];
    __shared__ int any_bad;
    if (threadIdx.x == 0) any_bad = 0;
    __syncthreads();
    double l = 0.0, w = 0.0;
    for (int64_t r = threadIdx.x; r < rows; r += kNllThreads) {
        const int64_t t = static_cast<int64_t>(target[r]);
        if (t != ignore && (t < 0 || t >= classes)) any_bad = 1;
        l += static_cast<double>(row_v[r]);
        w += static_cast<double>(row_w[r]);
    }
    sl[threadIdx.x] = l;
    sw[threadIdx.x] = w;
    __syncthreads();
    for (int half = kNllThreads / 2; half > 0; half >>= 1) {  // pairwise halving, fixed order
        if (static_cast<int>(threadIdx.x) < half) {
            sl[threadIdx.x] += sl[threadIdx.x + half];
            sw[threadIdx.x] += sw[threadIdx.x + half];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const double W = sw[0];
        const float value = reduction == 2 ? static_cast<float>(sl[0]) : static_cast<float>(sl[0] / W);
        const float tw = reduction == 0 ? 0.0f : static_cast<float>(W);
        if (out_dtype == 0) {
            if (reduction != 0) static_cast<float*>(out)[0] = value;
            static_cast<float*>(total)[0] = tw;
        } else if (out_dtype == 1) {
            if (reduction != 0) static_cast<_Float16*>(out)[0] = static_cast<_Float16>(value);
            static_cast<_Float16*>(total)[0] = static_cast<_Float16>(tw);
        } else {
            if (reduction != 0) static_cast<uint16_t*>(out)[0] = f32_to_bf16(value);
            static_cast<uint16_t*>(total)[0] = f32_to_bf16(tw);
        }
        *bad = any_bad;
    }
}

template <typename T, typename I>
__global__ void __launch_bounds__(kNllBwdThreads)
nll_backward_kernel(const T* __restrict__ grad, const I* __restrict__ target, const T* __restrict__ weight,
                    const T* __restrict__ total, T* __restrict__ dinput, int64_t rows, int64_t classes,
                    int reduction, int64_t ignore) {
    const int64_t count = rows * classes;
    for (int64_t i = flat_begin(kNllBwdThreads); i < count; i += flat_stride(kNllBwdThreads)) {
        const int64_t r = i / classes, c = i - r * classes;
        const int64_t t = static_cast<int64_t>(target[r]);
        float v = 0.0f;
        if (c == t && t != ignore) {
            float g = Elem<T>::load(grad, reduction == 0 ? r : 0);
            if (reduction == 1) g = g / Elem<T>::load(total, 0);
            v = -(Elem<T>::load(weight, t) * g);
        }
        Elem<T>::store(dinput, i, v);
    }
}

// workspace: the flag (first 256 bytes), then the per-row terms row_v[rows] and row_w[rows] (F32)
template <typename T, typename I>
hipError_t nll_forward_t(int dtype, const void* input, const void* target, const void* weight, void* out,
                         void* total, int64_t rows, int64_t classes, int reduction, int64_t ignore, void* ws,
                         hipStream_t s) {
    int* bad = static_cast<int*>(ws);
    float* row_v = reinterpret_cast<float*>(static_cast<char*>(ws) + 256);
    float* row_w = row_v + rows;
    if (rows > 0)
        hipLaunchKernelGGL((nll_rows_kernel<T, I>), dim3(flat_blocks(rows, kNllBwdThreads)), dim3(kNllBwdThreads), 0, s,
                           static_cast<const T*>(input), static_cast<const I*>(target), static_cast<const T*>(weight),
                           static_cast<T*>(out), row_v, row_w, rows, classes, reduction, ignore);
    hipLaunchKernelGGL((nll_reduce_kernel<I>), dim3(1), dim3(kNllThreads), 0, s, static_cast<const I*>(target), row_v,
                       row_w, out, total, dtype, rows, classes, reduction, ignore, bad);
    return hipGetLastError();
}

template <typename T, typename I>
hipError_t nll_backward_t(const void* grad, const void* target, const void* weight, const void* total, void* dinput,
                          int64_t rows, int64_t classes, int reduction, int64_t ignore, hipStream_t s) {
    const int64_t n = rows * classes;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL((nll_backward_kernel<T, I>), dim3(flat_blocks(n, kNllBwdThreads)),
                       dim3(kNllBwdThreads), 0, s, static_cast<const T*>(grad), static_cast<const I*>(target),
                       static_cast<const T*>(weight), static_cast<const T*>(total), static_cast<T*>(dinput), rows,
                       classes, reduction, ignore);
    return hipGetLastError();
}

}  // namespace

// dtype: 0 F32, 1 F16, 2 BF16; id_bytes: 4 or 8.
size_t nll_loss_workspace_bytes(int64_t rows) { return 256 + static_cast<size_t>(rows) * 2 * sizeof(float); }

hipError_t nll_loss(int dtype, int id_bytes, const void* input, const void* target, const void* weight, void* out,
                    void* total, int64_t rows, int64_t classes, int reduction, int64_t ignore, void* ws, hipStream_t s) {
    const bool i64 = id_bytes == 8;
    if (dtype == 0)
        return i64 ? nll_forward_t<float, int64_t>(dtype, input, target, weight, out, total, rows, classes, reduction, ignore, ws, s)
                   : nll_forward_t<float, int32_t>(dtype, input, target, weight, out, total, rows, classes, reduction, ignore, ws, s);
    if (dtype == 1)
        return i64 ? nll_forward_t<_Float16, int64_t>(dtype, input, target, weight, out, total, rows, classes, reduction, ignore, ws, s)
                   : nll_forward_t<_Float16, int32_t>(dtype, input, target, weight, out, total, rows, classes, reduction, ignore, ws, s);
    return i64 ? nll_forward_t<uint16_t, int64_t>(dtype, input, target, weight, out, total, rows, classes, reduction, ignore, ws, s)
               : nll_forward_t<uint16_t, int32_t>(dtype, input, target, weight, out, total, rows, classes, reduction, ignore, ws, s);
}

hipError_t nll_loss_backward(int dtype, int id_bytes, const void* grad, const void* target, const void* weight,
                             const void* total, void* dinput, int64_t rows, int64_t classes, int reduction,
                             int64_t ignore, hipStream_t s) {
    const bool i64 = id_bytes == 8;
    if (dtype == 0)
        return i64 ? nll_backward_t<float, int64_t>(grad, target, weight, total, dinput, rows, classes, reduction, ignore, s)
                   : nll_backward_t<float, int32_t>(grad, target, weight, total, dinput, rows, classes, reduction, ignore, s);
    if (dtype == 1)
        return i64 ? nll_backward_t<_Float16, int64_t>(grad, target, weight, total, dinput, rows, classes, reduction, ignore, s)
                   : nll_backward_t<_Float16, int32_t>(grad, target, weight, total, dinput, rows, classes, reduction, ignore, s);
    return i64 ? nll_backward_t<uint16_t, int64_t>(grad, target, weight, total, dinput, rows, classes, reduction, ignore, s)
               : nll_backward_t<uint16_t, int32_t>(grad, target, weight, total, dinput, rows, classes, reduction, ignore, s);
}

}  // namespace hk
