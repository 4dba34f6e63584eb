/*
 * hk_oracle.c — CPU restatement of the reference's host-side computations for the
 * BF16 transformer kernel path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker or the timed CPU
 * baseline. The product path (libhk.so) never calls it.
 *
 * Each function cites the reference file:line it restates (paths relative to the
 * shuqi2077/rust-ascend repository root). Inputs that the reference keeps in BF16
 * are passed here already decoded to float (exact). The f64 functions follow the
 * reference's f64 expectation loops; the f32 "lanes" functions follow the device
 * programs' FP32 operation order. OpenMP parallelizes over independent rows/heads
 * only, so every output element is computed in a fixed sequential order whatever
 * the thread count.
 *
 * How each function is pinned (checked by tests/test_oracle.py) is listed in the
 * header comment of oracle/oracle.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ BF16 */

/* Round-to-nearest-even to BF16, Inf/NaN keep their sign and payload top bits.
 * Reference: rust-ascend-kernels/src/tests.rs:7-11 (and the RNE formula of
 * rust-ascend-driver/examples/deepgemm_validate.rs:5). */
static inline float bf16r(float x) {
    uint32_t b;
    memcpy(&b, &x, 4);
    if ((b & 0x7f800000u) == 0x7f800000u) {
        b &= 0xffff0000u;
    } else {
        b = (b + 0x7fffu + ((b >> 16) & 1u)) & 0xffff0000u;
    }
    float y;
    memcpy(&y, &b, 4);
    return y;
}

float or_bf16(float x) { return bf16r(x); }

void or_round_bf16(const float* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = bf16r(in[i]);
}

int or_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void or_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* ------------------------------------------------------------------ GEMM */

static inline int64_t a_index(int64_t i, int64_t p, int64_t m, int64_t k, int ta) {
    return ta ? p * m + i : i * k + p;
}
static inline int64_t b_index(int64_t p, int64_t j, int64_t n, int64_t k, int tb) {
    return tb ? j * k + p : p * n + j;
}

/* out[b,i,j] = sum_q A'[b,i,q] * B'[b,q,j] in f64, q ascending.
 * Reference: examples/matrix_runtime.rs:28-39 (address formula also
 * rust-ascend-kernels/src/tests.rs:97-100). */
void or_gemm_f64(const float* a, const float* b, int64_t batch, int64_t m, int64_t n, int64_t k,
                 int ta, int tb, double* out) {
    for (int64_t g = 0; g < batch; ++g) {
        const float* ag = a + g * m * k;
        const float* bg = b + g * k * n;
        double* og = out + g * m * n;
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < m; ++i) {
            for (int64_t j = 0; j < n; ++j) {
                double s = 0.0;
                for (int64_t q = 0; q < k; ++q)
                    s += (double)ag[a_index(i, q, m, k, ta)] * (double)bg[b_index(q, j, n, k, tb)];
                og[i * n + j] = s;
            }
        }
    }
}

/* M-grouped NT: out[i,j] = sum_q A[i,q] * W[g,j,q] in f64, q ascending, where g is the first
 * group whose end exceeds i (empty groups, whose end repeats the previous one, own no row).
 * A [m,k], W [groups,n,k]. Reference: rust-ascend-kernels/src/tests.rs:89-103 (group lookup
 * :95, weight address :99). */
void or_gemm_grouped_nt_f64(const float* a, const float* w, int64_t m, int64_t n, int64_t k,
                            const int32_t* ends, int64_t groups, double* out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < m; ++i) {
        int64_t g = 0;
        while (g < groups && i >= (int64_t)ends[g]) ++g;
        for (int64_t j = 0; j < n; ++j) {
            double s = 0.0;
            if (g < groups) {
                const float* wr = w + (g * n + j) * k;
                for (int64_t q = 0; q < k; ++q) s += (double)a[i * k + q] * (double)wr[q];
            }
            out[i * n + j] = g < groups ? s : NAN;
        }
    }
}

/* Same, evaluated only at the listed (row, col) pairs of batch 0 (sampled parity
 * for shapes too large to evaluate whole on the CPU). */
void or_gemm_f64_sampled(const float* a, const float* b, int64_t m, int64_t n, int64_t k,
                         int ta, int tb, const int64_t* rows, const int64_t* cols, int64_t count,
                         double* out) {
#pragma omp parallel for schedule(static)
    for (int64_t s = 0; s < count; ++s) {
        int64_t i = rows[s], j = cols[s];
        double acc = 0.0;
        for (int64_t q = 0; q < k; ++q)
            acc += (double)a[a_index(i, q, m, k, ta)] * (double)b[b_index(q, j, n, k, tb)];
        out[s] = acc;
    }
}

/* f32 products summed sequentially over k without fused multiply-add (built with
 * -ffp-contract=off). Reference: rust-ascend-driver/examples/deepgemm_validate.rs:19-21.
 * This is the CPU baseline's GEMM. */
void or_gemm_f32(const float* a, const float* b, int64_t batch, int64_t m, int64_t n, int64_t k,
                 int ta, int tb, float* out) {
    for (int64_t g = 0; g < batch; ++g) {
        const float* ag = a + g * m * k;
        const float* bg = b + g * k * n;
        float* og = out + g * m * n;
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < m; ++i) {
            for (int64_t j = 0; j < n; ++j) {
                float s = 0.0f;
                for (int64_t q = 0; q < k; ++q) {
                    float prod = ag[a_index(i, q, m, k, ta)] * bg[b_index(q, j, n, k, tb)];
                    s = s + prod;
                }
                og[i * n + j] = s;
            }
        }
    }
}

/* ------------------------------------------------------------------ RMSNorm */

/* y = x*r*w, r = 1/sqrt(sum(x^2)/W + eps) in f64.
 * Reference: examples/rms_norm_runtime.rs:55-65. */
void or_rms_norm_f64(const float* x, const float* w, int64_t rows, int64_t width, double eps,
                     double* y, double* rstd) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float* a = x + r * width;
        double ss = 0.0;
        for (int64_t c = 0; c < width; ++c) ss += (double)a[c] * (double)a[c];
        double rr = 1.0 / sqrt(ss / (double)width + eps);
        rstd[r] = rr;
        for (int64_t c = 0; c < width; ++c) y[r * width + c] = (double)a[c] * rr * (double)w[c];
    }
}

/* dx = r*(dy*w - x*r^2*mean(dy*w*x)), dw[c] = sum_rows dy*x*r, in f64, using the
 * given per-row r (the forward's saved rstd, as the backward does not recompute eps).
 * Reference: examples/rms_norm_runtime.rs:60-67 and normalization.rs:180. The dw sum
 * runs over rows in ascending order per column. */
void or_rms_norm_backward_f64(const float* x, const float* w, const float* dy, const double* rstd,
                              int64_t rows, int64_t width, double* dx, double* dw) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float* a = x + r * width;
        const float* g = dy + r * width;
        double rr = rstd[r];
        double mean_gx = 0.0;
        for (int64_t c = 0; c < width; ++c) mean_gx += (double)g[c] * (double)w[c] * (double)a[c];
        mean_gx /= (double)width;
        for (int64_t c = 0; c < width; ++c)
            dx[r * width + c] = rr * ((double)g[c] * (double)w[c] - (double)a[c] * rr * rr * mean_gx);
    }
#pragma omp parallel for schedule(static)
    for (int64_t c = 0; c < width; ++c) {
        double s = 0.0;
        for (int64_t r = 0; r < rows; ++r) s += (double)dy[r * width + c] * ((double)x[r * width + c] * rstd[r]);
        dw[c] = s;
    }
}

/* The device row program's FP32 order: lane l (0..31) accumulates sum_j v[l+32j] in
 * j order, then the 32 lane sums are added (Plane::Sum). Requires width % 32 == 0.
 * Reference: rust-ascend-compiler/src/ascend/row_programs.rs:67-85. The 32-lane
 * plane reduction is hardware-defined; this takes lanes in ascending order. */
static float plane_sum(const float* v, int64_t width) {
    float lane[32];
    for (int l = 0; l < 32; ++l) lane[l] = v[l];
    for (int64_t j = 1; j < width / 32; ++j)
        for (int l = 0; l < 32; ++l) lane[l] = lane[l] + v[l + 32 * j];
    float s = 0.0f;
    for (int l = 0; l < 32; ++l) s = s + lane[l];
    return s;
}

/* RMSNorm forward in the row program's FP32 order.
 * Reference: row_programs.rs:144-151 (square, Plane::Sum, /W, +eps, rsqrt, (x*r)*w). */
int or_rms_norm_lanes_f32(const float* x, const float* w, int64_t rows, int64_t width, float eps,
                          float* y, float* rstd) {
    if (width < 32 || width % 32 != 0) return -1;
    float* sq = (float*)malloc(sizeof(float) * (size_t)width * (size_t)or_num_threads());
    if (!sq) return -2;
#pragma omp parallel
    {
        int t = 0;
#ifdef _OPENMP
        t = omp_get_thread_num();
#endif
        float* s = sq + (size_t)t * (size_t)width;
#pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            const float* a = x + r * width;
            for (int64_t c = 0; c < width; ++c) s[c] = a[c] * a[c];
            float mean = plane_sum(s, width) / (float)width;
            float rr = 1.0f / sqrtf(mean + eps);
            rstd[r] = rr;
            for (int64_t c = 0; c < width; ++c) y[r * width + c] = (a[c] * rr) * w[c];
        }
    }
    free(sq);
    return 0;
}

/* Pairwise column sum over rows, preserving an odd trailing row at each level.
 * Reference: rust-ascend-driver/src/tensor/runtime/normalization.rs:95-114. Sums in
 * place over `parts` ([rows, width]) and writes the result to out[width]; rows == 0
 * gives zeros (normalization.rs:96). */
void or_column_sum_pairwise(float* parts, int64_t rows, int64_t width, float* out) {
    if (rows == 0) {
        for (int64_t c = 0; c < width; ++c) out[c] = 0.0f;
        return;
    }
    while (rows > 1) {
        int64_t pairs = rows / 2;
        int64_t next = (rows + 1) / 2;
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < pairs * width; ++i) parts[i] = parts[i] + parts[pairs * width + i];
        if (rows % 2) memmove(parts + pairs * width, parts + (rows - 1) * width, sizeof(float) * (size_t)width);
        rows = next;
    }
    memcpy(out, parts, sizeof(float) * (size_t)width);
}

/* RMSNorm backward in the row programs' FP32 order, dw via the pairwise tree.
 * Reference: row_programs.rs:200-207 (contributions (x*r)*dy), :208-217 (g = dy*w,
 * Plane::Sum(g*x)/W, r*r, mean*rr, dx = (g - x*corr)*r) and normalization.rs:180-185. */
int or_rms_norm_backward_lanes_f32(const float* x, const float* w, const float* dy, const float* rstd,
                                   int64_t rows, int64_t width, float* dx, float* dw) {
    if (width < 32 || width % 32 != 0) return -1;
    float* parts = (float*)malloc(sizeof(float) * (size_t)(rows > 0 ? rows : 1) * (size_t)width);
    float* tmp = (float*)malloc(sizeof(float) * (size_t)width * (size_t)or_num_threads());
    if (!parts || !tmp) { free(parts); free(tmp); return -2; }
#pragma omp parallel
    {
        int t = 0;
#ifdef _OPENMP
        t = omp_get_thread_num();
#endif
        float* gx = tmp + (size_t)t * (size_t)width;
#pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            const float* a = x + r * width;
            const float* d = dy + r * width;
            float rr = rstd[r];
            for (int64_t c = 0; c < width; ++c) gx[c] = (d[c] * w[c]) * a[c];
            float mean = plane_sum(gx, width) / (float)width;
            float corr = mean * (rr * rr);
            for (int64_t c = 0; c < width; ++c) {
                float g = d[c] * w[c];
                dx[r * width + c] = (g - a[c] * corr) * rr;
                parts[r * width + c] = (a[c] * rr) * d[c];
            }
        }
    }
    or_column_sum_pairwise(parts, rows, width, dw);
    free(parts);
    free(tmp);
    return 0;
}

/* ------------------------------------------------------------------ RoPE */

/* Pair (a, b) of column `col` and its side: Interleaved pairs (2p, 2p+1), SplitHalf
 * pairs (p, p+P/2). Reference: rotary_programs.rs:62-77. */
static inline void rope_pair(int64_t col, int64_t p, int layout, int64_t* paired, int64_t* pair, int* side) {
    int64_t half = p / 2;
    if (layout == 0) {
        *pair = col / 2;
        *paired = (col / 2) * 2 + (col + 1) % 2;
        *side = (int)(col % 2);
    } else {
        *paired = (col + half) % p;
        *pair = col % half;
        *side = (int)(col / half);
    }
}

/* Full last-axis rotation with same-row tables, FP32 device order:
 * out = x*cos + sign*paired*sin (forward), x*cos - sign*paired*sin (backward), with
 * sign = 2*side - 1. Reference: rotary_programs.rs:47-97. */
void or_rotary(const float* x, const float* cos_t, const float* sin_t, int64_t rows, int64_t width,
               int layout, int backward, float* y) {
    int64_t half = width / 2;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t col = 0; col < width; ++col) {
            int64_t paired, pair;
            int side;
            rope_pair(col, width, layout, &paired, &pair, &side);
            float sign = (float)side * 2.0f - 1.0f;
            float c = cos_t[r * half + pair], s = sin_t[r * half + pair];
            float direct = x[r * width + col] * c;
            float rot = (x[r * width + paired] * s) * sign;
            y[r * width + col] = backward ? direct - rot : direct + rot;
        }
    }
}

/* The same in f64, pair-wise as the example's expectation is written:
 * y_a = x_a c - x_b s, y_b = x_b c + x_a s; dx_a = dy_a c + dy_b s, dx_b = dy_b c - dy_a s.
 * Reference: examples/rotary_tensor.rs:36-43. */
void or_rotary_f64(const float* x, const float* cos_t, const float* sin_t, int64_t rows, int64_t width,
                   int layout, int backward, double* y) {
    int64_t half = width / 2;
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t p = 0; p < half; ++p) {
            int64_t a = layout == 0 ? r * width + 2 * p : r * width + p;
            int64_t b = layout == 0 ? r * width + 2 * p + 1 : r * width + half + p;
            double c = cos_t[r * half + p], s = sin_t[r * half + p];
            if (!backward) {
                y[a] = (double)x[a] * c - (double)x[b] * s;
                y[b] = (double)x[b] * c + (double)x[a] * s;
            } else {
                y[a] = (double)x[a] * c + (double)x[b] * s;
                y[b] = (double)x[b] * c - (double)x[a] * s;
            }
        }
    }
}

/* Prefix rotation: the first p columns rotate with tables whose leading axes are 1
 * (broadcast) or equal to the input's and whose last axis is p/2; columns >= p are
 * copied bit-exactly. Reference: rotary_programs.rs:7-23 (validation), :101-156. */
int or_rotary_prefix(const float* x, const int64_t* in_shape, const int64_t* table_shape, int rank,
                     int64_t p, int layout, int backward, const float* cos_t, const float* sin_t,
                     float* y) {
    if (rank < 1 || rank > 8) return -1;
    int64_t width = in_shape[rank - 1];
    if (p <= 0 || p % 2 || p > width || table_shape[rank - 1] != p / 2) return -1;
    for (int a = 0; a < rank - 1; ++a)
        if (table_shape[a] != 1 && table_shape[a] != in_shape[a]) return -1;
    int64_t rows = 1;
    for (int a = 0; a < rank - 1; ++a) rows *= in_shape[a];
    int64_t half = p / 2;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        /* table row: coordinates of r over the leading axes, singleton table axes -> 0 */
        int64_t rem = r, trow = 0, tstride = 1;
        for (int a = rank - 2; a >= 0; --a) {
            int64_t coord = rem % in_shape[a];
            rem /= in_shape[a];
            if (table_shape[a] != 1) trow += coord * tstride;
            tstride *= table_shape[a];
        }
        for (int64_t col = 0; col < width; ++col) {
            if (col >= p) {
                memcpy(&y[r * width + col], &x[r * width + col], 4);
                continue;
            }
            int64_t paired, pair;
            int side;
            rope_pair(col, p, layout, &paired, &pair, &side);
            float sign = (float)side * 2.0f - 1.0f;
            float c = cos_t[trow * half + pair], s = sin_t[trow * half + pair];
            float direct = x[r * width + col] * c;
            float rot = (x[r * width + paired] * s) * sign;
            y[r * width + col] = backward ? direct - rot : direct + rot;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------ attention */

/* Grouped-query attention forward and backward in f64 with the reference's BF16
 * rounding points: Q, K, V and dY rounded to BF16 for every product; P rounded to
 * BF16 for P.V and P^T.dY; dS scaled then rounded to BF16 for dQ and dK.
 * Reference: examples/grouped_attention_tensor.rs:14-44 (loop structure and rounding),
 * src/nn/attention.rs:25-28,62-66 (QK^T*scale + mask, softmax, P.V; head h reads KV
 * head h/group), mask_programs.rs:5-40 (causal mask: key_start+j > query_start+i is
 * excluded). `mask` (optional, [B,Hq,M,N] additive) is used when causal == 0.
 * Rows whose keys are all excluded produce zeros and lse = -inf (the composed
 * reference produces NaN there; see the attention kernel's documentation).
 * V, dY and the output have the value width dw (d == dw in the fused kernels' domain;
 * src/nn/attention.rs:49-52 allows any). dmask (optional, [B,Hq,M,N]) receives the mask
 * gradient dS = P (dP - rowsum(P dP)), the scores' gradient before the scale.
 * Any of out/lse/dq/dk/dv/mag/dmask may be NULL; dq/dk/dv/dmask require dy. Outputs are
 * overwritten. */
void or_attention_f64(const float* q, const float* k, const float* v, const float* dy,
                      const float* mask, int64_t batch, int64_t heads, int64_t kv_heads,
                      int64_t m, int64_t n, int64_t d, int64_t dw, double scale, int causal,
                      uint64_t query_start, uint64_t key_start, double* out, double* lse,
                      double* dq, double* dk, double* dv, double* mag, double* dmask) {
    int64_t group = heads / kv_heads;
    if (out) memset(out, 0, sizeof(double) * (size_t)(batch * heads * m * dw));
    if (dq) memset(dq, 0, sizeof(double) * (size_t)(batch * heads * m * d));
    if (dk) memset(dk, 0, sizeof(double) * (size_t)(batch * kv_heads * n * d));
    if (dv) memset(dv, 0, sizeof(double) * (size_t)(batch * kv_heads * n * dw));
    if (dmask) memset(dmask, 0, sizeof(double) * (size_t)(batch * heads * m * n));
    /* mag (optional): the same sums over the absolute values of their terms, laid out as
     * [out | dq | dk | dv]; sum |terms| bounds the effect of rounding any term. */
    double* out_m = mag;
    double* dq_m = mag ? mag + batch * heads * m * dw : NULL;
    double* dk_m = mag ? dq_m + batch * heads * m * d : NULL;
    double* dv_m = mag ? dk_m + batch * kv_heads * n * d : NULL;
    if (mag)
        memset(mag, 0, sizeof(double) * (size_t)(batch * heads * m * (d + dw) + batch * kv_heads * n * (d + dw)));
    /* Parallel over (batch, kv head): the group's query heads run sequentially inside,
     * so dk/dv accumulate in a fixed order without races. */
#pragma omp parallel for schedule(dynamic) collapse(2)
    for (int64_t b = 0; b < batch; ++b) {
        for (int64_t kv = 0; kv < kv_heads; ++kv) {
            double* s = (double*)malloc(sizeof(double) * (size_t)n);
            double* p = (double*)malloc(sizeof(double) * (size_t)n);
            double* dp = (double*)malloc(sizeof(double) * (size_t)n);
            for (int64_t h = kv * group; h < (kv + 1) * group; ++h) {
                const float* qh = q + ((b * heads + h) * m) * d;
                const float* kh = k + ((b * kv_heads + kv) * n) * d;
                const float* vh = v + ((b * kv_heads + kv) * n) * dw;
                for (int64_t row = 0; row < m; ++row) {
                    double mx = -INFINITY;
                    for (int64_t j = 0; j < n; ++j) {
                        int excluded = causal && (key_start + (uint64_t)j > query_start + (uint64_t)row);
                        if (excluded) { s[j] = -INFINITY; continue; }
                        double acc = 0.0;
                        for (int64_t c = 0; c < d; ++c)
                            acc += (double)bf16r(qh[row * d + c]) * (double)bf16r(kh[j * d + c]);
                        s[j] = scale * acc;
                        if (!causal && mask) s[j] += (double)mask[((b * heads + h) * m + row) * n + j];
                        if (s[j] > mx) mx = s[j];
                    }
                    int64_t oi = ((b * heads + h) * m + row);
                    if (mx == -INFINITY) {
                        if (lse) lse[oi] = -INFINITY;
                        continue; /* zero output and zero gradients for this row */
                    }
                    double total = 0.0;
                    for (int64_t j = 0; j < n; ++j) { p[j] = exp(s[j] - mx); total += p[j]; }
                    for (int64_t j = 0; j < n; ++j) p[j] /= total;
                    if (lse) lse[oi] = mx + log(total);
                    if (out) {
                        for (int64_t j = 0; j < n; ++j) {
                            double pb = (double)bf16r((float)p[j]);
                            if (pb == 0.0) continue;
                            for (int64_t c = 0; c < dw; ++c) out[oi * dw + c] += pb * (double)bf16r(vh[j * dw + c]);
                            if (out_m)
                                for (int64_t c = 0; c < dw; ++c) out_m[oi * dw + c] += fabs(pb * (double)bf16r(vh[j * dw + c]));
                        }
                    }
                    if (!dy) continue;
                    const float* g = dy + oi * dw;
                    double dot = 0.0, dot_mag = 0.0, dot_mag_o = 0.0;
                    for (int64_t j = 0; j < n; ++j) {
                        double acc = 0.0;
                        for (int64_t c = 0; c < dw; ++c) acc += (double)bf16r(g[c]) * (double)bf16r(vh[j * dw + c]);
                        dp[j] = acc;
                        dot += p[j] * acc;
                        dot_mag += p[j] * fabs(acc);
                    }
                    if (mag && out) {
                        for (int64_t c = 0; c < dw; ++c) dot_mag_o += fabs((double)bf16r(g[c]) * out[oi * dw + c]);
                        if (dot_mag_o > dot_mag) dot_mag = dot_mag_o;
                    }
                    for (int64_t j = 0; j < n; ++j) {
                        double ds = p[j] * (dp[j] - dot);
                        double pb = (double)bf16r((float)p[j]);
                        double dsb = (double)bf16r((float)(scale * ds));
                        if (dmask) dmask[oi * n + j] = ds;
                        if (dv) {
                            double* dvh = dv + ((b * kv_heads + kv) * n + j) * dw;
                            for (int64_t c = 0; c < dw; ++c) dvh[c] += pb * (double)bf16r(g[c]);
                        }
                        if (dq) {
                            for (int64_t c = 0; c < d; ++c) dq[oi * d + c] += dsb * (double)bf16r(kh[j * d + c]);
                        }
                        if (dk) {
                            double* dkh = dk + ((b * kv_heads + kv) * n + j) * d;
                            for (int64_t c = 0; c < d; ++c) dkh[c] += dsb * (double)bf16r(qh[row * d + c]);
                        }
                        if (mag) {
                            /* |dS| term magnitude: p*(|dp| + |row term|), where the row term's own
                             * magnitude is the larger of sum_j p_j |dp_j| (its form here) and
                             * sum_d |dY_d O_d| (the form rowsum(dY o O) a fused kernel uses). */
                            double dsm = scale * p[j] * (fabs(dp[j]) + dot_mag);
                            double* dvm = dv_m + ((b * kv_heads + kv) * n + j) * dw;
                            double* dkm = dk_m + ((b * kv_heads + kv) * n + j) * d;
                            for (int64_t c = 0; c < dw; ++c) dvm[c] += fabs(pb * (double)bf16r(g[c]));
                            for (int64_t c = 0; c < d; ++c) {
                                dq_m[oi * d + c] += dsm * fabs((double)bf16r(kh[j * d + c]));
                                dkm[c] += dsm * fabs((double)bf16r(qh[row * d + c]));
                            }
                        }
                    }
                }
            }
            free(s);
            free(p);
            free(dp);
        }
    }
}

/* Causal additive mask [batch, queries, keys]: -inf where key_start+key >
 * query_start+query, else +0. Reference: mask_programs.rs:5-40. */
void or_causal_mask(int64_t batch, int64_t queries, int64_t keys, uint64_t query_start,
                    uint64_t key_start, float* out) {
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t i = 0; i < queries; ++i)
            for (int64_t j = 0; j < keys; ++j)
                out[(b * queries + i) * keys + j] =
                    (key_start + (uint64_t)j > query_start + (uint64_t)i) ? -INFINITY : 0.0f;
}

/* Row softmax / log-softmax in double over [rows, width] F32 input.
 * Reference: the host check of rust-ascend-driver/examples/common_rows_validate.rs:55-58
 * (m = max, exp(x - m), sum; y = e / sum or x - m - ln(sum)), i.e. the arithmetic of
 * row_programs.rs:135-143. */
void or_softmax_f64(const float* x, int64_t rows, int64_t width, int logarithmic, double* out) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float* a = x + r * width;
        double* o = out + r * width;
        double m = -INFINITY;
        for (int64_t j = 0; j < width; ++j) m = a[j] > m ? (double)a[j] : m;
        double sum = 0.0;
        for (int64_t j = 0; j < width; ++j) sum += exp((double)a[j] - m);
        for (int64_t j = 0; j < width; ++j)
            o[j] = logarithmic ? ((double)a[j] - m) - log(sum) : exp((double)a[j] - m) / sum;
    }
}

/* Backward from the saved output y. Reference: common_rows_validate.rs:82-85
 * (row_programs.rs:152-163): softmax dx = y (dy - sum(y dy)); log-softmax
 * dx = dy - exp(y) sum(dy). */
void or_softmax_backward_f64(const float* y, const float* dy, int64_t rows, int64_t width, int logarithmic,
                             double* out) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float* a = y + r * width;
        const float* g = dy + r * width;
        double* o = out + r * width;
        double dot = 0.0;
        for (int64_t j = 0; j < width; ++j) dot += logarithmic ? (double)g[j] : (double)a[j] * (double)g[j];
        for (int64_t j = 0; j < width; ++j)
            o[j] = logarithmic ? (double)g[j] - exp((double)a[j]) * dot : (double)a[j] * ((double)g[j] - dot);
    }
}

/* KV-head repetition backward in F32, in the reference's level order: each level adds the
 * neighbouring groups (2i, 2i+1) of every row and carries an odd last group through, until one
 * group is left. dy is [rows, groups, width] (rows = B*Hkv, groups = Hq/Hkv, width = N*D).
 * Reference: rust-ascend-driver/src/tensor/runtime/heads.rs:29-51 with the pair/tail
 * programs of heads_programs.rs:56-86. */
void or_repeat_kv_backward(const float* dy, int64_t rows, int64_t groups, int64_t width, float* out) {
    float* value = (float*)malloc((size_t)(rows * groups * width) * sizeof(float));
    memcpy(value, dy, (size_t)(rows * groups * width) * sizeof(float));
    while (groups > 1) {
        const int64_t next_groups = (groups + 1) / 2;
        float* next = (float*)malloc((size_t)(rows * next_groups * width) * sizeof(float));
        for (int64_t r = 0; r < rows; ++r)
            for (int64_t g = 0; g < next_groups; ++g)
                for (int64_t c = 0; c < width; ++c) {
                    const float* src = value + (r * groups + 2 * g) * width + c;
                    next[(r * next_groups + g) * width + c] = 2 * g + 1 < groups ? src[0] + src[width] : src[0];
                }
        free(value);
        value = next;
        groups = next_groups;
    }
    memcpy(out, value, (size_t)(rows * width) * sizeof(float));
    free(value);
}
