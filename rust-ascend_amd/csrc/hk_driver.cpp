// hk_driver.cpp — the C ABI of libhk.so (declared in include/hk.h).
//
// Replaces the reference's AscendCL loader and launch layers
// (rust-ascend-driver/src/{api,sys,lib}.rs, tensor/deepgemm/mod.rs, tensor/common_ir/mod.rs,
// tensor/runtime/{mod,worker,matrix,normalization,rotary}.rs) with a HIP runtime driver:
//   * one process-wide context (initialize_exclusive, runtime/mod.rs:424-435),
//   * every shape/dtype/domain check before any device work (plan.rs:49-80,
//     normalization.rs:12-48, rotary_programs.rs:7-23, attention.rs:81-104),
//   * output/input overlap rejection (deepgemm/mod.rs:99-100,117-119),
//   * launch, then stream synchronization unless async mode is on (deepgemm/mod.rs:134-145),
//   * a sticky poison flag after a failed launch or synchronization (deepgemm/mod.rs:39,143),
//   * launch/sync counters (deepgemm/mod.rs:15-16,142).
// The gfx950 code object is linked into this library as a fat binary and registered by
// the HIP runtime when the library loads; there is no JIT build step and no CPU fallback.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/hk.h"
#include "hk_kernels.hpp"

namespace {

thread_local std::string g_last_error;

hk_status fail(hk_status st, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return st;
}

struct GroupEndsDev;
struct ModuleDev;

struct Ctx {
    int device = 0;
    int num_cus = 256;
    hipStream_t stream = nullptr;
    bool async = false;
    bool poisoned = false;
    std::mutex mu;
    hk_stats stats{};
    void* workspace = nullptr;
    size_t ws_bytes = 0;
    void* scratch = nullptr;  // device address of `scratch` below on this context's device
    int* flags = nullptr;     // device address of `check_flags` below
    uint32_t flag_seq = 0;    // sequence number of the last embedding lookup
    std::vector<GroupEndsDev*> group_tables;  // live uploads, for the device programs' checks
    std::vector<ModuleDev*> modules;          // loaded device-program code objects
};

// Device memory of the allocation-free entry point (hk_rms_norm_backward_noalloc): its dgamma
// partials live in this fixed array instead of the context workspace, so the call makes no
// allocation. The array exists once per GPU for the life of the process. In host code its name
// is only a stand-in for the symbol, not a device address: hk_init resolves the address with
// hipGetSymbolAddress on the context's device, and every host-side use goes through Ctx::scratch.
constexpr size_t kScratchBytes = size_t(8) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// The embedding lookup's index check: a lookup that meets an index outside the table writes its
// own sequence number into check_flags[0], so no launch has to clear the word first. Zeroed by
// hk_init; only embedding lookups write it (one context per process).
static __device__ __align__(256) int check_flags[64];

std::mutex g_init_mu;
Ctx* g_ctx = nullptr;

int64_t dtype_size(int32_t dt) {
    switch (dt) {
        case HK_F32:
        case HK_I32: return 4;
        case HK_I64: return 8;
        case HK_BOOL: return 1;
        case HK_F16:
        case HK_BF16: return 2;
        default: return 0;
    }
}

bool is_float(int32_t dt) { return dt == HK_F32 || dt == HK_F16 || dt == HK_BF16; }

const char* dtype_name(int32_t dt) {
    switch (dt) {
        case HK_F32: return "F32";
        case HK_F16: return "F16";
        case HK_BF16: return "BF16";
        case HK_I32: return "I32";
        case HK_I64: return "I64";
        case HK_BOOL: return "BOOL";
        default: return "?";
    }
}

// Element count with overflow and sign checks; -1 on an invalid descriptor.
int64_t numel(const hk_tensor* t) {
    if (!t || t->rank < 0 || t->rank > HK_MAX_RANK) return -1;
    int64_t n = 1;
    for (int i = 0; i < t->rank; ++i) {
        if (t->shape[i] < 0) return -1;
        if (t->shape[i] != 0 && n > INT64_MAX / 4 / t->shape[i]) return -1;
        n *= t->shape[i];
    }
    return n;
}

int64_t nbytes(const hk_tensor* t) { return numel(t) * dtype_size(t->dtype); }

std::string shape_str(const hk_tensor* t) {
    std::string s = "[";
    for (int i = 0; i < t->rank; ++i) {
        if (i) s += ",";
        s += std::to_string(t->shape[i]);
    }
    return s + "]";
}

// Basic descriptor check: floating dtype, valid rank/shape, non-null data unless empty.
// Integer tensors (embedding IDs) are checked by ids_ok instead.
bool tensor_ok(const hk_tensor* t, const char* name, bool integer = false) {
    if (!t) {
        fail(HK_INVALID_ARGUMENT, "%s: null tensor descriptor", name);
        return false;
    }
    if (integer ? (t->dtype != HK_I32 && t->dtype != HK_I64) : !is_float(t->dtype)) {
        fail(HK_INVALID_ARGUMENT, "%s: unsupported dtype code %d", name, t->dtype);
        return false;
    }
    const int64_t n = numel(t);
    if (n < 0) {
        fail(HK_INVALID_ARGUMENT, "%s: invalid rank or shape", name);
        return false;
    }
    if (n > 0 && t->data == nullptr) {
        fail(HK_INVALID_ARGUMENT, "%s: null data pointer for a non-empty tensor", name);
        return false;
    }
    return true;
}

bool same_shape(const hk_tensor* a, const hk_tensor* b) {
    if (a->rank != b->rank) return false;
    for (int i = 0; i < a->rank; ++i)
        if (a->shape[i] != b->shape[i]) return false;
    return true;
}

bool overlaps(const hk_tensor* a, const hk_tensor* b) {
    const int64_t na = nbytes(a), nb = nbytes(b);
    if (na <= 0 || nb <= 0) return false;
    const uintptr_t a0 = reinterpret_cast<uintptr_t>(a->data), b0 = reinterpret_cast<uintptr_t>(b->data);
    return a0 < b0 + static_cast<uintptr_t>(nb) && b0 < a0 + static_cast<uintptr_t>(na);
}

// Every output must be disjoint from every input and from the other outputs.
bool disjoint(std::initializer_list<const hk_tensor*> outs, std::initializer_list<const hk_tensor*> ins) {
    std::vector<const hk_tensor*> o(outs), in(ins);
    for (size_t i = 0; i < o.size(); ++i) {
        for (const hk_tensor* x : in)
            if (overlaps(o[i], x)) {
                fail(HK_INVALID_ARGUMENT, "output overlaps an input");
                return false;
            }
        for (size_t j = i + 1; j < o.size(); ++j)
            if (overlaps(o[i], o[j])) {
                fail(HK_INVALID_ARGUMENT, "outputs overlap each other");
                return false;
            }
    }
    return true;
}

hk_tensor make_view(void* data, int32_t dtype, std::initializer_list<int64_t> shape) {
    hk_tensor t{};
    t.data = data;
    t.dtype = dtype;
    t.rank = static_cast<int32_t>(shape.size());
    int i = 0;
    for (int64_t d : shape) t.shape[i++] = d;
    return t;
}

// Acquire the context for an op: initialized, not poisoned; holds its mutex.
struct OpGuard {
    Ctx* c;
    std::unique_lock<std::mutex> lock;
    hk_status st = HK_OK;
    explicit OpGuard(hk_context* h) : c(reinterpret_cast<Ctx*>(h)) {
        if (!c || c != g_ctx) {
            st = fail(HK_NOT_INITIALIZED, "runtime is not initialized (call hk_init)");
            return;
        }
        lock = std::unique_lock<std::mutex>(c->mu);
        if (c->poisoned) st = fail(HK_POISONED, "context poisoned by an earlier completion failure");
    }
};

// After enqueuing an op: check the launch, then synchronize unless async. A failure
// poisons the context, as a failed launch/sync poisons the reference's provider.
hk_status complete(Ctx* c, hipError_t launch, const char* op, int kernels) {
    c->stats.launches += static_cast<uint64_t>(kernels);
    hipError_t sync = hipSuccess;
    if (launch == hipSuccess && !c->async) {
        sync = hipStreamSynchronize(c->stream);
        c->stats.synchronizations += 1;
    }
    if (launch != hipSuccess || sync != hipSuccess) {
        c->poisoned = true;
        return fail(HK_COMPLETION_ERROR, "%s: launch status %d (%s), synchronization status %d (%s)", op,
                    static_cast<int>(launch), hipGetErrorString(launch), static_cast<int>(sync),
                    hipGetErrorString(sync));
    }
    return HK_OK;
}

// Upper bound on the workspace, in bytes: the environment variable HK_WORKSPACE_LIMIT (read on
// every resize), else none. A larger request fails as an allocation failure does, so callers
// that cap the library's device memory get the same fallbacks (the recompute form of the
// attention backward) as when HBM is short.
size_t workspace_limit() {
    const char* env = std::getenv("HK_WORKSPACE_LIMIT");
    if (env == nullptr || *env == '\0') return SIZE_MAX;
    char* end = nullptr;
    const unsigned long long v = std::strtoull(env, &end, 10);
    return end != nullptr && *end == '\0' ? static_cast<size_t>(v) : SIZE_MAX;
}

hk_status ensure_workspace(Ctx* c, size_t bytes) {
    if (bytes <= c->ws_bytes) return HK_OK;
    const size_t limit = workspace_limit();
    if (bytes > limit)
        return fail(HK_HIP_ERROR, "workspace of %zu bytes exceeds HK_WORKSPACE_LIMIT (%zu bytes)", bytes, limit);
    if (c->workspace) {
        // queued work may still read the old buffer
        hipError_t e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) {
            c->poisoned = true;
            return fail(HK_COMPLETION_ERROR, "workspace resize: synchronization status %d", static_cast<int>(e));
        }
        (void)hipFree(c->workspace);
        c->workspace = nullptr;
        c->ws_bytes = 0;
    }
    size_t want = bytes < (size_t(1) << 20) ? std::min(size_t(1) << 20, limit) : bytes;
    hipError_t e = hipMalloc(&c->workspace, want);
    if (e != hipSuccess) {
        c->workspace = nullptr;
        // a failed allocation leaves HIP's last error set; every launch wrapper returns
        // hipGetLastError(), so clear it here or the next op reports it and poisons the context
        (void)hipGetLastError();
        return fail(HK_HIP_ERROR, "workspace allocation of %zu bytes failed: %s", want, hipGetErrorString(e));
    }
    c->ws_bytes = want;
    return HK_OK;
}

// Frees the workspace when it holds more than keep bytes (after the queued work that may use it).
hk_status trim_workspace(Ctx* c, size_t keep) {
    if (!c->workspace || c->ws_bytes <= keep) return HK_OK;
    hipError_t e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        c->poisoned = true;
        return fail(HK_COMPLETION_ERROR, "workspace trim: synchronization status %d", static_cast<int>(e));
    }
    e = hipFree(c->workspace);
    c->workspace = nullptr;
    c->ws_bytes = 0;
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(HK_HIP_ERROR, "workspace release failed: %s", hipGetErrorString(e));
    }
    return HK_OK;
}

// ------------------------------------------------------------------ GEMM contract

struct GemmSpec {
    int kind = 0;  // 0 dense, 1 batched
    int64_t batch = 1, m = 0, n = 0, k = 0;
    int32_t out_dtype = HK_BF16;
};

// Reference: GemmSpec::new + GemmSpec::checked, rust-ascend-driver/src/tensor/deepgemm/plan.rs:49-80.
hk_status gemm_spec(const hk_tensor* a, const hk_tensor* b, int32_t ta, int32_t tb, int32_t out_dtype,
                    GemmSpec* s) {
    if (!tensor_ok(a, "A") || !tensor_ok(b, "B")) return HK_INVALID_ARGUMENT;
    if ((ta != HK_NO && ta != HK_YES) || (tb != HK_NO && tb != HK_YES))
        return fail(HK_INVALID_ARGUMENT, "transpose flags must be 0 (No) or 1 (Yes)");
    const int r = a->rank;
    if (!(r == 2 || r == 3) || b->rank != r) return fail(HK_INVALID_ARGUMENT, "GEMM requires matching rank 2 or rank 3");
    if (r == 3 && a->shape[0] != b->shape[0]) return fail(HK_INVALID_ARGUMENT, "batch broadcasting is not supported");
    const int64_t* a2 = a->shape + (r - 2);
    const int64_t* b2 = b->shape + (r - 2);
    const int64_t m = ta == HK_NO ? a2[0] : a2[1];
    const int64_t k = ta == HK_NO ? a2[1] : a2[0];
    const int64_t kb = tb == HK_NO ? b2[0] : b2[1];
    const int64_t n = tb == HK_NO ? b2[1] : b2[0];
    if (kb != k) return fail(HK_INVALID_ARGUMENT, "GEMM contraction mismatch (%lld vs %lld)", (long long)k, (long long)kb);
    const int64_t groups = r == 3 ? a->shape[0] : 1;
    if (a->dtype != HK_BF16 || b->dtype != HK_BF16 || !(out_dtype == HK_BF16 || out_dtype == HK_F32))
        return fail(HK_INVALID_ARGUMENT, "GEMM accepts BF16 inputs and BF16/F32 output only (got %s, %s -> %s)",
                    dtype_name(a->dtype), dtype_name(b->dtype), dtype_name(out_dtype));
    for (int64_t x : {m, n, k})
        if (x <= 0 || x % 16 != 0 || x > INT32_MAX)
            return fail(HK_INVALID_ARGUMENT,
                        "M/N/K must be positive multiples of 16 <= INT32_MAX; batches 1..=4096 (M=%lld N=%lld K=%lld)",
                        (long long)m, (long long)n, (long long)k);
    if (groups <= 0 || groups > 4096)
        return fail(HK_INVALID_ARGUMENT, "M/N/K must be positive multiples of 16 <= INT32_MAX; batches 1..=4096");
    const int64_t tiles = ((m + 63) / 64) * ((n + 63) / 64) * groups;
    if (tiles > static_cast<int64_t>(INT32_MAX) - 32) return fail(HK_INVALID_ARGUMENT, "tile range overflows");
    s->kind = r == 3 ? 1 : 0;
    s->batch = groups;
    s->m = m;
    s->n = n;
    s->k = k;
    s->out_dtype = out_dtype;
    return HK_OK;
}

// Reference: GroupEnds::new, deepgemm/plan.rs:16-26.
hk_status group_ends_check(const int32_t* ends, int32_t count) {
    if (count <= 0 || count > 4096 || ends == nullptr) return fail(HK_INVALID_ARGUMENT, "group count must be 1..=4096");
    int32_t previous = 0;
    for (int32_t i = 0; i < count; ++i) {
        if (ends[i] < previous || ends[i] % 256 != 0)
            return fail(HK_INVALID_ARGUMENT, "group ends must be nondecreasing multiples of 256");
        previous = ends[i];
    }
    if (previous == 0) return fail(HK_INVALID_ARGUMENT, "all-empty grouped GEMM is not implemented");
    return HK_OK;
}

// Reference: GemmSpec::grouped_nt (deepgemm/plan.rs:61-67), then GemmSpec::checked (:68-80) with
// 256-row M blocks for the tile-range bound.
hk_status grouped_spec(const hk_tensor* a, const hk_tensor* w, const int32_t* ends, int32_t count, int32_t out_dtype,
                       GemmSpec* s) {
    if (!tensor_ok(a, "A") || !tensor_ok(w, "weights")) return HK_INVALID_ARGUMENT;
    hk_status st = group_ends_check(ends, count);
    if (st != HK_OK) return st;
    if (a->rank != 2 || w->rank != 3) return fail(HK_INVALID_ARGUMENT, "grouped NT requires [M,K] and [G,N,K]");
    if (a->shape[0] != ends[count - 1] || w->shape[0] != count || a->shape[1] != w->shape[2])
        return fail(HK_INVALID_ARGUMENT, "grouped NT dimensions do not match the physical prefix sums");
    if (a->dtype != HK_BF16 || w->dtype != HK_BF16 || !(out_dtype == HK_BF16 || out_dtype == HK_F32))
        return fail(HK_INVALID_ARGUMENT, "GEMM accepts BF16 inputs and BF16/F32 output only (got %s, %s -> %s)",
                    dtype_name(a->dtype), dtype_name(w->dtype), dtype_name(out_dtype));
    const int64_t m = a->shape[0], n = w->shape[1], k = a->shape[1];
    for (int64_t x : {m, n, k})
        if (x <= 0 || x % 16 != 0 || x > INT32_MAX)
            return fail(HK_INVALID_ARGUMENT,
                        "M/N/K must be positive multiples of 16 <= INT32_MAX; batches/groups 1..=4096 (M=%lld N=%lld K=%lld)",
                        (long long)m, (long long)n, (long long)k);
    const int64_t tiles = ((m + 255) / 256) * ((n + 63) / 64);
    if (tiles > static_cast<int64_t>(INT32_MAX) - 32) return fail(HK_INVALID_ARGUMENT, "tile range overflows");
    s->kind = 2;
    s->batch = count;
    s->m = m;
    s->n = n;
    s->k = k;
    s->out_dtype = out_dtype;
    return HK_OK;
}

// Uploaded group ends: the checked host copy and, in one device allocation, the ends themselves
// (the grouped_layout argument of the M-grouped device programs) followed by the group of every
// 256-row block of A (what libhk.so's grouped kernels index).
struct GroupEndsDev {
    Ctx* ctx = nullptr;
    std::vector<int32_t> ends;
    int32_t* mem = nullptr;          // the allocation
    int32_t* ends_dev = nullptr;     // mem: the ends, padded to 64 entries
    int32_t* block_group = nullptr;  // after the padded ends
};

bool live_group_table(const Ctx* c, const void* h) {
    return std::find(c->group_tables.begin(), c->group_tables.end(), h) != c->group_tables.end();
}

// A loaded device-program code object and the entry points looked up in it. The image stays
// allocated with the module, as the reference keeps the verified ELF bytes alive
// (deepgemm/native.rs:41-43).
enum class ProgramKind { Dense, Batched, MGrouped };
struct FunctionDev {
    hipFunction_t fn = nullptr;
    hipFunction_t fn_wide = nullptr;  // NAME_wide: operand slices past 32-bit offsets (null if absent)
    std::string name;
    ProgramKind kind = ProgramKind::Dense;
    bool ta = false, tb = false, out_bf16 = true;
};
struct ModuleDev {
    Ctx* ctx = nullptr;
    hipModule_t module = nullptr;
    std::vector<unsigned char> image;
    std::vector<std::unique_ptr<FunctionDev>> functions;
};

// Unload every module and free every group-ends table of a context whose stream has completed.
void release_programs(Ctx* c) {
    for (ModuleDev* m : c->modules) {
        (void)hipModuleUnload(m->module);
        delete m;
    }
    c->modules.clear();
    for (GroupEndsDev* d : c->group_tables) {
        (void)hipFree(d->mem);
        delete d;
    }
    c->group_tables.clear();
}

bool out_matches(const GemmSpec& s, const hk_tensor* out) {
    if (out->dtype != s.out_dtype) return false;
    if (s.kind != 1) return out->rank == 2 && out->shape[0] == s.m && out->shape[1] == s.n;
    return out->rank == 3 && out->shape[0] == s.batch && out->shape[1] == s.m && out->shape[2] == s.n;
}

hk_status run_gemm(Ctx* c, const GemmSpec& s, const void* a, const void* b, void* out, int ta, int tb,
                   void* ws, hipError_t* err) {
    *err = hk::gemm_bf16(a, b, out, s.out_dtype == HK_BF16, s.batch, s.m, s.n, s.k, ta, tb, ws, c->num_cus,
                         c->stream);
    return HK_OK;
}

// The reference's FP32-storage wrappers take F32 A/B; the GEMM runs on BF16 copies.
hk_status mixed_spec(const hk_tensor* a, const hk_tensor* b, int32_t ta, int32_t tb, GemmSpec* s) {
    if (!tensor_ok(a, "A") || !tensor_ok(b, "B")) return HK_INVALID_ARGUMENT;
    if (a->dtype != HK_F32 || b->dtype != HK_F32)
        return fail(HK_INVALID_ARGUMENT, "BF16-compute FP32 matmul requires FP32 inputs");
    hk_tensor ab = *a, bb = *b;
    ab.dtype = HK_BF16;
    bb.dtype = HK_BF16;
    return gemm_spec(&ab, &bb, ta, tb, HK_F32, s);
}

bool is_bf16_copy_of(const hk_tensor* snap, const hk_tensor* src) {
    return snap && snap->dtype == HK_BF16 && same_shape(snap, src);
}

// ------------------------------------------------------------------ row layouts

// rows x width of a contiguous tensor whose last axis is the row.
bool row_layout(const hk_tensor* x, int64_t* rows, int64_t* width, const char* op) {
    if (x->rank < 1) {
        fail(HK_INVALID_ARGUMENT, "%s requires a last dimension", op);
        return false;
    }
    *width = x->shape[x->rank - 1];
    if (*width <= 0) {
        fail(HK_INVALID_ARGUMENT, "%s width must be positive", op);
        return false;
    }
    if (*width > INT32_MAX) {
        fail(HK_INVALID_ARGUMENT, "%s width must not exceed INT32_MAX", op);
        return false;
    }
    *rows = numel(x) / *width;
    return true;
}

}  // namespace

// ====================================================================== C ABI

extern "C" {

const char* hk_last_error(void) { return g_last_error.c_str(); }

int32_t hk_abi_version(void) { return 1; }

hk_status hk_init(int32_t device, hk_context** out) {
    if (!out) return fail(HK_INVALID_ARGUMENT, "null output handle");
    std::lock_guard<std::mutex> lk(g_init_mu);
    if (g_ctx) return fail(HK_INVALID_ARGUMENT, "HIP runtime already initialized");
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count <= 0)
        return fail(HK_LOAD_ERROR, "no HIP device available (%s)", hipGetErrorString(e));
    if (device < 0 || device >= count) return fail(HK_INVALID_ARGUMENT, "device ordinal %d out of range 0..%d", device, count - 1);
    e = hipSetDevice(device);
    if (e != hipSuccess) return fail(HK_HIP_ERROR, "hipSetDevice(%d): %s", device, hipGetErrorString(e));
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return fail(HK_HIP_ERROR, "hipGetDeviceProperties: %s", hipGetErrorString(e));
    // Reference: NativeApi::check_soc requires the one supported SoC (deepgemm/native.rs:16-35).
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(HK_LOAD_ERROR, "device %d is %s; libhk.so carries gfx950 code only", device, prop.gcnArchName);
    void* scratch_ptr = nullptr;
    e = hipGetSymbolAddress(&scratch_ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || scratch_ptr == nullptr)
        return fail(HK_LOAD_ERROR, "hipGetSymbolAddress(scratch) on device %d: %s", device, hipGetErrorString(e));
    void* flags_ptr = nullptr;
    e = hipGetSymbolAddress(&flags_ptr, HIP_SYMBOL(check_flags));
    if (e == hipSuccess && flags_ptr != nullptr) e = hipMemset(flags_ptr, 0, sizeof(check_flags));
    if (e != hipSuccess || flags_ptr == nullptr)
        return fail(HK_LOAD_ERROR, "check flags on device %d: %s", device, hipGetErrorString(e));
    Ctx* c = new Ctx();
    c->device = device;
    c->scratch = scratch_ptr;
    c->flags = static_cast<int*>(flags_ptr);
    c->num_cus = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
    c->stats.modules_loaded = 1;  // the fat binary linked into this library
    g_ctx = c;
    *out = reinterpret_cast<hk_context*>(c);
    return HK_OK;
}

hk_status hk_shutdown(hk_context* h) {
    std::lock_guard<std::mutex> lk(g_init_mu);
    Ctx* c = reinterpret_cast<Ctx*>(h);
    if (!c || c != g_ctx) return fail(HK_NOT_INITIALIZED, "runtime is not initialized");
    {
        std::lock_guard<std::mutex> g(c->mu);
        // after a failed synchronization (or on a poisoned context) device memory and code objects
        // are leaked, never freed under queued work
        if (!c->poisoned && hipStreamSynchronize(c->stream) == hipSuccess) {
            if (c->workspace) (void)hipFree(c->workspace);
            release_programs(c);
        }
    }
    delete c;
    g_ctx = nullptr;
    return HK_OK;
}

hk_status hk_set_stream(hk_context* h, void* stream) {
    OpGuard g(h);
    if (g.st != HK_OK && g.st != HK_POISONED) return g.st;
    hipStream_t next = static_cast<hipStream_t>(stream);
    if (next == g.c->stream) return HK_OK;
    // The context's workspace serves one stream at a time: in async mode, work queued on the old
    // stream may still use it, so that stream drains before ops on the new one can reuse it.
    if (g.c->async && !g.c->poisoned) {
        hipError_t e = hipStreamSynchronize(g.c->stream);
        g.c->stats.synchronizations += 1;
        if (e != hipSuccess) {
            g.c->poisoned = true;
            return fail(HK_COMPLETION_ERROR, "stream switch: synchronization status %d (%s)", static_cast<int>(e),
                        hipGetErrorString(e));
        }
    }
    g.c->stream = next;
    return HK_OK;
}

void* hk_get_stream(hk_context* h) {
    Ctx* c = reinterpret_cast<Ctx*>(h);
    return (c && c == g_ctx) ? static_cast<void*>(c->stream) : nullptr;
}

hk_status hk_set_async(hk_context* h, int32_t mode) {
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    g.c->async = mode != 0;
    return HK_OK;
}

hk_status hk_sync(hk_context* h) {
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    hipError_t e = hipStreamSynchronize(g.c->stream);
    g.c->stats.synchronizations += 1;
    if (e != hipSuccess) {
        g.c->poisoned = true;
        return fail(HK_COMPLETION_ERROR, "synchronization status %d (%s)", static_cast<int>(e), hipGetErrorString(e));
    }
    return HK_OK;
}

hk_status hk_get_stats(hk_context* h, hk_stats* out) {
    OpGuard g(h);
    if (g.st != HK_OK && g.st != HK_POISONED) return g.st;
    if (!out) return fail(HK_INVALID_ARGUMENT, "null stats pointer");
    *out = g.c->stats;
    return HK_OK;
}

hk_status hk_workspace_size(hk_context* h, uint64_t* bytes) {
    OpGuard g(h);
    if (g.st != HK_OK && g.st != HK_POISONED) return g.st;
    if (!bytes) return fail(HK_INVALID_ARGUMENT, "null output pointer");
    *bytes = g.c->ws_bytes;
    return HK_OK;
}

hk_status hk_trim_workspace(hk_context* h, uint64_t keep_bytes) {
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    return trim_workspace(g.c, static_cast<size_t>(keep_bytes));
}

hk_status hk_alloc(hk_context* h, size_t bytes, void** out) {
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    if (!out) return fail(HK_INVALID_ARGUMENT, "null output pointer");
    *out = nullptr;
    if (bytes == 0) return HK_OK;
    hipError_t e = hipMalloc(out, bytes);  // 256-byte aligned (the reference aligns to 32 B)
    if (e != hipSuccess) return fail(HK_HIP_ERROR, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    return HK_OK;
}

hk_status hk_free(hk_context* h, void* p) {
    OpGuard g(h);
    if (g.st != HK_OK && g.st != HK_POISONED) return g.st;
    if (!p) return HK_OK;
    if (g.c->poisoned) return fail(HK_POISONED, "poisoned context: memory is leaked rather than freed");
    // queued work may still use the buffer (async mode)
    hipError_t e = hipStreamSynchronize(g.c->stream);
    if (e == hipSuccess) e = hipFree(p);
    if (e != hipSuccess) return fail(HK_HIP_ERROR, "hipFree: %s", hipGetErrorString(e));
    return HK_OK;
}

hk_status hk_upload(hk_context* h, void* dst, const void* src, size_t bytes) {
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    if (bytes == 0) return HK_OK;
    if (!dst || !src) return fail(HK_INVALID_ARGUMENT, "null pointer");
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g.c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g.c->stream);
    if (e != hipSuccess) return fail(HK_HIP_ERROR, "upload: %s", hipGetErrorString(e));
    return HK_OK;
}

hk_status hk_download(hk_context* h, void* dst, const void* src, size_t bytes) {
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    if (bytes == 0) return HK_OK;
    if (!dst || !src) return fail(HK_INVALID_ARGUMENT, "null pointer");
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g.c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g.c->stream);
    if (e != hipSuccess) return fail(HK_HIP_ERROR, "download: %s", hipGetErrorString(e));
    return HK_OK;
}

// ------------------------------------------------------------------ GEMM

hk_status hk_gemm_plan_check(const hk_tensor* a, const hk_tensor* b, int32_t ta, int32_t tb, int32_t out_dtype,
                             hk_gemm_plan* plan) {
    GemmSpec s;
    hk_status st = gemm_spec(a, b, ta, tb, out_dtype, &s);
    if (st != HK_OK) return st;
    if (plan) {
        std::memset(plan, 0, sizeof *plan);
        plan->kind = s.kind;
        plan->batch = s.batch;
        plan->m = s.m;
        plan->n = s.n;
        plan->k = s.k;
        if (s.kind == 0) {
            plan->out_rank = 2;
            plan->out_shape[0] = s.m;
            plan->out_shape[1] = s.n;
        } else {
            plan->out_rank = 3;
            plan->out_shape[0] = s.batch;
            plan->out_shape[1] = s.m;
            plan->out_shape[2] = s.n;
        }
        std::snprintf(plan->key, sizeof plan->key, "bf16_%s_%c%c_%s", s.kind ? "batched" : "dense",
                      ta ? 't' : 'n', tb ? 't' : 'n', out_dtype == HK_BF16 ? "bf16" : "f32");
    }
    return HK_OK;
}

hk_status hk_gemm_into(hk_context* h, const hk_tensor* a, const hk_tensor* b, int32_t ta, int32_t tb, hk_tensor* out) {
    if (!tensor_ok(out, "out")) return HK_INVALID_ARGUMENT;
    GemmSpec s;
    hk_status st = gemm_spec(a, b, ta, tb, out->dtype, &s);
    if (st != HK_OK) return st;
    if (!out_matches(s, out)) return fail(HK_INVALID_ARGUMENT, "GEMM output layout mismatch: %s", shape_str(out).c_str());
    if (!disjoint({out}, {a, b})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    st = ensure_workspace(g.c, hk::gemm_workspace_bytes(s.batch, s.m, s.n, s.k, ta, tb));
    if (st != HK_OK) return st;
    hipError_t e;
    run_gemm(g.c, s, a->data, b->data, out->data, ta, tb, g.c->workspace, &e);
    return complete(g.c, e, "gemm", 1);
}

hk_status hk_group_ends_check(const int32_t* ends, int32_t count) { return group_ends_check(ends, count); }

hk_status hk_group_ends_upload(hk_context* h, const int32_t* ends, int32_t count, hk_group_ends** out) {
    // Reference: DeepGemm::upload_group_ends, deepgemm/mod.rs:61-67.
    if (!out) return fail(HK_INVALID_ARGUMENT, "null output handle");
    *out = nullptr;
    hk_status st = group_ends_check(ends, count);
    if (st != HK_OK) return st;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    const int64_t blocks = ends[count - 1] / 256;
    std::vector<int32_t> table(static_cast<size_t>(blocks));
    int32_t grp = 0;
    for (int64_t b = 0; b < blocks; ++b) {
        while (ends[grp] <= b * 256) ++grp;  // first group whose end lies beyond the block's first row
        table[static_cast<size_t>(b)] = grp;
    }
    const size_t padded = (static_cast<size_t>(count) + 63) & ~size_t(63);
    std::vector<int32_t> image(padded + table.size(), 0);
    std::copy(ends, ends + count, image.begin());
    std::copy(table.begin(), table.end(), image.begin() + static_cast<std::ptrdiff_t>(padded));
    GroupEndsDev* d = new GroupEndsDev();
    d->ctx = g.c;
    d->ends.assign(ends, ends + count);
    hipError_t e = hipMalloc(&d->mem, image.size() * sizeof(int32_t));
    if (e == hipSuccess)
        e = hipMemcpyAsync(d->mem, image.data(), image.size() * sizeof(int32_t), hipMemcpyHostToDevice, g.c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g.c->stream);
    if (e != hipSuccess) {
        if (d->mem) (void)hipFree(d->mem);
        delete d;
        return fail(HK_HIP_ERROR, "group ends upload: %s", hipGetErrorString(e));
    }
    d->ends_dev = d->mem;
    d->block_group = d->mem + padded;
    g.c->group_tables.push_back(d);
    *out = reinterpret_cast<hk_group_ends*>(d);
    return HK_OK;
}

hk_status hk_group_ends_free(hk_context* h, hk_group_ends* ends) {
    if (!ends) return HK_OK;
    GroupEndsDev* d = reinterpret_cast<GroupEndsDev*>(ends);
    OpGuard g(h);
    if (g.st != HK_OK && g.st != HK_POISONED) return g.st;
    if (!live_group_table(g.c, d)) return fail(HK_INVALID_ARGUMENT, "not a live group-ends handle of this context");
    if (g.c->poisoned) return fail(HK_POISONED, "poisoned context: memory is leaked rather than freed");
    hipError_t e = hipStreamSynchronize(g.c->stream);  // queued grouped GEMMs may still read the table
    if (e == hipSuccess) e = hipFree(d->mem);
    if (e != hipSuccess) return fail(HK_HIP_ERROR, "group ends free: %s", hipGetErrorString(e));
    auto& live = g.c->group_tables;
    live.erase(std::remove(live.begin(), live.end(), d), live.end());
    delete d;
    return HK_OK;
}

hk_status hk_gemm_grouped_plan_check(const hk_tensor* a, const hk_tensor* w, const int32_t* ends, int32_t count,
                                     int32_t out_dtype, hk_gemm_plan* plan) {
    GemmSpec s;
    hk_status st = grouped_spec(a, w, ends, count, out_dtype, &s);
    if (st != HK_OK) return st;
    if (plan) {
        std::memset(plan, 0, sizeof *plan);
        plan->kind = 2;
        plan->batch = s.batch;
        plan->m = s.m;
        plan->n = s.n;
        plan->k = s.k;
        plan->out_rank = 2;
        plan->out_shape[0] = s.m;
        plan->out_shape[1] = s.n;
        std::snprintf(plan->key, sizeof plan->key, "bf16_mgrouped_nt_%s", out_dtype == HK_BF16 ? "bf16" : "f32");
    }
    return HK_OK;
}

hk_status hk_gemm_grouped_nt_into(hk_context* h, const hk_tensor* a, const hk_tensor* w, const hk_group_ends* ends,
                                  hk_tensor* out) {
    // Reference: DeepGemm::grouped_nt_into, deepgemm/mod.rs:74-78 and run (:87-97).
    if (!tensor_ok(out, "out")) return HK_INVALID_ARGUMENT;
    if (!ends) return fail(HK_INVALID_ARGUMENT, "grouped GEMM requires uploaded group ends");
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    const GroupEndsDev* d = reinterpret_cast<const GroupEndsDev*>(ends);
    if (!live_group_table(g.c, d))
        return fail(HK_INVALID_ARGUMENT, "grouped GEMM requires group ends uploaded to this context");
    GemmSpec s;
    hk_status st = grouped_spec(a, w, d->ends.data(), static_cast<int32_t>(d->ends.size()), out->dtype, &s);
    if (st != HK_OK) return st;
    if (!out_matches(s, out)) return fail(HK_INVALID_ARGUMENT, "grouped GEMM output layout mismatch: %s", shape_str(out).c_str());
    if (!disjoint({out}, {a, w})) return HK_INVALID_ARGUMENT;
    hipError_t e = hk::gemm_bf16_grouped_nt(a->data, w->data, out->data, s.out_dtype == HK_BF16, s.m, s.n, s.k,
                                            d->block_group, g.c->num_cus, g.c->stream);
    return complete(g.c, e, "grouped_nt", 1);
}

// ------------------------------------------------------------------ GEMM device programs
//
// The reference reads each GEMM program from a checked artifact (deepgemm/artifact.rs:6-27), loads
// it with aclrtBinaryLoadFromData, looks its entry up with aclrtBinaryGetFunction (native.rs:46-64)
// and launches it with aclrtLaunchKernelWithArgsArray and a nine-pointer argv (native.rs:87-93,
// deepgemm/mod.rs:122-145). Here the 18 programs are one gfx950 code object built ahead of time
// (hk_programs.hip -> hk_programs.hsaco), loaded with hipModuleLoadData; the argv goes to
// hipModuleLaunchKernel unchanged, since it is the programs' own parameter list. The programs trust
// their arguments, so the launch checks every one against the reference's contract first.

namespace {

constexpr size_t kMaxImageBytes = size_t(128) << 20;  // artifact.rs:19
constexpr uint32_t kEfAmdgpuMachGfx950 = 0x4f;

uint16_t rd16(const unsigned char* p) {
    uint16_t v;
    std::memcpy(&v, p, sizeof v);
    return v;
}
uint32_t rd32(const unsigned char* p) {
    uint32_t v;
    std::memcpy(&v, p, sizeof v);
    return v;
}
uint64_t rd64(const unsigned char* p) {
    uint64_t v;
    std::memcpy(&v, p, sizeof v);
    return v;
}

// A complete little-endian ELF64 AMDGPU code object for gfx950 whose headers and sections lie
// inside the image (reference check: artifact.rs:18-22 for its own ELF64 object).
hk_status check_code_object(const unsigned char* p, size_t n) {
    if (n < 64 || n > kMaxImageBytes) return fail(HK_LOAD_ERROR, "invalid code object size %zu", n);
    if (std::memcmp(p, "\x7f" "ELF\x02\x01", 6) != 0)
        return fail(HK_LOAD_ERROR, "expected a little-endian ELF64 code object (an unbundled --genco image)");
    if (rd16(p + 16) != 3 || rd16(p + 18) != 224)
        return fail(HK_LOAD_ERROR, "not an AMDGPU code object (e_type %u, e_machine %u)", rd16(p + 16),
                    rd16(p + 18));
    const uint32_t mach = rd32(p + 48) & 0xff;
    if (mach != kEfAmdgpuMachGfx950)
        return fail(HK_LOAD_ERROR, "code object is for another GPU (e_flags machine 0x%x; gfx950 is 0x%x)", mach,
                    kEfAmdgpuMachGfx950);
    const uint64_t phoff = rd64(p + 32), shoff = rd64(p + 40);
    const uint16_t phentsize = rd16(p + 54), phnum = rd16(p + 56);
    const uint16_t shentsize = rd16(p + 58), shnum = rd16(p + 60);
    if (phoff > n || uint64_t(phentsize) * phnum > n - phoff || shoff > n || shentsize < 64 ||
        uint64_t(shentsize) * shnum > n - shoff)
        return fail(HK_LOAD_ERROR, "truncated code object (header tables past the end of %zu bytes)", n);
    for (uint16_t i = 0; i < shnum; ++i) {
        const unsigned char* sh = p + shoff + uint64_t(i) * shentsize;
        const uint32_t type = rd32(sh + 4);
        const uint64_t off = rd64(sh + 24), size = rd64(sh + 32);
        if (type != 8 /* SHT_NOBITS */ && (off > n || size > n - off))
            return fail(HK_LOAD_ERROR, "truncated code object (section %u past the end of %zu bytes)", i, n);
    }
    return HK_OK;
}

// The code object's entry points, by name: ruda_rust_bf16_{dense,batched}_{n,t}{n,t}_{bf16,f32} and
// ruda_rust_bf16_mgrouped_nt_{bf16,f32} (rust-ascend-kernels/src/config.rs:14-40; the name is
// "ruda_rust_" + GemmSpec::key, deepgemm/plan.rs:84-85).
bool program_spec(const char* name, FunctionDev* f) {
    for (int kind = 0; kind < 3; ++kind)
        for (int ta = 0; ta < 2; ++ta)
            for (int tb = 0; tb < 2; ++tb)
                for (int bf16 = 0; bf16 < 2; ++bf16) {
                    if (kind == 2 && (ta || !tb)) continue;  // M-grouped is NT only
                    char want[64];
                    std::snprintf(want, sizeof want, "ruda_rust_bf16_%s_%c%c_%s",
                                  kind == 0 ? "dense" : kind == 1 ? "batched" : "mgrouped", ta ? 't' : 'n',
                                  tb ? 't' : 'n', bf16 ? "bf16" : "f32");
                    if (std::strcmp(name, want) != 0) continue;
                    f->name = want;
                    f->kind = static_cast<ProgramKind>(kind);
                    f->ta = ta;
                    f->tb = tb;
                    f->out_bf16 = bf16;
                    return true;
                }
    return false;
}

ModuleDev* live_module(const Ctx* c, const void* h) {
    for (ModuleDev* m : c->modules)
        if (m == h) return m;
    return nullptr;
}

const FunctionDev* live_function(const Ctx* c, const void* h) {
    for (const ModuleDev* m : c->modules)
        for (const auto& f : m->functions)
            if (f.get() == h) return f.get();
    return nullptr;
}

// [addr, addr + bytes) inside one device allocation of this process.
bool in_device_allocation(uint64_t addr, uint64_t bytes) {
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    if (hipMemGetAddressRange(&base, &size, reinterpret_cast<hipDeviceptr_t>(addr)) != hipSuccess) {
        (void)hipGetLastError();  // not device memory: clear the error so no later launch check sees it
        return false;
    }
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    return addr >= b && bytes <= size && addr - b <= size - bytes;
}

}  // namespace

hk_status hk_module_load_data(hk_context* h, const void* image, size_t bytes, hk_module** out) {
    // Reference: Kernel::load (aclrtBinaryLoadFromData), deepgemm/native.rs:46-52, after
    // artifact::read's checks (artifact.rs:18-22).
    if (!out) return fail(HK_INVALID_ARGUMENT, "null output handle");
    *out = nullptr;
    if (!image) return fail(HK_INVALID_ARGUMENT, "null code object image");
    const unsigned char* p = static_cast<const unsigned char*>(image);
    hk_status st = check_code_object(p, bytes);
    if (st != HK_OK) return st;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    auto m = std::make_unique<ModuleDev>();
    m->ctx = g.c;
    m->image.assign(p, p + bytes);
    hipError_t e = hipModuleLoadData(&m->module, m->image.data());
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(HK_LOAD_ERROR, "hipModuleLoadData: %s", hipGetErrorString(e));
    }
    g.c->modules.push_back(m.get());
    g.c->stats.modules_loaded += 1;
    *out = reinterpret_cast<hk_module*>(m.release());
    return HK_OK;
}

hk_status hk_module_get_function(hk_context* h, hk_module* module, const char* name, hk_function** out) {
    // Reference: Kernel::load's aclrtBinaryGetFunction, deepgemm/native.rs:53-63.
    if (!out) return fail(HK_INVALID_ARGUMENT, "null output handle");
    *out = nullptr;
    if (!name) return fail(HK_INVALID_ARGUMENT, "null program name");
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    ModuleDev* m = live_module(g.c, module);
    if (!m) return fail(HK_INVALID_ARGUMENT, "not a loaded module of this context");
    auto f = std::make_unique<FunctionDev>();
    if (!program_spec(name, f.get()))
        return fail(HK_INVALID_ARGUMENT,
                    "unknown device program \"%.80s\" (the code object holds ruda_rust_bf16_{dense,batched}_{n,t}{n,t}_"
                    "{bf16,f32} and ruda_rust_bf16_mgrouped_nt_{bf16,f32})", name);
    for (const auto& have : m->functions)
        if (have->name == f->name) {
            *out = reinterpret_cast<hk_function*>(have.get());
            return HK_OK;
        }
    hipError_t e = hipModuleGetFunction(&f->fn, m->module, f->name.c_str());
    if (e != hipSuccess || !f->fn) {
        (void)hipGetLastError();
        return fail(HK_LOAD_ERROR, "hipModuleGetFunction(%s): %s", f->name.c_str(), hipGetErrorString(e));
    }
    // The companion for operand slices past 32-bit offsets; a code object without it serves only
    // the shapes within them.
    if (hipModuleGetFunction(&f->fn_wide, m->module, (f->name + "_wide").c_str()) != hipSuccess) {
        (void)hipGetLastError();
        f->fn_wide = nullptr;
    }
    m->functions.push_back(std::move(f));
    *out = reinterpret_cast<hk_function*>(m->functions.back().get());
    return HK_OK;
}

hk_status hk_launch_kernel_with_args(hk_context* h, const hk_function* function, uint32_t block_dim, void** args) {
    // Reference: aclrtLaunchKernelWithArgsArray(function, 32, stream, NULL, argv) and the argv it is
    // given, deepgemm/native.rs:11,87-93 and deepgemm/mod.rs:122-145; the contract checked here is
    // GemmSpec::checked's (plan.rs:68-80) plus the packing execute_addresses writes (mod.rs:125-131).
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    const FunctionDev* f = live_function(g.c, function);
    if (!f) return fail(HK_INVALID_ARGUMENT, "not a device program of a module loaded in this context");
    if (block_dim == 0) return fail(HK_INVALID_ARGUMENT, "block_dim must be positive");
    if (!args) return fail(HK_INVALID_ARGUMENT, "null argument array");
    for (int i = 0; i < 9; ++i)
        if (!args[i]) return fail(HK_INVALID_ARGUMENT, "argument pointer %d of 9 is null", i);
    hk_gm a, b, d;
    uint32_t m, n, k, groups;
    const int32_t* ends_ptr;
    hk_epilogue ep;
    std::memcpy(&a, args[0], sizeof a);
    std::memcpy(&b, args[1], sizeof b);
    std::memcpy(&d, args[2], sizeof d);
    std::memcpy(&m, args[3], sizeof m);
    std::memcpy(&n, args[4], sizeof n);
    std::memcpy(&k, args[5], sizeof k);
    std::memcpy(&ends_ptr, args[6], sizeof ends_ptr);
    std::memcpy(&groups, args[7], sizeof groups);
    std::memcpy(&ep, args[8], sizeof ep);
    for (uint32_t x : {m, n, k})
        if (x == 0 || x % 16 != 0 || x > INT32_MAX)
            return fail(HK_INVALID_ARGUMENT,
                        "M/N/K must be positive multiples of 16 <= INT32_MAX; batches/groups 1..=4096 (M=%u N=%u K=%u)",
                        m, n, k);
    if (ep.alpha != 1.0f || ep.pad0 != 0 || ep.sfd != 0 || ep.stride != 0 || ep.n != n || ep.pad1 != 0)
        return fail(HK_INVALID_ARGUMENT, "epilogue must be {alpha 1, pad 0, sfd 0, stride 0, n = N} (mod.rs:132)");
    int64_t batches = 1, slices = 1;
    if (f->kind == ProgramKind::Dense) {
        if (groups != 0 || ends_ptr) return fail(HK_INVALID_ARGUMENT, "dense programs take num_groups 0 and no grouped_layout");
    } else if (f->kind == ProgramKind::Batched) {
        if (groups == 0 || groups > 4096 || ends_ptr)
            return fail(HK_INVALID_ARGUMENT, "batched programs take num_groups 1..=4096 (the batch) and no grouped_layout");
        batches = slices = groups;
    } else {
        const GroupEndsDev* t = nullptr;
        for (const GroupEndsDev* x : g.c->group_tables)
            if (x->ends_dev == ends_ptr) t = x;
        if (!t) return fail(HK_INVALID_ARGUMENT, "grouped_layout must be the device ends of group ends uploaded to this context");
        if (groups != t->ends.size() || static_cast<int64_t>(m) != t->ends.back())
            return fail(HK_INVALID_ARGUMENT, "grouped NT dimensions do not match the physical prefix sums");
        slices = groups;
    }
    const bool batched = f->kind == ProgramKind::Batched;
    const uint64_t want_a = f->ta ? m : k, want_b = f->tb ? k : n;
    const uint64_t mk = uint64_t(m) * k, nk = uint64_t(n) * k, mn = uint64_t(m) * n;
    if (a.stride_outer != want_a || a.stride_batch != (batched ? mk : 0) || b.stride_outer != want_b ||
        b.stride_batch != (batched ? nk : 0) || d.stride_outer != n || d.stride_batch != (batched ? mn : 0))
        return fail(HK_INVALID_ARGUMENT,
                    "device programs take packed row-major operands: strides (outer, batch) A (%llu, %llu) B (%llu, "
                    "%llu) D (%llu, %llu), expected A (%llu, %llu) B (%llu, %llu) D (%u, %llu)",
                    (unsigned long long)a.stride_outer, (unsigned long long)a.stride_batch,
                    (unsigned long long)b.stride_outer, (unsigned long long)b.stride_batch,
                    (unsigned long long)d.stride_outer, (unsigned long long)d.stride_batch,
                    (unsigned long long)want_a, (unsigned long long)(batched ? mk : 0), (unsigned long long)want_b,
                    (unsigned long long)(batched ? nk : 0), n, (unsigned long long)(batched ? mn : 0));
    // The 256x256 tile kernel addresses each operand slice with 32-bit byte offsets up to the end of
    // the last 64-deep K stage; past that, the program's _wide companion addresses from each tile
    // (a K-major operand's 256 rows of K, an MN-major one's 64 k-rows of M or N columns per stage).
    const uint64_t k64 = (uint64_t(k) + 63) / 64 * 64, lim = uint64_t(1) << 31;
    hipFunction_t fn = f->fn;
    if (uint64_t(m) * k64 * 2 >= lim || uint64_t(n) * k64 * 2 >= lim) {
        auto reach = [&](bool mn_major, uint64_t cols) { return mn_major ? 64 * cols * 2 + 512 : 256 * k64 * 2; };
        if (!f->fn_wide || reach(f->ta, m) >= lim || reach(!f->tb, n) >= lim)
            return fail(HK_INVALID_ARGUMENT,
                        "operand slice too large for the device programs' offsets (M*K or N*K of 2^30 elements or "
                        "more needs K < 2^22 for a K-major operand and M or N < 2^24 for an MN-major one)");
        fn = f->fn_wide;
    }
    for (const hk_gm* x : {&a, &b, &d})
        if (x->addr == 0 || x->addr % 16 != 0)
            return fail(HK_INVALID_ARGUMENT, "operand addresses must be non-null and 16-byte aligned");
    const uint64_t a_bytes = uint64_t(batches) * mk * 2, b_bytes = uint64_t(slices) * nk * 2;
    const uint64_t d_bytes = uint64_t(batches) * mn * (f->out_bf16 ? 2 : 4);
    auto overlap = [](uint64_t p, uint64_t pn, uint64_t q, uint64_t qn) { return p < q + qn && q < p + pn; };
    if (overlap(d.addr, d_bytes, a.addr, a_bytes) || overlap(d.addr, d_bytes, b.addr, b_bytes))
        return fail(HK_INVALID_ARGUMENT, "GEMM output overlaps input");
    if (!in_device_allocation(a.addr, a_bytes) || !in_device_allocation(b.addr, b_bytes) ||
        !in_device_allocation(d.addr, d_bytes))
        return fail(HK_INVALID_ARGUMENT, "an operand range is not inside one device allocation of this process");
    const unsigned tiles = ((m + 255) / 256) * ((n + 255) / 256);
    hipError_t e = hipModuleLaunchKernel(fn, tiles, 1, static_cast<unsigned>(batches), 256, 1, 1, 0, g.c->stream,
                                         args, nullptr);
    return complete(g.c, e, f->name.c_str(), 1);
}

hk_status hk_module_unload(hk_context* h, hk_module* module) {
    // Reference: Drop for Kernel (aclrtBinaryUnLoad once the session's work is complete, else the
    // code is leaked), deepgemm/native.rs:66-76.
    if (!module) return HK_OK;
    OpGuard g(h);
    if (g.st != HK_OK && g.st != HK_POISONED) return g.st;
    ModuleDev* m = live_module(g.c, module);
    if (!m) return fail(HK_INVALID_ARGUMENT, "not a loaded module of this context");
    if (g.c->poisoned) return fail(HK_POISONED, "poisoned context: the code object stays loaded under queued work");
    hipError_t e = hipStreamSynchronize(g.c->stream);
    if (e != hipSuccess) {
        g.c->poisoned = true;
        return fail(HK_COMPLETION_ERROR, "module unload: synchronization status %d (%s)", static_cast<int>(e),
                    hipGetErrorString(e));
    }
    e = hipModuleUnload(m->module);
    auto& live = g.c->modules;
    live.erase(std::remove(live.begin(), live.end(), m), live.end());
    delete m;
    if (e != hipSuccess) return fail(HK_HIP_ERROR, "hipModuleUnload: %s", hipGetErrorString(e));
    return HK_OK;
}

hk_status hk_group_ends_data(hk_context* h, const hk_group_ends* ends, const int32_t** out) {
    // Reference: DeviceGroupEnds' device tensor, the grouped_layout argument (deepgemm/mod.rs:70,101).
    if (!out) return fail(HK_INVALID_ARGUMENT, "null output pointer");
    *out = nullptr;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    if (!live_group_table(g.c, ends)) return fail(HK_INVALID_ARGUMENT, "not a live group-ends handle of this context");
    *out = reinterpret_cast<const GroupEndsDev*>(ends)->ends_dev;
    return HK_OK;
}

// ------------------------------------------------------------------ generic floating matmul

namespace {

// Reference: generic_matrix::output_layout (runtime/generic_matrix.rs:4-15) over
// layout::matmul_shape and layout::broadcast (tensor/layout.rs:106-142): matching F32/F16/BF16,
// rank 2..6 each, A [..., M, K] and B [..., K, N], batch dims broadcast from the right.
hk_status matmul_spec(const hk_tensor* a, const hk_tensor* b, hk::MatmulSpec* s, hk_tensor* out_layout) {
    if (!tensor_ok(a, "A") || !tensor_ok(b, "B")) return HK_INVALID_ARGUMENT;
    if (b->dtype != a->dtype || !(a->rank >= 2 && a->rank <= 6) || !(b->rank >= 2 && b->rank <= 6))
        return fail(HK_INVALID_ARGUMENT, "generic matmul requires matching floating dtypes and rank 2..6");
    const int64_t m = a->shape[a->rank - 2], k = a->shape[a->rank - 1];
    const int64_t kb = b->shape[b->rank - 2], n = b->shape[b->rank - 1];
    if (k != kb) return fail(HK_INVALID_ARGUMENT, "matmul contraction dimensions differ");
    const int ra = a->rank - 2, rb = b->rank - 2, rank = ra > rb ? ra : rb;
    int64_t shape[4], sa[4], sb[4];
    int64_t stride_a = m * k, stride_b = k * n;  // elements per batch step of the innermost batch dim
    for (int i = 0; i < rank; ++i) {  // i-th batch dim from the right
        const int64_t x = i < ra ? a->shape[ra - 1 - i] : 1;
        const int64_t y = i < rb ? b->shape[rb - 1 - i] : 1;
        int64_t d;
        if (x == y || y == 1) d = x;
        else if (x == 1) d = y;
        else return fail(HK_INVALID_ARGUMENT, "incompatible broadcast dimensions");
        shape[rank - 1 - i] = d;
        sa[rank - 1 - i] = x == 1 ? 0 : stride_a;
        sb[rank - 1 - i] = y == 1 ? 0 : stride_b;
        stride_a *= x;
        stride_b *= y;
    }
    int64_t count = 1;
    for (int i = 0; i < rank; ++i) {
        if (shape[i] != 0 && count > INT64_MAX / 8 / shape[i])
            return fail(HK_INVALID_ARGUMENT, "matmul output is too large");
        count *= shape[i];
    }
    if (s) {
        s->dtype = a->dtype;
        s->m = m;
        s->n = n;
        s->k = k;
        for (hk::MatmulBatch* mb : {&s->batch, &s->a_batch, &s->b_batch}) {
            mb->dims = rank;
            mb->count = count;
            for (int i = 0; i < rank; ++i) mb->shape[i] = shape[i];
        }
        for (int i = 0; i < rank; ++i) {
            s->a_batch.stride[i] = sa[i];
            s->b_batch.stride[i] = sb[i];
        }
    }
    if (out_layout) {
        out_layout->dtype = a->dtype;
        out_layout->rank = rank + 2;
        for (int i = 0; i < rank; ++i) out_layout->shape[i] = shape[i];
        out_layout->shape[rank] = m;
        out_layout->shape[rank + 1] = n;
    }
    return HK_OK;
}

}  // namespace

hk_status hk_matmul_layout(const hk_tensor* a, const hk_tensor* b, hk_tensor* out) {
    // Reference: generic_matrix::output_layout, runtime/generic_matrix.rs:4-15 (host-only).
    if (!out) return fail(HK_INVALID_ARGUMENT, "null output layout");
    hk_tensor layout{};
    hk_status st = matmul_spec(a, b, nullptr, &layout);
    if (st != HK_OK) return st;
    out->dtype = layout.dtype;
    out->rank = layout.rank;
    for (int i = 0; i < HK_MAX_RANK; ++i) out->shape[i] = i < layout.rank ? layout.shape[i] : 0;
    return HK_OK;
}

hk_status hk_tensor_matmul(hk_context* h, const hk_tensor* a, const hk_tensor* b, hk_tensor* out) {
    // Reference: AscendRuntime::tensor_matmul (runtime/mod.rs:156-158) -> generic_matrix::matmul
    // (generic_matrix.rs:17-54) -> AscendState::tensor_matmul (worker.rs:128-162): KEEP_DTYPE.
    hk::MatmulSpec s;
    hk_tensor want{};
    hk_status st = matmul_spec(a, b, &s, &want);
    if (st != HK_OK) return st;
    if (!tensor_ok(out, "out")) return HK_INVALID_ARGUMENT;
    if (out->dtype != want.dtype || !same_shape(out, &want))
        return fail(HK_INVALID_ARGUMENT, "floating matmul resource/layout contract mismatch (output %s %s, want %s %s)",
                    dtype_name(out->dtype), shape_str(out).c_str(), dtype_name(want.dtype), shape_str(&want).c_str());
    if (!disjoint({out}, {a, b})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    if (numel(out) == 0) return HK_OK;
    if ((st = ensure_workspace(g.c, hk::matmul_workspace_bytes(s))) != HK_OK) return st;
    hipError_t e = hk::matmul(s, a->data, b->data, out->data, g.c->workspace, g.c->num_cus, g.c->stream);
    return complete(g.c, e, "tensor_matmul", 5);
}

hk_status hk_tensor_matmul_backward(hk_context* h, const hk_tensor* a, const hk_tensor* b, const hk_tensor* dy,
                                    hk_tensor* da, hk_tensor* db) {
    // The gradients of out = A @ B: dA = dY B^T and dB = A^T dY, each summed over the batch dims its
    // operand broadcasts along (the autodiff rule the reference's float_matmul takes from its
    // tensor library, src/backend.rs:692-703).
    hk::MatmulSpec s;
    hk_tensor want{};
    hk_status st = matmul_spec(a, b, &s, &want);
    if (st != HK_OK) return st;
    if (!tensor_ok(dy, "dY") || !tensor_ok(da, "dA") || !tensor_ok(db, "dB")) return HK_INVALID_ARGUMENT;
    if (dy->dtype != want.dtype || !same_shape(dy, &want))
        return fail(HK_INVALID_ARGUMENT, "matmul backward: dY must be %s %s", dtype_name(want.dtype), shape_str(&want).c_str());
    if (da->dtype != a->dtype || !same_shape(da, a) || db->dtype != b->dtype || !same_shape(db, b))
        return fail(HK_INVALID_ARGUMENT, "matmul backward: dA and dB must match A and B");
    if (!disjoint({da, db}, {a, b, dy})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    if (numel(da) == 0 && numel(db) == 0) return HK_OK;
    if ((st = ensure_workspace(g.c, hk::matmul_backward_workspace_bytes(s))) != HK_OK) return st;
    hipError_t e = hk::matmul_backward(s, a->data, b->data, dy->data, da->data, db->data, g.c->workspace,
                                       g.c->num_cus, g.c->stream);
    return complete(g.c, e, "tensor_matmul_backward", 8);
}

// ------------------------------------------------------------------ module attention pieces

hk_status hk_swap_last_dims(hk_context* h, const hk_tensor* x, hk_tensor* y) {
    // Reference: float_swap_dims(x, rank-2, rank-1) then contiguous() (src/backend.rs:133-140,641).
    if (!tensor_ok(x, "x") || !tensor_ok(y, "y")) return HK_INVALID_ARGUMENT;
    if (x->rank < 2 || y->rank != x->rank || y->dtype != x->dtype)
        return fail(HK_INVALID_ARGUMENT, "swap_last_dims requires rank >= 2 and an output of the same dtype and rank");
    for (int i = 0; i < x->rank - 2; ++i)
        if (y->shape[i] != x->shape[i]) return fail(HK_INVALID_ARGUMENT, "swap_last_dims output shape mismatch");
    const int64_t R = x->shape[x->rank - 2], C = x->shape[x->rank - 1];
    if (y->shape[x->rank - 2] != C || y->shape[x->rank - 1] != R)
        return fail(HK_INVALID_ARGUMENT, "swap_last_dims output shape mismatch");
    if (!disjoint({y}, {x})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    const int64_t n = numel(x);
    if (n == 0) return HK_OK;
    hipError_t e = hk::swap_last_dims(static_cast<int>(dtype_size(x->dtype)), x->data, y->data, n / (R * C), R, C,
                                      g.c->stream);
    return complete(g.c, e, "swap_last_dims", 1);
}

namespace {

// F32 rank-4 scores with an optional F32 bias and HK_BOOL mask broadcast onto them.
hk_status scores_spec(const hk_tensor* s, float scale, float softcap, const hk_tensor* bias, const hk_tensor* mask,
                      int32_t causal, hk::AttnScoreSpec* sp) {
    if (!tensor_ok(s, "scores")) return HK_INVALID_ARGUMENT;
    if (s->dtype != HK_F32 || s->rank != 4)
        return fail(HK_INVALID_ARGUMENT, "attention scores must be F32 [B, H, Sq, Sk], got %s %s", dtype_name(s->dtype),
                    shape_str(s).c_str());
    if (!std::isfinite(scale) || !std::isfinite(softcap) || softcap < 0.0f)
        return fail(HK_INVALID_ARGUMENT, "scale must be finite and softcap finite and >= 0 (0 = none)");
    if (causal != 0 && causal != 1) return fail(HK_INVALID_ARGUMENT, "causal must be 0 or 1");
    auto strides = [&](const hk_tensor* t, const char* what, int64_t (&st)[4]) {
        int64_t run = 1;
        for (int k = 3; k >= 0; --k) {
            if (t->shape[k] != s->shape[k] && t->shape[k] != 1) {
                fail(HK_INVALID_ARGUMENT, "attention %s %s does not broadcast onto the scores %s", what,
                     shape_str(t).c_str(), shape_str(s).c_str());
                return false;
            }
            st[k] = t->shape[k] == 1 ? 0 : run;
            run *= t->shape[k];
        }
        return true;
    };
    for (int k = 0; k < 4; ++k) sp->shape[k] = s->shape[k];
    if (bias) {
        if (!tensor_ok(bias, "bias")) return HK_INVALID_ARGUMENT;
        if (bias->dtype != HK_F32 || bias->rank != 4) return fail(HK_INVALID_ARGUMENT, "attention bias must be F32 rank 4");
        if (!strides(bias, "bias", sp->bias_stride)) return HK_INVALID_ARGUMENT;
    }
    if (mask) {
        if (mask->dtype != HK_BOOL || mask->rank != 4 || numel(mask) < 0 ||
            (numel(mask) > 0 && mask->data == nullptr))
            return fail(HK_INVALID_ARGUMENT, "attention mask must be a BOOL rank-4 tensor");
        if (!strides(mask, "mask", sp->mask_stride)) return HK_INVALID_ARGUMENT;
    }
    sp->scale = scale;
    sp->softcap = softcap;
    sp->causal = causal;
    return HK_OK;
}

}  // namespace

hk_status hk_attention_scores(hk_context* h, const hk_tensor* s, float scale, float softcap, const hk_tensor* bias,
                              const hk_tensor* mask, int32_t causal, hk_tensor* out) {
    hk::AttnScoreSpec sp;
    hk_status st = scores_spec(s, scale, softcap, bias, mask, causal, &sp);
    if (st != HK_OK) return st;
    if (!tensor_ok(out, "out")) return HK_INVALID_ARGUMENT;
    if (out->dtype != HK_F32 || !same_shape(out, s)) return fail(HK_INVALID_ARGUMENT, "scores output must match the scores");
    if (!disjoint({out}, {s}) || (bias && !disjoint({out}, {bias})) || (mask && !disjoint({out}, {mask})))
        return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    hipError_t e = hk::attention_scores(sp, static_cast<const float*>(s->data), static_cast<float*>(out->data),
                                        bias ? static_cast<const float*>(bias->data) : nullptr,
                                        mask ? static_cast<const uint8_t*>(mask->data) : nullptr, g.c->stream);
    return complete(g.c, e, "attention_scores", 1);
}

hk_status hk_attention_scores_backward(hk_context* h, const hk_tensor* s, const hk_tensor* dout, float scale,
                                       float softcap, const hk_tensor* mask, int32_t causal, hk_tensor* ds,
                                       hk_tensor* dbias) {
    hk::AttnScoreSpec sp;
    hk_status st = scores_spec(s, scale, softcap, nullptr, mask, causal, &sp);
    if (st != HK_OK) return st;
    if (!tensor_ok(dout, "dout") || !tensor_ok(ds, "ds")) return HK_INVALID_ARGUMENT;
    if (dout->dtype != HK_F32 || !same_shape(dout, s) || ds->dtype != HK_F32 || !same_shape(ds, s))
        return fail(HK_INVALID_ARGUMENT, "dout and ds must be F32 shaped like the scores");
    int64_t bias_shape[4] = {1, 1, 1, 1};
    if (dbias) {
        if (!tensor_ok(dbias, "dbias")) return HK_INVALID_ARGUMENT;
        if (dbias->dtype != HK_F32 || dbias->rank != 4) return fail(HK_INVALID_ARGUMENT, "dbias must be F32 rank 4");
        for (int k = 0; k < 4; ++k) {
            if (dbias->shape[k] != s->shape[k] && dbias->shape[k] != 1)
                return fail(HK_INVALID_ARGUMENT, "dbias %s does not broadcast onto the scores %s", shape_str(dbias).c_str(),
                            shape_str(s).c_str());
            bias_shape[k] = dbias->shape[k];
        }
    }
    if (!disjoint({ds}, {s, dout}) || (dbias && !disjoint({ds, dbias}, {s, dout})) ||
        (mask && !disjoint({ds}, {mask})) || (mask && dbias && !disjoint({dbias}, {mask})))
        return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    if (dbias && (st = ensure_workspace(g.c, static_cast<size_t>(numel(s)) * sizeof(float))) != HK_OK) return st;
    hipError_t e = hk::attention_scores_backward(
        sp, static_cast<const float*>(s->data), static_cast<const float*>(dout->data), static_cast<float*>(ds->data),
        mask ? static_cast<const uint8_t*>(mask->data) : nullptr, dbias ? static_cast<float*>(dbias->data) : nullptr,
        bias_shape, static_cast<float*>(g.c->workspace), g.c->stream);
    return complete(g.c, e, "attention_scores_backward", dbias ? 2 : 1);
}

hk_status hk_linear_nt_backward(hk_context* h, const hk_tensor* x, const hk_tensor* w, const hk_tensor* dy,
                                hk_tensor* dx, hk_tensor* dw) {
    // Reference: matrix.rs:60-74.
    GemmSpec fwd, sdx, sdw;
    hk_status st = gemm_spec(x, w, HK_NO, HK_YES, HK_BF16, &fwd);
    if (st != HK_OK) return st;
    if (!tensor_ok(dy, "dY") || !tensor_ok(dx, "dX") || !tensor_ok(dw, "dW")) return HK_INVALID_ARGUMENT;
    if (fwd.kind != 0 || !out_matches(fwd, dy))
        return fail(HK_INVALID_ARGUMENT, "linear backward requires rank-2 BF16 dY matching X @ W^T");
    if ((st = gemm_spec(dy, w, HK_NO, HK_NO, HK_BF16, &sdx)) != HK_OK) return st;
    if ((st = gemm_spec(dy, x, HK_YES, HK_NO, HK_F32, &sdw)) != HK_OK) return st;
    if (!out_matches(sdx, dx)) return fail(HK_INVALID_ARGUMENT, "dX must be BF16 shaped like X");
    if (!out_matches(sdw, dw)) return fail(HK_INVALID_ARGUMENT, "dW must be F32 shaped like W");
    if (!disjoint({dx, dw}, {x, w, dy})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    size_t ws = std::max(hk::gemm_workspace_bytes(1, sdx.m, sdx.n, sdx.k, HK_NO, HK_NO),
                         hk::gemm_workspace_bytes(1, sdw.m, sdw.n, sdw.k, HK_YES, HK_NO));
    if ((st = ensure_workspace(g.c, ws)) != HK_OK) return st;
    hipError_t e;
    run_gemm(g.c, sdx, dy->data, w->data, dx->data, HK_NO, HK_NO, g.c->workspace, &e);
    if (e == hipSuccess) run_gemm(g.c, sdw, dy->data, x->data, dw->data, HK_YES, HK_NO, g.c->workspace, &e);
    return complete(g.c, e, "linear_nt_backward", 2);
}

hk_status hk_gemm_bf16_fp32(hk_context* h, const hk_tensor* a, const hk_tensor* b, int32_t ta, int32_t tb,
                            hk_tensor* out, hk_tensor* a_bf16, hk_tensor* b_bf16) {
    // Reference: matrix.rs:84-93 (cast both inputs into independent snapshots, then GEMM).
    GemmSpec s;
    hk_status st = mixed_spec(a, b, ta, tb, &s);
    if (st != HK_OK) return st;
    if (!tensor_ok(out, "out") || !tensor_ok(a_bf16, "A_bf16") || !tensor_ok(b_bf16, "B_bf16")) return HK_INVALID_ARGUMENT;
    if (!out_matches(s, out)) return fail(HK_INVALID_ARGUMENT, "output must be F32 %s", shape_str(out).c_str());
    if (!is_bf16_copy_of(a_bf16, a) || !is_bf16_copy_of(b_bf16, b))
        return fail(HK_INVALID_ARGUMENT, "BF16 snapshots must match the inputs' shapes");
    if (!disjoint({out, a_bf16, b_bf16}, {a, b})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    if ((st = ensure_workspace(g.c, hk::gemm_workspace_bytes(s.batch, s.m, s.n, s.k, ta, tb))) != HK_OK) return st;
    hipError_t e = hk::cast_apply(1, a->data, a_bf16->data, numel(a), g.c->stream);
    if (e == hipSuccess) e = hk::cast_apply(1, b->data, b_bf16->data, numel(b), g.c->stream);
    if (e == hipSuccess) run_gemm(g.c, s, a_bf16->data, b_bf16->data, out->data, ta, tb, g.c->workspace, &e);
    return complete(g.c, e, "gemm_bf16_fp32", 3);
}

hk_status hk_gemm_bf16_fp32_backward(hk_context* h, const hk_tensor* a, const hk_tensor* b, const hk_tensor* dy,
                                     int32_t ta, int32_t tb, hk_tensor* da, hk_tensor* db) {
    // Reference: matrix.rs:95-121.
    GemmSpec fwd;
    hk_status st = gemm_spec(a, b, ta, tb, HK_F32, &fwd);
    if (st != HK_OK) return st;
    if (!tensor_ok(dy, "dY") || !tensor_ok(da, "dA") || !tensor_ok(db, "dB")) return HK_INVALID_ARGUMENT;
    if (!out_matches(fwd, dy))
        return fail(HK_INVALID_ARGUMENT, "BF16-compute matmul backward requires saved BF16 inputs and matching FP32 dY");
    if (da->dtype != HK_F32 || !same_shape(da, a) || db->dtype != HK_F32 || !same_shape(db, b))
        return fail(HK_INVALID_ARGUMENT, "gradients must be F32 in the inputs' physical shapes");
    if (!disjoint({da, db}, {a, b, dy})) return HK_INVALID_ARGUMENT;
    // dY rounded to BF16 in the workspace head, GEMM workspace after it.
    hk_tensor dyb = *dy;
    dyb.dtype = HK_BF16;
    const int opp_ta = ta == HK_NO ? HK_YES : HK_NO;
    const int opp_tb = tb == HK_NO ? HK_YES : HK_NO;
    // dX: ta == No -> dY . op'(B) ; else B . dY^T   (matrix.rs:104-105)
    const hk_tensor *dx_a = ta == HK_NO ? &dyb : b, *dx_b = ta == HK_NO ? b : &dyb;
    const int dx_ta = ta == HK_NO ? HK_NO : tb, dx_tb = ta == HK_NO ? opp_tb : HK_YES;
    // dW: tb == No -> op'(A) . dY ; else dY^T . A   (matrix.rs:106-107)
    const hk_tensor *dw_a = tb == HK_NO ? a : &dyb, *dw_b = tb == HK_NO ? &dyb : a;
    const int dw_ta = tb == HK_NO ? opp_ta : HK_YES, dw_tb = tb == HK_NO ? HK_NO : ta;
    GemmSpec sdx, sdw;
    if ((st = gemm_spec(dx_a, dx_b, dx_ta, dx_tb, HK_F32, &sdx)) != HK_OK) return st;
    if ((st = gemm_spec(dw_a, dw_b, dw_ta, dw_tb, HK_F32, &sdw)) != HK_OK) return st;
    const size_t dy_bytes = (static_cast<size_t>(numel(dy)) * 2 + 255) & ~size_t(255);
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    const size_t ws = dy_bytes + std::max(hk::gemm_workspace_bytes(sdx.batch, sdx.m, sdx.n, sdx.k, dx_ta, dx_tb),
                                          hk::gemm_workspace_bytes(sdw.batch, sdw.m, sdw.n, sdw.k, dw_ta, dw_tb));
    if ((st = ensure_workspace(g.c, ws)) != HK_OK) return st;
    void* dyb_ptr = g.c->workspace;
    void* gws = static_cast<char*>(g.c->workspace) + dy_bytes;
    dyb.data = dyb_ptr;
    hipError_t e = hk::cast_apply(1, dy->data, dyb_ptr, numel(dy), g.c->stream);
    if (e == hipSuccess) run_gemm(g.c, sdx, dx_a->data, dx_b->data, da->data, dx_ta, dx_tb, gws, &e);
    if (e == hipSuccess) run_gemm(g.c, sdw, dw_a->data, dw_b->data, db->data, dw_ta, dw_tb, gws, &e);
    return complete(g.c, e, "gemm_bf16_fp32_backward", 3);
}

hk_status hk_linear_bf16_fp32(hk_context* h, const hk_tensor* x, const hk_tensor* w, hk_tensor* y,
                              hk_tensor* x_bf16, hk_tensor* w_bf16) {
    // Reference: matrix.rs:123-133 (rank-2 check, then gemm_bf16_fp32 NT).
    if (!tensor_ok(x, "X") || !tensor_ok(w, "W")) return HK_INVALID_ARGUMENT;
    if (x->rank != 2 || w->rank != 2)
        return fail(HK_INVALID_ARGUMENT, "BF16-compute FP32 linear requires rank-2 input and weight");
    return hk_gemm_bf16_fp32(h, x, w, HK_NO, HK_YES, y, x_bf16, w_bf16);
}

hk_status hk_linear_bf16_fp32_backward(hk_context* h, const hk_tensor* x, const hk_tensor* w, const hk_tensor* dy,
                                       hk_tensor* dx, hk_tensor* dw) {
    // Reference: matrix.rs:134-145.
    if (!tensor_ok(x, "X") || !tensor_ok(w, "W")) return HK_INVALID_ARGUMENT;
    if (x->rank != 2 || w->rank != 2)
        return fail(HK_INVALID_ARGUMENT, "BF16-compute linear backward requires saved rank-2 inputs");
    return hk_gemm_bf16_fp32_backward(h, x, w, dy, HK_NO, HK_YES, dx, dw);
}

namespace {
// Reference: frozen_linear_spec, matrix.rs:147-153: rank-2 F32 X, fixed rank-2 BF16 W, NT, F32 out.
hk_status frozen_spec(const hk_tensor* x, const hk_tensor* w, GemmSpec* s) {
    if (!tensor_ok(x, "X") || !tensor_ok(w, "W")) return HK_INVALID_ARGUMENT;
    if (x->rank != 2 || w->rank != 2 || x->dtype != HK_F32 || w->dtype != HK_BF16)
        return fail(HK_INVALID_ARGUMENT, "frozen BF16 linear requires rank-2 FP32 input and fixed BF16 weight");
    hk_tensor xb = *x;
    xb.dtype = HK_BF16;
    return gemm_spec(&xb, w, HK_NO, HK_YES, HK_F32, s);
}
}  // namespace

hk_status hk_linear_frozen_bf16_fp32(hk_context* h, const hk_tensor* x, const hk_tensor* w, hk_tensor* y) {
    // Reference: matrix.rs:154-159: X rounded to BF16 on the device, the fixed W used in place.
    GemmSpec s;
    hk_status st = frozen_spec(x, w, &s);
    if (st != HK_OK) return st;
    if (!tensor_ok(y, "Y")) return HK_INVALID_ARGUMENT;
    if (!out_matches(s, y)) return fail(HK_INVALID_ARGUMENT, "output must be F32 [%lld,%lld]", (long long)s.m, (long long)s.n);
    if (!disjoint({y}, {x, w})) return HK_INVALID_ARGUMENT;
    const size_t x_bytes = (static_cast<size_t>(numel(x)) * 2 + 255) & ~size_t(255);
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    if ((st = ensure_workspace(g.c, x_bytes + hk::gemm_workspace_bytes(1, s.m, s.n, s.k, HK_NO, HK_YES))) != HK_OK)
        return st;
    void* xb = g.c->workspace;
    hipError_t e = hk::cast_apply(1, x->data, xb, numel(x), g.c->stream);
    if (e == hipSuccess)
        run_gemm(g.c, s, xb, w->data, y->data, HK_NO, HK_YES, static_cast<char*>(g.c->workspace) + x_bytes, &e);
    return complete(g.c, e, "linear_frozen_bf16_fp32", 2);
}

hk_status hk_linear_frozen_bf16_fp32_backward(hk_context* h, const hk_tensor* w, const hk_tensor* dy, hk_tensor* dx) {
    // Reference: matrix.rs:160-172: dX = bf16(dY) W (NN, F32 out); the weight gets no gradient.
    if (!tensor_ok(w, "W") || !tensor_ok(dy, "dY") || !tensor_ok(dx, "dX")) return HK_INVALID_ARGUMENT;
    if (dx->rank != 2 || dx->dtype != HK_F32)
        return fail(HK_INVALID_ARGUMENT, "frozen BF16 linear input gradient must be rank-2 FP32");
    GemmSpec fwd;
    hk_status st = frozen_spec(dx, w, &fwd);
    if (st != HK_OK) return st;
    if (!out_matches(fwd, dy)) return fail(HK_INVALID_ARGUMENT, "frozen BF16 linear backward requires matching FP32 dY");
    hk_tensor dyb = *dy;
    dyb.dtype = HK_BF16;
    GemmSpec s;
    if ((st = gemm_spec(&dyb, w, HK_NO, HK_NO, HK_F32, &s)) != HK_OK) return st;
    if (!out_matches(s, dx)) return fail(HK_INVALID_ARGUMENT, "frozen BF16 linear input gradient shape mismatch");
    if (!disjoint({dx}, {w, dy})) return HK_INVALID_ARGUMENT;
    const size_t dy_bytes = (static_cast<size_t>(numel(dy)) * 2 + 255) & ~size_t(255);
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    if ((st = ensure_workspace(g.c, dy_bytes + hk::gemm_workspace_bytes(1, s.m, s.n, s.k, HK_NO, HK_NO))) != HK_OK)
        return st;
    void* dyb_ptr = g.c->workspace;
    hipError_t e = hk::cast_apply(1, dy->data, dyb_ptr, numel(dy), g.c->stream);
    if (e == hipSuccess)
        run_gemm(g.c, s, dyb_ptr, w->data, dx->data, HK_NO, HK_NO, static_cast<char*>(g.c->workspace) + dy_bytes, &e);
    return complete(g.c, e, "linear_frozen_bf16_fp32_backward", 2);
}

// ------------------------------------------------------------------ padded GEMM

namespace {

int64_t round16(int64_t x) { return (x + 15) / 16 * 16; }

// Reference: PaddedGemmSpec::new, deepgemm/padded.rs:13-36. The matrix axes of A and B are
// rounded up to multiples of 16 (the "native" BF16 layouts); the logical output is F32.
struct PaddedSpec {
    int rank = 2;
    int64_t batch = 1, m = 0, n = 0, k = 0;
    int64_t a_rows = 0, a_cols = 0, b_rows = 0, b_cols = 0;  // physical matrix axes
    hk_tensor a_pad{}, b_pad{};                              // native BF16 layouts (data unset)
    GemmSpec native;
};

hk_status padded_spec(const hk_tensor* a, const hk_tensor* b, int32_t ta, int32_t tb, PaddedSpec* p) {
    if (!tensor_ok(a, "A") || !tensor_ok(b, "B")) return HK_INVALID_ARGUMENT;
    if ((ta != HK_NO && ta != HK_YES) || (tb != HK_NO && tb != HK_YES))
        return fail(HK_INVALID_ARGUMENT, "transpose flags must be 0 (No) or 1 (Yes)");
    const int r = a->rank;
    if (!(r == 2 || r == 3) || b->rank != r || !(a->dtype == HK_F32 || a->dtype == HK_BF16) ||
        !(b->dtype == HK_F32 || b->dtype == HK_BF16))
        return fail(HK_INVALID_ARGUMENT, "padded GEMM requires matching rank-2/3 FP32/BF16 inputs");
    if (r == 3 && a->shape[0] != b->shape[0]) return fail(HK_INVALID_ARGUMENT, "padded GEMM does not broadcast batches");
    const int64_t *a2 = a->shape + (r - 2), *b2 = b->shape + (r - 2);
    const int64_t m = ta == HK_NO ? a2[0] : a2[1], k = ta == HK_NO ? a2[1] : a2[0];
    const int64_t kb = tb == HK_NO ? b2[0] : b2[1], n = tb == HK_NO ? b2[1] : b2[0];
    if (k != kb) return fail(HK_INVALID_ARGUMENT, "padded GEMM logical contraction mismatch");
    p->a_pad = *a;
    p->b_pad = *b;
    for (hk_tensor* t : {&p->a_pad, &p->b_pad}) {
        t->dtype = HK_BF16;
        t->data = reinterpret_cast<void*>(uintptr_t{256});  // layout only; never dereferenced
        for (int i = r - 2; i < r; ++i) {
            if (t->shape[i] <= 0) return fail(HK_INVALID_ARGUMENT, "padded GEMM matrix axes must be positive");
            if (round16(t->shape[i]) > INT32_MAX) return fail(HK_INVALID_ARGUMENT, "padded GEMM aligned axis exceeds INT32_MAX");
            t->shape[i] = round16(t->shape[i]);
        }
    }
    hk_status st = gemm_spec(&p->a_pad, &p->b_pad, ta, tb, HK_F32, &p->native);
    if (st != HK_OK) return st;
    p->rank = r;
    p->batch = r == 3 ? a->shape[0] : 1;
    p->m = m;
    p->n = n;
    p->k = k;
    p->a_rows = a2[0];
    p->a_cols = a2[1];
    p->b_rows = b2[0];
    p->b_cols = b2[1];
    return HK_OK;
}

bool is_logical_out(const PaddedSpec& p, const hk_tensor* t) {
    if (t->dtype != HK_F32 || t->rank != p.rank) return false;
    const int64_t* s = t->shape + (p.rank - 2);
    return (p.rank == 2 || t->shape[0] == p.batch) && s[0] == p.m && s[1] == p.n;
}

bool same_layout(const hk_tensor* t, const hk_tensor& want) { return t->dtype == want.dtype && same_shape(t, &want); }

size_t ws_round(size_t x) { return (x + 255) & ~size_t(255); }

}  // namespace

hk_status hk_gemm_padded_bf16_fp32(hk_context* h, const hk_tensor* a, const hk_tensor* b, int32_t ta, int32_t tb,
                                   hk_tensor* out, hk_tensor* a_pad, hk_tensor* b_pad) {
    // Reference: padded_matrix::forward, runtime/padded_matrix.rs:39-46.
    PaddedSpec p;
    hk_status st = padded_spec(a, b, ta, tb, &p);
    if (st != HK_OK) return st;
    if (a->dtype != HK_F32 || b->dtype != HK_F32)
        return fail(HK_INVALID_ARGUMENT, "padded trainable matmul requires FP32 inputs");
    if (!tensor_ok(out, "out") || !tensor_ok(a_pad, "A_pad") || !tensor_ok(b_pad, "B_pad")) return HK_INVALID_ARGUMENT;
    if (!is_logical_out(p, out)) return fail(HK_INVALID_ARGUMENT, "output must be F32 of the logical shape");
    if (!same_layout(a_pad, p.a_pad) || !same_layout(b_pad, p.b_pad))
        return fail(HK_INVALID_ARGUMENT, "padded snapshots must be BF16 with matrix axes rounded up to 16");
    if (!disjoint({out, a_pad, b_pad}, {a, b})) return HK_INVALID_ARGUMENT;
    const GemmSpec& s = p.native;
    const bool crop = s.m != p.m || s.n != p.n;
    const size_t out_bytes = crop ? ws_round(static_cast<size_t>(s.batch * s.m * s.n) * 4) : 0;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    if ((st = ensure_workspace(g.c, out_bytes + hk::gemm_workspace_bytes(s.batch, s.m, s.n, s.k, ta, tb))) != HK_OK)
        return st;
    float* native_out = crop ? static_cast<float*>(g.c->workspace) : static_cast<float*>(out->data);
    void* gws = static_cast<char*>(g.c->workspace) + out_bytes;
    const int64_t ar = p.a_pad.shape[p.rank - 2], ac = p.a_pad.shape[p.rank - 1];
    const int64_t br = p.b_pad.shape[p.rank - 2], bc = p.b_pad.shape[p.rank - 1];
    hipError_t e = hk::pad_bf16(0, a->data, a_pad->data, p.batch, p.a_rows, p.a_cols, ar, ac, g.c->stream);
    if (e == hipSuccess) e = hk::pad_bf16(0, b->data, b_pad->data, p.batch, p.b_rows, p.b_cols, br, bc, g.c->stream);
    if (e == hipSuccess) run_gemm(g.c, s, a_pad->data, b_pad->data, native_out, ta, tb, gws, &e);
    if (e == hipSuccess && crop)
        e = hk::crop_f32(native_out, static_cast<float*>(out->data), p.batch, p.m, p.n, s.m, s.n, g.c->stream);
    return complete(g.c, e, "gemm_padded_bf16_fp32", crop ? 4 : 3);
}

hk_status hk_gemm_padded_bf16_fp32_backward(hk_context* h, const hk_tensor* a_pad, const hk_tensor* b_pad,
                                            const hk_tensor* dy, int32_t ta, int32_t tb, hk_tensor* da,
                                            hk_tensor* db) {
    // Reference: padded_matrix::backward, runtime/padded_matrix.rs:47-63, and
    // PaddedGemmSpec::backward_specs, deepgemm/padded.rs:39-50. da/db carry the original
    // physical input shapes (the reference's a_shape/b_shape).
    if (!tensor_ok(da, "dA") || !tensor_ok(db, "dB")) return HK_INVALID_ARGUMENT;
    if (da->dtype != HK_F32 || db->dtype != HK_F32) return fail(HK_INVALID_ARGUMENT, "padded gradients are F32");
    PaddedSpec p;
    hk_status st = padded_spec(da, db, ta, tb, &p);
    if (st != HK_OK) return st;
    if (!tensor_ok(a_pad, "A_pad") || !tensor_ok(b_pad, "B_pad") || !tensor_ok(dy, "dY")) return HK_INVALID_ARGUMENT;
    if (!same_layout(a_pad, p.a_pad) || !same_layout(b_pad, p.b_pad) || !is_logical_out(p, dy))
        return fail(HK_INVALID_ARGUMENT, "padded matmul backward saved input or logical dY layout mismatch");
    if (!disjoint({da, db}, {a_pad, b_pad, dy})) return HK_INVALID_ARGUMENT;
    const GemmSpec& s = p.native;
    hk_tensor dyp{};  // dY rounded to BF16 and padded to [batch, M16, N16]
    dyp.dtype = HK_BF16;
    dyp.rank = p.rank;
    dyp.data = reinterpret_cast<void*>(uintptr_t{256});
    if (p.rank == 3) dyp.shape[0] = p.batch;
    dyp.shape[p.rank - 2] = s.m;
    dyp.shape[p.rank - 1] = s.n;
    const int opp_ta = ta == HK_NO ? HK_YES : HK_NO, opp_tb = tb == HK_NO ? HK_YES : HK_NO;
    const hk_tensor *da_a = ta == HK_NO ? &dyp : b_pad, *da_b = ta == HK_NO ? b_pad : &dyp;
    const int da_ta = ta == HK_NO ? HK_NO : tb, da_tb = ta == HK_NO ? opp_tb : HK_YES;
    const hk_tensor *db_a = tb == HK_NO ? a_pad : &dyp, *db_b = tb == HK_NO ? &dyp : a_pad;
    const int db_ta = tb == HK_NO ? opp_ta : HK_YES, db_tb = tb == HK_NO ? HK_NO : ta;
    GemmSpec sda, sdb;
    if ((st = gemm_spec(da_a, da_b, da_ta, da_tb, HK_F32, &sda)) != HK_OK) return st;
    if ((st = gemm_spec(db_a, db_b, db_ta, db_tb, HK_F32, &sdb)) != HK_OK) return st;
    const bool crop_a = !same_shape(da, &p.a_pad), crop_b = !same_shape(db, &p.b_pad);
    const size_t dy_bytes = ws_round(static_cast<size_t>(s.batch * s.m * s.n) * 2);
    const size_t pa_bytes = crop_a ? ws_round(static_cast<size_t>(numel(&p.a_pad)) * 4) : 0;
    const size_t pb_bytes = crop_b ? ws_round(static_cast<size_t>(numel(&p.b_pad)) * 4) : 0;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    const size_t gws_bytes = std::max(hk::gemm_workspace_bytes(sda.batch, sda.m, sda.n, sda.k, da_ta, da_tb),
                                      hk::gemm_workspace_bytes(sdb.batch, sdb.m, sdb.n, sdb.k, db_ta, db_tb));
    if ((st = ensure_workspace(g.c, dy_bytes + pa_bytes + pb_bytes + gws_bytes)) != HK_OK) return st;
    char* w = static_cast<char*>(g.c->workspace);
    dyp.data = w;
    float* pa = crop_a ? reinterpret_cast<float*>(w + dy_bytes) : static_cast<float*>(da->data);
    float* pb = crop_b ? reinterpret_cast<float*>(w + dy_bytes + pa_bytes) : static_cast<float*>(db->data);
    void* gws = w + dy_bytes + pa_bytes + pb_bytes;
    int kernels = 3;
    hipError_t e = hk::pad_bf16(0, dy->data, dyp.data, p.batch, p.m, p.n, s.m, s.n, g.c->stream);
    if (e == hipSuccess) run_gemm(g.c, sda, da_a->data, da_b->data, pa, da_ta, da_tb, gws, &e);
    if (e == hipSuccess) run_gemm(g.c, sdb, db_a->data, db_b->data, pb, db_ta, db_tb, gws, &e);
    const int64_t ar = p.a_pad.shape[p.rank - 2], ac = p.a_pad.shape[p.rank - 1];
    const int64_t br = p.b_pad.shape[p.rank - 2], bc = p.b_pad.shape[p.rank - 1];
    if (e == hipSuccess && crop_a) {
        e = hk::crop_f32(pa, static_cast<float*>(da->data), p.batch, p.a_rows, p.a_cols, ar, ac, g.c->stream);
        ++kernels;
    }
    if (e == hipSuccess && crop_b) {
        e = hk::crop_f32(pb, static_cast<float*>(db->data), p.batch, p.b_rows, p.b_cols, br, bc, g.c->stream);
        ++kernels;
    }
    return complete(g.c, e, "gemm_padded_bf16_fp32_backward", kernels);
}

hk_status hk_linear_frozen_padded_bf16_fp32(hk_context* h, const hk_tensor* x, const hk_tensor* w, hk_tensor* y,
                                            hk_tensor* w_pad) {
    // Reference: padded_matrix::frozen_forward, runtime/padded_matrix.rs:64-76.
    if (!tensor_ok(x, "input") || !tensor_ok(w, "weight")) return HK_INVALID_ARGUMENT;
    if (x->rank != 2 || w->rank != 2 || x->dtype != HK_F32 || w->dtype != HK_BF16)
        return fail(HK_INVALID_ARGUMENT, "frozen padded linear requires rank-2 FP32 input and fixed BF16 weight");
    PaddedSpec p;
    hk_status st = padded_spec(x, w, HK_NO, HK_YES, &p);
    if (st != HK_OK) return st;
    if (!tensor_ok(y, "out")) return HK_INVALID_ARGUMENT;
    if (!is_logical_out(p, y)) return fail(HK_INVALID_ARGUMENT, "output must be F32 [M,N]");
    const bool w_tail = !same_shape(w, &p.b_pad);
    if (w_pad) {
        if (!tensor_ok(w_pad, "W_pad") || !same_layout(w_pad, p.b_pad))
            return fail(HK_INVALID_ARGUMENT, "padded weight must be BF16 with both axes rounded up to 16");
        if (!disjoint({y, w_pad}, {x, w})) return HK_INVALID_ARGUMENT;
    } else if (!disjoint({y}, {x, w})) {
        return HK_INVALID_ARGUMENT;
    }
    const GemmSpec& s = p.native;
    const bool crop = s.m != p.m || s.n != p.n;
    const size_t xb = ws_round(static_cast<size_t>(s.m * s.k) * 2);
    const size_t wb = (w_tail && !w_pad) ? ws_round(static_cast<size_t>(s.n * s.k) * 2) : 0;
    const size_t ob = crop ? ws_round(static_cast<size_t>(s.m * s.n) * 4) : 0;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    if ((st = ensure_workspace(g.c, xb + wb + ob + hk::gemm_workspace_bytes(1, s.m, s.n, s.k, HK_NO, HK_YES))) != HK_OK)
        return st;
    char* ws = static_cast<char*>(g.c->workspace);
    void* xpad = ws;
    // aligned weights are used in place (reference: "aligned weights reuse their actual handle")
    const void* wuse = w->data;
    int kernels = 2;
    hipError_t e = hk::pad_bf16(0, x->data, xpad, 1, p.m, p.k, s.m, s.k, g.c->stream);
    if (e == hipSuccess && (w_tail || w_pad)) {
        void* wdst = w_pad ? w_pad->data : ws + xb;
        e = hk::pad_bf16(1, w->data, wdst, 1, p.n, p.k, s.n, s.k, g.c->stream);
        wuse = wdst;
        ++kernels;
    }
    float* native_out = crop ? reinterpret_cast<float*>(ws + xb + wb) : static_cast<float*>(y->data);
    if (e == hipSuccess) run_gemm(g.c, s, xpad, wuse, native_out, HK_NO, HK_YES, ws + xb + wb + ob, &e);
    if (e == hipSuccess && crop) {
        e = hk::crop_f32(native_out, static_cast<float*>(y->data), 1, p.m, p.n, s.m, s.n, g.c->stream);
        ++kernels;
    }
    return complete(g.c, e, "linear_frozen_padded_bf16_fp32", kernels);
}

hk_status hk_linear_frozen_padded_bf16_fp32_backward(hk_context* h, const hk_tensor* w_pad, const hk_tensor* dy,
                                                     hk_tensor* dx) {
    // Reference: padded_matrix::frozen_backward, runtime/padded_matrix.rs:77-87. The logical
    // input shape is dx's; the logical weight shape is [dy's N, dx's K].
    if (!tensor_ok(w_pad, "weight") || !tensor_ok(dy, "dY") || !tensor_ok(dx, "dX")) return HK_INVALID_ARGUMENT;
    if (dx->rank != 2 || dy->rank != 2 || w_pad->rank != 2)
        return fail(HK_INVALID_ARGUMENT, "frozen padded linear backward requires rank-2 shapes");
    if (dx->dtype != HK_F32) return fail(HK_INVALID_ARGUMENT, "dX must be F32");
    hk_tensor wl = *w_pad;  // the logical weight layout [N, K]
    wl.shape[0] = dy->shape[1];
    wl.shape[1] = dx->shape[1];
    wl.dtype = HK_BF16;
    PaddedSpec p;
    hk_status st = padded_spec(dx, &wl, HK_NO, HK_YES, &p);
    if (st != HK_OK) return st;
    if (!same_layout(w_pad, p.b_pad) || !is_logical_out(p, dy))
        return fail(HK_INVALID_ARGUMENT, "frozen padded linear saved weight or dY layout mismatch");
    if (!disjoint({dx}, {w_pad, dy})) return HK_INVALID_ARGUMENT;
    const GemmSpec& s = p.native;
    hk_tensor dyp = make_view(reinterpret_cast<void*>(uintptr_t{256}), HK_BF16, {s.m, s.n});
    GemmSpec sdx;
    if ((st = gemm_spec(&dyp, w_pad, HK_NO, HK_NO, HK_F32, &sdx)) != HK_OK) return st;
    const bool crop = s.m != p.m || s.k != p.k;
    const size_t db = ws_round(static_cast<size_t>(s.m * s.n) * 2);
    const size_t ob = crop ? ws_round(static_cast<size_t>(s.m * s.k) * 4) : 0;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    if ((st = ensure_workspace(g.c, db + ob + hk::gemm_workspace_bytes(1, sdx.m, sdx.n, sdx.k, HK_NO, HK_NO))) != HK_OK)
        return st;
    char* ws = static_cast<char*>(g.c->workspace);
    float* native_out = crop ? reinterpret_cast<float*>(ws + db) : static_cast<float*>(dx->data);
    hipError_t e = hk::pad_bf16(0, dy->data, ws, 1, p.m, p.n, s.m, s.n, g.c->stream);
    if (e == hipSuccess) run_gemm(g.c, sdx, ws, w_pad->data, native_out, HK_NO, HK_NO, ws + db + ob, &e);
    if (e == hipSuccess && crop)
        e = hk::crop_f32(native_out, static_cast<float*>(dx->data), 1, p.m, p.k, s.m, s.k, g.c->stream);
    return complete(g.c, e, "linear_frozen_padded_bf16_fp32_backward", crop ? 3 : 2);
}

hk_status hk_cast_into(hk_context* h, const hk_tensor* in, hk_tensor* out) {
    // Reference: conversion.rs:21-62 (shape retained, distinct output storage).
    if (!tensor_ok(in, "input") || !tensor_ok(out, "output")) return HK_INVALID_ARGUMENT;
    if (!same_shape(in, out)) return fail(HK_INVALID_ARGUMENT, "cast output shape mismatch");
    const bool f2b = in->dtype == HK_F32 && out->dtype == HK_BF16;
    const bool b2f = in->dtype == HK_BF16 && out->dtype == HK_F32;
    if (!f2b && !b2f) return fail(HK_INVALID_ARGUMENT, "cast supports F32 <-> BF16");
    if (!disjoint({out}, {in})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    hipError_t e = hk::cast_apply(f2b ? 1 : 0, in->data, out->data, numel(in), g.c->stream);
    return complete(g.c, e, "cast", 1);
}

// ------------------------------------------------------------------ RMSNorm

namespace {
// Reference: elementwise.rs:5-11 (check_for: contiguous, one shape; element count <= u32).
static bool gate_shapes(std::initializer_list<const hk_tensor*> ts, const char* op) {
    const hk_tensor* first = *ts.begin();
    if (first->dtype != HK_F32 && first->dtype != HK_BF16)
        return fail(HK_INVALID_ARGUMENT, "%s requires F32 or BF16 tensors", op), false;
    for (const hk_tensor* t : ts)
        if (t->dtype != first->dtype || !same_shape(t, first))
            return fail(HK_INVALID_ARGUMENT, "%s requires tensors of one dtype and shape", op), false;
    if (numel(first) > static_cast<int64_t>(UINT32_MAX))
        return fail(HK_INVALID_ARGUMENT, "%s element count exceeds u32", op), false;
    return true;
}
}  // namespace

hk_status hk_silu_mul(hk_context* h, const hk_tensor* gate, const hk_tensor* up, hk_tensor* y) {
    // Reference: elementwise.rs:13-19.
    if (!tensor_ok(gate, "gate") || !tensor_ok(up, "up") || !tensor_ok(y, "Y")) return HK_INVALID_ARGUMENT;
    if (!gate_shapes({gate, up, y}, "SiLU Mul")) return HK_INVALID_ARGUMENT;
    if (!disjoint({y}, {gate, up})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    const int64_t n = numel(gate);
    hipError_t e = hk::silu_mul(gate->dtype == HK_BF16, gate->data, up->data, y->data, n, g.c->stream);
    return complete(g.c, e, "silu_mul", n ? 1 : 0);
}

hk_status hk_silu_mul_backward(hk_context* h, const hk_tensor* gate, const hk_tensor* up, const hk_tensor* dy,
                               hk_tensor* dgate, hk_tensor* dup) {
    // Reference: elementwise.rs:21-30.
    if (!tensor_ok(gate, "gate") || !tensor_ok(up, "up") || !tensor_ok(dy, "dY") || !tensor_ok(dgate, "dGate") ||
        !tensor_ok(dup, "dUp"))
        return HK_INVALID_ARGUMENT;
    if (!gate_shapes({gate, up, dy, dgate, dup}, "SiLU Mul backward")) return HK_INVALID_ARGUMENT;
    if (!disjoint({dgate, dup}, {gate, up, dy})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    const int64_t n = numel(gate);
    hipError_t e = hk::silu_mul_backward(gate->dtype == HK_BF16, gate->data, up->data, dy->data, dgate->data,
                                         dup->data, n, g.c->stream);
    return complete(g.c, e, "silu_mul_backward", n ? 1 : 0);
}

// ------------------------------------------------------------------ bias and residual add

namespace {
// Reference: affine.rs:6-9 with wide_rows.rs:13-20 (rank 1..8, positive width, count <= u32).
static bool affine_layout(const hk_tensor* t, int64_t* rows, int64_t* width, const char* op) {
    if (t->rank < 1 || t->rank > 8) return fail(HK_INVALID_ARGUMENT, "%s requires rank 1..8", op), false;
    *width = t->shape[t->rank - 1];
    if (*width <= 0) return fail(HK_INVALID_ARGUMENT, "%s requires a positive last axis", op), false;
    const int64_t n = numel(t);
    if (n > static_cast<int64_t>(UINT32_MAX)) return fail(HK_INVALID_ARGUMENT, "%s element count exceeds u32", op), false;
    *rows = n / *width;
    return true;
}
}  // namespace

hk_status hk_bias_add(hk_context* h, const hk_tensor* x, const hk_tensor* bias, const hk_tensor* residual,
                      hk_tensor* y) {
    // Reference: runtime/affine.rs:10-22 (forward), src/nn/affine.rs:17-25.
    if (!tensor_ok(x, "X") || !tensor_ok(y, "Y")) return HK_INVALID_ARGUMENT;
    if (!bias && !residual) return fail(HK_INVALID_ARGUMENT, "bias add needs a bias, a residual or both");
    if ((bias && !tensor_ok(bias, "bias")) || (residual && !tensor_ok(residual, "residual"))) return HK_INVALID_ARGUMENT;
    int64_t rows, width;
    if (!affine_layout(x, &rows, &width, "bias add")) return HK_INVALID_ARGUMENT;
    if (x->dtype != HK_F32 && x->dtype != HK_BF16) return fail(HK_INVALID_ARGUMENT, "bias add requires F32 or BF16 X");
    if (bias && (bias->dtype != HK_F32 || bias->rank != 1 || bias->shape[0] != width))
        return fail(HK_INVALID_ARGUMENT, "bias must be F32 [%lld]", static_cast<long long>(width));
    if (residual && (residual->dtype != x->dtype || !same_shape(residual, x)))
        return fail(HK_INVALID_ARGUMENT, "residual must match X exactly");
    if (y->dtype != x->dtype || !same_shape(y, x)) return fail(HK_INVALID_ARGUMENT, "bias add output must match X");
    if (!disjoint({y}, {x}) || (bias && !disjoint({y}, {bias})) || (residual && !disjoint({y}, {residual})))
        return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    const int64_t n = rows * width;
    hipError_t e = hk::bias_add(x->dtype == HK_BF16, x->data, bias ? static_cast<const float*>(bias->data) : nullptr,
                                residual ? residual->data : nullptr, y->data, n, width, g.c->stream);
    return complete(g.c, e, residual ? "residual_bias_add" : "bias_add", n ? 1 : 0);
}

hk_status hk_bias_add_backward(hk_context* h, const hk_tensor* dy, hk_tensor* dbias) {
    // Reference: runtime/affine.rs:23-26 -> normalization.rs:95-114 (column_sum).
    if (!tensor_ok(dy, "dY") || !tensor_ok(dbias, "dbias")) return HK_INVALID_ARGUMENT;
    int64_t rows, width;
    if (!affine_layout(dy, &rows, &width, "bias add backward")) return HK_INVALID_ARGUMENT;
    if (dy->dtype != HK_F32) return fail(HK_INVALID_ARGUMENT, "bias add backward requires F32 dY");
    if (dbias->dtype != HK_F32 || dbias->rank != 1 || dbias->shape[0] != width)
        return fail(HK_INVALID_ARGUMENT, "dbias must be F32 [%lld]", static_cast<long long>(width));
    if (!disjoint({dbias}, {dy})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    hk_status st = ensure_workspace(g.c, hk::column_sum_workspace_bytes(rows, width));
    if (st != HK_OK) return st;
    hipError_t e = hk::column_sum(static_cast<const float*>(dy->data), static_cast<float*>(dbias->data), rows, width,
                                  g.c->workspace, g.c->stream);
    return complete(g.c, e, "bias_add_backward", 1);
}

// ------------------------------------------------------------------ decoder-layer relayouts

namespace {
static bool aligned_bf16(std::initializer_list<const hk_tensor*> ts, const char* op) {
    for (const hk_tensor* t : ts) {
        if (t->dtype != HK_BF16) return fail(HK_INVALID_ARGUMENT, "%s requires BF16 tensors", op), false;
        if (reinterpret_cast<uintptr_t>(t->data) % 16 != 0)
            return fail(HK_INVALID_ARGUMENT, "%s requires 16-byte aligned tensors", op), false;
    }
    return true;
}
static bool dims_are(const hk_tensor* t, std::initializer_list<int64_t> dims) {
    if (t->rank != static_cast<int32_t>(dims.size())) return false;
    int i = 0;
    for (int64_t d : dims)
        if (t->shape[i++] != d) return false;
    return true;
}
// rows [B,S,(Hq+2Hkv)D], q [B,Hq,S,D], k/v [B,Hkv,S,D], tables [S, D/2] F32.
static hk_status qkv_rope_common(hk_context* h, bool merge, const hk_tensor* rows, const hk_tensor* q, const hk_tensor* k,
                          const hk_tensor* v, const hk_tensor* c, const hk_tensor* s, int32_t layout) {
    const char* op = merge ? "qkv_rope_merge" : "qkv_rope_split";
    if (!tensor_ok(rows, "QKV rows") || !tensor_ok(q, "Q") || !tensor_ok(k, "K") || !tensor_ok(v, "V") ||
        !tensor_ok(c, "cos") || !tensor_ok(s, "sin"))
        return HK_INVALID_ARGUMENT;
    if (layout != HK_ROTARY_INTERLEAVED && layout != HK_ROTARY_SPLIT_HALF)
        return fail(HK_INVALID_ARGUMENT, "rotary layout must be 0 (Interleaved) or 1 (SplitHalf)");
    if (!aligned_bf16({rows, q, k, v}, op)) return HK_INVALID_ARGUMENT;
    if (q->rank != 4 || k->rank != 4) return fail(HK_INVALID_ARGUMENT, "%s requires Q[B,Hq,S,D] and K/V[B,Hkv,S,D]", op);
    const int64_t B = q->shape[0], Hq = q->shape[1], S = q->shape[2], D = q->shape[3], Hkv = k->shape[1];
    if (B <= 0 || Hq <= 0 || Hkv <= 0 || S <= 0 || D <= 0 || D % 16 != 0)
        return fail(HK_INVALID_ARGUMENT, "%s requires positive dimensions and D %% 16 == 0", op);
    if (!dims_are(k, {B, Hkv, S, D}) || !dims_are(v, {B, Hkv, S, D}) || !dims_are(rows, {B, S, (Hq + 2 * Hkv) * D}))
        return fail(HK_INVALID_ARGUMENT, "%s requires rows [B,S,(Hq+2Hkv)D], Q [B,Hq,S,D], K/V [B,Hkv,S,D]", op);
    if (c->dtype != HK_F32 || s->dtype != HK_F32 || !dims_are(c, {S, D / 2}) || !dims_are(s, {S, D / 2}) ||
        reinterpret_cast<uintptr_t>(c->data) % 16 != 0 || reinterpret_cast<uintptr_t>(s->data) % 16 != 0)
        return fail(HK_INVALID_ARGUMENT, "%s requires 16-byte aligned F32 cos/sin tables [S, D/2]", op);
    if (merge ? !disjoint({rows}, {q, k, v, c, s}) : !disjoint({q, k, v}, {rows, c, s})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    hipError_t e = hk::qkv_rope(merge, layout, rows->data, q->data, k->data, v->data, static_cast<const float*>(c->data),
                                static_cast<const float*>(s->data), B, S, Hq, Hkv, D, g.c->stream);
    return complete(g.c, e, op, 1);
}
static hk_status heads_rows_common(hk_context* h, bool to_rows, const hk_tensor* x, hk_tensor* y) {
    const char* op = to_rows ? "heads_to_rows" : "rows_to_heads";
    if (!tensor_ok(x, "X") || !tensor_ok(y, "Y")) return HK_INVALID_ARGUMENT;
    if (!aligned_bf16({x, y}, op)) return HK_INVALID_ARGUMENT;
    const hk_tensor* planes = to_rows ? x : y;
    const hk_tensor* rows = to_rows ? y : x;
    if (planes->rank != 4) return fail(HK_INVALID_ARGUMENT, "%s requires head planes [B,H,S,D]", op);
    const int64_t B = planes->shape[0], H = planes->shape[1], S = planes->shape[2], D = planes->shape[3];
    if (D <= 0 || D % 8 != 0 || !dims_are(rows, {B, S, H * D}))
        return fail(HK_INVALID_ARGUMENT, "%s requires planes [B,H,S,D] (D %% 8 == 0) and rows [B,S,H*D]", op);
    if (!disjoint({y}, {x})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    hipError_t e = hk::heads_rows(to_rows, x->data, y->data, B, H, S, D, g.c->stream);
    return complete(g.c, e, op, 1);
}
}  // namespace

hk_status hk_qkv_rope_split(hk_context* h, const hk_tensor* qkv, const hk_tensor* cos, const hk_tensor* sin,
                            int32_t layout, hk_tensor* q, hk_tensor* k, hk_tensor* v) {
    return qkv_rope_common(h, false, qkv, q, k, v, cos, sin, layout);
}
hk_status hk_qkv_rope_merge(hk_context* h, const hk_tensor* dq, const hk_tensor* dk, const hk_tensor* dv,
                            const hk_tensor* cos, const hk_tensor* sin, int32_t layout, hk_tensor* dqkv) {
    return qkv_rope_common(h, true, dqkv, dq, dk, dv, cos, sin, layout);
}
hk_status hk_qkv_projection_rope(hk_context* h, const hk_tensor* x, const hk_tensor* w, const hk_tensor* cos,
                                 const hk_tensor* sin, int32_t layout, hk_tensor* q, hk_tensor* k, hk_tensor* v) {
    const char* op = "qkv_projection_rope";
    if (!tensor_ok(x, "X") || !tensor_ok(w, "W") || !tensor_ok(q, "Q") || !tensor_ok(k, "K") || !tensor_ok(v, "V") ||
        !tensor_ok(cos, "cos") || !tensor_ok(sin, "sin"))
        return HK_INVALID_ARGUMENT;
    if (layout != HK_ROTARY_INTERLEAVED && layout != HK_ROTARY_SPLIT_HALF)
        return fail(HK_INVALID_ARGUMENT, "rotary layout must be 0 (Interleaved) or 1 (SplitHalf)");
    if (!aligned_bf16({x, w, q, k, v}, op)) return HK_INVALID_ARGUMENT;
    if (q->rank != 4 || k->rank != 4) return fail(HK_INVALID_ARGUMENT, "%s requires Q[B,Hq,S,D] and K/V[B,Hkv,S,D]", op);
    const int64_t B = q->shape[0], Hq = q->shape[1], S = q->shape[2], D = q->shape[3], Hkv = k->shape[1];
    if (B <= 0 || Hq <= 0 || Hkv <= 0 || S <= 0 || D != 128)
        return fail(HK_INVALID_ARGUMENT, "%s requires positive dimensions and heads of width 128", op);
    const int64_t W = (Hq + 2 * Hkv) * D;
    const int64_t T = B * S;
    const int64_t H = x->shape[x->rank - 1];
    const bool x_ok = (x->rank == 2 && dims_are(x, {T, H})) || (x->rank == 3 && dims_are(x, {B, S, H}));
    if (!dims_are(k, {B, Hkv, S, D}) || !dims_are(v, {B, Hkv, S, D}) || !x_ok || !dims_are(w, {W, H}))
        return fail(HK_INVALID_ARGUMENT, "%s requires X [B*S,H] or [B,S,H], W [(Hq+2Hkv)*128,H], Q [B,Hq,S,128], "
                                         "K/V [B,Hkv,S,128]", op);
    if (cos->dtype != HK_F32 || sin->dtype != HK_F32 || !dims_are(cos, {S, D / 2}) || !dims_are(sin, {S, D / 2}) ||
        reinterpret_cast<uintptr_t>(cos->data) % 16 != 0 || reinterpret_cast<uintptr_t>(sin->data) % 16 != 0)
        return fail(HK_INVALID_ARGUMENT, "%s requires 16-byte aligned F32 cos/sin tables [S, D/2]", op);
    if (!hk::qkv_rope_applies(T, H, W))
        return fail(HK_INVALID_ARGUMENT, "%s requires H %% 8 == 0 and B*S*H, (Hq+2Hkv)*128*H below 2^30 elements", op);
    if (!disjoint({q, k, v}, {x, w, cos, sin})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    hipError_t e = hk::gemm_qkv_rope(x->data, w->data, T, H, S, Hq, Hkv, static_cast<const float*>(cos->data),
                                     static_cast<const float*>(sin->data), layout, q->data, k->data, v->data,
                                     g.c->stream);
    return complete(g.c, e, op, 1);
}

namespace {
// Rank-2 BF16 [rows, cols] with cols % mult == 0 (rows any positive count).
bool bf16_matrix(const hk_tensor* t, int64_t rows, int64_t cols) {
    return t->dtype == HK_BF16 && t->rank == 2 && t->shape[0] == rows && t->shape[1] == cols;
}
}  // namespace

hk_status hk_linear_residual(hk_context* h, const hk_tensor* x, const hk_tensor* w, const hk_tensor* residual,
                             hk_tensor* y) {
    const char* op = "linear_residual";
    if (!tensor_ok(x, "X") || !tensor_ok(w, "W") || !tensor_ok(residual, "residual") || !tensor_ok(y, "Y"))
        return HK_INVALID_ARGUMENT;
    if (x->rank != 2 || w->rank != 2) return fail(HK_INVALID_ARGUMENT, "%s requires X [M,K] and W [N,K]", op);
    const int64_t M = x->shape[0], K = x->shape[1], N = w->shape[0];
    if (!bf16_matrix(x, M, K) || !bf16_matrix(w, N, K) || !bf16_matrix(residual, M, N) || !bf16_matrix(y, M, N))
        return fail(HK_INVALID_ARGUMENT, "%s requires BF16 X [M,K], W [N,K], residual and Y [M,N]", op);
    if (!aligned_bf16({x, w, residual, y}, op)) return HK_INVALID_ARGUMENT;
    if (M <= 0 || N % 16 != 0 || !hk::epi_applies(M, N, K))
        return fail(HK_INVALID_ARGUMENT, "%s requires N %% 16 == 0, K %% 8 == 0 and M*K, N*K below 2^30 elements", op);
    if (!disjoint({y}, {x, w, residual})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    hipError_t e = hk::gemm_residual(x->data, w->data, residual->data, y->data, M, N, K, g.c->stream);
    return complete(g.c, e, op, 1);
}

hk_status hk_swiglu_projection(hk_context* h, const hk_tensor* x, const hk_tensor* w_gu, hk_tensor* gate,
                               hk_tensor* up, hk_tensor* act) {
    const char* op = "swiglu_projection";
    if (!tensor_ok(x, "X") || !tensor_ok(w_gu, "W_gu") || !tensor_ok(gate, "gate") || !tensor_ok(up, "up") ||
        !tensor_ok(act, "act"))
        return HK_INVALID_ARGUMENT;
    if (x->rank != 2 || w_gu->rank != 2) return fail(HK_INVALID_ARGUMENT, "%s requires X [T,H] and W_gu [2F,H]", op);
    const int64_t T = x->shape[0], H = x->shape[1], F = w_gu->shape[0] / 2;
    if (!bf16_matrix(x, T, H) || !bf16_matrix(w_gu, 2 * F, H) || !bf16_matrix(gate, T, F) || !bf16_matrix(up, T, F) ||
        !bf16_matrix(act, T, F))
        return fail(HK_INVALID_ARGUMENT, "%s requires BF16 X [T,H], W_gu [2F,H], gate/up/act [T,F]", op);
    if (!aligned_bf16({x, w_gu, gate, up, act}, op)) return HK_INVALID_ARGUMENT;
    if (T <= 0 || F <= 0 || F % 16 != 0 || !hk::epi_applies(T, 2 * F, H))
        return fail(HK_INVALID_ARGUMENT, "%s requires F %% 16 == 0, H %% 8 == 0 and T*H, 2F*H below 2^30 elements", op);
    if (!disjoint({gate, up, act}, {x, w_gu})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    hipError_t e = hk::gemm_swiglu(x->data, w_gu->data, gate->data, up->data, act->data, T, F, H, g.c->stream);
    return complete(g.c, e, op, 1);
}

hk_status hk_swiglu_projection_backward(hk_context* h, const hk_tensor* dy, const hk_tensor* wd, const hk_tensor* gate,
                                        const hk_tensor* up, hk_tensor* dgu) {
    const char* op = "swiglu_projection_backward";
    if (!tensor_ok(dy, "dY") || !tensor_ok(wd, "Wd") || !tensor_ok(gate, "gate") || !tensor_ok(up, "up") ||
        !tensor_ok(dgu, "dgu"))
        return HK_INVALID_ARGUMENT;
    if (dy->rank != 2 || wd->rank != 2) return fail(HK_INVALID_ARGUMENT, "%s requires dY [T,H] and Wd [H,F]", op);
    const int64_t T = dy->shape[0], H = dy->shape[1], F = wd->shape[1];
    if (!bf16_matrix(dy, T, H) || !bf16_matrix(wd, H, F) || !bf16_matrix(gate, T, F) || !bf16_matrix(up, T, F) ||
        !bf16_matrix(dgu, T, 2 * F))
        return fail(HK_INVALID_ARGUMENT, "%s requires BF16 dY [T,H], Wd [H,F], gate/up [T,F], dgu [T,2F]", op);
    if (!aligned_bf16({dy, wd, gate, up, dgu}, op)) return HK_INVALID_ARGUMENT;
    if (T <= 0 || F <= 0 || F % 16 != 0 || !hk::epi_applies(T, F, H))
        return fail(HK_INVALID_ARGUMENT, "%s requires F %% 16 == 0, H %% 8 == 0 and T*H, F*H below 2^30 elements", op);
    if (!disjoint({dgu}, {dy, wd, gate, up})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    hipError_t e = hk::gemm_swiglu_backward(dy->data, wd->data, gate->data, up->data, dgu->data, T, F, H, g.c->stream);
    return complete(g.c, e, op, 1);
}

hk_status hk_heads_to_rows(hk_context* h, const hk_tensor* x, hk_tensor* y) { return heads_rows_common(h, true, x, y); }
hk_status hk_rows_to_heads(hk_context* h, const hk_tensor* x, hk_tensor* y) { return heads_rows_common(h, false, x, y); }

// ------------------------------------------------------------------ embedding

namespace {
// Reference: embedding.rs:21-26 (indices_layout: contiguous rank 1..7 INT32/INT64).
static bool ids_layout(const hk_tensor* ids, int64_t* tokens) {
    if (!tensor_ok(ids, "IDs", true)) return false;
    if (ids->rank < 1 || ids->rank > 7)
        return fail(HK_INVALID_ARGUMENT, "embedding indices require contiguous rank 1..7 INT32/INT64 storage"), false;
    *tokens = numel(ids);
    if (*tokens > INT32_MAX) return fail(HK_INVALID_ARGUMENT, "embedding supports at most 2^31-1 IDs"), false;
    return true;
}
static bool ids_prefix(const hk_tensor* ids, const hk_tensor* t) {  // t = ids.shape + [H]
    if (t->rank != ids->rank + 1) return false;
    for (int i = 0; i < ids->rank; ++i)
        if (t->shape[i] != ids->shape[i]) return false;
    return true;
}
// After a synchronous call: read the kernel's out-of-range flag (the workspace's first int).
// The index check of a synchronous call: the flag word at `flag` equals `bad` when an index was
// outside the table.
static hk_status ids_in_range(Ctx* c, hk_status st, int64_t vocab, const void* flag, int bad) {
    if (st != HK_OK || c->async) return st;
    int value = 0;
    if (hipMemcpy(&value, flag, sizeof(value), hipMemcpyDeviceToHost) != hipSuccess) {
        c->poisoned = true;
        return fail(HK_COMPLETION_ERROR, "embedding: reading the index check failed");
    }
    if (value == bad) return fail(HK_INVALID_ARGUMENT, "embedding index outside [0, %lld)", static_cast<long long>(vocab));
    return HK_OK;
}
}  // namespace

// ------------------------------------------------------------------ NLLLoss

namespace {
int float_code(int32_t dt) { return dt == HK_F32 ? 0 : (dt == HK_F16 ? 1 : 2); }

// Reference: forward_layouts, rust-ascend-driver/src/tensor/loss.rs:17-27.
hk_status nll_layouts(const hk_tensor* input, const hk_tensor* target, const hk_tensor* weight, int32_t reduction) {
    if (!tensor_ok(input, "input") || !tensor_ok(weight, "weight") || !tensor_ok(target, "target", true))
        return fail(HK_INVALID_ARGUMENT, "NLLLoss requires floating input[N,C], matching integer target[N] and same-dtype class weight[C]");
    if (input->rank != 2 || input->shape[1] <= 0 || target->rank != 1 || target->shape[0] != input->shape[0] ||
        weight->rank != 1 || weight->shape[0] != input->shape[1] || weight->dtype != input->dtype)
        return fail(HK_INVALID_ARGUMENT, "NLLLoss requires floating input[N,C], matching integer target[N] and same-dtype class weight[C]");
    if (reduction < HK_LOSS_NONE || reduction > HK_LOSS_SUM)
        return fail(HK_INVALID_ARGUMENT, "NLLLoss reduction must be None (0), Mean (1) or Sum (2)");
    return HK_OK;
}
bool nll_out_ok(const hk_tensor* t, int64_t len, int32_t dtype) {
    return t && t->dtype == dtype && t->rank == 1 && t->shape[0] == len && (len == 0 || t->data);
}
}  // namespace

hk_status hk_nll_loss(hk_context* h, const hk_tensor* input, const hk_tensor* target, const hk_tensor* weight,
                      int32_t reduction, int64_t ignore_index, hk_tensor* out, hk_tensor* total_weight) {
    // Reference: CannSession::nll_loss, tensor/loss.rs:31-46 (runtime/loss.rs:15-20).
    hk_status st = nll_layouts(input, target, weight, reduction);
    if (st != HK_OK) return st;
    const int64_t rows = input->shape[0], classes = input->shape[1];
    if (!nll_out_ok(out, reduction == HK_LOSS_NONE ? rows : 1, input->dtype) || !nll_out_ok(total_weight, 1, input->dtype))
        return fail(HK_INVALID_ARGUMENT, "NLLLoss output must be [N] (None) or [1], total weight [1], in the input's dtype");
    if (!disjoint({out, total_weight}, {input, target, weight})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    if ((st = ensure_workspace(g.c, hk::nll_loss_workspace_bytes(rows))) != HK_OK) return st;
    hipError_t e = hk::nll_loss(float_code(input->dtype), target->dtype == HK_I64 ? 8 : 4, input->data, target->data,
                                weight->data, out->data, total_weight->data, rows, classes, reduction, ignore_index,
                                g.c->workspace, g.c->stream);
    st = complete(g.c, e, "nll_loss", 1);
    if (st != HK_OK || g.c->async) return st;
    int flag = 0;
    if (hipMemcpy(&flag, g.c->workspace, sizeof(flag), hipMemcpyDeviceToHost) != hipSuccess) {
        g.c->poisoned = true;
        return fail(HK_COMPLETION_ERROR, "nll_loss: reading the label check failed");
    }
    if (flag)
        return fail(HK_INVALID_ARGUMENT, "NLLLoss target outside [0, %lld) that is not the ignore index %lld",
                    static_cast<long long>(classes), static_cast<long long>(ignore_index));
    return HK_OK;
}

hk_status hk_nll_loss_backward(hk_context* h, const hk_tensor* grad, const hk_tensor* input, const hk_tensor* target,
                               const hk_tensor* weight, const hk_tensor* total_weight, int32_t reduction,
                               int64_t ignore_index, hk_tensor* dinput) {
    // Reference: CannSession::nll_loss_backward, tensor/loss.rs:47-60 (backward_layout, :28-36).
    hk_status st = nll_layouts(input, target, weight, reduction);
    if (st != HK_OK) return st;
    const int64_t rows = input->shape[0], classes = input->shape[1];
    if (!nll_out_ok(grad, reduction == HK_LOSS_NONE ? rows : 1, input->dtype) ||
        !nll_out_ok(total_weight, 1, input->dtype))
        return fail(HK_INVALID_ARGUMENT, "NLLLoss upstream gradient or saved total weight does not match forward reduction/dtype");
    if (!tensor_ok(dinput, "dinput") || dinput->dtype != input->dtype || !same_shape(dinput, input))
        return fail(HK_INVALID_ARGUMENT, "NLLLoss input gradient must match the input");
    if (!disjoint({dinput}, {grad, input, target, weight, total_weight})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    hipError_t e = hk::nll_loss_backward(float_code(input->dtype), target->dtype == HK_I64 ? 8 : 4, grad->data,
                                         target->data, weight->data, total_weight->data, dinput->data, rows, classes,
                                         reduction, ignore_index, g.c->stream);
    return complete(g.c, e, "nll_loss_backward", 1);
}

hk_status hk_embedding(hk_context* h, const hk_tensor* weight, const hk_tensor* ids, hk_tensor* out) {
    // Reference: runtime/indexing.rs:33-37, embedding.rs:27-34 (forward_layout) and :46-60.
    int64_t tokens;
    if (!tensor_ok(weight, "weight") || !ids_layout(ids, &tokens) || !tensor_ok(out, "out")) return HK_INVALID_ARGUMENT;
    if (weight->rank != 2 || (weight->shape[0] == 0 && tokens != 0))
        return fail(HK_INVALID_ARGUMENT,
                    "embedding weight requires a rank-2 FP32/FP16/BF16 table; nonempty indices require weight rows");
    if (weight->shape[0] > INT32_MAX) return fail(HK_INVALID_ARGUMENT, "embedding supports at most 2^31-1 table rows");
    if (out->dtype != weight->dtype || !ids_prefix(ids, out) || out->shape[ids->rank] != weight->shape[1])
        return fail(HK_INVALID_ARGUMENT, "embedding output must be [ids..., H] in the table's dtype");
    if (!disjoint({out}, {weight, ids})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    const int64_t vocab = weight->shape[0];
    g.c->flag_seq = g.c->flag_seq + 1 == 0 ? 1 : g.c->flag_seq + 1;  // never 0, the word's initial value
    const int seq = static_cast<int>(g.c->flag_seq);
    hipError_t e = hk::embedding(weight->data, static_cast<int>(dtype_size(ids->dtype)), ids->data, out->data, tokens,
                                 vocab, weight->shape[1] * dtype_size(weight->dtype), g.c->flags, seq, g.c->stream);
    return ids_in_range(g.c, complete(g.c, e, "embedding", 1), vocab, g.c->flags, seq);
}

hk_status hk_embedding_backward(hk_context* h, const hk_tensor* grad, const hk_tensor* ids, uint64_t num_weights,
                                uint64_t padding_idx, int32_t scale_grad_by_freq, hk_tensor* dweight) {
    // Reference: runtime/indexing.rs:60-64, embedding.rs:35-44 (backward_layout), :9-18 (padding
    // sentinel) and :60-79 (dense backward).
    int64_t tokens;
    if (!tensor_ok(grad, "grad") || !ids_layout(ids, &tokens) || !tensor_ok(dweight, "dweight"))
        return HK_INVALID_ARGUMENT;
    if (num_weights > static_cast<uint64_t>(INT32_MAX))
        return fail(HK_INVALID_ARGUMENT, "embedding supports at most 2^31-1 table rows");
    if (padding_idx != HK_NO_PADDING && padding_idx >= num_weights)
        return fail(HK_INVALID_ARGUMENT, "embedding padding index must be within the weight rows");
    if (scale_grad_by_freq != 0 && scale_grad_by_freq != 1)
        return fail(HK_INVALID_ARGUMENT, "scale_grad_by_freq must be 0 or 1");
    const int64_t vocab = static_cast<int64_t>(num_weights);
    if (!ids_prefix(ids, grad) || (vocab == 0 && tokens != 0))
        return fail(HK_INVALID_ARGUMENT,
                    "embedding gradient must have the index shape followed by the embedding width and floating dtype");
    const int64_t width = grad->shape[ids->rank];
    if (dweight->dtype != grad->dtype || dweight->rank != 2 || dweight->shape[0] != vocab || dweight->shape[1] != width)
        return fail(HK_INVALID_ARGUMENT, "dweight must be [num_weights, H] in the gradient's dtype");
    if (!disjoint({dweight}, {grad, ids})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    hk_status st = ensure_workspace(g.c, hk::embedding_workspace_bytes(tokens, vocab, true));
    if (st != HK_OK) return st;
    hipError_t e = hk::embedding_backward(grad->dtype, grad->data, static_cast<int>(dtype_size(ids->dtype)), ids->data,
                                          dweight->data, tokens, vocab, width, padding_idx, scale_grad_by_freq,
                                          g.c->workspace, g.c->stream);
    st = complete(g.c, e, "embedding_backward", hk::embedding_backward_launches(tokens, vocab, width));
    return ids_in_range(g.c, st, vocab, g.c->workspace, 1);
}

hk_status hk_softmax(hk_context* h, const hk_tensor* x, int32_t logarithmic, hk_tensor* y) {
    // Reference: rows.rs:50-62 (layout_for / check_for: contiguous F32, positive width).
    if (!tensor_ok(x, "X") || !tensor_ok(y, "Y")) return HK_INVALID_ARGUMENT;
    int64_t rows, width;
    if (!row_layout(x, &rows, &width, "softmax")) return HK_INVALID_ARGUMENT;
    if (x->dtype != HK_F32) return fail(HK_INVALID_ARGUMENT, "softmax input must be F32");
    if (y->dtype != HK_F32 || !same_shape(x, y)) return fail(HK_INVALID_ARGUMENT, "softmax output must match the input");
    if (logarithmic != 0 && logarithmic != 1) return fail(HK_INVALID_ARGUMENT, "logarithmic must be 0 or 1");
    if (rows > INT32_MAX) return fail(HK_INVALID_ARGUMENT, "softmax supports at most 2^31-1 rows");
    if (!disjoint({y}, {x})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    hipError_t e = hk::softmax_forward(static_cast<const float*>(x->data), static_cast<float*>(y->data), rows, width,
                                       logarithmic, g.c->stream);
    return complete(g.c, e, logarithmic ? "log_softmax" : "softmax", rows ? 1 : 0);
}

hk_status hk_softmax_backward(hk_context* h, const hk_tensor* y, const hk_tensor* dy, int32_t logarithmic,
                              hk_tensor* dx) {
    // Reference: rows.rs:64-79.
    if (!tensor_ok(y, "Y") || !tensor_ok(dy, "dY") || !tensor_ok(dx, "dX")) return HK_INVALID_ARGUMENT;
    int64_t rows, width;
    if (!row_layout(y, &rows, &width, "softmax backward")) return HK_INVALID_ARGUMENT;
    if (y->dtype != HK_F32) return fail(HK_INVALID_ARGUMENT, "softmax backward input must be F32");
    if (dy->dtype != HK_F32 || !same_shape(dy, y)) return fail(HK_INVALID_ARGUMENT, "dY must match Y");
    if (dx->dtype != HK_F32 || !same_shape(dx, y)) return fail(HK_INVALID_ARGUMENT, "dX must match Y");
    if (logarithmic != 0 && logarithmic != 1) return fail(HK_INVALID_ARGUMENT, "logarithmic must be 0 or 1");
    if (rows > INT32_MAX) return fail(HK_INVALID_ARGUMENT, "softmax supports at most 2^31-1 rows");
    if (!disjoint({dx}, {y, dy})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    hipError_t e = hk::softmax_backward(static_cast<const float*>(y->data), static_cast<const float*>(dy->data),
                                        static_cast<float*>(dx->data), rows, width, logarithmic, g.c->stream);
    return complete(g.c, e, logarithmic ? "log_softmax_backward" : "softmax_backward", rows ? 1 : 0);
}

hk_status hk_causal_mask(hk_context* h, uint64_t query_start, uint64_t key_start, hk_tensor* out) {
    // Reference: CausalMaskSpec::elements (mask_programs.rs:7-19), mask.rs via runtime/mod.rs:205-206.
    if (!tensor_ok(out, "mask")) return HK_INVALID_ARGUMENT;
    if (out->dtype != HK_F32 || out->rank != 3) return fail(HK_INVALID_ARGUMENT, "causal mask output must be F32 [B,Q,K]");
    const int64_t batch = out->shape[0], queries = out->shape[1], keys = out->shape[2];
    if (queries <= 0 || keys <= 0) return fail(HK_INVALID_ARGUMENT, "causal mask requires positive query/key lengths");
    if (query_start > UINT64_MAX - static_cast<uint64_t>(queries - 1) ||
        key_start > UINT64_MAX - static_cast<uint64_t>(keys - 1))
        return fail(HK_INVALID_ARGUMENT, "causal absolute position overflow");
    if (batch < 0 || numel(out) > static_cast<int64_t>(UINT32_MAX))
        return fail(HK_INVALID_ARGUMENT, "causal mask domain exceeds u32");
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    hipError_t e = hk::causal_mask(static_cast<float*>(out->data), batch, queries, keys, query_start, key_start,
                                   g.c->stream);
    return complete(g.c, e, "causal_mask", numel(out) ? 1 : 0);
}

namespace {
// [B, H, N, D] F32 with both element counts within u32 (RepeatKvSpec::elements, heads_programs.rs:5-18).
static bool kv_shapes(const hk_tensor* kv, const hk_tensor* qh, const char* kv_name, const char* q_name) {
    if (kv->dtype != HK_F32 || qh->dtype != HK_F32 || kv->rank != 4 || qh->rank != 4)
        return fail(HK_INVALID_ARGUMENT, "KV repetition requires F32 [B,Hkv,N,D] %s and [B,Hq,N,D] %s", kv_name, q_name),
               false;
    if (kv->shape[0] != qh->shape[0] || kv->shape[2] != qh->shape[2] || kv->shape[3] != qh->shape[3])
        return fail(HK_INVALID_ARGUMENT, "%s and %s must agree in B, N and D", kv_name, q_name), false;
    if (kv->shape[1] <= 0 || qh->shape[1] <= 0 || qh->shape[1] % kv->shape[1] != 0)
        return fail(HK_INVALID_ARGUMENT, "KV repetition requires positive heads and query_heads divisible by kv_heads"),
               false;
    if (numel(kv) > static_cast<int64_t>(UINT32_MAX) || numel(qh) > static_cast<int64_t>(UINT32_MAX))
        return fail(HK_INVALID_ARGUMENT, "KV repetition complete domain exceeds u32"), false;
    return true;
}
}  // namespace

hk_status hk_repeat_kv_heads(hk_context* h, const hk_tensor* x, hk_tensor* y) {
    // Reference: runtime/heads.rs:21-28.
    if (!tensor_ok(x, "X") || !tensor_ok(y, "Y")) return HK_INVALID_ARGUMENT;
    if (!kv_shapes(x, y, "X", "Y")) return HK_INVALID_ARGUMENT;
    if (!disjoint({y}, {x})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    hipError_t e = hk::repeat_kv_heads(static_cast<const float*>(x->data), static_cast<float*>(y->data), x->shape[0],
                                       x->shape[1], y->shape[1], x->shape[2] * x->shape[3], g.c->stream);
    return complete(g.c, e, "repeat_kv_heads", numel(y) ? 1 : 0);
}

hk_status hk_repeat_kv_heads_backward(hk_context* h, const hk_tensor* dy, hk_tensor* dx) {
    // Reference: runtime/heads.rs:29-51.
    if (!tensor_ok(dy, "dY") || !tensor_ok(dx, "dX")) return HK_INVALID_ARGUMENT;
    if (!kv_shapes(dx, dy, "dX", "dY")) return HK_INVALID_ARGUMENT;
    if (!disjoint({dx}, {dy})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    const int64_t plane = dx->shape[2] * dx->shape[3];
    hk_status st = ensure_workspace(g.c, hk::repeat_kv_backward_workspace_bytes(dx->shape[0], dx->shape[1],
                                                                                dy->shape[1], plane));
    if (st != HK_OK) return st;
    hipError_t e = hk::repeat_kv_heads_backward(static_cast<const float*>(dy->data), static_cast<float*>(dx->data),
                                                dx->shape[0], dx->shape[1], dy->shape[1], plane, g.c->workspace,
                                                g.c->stream);
    return complete(g.c, e, "repeat_kv_heads_backward", numel(dx) ? 1 : 0);
}

// The RMSNorm row-split exchange's check word (check_flags[1]): a new sequence number per call,
// the wait bound from HK_ROW_SPIN_LIMIT (polls per wait; default 2^24, ~1 s), and after a
// synchronous call that launched a split kernel, a word equal to the call's number means a
// wait ran out and the results are invalid. The device is left healthy (every wait is bounded),
// so the context is not poisoned.
static hk::RowCheck row_check(Ctx* c) {
    c->flag_seq = c->flag_seq + 1 == 0 ? 1 : c->flag_seq + 1;
    int limit = 1 << 24;
    if (const char* env = std::getenv("HK_ROW_SPIN_LIMIT")) {
        char* end = nullptr;
        const long v = std::strtol(env, &end, 10);
        if (end != nullptr && *end == '\0' && v > 0 && v <= INT32_MAX) limit = static_cast<int>(v);
    }
    return hk::RowCheck{c->flags + 1, static_cast<int>(c->flag_seq), limit, 0};
}

static hk_status row_check_result(Ctx* c, hk_status st, const hk::RowCheck& rc, const char* op) {
    if (st != HK_OK || c->async || !rc.used) return st;
    int value = 0;
    if (hipMemcpy(&value, rc.flag, sizeof(value), hipMemcpyDeviceToHost) != hipSuccess) {
        c->poisoned = true;
        return fail(HK_COMPLETION_ERROR, "%s: reading the row exchange check failed", op);
    }
    if (value == rc.seq)
        return fail(HK_COMPLETION_ERROR,
                    "%s: a row-split exchange wait ran out after %d polls; the results of this call are invalid", op,
                    rc.spin_limit);
    return HK_OK;
}

hk_status hk_rms_norm(hk_context* h, const hk_tensor* x, const hk_tensor* w, double eps, hk_tensor* y,
                      hk_tensor* rstd) {
    // Reference: normalization.rs:153-166 (+ layout_for / epsilon_for, :12-48).
    if (!tensor_ok(x, "X") || !tensor_ok(w, "weight") || !tensor_ok(y, "Y") || !tensor_ok(rstd, "rstd"))
        return HK_INVALID_ARGUMENT;
    int64_t rows, width;
    if (!row_layout(x, &rows, &width, "RMSNorm")) return HK_INVALID_ARGUMENT;
    if (x->dtype != HK_F32 && x->dtype != HK_BF16) return fail(HK_INVALID_ARGUMENT, "RMSNorm input must be F32 or BF16");
    const float e32 = static_cast<float>(eps);
    if (!std::isfinite(eps) || !std::isfinite(e32) || !(e32 > 0.0f))
        return fail(HK_INVALID_ARGUMENT, "RMSNorm epsilon must be positive and representable in FP32");
    if (w->dtype != HK_F32 || w->rank != 1 || w->shape[0] != width)
        return fail(HK_INVALID_ARGUMENT, "RMSNorm weight must be F32 [%lld]", (long long)width);
    if (y->dtype != x->dtype || !same_shape(x, y)) return fail(HK_INVALID_ARGUMENT, "RMSNorm output must match the input");
    if (rstd->dtype != HK_F32 || numel(rstd) != rows)
        return fail(HK_INVALID_ARGUMENT, "rstd must be F32 with one value per row (%lld)", (long long)rows);
    if (!disjoint({y, rstd}, {x, w})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    hk::RowCheck rc = row_check(g.c);
    hipError_t e = hk::rms_norm_forward(x->dtype == HK_BF16, x->data, static_cast<const float*>(w->data), y->data,
                                        static_cast<float*>(rstd->data), rows, width, e32, rc, g.c->stream);
    return row_check_result(g.c, complete(g.c, e, "rms_norm", rows ? 1 : 0), rc, "rms_norm");
}

static hk_status rms_backward_args(const hk_tensor* x, const hk_tensor* w, const hk_tensor* dy, const hk_tensor* rstd,
                                   const hk_tensor* dx, const hk_tensor* dw, int64_t* rows_out, int64_t* width_out) {
    // Reference: normalization.rs:168-186.
    if (!tensor_ok(x, "X") || !tensor_ok(w, "weight") || !tensor_ok(dy, "dY") || !tensor_ok(rstd, "rstd") ||
        !tensor_ok(dx, "dX") || !tensor_ok(dw, "dW"))
        return HK_INVALID_ARGUMENT;
    int64_t rows, width;
    if (!row_layout(x, &rows, &width, "RMSNorm")) return HK_INVALID_ARGUMENT;
    if (x->dtype != HK_F32 && x->dtype != HK_BF16) return fail(HK_INVALID_ARGUMENT, "RMSNorm input must be F32 or BF16");
    if (w->dtype != HK_F32 || w->rank != 1 || w->shape[0] != width)
        return fail(HK_INVALID_ARGUMENT, "RMSNorm weight must be F32 [%lld]", (long long)width);
    if (dy->dtype != x->dtype || !same_shape(dy, x)) return fail(HK_INVALID_ARGUMENT, "dY must match X");
    if (dx->dtype != x->dtype || !same_shape(dx, x)) return fail(HK_INVALID_ARGUMENT, "dX must match X");
    if (rstd->dtype != HK_F32 || numel(rstd) != rows) return fail(HK_INVALID_ARGUMENT, "rstd must be F32 [rows]");
    if (dw->dtype != HK_F32 || numel(dw) != width) return fail(HK_INVALID_ARGUMENT, "dW must be F32 [width]");
    if (!disjoint({dx, dw}, {x, w, dy, rstd})) return HK_INVALID_ARGUMENT;
    *rows_out = rows;
    *width_out = width;
    return HK_OK;
}

hk_status hk_rms_norm_backward(hk_context* h, const hk_tensor* x, const hk_tensor* w, const hk_tensor* dy,
                               const hk_tensor* rstd, hk_tensor* dx, hk_tensor* dw) {
    int64_t rows, width;
    hk_status st = rms_backward_args(x, w, dy, rstd, dx, dw, &rows, &width);
    if (st != HK_OK) return st;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    if ((st = ensure_workspace(g.c, hk::rms_backward_workspace_bytes(rows, width, x->data, w->data, dy->data,
                                                                     dx->data))) != HK_OK)
        return st;
    hk::RowCheck rc = row_check(g.c);
    hipError_t e = hk::rms_norm_backward(x->dtype == HK_BF16, x->data, static_cast<const float*>(w->data), dy->data,
                                         static_cast<const float*>(rstd->data), nullptr, dx->data,
                                         static_cast<float*>(dw->data), static_cast<float*>(g.c->workspace), rows,
                                         width, rc, g.c->stream);
    return row_check_result(g.c, complete(g.c, e, "rms_norm_backward", 2), rc, "rms_norm_backward");
}

hk_status hk_rms_norm_backward_residual(hk_context* h, const hk_tensor* x, const hk_tensor* w, const hk_tensor* dy,
                                        const hk_tensor* rstd, const hk_tensor* residual, hk_tensor* dx, hk_tensor* dw) {
    const char* op = "rms_norm_backward_residual";
    int64_t rows, width;
    hk_status st = rms_backward_args(x, w, dy, rstd, dx, dw, &rows, &width);
    if (st != HK_OK) return st;
    if (!tensor_ok(residual, "residual")) return HK_INVALID_ARGUMENT;
    if (residual->dtype != dx->dtype || !same_shape(residual, dx))
        return fail(HK_INVALID_ARGUMENT, "%s requires a residual gradient of dX's dtype and shape", op);
    if (!disjoint({dx}, {residual})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    if ((st = ensure_workspace(g.c, hk::rms_backward_workspace_bytes(rows, width, x->data, w->data, dy->data,
                                                                     dx->data))) != HK_OK)
        return st;
    hk::RowCheck rc = row_check(g.c);
    hipError_t e = hk::rms_norm_backward(x->dtype == HK_BF16, x->data, static_cast<const float*>(w->data), dy->data,
                                         static_cast<const float*>(rstd->data), residual->data, dx->data,
                                         static_cast<float*>(dw->data), static_cast<float*>(g.c->workspace), rows,
                                         width, rc, g.c->stream);
    return row_check_result(g.c, complete(g.c, e, op, 2), rc, op);
}

hk_status hk_rms_norm_backward_noalloc(hk_context* h, const hk_tensor* x, const hk_tensor* w, const hk_tensor* dy,
                                       const hk_tensor* rstd, hk_tensor* dx, hk_tensor* dw) {
    int64_t rows, width;
    hk_status st = rms_backward_args(x, w, dy, rstd, dx, dw, &rows, &width);
    if (st != HK_OK) return st;
    const size_t need = hk::rms_backward_workspace_bytes(rows, width, x->data, w->data, dy->data, dx->data);
    if (need > kScratchBytes)
        return fail(HK_INVALID_ARGUMENT,
                    "rms_norm_backward_noalloc: %zu bytes of dgamma partials exceed its fixed %zu-byte device scratch "
                    "(any row count fits up to width 4096 when the width is a multiple of 8 and the tensors are "
                    "16-byte aligned, up to width 2048 otherwise; use hk_rms_norm_backward)",
                    need, kScratchBytes);
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    // The same kernels as hk_rms_norm_backward; every partial is written before it is read, so the
    // scratch needs no clearing. Overlapping calls on one GPU share the array and race.
    hk::RowCheck rc = row_check(g.c);
    hipError_t e = hk::rms_norm_backward(x->dtype == HK_BF16, x->data, static_cast<const float*>(w->data), dy->data,
                                         static_cast<const float*>(rstd->data), nullptr, dx->data,
                                         static_cast<float*>(dw->data), static_cast<float*>(g.c->scratch), rows, width,
                                         rc, g.c->stream);
    return row_check_result(g.c, complete(g.c, e, "rms_norm_backward_noalloc", 2), rc, "rms_norm_backward_noalloc");
}

// ------------------------------------------------------------------ RoPE

static hk_status rotary_common(hk_context* h, const hk_tensor* x, const hk_tensor* c, const hk_tensor* s,
                               int64_t p, bool prefix, int32_t layout, bool backward, hk_tensor* y) {
    if (!tensor_ok(x, "X") || !tensor_ok(c, "cos") || !tensor_ok(s, "sin") || !tensor_ok(y, "Y"))
        return HK_INVALID_ARGUMENT;
    if (layout != HK_ROTARY_INTERLEAVED && layout != HK_ROTARY_SPLIT_HALF)
        return fail(HK_INVALID_ARGUMENT, "rotary layout must be 0 (Interleaved) or 1 (SplitHalf)");
    if (x->dtype != HK_F32 && x->dtype != HK_BF16) return fail(HK_INVALID_ARGUMENT, "rotary input must be F32 or BF16");
    if (c->dtype != HK_F32 || s->dtype != HK_F32) return fail(HK_INVALID_ARGUMENT, "rotary tables must be F32");
    if (y->dtype != x->dtype || !same_shape(x, y)) return fail(HK_INVALID_ARGUMENT, "rotary output must match the input");
    if (!same_shape(c, s)) return fail(HK_INVALID_ARGUMENT, "cos and sin tables must have one shape");
    const int rank = x->rank;
    hk::RopeMap map{};
    if (rank < 1 || rank > 8) return fail(HK_INVALID_ARGUMENT, "rotary requires rank 1..8");
    const int64_t width = x->shape[rank - 1];
    if (!prefix) {
        // Reference: runtime/rotary.rs:6-14 (table shape = input shape with the width halved).
        p = width;
        if (width <= 0 || width % 2 != 0)
            return fail(HK_INVALID_ARGUMENT, "rotary requires a positive even width");
        bool ok = c->rank == rank;
        for (int i = 0; ok && i < rank - 1; ++i) ok = c->shape[i] == x->shape[i];
        if (!ok || c->shape[rank - 1] != width / 2)
            return fail(HK_INVALID_ARGUMENT, "rotary tables must have the input shape with the last axis halved");
        map.same_row = 1;
    } else {
        // Reference: PrefixRotarySpec::elements, rotary_programs.rs:11-23.
        if (c->rank != rank)
            return fail(HK_INVALID_ARGUMENT, "rotary prefix requires equal input/table ranks within 1..8");
        bool ok = p > 0 && p % 2 == 0 && p <= width && c->shape[rank - 1] == p / 2;
        for (int i = 0; ok && i < rank - 1; ++i) ok = c->shape[i] == 1 || c->shape[i] == x->shape[i];
        if (!ok)
            return fail(HK_INVALID_ARGUMENT,
                        "rotary prefix requires positive even P<=D, table last axis P/2 and singleton or matching leading axes");
        map.same_row = 0;
        map.nlead = rank - 1;
        int64_t tstride = 1;  // in units of table rows
        for (int a = rank - 2; a >= 0; --a) {
            map.shape[a] = x->shape[a];
            map.tstride[a] = c->shape[a] == 1 ? 0 : tstride;
            tstride *= c->shape[a];
        }
    }
    if (!disjoint({y}, {x, c, s})) return HK_INVALID_ARGUMENT;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    const int64_t rows = width > 0 ? numel(x) / width : 0;
    hipError_t e = hk::rope_apply(x->dtype == HK_BF16, x->data, static_cast<const float*>(c->data),
                                  static_cast<const float*>(s->data), y->data, rows, width, p, layout,
                                  backward ? 1 : 0, map, g.c->stream);
    return complete(g.c, e, prefix ? "rotary_prefix" : "rotary", rows ? 1 : 0);
}

hk_status hk_rotary(hk_context* h, const hk_tensor* x, const hk_tensor* c, const hk_tensor* s, int32_t layout,
                    hk_tensor* y) {
    return rotary_common(h, x, c, s, 0, false, layout, false, y);
}
hk_status hk_rotary_backward(hk_context* h, const hk_tensor* dy, const hk_tensor* c, const hk_tensor* s,
                             int32_t layout, hk_tensor* dx) {
    return rotary_common(h, dy, c, s, 0, false, layout, true, dx);
}
hk_status hk_rotary_prefix(hk_context* h, const hk_tensor* x, const hk_tensor* c, const hk_tensor* s, int32_t width,
                           int32_t layout, hk_tensor* y) {
    return rotary_common(h, x, c, s, width, true, layout, false, y);
}
hk_status hk_rotary_prefix_backward(hk_context* h, const hk_tensor* dy, const hk_tensor* c, const hk_tensor* s,
                                    int32_t width, int32_t layout, hk_tensor* dx) {
    return rotary_common(h, dy, c, s, width, true, layout, true, dx);
}

// ------------------------------------------------------------------ attention

static hk_status attention_shape(const hk_tensor* q, const hk_tensor* k, const hk_tensor* v, float scale,
                                 int32_t causal, uint64_t qs, uint64_t ks, hk::AttnShape* sh) {
    if (!tensor_ok(q, "Q") || !tensor_ok(k, "K") || !tensor_ok(v, "V")) return HK_INVALID_ARGUMENT;
    if (q->rank != 4 || k->rank != 4 || v->rank != 4)
        return fail(HK_INVALID_ARGUMENT, "attention requires rank-4 Q[B,Hq,M,D], K/V[B,Hkv,N,D]");
    if ((q->dtype != HK_BF16 && q->dtype != HK_F32) || k->dtype != q->dtype || v->dtype != q->dtype)
        return fail(HK_INVALID_ARGUMENT, "fused attention requires Q/K/V all BF16 or all F32");
    const int64_t B = q->shape[0], H = q->shape[1], M = q->shape[2], D = q->shape[3];
    const int64_t Hkv = k->shape[1], N = k->shape[2];
    // Reference: validate_gqa / validate_dimensions, src/nn/attention.rs:81-104.
    if (H <= 0 || Hkv <= 0 || H % Hkv != 0 || k->shape[0] != B || v->shape[0] != B || v->shape[1] != Hkv ||
        k->shape[3] != D || v->shape[2] != N)
        return fail(HK_INVALID_ARGUMENT,
                    "GQA requires matching batches, positive divisible Q/KV heads and matching K/V lengths and Q/K widths");
    if (v->shape[3] != D) return fail(HK_INVALID_ARGUMENT, "fused attention requires the value width to equal D");
    if (B <= 0 || B * H > 4096 || M <= 0 || N <= 0 || M > INT32_MAX || N > INT32_MAX || !std::isfinite(scale))
        return fail(HK_INVALID_ARGUMENT,
                    "attention requires 1..4096 flattened batches, positive M/N within INT32_MAX and a finite scale");
    if (!(D == 16 || D == 32 || D == 64 || D == 128))
        return fail(HK_INVALID_ARGUMENT, "fused attention supports head dims 16, 32, 64 and 128 (got %lld)", (long long)D);
    if (causal && (qs > UINT64_MAX - static_cast<uint64_t>(M - 1) || ks > UINT64_MAX - static_cast<uint64_t>(N - 1)))
        return fail(HK_INVALID_ARGUMENT, "causal absolute position overflow");
    sh->batch = B;
    sh->heads = H;
    sh->kv_heads = Hkv;
    sh->m = M;
    sh->n = N;
    sh->d = D;
    sh->scale = scale;
    sh->causal = causal ? 1 : 0;
    sh->query_start = causal ? qs : 0;
    sh->key_start = causal ? ks : 0;
    // Rejected here, before any device work, so an oversized shape leaves the context healthy.
    if (!hk::attention_shape_fits(*sh))
        return fail(HK_INVALID_ARGUMENT,
                    "attention shape too large for the fused kernels: M*D and N*D must stay below 2^30 elements per "
                    "head and each launch below 2^32 work items (M=%lld N=%lld D=%lld)",
                    (long long)M, (long long)N, (long long)D);
    return HK_OK;
}

namespace {
// F32 Q/K/V/dO (the reference's FP32 attention surface) are rounded to BF16 (RNE) into the
// workspace before the fused kernels run, as the reference's matmul_bf16_fp32 rounds every GEMM
// operand; BF16 inputs are used in place.
struct Staged {
    const void* p;
    size_t bytes;  // workspace bytes it takes (0 when used in place)
};
Staged staged(const hk_tensor* t) {
    return {t->data, t->dtype == HK_F32 ? ws_round(static_cast<size_t>(numel(t)) * 2) : 0};
}
hipError_t stage(const hk_tensor* t, Staged& st, char*& cursor, hipStream_t s) {
    if (!st.bytes) return hipSuccess;
    st.p = cursor;
    cursor += st.bytes;
    return hk::cast_apply(1, t->data, const_cast<void*>(st.p), numel(t), s);
}
}  // namespace

hk_status hk_attention_forward(hk_context* h, const hk_tensor* q, const hk_tensor* k, const hk_tensor* v, float scale,
                               int32_t causal, uint64_t qs, uint64_t ks, hk_tensor* o, hk_tensor* lse) {
    hk::AttnShape sh;
    hk_status st = attention_shape(q, k, v, scale, causal, qs, ks, &sh);
    if (st != HK_OK) return st;
    if (!tensor_ok(o, "O") || !tensor_ok(lse, "lse")) return HK_INVALID_ARGUMENT;
    if ((o->dtype != HK_BF16 && o->dtype != HK_F32) || !same_shape(o, q))
        return fail(HK_INVALID_ARGUMENT, "O must be BF16 or F32 shaped like Q");
    if (lse->dtype != HK_F32 || lse->rank != 3 || lse->shape[0] != sh.batch || lse->shape[1] != sh.heads ||
        lse->shape[2] != sh.m)
        return fail(HK_INVALID_ARGUMENT, "lse must be F32 [B,Hq,M]");
    if (!disjoint({o, lse}, {q, k, v})) return HK_INVALID_ARGUMENT;
    sh.o_f32 = o->dtype == HK_F32;
    Staged sq = staged(q), sk = staged(k), sv = staged(v);
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    if ((st = ensure_workspace(g.c, sq.bytes + sk.bytes + sv.bytes)) != HK_OK) return st;
    char* cursor = static_cast<char*>(g.c->workspace);
    hipError_t e = stage(q, sq, cursor, g.c->stream);
    if (e == hipSuccess) e = stage(k, sk, cursor, g.c->stream);
    if (e == hipSuccess) e = stage(v, sv, cursor, g.c->stream);
    if (e == hipSuccess)
        e = hk::attention_forward(sh, sq.p, sk.p, sv.p, o->data, static_cast<float*>(lse->data), g.c->stream);
    return complete(g.c, e, "attention_forward", 1 + (sq.bytes ? 3 : 0));
}

namespace {
// The checks and the call of hk_attention_backward and its rows form (`rows` set: dQ/dK/dV go
// to the fused QKV gradient rows, and dq/dk/dv are null).
hk_status attention_backward_common(hk_context* h, const hk_tensor* q, const hk_tensor* k, const hk_tensor* v,
                                    const hk_tensor* o, const hk_tensor* lse, const hk_tensor* dout, float scale,
                                    int32_t causal, uint64_t qs, uint64_t ks, hk_tensor* dq, hk_tensor* dk,
                                    hk_tensor* dv, const hk_tensor* cos, const hk_tensor* sin, int32_t layout,
                                    hk_tensor* rows) {
    hk::AttnShape sh;
    hk_status st = attention_shape(q, k, v, scale, causal, qs, ks, &sh);
    if (st != HK_OK) return st;
    if (!tensor_ok(o, "O") || !tensor_ok(lse, "lse") || !tensor_ok(dout, "dO")) return HK_INVALID_ARGUMENT;
    if ((o->dtype != HK_BF16 && o->dtype != HK_F32) || !same_shape(o, q) ||
        (dout->dtype != HK_BF16 && dout->dtype != HK_F32) || !same_shape(dout, q))
        return fail(HK_INVALID_ARGUMENT, "O and dO must be BF16 or F32 shaped like Q");
    if (lse->dtype != HK_F32 || lse->rank != 3 || lse->shape[0] != sh.batch || lse->shape[1] != sh.heads ||
        lse->shape[2] != sh.m)
        return fail(HK_INVALID_ARGUMENT, "lse must be F32 [B,Hq,M]");
    hk::AttnRowsOut rows_out{};
    if (rows == nullptr) {
        if (!tensor_ok(dq, "dQ") || !tensor_ok(dk, "dK") || !tensor_ok(dv, "dV")) return HK_INVALID_ARGUMENT;
        if (!same_shape(dq, q) || !same_shape(dk, k) || !same_shape(dv, v))
            return fail(HK_INVALID_ARGUMENT, "dQ/dK/dV must have the shapes of Q/K/V");
        if ((dq->dtype != HK_F32 && dq->dtype != HK_BF16) || (dk->dtype != HK_F32 && dk->dtype != HK_BF16) ||
            dv->dtype != dk->dtype)
            return fail(HK_INVALID_ARGUMENT, "dQ/dK/dV must be F32 or BF16 (dK and dV alike)");
        if (!disjoint({dq, dk, dv}, {q, k, v, o, lse, dout})) return HK_INVALID_ARGUMENT;
    } else {
        const char* op = "attention_backward_qkv_rows";
        if (!tensor_ok(rows, "dQKV rows") || !tensor_ok(cos, "cos") || !tensor_ok(sin, "sin")) return HK_INVALID_ARGUMENT;
        if (layout != HK_ROTARY_INTERLEAVED && layout != HK_ROTARY_SPLIT_HALF)
            return fail(HK_INVALID_ARGUMENT, "rotary layout must be 0 (Interleaved) or 1 (SplitHalf)");
        if ((sh.d != 64 && sh.d != 128) || sh.m != sh.n)
            return fail(HK_INVALID_ARGUMENT, "%s requires heads of width 64 or 128 and as many keys as queries", op);
        const int64_t S = sh.m, D = sh.d, W = (sh.heads + 2 * sh.kv_heads) * D;
        if (!aligned_bf16({rows}, op)) return HK_INVALID_ARGUMENT;
        if (!dims_are(rows, {sh.batch, S, W}))
            return fail(HK_INVALID_ARGUMENT, "%s requires dQKV rows BF16 [B, S, (Hq+2Hkv)*D]", op);
        if (cos->dtype != HK_F32 || sin->dtype != HK_F32 || !dims_are(cos, {S, D / 2}) || !dims_are(sin, {S, D / 2}) ||
            reinterpret_cast<uintptr_t>(cos->data) % 16 != 0 || reinterpret_cast<uintptr_t>(sin->data) % 16 != 0)
            return fail(HK_INVALID_ARGUMENT, "%s requires 16-byte aligned F32 cos/sin tables [S, D/2]", op);
        if (!disjoint({rows}, {q, k, v, o, lse, dout, cos, sin})) return HK_INVALID_ARGUMENT;
        rows_out = hk::AttnRowsOut{rows->data, W, static_cast<const float*>(cos->data),
                                   static_cast<const float*>(sin->data), layout};
    }
    sh.o_f32 = o->dtype == HK_F32;
    Staged sq = staged(q), sk = staged(k), sv = staged(v), sd = staged(dout);
    const size_t staging = sq.bytes + sk.bytes + sv.bytes + sd.bytes;
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    hk::attention_bwd_plan(sh, g.c->num_cus);
    size_t stat_bytes = ws_round(hk::attention_bwd_workspace_bytes(sh));
    st = ensure_workspace(g.c, stat_bytes + staging);
    if (st == HK_HIP_ERROR && (sh.store_ds || sh.dkv_splits > 1)) {
        // the stored-dS buffer or the split's partial sums do not fit in free device memory (or
        // the workspace limit): the recompute form of dQ, unsplit, needs only the row statistics
        sh.store_ds = 0;
        sh.dkv_splits = 1;
        stat_bytes = ws_round(hk::attention_bwd_workspace_bytes(sh));
        st = ensure_workspace(g.c, stat_bytes + staging);
    }
    if (st != HK_OK) return st;
    char* cursor = static_cast<char*>(g.c->workspace) + stat_bytes;
    hipError_t e = stage(q, sq, cursor, g.c->stream);
    if (e == hipSuccess) e = stage(k, sk, cursor, g.c->stream);
    if (e == hipSuccess) e = stage(v, sv, cursor, g.c->stream);
    if (e == hipSuccess) e = stage(dout, sd, cursor, g.c->stream);
    if (e == hipSuccess)
        e = hk::attention_backward(sh, sq.p, sk.p, sv.p, o->data, static_cast<const float*>(lse->data), sd.p,
                                   rows ? nullptr : dq->data, rows ? 1 : dq->dtype == HK_BF16,
                                   rows ? nullptr : dk->data, rows ? nullptr : dv->data,
                                   rows ? 1 : dk->dtype == HK_BF16, rows ? &rows_out : nullptr, g.c->workspace,
                                   g.c->stream);
    return complete(g.c, e, rows ? "attention_backward_qkv_rows" : "attention_backward",
                    3 + (sq.bytes ? 3 : 0) + (sd.bytes ? 1 : 0));
}
}  // namespace

hk_status hk_attention_backward(hk_context* h, const hk_tensor* q, const hk_tensor* k, const hk_tensor* v,
                                const hk_tensor* o, const hk_tensor* lse, const hk_tensor* dout, float scale,
                                int32_t causal, uint64_t qs, uint64_t ks, hk_tensor* dq, hk_tensor* dk,
                                hk_tensor* dv) {
    return attention_backward_common(h, q, k, v, o, lse, dout, scale, causal, qs, ks, dq, dk, dv, nullptr, nullptr,
                                     0, nullptr);
}

hk_status hk_attention_backward_qkv_rows(hk_context* h, const hk_tensor* q, const hk_tensor* k, const hk_tensor* v,
                                         const hk_tensor* o, const hk_tensor* lse, const hk_tensor* dout, float scale,
                                         int32_t causal, uint64_t qs, uint64_t ks, const hk_tensor* cos,
                                         const hk_tensor* sin, int32_t layout, hk_tensor* dqkv) {
    return attention_backward_common(h, q, k, v, o, lse, dout, scale, causal, qs, ks, nullptr, nullptr, nullptr, cos,
                                     sin, layout, dqkv);
}

// ------------------------------------------------------------------ composed attention
//
// The reference's materialized attention (src/nn/attention.rs:10-67): additive masks, value widths
// other than the head width, and head widths the fused kernels do not take. Same rounding points as
// the reference's chain of matmul_bf16_fp32 / softmax: S = bf16(Q) bf16(K)^T (F32), S = S * scale
// (+ mask), P = softmax(S) (F32), O = bf16(P) bf16(V). GQA needs no repeated K/V: the Hq/Hkv query
// heads of one KV head are consecutive, so Q viewed as [B*Hkv, (Hq/Hkv)*M, D] multiplies that KV
// head's [N, D] directly, and the scores come out in the [B, Hq, M, N] layout of the mask.

namespace {

struct ComposedShape {
    int64_t batch = 0, heads = 1, kv_heads = 1, m = 0, n = 0, d = 0, dv = 0;
    int64_t groups() const { return batch * kv_heads; }      // GEMM batches: one per (b, KV head)
    int64_t rows() const { return heads / kv_heads * m; }    // query rows per GEMM batch
    int64_t scores() const { return batch * heads * m * n; }
};

hk_status composed_shape(const hk_tensor* q, const hk_tensor* k, const hk_tensor* v, float scale,
                         const hk_tensor* mask, ComposedShape* sh) {
    if (!tensor_ok(q, "Q") || !tensor_ok(k, "K") || !tensor_ok(v, "V")) return HK_INVALID_ARGUMENT;
    if (q->rank != k->rank || q->rank != v->rank || (q->rank != 3 && q->rank != 4))
        return fail(HK_INVALID_ARGUMENT,
                    "attention requires rank-3 Q[B,M,D], K[B,N,D], V[B,N,Dv] or rank-4 Q[B,Hq,M,D], K[B,Hkv,N,D], "
                    "V[B,Hkv,N,Dv]");
    if ((q->dtype != HK_F32 && q->dtype != HK_BF16) || k->dtype != q->dtype || v->dtype != q->dtype)
        return fail(HK_INVALID_ARGUMENT, "attention requires FP32 (or BF16) Q/K/V of one dtype");
    const bool r4 = q->rank == 4;
    const int o = r4 ? 1 : 0;
    const int64_t B = q->shape[0], H = r4 ? q->shape[1] : 1, M = q->shape[1 + o], D = q->shape[2 + o];
    const int64_t Hkv = r4 ? k->shape[1] : 1, N = k->shape[1 + o], Dv = v->shape[2 + o];
    // Reference: validate_gqa and validate_dimensions, src/nn/attention.rs:81-104.
    if (H <= 0 || Hkv <= 0 || H % Hkv != 0 || k->shape[0] != B || v->shape[0] != B || (r4 && v->shape[1] != Hkv) ||
        k->shape[2 + o] != D || v->shape[1 + o] != N)
        return fail(HK_INVALID_ARGUMENT,
                    "GQA requires matching batches, positive divisible Q/KV heads and matching K/V lengths and Q/K widths");
    const int64_t flat = B * H;
    auto aligned = [](int64_t x) { return x > 0 && x % 16 == 0 && x <= INT32_MAX; };
    if (flat <= 0 || flat > 4096 || !aligned(M) || !aligned(D) || !aligned(Dv) || N <= 0 || N > INT32_MAX ||
        N % 32 != 0 || !std::isfinite(scale) || flat * M * N > static_cast<int64_t>(UINT32_MAX))
        return fail(HK_INVALID_ARGUMENT,
                    "attention requires matching batches/contractions, aligned positive matrix dimensions, positive N "
                    "divisible by 32 within INT32_MAX, a finite FP32 scale and scores within u32");
    if (flat * N * std::max(D, Dv) > static_cast<int64_t>(UINT32_MAX))  // RepeatKvSpec::elements, heads_programs.rs:9-17
        return fail(HK_INVALID_ARGUMENT, "KV repetition complete domain exceeds u32");
    if (mask) {
        if (!tensor_ok(mask, "mask")) return HK_INVALID_ARGUMENT;
        const bool ok = mask->dtype == HK_F32 && mask->rank == q->rank && mask->shape[0] == B &&
                        (!r4 || mask->shape[1] == H) && mask->shape[1 + o] == M && mask->shape[2 + o] == N;
        if (!ok)
            return fail(HK_INVALID_ARGUMENT, r4 ? "GQA additive mask must be FP32 [B,Hq,M,N]"
                                               : "attention additive mask must be FP32 [B,M,N]");
    }
    sh->batch = B;
    sh->heads = H;
    sh->kv_heads = Hkv;
    sh->m = M;
    sh->n = N;
    sh->d = D;
    sh->dv = Dv;
    return HK_OK;
}

bool shaped_like(const hk_tensor* t, const hk_tensor* like, int64_t last) {
    if (t->rank != like->rank) return false;
    for (int i = 0; i + 1 < t->rank; ++i)
        if (t->shape[i] != like->shape[i]) return false;
    return t->shape[t->rank - 1] == last;
}

// Workspace carving for the composed path (256-byte aligned pieces).
struct Carve {
    char* base;
    size_t used = 0;
    void* take(size_t bytes) {
        void* p = base ? base + used : nullptr;
        used += ws_round(bytes);
        return p;
    }
};

// BF16 operand: `t` itself when BF16, else its RNE rounding into the workspace.
const void* bf16_operand(const hk_tensor* t, Carve& w, hipError_t* e, hipStream_t s) {
    if (t->dtype == HK_BF16) return t->data;
    void* p = w.take(static_cast<size_t>(numel(t)) * 2);
    if (w.base && *e == hipSuccess) *e = hk::cast_apply(1, t->data, p, numel(t), s);
    return p;
}

// S = bf16(Q) bf16(K)^T * scale (+ mask) and P = softmax(S), both F32 [B*Hkv, rows, N].
void composed_probs(const ComposedShape& sh, const void* qb, const void* kb, float scale, const hk_tensor* mask,
                    float* sbuf, float* p, void* gws, int num_cus, hipStream_t s, hipError_t* e) {
    const int64_t G = sh.groups(), R = sh.rows();
    if (*e == hipSuccess) *e = hk::gemm_bf16(qb, kb, sbuf, false, G, R, sh.n, sh.d, HK_NO, HK_YES, gws, num_cus, s);
    if (*e == hipSuccess)
        *e = hk::scale_mask(sbuf, mask ? static_cast<const float*>(mask->data) : nullptr, scale, sh.scores(), s);
    if (*e == hipSuccess) *e = hk::softmax_forward(sbuf, p, G * R, sh.n, 0, s);
}

size_t composed_gemm_ws(const ComposedShape& sh) {
    const int64_t G = sh.groups(), R = sh.rows();
    size_t w = hk::gemm_workspace_bytes(G, R, sh.n, sh.d, HK_NO, HK_YES);
    w = std::max(w, hk::gemm_workspace_bytes(G, R, sh.dv, sh.n, HK_NO, HK_NO));   // O, dQ (Dv or D wide)
    w = std::max(w, hk::gemm_workspace_bytes(G, R, sh.d, sh.n, HK_NO, HK_NO));
    w = std::max(w, hk::gemm_workspace_bytes(G, R, sh.n, sh.dv, HK_NO, HK_YES));  // dP
    w = std::max(w, hk::gemm_workspace_bytes(G, sh.n, sh.d, R, HK_YES, HK_NO));   // dK
    w = std::max(w, hk::gemm_workspace_bytes(G, sh.n, sh.dv, R, HK_YES, HK_NO));  // dV
    return w;
}

}  // namespace

hk_status hk_attention_masked_forward(hk_context* h, const hk_tensor* q, const hk_tensor* k, const hk_tensor* v,
                                      float scale, const hk_tensor* mask, hk_tensor* o) {
    ComposedShape sh;
    hk_status st = composed_shape(q, k, v, scale, mask, &sh);
    if (st != HK_OK) return st;
    if (!tensor_ok(o, "O")) return HK_INVALID_ARGUMENT;
    if ((o->dtype != HK_F32 && o->dtype != HK_BF16) || !shaped_like(o, q, sh.dv))
        return fail(HK_INVALID_ARGUMENT, "O must be F32 (or BF16) shaped like Q with the value width");
    if (mask ? !disjoint({o}, {q, k, v, mask}) : !disjoint({o}, {q, k, v})) return HK_INVALID_ARGUMENT;
    const int64_t G = sh.groups(), R = sh.rows();
    auto plan = [&](Carve& w, hipError_t* e, Ctx* c) {
        const void* qb = bf16_operand(q, w, e, c ? c->stream : nullptr);
        const void* kb = bf16_operand(k, w, e, c ? c->stream : nullptr);
        const void* vb = bf16_operand(v, w, e, c ? c->stream : nullptr);
        float* sbuf = static_cast<float*>(w.take(sh.scores() * 4));
        float* p = static_cast<float*>(w.take(sh.scores() * 4));
        void* pb = w.take(sh.scores() * 2);
        void* gws = w.take(composed_gemm_ws(sh));
        if (!c) return;
        composed_probs(sh, qb, kb, scale, mask, sbuf, p, gws, c->num_cus, c->stream, e);
        if (*e == hipSuccess) *e = hk::cast_apply(1, p, pb, sh.scores(), c->stream);
        if (*e == hipSuccess)
            *e = hk::gemm_bf16(pb, vb, o->data, o->dtype == HK_BF16, G, R, sh.dv, sh.n, HK_NO, HK_NO, gws,
                               c->num_cus, c->stream);
    };
    Carve size{nullptr};
    hipError_t e = hipSuccess;
    plan(size, &e, nullptr);
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    if ((st = ensure_workspace(g.c, size.used)) != HK_OK) return st;
    Carve w{static_cast<char*>(g.c->workspace)};
    plan(w, &e, g.c);
    return complete(g.c, e, "attention_masked_forward", 6);
}

hk_status hk_attention_masked_backward(hk_context* h, const hk_tensor* q, const hk_tensor* k, const hk_tensor* v,
                                       const hk_tensor* mask, const hk_tensor* dout, float scale, hk_tensor* dq,
                                       hk_tensor* dk, hk_tensor* dv, hk_tensor* dmask) {
    ComposedShape sh;
    hk_status st = composed_shape(q, k, v, scale, mask, &sh);
    if (st != HK_OK) return st;
    if (!tensor_ok(dout, "dO") || !tensor_ok(dq, "dQ") || !tensor_ok(dk, "dK") || !tensor_ok(dv, "dV"))
        return HK_INVALID_ARGUMENT;
    if ((dout->dtype != HK_F32 && dout->dtype != HK_BF16) || !shaped_like(dout, q, sh.dv))
        return fail(HK_INVALID_ARGUMENT, "dO must be F32 (or BF16) shaped like the output");
    if (!same_shape(dq, q) || !same_shape(dk, k) || !same_shape(dv, v) ||
        (dq->dtype != HK_F32 && dq->dtype != HK_BF16) || (dk->dtype != HK_F32 && dk->dtype != HK_BF16) ||
        dv->dtype != dk->dtype)
        return fail(HK_INVALID_ARGUMENT, "dQ/dK/dV must be F32 or BF16 (dK and dV alike) with the shapes of Q/K/V");
    if (dmask) {
        if (!mask) return fail(HK_INVALID_ARGUMENT, "a mask gradient needs the mask");
        if (!tensor_ok(dmask, "dMask")) return HK_INVALID_ARGUMENT;
        if (dmask->dtype != HK_F32 || !same_shape(dmask, mask))
            return fail(HK_INVALID_ARGUMENT, "the mask gradient must be F32 shaped like the mask");
    }
    std::vector<const hk_tensor*> ins = {q, k, v, dout};
    if (mask) ins.push_back(mask);
    std::vector<const hk_tensor*> outs = {dq, dk, dv};
    if (dmask) outs.push_back(dmask);
    for (size_t i = 0; i < outs.size(); ++i) {
        for (const hk_tensor* x : ins)
            if (overlaps(outs[i], x)) return fail(HK_INVALID_ARGUMENT, "output overlaps an input");
        for (size_t j = i + 1; j < outs.size(); ++j)
            if (overlaps(outs[i], outs[j])) return fail(HK_INVALID_ARGUMENT, "outputs overlap each other");
    }
    const int64_t G = sh.groups(), R = sh.rows();
    auto plan = [&](Carve& w, hipError_t* e, Ctx* c) {
        hipStream_t s = c ? c->stream : nullptr;
        const void* qb = bf16_operand(q, w, e, s);
        const void* kb = bf16_operand(k, w, e, s);
        const void* vb = bf16_operand(v, w, e, s);
        const void* dob = bf16_operand(dout, w, e, s);
        float* sbuf = static_cast<float*>(w.take(sh.scores() * 4));  // scores, then dP
        float* p = static_cast<float*>(w.take(sh.scores() * 4));
        float* ds = dmask ? static_cast<float*>(dmask->data) : static_cast<float*>(w.take(sh.scores() * 4));
        void* b16 = w.take(sh.scores() * 2);  // bf16(scale * dS), then bf16(P)
        void* gws = w.take(composed_gemm_ws(sh));
        if (!c) return;
        const int cus = c->num_cus;
        // recompute P (the reference keeps it in its autodiff graph)
        composed_probs(sh, qb, kb, scale, mask, sbuf, p, gws, cus, s, e);
        // dP = bf16(dO) bf16(V)^T; dS = P * (dP - rowsum(P * dP)) (softmax_backward); dMask = dS
        if (*e == hipSuccess) *e = hk::gemm_bf16(dob, vb, sbuf, false, G, R, sh.n, sh.dv, HK_NO, HK_YES, gws, cus, s);
        if (*e == hipSuccess) *e = hk::softmax_backward(p, sbuf, ds, G * R, sh.n, 0, s);
        // dQ = bf16(scale dS) bf16(K); dK = bf16(scale dS)^T bf16(Q) (the group's heads summed in the GEMM)
        if (*e == hipSuccess) *e = hk::scale_to_bf16(ds, scale, b16, sh.scores(), s);
        if (*e == hipSuccess)
            *e = hk::gemm_bf16(b16, kb, dq->data, dq->dtype == HK_BF16, G, R, sh.d, sh.n, HK_NO, HK_NO, gws, cus, s);
        if (*e == hipSuccess)
            *e = hk::gemm_bf16(b16, qb, dk->data, dk->dtype == HK_BF16, G, sh.n, sh.d, R, HK_YES, HK_NO, gws, cus, s);
        // dV = bf16(P)^T bf16(dO)
        if (*e == hipSuccess) *e = hk::cast_apply(1, p, b16, sh.scores(), s);
        if (*e == hipSuccess)
            *e = hk::gemm_bf16(b16, dob, dv->data, dv->dtype == HK_BF16, G, sh.n, sh.dv, R, HK_YES, HK_NO, gws, cus, s);
    };
    Carve size{nullptr};
    hipError_t e = hipSuccess;
    plan(size, &e, nullptr);
    OpGuard g(h);
    if (g.st != HK_OK) return g.st;
    if ((st = ensure_workspace(g.c, size.used)) != HK_OK) return st;
    Carve w{static_cast<char*>(g.c->workspace)};
    plan(w, &e, g.c);
    return complete(g.c, e, "attention_masked_backward", 11);
}

}  // extern "C"
