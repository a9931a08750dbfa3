// libluxgpu_backend_hip.so -- Lux GPU backend plugin for AMD Instinct MI355X.
//
// Host side: plugin entry (lux_gpu_backend_init), the ABI-v3 vtable, device /
// stream / buffer layer on HIP, and the quantized-matmul entry points of
// <lux/gpu/hip_quant.h>.  Kernels live in the other .hip files of this directory.
//
// Reference counterparts (luxcpp/webgpu):
//   plugin entry + vtable      src/webgpu_plugin.cpp:4018-4154
//   context / device info      src/webgpu_plugin.cpp:1218-1430
//   buffers                    src/webgpu_plugin.cpp:1432-1566
//   bounded waits              src/webgpu_plugin.cpp:61-83 (timeout -> DEVICE_LOST)
//   op_matmul_f32              src/webgpu_plugin.cpp:1721-1771
// Differences by design: a context owns a hipStream_t instead of a queue and a
// shared uniform buffer; kernel arguments travel with each launch, so ops on
// different contexts (or threads) never share parameter memory.
#include <algorithm>
#include <chrono>
#include <cstdarg>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "common.hpp"
#include "lux/gpu/backend_plugin.h"
#include "lux/gpu/hip_quant.h"

#define LUX_EXPORT extern "C" __attribute__((visibility("default")))

namespace {

using namespace luxhip;

thread_local std::string g_last_error;

LuxBackendError fail(LuxBackendError code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
LuxBackendError fail(LuxBackendError code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

struct HipCtx {
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    bool synchronous = true;
    double timeout_s = 5.0;
    std::string name;
    std::string force_fail;  // LUX_HIP_FORCE_FAIL test hook: op name that fails
    hipDeviceProp_t props{};
    void* ws = nullptr;      // device workspace (staged activations, partial sums), grown on demand
    size_t ws_size = 0;
    // Workspaces replaced by a larger one.  They stay allocated until destroy_context: a
    // HIP graph captured earlier on this context still holds their addresses.  Growth is
    // at least 2x, so the retired blocks together are smaller than the current one.
    std::vector<void*> ws_retired;
};

// Workspace of at least `bytes` on the context's device, in *out.  Growing it calls
// hipMalloc, which stream capture does not allow: a call inside capture that needs a
// larger workspace returns NOT_SUPPORTED (run the shape once eagerly before capturing).
// The old block is kept (not freed), so graphs captured before the growth replay
// unchanged.  Every op of a context shares the one workspace, so work on one context must
// not run concurrently with itself (graph replays included).
LuxBackendError get_workspace(HipCtx* c, size_t bytes, void** out, const char* op) {
    *out = nullptr;
    if (bytes <= c->ws_size) {
        *out = c->ws;
        return LUX_BACKEND_OK;
    }
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(c->stream, &cs) != hipSuccess) (void)hipGetLastError();
    if (cs != hipStreamCaptureStatusNone)
        return fail(LUX_BACKEND_ERROR_NOT_SUPPORTED,
                    "%s: workspace must grow to %zu bytes during stream capture; run this shape once "
                    "eagerly before capturing", op, bytes);
    size_t sz = std::max(bytes, 2 * c->ws_size);
    sz = (sz + 0xFFFFF) & ~(size_t)0xFFFFF;  // 1 MiB granules
    void* p = nullptr;
    if (hipMalloc(&p, sz) != hipSuccess) {
        (void)hipGetLastError();
        return fail(LUX_BACKEND_ERROR_OUT_OF_MEMORY, "%s: workspace allocation of %zu bytes failed", op, sz);
    }
    if (c->ws) c->ws_retired.push_back(c->ws);
    c->ws = p;
    c->ws_size = sz;
    *out = p;
    return LUX_BACKEND_OK;
}

// ---- fixed scratch of lux_hip_qmatmul_noalloc -------------------------------------
// One array per GPU, in the code object's device memory (allocated when the library's
// code is loaded on that device, held until the process ends).  In host code `scratch`
// names a host-side stand-in, not the device array: kernels and copies get the address
// from scratch_device_ptr(), which asks HIP for it once per device.
constexpr size_t kScratchBytes = LUX_HIP_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on `device`, which must be the current device.
LuxBackendError scratch_device_ptr(int device, void** out) {
    *out = nullptr;
    if (device < 0 || device >= kMaxDevices)
        return fail(LUX_BACKEND_ERROR_NOT_SUPPORTED, "qmatmul_noalloc: device %d beyond %d", device, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            (void)hipGetLastError();
            return fail(LUX_BACKEND_ERROR_INTERNAL, "qmatmul_noalloc: hipGetSymbolAddress(scratch) on device %d: %s",
                        device, hipGetErrorString(e));
        }
        g_scratch_ptr[device] = p;
    }
    *out = g_scratch_ptr[device];
    return LUX_BACKEND_OK;
}

struct HipBuf {
    void* ptr = nullptr;
    size_t size = 0;
    bool owned = true;
    int device = 0;
};

inline HipCtx* C(LuxBackendContext* c) { return reinterpret_cast<HipCtx*>(c); }
inline HipBuf* B(LuxBackendBuffer* b) { return reinterpret_cast<HipBuf*>(b); }

double env_double(const char* name, double dflt) {
    const char* v = getenv(name);
    if (!v || !*v) return dflt;
    char* end = nullptr;
    double d = strtod(v, &end);
    return (end && end != v && d >= 0.0) ? d : dflt;
}

// Bounded wait for the context stream (the counterpart of wgpu_wait_until,
// src/webgpu_plugin.cpp:74-82): spin on hipStreamQuery, back off after 1 ms,
// give up with DEVICE_LOST at the deadline.
LuxBackendError wait_stream(HipCtx* c) {
    const auto t0 = std::chrono::steady_clock::now();
    const auto deadline = t0 + std::chrono::duration<double>(c->timeout_s);
    for (;;) {
        hipError_t e = hipStreamQuery(c->stream);
        if (e == hipSuccess) return LUX_BACKEND_OK;
        if (e != hipErrorNotReady)
            return fail(LUX_BACKEND_ERROR_INTERNAL, "stream error: %s", hipGetErrorString(e));
        auto now = std::chrono::steady_clock::now();
        if (now > deadline)
            return fail(LUX_BACKEND_ERROR_DEVICE_LOST, "wait exceeded %.3f s", c->timeout_s);
        if (now - t0 > std::chrono::milliseconds(1))
            std::this_thread::sleep_for(std::chrono::microseconds(50));
    }
}

LuxBackendError begin_op(HipCtx* c, const char* op) {
    if (!c->force_fail.empty() && c->force_fail == op)
        return fail(LUX_BACKEND_ERROR_INTERNAL, "%s: forced failure (LUX_HIP_FORCE_FAIL)", op);
    hipError_t e = hipSetDevice(c->device);
    if (e != hipSuccess) return fail(LUX_BACKEND_ERROR_INTERNAL, "hipSetDevice: %s", hipGetErrorString(e));
    return LUX_BACKEND_OK;
}

LuxBackendError end_op(HipCtx* c, hipError_t launch, const char* op) {
    if (launch != hipSuccess)
        return fail(LUX_BACKEND_ERROR_INTERNAL, "%s: launch failed: %s", op, hipGetErrorString(launch));
    if (c->synchronous) return wait_stream(c);
    return LUX_BACKEND_OK;
}

// ---------------------------------------------------------------- lifecycle
LuxBackendContext* hip_create_context(int device_index) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        fail(LUX_BACKEND_ERROR_NOT_SUPPORTED, "no HIP device");
        return nullptr;
    }
    if (device_index < 0 || device_index >= n) {
        fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "device index %d out of range (%d)", device_index, n);
        return nullptr;
    }
    auto* c = new HipCtx();
    c->device = device_index;
    if (hipSetDevice(device_index) != hipSuccess ||
        hipGetDeviceProperties(&c->props, device_index) != hipSuccess ||
        hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        fail(LUX_BACKEND_ERROR_INTERNAL, "HIP device %d initialisation failed", device_index);
        return nullptr;
    }
    c->stream = c->own_stream;
    c->timeout_s = env_double("LUX_HIP_WAIT_TIMEOUT_S", 5.0);
    if (const char* f = getenv("LUX_HIP_FORCE_FAIL")) c->force_fail = f;
    c->name = c->props.name[0] ? c->props.name : "AMD GPU";
    c->name += " (";
    c->name += c->props.gcnArchName;
    c->name += ")";
    return reinterpret_cast<LuxBackendContext*>(c);
}

void hip_destroy_context(LuxBackendContext* ctx) {
    HipCtx* c = C(ctx);
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->own_stream) {
        (void)hipStreamSynchronize(c->own_stream);
        (void)hipStreamDestroy(c->own_stream);
    }
    if (c->ws) (void)hipFree(c->ws);
    for (void* p : c->ws_retired) (void)hipFree(p);
    delete c;
}

LuxBackendError hip_get_device_count(int* count) {
    if (!count) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "count is NULL");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
    *count = n;
    return LUX_BACKEND_OK;
}

LuxBackendError hip_get_device_info(LuxBackendContext* ctx, LuxBackendDeviceInfo* info) {
    if (!info) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "info is NULL");
    HipCtx* c = C(ctx);
    if (!c) return fail(LUX_BACKEND_ERROR_INTERNAL, "context is NULL");
    size_t free_b = 0, total_b = 0;
    (void)hipSetDevice(c->device);
    if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) {
        free_b = c->props.totalGlobalMem;
        total_b = c->props.totalGlobalMem;
    }
    info->name = c->name.c_str();
    info->vendor = "AMD HIP";
    info->memory_total = (uint64_t)total_b;
    info->memory_available = (uint64_t)free_b;
    info->compute_units = c->props.multiProcessorCount;
    info->max_workgroup_size = c->props.maxThreadsPerBlock;
    info->is_discrete = true;
    info->is_unified_memory = false;
    return LUX_BACKEND_OK;
}

LuxBackendError hip_sync(LuxBackendContext* ctx) {
    HipCtx* c = C(ctx);
    if (!c) return fail(LUX_BACKEND_ERROR_INTERNAL, "context is NULL");
    if (hipSetDevice(c->device) != hipSuccess) return fail(LUX_BACKEND_ERROR_INTERNAL, "hipSetDevice");
    return wait_stream(c);
}

// ---------------------------------------------------------------- buffers
LuxBackendBuffer* hip_buffer_alloc(LuxBackendContext* ctx, size_t bytes) {
    HipCtx* c = C(ctx);
    if (!c) return nullptr;
    (void)hipSetDevice(c->device);
    auto* b = new HipBuf();
    b->size = bytes;
    b->device = c->device;
    if (bytes > 0 && hipMalloc(&b->ptr, bytes) != hipSuccess) {
        (void)hipGetLastError();
        delete b;
        fail(LUX_BACKEND_ERROR_OUT_OF_MEMORY, "hipMalloc(%zu) failed", bytes);
        return nullptr;
    }
    return reinterpret_cast<LuxBackendBuffer*>(b);
}

LuxBackendError hip_buffer_copy_from_host(LuxBackendContext* ctx, LuxBackendBuffer* buf,
                                          const void* src, size_t bytes);

LuxBackendBuffer* hip_buffer_alloc_with_data(LuxBackendContext* ctx, const void* data, size_t bytes) {
    LuxBackendBuffer* b = hip_buffer_alloc(ctx, bytes);
    if (!b) return nullptr;
    if (data && bytes && hip_buffer_copy_from_host(ctx, b, data, bytes) != LUX_BACKEND_OK) {
        HipBuf* hb = B(b);
        (void)hipFree(hb->ptr);
        delete hb;
        return nullptr;
    }
    return b;
}

void hip_buffer_free(LuxBackendContext* ctx, LuxBackendBuffer* buf) {
    HipBuf* b = B(buf);
    if (!b) return;
    if (b->owned && b->ptr) {
        (void)hipSetDevice(b->device);
        if (HipCtx* c = C(ctx)) (void)hipStreamSynchronize(c->stream);
        (void)hipFree(b->ptr);
    }
    delete b;
}

LuxBackendError hip_buffer_copy_to_host(LuxBackendContext* ctx, LuxBackendBuffer* buf, void* dst,
                                        size_t bytes) {
    HipCtx* c = C(ctx);
    HipBuf* b = B(buf);
    if (!c || !b || !dst) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "copy_to_host: NULL argument");
    size_t n = std::min(bytes, b->size);  // clamp, as src/webgpu_plugin.cpp:1495
    if (n == 0) return LUX_BACKEND_OK;
    if (LuxBackendError e = begin_op(c, "buffer_copy_to_host")) return e;
    hipError_t he = hipMemcpyAsync(dst, b->ptr, n, hipMemcpyDeviceToHost, c->stream);
    if (he != hipSuccess) return fail(LUX_BACKEND_ERROR_INTERNAL, "D2H copy: %s", hipGetErrorString(he));
    return wait_stream(c);  // the host pointer must hold the data on return
}

LuxBackendError hip_buffer_copy_from_host(LuxBackendContext* ctx, LuxBackendBuffer* buf,
                                          const void* src, size_t bytes) {
    HipCtx* c = C(ctx);
    HipBuf* b = B(buf);
    if (!c || !b || !src) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "copy_from_host: NULL argument");
    size_t n = std::min(bytes, b->size);  // clamp, as src/webgpu_plugin.cpp:1553
    if (n == 0) return LUX_BACKEND_OK;
    if (LuxBackendError e = begin_op(c, "buffer_copy_from_host")) return e;
    hipError_t he = hipMemcpyAsync(b->ptr, src, n, hipMemcpyHostToDevice, c->stream);
    if (he != hipSuccess) return fail(LUX_BACKEND_ERROR_INTERNAL, "H2D copy: %s", hipGetErrorString(he));
    return wait_stream(c);  // the caller may reuse src on return
}

void* hip_buffer_get_host_ptr(LuxBackendContext*, LuxBackendBuffer*) {
    return nullptr;  // device memory is not host-visible (as src/webgpu_plugin.cpp:1564)
}

// ---------------------------------------------------------------- matmul
bool fits(const HipBuf* b, size_t need) { return b && (need == 0 || (b->ptr && b->size >= need)); }

LuxBackendError hip_op_matmul_f32(LuxBackendContext* ctx, LuxBackendBuffer* a, LuxBackendBuffer* b,
                                  LuxBackendBuffer* out, int M, int K, int N) {
    HipCtx* c = C(ctx);
    HipBuf *A = B(a), *Bm = B(b), *O = B(out);
    if (!c || !A || !Bm || !O) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "matmul: NULL argument");
    if (M < 0 || K < 0 || N < 0) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "matmul: negative size");
    const size_t m = M, k = K, n = N;
    if (!fits(A, m * k * 4) || !fits(Bm, k * n * 4) || !fits(O, m * n * 4))
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "matmul: buffer smaller than M*K/K*N/M*N floats");
    if (LuxBackendError e = begin_op(c, "op_matmul_f32")) return e;
    if (M == 0 || N == 0) return LUX_BACKEND_OK;
    const float* pa = static_cast<const float*>(A->ptr);
    const float* pb = static_cast<const float*>(Bm->ptr);
    float* po = static_cast<float*>(O->ptr);
    hipError_t he;
    if (K == 0) {
        he = launch_fill_f32(po, m * n, 0.0f, c->stream);
    } else if (N == 1) {
        // GEMV: C[M] = A[M x K] . B[K]  (the reference runs this through the 16x16
        // GEMM with 15/16 lanes idle, src/webgpu_plugin.cpp:1759-1763).
        he = launch_gemv_f32(pa, pb, po, M, K, K, 1.0f, 0.0f, c->stream);
    } else if (M == 1) {
        // Row vector: C[N] = B^T[N x K] . a[K].
        void* ws = nullptr;
        if (LuxBackendError e = get_workspace(c, gemv_t_workspace(K, N), &ws, "op_matmul_f32")) return e;
        he = launch_gemv_f32_t(pb, pa, po, K, N, N, 1.0f, 0.0f, static_cast<float*>(ws), c->stream);
    } else {
        he = launch_gemm_f32(pa, pb, po, M, K, N, c->stream);
    }
    return end_op(c, he, "op_matmul_f32");
}

// Elementwise slots (src/webgpu_plugin.cpp:1637-1719, WGSL_BINARY_OPS :92-135): out[i] =
// a[i] op b[i] for i < n, strides 1.  The reference leaves op_div_f32 NOT_SUPPORTED
// (:3548); it is filled here with the same elementwise form.
LuxBackendError hip_binary(LuxBackendContext* ctx, LuxBackendBuffer* a, LuxBackendBuffer* b, LuxBackendBuffer* out,
                           size_t n, int op, const char* name) {
    HipCtx* c = C(ctx);
    HipBuf *A = B(a), *Bb = B(b), *O = B(out);
    if (!c || !A || !Bb || !O) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "%s: NULL argument", name);
    if (!fits(A, n * 4) || !fits(Bb, n * 4) || !fits(O, n * 4))
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "%s: buffer smaller than %zu floats", name, n);
    if (LuxBackendError e = begin_op(c, name)) return e;
    if (n == 0) return LUX_BACKEND_OK;
    return end_op(c, launch_binary_f32(op, static_cast<const float*>(A->ptr), static_cast<const float*>(Bb->ptr),
                                       static_cast<float*>(O->ptr), n, c->stream),
                  name);
}
LuxBackendError hip_op_add_f32(LuxBackendContext* c, LuxBackendBuffer* a, LuxBackendBuffer* b, LuxBackendBuffer* o,
                               size_t n) {
    return hip_binary(c, a, b, o, n, 0, "op_add_f32");
}
LuxBackendError hip_op_sub_f32(LuxBackendContext* c, LuxBackendBuffer* a, LuxBackendBuffer* b, LuxBackendBuffer* o,
                               size_t n) {
    return hip_binary(c, a, b, o, n, 1, "op_sub_f32");
}
LuxBackendError hip_op_mul_f32(LuxBackendContext* c, LuxBackendBuffer* a, LuxBackendBuffer* b, LuxBackendBuffer* o,
                               size_t n) {
    return hip_binary(c, a, b, o, n, 2, "op_mul_f32");
}
LuxBackendError hip_op_div_f32(LuxBackendContext* c, LuxBackendBuffer* a, LuxBackendBuffer* b, LuxBackendBuffer* o,
                               size_t n) {
    return hip_binary(c, a, b, o, n, 3, "op_div_f32");
}

// ---------------------------------------------------------------- vtable
const lux_gpu_backend_vtbl g_vtbl = [] {
    lux_gpu_backend_vtbl v;
    std::memset(&v, 0, sizeof v);  // every slot not named below stays NULL -> CPU fallback
    v.create_context = hip_create_context;
    v.destroy_context = hip_destroy_context;
    v.get_device_count = hip_get_device_count;
    v.get_device_info = hip_get_device_info;
    v.sync = hip_sync;
    v.buffer_alloc = hip_buffer_alloc;
    v.buffer_alloc_with_data = hip_buffer_alloc_with_data;
    v.buffer_free = hip_buffer_free;
    v.buffer_copy_to_host = hip_buffer_copy_to_host;
    v.buffer_copy_from_host = hip_buffer_copy_from_host;
    v.buffer_get_host_ptr = hip_buffer_get_host_ptr;
    v.op_add_f32 = hip_op_add_f32;
    v.op_sub_f32 = hip_op_sub_f32;
    v.op_mul_f32 = hip_op_mul_f32;
    v.op_div_f32 = hip_op_div_f32;
    v.op_matmul_f32 = hip_op_matmul_f32;
    return v;
}();

// ---------------------------------------------------------------- quantized
size_t dtype_bytes(int dt) {
    switch (dt) {
        case LUX_HIP_F32: case LUX_HIP_I32: return 4;
        case LUX_HIP_F16: case LUX_HIP_BF16: return 2;
        case LUX_HIP_I8: return 1;
        default: return 0;
    }
}

size_t scale_bytes(int fmt) {
    switch (fmt) {
        case LUX_HIP_SCALE_F16: return 2;
        case LUX_HIP_SCALE_F32: return 4;
        case LUX_HIP_SCALE_GROUPSCALE: return 16;
        default: return 0;
    }
}

}  // namespace

// ============================================================== exports
LUX_EXPORT bool lux_gpu_backend_init(lux_gpu_backend_desc* out) {
    if (!out) return false;
    out->abi_version = LUX_GPU_BACKEND_ABI_VERSION;
    out->vtbl_size = (uint32_t)sizeof(lux_gpu_backend_vtbl);
    out->backend_name = "hip";
    out->backend_version = "0.1.0";
    out->capabilities = LUX_CAP_TENSOR_OPS | LUX_CAP_MATMUL;
    out->vtbl = &g_vtbl;
    return true;
}

LUX_EXPORT uint32_t lux_hip_quant_api_version(void) { return LUX_HIP_QUANT_API_VERSION; }

LUX_EXPORT const char* lux_hip_last_error(void) { return g_last_error.c_str(); }

LUX_EXPORT LuxBackendBuffer* lux_hip_buffer_wrap(LuxBackendContext* ctx, void* device_ptr, size_t bytes) {
    HipCtx* c = C(ctx);
    if (!c || (!device_ptr && bytes)) {
        fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "buffer_wrap: NULL argument");
        return nullptr;
    }
    auto* b = new HipBuf();
    b->ptr = device_ptr;
    b->size = bytes;
    b->owned = false;
    b->device = c->device;
    return reinterpret_cast<LuxBackendBuffer*>(b);
}

LUX_EXPORT void* lux_hip_buffer_device_ptr(LuxBackendBuffer* buf) { return buf ? B(buf)->ptr : nullptr; }
LUX_EXPORT size_t lux_hip_buffer_size(LuxBackendBuffer* buf) { return buf ? B(buf)->size : 0; }

LUX_EXPORT LuxBackendError lux_hip_context_set_stream(LuxBackendContext* ctx, void* stream) {
    HipCtx* c = C(ctx);
    if (!c) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "set_stream: NULL context");
    c->stream = stream ? static_cast<hipStream_t>(stream) : c->own_stream;
    return LUX_BACKEND_OK;
}

LUX_EXPORT void* lux_hip_context_get_stream(LuxBackendContext* ctx) {
    HipCtx* c = C(ctx);
    return c ? static_cast<void*>(c->stream) : nullptr;
}

LUX_EXPORT LuxBackendError lux_hip_context_set_synchronous(LuxBackendContext* ctx, int synchronous) {
    HipCtx* c = C(ctx);
    if (!c) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "set_synchronous: NULL context");
    c->synchronous = synchronous != 0;
    return LUX_BACKEND_OK;
}

LUX_EXPORT LuxBackendError lux_hip_gemv_f32(LuxBackendContext* ctx, LuxBackendBuffer* a,
                                            LuxBackendBuffer* x, LuxBackendBuffer* y,
                                            const LuxHipGemvParams* p) {
    HipCtx* c = C(ctx);
    HipBuf *A = B(a), *X = B(x), *Y = B(y);
    if (!c || !A || !X || !Y || !p) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "gemv_f32: NULL argument");
    const size_t M = p->M, N = p->N, lda = p->lda;
    if (lda < N || M > INT32_MAX || N > INT32_MAX || lda > INT32_MAX)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "gemv_f32: lda < N or size too large");
    const size_t a_need = M ? ((M - 1) * lda + N) * 4 : 0;
    const size_t x_need = (p->trans ? M : N) * 4, y_need = (p->trans ? N : M) * 4;
    if (!fits(A, a_need) || !fits(X, x_need) || !fits(Y, y_need))
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "gemv_f32: buffer too small");
    if (LuxBackendError e = begin_op(c, "gemv_f32")) return e;
    const size_t outn = p->trans ? N : M;
    if (outn == 0) return LUX_BACKEND_OK;
    hipError_t he;
    if (p->trans) {
        void* ws = nullptr;
        if (LuxBackendError e = get_workspace(c, gemv_t_workspace((int)M, (int)N), &ws, "gemv_f32")) return e;
        he = launch_gemv_f32_t((const float*)A->ptr, (const float*)X->ptr, (float*)Y->ptr, (int)M, (int)N,
                               (int)lda, p->alpha, p->beta, static_cast<float*>(ws), c->stream);
    }
    else {
        he = launch_gemv_f32((const float*)A->ptr, (const float*)X->ptr, (float*)Y->ptr, (int)M, (int)N,
                             (int)lda, p->alpha, p->beta, c->stream);
    }
    return end_op(c, he, "gemv_f32");
}

LUX_EXPORT LuxBackendError lux_hip_gemv_f32_batched(LuxBackendContext* ctx, LuxBackendBuffer* a,
                                                    LuxBackendBuffer* x, LuxBackendBuffer* y,
                                                    const LuxHipGemvBatchedParams* p) {
    HipCtx* c = C(ctx);
    HipBuf *A = B(a), *X = B(x), *Y = B(y);
    if (!c || !A || !X || !Y || !p)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "gemv_f32_batched: NULL argument");
    const size_t M = p->M, N = p->N, lda = p->lda, nb = p->batch_count;
    const size_t sa = p->stride_a, sx = p->stride_x, sy = p->stride_y;
    if (lda < N || M > INT32_MAX || N > INT32_MAX || lda > INT32_MAX || nb > INT32_MAX)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "gemv_f32_batched: lda < N or size too large");
    if (nb > 1 && M > 0 && sy < M)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT,
                    "gemv_f32_batched: stride_y %zu < M %zu makes the y vectors overlap", sy, M);
    if (M > 0 && nb > 0) {
        const size_t a_need = ((nb - 1) * sa + (M - 1) * lda + N) * 4;
        const size_t x_need = ((nb - 1) * sx + N) * 4, y_need = ((nb - 1) * sy + M) * 4;
        if (!fits(A, a_need) || !fits(X, x_need) || !fits(Y, y_need))
            return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "gemv_f32_batched: buffer too small");
    }
    if (LuxBackendError e = begin_op(c, "gemv_f32_batched")) return e;
    if (M == 0 || nb == 0) return LUX_BACKEND_OK;
    hipError_t he = launch_gemv_f32_batched((const float*)A->ptr, (const float*)X->ptr, (float*)Y->ptr,
                                            (int)M, (int)N, (int)lda, p->alpha, p->beta, (int)nb, sa, sx,
                                            sy, c->stream);
    return end_op(c, he, "gemv_f32_batched");
}

LUX_EXPORT LuxBackendError lux_hip_dot_f16(LuxBackendContext* ctx, LuxBackendBuffer* a, LuxBackendBuffer* b,
                                           LuxBackendBuffer* result, const LuxHipDotParams* p) {
    HipCtx* c = C(ctx);
    HipBuf *A = B(a), *Bv = B(b), *R = B(result);
    if (!c || !A || !Bv || !R || !p) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "dot_f16: NULL argument");
    const size_t size = p->size, nv = p->num_vectors, stride = p->vector_stride;
    if (size > INT32_MAX || nv > INT32_MAX)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "dot_f16: size too large");
    if (nv > 0) {
        const size_t need = (2 * ((nv - 1) * stride / 2) + size) * 2;  // bytes of a and b
        if (!fits(A, need) || !fits(Bv, need) || !fits(R, nv * 4))
            return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "dot_f16: buffer too small");
    }
    if (LuxBackendError e = begin_op(c, "dot_f16")) return e;
    if (nv == 0) return LUX_BACKEND_OK;
    return end_op(c, launch_dot_f16(A->ptr, Bv->ptr, (float*)R->ptr, (int)size, (int)nv, stride, c->stream),
                  "dot_f16");
}

LUX_EXPORT LuxBackendError lux_hip_gemv_f16(LuxBackendContext* ctx, LuxBackendBuffer* a,
                                            LuxBackendBuffer* x, LuxBackendBuffer* y, uint32_t M,
                                            uint32_t N, uint32_t lda) {
    HipCtx* c = C(ctx);
    HipBuf *A = B(a), *X = B(x), *Y = B(y);
    if (!c || !A || !X || !Y) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "gemv_f16: NULL argument");
    if (lda < N || M > INT32_MAX || lda > INT32_MAX)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "gemv_f16: lda < N or size too large");
    const size_t a_need = M ? (((size_t)M - 1) * lda + N) * 2 : 0;
    if (!fits(A, a_need) || !fits(X, (size_t)N * 2) || !fits(Y, (size_t)M * 4))
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "gemv_f16: buffer too small");
    if (LuxBackendError e = begin_op(c, "gemv_f16")) return e;
    if (M == 0) return LUX_BACKEND_OK;
    hipError_t he = launch_gemv_f16(A->ptr, X->ptr, (float*)Y->ptr, (int)M, (int)N, (int)lda, c->stream);
    return end_op(c, he, "gemv_f16");
}

namespace {
// noalloc: staging buffers come from the device's fixed `scratch` array (at most
// kScratchBytes) instead of the context workspace; nothing is allocated.
// ws_offset: the first ws_offset bytes of the context workspace hold a caller's data
// (rms_norm_qmatmul's normalised rows) and are left alone.
// rn: x is the row before rms_norm, normalised by the GEMV itself (the caller checked
// qgemv_i4_rn_supported; x_dtype F16 names the normalised row's type).
LuxBackendError qmatmul_impl(LuxBackendContext* ctx, const LuxHipQMatmulDesc* d, LuxBackendBuffer* w,
                             LuxBackendBuffer* w_scales, LuxBackendBuffer* x, LuxBackendBuffer* x_scales,
                             int epilogue, LuxBackendBuffer* bias, LuxBackendBuffer* residual,
                             LuxBackendBuffer* y, bool noalloc = false, size_t ws_offset = 0,
                             const RnArgs* rn = nullptr) {
    HipCtx* c = C(ctx);
    if (!c || !d || !w || !x || !y) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "qmatmul: NULL argument");
    if (epilogue < LUX_HIP_EPILOGUE_NONE || epilogue > LUX_HIP_EPILOGUE_SILU_MUL)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "qmatmul: bad epilogue %d", epilogue);
    const bool silu_mul = epilogue == LUX_HIP_EPILOGUE_SILU_MUL;
    if (d->struct_size < sizeof(LuxHipQMatmulDesc))
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "qmatmul: struct_size %u too small", d->struct_size);
    const int n_out = d->n_out, K = d->k, M = d->m, gs = d->group_size;
    if (n_out < 0 || K < 0 || M < 0) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "qmatmul: negative size");
    if (d->weight_bits != 4 && d->weight_bits != 8)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "qmatmul: weight_bits must be 4 or 8");
    if (K % 32 != 0) return fail(LUX_BACKEND_ERROR_NOT_SUPPORTED, "qmatmul: k %% 32 != 0");
    // QUANTIZE_X: fp activations are quantized per token to int8 first (W4A8 prologue)
    const bool qx = (d->flags & LUX_HIP_QFLAG_QUANTIZE_X) != 0;
    if (qx && !((d->x_dtype == LUX_HIP_F32 || d->x_dtype == LUX_HIP_F16 || d->x_dtype == LUX_HIP_BF16) &&
                d->y_dtype != LUX_HIP_I32 && d->scale_format != LUX_HIP_SCALE_NONE && !x_scales))
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT,
                    "qmatmul: QUANTIZE_X needs fp x and y, weight scales and no x_scales");
    const bool w4a8 = d->x_dtype == LUX_HIP_I8 || qx;
    const bool no_scale = d->scale_format == LUX_HIP_SCALE_NONE;
    if (!no_scale && (gs <= 0 || K % gs != 0 || gs % 8 != 0))
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "qmatmul: group_size %d must divide k and be a multiple of 8", gs);
    if (d->nibble_coding != LUX_HIP_NIBBLE_OFFSET_BINARY && d->nibble_coding != LUX_HIP_NIBBLE_TWOS_COMPLEMENT)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "qmatmul: bad nibble_coding");
    const size_t xb = dtype_bytes(d->x_dtype), yb = dtype_bytes(d->y_dtype);
    if (!xb || !yb || (d->x_dtype == LUX_HIP_I32) || (!w4a8 && d->y_dtype == LUX_HIP_I32))
        return fail(LUX_BACKEND_ERROR_NOT_SUPPORTED, "qmatmul: dtype combination");
    if (scale_bytes(d->scale_format) == 0 && !no_scale)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "qmatmul: bad scale_format");
    const bool partials = (d->flags & LUX_HIP_QFLAG_GROUP_PARTIALS) != 0;
    if (partials && !(w4a8 && d->y_dtype == LUX_HIP_I32 && !no_scale))
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "qmatmul: GROUP_PARTIALS needs W4A8, I32 out and a group_size");

    if (epilogue != LUX_HIP_EPILOGUE_NONE && w4a8)
        return fail(LUX_BACKEND_ERROR_NOT_SUPPORTED, "qmatmul: epilogues are not fused into the W4A8/W8A8 kernel");
    if (silu_mul && n_out % 2 != 0)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "qmatmul: SILU_MUL needs an even n_out (gate rows, then up rows)");
    const int ny = silu_mul ? n_out / 2 : n_out;  // output columns
    const size_t wn = (size_t)n_out * K * d->weight_bits / 8;
    const size_t groups = no_scale ? 0 : (size_t)n_out * (K / gs);
    const size_t yn = partials ? (size_t)M * n_out * (K / gs) * 4 : (size_t)M * ny * yb;
    HipBuf *W = B(w), *S = B(w_scales), *X = B(x), *XS = B(x_scales), *Y = B(y);
    HipBuf *BI = B(bias), *RE = B(residual);
    if (epilogue == LUX_HIP_EPILOGUE_ADD_BIAS && !fits(BI, (size_t)ny * 4))
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "qmatmul: ADD_BIAS needs an f32 bias of n_out elements");
    if (epilogue == LUX_HIP_EPILOGUE_ADD_RESIDUAL && !fits(RE, (size_t)M * ny * 4))
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "qmatmul: ADD_RESIDUAL needs an f32 residual of m x n_out");
    if (!fits(W, wn) || !fits(X, (size_t)M * K * xb) || !fits(Y, yn))
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "qmatmul: weight/activation/output buffer too small");
    if (!no_scale && !fits(S, groups * scale_bytes(d->scale_format)))
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "qmatmul: scale buffer too small");
    const bool need_xs = w4a8 && d->y_dtype != LUX_HIP_I32 && !qx;
    if (need_xs && !fits(XS, (size_t)M * 4))
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "qmatmul: x_scales (f32 [m]) required for W4A8 fp output");
    // Natural alignment of every element type (wrapped views may start anywhere); the
    // kernels' 16-byte vector paths check their own stronger requirements and fall back
    // or refuse.  QUANTIZE_X reads x with 16-byte loads.
    {
        const uintptr_t wa = (uintptr_t)W->ptr, xa = (uintptr_t)X->ptr, ya = (uintptr_t)Y->ptr;
        const uintptr_t sa = no_scale ? 0 : (uintptr_t)S->ptr;
        const size_t sal = no_scale ? 1 : std::min<size_t>(scale_bytes(d->scale_format), 4);
        if ((d->weight_bits == 4 && (wa & 3u)) || (sa & (sal - 1)) || (xa & (xb - 1)) || (ya & (yb - 1)) ||
            (qx && (xa & 15u)) || (need_xs && ((uintptr_t)XS->ptr & 3u)))
            return fail(LUX_BACKEND_ERROR_NOT_SUPPORTED,
                        "qmatmul: misaligned buffer (w, scales, x or y not naturally aligned, or x not 16-byte "
                        "aligned for QUANTIZE_X)");
    }

    if (LuxBackendError e = begin_op(c, "qmatmul")) return e;
    if (M == 0 || n_out == 0) return LUX_BACKEND_OK;
    auto workspace = [&](size_t bytes, void** out) -> LuxBackendError {
        if (!noalloc) {
            void* base = nullptr;
            if (LuxBackendError e = get_workspace(c, ws_offset + bytes, &base, "qmatmul")) return e;
            *out = static_cast<unsigned char*>(base) + ws_offset;
            return LUX_BACKEND_OK;
        }
        if (bytes > kScratchBytes)
            return fail(LUX_BACKEND_ERROR_NOT_SUPPORTED,
                        "qmatmul_noalloc: this shape needs %zu bytes of scratch, above the maximum of %zu", bytes,
                        kScratchBytes);
        return scratch_device_ptr(c->device, out);
    };

    QArgs a{};
    a.w = W->ptr;
    a.s = no_scale ? nullptr : S->ptr;
    a.x = X->ptr;
    a.xs = need_xs ? static_cast<const float*>(XS->ptr) : nullptr;
    a.y = Y->ptr;
    a.n_out = n_out;
    a.k = K;
    a.m = M;
    a.group_size = no_scale ? K : gs;
    a.wbits = d->weight_bits;
    a.scale_kind = static_cast<ScaleKind>(d->scale_format);
    a.x_kind = static_cast<XKind>(d->x_dtype);
    a.y_kind = static_cast<YKind>(d->y_dtype);
    a.group_partials = partials;
    a.epi.kind = epilogue;
    a.epi.bias = epilogue == LUX_HIP_EPILOGUE_ADD_BIAS ? static_cast<const float*>(BI->ptr) : nullptr;
    a.epi.residual = epilogue == LUX_HIP_EPILOGUE_ADD_RESIDUAL ? static_cast<const float*>(RE->ptr) : nullptr;
    // Kernels decode offset-binary nibbles; two's complement becomes offset-binary
    // with one xor per word (ob = tc ^ 0x8, quantized.wgsl:152 vs quantized_nax.wgsl:109).
    a.xor_mask = (d->weight_bits == 4 && d->nibble_coding == LUX_HIP_NIBBLE_TWOS_COMPLEMENT) ? 0x88888888u : 0u;

    hipError_t he;
    if (rn) {
        a.rn = *rn;
        if (w4a8 || !qgemv_i4_rn_supported(a))
            return fail(LUX_BACKEND_ERROR_INTERNAL, "qmatmul: fused rms_norm on a path without it");
        he = launch_qgemv_i4(a, c->stream);
    } else if (w4a8) {
        if (qx) {  // int8 activations and their f32 per-token scales in the workspace
            a.x_kind = XKind::I8;
            void* wsv = nullptr;
            if (LuxBackendError e = workspace((size_t)M * K + (size_t)M * 4, &wsv)) return e;
            uint8_t* ws = static_cast<uint8_t*>(wsv);
            a.x = ws;
            a.xs = reinterpret_cast<const float*>(ws + (size_t)M * K);
            if (!w4a8_supported(a))
                return fail(LUX_BACKEND_ERROR_NOT_SUPPORTED, "qmatmul: W4A8/W8A8 shape/format not supported");
            QuantArgs qa{};
            qa.x = X->ptr;
            qa.q = ws;
            qa.s = ws + (size_t)M * K;  // k % 32 == 0: 4-byte aligned
            qa.rows = M;
            qa.k = K;
            qa.group_size = K;
            qa.bits = 8;
            qa.offset_binary = true;
            qa.scale_kind = ScaleKind::F32;
            qa.x_kind = static_cast<XKind>(d->x_dtype);
            if (hipError_t qe = launch_quantize(qa, c->stream); qe != hipSuccess)
                return end_op(c, qe, "qmatmul (activation quantization)");
        }
        if (!w4a8_supported(a))
            return fail(LUX_BACKEND_ERROR_NOT_SUPPORTED, "qmatmul: W4A8/W8A8 shape/format not supported");
        he = launch_w4a8(a, c->stream);
    } else if (d->weight_bits == 4 && M == 1 && (!silu_mul || qgemv_i4_fast(a))) {
        he = launch_qgemv_i4(a, c->stream);
    } else if (M <= 64 && qgemm_small_supported(a)) {
        // decode batches: bandwidth regime, weights streamed once per 64 tokens
        const size_t wsb = qgemm_small_workspace(a);
        void* ws = nullptr;
        if (wsb)
            if (LuxBackendError e = workspace(wsb, &ws)) return e;
        he = launch_qgemm_small(a, ws, c->stream);
    } else if (d->weight_bits == 4 && qgemm_i4_large_supported(a)) {
        void* ws = nullptr;
        if (LuxBackendError e = workspace(qgemm_i4_large_workspace(a), &ws)) return e;
        he = launch_qgemm_i4_large(a, ws, c->stream);
    } else if (qgemm_small_supported(a)) {
        const size_t wsb = qgemm_small_workspace(a);
        void* ws = nullptr;
        if (wsb)
            if (LuxBackendError e = workspace(wsb, &ws)) return e;
        he = launch_qgemm_small(a, ws, c->stream);
    } else {
        return fail(LUX_BACKEND_ERROR_NOT_SUPPORTED, "qmatmul: no kernel for this descriptor");
    }
    return end_op(c, he, "qmatmul");
}
}  // namespace

LUX_EXPORT LuxBackendError lux_hip_qmatmul(LuxBackendContext* ctx, const LuxHipQMatmulDesc* d,
                                           LuxBackendBuffer* w, LuxBackendBuffer* w_scales,
                                           LuxBackendBuffer* x, LuxBackendBuffer* x_scales,
                                           LuxBackendBuffer* y) {
    return qmatmul_impl(ctx, d, w, w_scales, x, x_scales, LUX_HIP_EPILOGUE_NONE, nullptr, nullptr, y);
}

LUX_EXPORT LuxBackendError lux_hip_qmatmul_ex(LuxBackendContext* ctx, const LuxHipQMatmulDesc* d,
                                              LuxBackendBuffer* w, LuxBackendBuffer* w_scales,
                                              LuxBackendBuffer* x, LuxBackendBuffer* x_scales, int epilogue,
                                              LuxBackendBuffer* bias, LuxBackendBuffer* residual,
                                              LuxBackendBuffer* y) {
    return qmatmul_impl(ctx, d, w, w_scales, x, x_scales, epilogue, bias, residual, y);
}

LUX_EXPORT LuxBackendError lux_hip_qmatmul_noalloc(LuxBackendContext* ctx, const LuxHipQMatmulDesc* d,
                                                   LuxBackendBuffer* w, LuxBackendBuffer* w_scales,
                                                   LuxBackendBuffer* x, LuxBackendBuffer* x_scales, int epilogue,
                                                   LuxBackendBuffer* bias, LuxBackendBuffer* residual,
                                                   LuxBackendBuffer* y) {
    return qmatmul_impl(ctx, d, w, w_scales, x, x_scales, epilogue, bias, residual, y, true);
}

// ---------------------------------------------------------------- producers / codecs
// Symmetric group quantizer: compute_group_scales + quantize_nax_int4_sym /
// quantize_nax_int8_group (quantized_nax.wgsl:157-262,336-362) in one pass.
LUX_EXPORT LuxBackendError lux_hip_quantize(LuxBackendContext* ctx, const LuxHipQuantizeDesc* d,
                                            LuxBackendBuffer* x, LuxBackendBuffer* q,
                                            LuxBackendBuffer* scales) {
    HipCtx* c = C(ctx);
    if (!c || !d || !x || !q || !scales) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "quantize: NULL argument");
    if (d->struct_size < sizeof(LuxHipQuantizeDesc))
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "quantize: struct_size %u too small", d->struct_size);
    const int rows = d->rows, K = d->k, gs = d->group_size;
    if (rows < 0 || K < 0) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "quantize: negative size");
    if (d->weight_bits != 4 && d->weight_bits != 8)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "quantize: weight_bits must be 4 or 8");
    if (gs < 8 || (gs & (gs - 1)) != 0 || K % gs != 0)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "quantize: group_size %d must be a power of two >= 8 dividing k", gs);
    if (d->nibble_coding != LUX_HIP_NIBBLE_OFFSET_BINARY && d->nibble_coding != LUX_HIP_NIBBLE_TWOS_COMPLEMENT)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "quantize: bad nibble_coding");
    if (d->x_dtype != LUX_HIP_F32 && d->x_dtype != LUX_HIP_F16 && d->x_dtype != LUX_HIP_BF16)
        return fail(LUX_BACKEND_ERROR_NOT_SUPPORTED, "quantize: x_dtype must be F32, F16 or BF16");
    if (scale_bytes(d->scale_format) == 0)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "quantize: bad scale_format");
    const size_t n = (size_t)rows * K;
    HipBuf *X = B(x), *Q = B(q), *S = B(scales);
    if (!fits(X, n * dtype_bytes(d->x_dtype)) || !fits(Q, n * d->weight_bits / 8) ||
        !fits(S, (size_t)rows * (K / gs) * scale_bytes(d->scale_format)))
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "quantize: buffer too small");
    if (((uintptr_t)X->ptr | (uintptr_t)Q->ptr) & 15u)
        return fail(LUX_BACKEND_ERROR_NOT_SUPPORTED, "quantize: x and q must be 16-byte aligned");
    if (LuxBackendError e = begin_op(c, "quantize")) return e;
    if (n == 0) return LUX_BACKEND_OK;
    QuantArgs a{};
    a.x = X->ptr;
    a.q = Q->ptr;
    a.s = S->ptr;
    a.rows = rows;
    a.k = K;
    a.group_size = gs;
    a.bits = d->weight_bits;
    a.offset_binary = d->nibble_coding == LUX_HIP_NIBBLE_OFFSET_BINARY;
    a.scale_kind = static_cast<ScaleKind>(d->scale_format);
    a.x_kind = static_cast<XKind>(d->x_dtype);
    return end_op(c, launch_quantize(a, c->stream), "quantize");
}

// Dequantizers dequantize_nax_int4_sym / dequantize_nax_int8_group (symmetric branch),
// quantized_nax.wgsl:264-282,364-386: out = f32(q) * s, then rounded to x_dtype.
LUX_EXPORT LuxBackendError lux_hip_dequantize(LuxBackendContext* ctx, const LuxHipQuantizeDesc* d,
                                              LuxBackendBuffer* q, LuxBackendBuffer* scales,
                                              LuxBackendBuffer* out) {
    HipCtx* c = C(ctx);
    if (!c || !d || !q || !scales || !out) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "dequantize: NULL argument");
    if (d->struct_size < sizeof(LuxHipQuantizeDesc))
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "dequantize: struct_size %u too small", d->struct_size);
    const int rows = d->rows, K = d->k, gs = d->group_size;
    if (rows < 0 || K < 0) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "dequantize: negative size");
    if (d->weight_bits != 4 && d->weight_bits != 8)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "dequantize: weight_bits must be 4 or 8");
    if (gs < 8 || gs % 8 != 0 || K % gs != 0)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "dequantize: group_size %d must be a multiple of 8 dividing k", gs);
    if (d->nibble_coding != LUX_HIP_NIBBLE_OFFSET_BINARY && d->nibble_coding != LUX_HIP_NIBBLE_TWOS_COMPLEMENT)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "dequantize: bad nibble_coding");
    if (d->x_dtype != LUX_HIP_F32 && d->x_dtype != LUX_HIP_F16 && d->x_dtype != LUX_HIP_BF16)
        return fail(LUX_BACKEND_ERROR_NOT_SUPPORTED, "dequantize: output dtype must be F32, F16 or BF16");
    if (scale_bytes(d->scale_format) == 0)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "dequantize: bad scale_format");
    const size_t n = (size_t)rows * K;
    HipBuf *Q = B(q), *S = B(scales), *X = B(out);
    if (!fits(Q, n * d->weight_bits / 8) || !fits(X, n * dtype_bytes(d->x_dtype)) ||
        !fits(S, (size_t)rows * (K / gs) * scale_bytes(d->scale_format)))
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "dequantize: buffer too small");
    if (((uintptr_t)Q->ptr | (uintptr_t)X->ptr) & 15u)
        return fail(LUX_BACKEND_ERROR_NOT_SUPPORTED, "dequantize: q and out must be 16-byte aligned");
    if (LuxBackendError e = begin_op(c, "dequantize")) return e;
    if (n == 0) return LUX_BACKEND_OK;
    QuantArgs a{};
    a.q = Q->ptr;
    a.s = S->ptr;
    a.rows = rows;
    a.k = K;
    a.group_size = gs;
    a.bits = d->weight_bits;
    a.offset_binary = d->nibble_coding == LUX_HIP_NIBBLE_OFFSET_BINARY;
    a.scale_kind = static_cast<ScaleKind>(d->scale_format);
    a.x_kind = static_cast<XKind>(d->x_dtype);
    return end_op(c, launch_dequantize(a, X->ptr, c->stream), "dequantize");
}

// Nibble re-coding: offset-binary <-> two's complement (each nibble xor 8).
LUX_EXPORT LuxBackendError lux_hip_convert_nibbles(LuxBackendContext* ctx, LuxBackendBuffer* in,
                                                   LuxBackendBuffer* out, size_t words, int from_coding,
                                                   int to_coding) {
    HipCtx* c = C(ctx);
    HipBuf *I = B(in), *O = B(out);
    if (!c || !I || !O) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "convert_nibbles: NULL argument");
    auto ok = [](int v) { return v == LUX_HIP_NIBBLE_OFFSET_BINARY || v == LUX_HIP_NIBBLE_TWOS_COMPLEMENT; };
    if (!ok(from_coding) || !ok(to_coding))
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "convert_nibbles: bad coding");
    if (!fits(I, words * 4) || !fits(O, words * 4))
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "convert_nibbles: buffer too small");
    if (((uintptr_t)I->ptr | (uintptr_t)O->ptr) & 3u)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "convert_nibbles: buffers must be 4-byte aligned");
    if (LuxBackendError e = begin_op(c, "convert_nibbles")) return e;
    if (words == 0) return LUX_BACKEND_OK;
    const uint32_t mask = from_coding == to_coding ? 0u : 0x88888888u;
    return end_op(c, launch_xor_words(I->ptr, O->ptr, words, mask, c->stream), "convert_nibbles");
}

// Scale storage conversion between F16, F32 and the 16-byte GroupScale.
LUX_EXPORT LuxBackendError lux_hip_convert_scales(LuxBackendContext* ctx, LuxBackendBuffer* in, int in_format,
                                                  LuxBackendBuffer* out, int out_format, size_t count) {
    HipCtx* c = C(ctx);
    HipBuf *I = B(in), *O = B(out);
    if (!c || !I || !O) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "convert_scales: NULL argument");
    const size_t ib = scale_bytes(in_format), ob = scale_bytes(out_format);
    if (!ib || !ob) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "convert_scales: bad scale format");
    if (!fits(I, count * ib) || !fits(O, count * ob))
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "convert_scales: buffer too small");
    if (LuxBackendError e = begin_op(c, "convert_scales")) return e;
    if (count == 0) return LUX_BACKEND_OK;
    return end_op(c, launch_convert_scales(I->ptr, static_cast<ScaleKind>(in_format), O->ptr,
                                           static_cast<ScaleKind>(out_format), count, c->stream),
                  "convert_scales");
}

// rms_norm.wgsl:25-110 (RMSNormParams {batch_size, hidden_size, eps}; bindings input,
// output, gamma, rms_out).  The ABI-v3 slot op_rms_norm_f32 exists but its signature is
// not recoverable (the reference leaves it NULL, src/webgpu_plugin.cpp:4072), so the
// kernel is exposed here.
LUX_EXPORT LuxBackendError lux_hip_rms_norm(LuxBackendContext* ctx, const LuxHipRmsNormParams* p,
                                            LuxBackendBuffer* input, LuxBackendBuffer* gamma,
                                            LuxBackendBuffer* output, LuxBackendBuffer* rms_out) {
    HipCtx* c = C(ctx);
    HipBuf *X = B(input), *G = B(gamma), *Y = B(output), *R = B(rms_out);
    if (!c || !p || !X || !G || !Y) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "rms_norm: NULL argument");
    const size_t xb = dtype_bytes(p->x_dtype), yb = dtype_bytes(p->y_dtype);
    if (!xb || !yb || p->x_dtype == LUX_HIP_I32 || p->x_dtype == LUX_HIP_I8 || p->y_dtype == LUX_HIP_I32 ||
        p->y_dtype == LUX_HIP_I8)
        return fail(LUX_BACKEND_ERROR_NOT_SUPPORTED, "rms_norm: dtypes must be F32, F16 or BF16");
    if (p->hidden_size == 0 && p->batch_size != 0)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "rms_norm: hidden_size 0");
    if (p->batch_size > INT32_MAX || p->hidden_size > INT32_MAX)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "rms_norm: size too large");
    const size_t n = (size_t)p->batch_size * p->hidden_size;
    if (!fits(X, n * xb) || !fits(Y, n * yb) || !fits(G, (size_t)p->hidden_size * 4) ||
        (R && !fits(R, (size_t)p->batch_size * 4)))
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "rms_norm: buffer too small");
    if (LuxBackendError e = begin_op(c, "rms_norm")) return e;
    if (n == 0) return LUX_BACKEND_OK;
    return end_op(c, launch_rms_norm(X->ptr, static_cast<XKind>(p->x_dtype), static_cast<const float*>(G->ptr), Y->ptr,
                                     static_cast<YKind>(p->y_dtype), R ? static_cast<float*>(R->ptr) : nullptr,
                                     (int)p->batch_size, (int)p->hidden_size, p->eps, c->stream),
                  "rms_norm");
}

// rms_norm (rms_norm.wgsl:50-110) of X into desc->x_dtype, then the quantized matmul of
// lux_hip_qmatmul_ex on the normalised rows.  At m == 1 with int4 weights, fp16 scales and
// an fp16 activation type, the GEMV normalises the row in its own prologue: one launch and
// no intermediate row in memory.  Otherwise the two kernels run back to back with the
// normalised rows at the start of the context workspace.  Both routes give the bits of
// lux_hip_rms_norm followed by lux_hip_qmatmul_ex.
LUX_EXPORT LuxBackendError lux_hip_rms_norm_qmatmul(LuxBackendContext* ctx, const LuxHipRmsNormParams* p,
                                                    LuxBackendBuffer* gamma, const LuxHipQMatmulDesc* d,
                                                    LuxBackendBuffer* w, LuxBackendBuffer* w_scales,
                                                    LuxBackendBuffer* x, int epilogue, LuxBackendBuffer* bias,
                                                    LuxBackendBuffer* residual, LuxBackendBuffer* y) {
    HipCtx* c = C(ctx);
    HipBuf *X = B(x), *G = B(gamma), *W = B(w), *S = B(w_scales);
    if (!c || !p || !d || !X || !G || !W || !y)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "rms_norm_qmatmul: NULL argument");
    if (d->struct_size < sizeof(LuxHipQMatmulDesc))
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "rms_norm_qmatmul: struct_size %u too small", d->struct_size);
    auto fp = [](int t) { return t == LUX_HIP_F32 || t == LUX_HIP_F16 || t == LUX_HIP_BF16; };
    if (!fp(p->x_dtype) || !fp(d->x_dtype))
        return fail(LUX_BACKEND_ERROR_NOT_SUPPORTED,
                    "rms_norm_qmatmul: x and the normalised rows must be F32, F16 or BF16");
    if (p->y_dtype != d->x_dtype)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT,
                    "rms_norm_qmatmul: the norm's y_dtype must equal the matmul's x_dtype");
    if (d->m < 0 || d->k < 0 || (int64_t)p->batch_size != d->m || (int64_t)p->hidden_size != d->k)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT,
                    "rms_norm_qmatmul: batch_size and hidden_size must equal the matmul's m and k");
    if (d->k == 0 && d->m != 0) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "rms_norm_qmatmul: hidden_size 0");
    const size_t xb = dtype_bytes(p->x_dtype), n = (size_t)d->m * d->k;
    if (!fits(X, n * xb) || !fits(G, (size_t)d->k * 4))
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "rms_norm_qmatmul: x or gamma buffer too small");
    if (((uintptr_t)X->ptr & (xb - 1)) || ((uintptr_t)G->ptr & 3u))
        return fail(LUX_BACKEND_ERROR_NOT_SUPPORTED, "rms_norm_qmatmul: x or gamma not naturally aligned");
    const RnArgs rn{X->ptr, static_cast<const float*>(G->ptr), p->eps, p->x_dtype};

    QArgs probe{};
    probe.w = W->ptr;
    probe.s = S ? S->ptr : nullptr;
    probe.n_out = d->n_out;
    probe.k = d->k;
    probe.m = d->m;
    probe.group_size = d->group_size;
    probe.wbits = d->weight_bits;
    probe.scale_kind = static_cast<ScaleKind>(d->scale_format);
    probe.x_kind = static_cast<XKind>(d->x_dtype);
    probe.rn = rn;
    if (d->flags == 0 && S && d->n_out > 0 && d->x_dtype == LUX_HIP_F16 && d->scale_format == LUX_HIP_SCALE_F16 &&
        qgemv_i4_rn_supported(probe))
        return qmatmul_impl(ctx, d, w, w_scales, x, nullptr, epilogue, bias, residual, y, false, 0, &rn);

    if (LuxBackendError e = begin_op(c, "rms_norm_qmatmul")) return e;
    HipBuf xn;
    xn.size = (n * dtype_bytes(d->x_dtype) + 255) & ~(size_t)255;
    xn.owned = false;
    xn.device = c->device;
    if (n) {
        if (LuxBackendError e = get_workspace(c, xn.size, &xn.ptr, "rms_norm_qmatmul")) return e;
        if (hipError_t he = launch_rms_norm(X->ptr, static_cast<XKind>(p->x_dtype), rn.gamma, xn.ptr,
                                            static_cast<YKind>(d->x_dtype), nullptr, d->m, d->k, p->eps, c->stream);
            he != hipSuccess)
            return end_op(c, he, "rms_norm_qmatmul (rms_norm)");
    } else {
        xn.ptr = X->ptr;  // nothing to normalise; the matmul validates and returns
    }
    return qmatmul_impl(ctx, d, w, w_scales, reinterpret_cast<LuxBackendBuffer*>(&xn), nullptr, epilogue, bias,
                        residual, y, false, xn.size);
}

// quantize_int8_per_channel / dequantize_int8_per_channel (quantized.wgsl:264-297):
// QuantParams.size and .quant_type (:37-42), ChannelQuantParams.channel_stride (:44-49),
// channel_scales: PerChannelScale[ceil(size / channel_stride)] (:51-56).
static LuxBackendError int8_per_channel(LuxBackendContext* ctx, bool dequantize, LuxBackendBuffer* in,
                                        LuxBackendBuffer* channel_scales, LuxBackendBuffer* out, size_t size,
                                        uint32_t channel_stride, uint32_t quant_type) {
    const char* op = dequantize ? "dequantize_int8_per_channel" : "quantize_int8_per_channel";
    HipCtx* c = C(ctx);
    HipBuf *I = B(in), *S = B(channel_scales), *O = B(out);
    if (!c || !I || !S || !O) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "%s: NULL argument", op);
    if (channel_stride == 0) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "%s: channel_stride is 0", op);
    const size_t channels = size / channel_stride + (size % channel_stride != 0);
    if (!fits(I, size * 4) || !fits(O, size * 4) || !fits(S, channels * sizeof(ChannelScale)))
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "%s: buffer too small", op);
    if (((uintptr_t)I->ptr | (uintptr_t)O->ptr | (uintptr_t)S->ptr) & 3u)
        return fail(LUX_BACKEND_ERROR_NOT_SUPPORTED, "%s: buffers must be 4-byte aligned", op);
    if (LuxBackendError e = begin_op(c, op)) return e;
    if (size == 0) return LUX_BACKEND_OK;
    return end_op(c,
                  launch_int8_per_channel(dequantize, I->ptr, static_cast<const ChannelScale*>(S->ptr), O->ptr, size,
                                          channel_stride, quant_type != 0, c->stream),
                  op);
}

LUX_EXPORT LuxBackendError lux_hip_quantize_int8_per_channel(LuxBackendContext* ctx, LuxBackendBuffer* in,
                                                             LuxBackendBuffer* channel_scales,
                                                             LuxBackendBuffer* out, size_t size,
                                                             uint32_t channel_stride, uint32_t quant_type) {
    return int8_per_channel(ctx, false, in, channel_scales, out, size, channel_stride, quant_type);
}

LUX_EXPORT LuxBackendError lux_hip_dequantize_int8_per_channel(LuxBackendContext* ctx, LuxBackendBuffer* in,
                                                               LuxBackendBuffer* channel_scales,
                                                               LuxBackendBuffer* out, size_t size,
                                                               uint32_t channel_stride, uint32_t quant_type) {
    return int8_per_channel(ctx, true, in, channel_scales, out, size, channel_stride, quant_type);
}

// requantize_int32_to_int8 (quantized.wgsl:560-580): RequantParams {size, input_scale,
// output_scale, output_zero_point}; i32 in, i32 out clamped to [-128, 127].
LUX_EXPORT LuxBackendError lux_hip_requantize_i32(LuxBackendContext* ctx, LuxBackendBuffer* in,
                                                  LuxBackendBuffer* out, size_t size, float input_scale,
                                                  float output_scale, int32_t output_zero_point) {
    HipCtx* c = C(ctx);
    HipBuf *I = B(in), *O = B(out);
    if (!c || !I || !O) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "requantize: NULL argument");
    if (!fits(I, size * 4) || !fits(O, size * 4))
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "requantize: buffer too small");
    if (LuxBackendError e = begin_op(c, "requantize")) return e;
    if (size == 0) return LUX_BACKEND_OK;
    return end_op(c, launch_requantize(static_cast<const int32_t*>(I->ptr), static_cast<int32_t*>(O->ptr), size,
                                       input_scale, output_scale, output_zero_point, c->stream),
                  "requantize");
}

// ---------------------------------------------------------------- host packers
// CPU-side producers of the hot path's inputs, for a loader that prepares weights on the
// host before upload (no device, no context).  Bit-identical to the device codecs
// (lux_hip_convert_nibbles, lux_hip_convert_scales).
namespace {

// binary32 -> binary16, round to nearest even (subnormals kept, overflow to inf, NaN
// stays NaN with its top payload bits), the rounding the device's conversion uses.
uint16_t host_f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);  // >= 65520 rounds to inf
    const uint32_t eb = ax >> 23;
    if (eb >= 113) {  // normal binary16: exponent eb - 127 + 15 >= 1
        uint32_t h = ((eb - 112) << 10) | ((ax & 0x7FFFFFu) >> 13);
        const uint32_t rem = ax & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;  // a carry moves up the exponent
        return (uint16_t)(sign | h);
    }
    if (eb < 102) return (uint16_t)sign;  // below 2^-25 (and 2^-25 itself ties to 0)
    const uint32_t m = (ax & 0x7FFFFFu) | 0x800000u, r = 126 - eb;  // value = m * 2^-(24 + r)
    uint32_t h = m >> r;
    const uint32_t rem = m & ((1u << r) - 1u), half = 1u << (r - 1);
    if (rem > half || (rem == half && (h & 1u))) ++h;  // may reach 0x400, the least normal
    return (uint16_t)(sign | h);
}

float host_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t x;
    if (e == 0x1F) x = sign | 0x7F800000u | (m << 13);
    else if (e) x = sign | ((e + 112) << 23) | (m << 13);
    else if (!m) x = sign;
    else {  // subnormal: m * 2^-24, exact in binary32
        const float v = std::ldexp((float)m, -24);
        std::memcpy(&x, &v, 4);
        x |= sign;
    }
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}

bool valid_coding(int c) { return c == LUX_HIP_NIBBLE_OFFSET_BINARY || c == LUX_HIP_NIBBLE_TWOS_COMPLEMENT; }

}  // namespace

LUX_EXPORT LuxBackendError lux_hip_pack_int4_host(const int8_t* q, size_t n, int coding, uint32_t* words) {
    if (n % 8 != 0) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "pack_int4_host: n = %zu is not a multiple of 8", n);
    if (!valid_coding(coding)) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "pack_int4_host: bad coding %d", coding);
    if (n && (!q || !words)) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "pack_int4_host: NULL argument");
    const uint32_t ob = coding == LUX_HIP_NIBBLE_OFFSET_BINARY ? 8u : 0u;
    for (size_t w = 0; w < n / 8; ++w) {
        uint32_t word = 0;
        for (int i = 0; i < 8; ++i) {
            const int v = q[8 * w + i];
            if (v < -8 || v > 7)
                return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "pack_int4_host: value %d at %zu outside [-8, 7]", v,
                            8 * w + i);
            word |= (((uint32_t)v & 0xFu) ^ ob) << (4 * i);  // element i in bits 4i .. 4i+3
        }
        words[w] = word;
    }
    return LUX_BACKEND_OK;
}

LUX_EXPORT LuxBackendError lux_hip_unpack_int4_host(const uint32_t* words, size_t n, int coding, int8_t* q) {
    if (n % 8 != 0) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "unpack_int4_host: n = %zu is not a multiple of 8", n);
    if (!valid_coding(coding)) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "unpack_int4_host: bad coding %d", coding);
    if (n && (!q || !words)) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "unpack_int4_host: NULL argument");
    const uint32_t ob = coding == LUX_HIP_NIBBLE_OFFSET_BINARY ? 8u : 0u;
    for (size_t w = 0; w < n / 8; ++w)
        for (int i = 0; i < 8; ++i) {
            const uint32_t t = ((words[w] >> (4 * i)) & 0xFu) ^ ob;  // two's complement nibble
            q[8 * w + i] = (int8_t)((int)t - (t >= 8 ? 16 : 0));
        }
    return LUX_BACKEND_OK;
}

LUX_EXPORT LuxBackendError lux_hip_convert_scales_host(const void* in, int in_format, void* out, int out_format,
                                                       size_t count) {
    if (scale_bytes(in_format) == 0 || scale_bytes(out_format) == 0)
        return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "convert_scales_host: bad format");
    if (count && (!in || !out)) return fail(LUX_BACKEND_ERROR_INVALID_ARGUMENT, "convert_scales_host: NULL argument");
    for (size_t i = 0; i < count; ++i) {
        float sc;
        GroupScale g{};
        if (in_format == LUX_HIP_SCALE_F16) sc = host_f16_to_f32(static_cast<const uint16_t*>(in)[i]);
        else if (in_format == LUX_HIP_SCALE_F32) sc = static_cast<const float*>(in)[i];
        else {
            std::memcpy(&g, static_cast<const uint8_t*>(in) + 16 * i, 16);
            sc = g.scale;
        }
        if (out_format == LUX_HIP_SCALE_F16) static_cast<uint16_t*>(out)[i] = host_f32_to_f16(sc);
        else if (out_format == LUX_HIP_SCALE_F32) static_cast<float*>(out)[i] = sc;
        else {
            const GroupScale o = in_format == LUX_HIP_SCALE_GROUPSCALE ? g : GroupScale{sc, 0, 0.0f, 0.0f};
            std::memcpy(static_cast<uint8_t*>(out) + 16 * i, &o, 16);
        }
    }
    return LUX_BACKEND_OK;
}
