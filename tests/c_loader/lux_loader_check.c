/*
 * A compiled C caller of libluxgpu_backend_hip.so, written the way luxcpp/gpu's loader
 * binds a backend plugin (reference docs/architecture.md:89-107: dlopen the plugin,
 * dlsym "lux_gpu_backend_init", check abi_version and vtbl_size, keep the vtable) and
 * binds the quantized lux_hip_* extensions with dlsym into a LuxHipQuantApi table.
 * It includes only the lux/gpu headers and builds with `gcc -std=c11`; nothing here knows
 * about HIP or PyTorch.
 *
 * Usage: lux_loader_check <plugin.so> <dir>
 * Reads from <dir> (little-endian raw arrays written by tests/test_gpu_c_loader.py):
 *   gemv_A.f32 [GM x GK], gemv_x.f32 [GK]           op_matmul_f32(M = GM, K = GK, N = 1)
 *   gemm_A.f32 [MM x MK], gemm_B.f32 [MK x MN]      op_matmul_f32(M = MM, K = MK, N = MN)
 *   q_W.u32 [QN x QK/8], q_S.f16 [QN x QK/32], q_x.f16 [QK]
 *                                                   lux_hip_qmatmul int4 g32 GEMV
 * Writes gemv_y.f32, gemm_C.f32 and q_y.f16 to <dir>.  Prints one "ok ..." line per
 * check and exits 0 when every call and check passed.
 */
#define _POSIX_C_SOURCE 200809L
#include <dlfcn.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "lux/gpu/backend_plugin.h"
#include "lux/gpu/hip_quant.h"

enum { GM = 1000, GK = 4096, MM = 70, MK = 300, MN = 130, QN = 4096, QK = 4096 };

typedef struct LuxHipQuantApi {
    uint32_t (*api_version)(void);
    LuxBackendError (*qmatmul)(LuxBackendContext*, const LuxHipQMatmulDesc*, LuxBackendBuffer* w,
                               LuxBackendBuffer* w_scales, LuxBackendBuffer* x, LuxBackendBuffer* x_scales,
                               LuxBackendBuffer* y);
    const char* (*last_error)(void);
} LuxHipQuantApi;

static int failures = 0;

#define CHECK(cond, ...)                   \
    do {                                   \
        if (cond) {                        \
            printf("ok   ");               \
        } else {                           \
            printf("FAIL ");               \
            ++failures;                    \
        }                                  \
        printf(__VA_ARGS__);               \
        printf("\n");                      \
    } while (0)

static void* read_file(const char* dir, const char* name, size_t bytes) {
    char path[4096];
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE* f = fopen(path, "rb");
    if (!f) return NULL;
    void* p = malloc(bytes);
    size_t got = p ? fread(p, 1, bytes, f) : 0;
    fclose(f);
    if (got != bytes) {
        free(p);
        return NULL;
    }
    return p;
}

static int write_file(const char* dir, const char* name, const void* data, size_t bytes) {
    char path[4096];
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE* f = fopen(path, "wb");
    if (!f) return 0;
    size_t put = fwrite(data, 1, bytes, f);
    fclose(f);
    return put == bytes;
}

/* dlsym returns an object pointer; POSIX guarantees it converts to a function pointer. */
#define BIND(handle, name, dst) memcpy(&(dst), &(void*){dlsym((handle), (name))}, sizeof(dst))

int main(int argc, char** argv) {
    if (argc != 3) {
        fprintf(stderr, "usage: %s <plugin.so> <dir>\n", argv[0]);
        return 2;
    }
    const char* dir = argv[2];
    void* h = dlopen(argv[1], RTLD_NOW | RTLD_LOCAL);
    CHECK(h != NULL, "dlopen %s", argv[1]);
    if (!h) {
        fprintf(stderr, "%s\n", dlerror());
        return 1;
    }

    /* The core's half of the contract: one symbol, descriptor checks, then the vtable. */
    lux_gpu_backend_init_fn init = NULL;
    BIND(h, "lux_gpu_backend_init", init);
    CHECK(init != NULL, "dlsym lux_gpu_backend_init");
    if (!init) return 1;
    lux_gpu_backend_desc desc;
    memset(&desc, 0, sizeof desc);
    const int inited = init(&desc);
    CHECK(inited, "lux_gpu_backend_init returned true");
    CHECK(desc.abi_version == LUX_GPU_BACKEND_ABI_VERSION, "abi_version %u", desc.abi_version);
    CHECK(desc.vtbl_size == sizeof(lux_gpu_backend_vtbl), "vtbl_size %u == sizeof(lux_gpu_backend_vtbl) %zu",
          desc.vtbl_size, sizeof(lux_gpu_backend_vtbl));
    CHECK(desc.backend_name && strcmp(desc.backend_name, "hip") == 0, "backend_name \"%s\"",
          desc.backend_name ? desc.backend_name : "(null)");
    CHECK((desc.capabilities & (LUX_CAP_TENSOR_OPS | LUX_CAP_MATMUL)) == (LUX_CAP_TENSOR_OPS | LUX_CAP_MATMUL),
          "capabilities 0x%x", desc.capabilities);
    const lux_gpu_backend_vtbl* vt = desc.vtbl;
    if (!inited || !vt || desc.vtbl_size != sizeof(lux_gpu_backend_vtbl)) return 1;
    CHECK(vt->op_matmul_f32 && vt->create_context && vt->buffer_alloc && vt->buffer_copy_to_host,
          "matmul, lifecycle and buffer slots filled");
    CHECK(vt->op_ntt_forward == NULL && vt->op_softmax_f32 == NULL, "slots off the path are NULL (CPU fallback)");

    /* Optional quantized extensions, bound as a loader would (LuxHipQuantApi). */
    LuxHipQuantApi api;
    memset(&api, 0, sizeof api);
    BIND(h, "lux_hip_quant_api_version", api.api_version);
    BIND(h, "lux_hip_qmatmul", api.qmatmul);
    BIND(h, "lux_hip_last_error", api.last_error);
    CHECK(api.api_version && api.qmatmul && api.last_error, "dlsym lux_hip_* extensions");
    if (!api.api_version || !api.qmatmul || !api.last_error) return 1;
    CHECK(api.api_version() == LUX_HIP_QUANT_API_VERSION, "lux_hip_quant_api_version %u", api.api_version());

    int ndev = 0;
    CHECK(vt->get_device_count(&ndev) == LUX_BACKEND_OK && ndev > 0, "get_device_count %d", ndev);
    LuxBackendContext* ctx = vt->create_context(0);
    CHECK(ctx != NULL, "create_context(0)");
    if (!ctx) return 1;
    LuxBackendDeviceInfo info;
    memset(&info, 0, sizeof info);
    CHECK(vt->get_device_info(ctx, &info) == LUX_BACKEND_OK && info.compute_units > 0, "device %s, %d CUs",
          info.name ? info.name : "?", info.compute_units);

    /* lux_tensor_matmul -> op_matmul_f32: a GEMV (N = 1) and a general GEMM. */
    float* gA = read_file(dir, "gemv_A.f32", (size_t)GM * GK * 4);
    float* gx = read_file(dir, "gemv_x.f32", (size_t)GK * 4);
    float* mA = read_file(dir, "gemm_A.f32", (size_t)MM * MK * 4);
    float* mB = read_file(dir, "gemm_B.f32", (size_t)MK * MN * 4);
    uint32_t* qW = read_file(dir, "q_W.u32", (size_t)QN * QK / 2);
    uint16_t* qS = read_file(dir, "q_S.f16", (size_t)QN * (QK / 32) * 2);
    uint16_t* qx = read_file(dir, "q_x.f16", (size_t)QK * 2);
    CHECK(gA && gx && mA && mB && qW && qS && qx, "inputs read from %s", dir);
    if (!(gA && gx && mA && mB && qW && qS && qx)) return 1;

    LuxBackendBuffer* bA = vt->buffer_alloc_with_data(ctx, gA, (size_t)GM * GK * 4);
    LuxBackendBuffer* bx = vt->buffer_alloc_with_data(ctx, gx, (size_t)GK * 4);
    LuxBackendBuffer* by = vt->buffer_alloc(ctx, (size_t)GM * 4);
    LuxBackendError e = vt->op_matmul_f32(ctx, bA, bx, by, GM, GK, 1);
    CHECK(e == LUX_BACKEND_OK, "op_matmul_f32 GEMV %dx%d: %d %s", GM, GK, (int)e, e ? api.last_error() : "");
    float* y = malloc((size_t)GM * 4);
    CHECK(vt->buffer_copy_to_host(ctx, by, y, (size_t)GM * 4) == LUX_BACKEND_OK, "copy GEMV result to host");
    CHECK(write_file(dir, "gemv_y.f32", y, (size_t)GM * 4), "write gemv_y.f32");

    LuxBackendBuffer* bmA = vt->buffer_alloc_with_data(ctx, mA, (size_t)MM * MK * 4);
    LuxBackendBuffer* bmB = vt->buffer_alloc_with_data(ctx, mB, (size_t)MK * MN * 4);
    LuxBackendBuffer* bmC = vt->buffer_alloc(ctx, (size_t)MM * MN * 4);
    e = vt->op_matmul_f32(ctx, bmA, bmB, bmC, MM, MK, MN);
    CHECK(e == LUX_BACKEND_OK, "op_matmul_f32 GEMM %dx%dx%d: %d", MM, MK, MN, (int)e);
    float* C = malloc((size_t)MM * MN * 4);
    CHECK(vt->buffer_copy_to_host(ctx, bmC, C, (size_t)MM * MN * 4) == LUX_BACKEND_OK, "copy GEMM result");
    CHECK(write_file(dir, "gemm_C.f32", C, (size_t)MM * MN * 4), "write gemm_C.f32");

    /* Error paths the core relies on. */
    CHECK(vt->op_matmul_f32(ctx, NULL, bmB, bmC, MM, MK, MN) == LUX_BACKEND_ERROR_INVALID_ARGUMENT,
          "NULL buffer -> INVALID_ARGUMENT");
    CHECK(vt->op_matmul_f32(ctx, bmA, bmB, bmC, MM + 1, MK, MN) == LUX_BACKEND_ERROR_INVALID_ARGUMENT,
          "buffer smaller than M*K -> INVALID_ARGUMENT");

    /* Config-2-shaped int4 GEMV through the extension (weights QN x QK, g32, fp16). */
    LuxBackendBuffer* bW = vt->buffer_alloc_with_data(ctx, qW, (size_t)QN * QK / 2);
    LuxBackendBuffer* bS = vt->buffer_alloc_with_data(ctx, qS, (size_t)QN * (QK / 32) * 2);
    LuxBackendBuffer* bqx = vt->buffer_alloc_with_data(ctx, qx, (size_t)QK * 2);
    LuxBackendBuffer* bqy = vt->buffer_alloc(ctx, (size_t)QN * 2);
    LuxHipQMatmulDesc d;
    memset(&d, 0, sizeof d);
    d.struct_size = sizeof d;
    d.n_out = QN;
    d.k = QK;
    d.m = 1;
    d.weight_bits = 4;
    d.group_size = 32;
    d.nibble_coding = LUX_HIP_NIBBLE_OFFSET_BINARY;
    d.scale_format = LUX_HIP_SCALE_F16;
    d.x_dtype = LUX_HIP_F16;
    d.y_dtype = LUX_HIP_F16;
    e = api.qmatmul(ctx, &d, bW, bS, bqx, NULL, bqy);
    CHECK(e == LUX_BACKEND_OK, "lux_hip_qmatmul int4 g32 GEMV %dx%d: %d %s", QN, QK, (int)e, e ? api.last_error() : "");
    uint16_t* qy = malloc((size_t)QN * 2);
    CHECK(vt->buffer_copy_to_host(ctx, bqy, qy, (size_t)QN * 2) == LUX_BACKEND_OK, "copy qmatmul result");
    CHECK(write_file(dir, "q_y.f16", qy, (size_t)QN * 2), "write q_y.f16");
    d.k = 100; /* not a multiple of 32: no kernel, the core must fall back */
    CHECK(api.qmatmul(ctx, &d, bW, bS, bqx, NULL, bqy) == LUX_BACKEND_ERROR_NOT_SUPPORTED,
          "k %% 32 != 0 -> NOT_SUPPORTED");

    LuxBackendBuffer* bufs[] = {bA, bx, by, bmA, bmB, bmC, bW, bS, bqx, bqy};
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; ++i) vt->buffer_free(ctx, bufs[i]);
    vt->destroy_context(ctx);
    free(gA), free(gx), free(mA), free(mB), free(qW), free(qS), free(qx), free(y), free(C), free(qy);
    printf("%s: %d failed checks\n", failures ? "FAILED" : "PASSED", failures);
    return failures ? 1 : 0;
}
