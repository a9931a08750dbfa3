/*
 * lux/gpu/backend_plugin.h -- Lux GPU backend plugin ABI (v3), as implemented by
 * libluxgpu_backend_hip.so.
 *
 * INFERRED HEADER.  The canonical header lives in the luxcpp/gpu repository, which
 * is not available here.  Everything below is reconstructed from the way the
 * WebGPU plugin uses it:
 *   - the vtable slot order follows the C++ designated initializers of
 *     `webgpu_vtbl` (reference src/webgpu_plugin.cpp:4022-4123).  Designated
 *     initializers must follow declaration order, so this order is a lower bound:
 *     the real header could interleave fields that the WebGPU plugin never names;
 *   - the descriptor fields follow webgpu_backend_init_impl
 *     (src/webgpu_plugin.cpp:4129-4152);
 *   - the device-info fields follow webgpu_get_device_info (:1369-1389);
 *   - the capability bits follow docs/architecture.md:112-123;
 *   - the error names follow every `return LUX_BACKEND_*` in the plugin.  Their
 *     numeric values are not recoverable from the reference.  OK, INVALID_ARGUMENT
 *     and OUT_OF_MEMORY take the values of the same-named codes of the public
 *     LuxError enum (0, 1, 2; docs/api.md:662-670).  NOT_SUPPORTED (3), DEVICE_LOST
 *     (4) and INTERNAL (5) are numbered here; they do NOT follow LuxError, whose
 *     NOT_SUPPORTED is 6 and whose 3-5 are BACKEND_NOT_AVAILABLE, DEVICE_NOT_FOUND
 *     and KERNEL_FAILED.  A core built against the canonical header maps by name.
 * A loader guards against a layout mismatch through `vtbl_size`
 * (src/webgpu_plugin.cpp:4133).
 *
 * Slots outside the quantized-matmul path (NTT, FHE, hashes, curves, MSM, KZG,
 * signatures) keep their position but are typed as an opaque function pointer:
 * the HIP plugin leaves all of them NULL, which tells the core to fall back to
 * its CPU implementation (src/webgpu_plugin.cpp:3596-3602).
 */
#ifndef LUX_GPU_BACKEND_PLUGIN_H
#define LUX_GPU_BACKEND_PLUGIN_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LUX_GPU_BACKEND_ABI_VERSION 3u

typedef struct LuxBackendContext LuxBackendContext; /* opaque, owned by the plugin */
typedef struct LuxBackendBuffer LuxBackendBuffer;   /* opaque, owned by the plugin */

typedef enum LuxBackendError {
    LUX_BACKEND_OK = 0,
    LUX_BACKEND_ERROR_INVALID_ARGUMENT = 1, /* NULL or inconsistent arguments   */
    LUX_BACKEND_ERROR_OUT_OF_MEMORY = 2,    /* device allocation failed        */
    LUX_BACKEND_ERROR_NOT_SUPPORTED = 3,    /* core falls back to CPU           */
    LUX_BACKEND_ERROR_DEVICE_LOST = 4,      /* wait deadline expired            */
    LUX_BACKEND_ERROR_INTERNAL = 5          /* launch or runtime failure        */
} LuxBackendError;

/* Capability bits (docs/architecture.md:112-123). */
#define LUX_CAP_TENSOR_OPS (1u << 0)
#define LUX_CAP_MATMUL (1u << 1)
#define LUX_CAP_NTT (1u << 2)
#define LUX_CAP_MSM (1u << 3)
#define LUX_CAP_CUSTOM_KERNELS (1u << 4)
#define LUX_CAP_UNIFIED_MEMORY (1u << 5)
#define LUX_CAP_FHE (1u << 6)
#define LUX_CAP_TFHE (1u << 7)
#define LUX_CAP_BLS12_381 (1u << 12)
#define LUX_CAP_BN254 (1u << 13)
#define LUX_CAP_KZG (1u << 14)
#define LUX_CAP_POSEIDON2 (1u << 15)

/* Fields written by webgpu_get_device_info (src/webgpu_plugin.cpp:1375-1382). */
typedef struct LuxBackendDeviceInfo {
    const char* name;
    const char* vendor;
    uint64_t memory_total;
    uint64_t memory_available;
    int compute_units;
    int max_workgroup_size;
    bool is_discrete;
    bool is_unified_memory;
} LuxBackendDeviceInfo;

/* Position holder for a slot this plugin never fills. */
typedef void (*lux_gpu_backend_unused_slot)(void);

typedef LuxBackendError (*lux_backend_binary_f32_fn)(LuxBackendContext*, LuxBackendBuffer* a,
                                                     LuxBackendBuffer* b, LuxBackendBuffer* out,
                                                     size_t n);

typedef struct lux_gpu_backend_vtbl {
    /* Lifecycle (src/webgpu_plugin.cpp:4024-4025) */
    LuxBackendContext* (*create_context)(int device_index);
    void (*destroy_context)(LuxBackendContext* ctx);

    /* Device info & sync (:4028-4030) */
    LuxBackendError (*get_device_count)(int* count);
    LuxBackendError (*get_device_info)(LuxBackendContext* ctx, LuxBackendDeviceInfo* info);
    LuxBackendError (*sync)(LuxBackendContext* ctx);

    /* Buffer management (:4033-4038) */
    LuxBackendBuffer* (*buffer_alloc)(LuxBackendContext* ctx, size_t bytes);
    LuxBackendBuffer* (*buffer_alloc_with_data)(LuxBackendContext* ctx, const void* data,
                                                size_t bytes);
    void (*buffer_free)(LuxBackendContext* ctx, LuxBackendBuffer* buf);
    LuxBackendError (*buffer_copy_to_host)(LuxBackendContext* ctx, LuxBackendBuffer* buf,
                                           void* dst, size_t bytes);
    LuxBackendError (*buffer_copy_from_host)(LuxBackendContext* ctx, LuxBackendBuffer* buf,
                                             const void* src, size_t bytes);
    void* (*buffer_get_host_ptr)(LuxBackendContext* ctx, LuxBackendBuffer* buf);

    /* Tensor (:4041-4044) */
    lux_backend_binary_f32_fn op_add_f32;
    lux_backend_binary_f32_fn op_sub_f32;
    lux_backend_binary_f32_fn op_mul_f32;
    lux_backend_binary_f32_fn op_div_f32;

    /* C[M x N] = A[M x K] . B[K x N], fp32, row-major (signature :1721) */
    LuxBackendError (*op_matmul_f32)(LuxBackendContext* ctx, LuxBackendBuffer* a,
                                     LuxBackendBuffer* b, LuxBackendBuffer* out, int M, int K,
                                     int N);
    LuxBackendError (*op_transpose_f32)(LuxBackendContext* ctx, LuxBackendBuffer* in,
                                        LuxBackendBuffer* out, int rows, int cols);

    /* Reductions, softmax, unary, copy, norms (:4049-4072) */
    lux_gpu_backend_unused_slot op_reduce_sum_f32;
    lux_gpu_backend_unused_slot op_reduce_max_f32;
    lux_gpu_backend_unused_slot op_reduce_min_f32;
    lux_gpu_backend_unused_slot op_reduce_mean_f32;
    lux_gpu_backend_unused_slot op_reduce_sum_axis_f32;
    lux_gpu_backend_unused_slot op_reduce_max_axis_f32;
    lux_gpu_backend_unused_slot op_softmax_f32;
    lux_gpu_backend_unused_slot op_log_softmax_f32;
    lux_gpu_backend_unused_slot op_exp_f32;
    lux_gpu_backend_unused_slot op_log_f32;
    lux_gpu_backend_unused_slot op_sqrt_f32;
    lux_gpu_backend_unused_slot op_neg_f32;
    lux_gpu_backend_unused_slot op_abs_f32;
    lux_gpu_backend_unused_slot op_tanh_f32;
    lux_gpu_backend_unused_slot op_sigmoid_f32;
    lux_gpu_backend_unused_slot op_relu_f32;
    lux_gpu_backend_unused_slot op_gelu_f32;
    lux_gpu_backend_unused_slot op_copy_f32;
    lux_gpu_backend_unused_slot op_layer_norm_f32;
    lux_gpu_backend_unused_slot op_rms_norm_f32;

    /* NTT, FHE (:4074-4082) */
    lux_gpu_backend_unused_slot op_ntt_forward;
    lux_gpu_backend_unused_slot op_ntt_inverse;
    lux_gpu_backend_unused_slot op_poly_mul;
    lux_gpu_backend_unused_slot op_tfhe_bootstrap;
    lux_gpu_backend_unused_slot op_tfhe_keyswitch;
    lux_gpu_backend_unused_slot op_blind_rotate;

    /* Hashes, curves, MSM, KZG (:4084-4104) */
    lux_gpu_backend_unused_slot op_poseidon2_hash;
    lux_gpu_backend_unused_slot op_blake3_hash;
    lux_gpu_backend_unused_slot op_keccak256_hash;
    lux_gpu_backend_unused_slot op_bls12_381_add;
    lux_gpu_backend_unused_slot op_bls12_381_mul;
    lux_gpu_backend_unused_slot op_bls12_381_pairing;
    lux_gpu_backend_unused_slot op_bn254_add;
    lux_gpu_backend_unused_slot op_bn254_mul;
    lux_gpu_backend_unused_slot op_msm;
    lux_gpu_backend_unused_slot op_kzg_commit;
    lux_gpu_backend_unused_slot op_kzg_open;
    lux_gpu_backend_unused_slot op_kzg_verify;

    /* ecrecover, post-quantum, threshold, Schnorr (:4106-4122) */
    lux_gpu_backend_unused_slot op_ecrecover_batch;
    lux_gpu_backend_unused_slot op_mldsa_verify_batch;
    lux_gpu_backend_unused_slot op_mlkem_decapsulate_batch;
    lux_gpu_backend_unused_slot op_slhdsa_verify_batch;
    lux_gpu_backend_unused_slot op_ringtail_partial_sign_batch;
    lux_gpu_backend_unused_slot op_ringtail_combine_batch;
    lux_gpu_backend_unused_slot op_frost_partial_verify_batch;
    lux_gpu_backend_unused_slot op_cggmp21_partial_sign_batch;
    lux_gpu_backend_unused_slot op_ed25519_verify_batch;
    lux_gpu_backend_unused_slot op_sr25519_verify_batch;
} lux_gpu_backend_vtbl;

/* Filled by lux_gpu_backend_init (src/webgpu_plugin.cpp:4129-4148). */
typedef struct lux_gpu_backend_desc {
    uint32_t abi_version;
    uint32_t vtbl_size;
    const char* backend_name;
    const char* backend_version;
    uint32_t capabilities;
    const lux_gpu_backend_vtbl* vtbl;
} lux_gpu_backend_desc;

typedef bool (*lux_gpu_backend_init_fn)(lux_gpu_backend_desc* out);

/* The one symbol the core resolves with dlsym (docs/architecture.md:91,102;
 * generated by LUX_GPU_DECLARE_BACKEND at src/webgpu_plugin.cpp:4154). */
bool lux_gpu_backend_init(lux_gpu_backend_desc* out);

#ifdef __cplusplus
}
#endif

#endif /* LUX_GPU_BACKEND_PLUGIN_H */
