/*
 * rsinfer native plugin ABI, version 1 — the contract this plugin exports.
 *
 * The engine's loader (src/backend/mod.rs:137-234 in the reference) dlopens a
 * shared library, resolves the nine symbols below, requires
 * safetyraise_kernel_abi_version() == 1, creates one context, reads the
 * capabilities (struct_size >= 40) and requires a non-empty name.  The types,
 * enum values and symbol signatures below therefore have to be identical to
 * the reference declaration (native/include/safetyraise_kernel.h:26-127);
 * the wording of this file is this project's own.
 *
 * Conventions the plugin honours (reference header :7-11, :94-114):
 *  - fixed-width integers, plain C pointers and explicit lengths only;
 *  - inputs are copied (or uploaded) before a call returns, no pointer is kept;
 *  - calls on one context are serial; the caller holds a lock around them;
 *  - results are complete when a call returns (synchronous contract);
 *  - a non-zero status comes with text available from last_error(context).
 */
#ifndef SAFETYRAISE_KERNEL_H
#define SAFETYRAISE_KERNEL_H

#include <stdint.h>

#define SAFETYRAISE_KERNEL_EXPORT __attribute__((visibility("default")))

#ifdef __cplusplus
extern "C" {
#endif

#define SAFETYRAISE_KERNEL_ABI_VERSION UINT32_C(1)

typedef struct safetyraise_kernel_context safetyraise_kernel_context;
typedef struct safetyraise_kernel_weight safetyraise_kernel_weight;

/* Status codes (reference :32-41).  Zero is success. */
typedef enum safetyraise_kernel_status {
    SAFETYRAISE_KERNEL_STATUS_OK = 0,
    SAFETYRAISE_KERNEL_STATUS_INVALID_ARGUMENT = 1,
    SAFETYRAISE_KERNEL_STATUS_UNSUPPORTED_DTYPE = 2,
    SAFETYRAISE_KERNEL_STATUS_DIMENSION_OVERFLOW = 3,
    SAFETYRAISE_KERNEL_STATUS_OUT_OF_MEMORY = 4,
    SAFETYRAISE_KERNEL_STATUS_DEVICE_ERROR = 5,
    SAFETYRAISE_KERNEL_STATUS_INTERNAL_ERROR = 6,
    SAFETYRAISE_KERNEL_STATUS_ABI_MISMATCH = 7
} safetyraise_kernel_status;

/* Weight dtypes (reference :44-52).  Bit n of dtype_mask means dtype n. */
typedef enum safetyraise_kernel_dtype {
    SAFETYRAISE_KERNEL_DTYPE_F32 = 1,
    SAFETYRAISE_KERNEL_DTYPE_F16 = 2,
    SAFETYRAISE_KERNEL_DTYPE_BF16 = 3,
    SAFETYRAISE_KERNEL_DTYPE_Q4_0 = 4,
    SAFETYRAISE_KERNEL_DTYPE_Q8_0 = 5,
    SAFETYRAISE_KERNEL_DTYPE_Q4K = 6,
    SAFETYRAISE_KERNEL_DTYPE_Q6K = 7
} safetyraise_kernel_dtype;

/* Device kinds (reference :54-58).  The loader maps any unknown value to
 * Other (src/backend/mod.rs:80-86); an AMD GPU plugin reports OTHER. */
typedef enum safetyraise_kernel_device_kind {
    SAFETYRAISE_KERNEL_DEVICE_HOST = 1,
    SAFETYRAISE_KERNEL_DEVICE_CUDA = 2,
    SAFETYRAISE_KERNEL_DEVICE_OTHER = 3
} safetyraise_kernel_device_kind;

/* create_context input (reference :61-65); 16 bytes. */
typedef struct safetyraise_kernel_context_options {
    uint32_t abi_version;
    uint32_t struct_size;
    uint64_t flags;
} safetyraise_kernel_context_options;

/* get_capabilities output (reference :68-76); 40 bytes.  max_rows and
 * max_cols of zero mean "no limit"; flags are plugin-defined. */
typedef struct safetyraise_kernel_capabilities {
    uint32_t abi_version;
    uint32_t struct_size;
    uint64_t dtype_mask;
    uint32_t device_kind;
    uint32_t flags;
    uint64_t max_rows;
    uint64_t max_cols;
} safetyraise_kernel_capabilities;

/* reference :78 */
SAFETYRAISE_KERNEL_EXPORT uint32_t safetyraise_kernel_abi_version(void);

/* reference :80 — must be non-NULL and non-empty (src/backend/mod.rs:198-211). */
SAFETYRAISE_KERNEL_EXPORT const char *safetyraise_kernel_name(void);

/* reference :82-84 — rejects abi_version != 1 or struct_size < 16. */
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_create_context(
    const safetyraise_kernel_context_options *options,
    safetyraise_kernel_context **out_context);

/* reference :86-88 — synchronises the device and frees the context's
 * resources; called before the library is unloaded. */
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_destroy_context(
    safetyraise_kernel_context *context);

/* reference :90-92 — the caller pre-fills struct_size. */
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_get_capabilities(
    safetyraise_kernel_context *context,
    safetyraise_kernel_capabilities *out_capabilities);

/* reference :98-105 — data is a contiguous weight[rows][cols]. */
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_create_weight(
    safetyraise_kernel_context *context,
    const uint8_t *data,
    uint64_t byte_len,
    uint64_t rows,
    uint64_t cols,
    uint32_t dtype,
    safetyraise_kernel_weight **out_weight);

/* reference :107-109 */
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_destroy_weight(
    safetyraise_kernel_context *context,
    safetyraise_kernel_weight *weight);

/* reference :115-123 — host f32 matrices in and out, synchronous. */
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_linear(
    safetyraise_kernel_context *context,
    safetyraise_kernel_weight *weight,
    const float *input,
    uint64_t input_rows,
    uint64_t input_cols,
    float *output,
    uint64_t output_rows,
    uint64_t output_cols);

/* reference :126-127 — NUL-terminated UTF-8 owned by the context. */
SAFETYRAISE_KERNEL_EXPORT const char *safetyraise_kernel_last_error(
    safetyraise_kernel_context *context);

#ifdef __cplusplus
}
#endif

#endif /* SAFETYRAISE_KERNEL_H */
