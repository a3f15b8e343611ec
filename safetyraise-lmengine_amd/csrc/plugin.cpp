// Context lifetime, the nine ABI v1 symbols and the shared host helpers.
//
// ABI v1 is declared in include/safetyraise_kernel.h.  This plugin reports
// dtype_mask = 0, so the engine's loader never routes a projection here
// (src/backend/mod.rs:259-264 falls back to its CPU matmul); linear and
// create_weight exist because the loader requires every v1 symbol
// (src/backend/mod.rs:553-575), and answer UNSUPPORTED_DTYPE.

#include <cmath>
#include <cstdio>
#include <cstring>
#include <new>

#include "sr_internal.hpp"

namespace sr {

int32_t fail(Ctx *ctx, int32_t status, const std::string &message) {
    if (ctx != nullptr) {
        ctx->error = message;
    }
    return status;
}

int32_t hip_fail(Ctx *ctx, hipError_t err, const char *what) {
    std::string message = "HIP error ";
    message += hipGetErrorName(err);
    message += " (";
    message += hipGetErrorString(err);
    message += ") in ";
    message += what;
    return fail(ctx, err == hipErrorOutOfMemory ? kNoMemory : kDeviceError, message);
}

bool checked_mul(uint64_t a, uint64_t b, uint64_t *out) {
    if (b != 0 && a > UINT64_MAX / b) {
        return false;
    }
    *out = a * b;
    return true;
}

int32_t ensure_buffer(Ctx *ctx, DeviceBuffer &buf, size_t bytes, bool zero) {
    if (bytes <= buf.bytes) {
        return kOk;
    }
    // Growing frees the old allocation; finish queued work that may use it.
    SR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (buf.ptr != nullptr) {
        SR_HIP(ctx, hipFree(buf.ptr));
        buf.ptr = nullptr;
        buf.bytes = 0;
    }
    size_t rounded = (bytes + ((size_t)1 << 20) - 1) & ~(((size_t)1 << 20) - 1);
    SR_HIP(ctx, hipMalloc(&buf.ptr, rounded));
    if (zero) {
        SR_HIP(ctx, hipMemset(buf.ptr, 0, rounded));
    }
    buf.bytes = rounded;
    return kOk;
}

int32_t take_error_word(Ctx *ctx, uint32_t *word) {
    SR_HIP(ctx, hipGetLastError());
    SR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    *word = 0;
    SR_HIP(ctx, hipMemcpy(word, ctx->d_error_word, sizeof *word, hipMemcpyDeviceToHost));
    if (*word != 0) {
        uint32_t zero = 0;
        SR_HIP(ctx, hipMemcpy(ctx->d_error_word, &zero, sizeof zero, hipMemcpyHostToDevice));
    }
    return kOk;
}

int32_t error_word_status(Ctx *ctx, uint32_t word) {
    if (word == 0) return kOk;
    if (word & kErrNonFiniteVariance) {
        return fail(ctx, kInvalid, "RMSNorm variance is not finite (activation overflow)");
    }
    if (word & kErrNonFiniteKv) {
        return fail(ctx, kInvalid, "KV append contains a non-finite value");
    }
    return fail(ctx, kInvalid,
                "prefill attention met a K/V/q value outside the fp16 range of its MFMA "
                "operands; repeat the call synchronously to recompute it on the f32 path");
}

int32_t finish_call(Ctx *ctx, bool async) {
    SR_HIP(ctx, hipGetLastError());
    if (async) {
        return kOk;
    }
    uint32_t word = 0;
    int32_t st = take_error_word(ctx, &word);
    if (st != kOk) return st;
    return error_word_status(ctx, word);
}

const RopeTable &rope_table(Ctx *ctx, float theta, uint32_t rotary_dim) {
    if (ctx->rope_theta != theta || ctx->rope_dim != rotary_dim) {
        for (uint32_t i = 0; i < rotary_dim / 2 && i < 128; ++i) {
            // src/model/math.rs:90-91: theta.powf((2*i) as f32 / rotary_dim as f32)
            const float exponent = (float)(2 * i) / (float)rotary_dim;
            ctx->rope.denom[i] = powf(theta, exponent);
        }
        ctx->rope_theta = theta;
        ctx->rope_dim = rotary_dim;
    }
    return ctx->rope;
}

}  // namespace sr

using namespace sr;

extern "C" {

SAFETYRAISE_KERNEL_EXPORT uint32_t safetyraise_kernel_abi_version(void) {
    return SAFETYRAISE_KERNEL_ABI_VERSION;
}

SAFETYRAISE_KERNEL_EXPORT const char *safetyraise_kernel_name(void) {
    return "safetyraise-mi355x-gfx950";
}

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_create_context(
    const safetyraise_kernel_context_options *options, safetyraise_kernel_context **out_context) {
    if (options == nullptr || out_context == nullptr ||
        options->abi_version != SAFETYRAISE_KERNEL_ABI_VERSION ||
        options->struct_size < sizeof(safetyraise_kernel_context_options)) {
        return kInvalid;
    }
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
        return kDeviceError;  // no GPU: this plugin has no host fallback
    }
    Ctx *ctx = new (std::nothrow) Ctx();
    if (ctx == nullptr) {
        return kNoMemory;
    }
    hipError_t err = hipGetDevice(&ctx->device);
    if (err == hipSuccess) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, ctx->device) == hipSuccess &&
            prop.multiProcessorCount > 0) {
            ctx->num_cus = prop.multiProcessorCount;
        }
        // A blocking stream: ordered with the legacy default stream, so work a
        // caller queues there (e.g. a framework's allocations) precedes ours.
        err = hipStreamCreate(&ctx->own_stream);
    }
    if (err == hipSuccess) {
        ctx->stream = ctx->own_stream;
        // word 0 is the error word; the rest stays zero and serves the
        // prefill kernels as a readable stand-in for absent norm weights
        // (up to 256 floats)
        err = hipMalloc(&ctx->d_error_word, kErrorBlockBytes);
    }
    if (err == hipSuccess) {
        err = hipMemset(ctx->d_error_word, 0, kErrorBlockBytes);
    }
    if (err != hipSuccess) {
        if (ctx->d_error_word != nullptr) (void)hipFree(ctx->d_error_word);
        if (ctx->own_stream != nullptr) (void)hipStreamDestroy(ctx->own_stream);
        delete ctx;
        return err == hipErrorOutOfMemory ? kNoMemory : kDeviceError;
    }
    *out_context = ctx;
    return kOk;
}

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_destroy_context(
    safetyraise_kernel_context *context) {
    if (context == nullptr) {
        return kInvalid;
    }
    int32_t status = kOk;
    if (hipStreamSynchronize(context->stream) != hipSuccess) {
        status = kDeviceError;
    }
    for (DeviceBuffer *b : {&context->staging, &context->partials, &context->rope_scratch}) {
        if (b->ptr != nullptr) (void)hipFree(b->ptr);
    }
    if (context->d_error_word != nullptr) (void)hipFree(context->d_error_word);
    if (context->own_stream != nullptr) (void)hipStreamDestroy(context->own_stream);
    delete context;
    return status;
}

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_get_capabilities(
    safetyraise_kernel_context *context, safetyraise_kernel_capabilities *out_capabilities) {
    if (context == nullptr || out_capabilities == nullptr ||
        out_capabilities->struct_size < sizeof(safetyraise_kernel_capabilities)) {
        return fail(context, kInvalid, "capabilities pointer or struct_size is invalid");
    }
    out_capabilities->abi_version = SAFETYRAISE_KERNEL_ABI_VERSION;
    out_capabilities->struct_size = sizeof(safetyraise_kernel_capabilities);
    out_capabilities->dtype_mask = 0;  // no linear weights: the engine keeps projections
    out_capabilities->device_kind = SAFETYRAISE_KERNEL_DEVICE_OTHER;
    out_capabilities->flags = SAFETYRAISE_MI355X_CAP_ATTENTION | SAFETYRAISE_MI355X_CAP_GDN |
                              SAFETYRAISE_MI355X_CAP_DEVICE_STATE;
    out_capabilities->max_rows = 0;
    out_capabilities->max_cols = 0;
    return kOk;
}

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_create_weight(
    safetyraise_kernel_context *context, const uint8_t *data, uint64_t byte_len, uint64_t rows,
    uint64_t cols, uint32_t dtype, safetyraise_kernel_weight **out_weight) {
    (void)data;
    (void)byte_len;
    (void)rows;
    (void)cols;
    if (context == nullptr || out_weight == nullptr) {
        return fail(context, kInvalid, "weight arguments are invalid");
    }
    char message[128];
    snprintf(message, sizeof message,
             "dtype %u is not supported: this plugin provides attention and GDN only", dtype);
    return fail(context, kUnsupportedDtype, message);
}

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_destroy_weight(
    safetyraise_kernel_context *context, safetyraise_kernel_weight *weight) {
    if (weight == nullptr) {
        return fail(context, kInvalid, "weight handle is NULL");
    }
    delete weight;
    return kOk;
}

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_linear(
    safetyraise_kernel_context *context, safetyraise_kernel_weight *weight, const float *input,
    uint64_t input_rows, uint64_t input_cols, float *output, uint64_t output_rows,
    uint64_t output_cols) {
    (void)input;
    (void)input_rows;
    (void)input_cols;
    (void)output;
    (void)output_rows;
    (void)output_cols;
    if (context == nullptr || weight == nullptr) {
        return fail(context, kInvalid, "linear arguments are invalid");
    }
    return fail(context, kUnsupportedDtype, "linear is not provided by this plugin");
}

SAFETYRAISE_KERNEL_EXPORT const char *safetyraise_kernel_last_error(
    safetyraise_kernel_context *context) {
    return context == nullptr ? "no context to read an error from" : context->error.c_str();
}

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_set_stream(
    safetyraise_kernel_context *context, void *hip_stream) {
    if (context == nullptr) {
        return kInvalid;
    }
    hipStream_t next = hip_stream == nullptr ? context->own_stream : (hipStream_t)hip_stream;
    if (next != context->stream) {
        SR_HIP(context, hipStreamSynchronize(context->stream));
        context->stream = next;
    }
    return kOk;
}

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_synchronize(
    safetyraise_kernel_context *context) {
    if (context == nullptr) {
        return kInvalid;
    }
    return finish_call(context, false);
}

}  // extern "C"
