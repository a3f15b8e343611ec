// Context lifetime, the nine ABI v1 symbols and the shared host helpers.
//
// ABI v1 is declared in include/safetyraise_kernel.h.  linear takes F32, F16
// and BF16 weights (dtype_mask bits 1-3), kept on the device from
// create_weight to destroy_weight, and runs on f32 MFMA (linear_kernels.hip);
// the engine's loader routes a projection here when its weight format's bit
// is set (src/backend/mod.rs:259-264) and falls back to its CPU matmul
// otherwise.

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
    ctx->async_pending = false;
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
                "an asynchronous prefill or verify call met a K/V/q value outside the fp16 "
                "range of its MFMA operands; truncate its sequences back (kv_truncate) and "
                "repeat it synchronously to recompute it on the f32 path");
}

int32_t finish_call(Ctx *ctx, bool async) {
    SR_HIP(ctx, hipGetLastError());
    if (async) {
        ctx->async_pending = true;
        return kOk;
    }
    uint32_t word = 0;
    int32_t st = take_error_word(ctx, &word);
    if (st != kOk) return st;
    return error_word_status(ctx, word);
}

int32_t refuse_under_capture(Ctx *ctx, const char *what) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(ctx->stream, &status) != hipSuccess) {
        (void)hipGetLastError();  // the query's own error is not this call's
        return kOk;
    }
    if (status == hipStreamCaptureStatusNone) return kOk;
    std::string message = what;
    message += " cannot be captured into a HIP graph: a call appends at the sequences' "
               "current lengths and advances them and their page lists on the host when it is "
               "made, so a replay would write the same cache positions again and never advance "
               "them";
    return fail(ctx, kInvalid, message.c_str());
}

int32_t report_pending_async(Ctx *ctx) {
    if (!ctx->async_pending) return kOk;
    uint32_t word = 0;
    const int32_t st = take_error_word(ctx, &word);
    if (st != kOk) return st;
    return error_word_status(ctx, word);
}

namespace {
thread_local KernelTimer *t_timer = nullptr;
}

TimerScope::TimerScope(Ctx *ctx) : prev_(t_timer) {
    t_timer = (ctx != nullptr && ctx->timer.enabled) ? &ctx->timer : nullptr;
}
TimerScope::~TimerScope() { t_timer = prev_; }

LaunchEvents timed_launch(const char *kernel) {
    KernelTimer *t = t_timer;
    if (t == nullptr) return {};
    if (t->used == t->records.size()) {
        if (t->records.size() >= KernelTimer::kMaxRecords) return {};  // window full: untimed
        KernelTimer::Record r{kernel, nullptr, nullptr};
        if (hipEventCreate(&r.start) != hipSuccess) return {};
        if (hipEventCreate(&r.stop) != hipSuccess) {
            (void)hipEventDestroy(r.start);
            return {};
        }
        t->records.push_back(r);
    }
    KernelTimer::Record &r = t->records[t->used++];
    r.name = kernel;
    return {r.start, r.stop};
}

static void destroy_timer_events(KernelTimer &t) {
    for (auto &r : t.records) {
        (void)hipEventDestroy(r.start);
        (void)hipEventDestroy(r.stop);
    }
    t.records.clear();
    t.used = 0;
}

float rope_denominator(float theta, uint32_t i, uint32_t rotary_dim) {
    // src/model/math.rs:90-91: theta.powf((2*i) as f32 / rotary_dim as f32)
    const float exponent = (float)(2 * i) / (float)rotary_dim;
    return powf(theta, exponent);
}

const RopeTable &rope_table(Ctx *ctx, float theta, uint32_t rotary_dim) {
    if (ctx->rope_theta != theta || ctx->rope_dim != rotary_dim) {
        for (uint32_t i = 0; i < rotary_dim / 2 && i < 128; ++i) {
            ctx->rope.denom[i] = rope_denominator(theta, i, rotary_dim);
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
    for (DeviceBuffer *b : {&context->staging, &context->partials, &context->rope_scratch,
                            &context->linear_in, &context->linear_out,
                            &context->linear_part}) {
        if (b->ptr != nullptr) (void)hipFree(b->ptr);
    }
    destroy_timer_events(context->timer);
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
    out_capabilities->dtype_mask = (UINT64_C(1) << SAFETYRAISE_KERNEL_DTYPE_F32) |
                                   (UINT64_C(1) << SAFETYRAISE_KERNEL_DTYPE_F16) |
                                   (UINT64_C(1) << SAFETYRAISE_KERNEL_DTYPE_BF16);
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
    // native/cpu/safetyraise_cpu.c:140-189: byte_len must equal
    // rows * cols * element size, and the bytes are copied before returning
    if (context == nullptr || out_weight == nullptr) {
        return fail(context, kInvalid, "weight arguments are invalid");
    }
    if (dtype != SAFETYRAISE_KERNEL_DTYPE_F32 && dtype != SAFETYRAISE_KERNEL_DTYPE_F16 &&
        dtype != SAFETYRAISE_KERNEL_DTYPE_BF16) {
        char message[128];
        snprintf(message, sizeof message, "weight dtype %u is not supported (F32, F16, BF16 are)",
                 dtype);
        return fail(context, kUnsupportedDtype, message);
    }
    const uint64_t element = dtype == SAFETYRAISE_KERNEL_DTYPE_F32 ? 4 : 2;
    uint64_t count = 0, bytes = 0;
    if (!checked_mul(rows, cols, &count) || !checked_mul(count, element, &bytes) ||
        bytes != byte_len || (byte_len != 0 && data == nullptr)) {
        return fail(context, kInvalid, "weight byte length does not match its shape and dtype");
    }
    if (rows > UINT32_MAX || cols > UINT32_MAX) {
        return fail(context, kOverflow, "weight dimensions exceed 2^32 - 1");
    }
    auto *weight = new (std::nothrow) safetyraise_kernel_weight;
    if (weight == nullptr) {
        return fail(context, kNoMemory, "cannot allocate a weight handle");
    }
    weight->rows = rows;
    weight->cols = cols;
    weight->dtype = dtype;
    if (bytes != 0) {
        hipError_t e = hipMalloc(&weight->d_data, sr::linear_weight_bytes(rows, cols, dtype));
        if (dtype == SAFETYRAISE_KERNEL_DTYPE_BF16) {
            // the row-major bytes go through a temporary device buffer into
            // the tile layout the bf16 kernels read
            void *rowmajor = nullptr;
            if (e == hipSuccess) e = hipMalloc(&rowmajor, bytes);
            if (e == hipSuccess) e = hipMemcpy(rowmajor, data, bytes, hipMemcpyHostToDevice);
            if (e == hipSuccess) {
                e = sr::linear_pack_bf16(context->stream, rowmajor, weight->d_data, rows, cols);
            }
            if (e == hipSuccess) e = hipStreamSynchronize(context->stream);
            if (rowmajor != nullptr) {
                const hipError_t f = hipFree(rowmajor);
                if (e == hipSuccess) e = f;
            }
        } else if (e == hipSuccess) {
            e = hipMemcpy(weight->d_data, data, bytes, hipMemcpyHostToDevice);
        }
        if (e != hipSuccess) {
            if (weight->d_data != nullptr) (void)hipFree(weight->d_data);
            delete weight;
            return hip_fail(context, e, "create_weight");
        }
    }
    *out_weight = weight;
    return kOk;
}

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_destroy_weight(
    safetyraise_kernel_context *context, safetyraise_kernel_weight *weight) {
    if (weight == nullptr) {
        return fail(context, kInvalid, "weight handle is NULL");
    }
    int32_t status = kOk;
    if (weight->d_data != nullptr) {
        // queued linear calls may still read it
        if (context != nullptr) SR_HIP(context, hipStreamSynchronize(context->stream));
        const hipError_t e = hipFree(weight->d_data);
        if (e != hipSuccess) status = hip_fail(context, e, "destroy_weight");
    }
    delete weight;
    return status;
}

namespace sr {
// The shape rules of native/cpu/safetyraise_cpu.c:214-220.
static int32_t check_linear(Ctx *ctx, const safetyraise_kernel_weight *w, const float *input,
                            uint64_t in_rows, uint64_t in_cols, const float *output,
                            uint64_t out_rows, uint64_t out_cols, uint64_t *in_count,
                            uint64_t *out_count) {
    if (w == nullptr || in_rows != out_rows || in_cols != w->cols || out_cols != w->rows ||
        !checked_mul(in_rows, in_cols, in_count) || !checked_mul(out_rows, out_cols, out_count) ||
        (*in_count != 0 && input == nullptr) || (*out_count != 0 && output == nullptr)) {
        return fail(ctx, kInvalid, "linear shapes or pointers are invalid");
    }
    if (in_rows > UINT32_MAX || *in_count > (UINT64_MAX >> 3) || *out_count > (UINT64_MAX >> 3)) {
        return fail(ctx, kOverflow, "linear dimensions are too large");
    }
    return kOk;
}

// The partial-sum buffer of a call that splits K (nullptr when it does not).
static int32_t linear_scratch(Ctx *ctx, const safetyraise_kernel_weight *w, uint64_t rows,
                              float **part) {
    const size_t bytes = linear_scratch_bytes((uint32_t)rows, (uint32_t)w->rows,
                                              (uint32_t)w->cols, w->dtype, ctx->num_cus);
    *part = nullptr;
    if (bytes == 0) return kOk;
    const int32_t e = ensure_buffer(ctx, ctx->linear_part, bytes, false);
    if (e != kOk) return e;
    *part = (float *)ctx->linear_part.ptr;
    return kOk;
}
}  // namespace sr

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_linear(
    safetyraise_kernel_context *context, safetyraise_kernel_weight *weight, const float *input,
    uint64_t input_rows, uint64_t input_cols, float *output, uint64_t output_rows,
    uint64_t output_cols) {
    if (context == nullptr) {
        return kInvalid;
    }
    TimerScope timer_scope(context);
    uint64_t in_count = 0, out_count = 0;
    const int32_t st = check_linear(context, weight, input, input_rows, input_cols, output,
                                    output_rows, output_cols, &in_count, &out_count);
    if (st != kOk) return st;
    // native/cpu/safetyraise_cpu.c:221-226: every input must be finite
    for (uint64_t i = 0; i < in_count; ++i) {
        if (!std::isfinite(input[i])) {
            return fail(context, kInvalid, "linear input contains non-finite values");
        }
    }
    if (out_count == 0) return kOk;
    int32_t e = ensure_buffer(context, context->linear_in, (size_t)(in_count ? in_count : 1) * 4,
                              false);
    if (e != kOk) return e;
    e = ensure_buffer(context, context->linear_out, (size_t)out_count * 4, false);
    if (e != kOk) return e;
    float *part = nullptr;
    e = linear_scratch(context, weight, input_rows, &part);
    if (e != kOk) return e;
    float *d_in = (float *)context->linear_in.ptr;
    float *d_out = (float *)context->linear_out.ptr;
    if (in_count != 0) {
        SR_HIP(context, hipMemcpyAsync(d_in, input, in_count * 4, hipMemcpyHostToDevice,
                                       context->stream));
    }
    SR_HIP(context, launch_linear(context->stream, d_in, weight->d_data, weight->dtype, d_out,
                                  (uint32_t)input_rows, (uint32_t)weight->rows,
                                  (uint32_t)weight->cols, part, context->num_cus));
    SR_HIP(context, hipMemcpyAsync(output, d_out, out_count * 4, hipMemcpyDeviceToHost,
                                   context->stream));
    SR_HIP(context, hipStreamSynchronize(context->stream));
    return kOk;
}

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_linear_device(
    safetyraise_kernel_context *context, safetyraise_kernel_weight *weight, const float *input,
    uint64_t input_rows, uint64_t input_cols, float *output, uint64_t output_rows,
    uint64_t output_cols) {
    if (context == nullptr) {
        return kInvalid;
    }
    TimerScope timer_scope(context);
    uint64_t in_count = 0, out_count = 0;
    const int32_t st = check_linear(context, weight, input, input_rows, input_cols, output,
                                    output_rows, output_cols, &in_count, &out_count);
    if (st != kOk) return st;
    if (out_count == 0) return kOk;
    float *part = nullptr;
    const int32_t e = linear_scratch(context, weight, input_rows, &part);
    if (e != kOk) return e;
    SR_HIP(context, launch_linear(context->stream, input, weight->d_data, weight->dtype, output,
                                  (uint32_t)input_rows, (uint32_t)weight->rows,
                                  (uint32_t)weight->cols, part, context->num_cus));
    return kOk;
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

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_timing_enable(
    safetyraise_kernel_context *context, uint32_t enable) {
    if (context == nullptr) {
        return kInvalid;
    }
    // records of launches still queued must not be reused under them
    SR_HIP(context, hipStreamSynchronize(context->stream));
    context->timer.enabled = enable != 0;
    context->timer.used = 0;
    if (!context->timer.enabled) destroy_timer_events(context->timer);
    return kOk;
}

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_timing_read(
    safetyraise_kernel_context *context, uint32_t index, const char **out_name,
    uint64_t *out_launches, double *out_total_ms) {
    if (context == nullptr) {
        return kInvalid;
    }
    if (out_name == nullptr || out_launches == nullptr || out_total_ms == nullptr) {
        return fail(context, kInvalid, "timing_read output pointer is NULL");
    }
    SR_HIP(context, hipStreamSynchronize(context->stream));
    const KernelTimer &t = context->timer;
    // distinct names in order of first launch
    std::vector<const char *> names;
    for (size_t i = 0; i < t.used; ++i) {
        bool seen = false;
        for (const char *n : names) seen = seen || std::strcmp(n, t.records[i].name) == 0;
        if (!seen) names.push_back(t.records[i].name);
    }
    if (index >= names.size()) {
        return fail(context, kInvalid, "timing_read index is past the last kernel name");
    }
    double total = 0.0;
    uint64_t launches = 0;
    for (size_t i = 0; i < t.used; ++i) {
        if (std::strcmp(names[index], t.records[i].name) != 0) continue;
        float ms = 0.0f;
        SR_HIP(context, hipEventElapsedTime(&ms, t.records[i].start, t.records[i].stop));
        total += ms;
        ++launches;
    }
    *out_name = names[index];
    *out_launches = launches;
    *out_total_ms = total;
    return kOk;
}

}  // extern "C"
