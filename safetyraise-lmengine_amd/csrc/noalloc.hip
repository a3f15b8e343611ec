// safetyraise_kernel_attention_forward_noalloc: safetyraise_kernel_attention_forward
// for callers that cannot allocate device memory (tight serving loops,
// harnesses that forbid hipMalloc).  Like the ordinary entry point it refuses
// calls while the stream is capturing a HIP graph: the sequences' lengths and
// page lists advance on the host when a call is made, so a replayed call
// would not advance them.  It runs the same kernels; the call's
// scratch (the split-K partial records of the decode and verify kernels, the
// per-row RoPE table of the verify and prefill kernels) comes from a fixed
// file-scope device array instead of the context's grow-on-demand buffers,
// and no staging is needed because the inputs must be device pointers.
//
// The array is one per GPU the library runs on: it is part of the library's
// code object, so it is reserved on a GPU (64 MiB of device memory) as soon
// as that code object is loaded there, i.e. at the library's first kernel
// launch on that GPU, whether or not this entry point is ever called, and it
// is held until the process ends.
// Its device address is looked up once per device (hipGetSymbolAddress, with
// that device current) and kept; host code never passes the array's name to
// a kernel, only that address.  Every call on a GPU shares its array: calls
// that overlap on one GPU (other threads, other contexts, other streams)
// race.  Nothing in it has to start at zero: every record and table entry is
// written before it is read within the call.
#include <cstdio>
#include <mutex>

#include "sr_device.hpp"

namespace sr {
namespace {

constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
constexpr int kMaxDevices = 64;
constexpr size_t kScratchAlign = 256;

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mutex;
void *g_scratch_ptr[kMaxDevices];  // device address of `scratch`, per device

// The device address of this GPU's `scratch`, looked up on the first call
// for the context's device with that device current.
int32_t scratch_address(Ctx *ctx, unsigned char **out) {
    if (ctx->device < 0 || ctx->device >= kMaxDevices) {
        return fail(ctx, kDeviceError, "device index out of range for the no-allocation scratch");
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[ctx->device] == nullptr) {
        int current = -1;
        SR_HIP(ctx, hipGetDevice(&current));
        if (current != ctx->device) SR_HIP(ctx, hipSetDevice(ctx->device));
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (current != ctx->device) (void)hipSetDevice(current);
        if (e != hipSuccess) return hip_fail(ctx, e, "hipGetSymbolAddress(scratch)");
        if (p == nullptr) return fail(ctx, kDeviceError, "the no-allocation scratch has no address");
        g_scratch_ptr[ctx->device] = p;
    }
    *out = (unsigned char *)g_scratch_ptr[ctx->device];
    return kOk;
}

// Parts of the region for one call.  attention_forward_impl asks for the
// RoPE table (at most once, before any partial records); the partial records
// of every launch then take the rest of the region (launches of one call run
// in stream order, so each reuses it, as the default buffers are reused).
struct FixedScratch {
    Ctx *ctx;
    unsigned char *base;
    size_t used;  // bytes held by the RoPE table
};

int32_t too_large(Ctx *ctx, size_t bytes, const char *what) {
    char message[224];
    snprintf(message, sizeof message,
             "attention_forward_noalloc: the call needs %zu more bytes of %s than the fixed "
             "%zu-byte scratch holds (use attention_forward, or split the call)",
             bytes, what, kNoAllocScratchBytes);
    return fail(ctx, kNoMemory, message);
}

void *fixed_rope(void *user, size_t bytes) {
    auto *s = (FixedScratch *)user;
    const size_t need = (bytes + kScratchAlign - 1) & ~(kScratchAlign - 1);
    if (s->used != 0 || need > kNoAllocScratchBytes) {
        too_large(s->ctx, need, "RoPE table");
        return nullptr;
    }
    s->used = need;
    return s->base;
}

float *fixed_partials(void *user, size_t bytes) {
    auto *s = (FixedScratch *)user;
    if (bytes > kNoAllocScratchBytes - s->used) {
        too_large(s->ctx, bytes - (kNoAllocScratchBytes - s->used), "split-K records");
        return nullptr;
    }
    return (float *)(s->base + s->used);
}

}  // namespace
}  // namespace sr

using namespace sr;

extern "C" SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_attention_forward_noalloc(
    safetyraise_kernel_context *context, const safetyraise_kernel_attention_args *args) {
    if (context == nullptr) return kInvalid;
    const int32_t capture = refuse_under_capture(context, "attention_forward_noalloc");
    if (capture != kOk) return capture;
    if (args == nullptr || args->struct_size < sizeof(safetyraise_kernel_attention_args)) {
        return fail(context, kInvalid, "attention args pointer or struct_size is invalid");
    }
    if ((args->flags & SAFETYRAISE_MI355X_DEVICE_POINTERS) == 0) {
        return fail(context, kInvalid,
                    "attention_forward_noalloc needs DEVICE_POINTERS (host inputs would need a "
                    "device staging allocation)");
    }
    unsigned char *base = nullptr;
    const int32_t st = scratch_address(context, &base);
    if (st != kOk) return st;
    // no TimerScope: kernel timing creates events, which this entry point does not
    FixedScratch fs{context, base, 0};
    const AttnScratch s{fixed_partials, fixed_rope, &fs};
    return attention_forward_impl(context, args, s);
}
