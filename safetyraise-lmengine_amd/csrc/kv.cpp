// Paged bf16 KV cache in HBM — the device-resident counterpart of the
// reference PagedKvCache (src/engine/state.rs:19-127) and of the snapshot
// semantics of SequenceState::checkpoint (state.rs:222-224).
//
// Host side keeps, per sequence slot, the length and the page list; pages are
// reference counted.  A fork shares every page (O(pages) host work, one
// device-side copy of the page-table row).  The first write into a shared,
// partly filled last page copies that page first, as Arc::make_mut does for
// the reference's last page (state.rs:70).  The device page table
// [max_sequences][pages_per_seq] is kept in step with the host lists by small
// kernels whose updates travel as kernel arguments, so nothing reads host
// memory after a call returns.

#include <algorithm>
#include <cstring>
#include <new>

#include "sr_internal.hpp"

namespace sr {

namespace {

using Pool = safetyraise_kernel_kv_pool;

int32_t check_seq(Ctx *ctx, Pool *pool, uint32_t seq) {
    if (pool == nullptr || seq >= pool->max_sequences || !pool->seqs[seq].open) {
        return fail(ctx, kInvalid, "KV sequence handle is not open");
    }
    return kOk;
}

void release_page(Pool *pool, int32_t page) {
    if (--pool->refcount[page] == 0) {
        pool->free_pages.push_back(page);
    }
}

int32_t alloc_page(Pool *pool) {
    const int32_t page = pool->free_pages.back();
    pool->free_pages.pop_back();
    pool->refcount[page] = 1;
    return page;
}

int32_t upload_entries(Ctx *ctx, Pool *pool, uint32_t seq, const std::vector<uint32_t> &index,
                       TableBatch *batch) {
    if (index.empty()) {
        return kOk;
    }
    TableBatch local;
    TableBatch &b = batch != nullptr ? *batch : local;
    for (size_t i = 0; i < index.size(); ++i) {
        b.idx.push_back(seq * pool->pages_per_seq + index[i]);
        b.val.push_back(pool->seqs[seq].pages[index[i]]);
    }
    return batch != nullptr ? kOk : kv_flush_table(ctx, pool, local);
}

}  // namespace

// Makes pages [len, len+n) of the sequence writable: copies a shared partial
// last page, allocates fresh pages, and queues the page-table update.
// Rejects writes past max_tokens (state.rs:53-55).
int32_t kv_flush_table(Ctx *ctx, Pool *pool, TableBatch &batch) {
    if (!batch.idx.empty()) {
        SR_HIP(ctx, launch_page_table_set(ctx->stream, pool->d_page_table, batch.idx.data(),
                                          batch.val.data(), (int)batch.idx.size()));
    }
    batch.idx.clear();
    batch.val.clear();
    return kOk;
}

int32_t kv_prepare_append(Ctx *ctx, Pool *pool, uint32_t seq, uint64_t n, TableBatch *batch) {
    auto &s = pool->seqs[seq];
    const uint64_t new_len = s.len + n;
    if (n == 0 || new_len > pool->max_tokens) {
        return fail(ctx, kInvalid, "KV write would exceed the sequence capacity");
    }
    const uint64_t pt = pool->page_tokens;
    // Pages past the length (left by an earlier failed call) hold no data:
    // return them so that only a partial last page can ever be shared.
    while (s.pages.size() > (s.len + pt - 1) / pt) {
        release_page(pool, s.pages.back());
        s.pages.pop_back();
    }
    const bool cow = (s.len % pt != 0) && pool->refcount[s.pages[s.len / pt]] > 1;
    const uint64_t have = s.pages.size();
    const uint64_t need = (new_len + pt - 1) / pt;
    const uint64_t fresh = need > have ? need - have : 0;
    if (pool->free_pages.size() < fresh + (cow ? 1 : 0)) {
        return fail(ctx, kNoMemory, "KV page pool exhausted");
    }
    std::vector<uint32_t> changed;
    if (cow) {
        const uint32_t at = (uint32_t)(s.len / pt);
        const int32_t old = s.pages[at];
        const int32_t page = alloc_page(pool);
        SR_HIP(ctx, launch_page_copy(ctx->stream, pool, page, old));
        release_page(pool, old);
        s.pages[at] = page;
        changed.push_back(at);
    }
    for (uint64_t i = 0; i < fresh; ++i) {
        s.pages.push_back(alloc_page(pool));
        changed.push_back((uint32_t)(s.pages.size() - 1));
    }
    return upload_entries(ctx, pool, seq, changed, batch);
}

}  // namespace sr

using namespace sr;

extern "C" {

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_kv_create(
    safetyraise_kernel_context *context, const safetyraise_kernel_kv_options *options,
    safetyraise_kernel_kv_pool **out_pool) {
    if (context == nullptr) return kInvalid;
    if (options == nullptr || out_pool == nullptr ||
        options->struct_size < sizeof(safetyraise_kernel_kv_options)) {
        return fail(context, kInvalid, "kv options pointer or struct_size is invalid");
    }
    const auto &o = *options;
    if (o.kv_heads == 0 || o.head_dim == 0 || o.head_dim > kGenericMaxHeadDim ||
        o.page_tokens < 16 || o.page_tokens > 65536 || (o.page_tokens & (o.page_tokens - 1)) != 0 ||
        o.num_pages == 0 || o.num_pages > INT32_MAX || o.max_tokens == 0 ||
        o.max_tokens > INT32_MAX || o.max_sequences == 0 || o.max_sequences > (1u << 20)) {
        return fail(context, kInvalid,
                    "kv geometry is invalid (head_dim 1..512, page_tokens a power of two in "
                    "16..65536, non-zero sizes)");
    }
    uint64_t page_elems, bytes, table;
    const uint64_t pages_per_seq = (o.max_tokens + o.page_tokens - 1) / o.page_tokens;
    if (!checked_mul((uint64_t)o.kv_heads * o.head_dim, o.page_tokens, &page_elems) ||
        !checked_mul(page_elems * 2, o.num_pages, &bytes) ||
        !checked_mul(pages_per_seq, o.max_sequences, &table) || table > (uint64_t)UINT32_MAX) {
        return fail(context, kOverflow, "kv pool size overflows");
    }
    Pool *pool = new (std::nothrow) Pool();
    if (pool == nullptr) return fail(context, kNoMemory, "kv pool allocation failed");
    pool->kv_heads = o.kv_heads;
    pool->head_dim = o.head_dim;
    pool->page_tokens = o.page_tokens;
    pool->num_pages = o.num_pages;
    pool->max_tokens = o.max_tokens;
    pool->max_sequences = o.max_sequences;
    pool->pages_per_seq = (uint32_t)pages_per_seq;
    hipError_t err = hipMalloc(&pool->k_pages, bytes);
    if (err == hipSuccess) err = hipMalloc(&pool->v_pages, bytes);
    if (err == hipSuccess) err = hipMalloc(&pool->d_page_table, table * sizeof(int32_t));
    if (err == hipSuccess) err = hipMemset(pool->d_page_table, 0, table * sizeof(int32_t));
    if (err != hipSuccess) {
        if (pool->k_pages) (void)hipFree(pool->k_pages);
        if (pool->v_pages) (void)hipFree(pool->v_pages);
        if (pool->d_page_table) (void)hipFree(pool->d_page_table);
        delete pool;
        return hip_fail(context, err, "kv pool allocation");
    }
    pool->seqs.resize(o.max_sequences);
    pool->refcount.assign(o.num_pages, 0);
    pool->free_pages.resize(o.num_pages);
    for (uint64_t i = 0; i < o.num_pages; ++i) {
        pool->free_pages[i] = (int32_t)(o.num_pages - 1 - i);  // page 0 handed out first
    }
    if (o.page_order_seed != 0) {
        // Fisher-Yates over the free list with a splitmix64 stream
        uint64_t state = o.page_order_seed;
        auto next = [&state]() {
            uint64_t z = (state += 0x9E3779B97F4A7C15ull);
            z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
            z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
            return z ^ (z >> 31);
        };
        for (uint64_t i = o.num_pages - 1; i > 0; --i) {
            const uint64_t j = next() % (i + 1);
            std::swap(pool->free_pages[i], pool->free_pages[j]);
        }
    }
    *out_pool = pool;
    return kOk;
}

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_kv_destroy(
    safetyraise_kernel_context *context, safetyraise_kernel_kv_pool *pool) {
    if (context == nullptr || pool == nullptr) return fail(context, kInvalid, "kv pool is NULL");
    SR_HIP(context, hipStreamSynchronize(context->stream));
    (void)hipFree(pool->k_pages);
    (void)hipFree(pool->v_pages);
    (void)hipFree(pool->d_page_table);
    delete pool;
    return kOk;
}

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_kv_open(
    safetyraise_kernel_context *context, safetyraise_kernel_kv_pool *pool, uint32_t *out_sequence) {
    if (context == nullptr) return kInvalid;
    if (pool == nullptr || out_sequence == nullptr) return fail(context, kInvalid, "NULL argument");
    for (uint32_t i = 0; i < pool->max_sequences; ++i) {
        if (!pool->seqs[i].open) {
            pool->seqs[i].open = true;
            pool->seqs[i].len = 0;
            pool->seqs[i].pages.clear();
            *out_sequence = i;
            return kOk;
        }
    }
    return fail(context, kNoMemory, "no free KV sequence slot");
}

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_kv_fork(
    safetyraise_kernel_context *context, safetyraise_kernel_kv_pool *pool, uint32_t source,
    uint32_t *out_sequence) {
    if (context == nullptr) return kInvalid;
    int32_t st = check_seq(context, pool, source);
    if (st != kOk) return st;
    if (out_sequence == nullptr) return fail(context, kInvalid, "NULL argument");
    uint32_t slot = 0;
    st = safetyraise_kernel_kv_open(context, pool, &slot);
    if (st != kOk) return st;
    auto &src = pool->seqs[source];
    auto &dst = pool->seqs[slot];
    dst.len = src.len;
    const uint64_t used = (src.len + pool->page_tokens - 1) / pool->page_tokens;
    dst.pages.assign(src.pages.begin(), src.pages.begin() + std::min<uint64_t>(used, src.pages.size()));
    for (int32_t page : dst.pages) {
        ++pool->refcount[page];
    }
    if (!dst.pages.empty()) {
        SR_HIP(context, hipMemcpyAsync(pool->d_page_table + (size_t)slot * pool->pages_per_seq,
                                       pool->d_page_table + (size_t)source * pool->pages_per_seq,
                                       dst.pages.size() * sizeof(int32_t), hipMemcpyDeviceToDevice,
                                       context->stream));
    }
    *out_sequence = slot;
    return kOk;
}

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_kv_close(
    safetyraise_kernel_context *context, safetyraise_kernel_kv_pool *pool, uint32_t sequence) {
    if (context == nullptr) return kInvalid;
    int32_t st = check_seq(context, pool, sequence);
    if (st != kOk) return st;
    auto &s = pool->seqs[sequence];
    for (int32_t page : s.pages) {
        release_page(pool, page);
    }
    s.pages.clear();
    s.len = 0;
    s.open = false;
    return kOk;
}

// state.rs:99-119: shrinking only; whole pages past the new length return
// to the pool, a partial tail page stays (and is copied on the next write if
// another sequence still shares it).
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_kv_truncate(
    safetyraise_kernel_context *context, safetyraise_kernel_kv_pool *pool, uint32_t sequence,
    uint64_t len) {
    if (context == nullptr) return kInvalid;
    int32_t st = check_seq(context, pool, sequence);
    if (st != kOk) return st;
    auto &s = pool->seqs[sequence];
    if (len > s.len) {
        return fail(context, kInvalid, "truncate cannot extend the KV cache");
    }
    const uint64_t keep = (len + pool->page_tokens - 1) / pool->page_tokens;
    while (s.pages.size() > keep) {
        release_page(pool, s.pages.back());
        s.pages.pop_back();
    }
    s.len = len;
    return kOk;
}

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_kv_len(
    safetyraise_kernel_context *context, safetyraise_kernel_kv_pool *pool, uint32_t sequence,
    uint64_t *out_len) {
    if (context == nullptr) return kInvalid;
    int32_t st = check_seq(context, pool, sequence);
    if (st != kOk) return st;
    if (out_len == nullptr) return fail(context, kInvalid, "NULL argument");
    *out_len = pool->seqs[sequence].len;
    return kOk;
}

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_kv_append(
    safetyraise_kernel_context *context, safetyraise_kernel_kv_pool *pool, uint32_t sequence,
    const void *keys, const void *values, uint64_t tokens, uint32_t flags) {
    if (context == nullptr) return kInvalid;
    int32_t st = check_seq(context, pool, sequence);
    if (st != kOk) return st;
    const bool device = (flags & SAFETYRAISE_MI355X_DEVICE_POINTERS) != 0;
    const bool async = (flags & SAFETYRAISE_MI355X_ASYNC) != 0;
    const bool bf16 = (flags & SAFETYRAISE_MI355X_INPUT_BF16) != 0;
    if (async && !device) {
        return fail(context, kInvalid, "ASYNC needs DEVICE_POINTERS");
    }
    if (tokens == 0 || keys == nullptr || values == nullptr) {
        return fail(context, kInvalid, "KV append needs at least one row and non-NULL data");
    }
    if (device && ((((uintptr_t)keys) | ((uintptr_t)values)) & 15u) != 0) {
        return fail(context, kInvalid, "device pointers must be 16-byte aligned");
    }
    uint64_t elems, bytes;
    if (!checked_mul(tokens, (uint64_t)pool->kv_heads * pool->head_dim, &elems) ||
        !checked_mul(elems, bf16 ? 2 : 4, &bytes)) {
        return fail(context, kOverflow, "KV append size overflows");
    }
    auto &s = pool->seqs[sequence];
    const uint64_t old_len = s.len;
    st = kv_prepare_append(context, pool, sequence, tokens);
    if (st != kOk) return st;
    const void *dk = keys;
    const void *dv = values;
    if (!device) {
        const size_t half = (bytes + 255) & ~(size_t)255;
        st = ensure_buffer(context, context->staging, 2 * half, false);
        if (st != kOk) return st;
        char *base = (char *)context->staging.ptr;
        SR_HIP(context, hipMemcpyAsync(base, keys, bytes, hipMemcpyHostToDevice, context->stream));
        SR_HIP(context,
               hipMemcpyAsync(base + half, values, bytes, hipMemcpyHostToDevice, context->stream));
        dk = base;
        dv = base + half;
    }
    SR_HIP(context, launch_kv_scatter(context->stream, pool, sequence, old_len, tokens, dk, dv, bf16,
                                      context->d_error_word));
    s.len = old_len + tokens;
    st = finish_call(context, async);
    if (st != kOk && !async) {
        s.len = old_len;  // the reference rejects the row before writing it
    }
    return st;
}

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_kv_read(
    safetyraise_kernel_context *context, safetyraise_kernel_kv_pool *pool, uint32_t sequence,
    uint64_t start, uint64_t tokens, float *keys, float *values) {
    if (context == nullptr) return kInvalid;
    int32_t st = check_seq(context, pool, sequence);
    if (st != kOk) return st;
    const auto &s = pool->seqs[sequence];
    if (start > s.len || tokens > s.len - start) {
        return fail(context, kInvalid, "KV token index out of range");
    }
    if (tokens == 0) return kOk;
    if (keys == nullptr || values == nullptr) return fail(context, kInvalid, "NULL argument");
    const uint64_t elems = tokens * pool->kv_heads * pool->head_dim;
    const size_t half = (elems * 4 + 255) & ~(size_t)255;
    st = ensure_buffer(context, context->staging, 2 * half, false);
    if (st != kOk) return st;
    float *dk = (float *)context->staging.ptr;
    float *dv = (float *)((char *)context->staging.ptr + half);
    SR_HIP(context, launch_kv_gather(context->stream, pool, sequence, start, tokens, dk, dv));
    SR_HIP(context, hipMemcpyAsync(keys, dk, elems * 4, hipMemcpyDeviceToHost, context->stream));
    SR_HIP(context, hipMemcpyAsync(values, dv, elems * 4, hipMemcpyDeviceToHost, context->stream));
    return finish_call(context, false);
}

}  // extern "C"
