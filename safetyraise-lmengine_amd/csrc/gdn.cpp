// Gated-delta-net state pool and forward entry point — the device-resident
// counterpart of RecurrentState (reference src/engine/state.rs:129-135) and
// of the Gdn::forward row loop (src/model/native.rs:720-742).
//
// Per sequence slot the pool holds the f32 state [Hv][Dv][Dk] and two
// buffers of the conv history [C][K-1] (oldest first, as state.rs:133); a
// host-side parity bit per slot says which buffer is current.  Each forward
// call reads the current buffer and writes the other, then flips the bit.

#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>
#include <vector>

#include "sr_internal.hpp"

namespace sr {


namespace {

using Pool = safetyraise_kernel_gdn_pool;

constexpr uint32_t kMaxKeepRows = 64;

int32_t check_seq(Ctx *ctx, Pool *pool, uint32_t seq) {
    if (pool == nullptr || seq >= pool->max_sequences || !pool->open[seq]) {
        return fail(ctx, kInvalid, "GDN sequence handle is not open");
    }
    return kOk;
}

// the sequence's current state buffer (which = 0) or its other one (1)
float *state_ptr(Pool *pool, uint32_t seq, uint32_t which = 0) {
    return pool->d_state + (size_t)pool->state_index(seq, which) * pool->state_elems();
}

float *history_ptr(Pool *pool, uint32_t seq, uint32_t parity) {
    return pool->d_history +
           ((size_t)parity * pool->max_sequences + seq) * pool->history_elems();
}

size_t align_up(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace

}  // namespace sr

using namespace sr;

extern "C" {

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_gdn_create(
    safetyraise_kernel_context *context, const safetyraise_kernel_gdn_options *options,
    safetyraise_kernel_gdn_pool **out_pool) {
    if (context == nullptr) return kInvalid;
    if (options == nullptr || out_pool == nullptr ||
        options->struct_size < sizeof(safetyraise_kernel_gdn_options)) {
        return fail(context, kInvalid, "gdn options pointer or struct_size is invalid");
    }
    const auto &o = *options;
    if (o.key_heads == 0 || o.value_heads == 0 || o.value_heads % o.key_heads != 0 ||
        o.key_dim == 0 || o.key_dim > kGdnMaxDim || o.value_dim == 0 || o.value_dim > kGdnMaxDim ||
        o.conv_kernel == 0 || o.conv_kernel > gdn_max_kernel() || o.max_sequences == 0 ||
        o.max_sequences > 65536) {
        return fail(context, kInvalid,
                    "GDN geometry is invalid (key_dim and value_dim 1..512, value_heads a "
                    "multiple of key_heads, conv kernel 1..8)");
    }
    if (o.keep_rows > kMaxKeepRows ||
        (o.keep_rows > 0 && o.value_dim % gdn_row_block() == 0 && o.key_dim == gdn_key_dim() &&
         o.value_dim != 128)) {
        return fail(context, kInvalid,
                    "GDN keep_rows must be at most 64 (value_dim 128 at key_dim 128)");
    }
    Pool *pool = new (std::nothrow) Pool();
    if (pool == nullptr) return fail(context, kNoMemory, "gdn pool allocation failed");
    pool->key_heads = o.key_heads;
    pool->value_heads = o.value_heads;
    pool->key_dim = o.key_dim;
    pool->value_dim = o.value_dim;
    pool->conv_kernel = o.conv_kernel;
    pool->max_sequences = o.max_sequences;
    pool->channels = 2 * o.key_heads * o.key_dim + o.value_heads * o.value_dim;
    pool->keep_rows = o.keep_rows;
    const size_t state_bytes =
        pool->state_elems() * pool->state_buffers() * o.max_sequences * sizeof(float);
    const size_t hist_bytes = std::max<size_t>(pool->history_elems(), 1) * 2 * o.max_sequences *
                              sizeof(float);
    const size_t rec_bytes =
        pool->record_elems() * o.keep_rows * (size_t)o.max_sequences * sizeof(float);
    hipError_t err = hipMalloc(&pool->d_state, state_bytes);
    if (err == hipSuccess) err = hipMalloc(&pool->d_history, hist_bytes);
    if (err == hipSuccess && rec_bytes > 0) err = hipMalloc(&pool->d_records, rec_bytes);
    if (err != hipSuccess) {
        if (pool->d_state) (void)hipFree(pool->d_state);
        if (pool->d_history) (void)hipFree(pool->d_history);
        if (pool->d_records) (void)hipFree(pool->d_records);
        delete pool;
        return hip_fail(context, err, "gdn pool allocation");
    }
    pool->open.assign(o.max_sequences, 0);
    pool->parity.assign(o.max_sequences, 0);
    pool->state_par.assign(o.max_sequences, 0);
    pool->kept.assign(o.max_sequences, Pool::kNoKept);
    pool->kept_at.assign(o.max_sequences, 0);
    *out_pool = pool;
    return kOk;
}

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_gdn_destroy(
    safetyraise_kernel_context *context, safetyraise_kernel_gdn_pool *pool) {
    if (context == nullptr || pool == nullptr) return fail(context, kInvalid, "gdn pool is NULL");
    SR_HIP(context, hipStreamSynchronize(context->stream));
    (void)hipFree(pool->d_state);
    (void)hipFree(pool->d_history);
    if (pool->d_records != nullptr) (void)hipFree(pool->d_records);
    delete pool;
    return kOk;
}

// New sequence: zero matrix and history (state.rs:167-180 `zeros`).
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_gdn_open(
    safetyraise_kernel_context *context, safetyraise_kernel_gdn_pool *pool,
    uint32_t *out_sequence) {
    if (context == nullptr) return kInvalid;
    if (pool == nullptr || out_sequence == nullptr) return fail(context, kInvalid, "NULL argument");
    for (uint32_t i = 0; i < pool->max_sequences; ++i) {
        if (!pool->open[i]) {
            pool->state_par[i] = 0;
            SR_HIP(context, hipMemsetAsync(state_ptr(pool, i), 0,
                                           pool->state_elems() * sizeof(float), context->stream));
            if (pool->history_elems() > 0) {
                SR_HIP(context, hipMemsetAsync(history_ptr(pool, i, 0), 0,
                                               pool->history_elems() * sizeof(float),
                                               context->stream));
            }
            pool->open[i] = 1;
            pool->parity[i] = 0;
            pool->kept[i] = Pool::kNoKept;
            *out_sequence = i;
            return kOk;
        }
    }
    return fail(context, kNoMemory, "no free GDN sequence slot");
}

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_gdn_fork(
    safetyraise_kernel_context *context, safetyraise_kernel_gdn_pool *pool, uint32_t source,
    uint32_t *out_sequence) {
    if (context == nullptr) return kInvalid;
    int32_t st = check_seq(context, pool, source);
    if (st != kOk) return st;
    if (out_sequence == nullptr) return fail(context, kInvalid, "NULL argument");
    uint32_t slot = 0;
    st = safetyraise_kernel_gdn_open(context, pool, &slot);
    if (st != kOk) return st;
    SR_HIP(context, hipMemcpyAsync(state_ptr(pool, slot), state_ptr(pool, source),
                                   pool->state_elems() * sizeof(float), hipMemcpyDeviceToDevice,
                                   context->stream));
    if (pool->history_elems() > 0) {
        SR_HIP(context,
               hipMemcpyAsync(history_ptr(pool, slot, 0),
                              history_ptr(pool, source, pool->parity[source]),
                              pool->history_elems() * sizeof(float), hipMemcpyDeviceToDevice,
                              context->stream));
    }
    pool->parity[slot] = 0;
    *out_sequence = slot;
    return kOk;
}

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_gdn_close(
    safetyraise_kernel_context *context, safetyraise_kernel_gdn_pool *pool, uint32_t sequence) {
    if (context == nullptr) return kInvalid;
    int32_t st = check_seq(context, pool, sequence);
    if (st != kOk) return st;
    pool->open[sequence] = 0;
    return kOk;
}

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_gdn_read(
    safetyraise_kernel_context *context, safetyraise_kernel_gdn_pool *pool, uint32_t sequence,
    float *matrix, float *history) {
    if (context == nullptr) return kInvalid;
    int32_t st = check_seq(context, pool, sequence);
    if (st != kOk) return st;
    if (matrix != nullptr) {
        SR_HIP(context, hipMemcpyAsync(matrix, state_ptr(pool, sequence),
                                       pool->state_elems() * sizeof(float), hipMemcpyDeviceToHost,
                                       context->stream));
    }
    if (history != nullptr && pool->history_elems() > 0) {
        SR_HIP(context, hipMemcpyAsync(history,
                                       history_ptr(pool, sequence, pool->parity[sequence]),
                                       pool->history_elems() * sizeof(float),
                                       hipMemcpyDeviceToHost, context->stream));
    }
    return finish_call(context, false);
}

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_gdn_write(
    safetyraise_kernel_context *context, safetyraise_kernel_gdn_pool *pool, uint32_t sequence,
    const float *matrix, const float *history) {
    if (context == nullptr) return kInvalid;
    int32_t st = check_seq(context, pool, sequence);
    if (st != kOk) return st;
    if (matrix != nullptr) {
        SR_HIP(context, hipMemcpyAsync(state_ptr(pool, sequence), matrix,
                                       pool->state_elems() * sizeof(float), hipMemcpyHostToDevice,
                                       context->stream));
    }
    pool->kept[sequence] = Pool::kNoKept;
    if (history != nullptr && pool->history_elems() > 0) {
        SR_HIP(context, hipMemcpyAsync(history_ptr(pool, sequence, pool->parity[sequence]), history,
                                       pool->history_elems() * sizeof(float),
                                       hipMemcpyHostToDevice, context->stream));
    }
    return finish_call(context, false);
}

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_gdn_forward(
    safetyraise_kernel_context *context, const safetyraise_kernel_gdn_args *args) {
    if (context == nullptr) return kInvalid;
    Ctx *ctx = context;
    TimerScope timer_scope(ctx);
    if (args == nullptr || args->struct_size < sizeof(safetyraise_kernel_gdn_args)) {
        return fail(ctx, kInvalid, "gdn args pointer or struct_size is invalid");
    }
    const auto &A = *args;
    Pool *pool = A.state;
    const bool device = (A.flags & SAFETYRAISE_MI355X_DEVICE_POINTERS) != 0;
    const bool async = (A.flags & SAFETYRAISE_MI355X_ASYNC) != 0;
    const bool bf16 = (A.flags & SAFETYRAISE_MI355X_INPUT_BF16) != 0;
    if (pool == nullptr) return fail(ctx, kInvalid, "gdn_forward needs a state pool");
    if (async && !device) return fail(ctx, kInvalid, "ASYNC needs DEVICE_POINTERS");
    if (!std::isfinite(A.eps) || A.eps <= 0.0f) {
        return fail(ctx, kInvalid, "RMSNorm shape or epsilon is invalid");
    }
    if (A.num_seqs == 0 || A.num_seqs > SAFETYRAISE_MI355X_MAX_BATCH || A.seq_ids == nullptr ||
        A.seq_rows == nullptr) {
        return fail(ctx, kInvalid, "GDN batch is empty or too large");
    }
    if (A.qkv == nullptr || A.z == nullptr || A.a == nullptr || A.b == nullptr ||
        A.a_log == nullptr || A.dt_bias == nullptr || A.conv_weight == nullptr ||
        A.norm == nullptr || A.out == nullptr) {
        return fail(ctx, kInvalid, "GDN input or output pointer is NULL");
    }
    const bool keep = (A.flags & SAFETYRAISE_MI355X_KEEP_ROWS) != 0;
    if (keep && pool->keep_rows == 0) {
        return fail(ctx, kInvalid, "KEEP_ROWS needs a GDN pool created with keep_rows > 0");
    }
    std::vector<GdnSeq> seqs(A.num_seqs);
    uint64_t total = 0;
    for (uint32_t i = 0; i < A.num_seqs; ++i) {
        const int32_t st = check_seq(ctx, pool, A.seq_ids[i]);
        if (st != kOk) return st;
        for (uint32_t j = 0; j < i; ++j) {
            if (A.seq_ids[j] == A.seq_ids[i]) {
                return fail(ctx, kInvalid, "a sequence appears twice in one call");
            }
        }
        if (A.seq_rows[i] == 0) return fail(ctx, kInvalid, "input is empty");
        if (keep && A.seq_rows[i] > pool->keep_rows) {
            return fail(ctx, kInvalid, "a KEEP_ROWS call has more rows than the pool's keep_rows");
        }
        const uint32_t id = A.seq_ids[i];
        GdnSeq &q = seqs[i];
        q.slot = id;
        q.rows = A.seq_rows[i];
        q.row0 = (uint32_t)total;
        q.parity = pool->parity[id];
        // KEEP_ROWS: read the current state buffer, write the other one (the
        // pre-call state stays for gdn_rollback); otherwise update in place
        q.state_in = pool->state_index(id, 0);
        q.state_out = keep ? pool->state_index(id, 1) : q.state_in;
        total += A.seq_rows[i];
    }
    if (total > INT32_MAX / std::max<uint32_t>(pool->channels, 1)) {
        return fail(ctx, kOverflow, "too many rows");
    }
    if (!async) {
        const int32_t pst = report_pending_async(ctx);
        if (pst != kOk) return pst;
    }
    const size_t esz = bf16 ? 2 : 4;
    const size_t width = (size_t)pool->value_heads * pool->value_dim;
    const size_t qkv_b = total * pool->channels * esz, z_b = total * width * esz;
    const size_t ab_b = total * pool->value_heads * esz, head_b = pool->value_heads * 4;
    const size_t conv_b = (size_t)pool->channels * pool->conv_kernel * 4;
    const size_t norm_b = pool->value_dim * 4, out_b = total * width * 4;

    GdnLaunch g{};
    g.pool = pool;
    g.err_word = ctx->d_error_word;
    g.eps = A.eps;
    g.bf16_in = bf16;
    g.qkv = A.qkv;
    g.z = A.z;
    g.a = A.a;
    g.b = A.b;
    g.a_log = A.a_log;
    g.dt_bias = A.dt_bias;
    g.conv_w = A.conv_weight;
    g.norm = A.norm;
    g.out = A.out;
    // raw delta-rule output [rows][Hv*Dv]
    size_t need = align_up(out_b);
    struct Region {
        const void *host;
        size_t bytes;
        size_t off;
    } regions[8] = {{A.qkv, qkv_b, 0},    {A.z, z_b, 0},           {A.a, ab_b, 0},
                    {A.b, ab_b, 0},       {A.a_log, head_b, 0},     {A.dt_bias, head_b, 0},
                    {A.conv_weight, conv_b, 0}, {A.norm, norm_b, 0}};
    size_t out_off = 0;
    if (!device) {
        for (auto &r : regions) {
            r.off = need;
            need += align_up(r.bytes);
        }
        out_off = need;
        need += align_up(out_b);
    }
    // per-chunk records of the chunked prefill form (host inputs are staged
    // at 256-byte offsets, so only device qkv can be unaligned)
    const size_t rec_b = gdn_chunk_rec_bytes(pool, seqs.data(), (int)A.num_seqs, keep,
                                             !device || ((uintptr_t)A.qkv & 15) == 0);
    const size_t rec_off = need;
    need += align_up(rec_b);
    int32_t st = ensure_buffer(ctx, ctx->staging, need, false);
    if (st != kOk) return st;
    char *base = (char *)ctx->staging.ptr;
    g.raw = (float *)base;
    g.chunk_rec = rec_b > 0 ? (float *)(base + rec_off) : nullptr;
    g.num_cus = ctx->num_cus;
    if (!device) {
        for (auto &r : regions) {
            SR_HIP(ctx, hipMemcpyAsync(base + r.off, r.host, r.bytes, hipMemcpyHostToDevice,
                                       ctx->stream));
        }
        g.qkv = base + regions[0].off;
        g.z = base + regions[1].off;
        g.a = base + regions[2].off;
        g.b = base + regions[3].off;
        g.a_log = (const float *)(base + regions[4].off);
        g.dt_bias = (const float *)(base + regions[5].off);
        g.conv_w = (const float *)(base + regions[6].off);
        g.norm = (const float *)(base + regions[7].off);
        g.out = (float *)(base + out_off);
    }
    g.keep = keep;
    g.records = pool->d_records;
    g.rec_stride = (uint32_t)pool->record_elems();
    g.keep_rows = pool->keep_rows;
    SR_HIP(ctx, launch_gdn(ctx->stream, g, seqs.data(), (int)A.num_seqs, (uint32_t)total));
    for (const GdnSeq &q : seqs) {
        pool->parity[q.slot] ^= 1u;
        if (keep) pool->state_par[q.slot] ^= 1u;
        pool->kept[q.slot] = keep ? q.rows : Pool::kNoKept;
        pool->kept_at[q.slot] = q.rows;
    }
    if (!device) {
        SR_HIP(ctx, hipMemcpyAsync(A.out, g.out, out_b, hipMemcpyDeviceToHost, ctx->stream));
    }
    return finish_call(ctx, async);
}

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_gdn_rollback(
    safetyraise_kernel_context *context, safetyraise_kernel_gdn_pool *pool, uint32_t sequence,
    uint32_t rows, uint32_t flags) {
    if (context == nullptr) return kInvalid;
    Ctx *ctx = context;
    TimerScope timer_scope(ctx);
    int32_t st = check_seq(ctx, pool, sequence);
    if (st != kOk) return st;
    const uint32_t kept = pool->kept[sequence];
    if (kept == Pool::kNoKept) {
        return fail(ctx, kInvalid,
                    "gdn_rollback: the sequence's last call was not a KEEP_ROWS call");
    }
    if (rows > kept) {
        return fail(ctx, kInvalid, "gdn_rollback: more rows than the KEEP_ROWS call had");
    }
    const bool async = (flags & SAFETYRAISE_MI355X_ASYNC) != 0;
    if (!async) {
        st = report_pending_async(ctx);
        if (st != kOk) return st;
    }
    if (rows != pool->kept_at[sequence]) {
        // rebuild the state and history after `rows` rows into the current
        // buffers from the pre-call ones (which the KEEP_ROWS call only read)
        GdnRollback r;
        r.state_in = state_ptr(pool, sequence, 1);
        r.state_out = state_ptr(pool, sequence, 0);
        r.hist_in = history_ptr(pool, sequence, pool->parity[sequence] ^ 1u);
        r.hist_out = history_ptr(pool, sequence, pool->parity[sequence]);
        r.records = pool->d_records + (size_t)sequence * pool->keep_rows * pool->record_elems();
        r.rec_stride = (uint32_t)pool->record_elems();
        r.keep = rows;
        r.value_heads = pool->value_heads;
        r.channels = pool->channels;
        r.conv_k = pool->conv_kernel;
        r.key_dim = pool->key_dim;
        r.value_dim = pool->value_dim;
        SR_HIP(ctx, launch_gdn_rollback(ctx->stream, r));
        pool->kept_at[sequence] = rows;
    }
    return finish_call(ctx, async);
}

}  // extern "C"
