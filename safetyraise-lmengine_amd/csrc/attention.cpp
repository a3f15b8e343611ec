// safetyraise_kernel_attention_forward: the Attention::forward row loop of
// the reference (src/model/native.rs:615-645, projections excluded) for a
// batch of sequences, on the paged bf16 KV cache of kv.cpp.
//
// Argument checks mirror the reference's errors: causal_attention geometry
// (src/model/math.rs:109-124), apply_rope shape (math.rs:58-65), rms_norm
// epsilon (math.rs:29-35), KV capacity (src/engine/state.rs:53-55) and empty
// input (SequenceState::ensure_room, state.rs:208-216).  Non-finite K/V or
// norm variance are detected on the device; a synchronous call then fails
// with INVALID_ARGUMENT and the sequences keep their previous length.

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "sr_internal.hpp"

namespace sr {

namespace {

constexpr size_t kAlign = 256;
// Rows per sequence from which a call takes the chunked prefill kernels.
constexpr uint32_t kPrefillMinRows = 16;

size_t align_up(size_t x) { return (x + kAlign - 1) & ~(kAlign - 1); }

struct Region {
    const void *host;
    size_t bytes;
    size_t offset;
};

// The default scratch: context-owned buffers grown on demand.
float *grow_partials(void *user, size_t bytes) {
    Ctx *ctx = (Ctx *)user;
    if (ensure_buffer(ctx, ctx->partials, bytes, false) != kOk) {
        return nullptr;
    }
    return (float *)ctx->partials.ptr;
}
void *grow_rope(void *user, size_t bytes) {
    Ctx *ctx = (Ctx *)user;
    if (ensure_buffer(ctx, ctx->rope_scratch, bytes, false) != kOk) {
        return nullptr;
    }
    return ctx->rope_scratch.ptr;
}

// One launch of the decode kernels over up to kMetaPerLaunch sequences, each
// contributing the row `row0` at cache length `ctx`.
int32_t run_decode_pack(Ctx *ctx, const AttnLaunch &a, const std::vector<SeqMeta> &pack,
                        const AttnScratch &scratch) {
    DecodePlanInput plan{ctx->num_cus, scratch.partials, scratch.user};
    const hipError_t e = launch_attn_decode(ctx->stream, a, pack.data(), (int)pack.size(), plan);
    if (e != hipSuccess) {
        // out of memory: the scratch could not be had (its provider set the text)
        return e == hipErrorOutOfMemory ? kNoMemory : hip_fail(ctx, e, "decode attention launch");
    }
    return kOk;
}

// The first pack launched carries the call's inline page-table entries
// (AttnLaunch::tbl_*); they are cleared once a launch has taken them.
int32_t run_verify_pack(Ctx *ctx, AttnLaunch &a, const std::vector<SeqMeta> &pack,
                        const AttnScratch &scratch, void *rope) {
    DecodePlanInput plan{ctx->num_cus, scratch.partials, scratch.user};
    const hipError_t e =
        launch_attn_verify(ctx->stream, a, pack.data(), (int)pack.size(), rope, plan);
    a.tbl_n = 0;
    if (e != hipSuccess) {
        return e == hipErrorOutOfMemory ? kNoMemory : hip_fail(ctx, e, "verify attention launch");
    }
    return kOk;
}

// Sends the call's page-table entries again when the call returns an error.
// kv_prepare_append has already changed the host page lists (fresh pages, a
// private copy of a shared partial page); an entry that was to travel in the
// arguments of the call's first append kernel never reaches the device if
// the call fails before that launch, and the next append into the copied
// page would then write into the page a forked sequence still holds.
// Writing an entry that did arrive again is harmless.
struct TableGuard {
    Ctx *ctx;
    safetyraise_kernel_kv_pool *pool;
    TableBatch &batch;
    bool armed = true;
    ~TableGuard() {
        if (!armed || batch.idx.empty()) return;
        const std::string saved = ctx->error;  // keep the call's own message
        (void)kv_flush_table(ctx, pool, batch);
        ctx->error = saved;
    }
};

int32_t run_prefill_pack(Ctx *ctx, AttnLaunch &a, const std::vector<SeqMeta> &pack, void *rope) {
    const hipError_t e = launch_attn_prefill(ctx->stream, a, pack.data(), (int)pack.size(), rope);
    a.tbl_n = 0;
    if (e != hipSuccess) return hip_fail(ctx, e, "prefill attention launch");
    return kOk;
}

// A call at a head width the tuned kernels are not built for: every row of
// every sequence through the generic kernels (append all rows, then attend).
// Ends the call as the routed path below does: lengths advanced, the output
// copied back for host pointers, and on a synchronous error the lengths of
// every sequence restored.
int32_t generic_forward(Ctx *ctx, const safetyraise_kernel_attention_args &A, AttnLaunch &L,
                        const std::vector<uint64_t> &row0, bool device, bool async,
                        size_t out_bytes) {
    auto *pool = A.kv;
    std::vector<float> denom(A.rotary_dim / 2);
    for (uint32_t i = 0; i < A.rotary_dim / 2; ++i) {
        denom[i] = rope_denominator(A.rope_theta, i, A.rotary_dim);
    }
    L.rope_denom = denom.data();
    std::vector<uint64_t> old_len(A.num_seqs);
    TableBatch batch;
    for (uint32_t i = 0; i < A.num_seqs; ++i) {
        old_len[i] = pool->seqs[A.seq_ids[i]].len;
        int32_t st = kv_prepare_append(ctx, pool, A.seq_ids[i], A.seq_rows[i], &batch);
        if (st != kOk) {
            kv_flush_table(ctx, pool, batch);
            return st;
        }
    }
    TableGuard table_guard{ctx, pool, batch};
    int32_t st = kv_flush_table(ctx, pool, batch);
    if (st != kOk) return st;
    std::vector<SeqMeta> seqs(A.num_seqs);
    for (uint32_t i = 0; i < A.num_seqs; ++i) {
        SeqMeta m{};
        m.slot = A.seq_ids[i];
        m.ctx = (uint32_t)old_len[i];
        m.rows = A.seq_rows[i];
        m.row0 = (uint32_t)row0[i];
        seqs[i] = m;
    }
    const hipError_t e = launch_attn_generic(ctx->stream, L, seqs.data(), (int)seqs.size());
    if (e != hipSuccess) return hip_fail(ctx, e, "generic attention launch");
    for (uint32_t i = 0; i < A.num_seqs; ++i) {
        pool->seqs[A.seq_ids[i]].len = old_len[i] + A.seq_rows[i];
    }
    if (!device) {
        SR_HIP(ctx, hipMemcpyAsync(A.out, L.out, out_bytes, hipMemcpyDeviceToHost, ctx->stream));
    }
    table_guard.armed = false;
    st = finish_call(ctx, async);
    if (st != kOk && !async) {
        for (uint32_t i = 0; i < A.num_seqs; ++i) {
            pool->seqs[A.seq_ids[i]].len = old_len[i];
        }
    }
    return st;
}

}  // namespace

int32_t attention_forward_impl(Ctx *ctx, const safetyraise_kernel_attention_args *args,
                               const AttnScratch &scratch) {
    if (args == nullptr || args->struct_size < sizeof(safetyraise_kernel_attention_args)) {
        return fail(ctx, kInvalid, "attention args pointer or struct_size is invalid");
    }
    const auto &A = *args;
    auto *pool = A.kv;
    const uint32_t flags = A.flags;
    const bool device = (flags & SAFETYRAISE_MI355X_DEVICE_POINTERS) != 0;
    const bool async = (flags & SAFETYRAISE_MI355X_ASYNC) != 0;
    const bool bf16 = (flags & SAFETYRAISE_MI355X_INPUT_BF16) != 0;
    const bool gated = (flags & SAFETYRAISE_MI355X_GATED) != 0;
    const bool qk_norm = (flags & SAFETYRAISE_MI355X_QK_NORM) != 0;
    if (pool == nullptr) return fail(ctx, kInvalid, "attention needs a KV pool");
    if (async && !device) return fail(ctx, kInvalid, "ASYNC needs DEVICE_POINTERS");
    // causal_attention geometry (math.rs:109-124)
    if (A.heads == 0 || A.kv_heads == 0 || A.head_dim == 0 || A.heads % A.kv_heads != 0 ||
        A.kv_heads != pool->kv_heads || A.head_dim != pool->head_dim) {
        return fail(ctx, kInvalid, "attention head mapping or cache geometry is invalid");
    }
    // apply_rope shape (math.rs:58-65)
    if (A.rotary_dim == 0 || A.rotary_dim > A.head_dim || A.rotary_dim % 2 != 0) {
        return fail(ctx, kInvalid, "RoPE input shape is invalid");
    }
    if (!(A.rope_theta > 0.0f) || !std::isfinite(A.rope_theta)) {
        return fail(ctx, kInvalid, "RoPE theta must be finite and positive");
    }
    if (qk_norm && (!std::isfinite(A.eps) || A.eps <= 0.0f)) {
        return fail(ctx, kInvalid, "RMSNorm shape or epsilon is invalid");
    }
    if (A.num_seqs == 0 || A.num_seqs > SAFETYRAISE_MI355X_MAX_BATCH || A.seq_ids == nullptr ||
        A.seq_rows == nullptr) {
        return fail(ctx, kInvalid, "attention batch is empty or too large");
    }
    if (A.q == nullptr || A.k == nullptr || A.v == nullptr || A.positions == nullptr ||
        A.out == nullptr || (qk_norm && (A.q_norm == nullptr || A.k_norm == nullptr))) {
        return fail(ctx, kInvalid, "attention input or output pointer is NULL");
    }
    uint64_t total_rows = 0;
    std::vector<uint64_t> row0(A.num_seqs);
    for (uint32_t i = 0; i < A.num_seqs; ++i) {
        const uint32_t id = A.seq_ids[i];
        if (id >= pool->max_sequences || !pool->seqs[id].open) {
            return fail(ctx, kInvalid, "KV sequence handle is not open");
        }
        for (uint32_t j = 0; j < i; ++j) {
            if (A.seq_ids[j] == id) return fail(ctx, kInvalid, "a sequence appears twice in one call");
        }
        if (A.seq_rows[i] == 0) return fail(ctx, kInvalid, "input is empty");  // ensure_room
        if (pool->seqs[id].len + A.seq_rows[i] > pool->max_tokens) {
            return fail(ctx, kInvalid, "KV write would exceed the sequence capacity");
        }
        row0[i] = total_rows;
        total_rows += A.seq_rows[i];
    }
    if (total_rows > INT32_MAX) return fail(ctx, kOverflow, "too many rows");
    if (!async) {
        // errors of earlier ASYNC work are reported before this call changes
        // anything, so the error word it reads at its end is its own
        const int32_t st = report_pending_async(ctx);
        if (st != kOk) return st;
    }

    const size_t esz = bf16 ? 2 : 4;
    const size_t hs = (size_t)A.head_dim * (gated ? 2 : 1);
    const size_t q_bytes = total_rows * A.heads * hs * esz;
    const size_t kv_bytes = total_rows * A.kv_heads * A.head_dim * esz;
    const size_t pos_bytes = total_rows * 3 * sizeof(int32_t);
    const size_t norm_bytes = (size_t)A.head_dim * sizeof(float);
    const size_t out_bytes = total_rows * A.heads * A.head_dim * sizeof(float);

    AttnLaunch L{};
    L.pool = pool;
    L.flags = flags;
    L.heads = A.heads;
    L.kv_heads = A.kv_heads;
    // The kernels take up to 8 query heads per KV head.  A larger group G
    // runs as kv_rep groups of G / kv_rep heads (the fewest that fit): query
    // heads are numbered KV head by KV head, so group j of cache head c holds
    // heads (c kv_rep + j) G / kv_rep onwards and reads c's cache, the KV
    // head h / G that math.rs:127 gives query head h.
    const uint32_t group = A.heads / A.kv_heads;
    L.kv_rep = 1;
    while (group / L.kv_rep > 8 || group % L.kv_rep != 0) ++L.kv_rep;
    L.head_dim = A.head_dim;
    L.rotary_dim = A.rotary_dim;
    L.eps = A.eps;
    std::memcpy(L.mrope, A.mrope_section, sizeof L.mrope);
    L.err_word = ctx->d_error_word;
    L.rope = &rope_table(ctx, A.rope_theta, A.rotary_dim);
    L.q = A.q;
    L.k = A.k;
    L.v = A.v;
    L.q_norm = A.q_norm;
    L.k_norm = A.k_norm;
    L.positions = A.positions;
    L.out = A.out;
    if (device) {
        if (((uintptr_t)A.q | (uintptr_t)A.k | (uintptr_t)A.v | (uintptr_t)A.out) & 15u) {
            return fail(ctx, kInvalid, "device pointers must be 16-byte aligned");
        }
    } else {
        Region regions[6] = {{A.q, q_bytes, 0},         {A.k, kv_bytes, 0},
                             {A.v, kv_bytes, 0},        {A.positions, pos_bytes, 0},
                             {A.q_norm, norm_bytes, 0}, {A.k_norm, norm_bytes, 0}};
        size_t off = 0;
        for (auto &r : regions) {
            r.offset = off;
            off += align_up(r.bytes);
        }
        const size_t out_off = off;
        off += align_up(out_bytes);
        int32_t st = ensure_buffer(ctx, ctx->staging, off, false);
        if (st != kOk) return st;
        char *base = (char *)ctx->staging.ptr;
        for (auto &r : regions) {
            if (r.host != nullptr && r.bytes != 0) {
                SR_HIP(ctx, hipMemcpyAsync(base + r.offset, r.host, r.bytes, hipMemcpyHostToDevice,
                                           ctx->stream));
            }
        }
        L.q = base + regions[0].offset;
        L.k = base + regions[1].offset;
        L.v = base + regions[2].offset;
        L.positions = (const int32_t *)(base + regions[3].offset);
        L.q_norm = qk_norm ? (const float *)(base + regions[4].offset) : nullptr;
        L.k_norm = qk_norm ? (const float *)(base + regions[5].offset) : nullptr;
        L.out = (float *)(base + out_off);
    }

    if (generic_head_dim(A.head_dim)) {
        return generic_forward(ctx, A, L, row0, device, async, out_bytes);
    }

    // Routing (below): 16+ rows -> prefill, 2..15 supported rows -> verify,
    // the rest -> row-serial decode.  When no row takes the decode path, the
    // call's page-table entries (if few) travel in the first append kernel's
    // arguments instead of a separate update launch.
    const bool prefill_ok = prefill_supported(L);
    bool any_serial_route = false, any_fast_route = false;
    for (uint32_t i = 0; i < A.num_seqs; ++i) {
        const uint32_t r = A.seq_rows[i];
        const bool fast = (r >= kPrefillMinRows && prefill_ok) ||
                          (r < kPrefillMinRows && verify_supported(L, r));
        any_serial_route = any_serial_route || !fast;
        any_fast_route = any_fast_route || fast;
    }
    std::vector<uint64_t> old_len(A.num_seqs);
    TableBatch batch;  // one page-table upload for the whole call
    for (uint32_t i = 0; i < A.num_seqs; ++i) {
        old_len[i] = pool->seqs[A.seq_ids[i]].len;
        int32_t st = kv_prepare_append(ctx, pool, A.seq_ids[i], A.seq_rows[i], &batch);
        if (st != kOk) {
            kv_flush_table(ctx, pool, batch);
            return st;
        }
    }
    TableGuard table_guard{ctx, pool, batch};
    if (!any_serial_route && batch.idx.size() <= kInlineTable) {
        L.tbl_idx = batch.idx.data();
        L.tbl_val = batch.val.data();
        L.tbl_n = (uint32_t)batch.idx.size();
    } else {
        int32_t st = kv_flush_table(ctx, pool, batch);
        if (st != kOk) return st;
    }

    // Sequences with at least kPrefillMinRows new rows take the chunked
    // prefill kernels: all their rows are appended, then every row attends
    // causally to the context plus the rows before it, in one launch pair.
    std::vector<uint8_t> serial(A.num_seqs, 1);
    uint32_t serial_rows = 0;
    bool any_prefill = false;
    // the per-row RoPE table of the verify and prefill kernels
    void *rope = nullptr;
    if (prefill_ok && any_fast_route) {
        rope = scratch.rope(scratch.user, prefill_rope_bytes(L, total_rows));
        if (rope == nullptr) return kNoMemory;
    }
    // Sequences with 2..15 rows (MTP verify drafts) take the multi-row
    // split-K kernel: every cached K/V tile is read once for all rows.
    {
        std::vector<SeqMeta> pack;
        for (uint32_t i = 0; i < A.num_seqs; ++i) {
            if (A.seq_rows[i] >= kPrefillMinRows || !verify_supported(L, A.seq_rows[i])) continue;
            serial[i] = 0;
            any_prefill = true;
            SeqMeta m{};
            m.slot = A.seq_ids[i];
            m.ctx = (uint32_t)old_len[i];
            m.rows = A.seq_rows[i];
            m.row0 = (uint32_t)row0[i];
            pack.push_back(m);
            if (pack.size() == (size_t)kMetaPerLaunch) {
                int32_t st = run_verify_pack(ctx, L, pack, scratch, rope);
                if (st != kOk) return st;
                pack.clear();
            }
        }
        if (!pack.empty()) {
            int32_t st = run_verify_pack(ctx, L, pack, scratch, rope);
            if (st != kOk) return st;
        }
    }
    {
        std::vector<SeqMeta> pack;
        for (uint32_t i = 0; i < A.num_seqs; ++i) {
            if (!serial[i]) continue;
            if (!prefill_ok || A.seq_rows[i] < kPrefillMinRows) {
                serial_rows = std::max(serial_rows, A.seq_rows[i]);
                continue;
            }
            serial[i] = 0;
            any_prefill = true;
            SeqMeta m{};
            m.slot = A.seq_ids[i];
            m.ctx = (uint32_t)old_len[i];
            m.rows = A.seq_rows[i];
            m.row0 = (uint32_t)row0[i];
            pack.push_back(m);
            if (pack.size() == (size_t)kMetaPerLaunch) {
                int32_t st = run_prefill_pack(ctx, L, pack, rope);
                if (st != kOk) return st;
                pack.clear();
            }
        }
        if (!pack.empty()) {
            int32_t st = run_prefill_pack(ctx, L, pack, rope);
            if (st != kOk) return st;
        }
    }

    // Row r of every selected sequence with more than r rows: one decode step
    // each, in row order, so row r sees the context plus rows 0..r (the
    // reference appends then attends row by row, native.rs:637-638).
    auto run_serial = [&](const std::vector<uint8_t> &which) -> int32_t {
        uint32_t nrows = 0;
        for (uint32_t i = 0; i < A.num_seqs; ++i) {
            if (which[i]) nrows = std::max(nrows, A.seq_rows[i]);
        }
        for (uint32_t r = 0; r < nrows; ++r) {
            std::vector<SeqMeta> pack;
            uint64_t pack_tokens = 0;
            for (uint32_t i = 0; i < A.num_seqs; ++i) {
                if (!which[i] || A.seq_rows[i] <= r) continue;
                SeqMeta m{};
                m.slot = A.seq_ids[i];
                m.ctx = (uint32_t)(old_len[i] + r);
                m.rows = 1;
                m.row0 = (uint32_t)(row0[i] + r);
                if (!pack.empty() && pack_tokens + m.ctx + 1 > 0x7fffffffull) {
                    int32_t st = run_decode_pack(ctx, L, pack, scratch);
                    if (st != kOk) return st;
                    pack.clear();
                    pack_tokens = 0;
                }
                pack.push_back(m);
                pack_tokens += (uint64_t)m.ctx + 1;
                if (pack.size() == (size_t)kMetaPerLaunch) {
                    int32_t st = run_decode_pack(ctx, L, pack, scratch);
                    if (st != kOk) return st;
                    pack.clear();
                    pack_tokens = 0;
                }
            }
            if (!pack.empty()) {
                int32_t st = run_decode_pack(ctx, L, pack, scratch);
                if (st != kOk) return st;
            }
        }
        return kOk;
    };
    if (serial_rows > 0) {
        int32_t st = run_serial(serial);
        if (st != kOk) return st;
    }
    if (any_prefill && !async) {
        // A synchronous call can recompute prefill rows whose MFMA operands
        // left the fp16 range on the f32 split-K path (same cache positions,
        // same values appended again).
        uint32_t word = 0;
        int32_t st = take_error_word(ctx, &word);
        if (st == kOk && word == kErrPrefillRange) {
            std::vector<uint8_t> redo(A.num_seqs);
            for (uint32_t i = 0; i < A.num_seqs; ++i) redo[i] = serial[i] ? 0 : 1;
            st = run_serial(redo);
        } else if (st == kOk) {
            st = error_word_status(ctx, word);
        }
        if (st != kOk) return st;
    }
    for (uint32_t i = 0; i < A.num_seqs; ++i) {
        pool->seqs[A.seq_ids[i]].len = old_len[i] + A.seq_rows[i];
    }
    if (!device) {
        SR_HIP(ctx, hipMemcpyAsync(A.out, L.out, out_bytes, hipMemcpyDeviceToHost, ctx->stream));
    }
    table_guard.armed = false;  // every launch went out: the entries are on the device
    int32_t st = finish_call(ctx, async);
    if (st != kOk && !async) {
        for (uint32_t i = 0; i < A.num_seqs; ++i) {
            pool->seqs[A.seq_ids[i]].len = old_len[i];
        }
    }
    return st;
}

}  // namespace sr

using namespace sr;

extern "C" SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_attention_forward(
    safetyraise_kernel_context *context, const safetyraise_kernel_attention_args *args) {
    if (context == nullptr) return kInvalid;
    const int32_t capture = refuse_under_capture(context, "attention_forward");
    if (capture != kOk) return capture;
    TimerScope timer_scope(context);
    const AttnScratch scratch{grow_partials, grow_rope, context};
    return attention_forward_impl(context, args, scratch);
}
