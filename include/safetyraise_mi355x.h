/*
 * MI355X (gfx950) attention / gated-delta-net extension to the rsinfer
 * plugin ABI v1.
 *
 * Everything here is optional for the engine's v1 loader: the loader resolves
 * only the nine v1 symbols (src/backend/mod.rs:553-575), so the library stays
 * a drop-in plugin.  A caller that wants the attention and GDN hot path reads
 * capabilities.flags (plugin-defined, reference header :73) and resolves the
 * symbols below with dlsym.
 *
 * The entry points replace the engine's in-process calls:
 *   - safetyraise_kernel_kv_*            PagedKvCache (src/engine/state.rs:19-127)
 *                                        plus SequenceState::checkpoint (:222-224)
 *   - safetyraise_kernel_attention_forward
 *                                        the Attention::forward row loop
 *                                        (src/model/native.rs:615-645): QK-RMSNorm,
 *                                        RoPE, KV append, causal_attention
 *                                        (src/model/math.rs:102-155), output gate
 *   - safetyraise_kernel_gdn_*           RecurrentState (src/engine/state.rs:129-135)
 *                                        and the Gdn::forward row loop
 *                                        (src/model/native.rs:720-742):
 *                                        causal_conv_silu, gated_delta_step,
 *                                        per-head RMSNorm, silu(z) gate
 *
 * Conventions are those of ABI v1: status codes from safetyraise_kernel_status,
 * text from safetyraise_kernel_last_error, calls on one context are serial.
 * Every args/options struct starts with struct_size so tail fields can be
 * added; the plugin rejects a struct_size smaller than the one it knows.
 *
 * Pointers are host memory unless SAFETYRAISE_MI355X_DEVICE_POINTERS is set,
 * in which case every tensor pointer of the call is a device address on the
 * context's GPU.  Calls return with results complete unless
 * SAFETYRAISE_MI355X_ASYNC is set (device pointers only): the work is then
 * enqueued on the context stream, and errors the kernels detect (non-finite
 * K/V or norm variance, as the reference rejects them) are reported by the
 * next synchronous attention or GDN call, before that call changes anything,
 * or by safetyraise_kernel_synchronize.  The asynchronous call has already
 * advanced its sequences by then: to repeat it, kv_truncate them to their
 * earlier lengths first.
 */
#ifndef SAFETYRAISE_MI355X_H
#define SAFETYRAISE_MI355X_H

#include "safetyraise_kernel.h"

#ifdef __cplusplus
extern "C" {
#endif

/* capabilities.flags bits reported by this plugin. */
#define SAFETYRAISE_MI355X_CAP_ATTENTION UINT32_C(0x1)    /* kv_* and attention_forward */
#define SAFETYRAISE_MI355X_CAP_GDN UINT32_C(0x2)          /* gdn_* */
#define SAFETYRAISE_MI355X_CAP_DEVICE_STATE UINT32_C(0x4) /* state lives in HBM, O(1) fork */

/* Per-call flags. */
#define SAFETYRAISE_MI355X_DEVICE_POINTERS UINT32_C(0x1)
#define SAFETYRAISE_MI355X_ASYNC UINT32_C(0x2)
#define SAFETYRAISE_MI355X_INPUT_BF16 UINT32_C(0x4)  /* q/k/v (gate, qkv, z, a, b) are bf16 */
#define SAFETYRAISE_MI355X_QK_NORM UINT32_C(0x8)     /* per-head RMSNorm of q and k */
#define SAFETYRAISE_MI355X_NORM_OFFSET UINT32_C(0x10) /* weight + 1 (Qwen3.5 norms) */
#define SAFETYRAISE_MI355X_GATED UINT32_C(0x20)      /* q rows are per-head [q, gate] */
#define SAFETYRAISE_MI355X_MROPE_INTERLEAVED UINT32_C(0x40)
#define SAFETYRAISE_MI355X_KEEP_ROWS UINT32_C(0x80) /* gdn_forward: allow gdn_rollback */

/* Largest number of sequences one call may carry. */
#define SAFETYRAISE_MI355X_MAX_BATCH 1024u

/* ------------------------------------------------------------------------
 * Context helpers (no counterpart in the reference: the v1 calls are
 * synchronous, these let a device-resident caller order work itself).
 * ---------------------------------------------------------------------- */

/* Sets the HIP stream (a hipStream_t, NULL = the context's own stream) on
 * which the context enqueues all later work. */
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_set_stream(
    safetyraise_kernel_context *context, void *hip_stream);

/* Waits for the context stream and reports errors detected by kernels of
 * earlier SAFETYRAISE_MI355X_ASYNC calls (then clears them). */
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_synchronize(
    safetyraise_kernel_context *context);

/* Kernel timing, for benchmarks (no counterpart in the reference).
 * enable != 0 waits for the context stream, clears earlier records and makes
 * every later kernel launch of this context record its device start and end
 * (the timestamps of the dispatch packet, as a profiler's kernel trace sees
 * them); enable == 0 stops and frees the records.  Recording costs one event
 * pair per launch, so timed calls are not the fastest.  A window (from one
 * enable to the next) records at most 65536 launches; later launches run
 * untimed, so a long run calls enable again to start a new window. */
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_timing_enable(
    safetyraise_kernel_context *context, uint32_t enable);
/* Waits for the context stream, then reports the index-th distinct kernel
 * name recorded (in order of first launch): the name (static storage), its
 * launches and their summed device milliseconds.  INVALID_ARGUMENT past the
 * last name. */
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_timing_read(
    safetyraise_kernel_context *context, uint32_t index, const char **out_name,
    uint64_t *out_launches, double *out_total_ms);

/* ------------------------------------------------------------------------
 * Paged bf16 KV cache — replaces PagedKvCache (src/engine/state.rs:19-127).
 *
 * A pool owns num_pages pages of K and of V in HBM.  One page holds
 * page_tokens tokens of every KV head in bf16; the pool is head-major,
 * [kv_head][page][token][head_dim], so a sequence whose pages are adjacent
 * is one contiguous stream per head.  A sequence is a slot holding a page list;
 * pages are reference counted so kv_fork is O(pages) host work and no device
 * copy (the snapshot shares every page; the first append into a shared,
 * partly filled page copies that page, as Arc::make_mut does at state.rs:70).
 * ---------------------------------------------------------------------- */
typedef struct safetyraise_kernel_kv_pool safetyraise_kernel_kv_pool;

typedef struct safetyraise_kernel_kv_options {
    uint32_t struct_size;   /* sizeof(safetyraise_kernel_kv_options) */
    uint32_t kv_heads;
    uint32_t head_dim;      /* 1..512 (64, 128 and 256 take the tuned kernels) */
    uint32_t page_tokens;   /* power of two >= 16 (reference: 64, state.rs:167) */
    uint64_t num_pages;     /* pages in the pool */
    uint64_t max_tokens;    /* per-sequence capacity (max_context) */
    uint32_t max_sequences; /* sequence slots */
    /* 0: pages are handed out in pool order (a sequence appended alone gets
     * adjacent pages).  Otherwise the free list starts as a random
     * permutation of the pool drawn from this seed, so every sequence's pages
     * are scattered over the pool, as in a long-running server's cache. */
    uint32_t page_order_seed;
} safetyraise_kernel_kv_options;

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_kv_create(
    safetyraise_kernel_context *context, const safetyraise_kernel_kv_options *options,
    safetyraise_kernel_kv_pool **out_pool);
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_kv_destroy(
    safetyraise_kernel_context *context, safetyraise_kernel_kv_pool *pool);

/* New empty sequence (PagedKvCache::new, state.rs:28-40). */
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_kv_open(
    safetyraise_kernel_context *context, safetyraise_kernel_kv_pool *pool,
    uint32_t *out_sequence);
/* Snapshot sharing every page (clone for SequenceState::checkpoint). */
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_kv_fork(
    safetyraise_kernel_context *context, safetyraise_kernel_kv_pool *pool,
    uint32_t source, uint32_t *out_sequence);
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_kv_close(
    safetyraise_kernel_context *context, safetyraise_kernel_kv_pool *pool, uint32_t sequence);
/* PagedKvCache::truncate (state.rs:99-119): len > current length is an error. */
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_kv_truncate(
    safetyraise_kernel_context *context, safetyraise_kernel_kv_pool *pool, uint32_t sequence,
    uint64_t len);
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_kv_len(
    safetyraise_kernel_context *context, safetyraise_kernel_kv_pool *pool, uint32_t sequence,
    uint64_t *out_len);
/* Appends tokens rows of already-normalised keys and values, each row
 * [kv_heads*head_dim] (PagedKvCache::append, state.rs:52-84, repeated).
 * Values are rounded to bf16 (round to nearest even) unless INPUT_BF16. */
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_kv_append(
    safetyraise_kernel_context *context, safetyraise_kernel_kv_pool *pool, uint32_t sequence,
    const void *keys, const void *values, uint64_t tokens, uint32_t flags);
/* Reads tokens rows starting at start as f32 [tokens][kv_heads*head_dim],
 * the layout of PagedKvCache::get (state.rs:86-96).  Host pointers. */
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_kv_read(
    safetyraise_kernel_context *context, safetyraise_kernel_kv_pool *pool, uint32_t sequence,
    uint64_t start, uint64_t tokens, float *keys, float *values);

/* ------------------------------------------------------------------------
 * Attention — replaces the per-row loop of Attention::forward
 * (src/model/native.rs:615-645) for a batch of sequences.
 *
 * Sequence i contributes seq_rows[i] consecutive rows (its new tokens, in
 * order).  For each row r at position p:
 *   q, k  = RMSNorm per head (if QK_NORM; weight+1 if NORM_OFFSET), then RoPE
 *           (rotate-half over the first rotary_dim dims, angle =
 *           p / theta^(2i/rotary_dim) in f32, MRoPE axes by mrope_section);
 *   append (k, v) to the sequence's cache, stored in bf16;
 *   out   = causal attention of q over every cached token, which is the
 *           context plus rows 0..r of this call (row r sees len+r+1 keys);
 *   out  *= sigmoid(gate) if GATED.
 * Inputs:  q [rows][heads*head_dim] (GATED: [rows][heads][2*head_dim] with the
 *          gate in the second half of each head), k and v
 *          [rows][kv_heads*head_dim], f32 or bf16 (INPUT_BF16);
 *          q_norm, k_norm [head_dim] f32 (QK_NORM only);
 *          positions [rows][3] int32 (the three MRoPE axes; text uses p,p,p).
 * Output:  out [rows][heads*head_dim] f32.
 * seq_ids and seq_rows are always host arrays.  The kernel is chosen per
 * sequence: one row goes to the split-K decode kernel; 2..15 rows (MTP
 * verify drafts) to the multi-row split-K verify kernel (every cached K/V
 * tile read once for up to 128 query vectors, rows * heads/kv_heads, at
 * head_dim <= 128 and 64 at head_dim 256; more rows run as row slices, each
 * reading the cache once); 16 or more rows to the MFMA prefill kernels.
 * Query-head groups other than 1..8 heads per KV head and RoPE widths not a
 * multiple of 32 go row by row to the decode kernel.  Head widths other than
 * 64, 128 and 256 (up to 512) take plain f32 kernels for every row: all rows
 * appended, then one wave per (row, query head) over the visible keys.  A synchronous call whose verify or prefill rows
 * meet a K/V/q value beyond the fp16 range of the MFMA operands
 * (|x| >= 65520) recomputes those sequences on the f32 split-K path; an
 * asynchronous one reports it at the next synchronous call.
 * ---------------------------------------------------------------------- */
typedef struct safetyraise_kernel_attention_args {
    uint32_t struct_size;
    uint32_t flags;
    uint32_t heads;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t rotary_dim;
    float eps;
    float rope_theta;
    uint32_t mrope_section[3]; /* all zero = no MRoPE */
    uint32_t num_seqs;
    const uint32_t *seq_ids;
    const uint32_t *seq_rows;
    const void *q;
    const void *k;
    const void *v;
    const float *q_norm;
    const float *k_norm;
    const int32_t *positions;
    float *out;
    safetyraise_kernel_kv_pool *kv;
} safetyraise_kernel_attention_args;

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_attention_forward(
    safetyraise_kernel_context *context, const safetyraise_kernel_attention_args *args);

/* safetyraise_kernel_attention_forward that allocates no device memory.  No
 * counterpart in the reference: it is for callers that cannot allocate
 * (tight serving loops, harnesses that forbid hipMalloc).  Same arguments,
 * kernels and results; DEVICE_POINTERS is required.  The call's scratch
 * (split-K partial records, the per-row RoPE table) comes from a fixed
 * 64 MiB device region per GPU.  The region is a static device array of the
 * library's code object, so every process that loads the library reserves
 * it on a GPU when the library's code is first loaded there (its first
 * kernel launch on that GPU), whether or not it calls this entry point, and
 * holds it until the process ends.  A call that needs more fails with
 * OUT_OF_MEMORY and its sequences keep their lengths.  Every call on one GPU
 * shares that region, so calls that overlap on one GPU (other threads,
 * contexts or streams) race; calls on one context are serial anyway.
 *
 * Neither attention entry point can be captured into a HIP graph: a call
 * appends at the sequences' current lengths and advances those lengths and
 * the page lists on the host when it is made, so a replay would rewrite the
 * same cache positions and never advance them.  Both return INVALID_ARGUMENT
 * while the context's stream is capturing. */
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_attention_forward_noalloc(
    safetyraise_kernel_context *context, const safetyraise_kernel_attention_args *args);

/* ------------------------------------------------------------------------
 * Gated delta net — replaces RecurrentState (src/engine/state.rs:129-135)
 * and the per-row loop of Gdn::forward (src/model/native.rs:720-742).
 *
 * A pool holds, per sequence slot, the f32 state [Hv][Dv][Dk] and the
 * causal-conv history of C = 2*Hk*Dk + Hv*Dv channels.
 * ---------------------------------------------------------------------- */
typedef struct safetyraise_kernel_gdn_pool safetyraise_kernel_gdn_pool;

typedef struct safetyraise_kernel_gdn_options {
    uint32_t struct_size;
    uint32_t key_heads;
    uint32_t value_heads;
    uint32_t key_dim;   /* 1..512 (128 takes the tuned kernels) */
    uint32_t value_dim; /* 1..512 (128, or a multiple of 16 at key_dim 128, tuned) */
    uint32_t conv_kernel;
    uint32_t max_sequences;
    /* 0, or the most rows per sequence a KEEP_ROWS call may carry (<= 64; at
     * key_dim 128 with value_dim a multiple of 16, value_dim must be 128):
     * every sequence then has two state buffers, so that gdn_rollback can
     * return it to the state after any row of such a call. */
    uint32_t keep_rows;
} safetyraise_kernel_gdn_options;

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_gdn_create(
    safetyraise_kernel_context *context, const safetyraise_kernel_gdn_options *options,
    safetyraise_kernel_gdn_pool **out_pool);
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_gdn_destroy(
    safetyraise_kernel_context *context, safetyraise_kernel_gdn_pool *pool);
/* New sequence with zero state and history (state.rs:167-180). */
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_gdn_open(
    safetyraise_kernel_context *context, safetyraise_kernel_gdn_pool *pool,
    uint32_t *out_sequence);
/* Copy of a sequence's state (SequenceState::checkpoint). */
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_gdn_fork(
    safetyraise_kernel_context *context, safetyraise_kernel_gdn_pool *pool, uint32_t source,
    uint32_t *out_sequence);
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_gdn_close(
    safetyraise_kernel_context *context, safetyraise_kernel_gdn_pool *pool, uint32_t sequence);
/* State in the reference layouts: matrix [Hv][Dv][Dk], history [C][K-1]
 * oldest first.  Host pointers. */
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_gdn_read(
    safetyraise_kernel_context *context, safetyraise_kernel_gdn_pool *pool, uint32_t sequence,
    float *matrix, float *history);
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_gdn_write(
    safetyraise_kernel_context *context, safetyraise_kernel_gdn_pool *pool, uint32_t sequence,
    const float *matrix, const float *history);

/* Commit of an MTP verify without re-running it.  Replaces the re-forward of
 * the committed tokens in decode_round (src/engine/speculative.rs:242-247)
 * for the recurrent layers; attention layers use kv_truncate.
 * After a gdn_forward call with SAFETYRAISE_MI355X_KEEP_ROWS (on a pool
 * created with keep_rows), returns the sequence's state and conv history to
 * what they were after its first `rows` rows of that call (0: before the
 * call; the call's own row count: unchanged).  The state is rebuilt from the
 * pre-call buffer, which the KEEP_ROWS call only read, and the per-row decay,
 * correction and key that call recorded: one state read and one write, with
 * the element-wise operations of the forward.  Allowed until the sequence's
 * next gdn_forward or gdn_write; repeated calls rebuild from the same
 * pre-call state.  flags: SAFETYRAISE_MI355X_ASYNC or 0. */
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_gdn_rollback(
    safetyraise_kernel_context *context, safetyraise_kernel_gdn_pool *pool, uint32_t sequence,
    uint32_t rows, uint32_t flags);

/* For each sequence's rows, in order (src/model/native.rs:720-742):
 *   x    = silu(causal conv over qkv with the history), history shifted;
 *   o    = gated_delta_step(x, a, b, A_log, dt_bias) on the state;
 *   out  = RMSNorm(o per value head, norm, eps, no offset) * silu(z).
 * Inputs: qkv [rows][C], z [rows][Hv*Dv], a and b [rows][Hv] (f32, or bf16
 * with INPUT_BF16); a_log, dt_bias [Hv], conv_weight [C][K], norm [Dv] f32.
 * Output: out [rows][Hv*Dv] f32.
 * KEEP_ROWS calls (see gdn_rollback), and calls with at most 8 rows per
 * sequence, run the recurrence token by token
 * (one workgroup per sequence and value head, state in registers); longer
 * calls with value_dim 128 and a 16-byte aligned qkv run the chunked (WY)
 * form in chunks of 32 rows (f32 MFMA), which equals the token-serial
 * result within the f32 tolerance.  The chunked form keeps 68 KB of device
 * scratch per (32-row chunk, value head) of the call in the context's
 * staging buffer (e.g. 280 MB for 4096 rows at 32 value heads), grown on
 * demand: OUT_OF_MEMORY when it cannot be.  Other key widths, and value
 * widths that are not a multiple of 16, run token by token in one workgroup
 * per (sequence, value head) with the state rows in HBM (a wave per row). */
typedef struct safetyraise_kernel_gdn_args {
    uint32_t struct_size;
    uint32_t flags;
    float eps;
    uint32_t num_seqs;
    const uint32_t *seq_ids;
    const uint32_t *seq_rows;
    const void *qkv;
    const void *z;
    const void *a;
    const void *b;
    const float *a_log;
    const float *dt_bias;
    const float *conv_weight;
    const float *norm;
    float *out;
    safetyraise_kernel_gdn_pool *state;
} safetyraise_kernel_gdn_args;

SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_gdn_forward(
    safetyraise_kernel_context *context, const safetyraise_kernel_gdn_args *args);

/* ABI v1 linear (safetyraise_kernel_linear, reference header :115-123) with
 * device pointers: input [rows][cols] and output [rows][out_cols] f32 in
 * device memory, queued on the context's stream and not waited for.  The
 * same shape checks as linear (status 1); the input is not scanned for
 * non-finite values (linear does that on the host, native/cpu/
 * safetyraise_cpu.c:221-226): non-finite inputs give non-finite outputs.
 * The weight is any handle from create_weight (dtype F32, F16 or BF16). */
SAFETYRAISE_KERNEL_EXPORT int32_t safetyraise_kernel_linear_device(
    safetyraise_kernel_context *context, safetyraise_kernel_weight *weight, const float *input,
    uint64_t input_rows, uint64_t input_cols, float *output, uint64_t output_rows,
    uint64_t output_cols);

#ifdef __cplusplus
}
#endif

#endif /* SAFETYRAISE_MI355X_H */
