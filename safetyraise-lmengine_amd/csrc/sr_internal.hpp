// Internal declarations shared by the plugin's host code and kernel launchers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "safetyraise_mi355x.h"

namespace sr {

constexpr int32_t kOk = SAFETYRAISE_KERNEL_STATUS_OK;
constexpr int32_t kInvalid = SAFETYRAISE_KERNEL_STATUS_INVALID_ARGUMENT;
constexpr int32_t kUnsupportedDtype = SAFETYRAISE_KERNEL_STATUS_UNSUPPORTED_DTYPE;
constexpr int32_t kOverflow = SAFETYRAISE_KERNEL_STATUS_DIMENSION_OVERFLOW;
constexpr int32_t kNoMemory = SAFETYRAISE_KERNEL_STATUS_OUT_OF_MEMORY;
constexpr int32_t kDeviceError = SAFETYRAISE_KERNEL_STATUS_DEVICE_ERROR;
constexpr int32_t kInternal = SAFETYRAISE_KERNEL_STATUS_INTERNAL_ERROR;
constexpr int32_t kAbiMismatch = SAFETYRAISE_KERNEL_STATUS_ABI_MISMATCH;

// Bits of the context's sticky device error word (set by kernels).
constexpr uint32_t kErrNonFiniteKv = 1u;        // PagedKvCache::append rejects (state.rs:56-58)
constexpr uint32_t kErrNonFiniteVariance = 2u;  // rms_norm rejects (math.rs:39-41)
constexpr size_t kErrorBlockBytes = 1024;  // error word + zero block (>= 256 floats)
// A prefill row's output is not finite: some K, V or q value is outside the fp16
// operand range of the MFMA prefill kernel; synchronous calls recompute on the
// f32 split-K path.
constexpr uint32_t kErrPrefillRange = 4u;

// Sequences per kernel launch whose metadata travels in the kernel arguments.
constexpr int kMetaPerLaunch = 64;
// Widest attention head the generic kernels take (head widths other than 64,
// 128 and 256; attn_generic.hip).
constexpr uint32_t kGenericMaxHeadDim = 512;
// Widest GDN key or value head the generic kernels take (gdn_kernels.hip).
constexpr uint32_t kGdnMaxDim = 512;

// Grow-only device allocation owned by a context.
struct DeviceBuffer {
    void *ptr = nullptr;
    size_t bytes = 0;
};

// Per-sequence launch metadata (kernel argument, by value).
struct SeqMeta {
    uint32_t slot;    // sequence slot in the pool (page-table row)
    uint32_t ctx;     // tokens cached before this call's rows
    uint32_t rows;    // new rows of this sequence in this launch
    uint32_t row0;    // first row index in the call's q/k/v/out/positions
    uint32_t split0;  // first global split index (decode kernel)
};

struct MetaPack {
    SeqMeta m[kMetaPerLaunch];
};

// Device durations of kernel launches, recorded on request
// (safetyraise_kernel_timing_enable) with the start/stop events of
// hipExtLaunchKernelGGL, i.e. the timestamps of the dispatch itself.  A
// launcher asks timed_launch(name) for the events of one launch; they are
// null (an ordinary launch) unless the calling thread is inside an entry
// point of a context whose timing is on (TimerScope).
struct KernelTimer {
    struct Record {
        const char *name;
        hipEvent_t start;
        hipEvent_t stop;
    };
    // launches recorded per window at most (one event pair each); later
    // launches of the window run untimed
    static constexpr size_t kMaxRecords = 65536;
    bool enabled = false;
    std::vector<Record> records;  // events are reused after timing_reset
    size_t used = 0;
};
struct LaunchEvents {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
};
LaunchEvents timed_launch(const char *kernel);

// RoPE denominators theta^(2i/rotary_dim) for i < rotary_dim/2, computed on
// the host with the C library powf in f32 exactly as math.rs:90-91 does.
struct RopeTable {
    float denom[128];
};

}  // namespace sr

struct safetyraise_kernel_context {
    int device = 0;
    int num_cus = 256;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    std::string error;
    uint32_t *d_error_word = nullptr;  // sticky kernel-detected errors
    bool async_pending = false;        // ASYNC work queued since the word was last read
    sr::DeviceBuffer staging;          // host-pointer mode device copies
    sr::DeviceBuffer partials;         // split-K partial (m, l, o) records
    sr::DeviceBuffer rope_scratch;     // prefill: per-row RoPE cos/sin
    sr::DeviceBuffer linear_in;        // linear: the host input's device copy
    sr::DeviceBuffer linear_out;       // linear: the output before it goes back
    sr::DeviceBuffer linear_part;      // linear: partial sums of calls that split K
    float rope_theta = 0.0f;
    uint32_t rope_dim = 0;
    sr::RopeTable rope{};
    sr::KernelTimer timer;
};

// A linear weight [rows][cols] in its own dtype (F32, F16 or BF16), on the
// device for the life of the handle: F32 and F16 row-major, BF16 in the 1 KB
// tiles of linear_pack_bf16.
struct safetyraise_kernel_weight {
    uint64_t rows = 0;
    uint64_t cols = 0;
    uint32_t dtype = 0;
    void *d_data = nullptr;
};

struct safetyraise_kernel_kv_pool {
    uint32_t kv_heads = 0;
    uint32_t head_dim = 0;
    uint32_t page_tokens = 0;
    uint64_t num_pages = 0;
    uint64_t max_tokens = 0;
    uint32_t max_sequences = 0;
    uint32_t pages_per_seq = 0;  // page-table row length
    // Head-major pool: [kv_heads][num_pages][page_tokens][head_dim] bf16, so
    // one head's pages are adjacent and a sequence on consecutive pages is
    // one contiguous stream per head.
    uint16_t *k_pages = nullptr;
    uint16_t *v_pages = nullptr;
    int32_t *d_page_table = nullptr;  // [max_sequences][pages_per_seq]
    struct Sequence {
        bool open = false;
        uint64_t len = 0;
        std::vector<int32_t> pages;
    };
    std::vector<Sequence> seqs;
    std::vector<uint32_t> refcount;
    std::vector<int32_t> free_pages;
    size_t page_elems() const { return (size_t)kv_heads * page_tokens * head_dim; }
    size_t head_page_elems() const { return (size_t)page_tokens * head_dim; }
    size_t head_stride() const { return (size_t)num_pages * page_tokens * head_dim; }
};

struct safetyraise_kernel_gdn_pool {
    uint32_t key_heads = 0;
    uint32_t value_heads = 0;
    uint32_t key_dim = 0;
    uint32_t value_dim = 0;
    uint32_t conv_kernel = 0;
    uint32_t max_sequences = 0;
    uint32_t channels = 0;
    // rows a KEEP_ROWS call may carry per sequence (0: no rollback); with it
    // every sequence has two state buffers and a record per row
    uint32_t keep_rows = 0;
    float *d_state = nullptr;    // [max_sequences][1 or 2][Hv][Dv][Dk]
    float *d_history = nullptr;  // [2][max_sequences][C][K-1], oldest first
    float *d_records = nullptr;  // [max_sequences][keep_rows][record_elems()]
    std::vector<uint8_t> open;
    std::vector<uint32_t> parity;     // which history buffer is current
    std::vector<uint32_t> state_par;  // which state buffer is current (keep_rows > 0)
    std::vector<uint32_t> kept;       // rows of the last KEEP_ROWS call, kNoKept if none since
    std::vector<uint32_t> kept_at;    // row of that call the current buffers hold
    static constexpr uint32_t kNoKept = 0xffffffffu;
    size_t state_elems() const { return (size_t)value_heads * value_dim * key_dim; }
    size_t history_elems() const { return (size_t)channels * (conv_kernel - 1); }
    uint32_t state_buffers() const { return keep_rows > 0 ? 2u : 1u; }
    // state buffer index of a sequence's current (which = 0) or other (1) buffer
    uint32_t state_index(uint32_t seq, uint32_t which) const {
        return seq * state_buffers() + (keep_rows > 0 ? (state_par[seq] ^ which) : 0u);
    }
    // alpha [Hv], delta [Hv][Dv], k^ [Hv][Dk], raw conv inputs [C]
    size_t record_elems() const {
        return (size_t)value_heads * (1 + value_dim + key_dim) + channels;
    }
};

namespace sr {

using Ctx = safetyraise_kernel_context;

int32_t fail(Ctx *ctx, int32_t status, const std::string &message);
int32_t hip_fail(Ctx *ctx, hipError_t err, const char *what);
#define SR_HIP(ctx, expr)                                    \
    do {                                                     \
        hipError_t _e = (expr);                              \
        if (_e != hipSuccess) return ::sr::hip_fail((ctx), _e, #expr); \
    } while (0)

// Makes ctx's kernel timer the calling thread's current one for the life of
// the scope (every entry point that launches kernels opens one).
class TimerScope {
  public:
    explicit TimerScope(Ctx *ctx);
    ~TimerScope();
    TimerScope(const TimerScope &) = delete;
    TimerScope &operator=(const TimerScope &) = delete;

  private:
    KernelTimer *prev_;
};

bool checked_mul(uint64_t a, uint64_t b, uint64_t *out);
int32_t ensure_buffer(Ctx *ctx, DeviceBuffer &buf, size_t bytes, bool zero);
int32_t finish_call(Ctx *ctx, bool async);  // sync + sticky error check unless async
// At the start of a synchronous call: waits for earlier ASYNC work, if any,
// and reports the errors its kernels raised (as the header promises), so
// that the error word the call reads at its end holds only its own bits.
// INVALID_ARGUMENT when the context's stream is capturing a HIP graph: the
// calls that advance host-side KV bookkeeping cannot be replayed.
int32_t refuse_under_capture(Ctx *ctx, const char *what);
int32_t report_pending_async(Ctx *ctx);
// Synchronises the context stream and returns the sticky error word, cleared.
int32_t take_error_word(Ctx *ctx, uint32_t *word);
// The status and message for a non-zero error word.
int32_t error_word_status(Ctx *ctx, uint32_t word);
const RopeTable &rope_table(Ctx *ctx, float theta, uint32_t rotary_dim);
// theta^(2i/rotary_dim) as math.rs:90-91 computes it (C library powf, f32)
float rope_denominator(float theta, uint32_t i, uint32_t rotary_dim);

// KV pool helpers used by attention.  Page-table entries changed by
// kv_prepare_append are queued in `batch` when it is given (and uploaded by
// kv_flush_table in one launch), else uploaded at once.
struct TableBatch {
    std::vector<uint32_t> idx;
    std::vector<int32_t> val;
};
int32_t kv_prepare_append(Ctx *ctx, safetyraise_kernel_kv_pool *pool, uint32_t seq, uint64_t n,
                          TableBatch *batch = nullptr);
int32_t kv_flush_table(Ctx *ctx, safetyraise_kernel_kv_pool *pool, TableBatch &batch);

// ---------------- kernel launchers (defined in the .hip files) ----------------
hipError_t launch_page_table_set(hipStream_t s, int32_t *table, const uint32_t *idx,
                                 const int32_t *val, int n);
hipError_t launch_kv_scatter(hipStream_t s, const safetyraise_kernel_kv_pool *pool, uint32_t slot,
                             uint64_t start, uint64_t tokens, const void *keys, const void *values,
                             bool bf16_in, uint32_t *err_word);
hipError_t launch_kv_gather(hipStream_t s, const safetyraise_kernel_kv_pool *pool, uint32_t slot,
                            uint64_t start, uint64_t tokens, float *keys, float *values);
hipError_t launch_page_copy(hipStream_t s, const safetyraise_kernel_kv_pool *pool, int32_t dst,
                            int32_t src);

struct AttnLaunch {
    const safetyraise_kernel_kv_pool *pool;
    uint32_t flags;
    uint32_t heads, kv_heads, head_dim, rotary_dim;
    // query-head groups per cache KV head: a GQA group of G > 8 heads runs
    // as kv_rep groups of G / kv_rep (the kernels' grids see kv_heads *
    // kv_rep KV heads, group g reading cache head g / kv_rep)
    uint32_t kv_rep = 1;
    float eps;
    uint32_t mrope[3];
    const void *q, *k, *v;
    const float *q_norm, *k_norm;
    const int32_t *positions;
    float *out;
    uint32_t *err_word;
    const RopeTable *rope;
    // generic head widths: theta^(2i/rotary_dim) for i < rotary_dim/2 (up to
    // kGenericMaxHeadDim/2 pairs, more than RopeTable holds)
    const float *rope_denom = nullptr;
    // page-table entries of this call not yet on the device (at most
    // kInlineTable): the first append kernel of the call writes them, and
    // resolves its own rows' pages from them
    const uint32_t *tbl_idx = nullptr;
    const int32_t *tbl_val = nullptr;
    uint32_t tbl_n = 0;
};
constexpr uint32_t kInlineTable = 64;

// Device scratch of one attention call: the split-K partial records (decode
// and verify) and the prefill RoPE table.  Each function returns nullptr,
// with the context's error text set, when it cannot provide `bytes`.  The
// default grows context-owned buffers; the no-allocation entry point hands
// out parts of a fixed region.
struct AttnScratch {
    float *(*partials)(void *user, size_t bytes);
    void *(*rope)(void *user, size_t bytes);
    void *user;
};
// safetyraise_kernel_attention_forward with the call's scratch from `scratch`.
int32_t attention_forward_impl(Ctx *ctx, const safetyraise_kernel_attention_args *args,
                               const AttnScratch &scratch);

// Host inputs of the decode launch plan: the CU count and a way to get the
// scratch for per-segment (max, sum, output) records (context-owned, grown
// on demand; returns nullptr when it cannot be allocated).
struct DecodePlanInput {
    int num_cus;
    float *(*reserve)(void *user, size_t bytes);
    void *user;
    float *reserve_partials(size_t bytes) const { return reserve(user, bytes); }
};

// Decode: one new row per sequence (seqs[i].ctx tokens cached before it,
// row seqs[i].row0 of the call's tensors).  Up to kMetaPerLaunch sequences
// whose visible tokens sum below 2^31.
hipError_t launch_attn_decode(hipStream_t s, const AttnLaunch &a, const SeqMeta *seqs, int nseq,
                              const DecodePlanInput &in);

// Chunked prefill: seqs[i].rows new rows appended after seqs[i].ctx cached
// tokens, row i attending to ctx + i + 1 keys.  Up to kMetaPerLaunch
// sequences; only for geometries where prefill_supported() holds.
// rope_scratch holds prefill_rope_bytes(a, rows of the call) bytes (per-row
// RoPE cos/sin shared by the two kernels).
bool prefill_supported(const AttnLaunch &a);
size_t prefill_rope_bytes(const AttnLaunch &a, uint64_t total_rows);
hipError_t launch_attn_prefill(hipStream_t s, const AttnLaunch &a, const SeqMeta *seqs, int nseq,
                               void *rope_scratch);
// Multi-row verify (2..15 rows per sequence, rows x heads/kv_heads <= 64,
// head_dim <= 128): split-K over key partitions with MFMA inner products,
// then a combine pass; partial records come from in.reserve_partials.
bool verify_supported(const AttnLaunch &a, uint32_t rows);
// Head widths other than 64, 128 and 256 (up to kGenericMaxHeadDim): every
// row of the call through the plain f32 kernels of attn_generic.hip (append,
// then attention); a.rope_denom must hold the rotary pairs' denominators.
bool generic_head_dim(uint32_t head_dim);
hipError_t launch_attn_generic(hipStream_t s, const AttnLaunch &a, const SeqMeta *seqs, int nseq);
hipError_t launch_attn_verify(hipStream_t s, const AttnLaunch &a, const SeqMeta *seqs, int nseq,
                              void *rope_scratch, const DecodePlanInput &in);

struct GdnLaunch {
    const safetyraise_kernel_gdn_pool *pool;
    const void *qkv, *z, *a, *b;
    const float *a_log, *dt_bias, *conv_w, *norm;
    float *raw, *out;
    uint32_t *err_word;
    float eps;
    bool bf16_in;
    // KEEP_ROWS: every row's record goes to records[slot][row] (rec_stride
    // floats each, keep_rows per slot)
    bool keep = false;
    float *records = nullptr;
    uint32_t rec_stride = 0, keep_rows = 0;
    // chunked prefill: gdn_chunk_rec_bytes(...) bytes of per-chunk records
    float *chunk_rec = nullptr;
    int num_cus = 256;
};

// One sequence of a GDN launch: pool slot, its rows in the call, the
// current history buffer, and the state buffers read and written (indices in
// units of one sequence's state; equal except for KEEP_ROWS calls).
struct GdnSeq {
    uint32_t slot, rows, row0, parity, state_in, state_out;
};

// gdn_rollback_kernel's inputs for one sequence.
struct GdnRollback {
    const float *state_in;
    float *state_out;
    const float *hist_in;
    float *hist_out;
    const float *records;
    uint32_t rec_stride, keep, value_heads, channels, conv_k;
    uint32_t key_dim, value_dim;
};
hipError_t launch_gdn_rollback(hipStream_t stream, const GdnRollback &r);

// y[M][N] = x[M][K] . W[N][K]^T with f32 products, W of dtype F32/F16/BF16
// (linear_kernels.hip).  scratch holds linear_scratch_bytes(...) bytes of
// partial sums (none when that is 0) for calls that split K.
size_t linear_scratch_bytes(uint32_t M, uint32_t N, uint32_t K, uint32_t dtype, int num_cus);
// Device bytes of a [rows][cols] weight as the kernels read it: row-major for
// F32 and F16, whole 1 KB tiles for BF16 (SIZE_MAX when that overflows).
size_t linear_weight_bytes(uint64_t rows, uint64_t cols, uint32_t dtype);
// The BF16 tile layout in dst from a row-major bf16 weight in device memory.
hipError_t linear_pack_bf16(hipStream_t stream, const void *src, void *dst, uint64_t rows,
                            uint64_t cols);
hipError_t launch_linear(hipStream_t stream, const float *x, const void *w, uint32_t dtype,
                         float *y, uint32_t M, uint32_t N, uint32_t K, float *scratch,
                         int num_cus);

// Conv + delta rule over every row of every sequence, then RMSNorm * silu(z).
// Calls that take the chunked form need g.chunk_rec with
// gdn_chunk_rec_bytes(...) bytes (0 for other calls; qkv_aligned: the qkv
// rows the kernels read start 16-byte aligned).
size_t gdn_chunk_rec_bytes(const safetyraise_kernel_gdn_pool *pool, const GdnSeq *seqs, int nseq,
                           bool keep, bool qkv_aligned);
hipError_t launch_gdn(hipStream_t stream, const GdnLaunch &g, const GdnSeq *seqs, int nseq,
                      uint32_t total_rows);
uint32_t gdn_key_dim();
uint32_t gdn_row_block();
uint32_t gdn_max_kernel();

}  // namespace sr
