// Gated delta net (Qwen3.5 linear attention) for gfx950.
//
// gdn_delta_kernel replaces, for a batch of sequences and all their rows,
// causal_conv_silu (reference src/model/math.rs:158-187) followed by
// gated_delta_step (math.rs:190-239); gdn_norm_gate_kernel applies the
// per-value-head RMSNorm and the silu(z) gate of Gdn::forward
// (src/model/native.rs:737-740).
//
// Work decomposition: one workgroup per (sequence, value head h, block of 16
// rows of the state S[h] in R^{Dv x Dk}).  Rows of S are independent given
// k^, q^, v, alpha and beta, so the state slice (16 x 128 f32, 8 per lane)
// stays in registers for all rows of the call and is read and written once.
// 16 lanes own one state row; the two dot products per row are 16-lane DPP
// reductions.  Each workgroup recomputes the causal conv for the q/k channels
// of its key head (shared with the sibling value heads and row blocks) and
// for its 16 v channels.  The conv history is double-buffered per sequence
// slot: every workgroup reads the current buffer and the owner of each
// channel writes the next one, so no workgroup can overwrite history that
// another still has to read.
#include "sr_device.hpp"

#include <type_traits>

namespace sr {

namespace {

constexpr int kThreads = 256;
constexpr int kRows = 16;   // state rows per workgroup
constexpr int kDk = 128;    // key dim (lanes x 8)
constexpr int kMaxK = 8;    // largest conv kernel
constexpr uint32_t kHeadKernelRows = 8;

struct GdnMeta {
    uint32_t slot;
    uint32_t rows;
    uint32_t row0;
    uint32_t parity;     // history buffer holding the current history
    uint32_t state_in;   // state buffer read (index in units of one state)
    uint32_t state_out;  // state buffer written (== state_in but for KEEP_ROWS calls)
    uint32_t chunk0;     // chunked prefill: the sequence's first chunk record in the launch
};

struct GdnParams {
    float *state;            // [slots][Hv][Dv][Dk]
    float *history;          // [2][slots][C][K-1]
    const void *qkv;         // [rows][C]
    const void *a;           // [rows][Hv]
    const void *b;
    const float *a_log;      // [Hv]
    const float *dt_bias;
    const float *conv_w;     // [C][K]
    float *raw_out;          // [rows][Hv*Dv]
    // chunked prefill: one record of kRecFloats per (chunk, value head), chunk
    // records of a sequence from meta.chunk0 on
    float *chunk_rec;
    // KEEP_ROWS calls (gdn_head_kernel only): per (slot, row) the row's decay
    // alpha [Hv], correction delta [Hv][Dv], normalised key k^ [Hv][Dk] and raw
    // conv inputs x [C], from which gdn_rollback_kernel rebuilds the state and
    // history after any row; nullptr otherwise
    float *records;
    uint32_t rec_stride;     // floats per (slot, row) record
    uint32_t keep_rows;      // records per slot
    uint32_t key_heads, value_heads, value_dim, conv_k, channels, max_slots;
    int bf16_in;
    uint32_t nseq;
    GdnMeta meta[kMetaPerLaunch];
};

__device__ __forceinline__ float softplus_ref(float x) {
    // src/model/math.rs:24-26
    return fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x)));
}

// One depthwise causal-conv channel held in a thread's registers
// (math.rs:158-187): the K-1 most recent raw inputs, oldest first, and the K
// weights.  All of it is loaded up front (compile-time bounds, so every load
// is in flight at once) and the per-row conv and history shift are register
// operations.
struct ConvChan {
    float hist[kMaxK - 1];
    float w[kMaxK];
    // Every load is unconditional, at an index clamped into the row (the
    // history allocation holds at least one value, for K = 1): conditional
    // loads would each end in a wait for all loads in flight.
    __device__ __forceinline__ void load(const float *history_row, const float *weights,
                                         uint32_t K) {
        const int last_h = K >= 2 ? (int)K - 2 : 0;
#pragma unroll
        for (int j = 0; j < kMaxK - 1; ++j) hist[j] = history_row[j < last_h ? j : last_h];
#pragma unroll
        for (int j = 0; j < kMaxK; ++j) w[j] = weights[j < (int)K - 1 ? j : (int)K - 1];
    }
    // the K-1 raw inputs before the next row from src[j * stride], oldest first
    __device__ __forceinline__ void set_hist(const float *src, int stride, uint32_t K) {
        const int last_h = K >= 2 ? (int)K - 2 : 0;
#pragma unroll
        for (int j = 0; j < kMaxK - 1; ++j) hist[j] = src[(j < last_h ? j : last_h) * stride];
    }
    static constexpr int kK = 0;  // kernel size known only at run time
    // silu(sum_{j<K-1} hist[j] * w[j] + x * w[K-1]), then append x
    __device__ __forceinline__ float step(float x, uint32_t K) {
        const float value = pre(x, K);
        return value * ref_sigmoid(value);
    }
    // the conv sum before silu, then append x
    __device__ __forceinline__ float pre(float x, uint32_t K) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < kMaxK - 1; ++j) {
            if (j + 1 < (int)K) acc += hist[j] * w[j];
        }
        float wl = 0.0f;
#pragma unroll
        for (int j = 0; j < kMaxK; ++j) {
            if (j + 1 == (int)K) wl = w[j];
        }
        const float value = acc + x * wl;
#pragma unroll
        for (int j = 0; j < kMaxK - 1; ++j) {
            if (j + 2 < (int)K) hist[j] = hist[j + 1];
            else if (j + 2 == (int)K) hist[j] = x;
        }
        return value;
    }
    __device__ __forceinline__ void store(float *history_row, uint32_t K) const {
#pragma unroll
        for (int j = 0; j < kMaxK - 1; ++j) {
            if (j + 1 < (int)K) history_row[j] = hist[j];
        }
    }
};

__global__ void __launch_bounds__(kThreads) gdn_delta_kernel(const GdnParams p) {
    constexpr int kCh = 2 * kDk + kRows;  // conv channels this workgroup needs
    __shared__ float conv_s[kCh];
    __shared__ float red_s[2][4];
    __shared__ float ab_s[2];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int group = tid >> 4;
    const int l16 = tid & 15;

    const uint32_t blocks_per_head = p.value_dim / kRows;
    const uint32_t rb = blockIdx.x % blocks_per_head;
    const uint32_t h = (blockIdx.x / blocks_per_head) % p.value_heads;
    const uint32_t s = blockIdx.x / (blocks_per_head * p.value_heads);
    const GdnMeta m = p.meta[s];
    const uint32_t groups = p.value_heads / p.key_heads;
    const uint32_t kh = h / groups;
    const uint32_t key_width = p.key_heads * kDk;
    const uint32_t K1 = p.conv_k - 1;
    const uint32_t v_row = rb * kRows + group;  // this group's state row

    // channel index of local channel c: q of kh, k of kh, then 16 v channels
    auto chan = [&](int c) -> uint32_t {
        if (c < kDk) return kh * kDk + c;
        if (c < 2 * kDk) return key_width + kh * kDk + (c - kDk);
        return 2 * key_width + h * p.value_dim + rb * kRows + (c - 2 * kDk);
    };

    // state slice: row v_row, dims [8*l16, 8*l16+8)
    float *srow = p.state + (((size_t)m.state_in * p.value_heads + h) * p.value_dim + v_row) * kDk +
                  l16 * 8;
    float S[8];
    {
        const float4 x0 = *(const float4 *)srow;
        const float4 x1 = *(const float4 *)(srow + 4);
        S[0] = x0.x; S[1] = x0.y; S[2] = x0.z; S[3] = x0.w;
        S[4] = x1.x; S[5] = x1.y; S[6] = x1.z; S[7] = x1.w;
    }
    const float a_log_e = expf(p.a_log[h]);
    const float dt = p.dt_bias[h];
    const float qscale = 1.0f / sqrtf((float)kDk);  // math.rs:213
    // a row's inputs (this thread's channels tid and tid + 256, a, b) are
    // loaded one row ahead, so a row never waits for its own loads
    const bool two = tid + kThreads < kCh;
    const uint32_t ch0 = chan(tid);
    const uint32_t ch1 = two ? chan(tid + kThreads) : 0;
    const size_t hist_slot = ((size_t)m.parity * p.max_slots + m.slot) * p.channels;
    const size_t hist_next = ((size_t)(1 - m.parity) * p.max_slots + m.slot) * p.channels;
    // (loads unconditional; a thread without a second channel reads its
    // first one again and ignores it)
    ConvChan cv0, cv1;
    cv0.load(p.history + (hist_slot + ch0) * K1, p.conv_w + (size_t)ch0 * p.conv_k, p.conv_k);
    const uint32_t ch1l = two ? ch1 : ch0;
    cv1.load(p.history + (hist_slot + ch1l) * K1, p.conv_w + (size_t)ch1l * p.conv_k, p.conv_k);
    float x0 = 0.0f, x1 = 0.0f, av = 0.0f, bv = 0.0f;
    auto load_row = [&](size_t row) {
        x0 = load_act_nb(p.qkv, row * p.channels + ch0, p.bf16_in != 0);
        x1 = load_act_nb(p.qkv, row * p.channels + ch1l, p.bf16_in != 0);
        av = load_act_nb(p.a, row * p.value_heads + h, p.bf16_in != 0);
        bv = load_act_nb(p.b, row * p.value_heads + h, p.bf16_in != 0);
    };
    load_row(m.row0);
    __syncthreads();

    for (uint32_t r = 0; r < m.rows; ++r) {
        const size_t row = (size_t)m.row0 + r;
        // A. causal conv + silu for the needed channels (math.rs:175-185)
        conv_s[tid] = cv0.step(x0, p.conv_k);
        if (two) conv_s[tid + kThreads] = cv1.step(x1, p.conv_k);
        if (tid == 0) {
            // math.rs:220-221
            ab_s[0] = expf(-a_log_e * softplus_ref(av + dt));
            ab_s[1] = ref_sigmoid(bv);
        }
        load_row(m.row0 + min(r + 1, m.rows - 1));  // next row's inputs (unconditional)
        __syncthreads();
        // B. L2 norms of q and k (math.rs:218-219): wave 0 -> q, wave 1 -> k
        if (wave < 2) {
            const float x0 = conv_s[wave * kDk + lane];
            const float x1 = conv_s[wave * kDk + lane + 64];
            const float ss = sum64(x0 * x0 + x1 * x1);
            if (lane == 0) red_s[wave][0] = 1.0f / sqrtf(ss + 1e-6f);
        }
        __syncthreads();
        // C. delta rule on this lane's 8 state values (math.rs:222-236)
        const float qi = red_s[0][0];
        const float ki = red_s[1][0];
        const float alpha = ab_s[0];
        const float beta = ab_s[1];
        float kh8[8], qh8[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            kh8[j] = conv_s[kDk + l16 * 8 + j] * ki;
            qh8[j] = conv_s[l16 * 8 + j] * qi;
        }
        float pred = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            S[j] *= alpha;
            pred += S[j] * kh8[j];
        }
        pred = sum16(pred);
        const float corr = beta * (conv_s[2 * kDk + group] - pred);
        float rd = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            S[j] += corr * kh8[j];
            rd += S[j] * qh8[j];
        }
        rd = sum16(rd);
        if (l16 == 0) {
            p.raw_out[row * p.value_heads * p.value_dim + (size_t)h * p.value_dim + v_row] =
                rd * qscale;
        }
        __syncthreads();  // conv_s / red_s are rewritten by the next row
    }

    *(float4 *)srow = make_float4(S[0], S[1], S[2], S[3]);
    *(float4 *)(srow + 4) = make_float4(S[4], S[5], S[6], S[7]);
    // next history: v channels by their owner; q/k channels by the first
    // value head of the key group, row block 0
    const bool owns_qk = (h % groups == 0) && rb == 0;
    if (tid >= 2 * kDk || owns_qk) cv0.store(p.history + (hist_next + ch0) * K1, p.conv_k);
    if (two) cv1.store(p.history + (hist_next + ch1) * K1, p.conv_k);  // v channels
}

// ---------------------------------------------------------------------------
// gdn_head_kernel: one workgroup per (sequence, value head) with Dv = 128.
// The head's whole 128 x 128 f32 state stays in registers (16 lanes per
// state row, 8 rows per 16-lane group, 8 dims per lane), so the q/k/v conv
// channels of the head are computed once and the per-head RMSNorm * silu(z)
// of Gdn::forward (native.rs:737-740) runs in the same kernel: no raw-output
// round trip and no second launch.  Every global input of the first row -
// state, history, conv weights, qkv, z, a, b - is requested before the
// first barrier, and each later row's inputs are loaded while the current
// row computes.  Used for decode-sized calls (few rows per sequence), where
// the sequences x heads workgroups fill the GPU.
// ---------------------------------------------------------------------------
constexpr int kHeadDv = 128;

// The kernel arguments gdn_head_kernel uses, held in scalar registers.
struct HeadArgs {
    float *state;
    float *history;
    const void *qkv;
    const void *a;
    const void *b;
    const float *a_log;
    const float *dt_bias;
    const float *conv_w;
    const float *norm;
    const void *z;
    float *out;
    uint32_t *err_word;
    float *records;
    float eps;
    uint32_t key_heads, value_heads, conv_k, channels, max_slots, rec_stride, keep_rows;
    int bf16_in;
    // forces every field into a register here, so all the reads are issued
    // together and waited for once
    __device__ __forceinline__ void pin() {
        state = pin_global(state);
        records = pin_global(records);
        history = pin_global(history);
        qkv = pin_global(qkv);
        a = pin_global(a);
        b = pin_global(b);
        a_log = pin_global(a_log);
        dt_bias = pin_global(dt_bias);
        conv_w = pin_global(conv_w);
        norm = pin_global(norm);
        z = pin_global(z);
        out = pin_global(out);
        err_word = pin_global(err_word);
        asm volatile("" : "+s"(eps), "+s"(key_heads), "+s"(value_heads), "+s"(conv_k),
                     "+s"(channels), "+s"(max_slots), "+s"(rec_stride), "+s"(keep_rows),
                     "+s"(bf16_in));
    }
};
constexpr int kHeadCh = 2 * kDk + kHeadDv;  // q, k and v channels of one head
constexpr int kHeadThreads = 512;

template <int NTH, class Conv>
__global__ void __launch_bounds__(NTH) gdn_head_kernel(const GdnParams p, const float *norm,
                                                            const void *z, float *out,
                                                            uint32_t *err_word, float eps) {
    __shared__ float conv_s[kHeadCh];
    __shared__ float out_s[kHeadDv];
    __shared__ float red_s[2];
    __shared__ float ab_s[2];

    constexpr int RPG = kHeadDv / (NTH / 16);  // state rows per 16-lane group
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int group = tid >> 4;
    const int l16 = tid & 15;
    // Every kernel argument used below is read here, in one batch of scalar
    // loads with one wait: left to itself the compiler reads each just before
    // its first use, and the state loads then sit behind several dependent
    // scalar round trips.
    // grid (value head, sequence): the sequence's entry needs no argument
    // to locate it, so it is read in the same batch
    const GdnMeta m = p.meta[blockIdx.y];
    HeadArgs a{p.state, p.history, p.qkv, p.a, p.b, p.a_log, p.dt_bias, p.conv_w, norm, z, out,
               err_word, p.records, eps, p.key_heads, p.value_heads, p.conv_k, p.channels,
               p.max_slots, p.rec_stride, p.keep_rows, p.bf16_in};
    a.pin();
    const bool bf16_in = a.bf16_in != 0;

    const uint32_t h = blockIdx.x;
    const uint32_t groups = a.value_heads / a.key_heads;
    const uint32_t kh = h / groups;
    const uint32_t key_width = a.key_heads * kDk;
    const uint32_t K1 = a.conv_k - 1;
    const size_t width = (size_t)a.value_heads * kHeadDv;
    auto chan = [&](int c) -> uint32_t {
        if (c < kDk) return kh * kDk + c;
        if (c < 2 * kDk) return key_width + kh * kDk + (c - kDk);
        return 2 * key_width + h * kHeadDv + (c - 2 * kDk);
    };
    // this thread's conv channels: tid (if < 384), and tid + NTH when that is
    // < 384 (only with fewer than 384 threads)
    constexpr bool kTwo = NTH < kHeadCh;
    const bool one = tid < kHeadCh;
    const bool two = kTwo && tid + NTH < kHeadCh;
    const uint32_t ch0 = one ? chan(tid) : 0;
    const uint32_t ch1 = two ? chan(tid + NTH) : 0;

    const size_t hist_slot = ((size_t)m.parity * a.max_slots + m.slot) * a.channels;
    const size_t hist_next = ((size_t)(1 - m.parity) * a.max_slots + m.slot) * a.channels;
    // (all loads unconditional: a conditional load ends in a wait for every
    // load in flight; threads without a channel read channel 0 and ignore it)
    Conv cv0, cv1;
    cv0.load(a.history + (hist_slot + ch0) * K1, a.conv_w + (size_t)ch0 * a.conv_k, a.conv_k);
    if constexpr (kTwo) {
        cv1.load(a.history + (hist_slot + ch1) * K1, a.conv_w + (size_t)ch1 * a.conv_k, a.conv_k);
    }
    // inputs of a row: qkv channels, z of this head (dims lane and lane + 64,
    // used by wave 0), a and b
    // a and b are the same for every lane; read through a per-lane offset the
    // compiler cannot fold (zero), they stay in vector registers.  As
    // wave-uniform values they were moved to scalar registers right after
    // the next row's loads, and that move waited for every load in flight,
    // the whole state included.
    uint32_t vzero = 0;
    asm volatile("" : "+v"(vzero));
    float x0 = 0.0f, x1 = 0.0f, z0 = 0.0f, z1 = 0.0f, av = 0.0f, bv = 0.0f;
    auto load_row = [&](size_t row) {
        x0 = load_act_nb(a.qkv, row * a.channels + ch0, bf16_in);
        if constexpr (kTwo) x1 = load_act_nb(a.qkv, row * a.channels + ch1, bf16_in);
        z0 = load_act_nb(a.z, row * width + h * kHeadDv + lane, bf16_in);
        z1 = load_act_nb(a.z, row * width + h * kHeadDv + lane + 64, bf16_in);
        av = load_act_nb(a.a, row * a.value_heads + h + vzero, bf16_in);
        bv = load_act_nb(a.b, row * a.value_heads + h + vzero, bf16_in);
    };
    load_row(m.row0);
    // state rows v = (NTH/16) i + group, dims [4 l16, 4 l16 + 4) and
    // [64 + 4 l16, 64 + 4 l16 + 4): each 16-byte load or store instruction
    // then covers 256 contiguous bytes of a row; requested after
    // the (branchy) conv loads so that nothing waits for them before the
    // delta step itself
    float *sbase = a.state + ((size_t)m.state_in * a.value_heads + h) * kHeadDv * kDk + l16 * 4;
    float *obase = a.state + ((size_t)m.state_out * a.value_heads + h) * kHeadDv * kDk + l16 * 4;
    // KEEP_ROWS: this head's part of each row's record (alpha, delta, k^, x)
    const bool keep = a.records != nullptr;  // uniform
    const uint32_t hv_dv = a.value_heads * kHeadDv;
    const bool owns_qk = (h % groups == 0);
    // the remaining small inputs are requested before the state: loads
    // complete in order for the wait counter, so a wait for one requested
    // after the state would wait for the whole state too, and the conv and
    // norms could no longer run while the state arrives
    const float a_log_v = a.a_log[h];
    const float dt = a.dt_bias[h];
    const float nw0 = a.norm[lane], nw1 = a.norm[lane + 64];
    // the state is read once and written once per call: nontemporal
    // accesses (streaming reads measured ~8 % faster than ordinary loads)
    typedef float nt_f32x4 __attribute__((ext_vector_type(4)));
    float S[RPG][8];
#pragma unroll
    for (int i = 0; i < RPG; ++i) {
        const float *src = sbase + (size_t)((NTH / 16) * i + group) * kDk;
        const nt_f32x4 x0 = __builtin_nontemporal_load((const nt_f32x4 *)src);
        const nt_f32x4 x1 = __builtin_nontemporal_load((const nt_f32x4 *)(src + kDk / 2));
        S[i][0] = x0.x; S[i][1] = x0.y; S[i][2] = x0.z; S[i][3] = x0.w;
        S[i][4] = x1.x; S[i][5] = x1.y; S[i][6] = x1.z; S[i][7] = x1.w;
    }
    const float a_log_e = expf(a_log_v);
    const float qscale = 1.0f / sqrtf((float)kDk);  // math.rs:213
    __syncthreads();

    for (uint32_t r = 0; r < m.rows; ++r) {
        const size_t row = (size_t)m.row0 + r;
        float *rec = keep ? a.records + ((size_t)m.slot * a.keep_rows + r) * a.rec_stride : nullptr;
        // A. causal conv + silu (math.rs:175-185), history in registers
        if (one) conv_s[tid] = cv0.step(x0, a.conv_k);
        if constexpr (kTwo) {
            if (two) conv_s[tid + NTH] = cv1.step(x1, a.conv_k);
        }
        if (keep) {
            // the row's raw conv inputs (q/k channels by the key group's first head)
            float *rx = rec + a.value_heads + 2 * hv_dv;
            if (one && (tid >= 2 * kDk || owns_qk)) rx[ch0] = x0;
            if constexpr (kTwo) {
                if (two && (tid + NTH >= 2 * kDk || owns_qk)) rx[ch1] = x1;
            }
        }
        if (tid == 0) {
            // math.rs:220-221
            ab_s[0] = expf(-a_log_e * softplus_ref(av + dt));
            ab_s[1] = ref_sigmoid(bv);
            if (keep) rec[h] = ab_s[0];
        }
        const float zc0 = z0, zc1 = z1;
        load_row(m.row0 + min(r + 1, m.rows - 1));  // next row's inputs (unconditional)
        __syncthreads();
        // B. L2 norms of q and k (math.rs:218-219): wave 0 -> q, wave 1 -> k
        if (wave < 2) {
            const float y0 = conv_s[wave * kDk + lane];
            const float y1 = conv_s[wave * kDk + lane + 64];
            const float ss = sum64(y0 * y0 + y1 * y1);
            if (lane == 0) red_s[wave] = 1.0f / sqrtf(ss + 1e-6f);
        }
        __syncthreads();
        // C. delta rule on the 8 state rows of this group (math.rs:222-236)
        const float qi = red_s[0];
        const float ki = red_s[1];
        const float alpha = ab_s[0];
        const float beta = ab_s[1];
        float kh8[8], qh8[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int dim = (j < 4) ? 4 * l16 + j : kDk / 2 + 4 * l16 + (j - 4);
            kh8[j] = conv_s[kDk + dim] * ki;
            qh8[j] = conv_s[dim] * qi;
            if (keep && group == 0) rec[a.value_heads + hv_dv + h * kDk + dim] = kh8[j];
        }
#pragma unroll
        for (int i = 0; i < RPG; ++i) {
            const int v = (NTH / 16) * i + group;
            float pred = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                S[i][j] *= alpha;
                pred += S[i][j] * kh8[j];
            }
            pred = sum16(pred);
            const float corr = beta * (conv_s[2 * kDk + v] - pred);
            if (keep && l16 == 0) rec[a.value_heads + h * kHeadDv + v] = corr;
            float rd = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                S[i][j] += corr * kh8[j];
                rd += S[i][j] * qh8[j];
            }
            rd = sum16(rd);
            if (l16 == 0) out_s[v] = rd * qscale;
            if (r + 1 == m.rows) {
                // final values of this slice: written now, so that the state
                // writes stream out while later slices are still arriving
                float *dst = obase + (size_t)v * kDk;
                __builtin_nontemporal_store(nt_f32x4{S[i][0], S[i][1], S[i][2], S[i][3]},
                                            (nt_f32x4 *)dst);
                __builtin_nontemporal_store(nt_f32x4{S[i][4], S[i][5], S[i][6], S[i][7]},
                                            (nt_f32x4 *)(dst + kDk / 2));
            }
        }
        __syncthreads();
        // D. RMSNorm without offset (math.rs:28-50), then * silu(z)
        if (wave == 0) {
            const float o0 = out_s[lane], o1 = out_s[lane + 64];
            const float ss = sum64(o0 * o0 + o1 * o1);
            const float variance = ss / (float)kHeadDv;
            if (!isfinite(variance) && lane == 0) atomicOr(a.err_word, kErrNonFiniteVariance);
            const float inv = 1.0f / sqrtf(variance + a.eps);
            float *dst = a.out + row * width + h * kHeadDv;
            dst[lane] = o0 * inv * nw0 * (zc0 * ref_sigmoid(zc0));
            dst[lane + 64] = o1 * inv * nw1 * (zc1 * ref_sigmoid(zc1));
        }
    }

    // next history: v channels here; q/k channels by the first value head of
    // the key group (the others compute the same values)
    if (one && (tid >= 2 * kDk || owns_qk)) cv0.store(a.history + (hist_next + ch0) * K1, a.conv_k);
    if constexpr (kTwo) {
        if (two && (tid + NTH >= 2 * kDk || owns_qk)) cv1.store(a.history + (hist_next + ch1) * K1, a.conv_k);
    }
}

// ---------------------------------------------------------------------------
// gdn_rollback_kernel: one sequence's state and conv history as they were
// after row `keep` of its last KEEP_ROWS call, rebuilt from the state before
// that call (the other state buffer, which the call only read) and the call's
// records.  Per row the state update is S = alpha S + delta k^T, applied
// element by element with the same operations gdn_head_kernel applies (a
// product, then a multiply-add), so the rebuilt state is the one the forward
// held after that row; the history is the last K-1 of (the history before
// the call, x_0 .. x_{keep-1}).  Blocks 0..Hv-1 rebuild one value head's
// state each, the others 256 conv channels each.
// ---------------------------------------------------------------------------
struct RollbackParams {
    const float *state_in;  // [Hv][Dv][Dk] before the call
    float *state_out;       // [Hv][Dv][Dk] the sequence's current buffer
    const float *hist_in;   // [C][K-1] before the call
    float *hist_out;        // [C][K-1] the current history buffer
    const float *records;   // the sequence's records, rows 0 .. keep-1
    uint32_t rec_stride, keep, value_heads, channels, conv_k;
};

__global__ void __launch_bounds__(256) gdn_rollback_kernel(const RollbackParams p) {
    const uint32_t tid = threadIdx.x;
    const uint32_t hv_dv = p.value_heads * kHeadDv;
    if (blockIdx.x < p.value_heads) {
        const uint32_t h = blockIdx.x;
        const uint32_t l16 = tid & 15, g = tid >> 4;  // rows g + 16 i, dims 8 l16 .. + 8
        const float *src = p.state_in + (size_t)h * kHeadDv * kDk + 8 * l16;
        float *dst = p.state_out + (size_t)h * kHeadDv * kDk + 8 * l16;
        float S[8][8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float *s = src + (size_t)(g + 16 * i) * kDk;
            const float4 x0 = *(const float4 *)s, x1 = *(const float4 *)(s + 4);
            S[i][0] = x0.x; S[i][1] = x0.y; S[i][2] = x0.z; S[i][3] = x0.w;
            S[i][4] = x1.x; S[i][5] = x1.y; S[i][6] = x1.z; S[i][7] = x1.w;
        }
        for (uint32_t r = 0; r < p.keep; ++r) {
            const float *rec = p.records + (size_t)r * p.rec_stride;
            const float alpha = rec[h];
            float kh[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) kh[j] = rec[p.value_heads + hv_dv + h * kDk + 8 * l16 + j];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float corr = rec[p.value_heads + h * kHeadDv + g + 16 * i];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    S[i][j] *= alpha;
                    S[i][j] += corr * kh[j];
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float *d = dst + (size_t)(g + 16 * i) * kDk;
            *(float4 *)d = make_float4(S[i][0], S[i][1], S[i][2], S[i][3]);
            *(float4 *)(d + 4) = make_float4(S[i][4], S[i][5], S[i][6], S[i][7]);
        }
        return;
    }
    const uint32_t c = (blockIdx.x - p.value_heads) * 256 + tid;
    const uint32_t K1 = p.conv_k - 1;
    if (c >= p.channels || K1 == 0) return;
    // position t of (history before the call, x_0, x_1, ...): the last K-1
    // positions up to row keep - 1 are t = keep .. keep + K1 - 1
    for (uint32_t i = 0; i < K1; ++i) {
        const uint32_t t = p.keep + i;
        p.hist_out[(size_t)c * K1 + i] =
            t < K1 ? p.hist_in[(size_t)c * K1 + t]
                   : p.records[(size_t)(t - K1) * p.rec_stride + p.value_heads + 2 * hv_dv + c];
    }
}

// ---------------------------------------------------------------------------
// Chunked prefill: the delta rule of prefill-sized calls in chunked form on
// f32 MFMA (v_mfma_f32_16x16x4f32).  With k^, q^ the L2-normalised conv
// outputs, g_t = sum_{i<=t} log(alpha_i) over the chunk and S0 the state at
// the chunk start, the token-serial recurrence (math.rs:222-236)
//     S_t = alpha_t S_{t-1} + delta_t k^_t^T,
//     delta_t = beta_t (v_t - alpha_t S_{t-1} k^_t)
// unrolls to S_t = e^{g_t} S0 + sum_{j<=t} e^{g_t-g_j} delta_j k^_j^T, and
// the deltas of a chunk solve the unit lower-triangular system
//     (I + A) Delta = diag(beta) V - diag(beta e^g) K^ S0^T,
//     A[t][j] = beta_t e^{g_t-g_j} (k^_t . k^_j)  (j < t),
// so with T = (I + A)^-1, W = T diag(beta e^g) K^, U = T diag(beta) V:
//     Delta = U - W S0^T
//     o_t   = (e^{g_t} S0 q^_t + sum_{j<=t} e^{g_t-g_j} (q^_t . k^_j) delta_j) / sqrt(Dk)
//     S_C   = e^{g_C} S0 + sum_j e^{g_C-g_j} delta_j k^_j^T.
// Decays enter only as e^{x} with x <= 0.
//
// Only the three products with S0 depend on the state.  Everything else --
// conv, norms, q.k, k.k, T, W, U -- depends on the chunk's own rows and the
// K-1 raw inputs before them, so it is computed in two kernels:
//   gdn_chunk_prep_kernel: one workgroup per (sequence, chunk, value head),
//     all chunks of the call at once; writes a record per (chunk, value head):
//       Qe = diag(e^{g_t} / |q_t|) Q,  -W,  U,  Ks = K^T diag(e^{g_C-g_j} / |k_j|),
//       Pm[t][j] = e^{g_t-g_j} (q^_t . k^_j) (j <= t),  e^{g_C}
//     and, from the last chunk, the next conv history (the records with
//     nontemporal stores: the scan reads them on other XCDs, from memory
//     anyway, and streaming them out took 0.5 us off the kernel);
//   gdn_chunk_scan_kernel: one workgroup per (sequence, value head, 32 of the
//     Dv = 128 state rows), the slice in LDS, walking the chunks in order:
//       Delta = U + (-W) S0^T,  o = (Qe S0^T + Pm Delta) / sqrt(Dk),
//       S_C = e^{g_C} S0 + Delta^T Ks^T.
// The conv history is double-buffered exactly as in gdn_delta_kernel.
// ---------------------------------------------------------------------------
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ void pin(T &x) {
    asm volatile("" : "+v"(x));
}

constexpr int kCk = 32;        // rows per chunk
constexpr int kVs = 32;        // state rows (value dims) per workgroup
constexpr int kPr = kDk + 4;   // pitch (floats) of [.][Dk] arrays
constexpr int kPc = kCk + 4;   // pitch of [.][chunk] arrays
constexpr int kScanThreads = 512;  // gdn_chunk_scan_kernel
constexpr int kPrepThreads = 512;  // gdn_chunk_prep_kernel

// x * sigmoid(x) with the hardware exp2 and reciprocal (a few ulp from the
// libm form; the chunked path is held to the f32 tolerance, not to ulps)
__device__ __forceinline__ float fast_silu(float x) {
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

// The value head of grid slot x (0 <= x < Hv) in the chunked kernels.  The
// dispatcher places workgroup i on XCD i % 8; with key_heads a multiple of 8
// the slots are ordered so that every value head of a key head lands on one
// XCD (key head (x % 8) + 8 (slot / groups), slot = x / 8), where the value
// heads share the key head's q/k rows and their records in its L2.
__device__ __forceinline__ uint32_t head_of_slot(uint32_t x, uint32_t key_heads, uint32_t groups) {
    if (key_heads % 8 != 0) return x;
    const uint32_t slot = x >> 3;
    return ((x & 7) + 8 * (slot / groups)) * groups + slot % groups;
}

// e^x with the hardware exp2 (e^{-inf} = 0); for the chunked form's decay
// factors, held to the f32 tolerance like fast_silu
__device__ __forceinline__ float fast_exp(float x) {
    return __builtin_amdgcn_exp2f(1.4426950408889634f * x);
}

// One (chunk, value head) record of gdn_chunk_prep_kernel, in floats.
constexpr int kRecQe = 0;                      // [kCk][kDk]     Qe
constexpr int kRecWn = kRecQe + kCk * kDk;     // [kCk][kDk]     -W
constexpr int kRecU = kRecWn + kCk * kDk;      // [kCk][kHeadDv] U
constexpr int kRecKs = kRecU + kCk * kHeadDv;  // [kDk][kCk]     Ks
constexpr int kRecPm = kRecKs + kDk * kCk;     // [kCk][kCk]     Pm
constexpr int kRecEc = kRecPm + kCk * kCk;     // e^{g_C}
constexpr int kRecFloats = kRecEc + 64;        // a 256-byte multiple
constexpr int kPre = kMaxK - 1;                // raw input rows staged before a chunk

struct ScanLds {
    float s0[kVs][kPr];  // state slice: rows v, dims d
    float dt[kVs][kPc];  // Delta of the slice, transposed: [v][t]
    struct Rec {         // a chunk's record, rows padded against bank conflicts
        float qe[kCk][kPr];
        float wn[kCk][kPr];
        float ks[kDk][kPc];
        float pm[kCk][kPc];
        float u[kCk][kPc];  // this slice's columns of U
    } r[2];
};

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// One lane's operand of a 16-row tile over NK steps of 16 k: row lane & 15,
// k = 16 s + 4 (lane >> 4) + i.  The tile's rows are k-contiguous in LDS.
// Every product below is acc += A . B^T with both operands in this form;
// the i-th MFMA of a step takes element i, so lane (r, slot) feeds A row r
// and B row r at the same k, and the tile's rows 4 slot + i, column r are
// acc[i].  All reads of an operand are issued before any MFMA uses them.
template <int NK>
struct Ops {
    f32x4 v[NK];
};

template <int NK>
__device__ __forceinline__ void load_ops(Ops<NK> &o, const float *row0, int ld, int lane) {
    const float *p = row0 + (lane & 15) * ld + 4 * (lane >> 4);
#pragma unroll
    for (int s = 0; s < NK; ++s) o.v[s] = *(const f32x4 *)(p + 16 * s);
}

// multiplies the operand's k-th element by scale[k]
template <int NK>
__device__ __forceinline__ void scale_ops(Ops<NK> &o, const float *scale, int lane) {
    const float *p = scale + 4 * (lane >> 4);
#pragma unroll
    for (int s = 0; s < NK; ++s) {
        o.v[s] *= *(const f32x4 *)(p + 16 * s);
    }
}

template <int NK>
__device__ __forceinline__ void mma(f32x4 &acc, const Ops<NK> &a, const Ops<NK> &b) {
#pragma unroll
    for (int s = 0; s < NK; ++s) {
        acc = mfma4(a.v[s].x, b.v[s].x, acc);
        acc = mfma4(a.v[s].y, b.v[s].y, acc);
        acc = mfma4(a.v[s].z, b.v[s].z, acc);
        acc = mfma4(a.v[s].w, b.v[s].w, acc);
    }
}

// Causal conv channel with the kernel size K known at compile time; same
// arithmetic and history layout as ConvChan.
template <int K>
struct ConvK {
    static constexpr int kK = K;
    static constexpr int H = K > 1 ? K - 1 : 1;
    float hist[H];
    float w[K];
    __device__ __forceinline__ void load(const float *history_row, const float *weights,
                                         uint32_t) {
#pragma unroll
        for (int j = 0; j < K - 1; ++j) hist[j] = history_row[j];
#pragma unroll
        for (int j = 0; j < K; ++j) w[j] = weights[j];
    }
    __device__ __forceinline__ void set_hist(const float *src, int stride, uint32_t) {
#pragma unroll
        for (int j = 0; j < K - 1; ++j) hist[j] = src[j * stride];
    }
    __device__ __forceinline__ float pre(float x, uint32_t) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < K - 1; ++j) acc += hist[j] * w[j];
        const float value = acc + x * w[K - 1];
#pragma unroll
        for (int j = 0; j + 1 < K - 1; ++j) hist[j] = hist[j + 1];
        if constexpr (K > 1) hist[K - 2] = x;
        return value;
    }
    __device__ __forceinline__ float step(float x, uint32_t K_) {
        const float value = pre(x, K_);
        return value * ref_sigmoid(value);
    }
    __device__ __forceinline__ void store(float *history_row, uint32_t) const {
#pragma unroll
        for (int j = 0; j < K - 1; ++j) history_row[j] = hist[j];
    }
};

// a[i] for a run-time i, as selects (a dynamically indexed register array
// would live in scratch memory)
template <int N>
__device__ __forceinline__ float pick(const float (&a)[N], int i) {
    float x = a[0];
#pragma unroll
    for (int j = 1; j < N; ++j) x = i == j ? a[j] : x;
    return x;
}

// Prep forms: one workgroup per (sequence, chunk, value head) forming the
// whole record, or (kSplit) two, one forming -W, Qe and Pm (grid slots
// 0 .. Hv-1) and the other U, Ks and e^{g_C} (slots Hv .. 2 Hv - 1), both
// forming A from k.k and inverting it.  Two per record keep every CU busy
// when a call has few chunks; with many chunks the shared part done twice
// costs more than it saves.
template <bool kSplit>
struct PrepLds {
    static constexpr int kIn = kSplit ? 2 * kDk : 2 * kDk + kHeadDv;  // staged channels
    struct Both {
        float q[kCk][kPr];        // conv(q) rows t
        float vc[kHeadDv][kPc];   // conv(v) transposed: [v][t]
    };
    union One {                   // a split workgroup uses one of them
        float q[kCk][kPr];
        float vc[kHeadDv][kPc];
    };
    typename std::conditional<kSplit, One, Both>::type qv;
    float k[kCk][kPr];        // conv(k) rows t
    float kc[kDk][kPc];       // conv(k) transposed: [d][t]
    float a[kCk][kPc];        // A (strictly lower)
    float t[kCk][kPc];        // T = (I + A)^-1
    float tt[kCk][kPc];       // T11^T, then M^T (P2 scratch)
    float g[kCk];             // cumulative log decay
    float beta[kCk];
    float rq[kCk];            // 1 / |q_t|
    float rk[kCk];            // 1 / |k_t|
    float sw[kCk];            // column scales of T: beta_j e^{g_j} / |k_j| (W)
    float su[kCk];            //   beta_j (U)
    float ss[kCk];            //   e^{g_C - g_j} / |k_j| (Ks; g_C: last row)
    float qs[kCk];            // Qe's row scales e^{g_t} / |q_t|
    f32x4 part[2][64];        // second k-halves of the q.k tiles (1, 0) and (1, 1)
    float xin[kPre + kCk][kIn];  // raw inputs: kPre rows before the chunk, then its rows
};

template <class Conv, bool kSplit>
__global__ void __launch_bounds__(kPrepThreads) gdn_chunk_prep_kernel(const GdnParams p) {
    extern __shared__ __align__(16) unsigned char lds_raw[];
    PrepLds<kSplit> &L = *(PrepLds<kSplit> *)lds_raw;
    constexpr int kIn = PrepLds<kSplit>::kIn;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int r16 = lane & 15;
    const int sl = lane >> 4;

    // the record parts this workgroup forms (uniform); grid slot: value
    // head x, or x + Hv for the U part of a split pair
    const bool u_only = kSplit && blockIdx.x >= p.value_heads;
    const bool kW = !u_only, kU = !kSplit || u_only;
    const uint32_t x = u_only ? blockIdx.x - p.value_heads : blockIdx.x;
    const uint32_t h = head_of_slot(x, p.key_heads, p.value_heads / p.key_heads);
    const uint32_t c = blockIdx.y;
    const GdnMeta m = p.meta[blockIdx.z];
    const uint32_t nchunks = (m.rows + kCk - 1) / kCk;
    if (c >= nchunks) return;
    const uint32_t r0 = c * kCk;
    const uint32_t nv = min((uint32_t)kCk, m.rows - r0);
    float *rec = p.chunk_rec + ((size_t)(m.chunk0 + c) * p.value_heads + h) * kRecFloats;
    const uint32_t groups = p.value_heads / p.key_heads;
    const uint32_t kh = h / groups;
    const uint32_t key_width = p.key_heads * kDk;
    const uint32_t K1 = p.conv_k - 1;
    const bool bf16_in = p.bf16_in != 0;
    constexpr int KC = Conv::kK;  // 0: run-time kernel size
    const int Kr = KC ? KC : (int)p.conv_k;

    // the staged channels, in order: q, k, v (whole record); q, k (W part);
    // k, v (U part); the global channel of staged channel lc
    auto chan = [&](int lc) -> uint32_t {
        const uint32_t qch = kh * kDk, kch = key_width + kh * kDk, vch = 2 * key_width + h * kHeadDv;
        if (u_only) return lc < kDk ? kch + lc : vch + (lc - kDk);
        return lc < kDk ? qch + lc : lc < 2 * kDk ? kch + (lc - kDk) : vch + (lc - 2 * kDk);
    };
    // conv work of this thread (row ranges wave-uniform): channel lc of the
    // first 256 over rows 16 half .. + 15; for the whole record also v channel vch
    // over rows 8 vquart .. + 7
    const int lc = tid & (2 * kDk - 1);
    const int half = tid >> 8;
    const int vch = tid & (kHeadDv - 1);
    const int vquart = tid >> 7;
    const uint32_t ch0 = chan(lc);
    const uint32_t ch1 = chan(2 * kDk + vch);  // used for the whole record only
    const size_t hist_slot = ((size_t)m.parity * p.max_slots + m.slot) * p.channels;
    const size_t hist_next = ((size_t)(1 - m.parity) * p.max_slots + m.slot) * p.channels;
    // weights and the stored history (used by the rows that start the call;
    // the others take the K-1 inputs before them from the staged rows)
    Conv cv0, cvv;
    cv0.load(p.history + (hist_slot + ch0) * K1, p.conv_w + (size_t)ch0 * p.conv_k, p.conv_k);
    if constexpr (!kSplit) {
        cvv.load(p.history + (hist_slot + ch1) * K1, p.conv_w + (size_t)ch1 * p.conv_k, p.conv_k);
    }

    // decay and write strength inputs first: wave 1 turns them into g and
    // beta while the raw inputs below are in flight
    const int cvl = lane & 31;
    float av = 0.0f, bv = 0.0f;
    {
        const size_t row = (size_t)m.row0 + r0 + min((uint32_t)cvl, nv - 1);
        av = load_act_nb(p.a, row * p.value_heads + h, bf16_in);
        bv = load_act_nb(p.b, row * p.value_heads + h, bf16_in);
    }
    const float a_log_e = expf(p.a_log[h]);
    const float dt_bias = p.dt_bias[h];
    auto decay_and_strength = [&]() __attribute__((always_inline)) {
        if (wave == 1) {
            // math.rs:220-221; padded rows: alpha 1, beta 0
            const bool valid = (uint32_t)cvl < nv;
            float la = valid ? -a_log_e * softplus_ref(av + dt_bias) : 0.0f;
            const float beta = valid ? ref_sigmoid(bv) : 0.0f;
#pragma unroll
            for (int o = 1; o < kCk; o <<= 1) {
                const float y = __shfl_up(la, o);
                if (cvl >= o) la += y;
            }
            if (lane < kCk) {
                L.g[lane] = la;
                L.beta[lane] = beta;
            }
        }
    };
    // ---- raw inputs: rows r0 - kPre .. r0 + kCk - 1 of the sequence, clamped
    //      into its rows (clamped copies are never used), in 16-byte segments
    //      of the staged channel ranges, every load in flight together
    {
        uint32_t lt = tid;
        pin(lt);
        auto seg_src = [&](int rr, int c0) -> size_t {
            const int row = min(max((int)r0 - kPre + rr, 0), (int)m.rows - 1);
            return ((size_t)m.row0 + row) * p.channels + chan(c0);
        };
        constexpr int R = kPre + kCk;
        if (!bf16_in) {
            constexpr int SEG = kIn / 4;
            constexpr int N = (R * SEG + kPrepThreads - 1) / kPrepThreads;
            f32x4 xs[N];
#pragma unroll
            for (int n = 0; n < N; ++n) {
                const int e = min((int)lt + n * kPrepThreads, R * SEG - 1);
                xs[n] = *(const f32x4 *)((const float *)p.qkv + seg_src(e / SEG, 4 * (e % SEG)));
            }
            decay_and_strength();
#pragma unroll
            for (int n = 0; n < N; ++n) {
                const int e = (int)lt + n * kPrepThreads;
                if (e < R * SEG) *(f32x4 *)&L.xin[e / SEG][4 * (e % SEG)] = xs[n];
            }
        } else {
            constexpr int SEG = kIn / 8;
            constexpr int N = (R * SEG + kPrepThreads - 1) / kPrepThreads;
            u32x4 xs[N];
#pragma unroll
            for (int n = 0; n < N; ++n) {
                const int e = min((int)lt + n * kPrepThreads, R * SEG - 1);
                xs[n] = *(const u32x4 *)((const uint16_t *)p.qkv + seg_src(e / SEG, 8 * (e % SEG)));
            }
            decay_and_strength();
#pragma unroll
            for (int n = 0; n < N; ++n) {
                const int e = (int)lt + n * kPrepThreads;
                if (e < R * SEG) {
                    float *dst = &L.xin[e / SEG][8 * (e % SEG)];
                    *(f32x4 *)dst = f32x4{__uint_as_float(xs[n][0] << 16), __uint_as_float(xs[n][0] & 0xffff0000u),
                                          __uint_as_float(xs[n][1] << 16), __uint_as_float(xs[n][1] & 0xffff0000u)};
                    *(f32x4 *)(dst + 4) = f32x4{__uint_as_float(xs[n][2] << 16), __uint_as_float(xs[n][2] & 0xffff0000u),
                                                __uint_as_float(xs[n][3] << 16), __uint_as_float(xs[n][3] & 0xffff0000u)};
                }
            }
        }
    }
    __syncthreads();
    // ---- causal conv + silu (math.rs:158-187); rows past nv are zero and do
    //      not advance the history
    const bool last_chunk = c + 1 == nchunks;
    if (c > 0 || half == 1) cv0.set_hist(&L.xin[kPre + 16 * half - (Kr - 1)][lc], kIn, p.conv_k);
    {
        const int tb = 16 * half;
        float xr[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) xr[i] = L.xin[kPre + tb + i][lc];
        float yr[16];
        if (tb + 16 <= (int)nv) {
#pragma unroll
            for (int i = 0; i < 16; ++i) yr[i] = fast_silu(cv0.pre(xr[i], p.conv_k));
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                yr[i] = 0.0f;
                if ((uint32_t)(tb + i) < nv) yr[i] = fast_silu(cv0.pre(xr[i], p.conv_k));
            }
        }
        // first range q (k for the U part), second range k (v for the U part)
        const bool is_k = u_only ? lc < kDk : lc >= kDk;  // wave-uniform
        const int d = lc & (kDk - 1);
        if (is_k) {
#pragma unroll
            for (int i = 0; i < 16; ++i) L.k[tb + i][d] = yr[i];
#pragma unroll
            for (int i = 0; i < 16; i += 4) {
                *(f32x4 *)&L.kc[d][tb + i] = f32x4{yr[i], yr[i + 1], yr[i + 2], yr[i + 3]};
            }
        } else if (!u_only) {
#pragma unroll
            for (int i = 0; i < 16; ++i) L.qv.q[tb + i][d] = yr[i];
        } else {
#pragma unroll
            for (int i = 0; i < 16; i += 4) {
                *(f32x4 *)&L.qv.vc[d][tb + i] = f32x4{yr[i], yr[i + 1], yr[i + 2], yr[i + 3]};
            }
        }
        // the history after the call: the last K-1 raw inputs, from the last
        // chunk, by the threads that hold the last row; q/k channels only in
        // the key head's first value head (a U part writes only its v channels)
        const bool writes = u_only ? lc >= kDk : h % groups == 0;
        if (last_chunk && half == (nv > 16 ? 1 : 0) && writes) {
            cv0.store(p.history + (hist_next + ch0) * K1, p.conv_k);
        }
    }
    if constexpr (!kSplit) {
        if (c > 0 || vquart > 0) {
            cvv.set_hist(&L.xin[kPre + 8 * vquart - (Kr - 1)][2 * kDk + vch], kIn, p.conv_k);
        }
        const int tb = 8 * vquart;
        float xr[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) xr[i] = L.xin[kPre + tb + i][2 * kDk + vch];
        float yv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            yv[i] = 0.0f;
            if ((uint32_t)(tb + i) < nv) yv[i] = fast_silu(cvv.pre(xr[i], p.conv_k));
        }
        *(f32x4 *)&L.qv.vc[vch][tb] = f32x4{yv[0], yv[1], yv[2], yv[3]};
        *(f32x4 *)&L.qv.vc[vch][tb + 4] = f32x4{yv[4], yv[5], yv[6], yv[7]};
        if (last_chunk && vquart == (int)(nv - 1) / 8) cvv.store(p.history + (hist_next + ch1) * K1, p.conv_k);
    }
    __syncthreads();
    // ---- L2 norms per row (math.rs:218-219): 16 lanes per row, 8 dims each,
    //      a reduction over the 16; then the row's scales
    {
        const int t = 4 * wave + (lane >> 4), part = lane & 15;
        float sq = 0.0f, sk = 0.0f;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const float4 b4 = *(const float4 *)&L.k[t][8 * part + 4 * i];
            sk += b4.x * b4.x + b4.y * b4.y + b4.z * b4.z + b4.w * b4.w;
            if (kW) {
                const float4 a4 = *(const float4 *)&L.qv.q[t][8 * part + 4 * i];
                sq += a4.x * a4.x + a4.y * a4.y + a4.z * a4.z + a4.w * a4.w;
            }
        }
        sk = sum16(sk);
        if (kW) sq = sum16(sq);
        if (part == 0) {
            const float rk = 1.0f / sqrtf(sk + 1e-6f);
            const float gt = L.g[t], bt = L.beta[t];
            L.rk[t] = rk;
            if (kW) {
                // Qe's row scale e^{g_t} / |q_t|; W's column scale of T,
                // beta_j e^{g_j} / |k_j|
                const float rq = 1.0f / sqrtf(sq + 1e-6f);
                L.rq[t] = rq;
                L.qs[t] = rq * fast_exp(gt);
                L.sw[t] = bt * fast_exp(gt) * rk;
            }
            if (kU) {
                // U's column scale beta_j; Ks's e^{g_C - g_j} / |k_j|
                L.su[t] = bt;
                L.ss[t] = fast_exp(L.g[kCk - 1] - gt) * rk;
            }
        }
    }
    __syncthreads();
    // ---- P1: the k.k tiles (0,0), (1,0), (1,1) -> A on waves 0..2.  With W:
    //      the q.k tiles too, wave 3 (0,0) -> Pm (and Pm's zero tile (0,1)),
    //      waves 4..7 halves over k of (1,0) (waves 4, 6) and (1,1) (5, 7),
    //      the second halves handed over in LDS, so every SIMD runs 48 MFMAs;
    //      waves 4..7 then write Qe (and with U, Ks).  U alone: waves 3..7
    //      write Ks.
    f32x4 acc = {0, 0, 0, 0}, acc2 = {0, 0, 0, 0};
    const int p1_tile = wave < 3 ? wave : wave == 3 ? 0 : 1 + (wave & 1);
    const int p1_tr = p1_tile == 0 ? 0 : 1, p1_tc = p1_tile == 2 ? 1 : 0;
    auto write_ks = [&](int first, int stride) __attribute__((always_inline)) {
        // Ks[d][j] = k[d][j] e^{g_C - g_j} / |k_j|
        for (int e = first; e < kDk * kCk / 4; e += stride) {
            const int d = e >> 3, j = 4 * (e & 7);
            __builtin_nontemporal_store(*(const f32x4 *)&L.kc[d][j] * *(const f32x4 *)&L.ss[j],
                                        (f32x4 *)(rec + kRecKs + d * kCk + j));
        }
    };
    if (wave < 3 || kW) {
        const float *arow = wave < 3 ? &L.k[16 * p1_tr][0] : &L.qv.q[16 * p1_tr][0];
        constexpr int NH = kDk / 32;
        // k range: both halves (waves 0..3), the first (4, 5) or second (6, 7)
        const int h0 = wave < 6 ? 0 : 1, h1 = wave < 4 ? 2 : h0 + 1;
        for (int hh = h0; hh < h1; ++hh) {
            Ops<NH> xa, kb;
            load_ops(xa, arow + NH * 16 * hh, kPr, lane);
            load_ops(kb, &L.k[16 * p1_tc][NH * 16 * hh], kPr, lane);
#pragma unroll
            for (int st = 0; st < NH; ++st) {
                acc = mfma4(xa.v[st].x, kb.v[st].x, acc);
                acc2 = mfma4(xa.v[st].y, kb.v[st].y, acc2);
                acc = mfma4(xa.v[st].z, kb.v[st].z, acc);
                acc2 = mfma4(xa.v[st].w, kb.v[st].w, acc2);
            }
        }
        acc += acc2;
    }
    if (wave < 3 || (kW && wave == 3)) {
        const int j = 16 * p1_tc + r16;
        const float gj = L.g[j], rkj = L.rk[j];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = 16 * p1_tr + 4 * sl + i;
            const float e = j <= t ? fast_exp(L.g[t] - gj) : 0.0f;
            if (wave < 3) {
                L.a[t][j] = j < t ? L.beta[t] * e * L.rk[t] * rkj * acc[i] : 0.0f;
            } else {
                rec[kRecPm + t * kCk + j] = e * L.rq[t] * rkj * acc[i];
                rec[kRecPm + t * kCk + 16 + r16] = 0.0f;
            }
        }
    } else if (kW) {
        if (wave >= 6) L.part[wave & 1][lane] = acc;
        const int u = tid - 4 * 64;  // 0..255
#pragma unroll
        for (int n = 0; n < 4; ++n) {
            // Qe = diag(e^{g_t} / |q_t|) Q
            const int e = u + n * 256;
            const int t = e >> 5, d = 4 * (e & 31);
            __builtin_nontemporal_store(*(const f32x4 *)&L.qv.q[t][d] * L.qs[t],
                                        (f32x4 *)(rec + kRecQe + t * kDk + d));
        }
        if (kU) write_ks(u, 256);
    } else {
        write_ks(tid - 3 * 64, kPrepThreads - 3 * 64);
    }
    __syncthreads();
    // ---- P2: T = (I + A)^-1.  Waves 0 and 1 invert the diagonal 16 x 16
    //      blocks by forward substitution (lane j: column j), storing T and
    //      its transpose; wave 2 clears the upper-right block; wave 3 writes
    //      e^{g_C} (with U); waves 4 and 5 finish their Pm tiles (with W).
    if (wave < 2) {
        const int b0 = 16 * wave;
        const int j = r16;
        f32x4 ar[16][4];
#pragma unroll
        for (int i = 1; i < 16; ++i)
#pragma unroll
            for (int qd = 0; 4 * qd < i; ++qd) ar[i][qd] = *(const f32x4 *)&L.a[b0 + i][b0 + 4 * qd];
        float xv[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float acc0 = i == j ? 1.0f : 0.0f, acc1 = 0.0f;
#pragma unroll
            for (int mm = 0; mm < i; ++mm) {
                const float am = ar[i][mm >> 2][mm & 3];
                if (mm & 1) acc1 -= am * xv[mm];
                else acc0 -= am * xv[mm];
            }
            xv[i] = acc0 + acc1;
        }
        if (lane < 16) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                L.t[b0 + i][b0 + j] = xv[i];
                L.tt[b0 + j][b0 + i] = xv[i];
            }
        }
    } else if (wave == 2) {
        for (int e = lane; e < 256; e += 64) L.t[e >> 4][16 + (e & 15)] = 0.0f;
    } else if (wave == 3) {
        if (kU && lane == 0) rec[kRecEc] = expf(L.g[kCk - 1]);
    } else if (wave < 6 && kW) {
        acc += L.part[wave & 1][lane];
        const int j = 16 * p1_tc + r16;
        const float gj = L.g[j], rkj = L.rk[j];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = 16 * p1_tr + 4 * sl + i;
            const float e = j <= t ? fast_exp(L.g[t] - gj) : 0.0f;
            rec[kRecPm + t * kCk + j] = e * L.rq[t] * rkj * acc[i];
        }
    }
    __syncthreads();
    //      T21 = -T22 A21 T11 (wave 0): M = A21 T11 with B = T11^T rows, M^T
    //      through LDS, then T21 = -T22 M.
    if (wave == 0) {
        Ops<1> a21, t11t;
        load_ops(a21, &L.a[16][0], kPc, lane);
        load_ops(t11t, &L.tt[0][0], kPc, lane);
        f32x4 mt = {0, 0, 0, 0};
        mma(mt, a21, t11t);
#pragma unroll
        for (int i = 0; i < 4; ++i) L.tt[16 + r16][4 * sl + i] = mt[i];  // M^T
        Ops<1> t22, mtr;
        load_ops(t22, &L.t[16][16], kPc, lane);
        load_ops(mtr, &L.tt[16][0], kPc, lane);
        f32x4 t21 = {0, 0, 0, 0};
        mma(t21, t22, mtr);
#pragma unroll
        for (int i = 0; i < 4; ++i) L.t[16 + 4 * sl + i][r16] = -t21[i];
    }
    __syncthreads();
    // ---- P3: W = T diag(sw) K (stored negated) and U = T diag(su) V, those
    //      of this mode; wave w owns rows 16 (w & 1).. and columns
    //      32 (w >> 1) .. + 31
    {
        const int tr = wave & 1, c0 = 32 * (wave >> 1);
        auto product = [&](const float *scale, const float (*rows)[kPc], float *dst, float sign)
                           __attribute__((always_inline)) {
            Ops<2> ta;
            load_ops(ta, &L.t[16 * tr][0], kPc, lane);
            scale_ops(ta, scale, lane);
            Ops<2> xb[2];
#pragma unroll
            for (int n = 0; n < 2; ++n) load_ops(xb[n], &rows[c0 + 16 * n][0], kPc, lane);
            f32x4 o[2] = {{0, 0, 0, 0}, {0, 0, 0, 0}};
#pragma unroll
            for (int st = 0; st < 2; ++st)
#pragma unroll
                for (int e = 0; e < 4; ++e)
#pragma unroll
                    for (int n = 0; n < 2; ++n) o[n] = mfma4(ta.v[st][e], xb[n].v[st][e], o[n]);
#pragma unroll
            for (int n = 0; n < 2; ++n)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int t = 16 * tr + 4 * sl + i, col = c0 + 16 * n + r16;
                    __builtin_nontemporal_store(sign * o[n][i], dst + t * kDk + col);
                }
        };
        if (kW) product(L.sw, L.kc, rec + kRecWn, -1.0f);
        if (kU) product(L.su, L.qv.vc, rec + kRecU, 1.0f);
    }
}

// The scan over a sequence's chunks for one 32-row slice of a value head's
// state, 8 waves: waves 0..3 own the output tiles (rows 16 (w >> 1)..,
// state rows 16 (w & 1)..), waves 4..7 the Delta tiles of the same places
// and then the state-update tiles (state rows 16 ((w - 4) >> 1)..,
// dims 64 ((w - 4) & 1)..), so each SIMD runs one wave of each kind and the
// same MFMA count in both phases.  Each chunk's record (Qe, -W, Pm, Ks and
// this slice's U columns) is staged once per workgroup into LDS,
// double-buffered: the loads for chunk c + 1 are issued into registers at
// the start of chunk c and written to the other buffer at its end, so they
// have a whole chunk to land.  xcd_map: the grid is ordered so that the four
// slices of a (sequence, value head) get workgroup ids 8 apart, which the
// dispatcher places on one XCD, so they share its L2 for the record.
__global__ void __launch_bounds__(kScanThreads) gdn_chunk_scan_kernel(const GdnParams p,
                                                                      uint32_t xcd_map) {
    extern __shared__ __align__(16) unsigned char lds_raw[];
    ScanLds &L = *(ScanLds *)lds_raw;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int r16 = lane & 15;
    const int sl = lane >> 4;
    const bool out_wave = wave < 4;  // wave-uniform role
    const int tr = (wave & 3) >> 1, tc = wave & 1;

    constexpr uint32_t nq = kHeadDv / kVs;  // slices per head
    const uint32_t b = blockIdx.x;
    uint32_t pair, vq;
    if (xcd_map) {
        vq = (b >> 3) % nq;
        pair = ((b >> 3) / nq) * 8 + (b & 7);
    } else {
        vq = b % nq;
        pair = b / nq;
    }
    const uint32_t h = head_of_slot(pair % p.value_heads, p.key_heads, p.value_heads / p.key_heads);
    const GdnMeta m = p.meta[pair / p.value_heads];
    const uint32_t nchunks = (m.rows + kCk - 1) / kCk;
    const float qscale = 1.0f / sqrtf((float)kDk);  // math.rs:234-235

    // record staging: 7 16-byte segments per thread; segment e = tid + 512 n
    // is in Qe (n < 2), -W (n < 4), Ks (n < 6), then Pm (waves 0..3) or U
    constexpr int kSeg = 7;
    auto rec_of = [&](uint32_t c) -> const float * {
        return p.chunk_rec + ((size_t)(m.chunk0 + c) * p.value_heads + h) * kRecFloats;
    };
    const int t2 = tid & 255;
    auto fetch = [&](const float *rec, f32x4 (&xs)[kSeg]) __attribute__((always_inline)) {
#pragma unroll
        for (int n = 0; n < kSeg; ++n) {
            const int e = tid + kScanThreads * (n & 1);
            int src;
            if (n < 2) src = kRecQe + (e >> 5) * kDk + 4 * (e & 31);
            else if (n < 4) src = kRecWn + (e >> 5) * kDk + 4 * (e & 31);
            else if (n < 6) src = kRecKs + (e >> 3) * kCk + 4 * (e & 7);
            else if (out_wave) src = kRecPm + (t2 >> 3) * kCk + 4 * (t2 & 7);
            else src = kRecU + (t2 >> 3) * kHeadDv + vq * kVs + 4 * (t2 & 7);
            xs[n] = *(const f32x4 *)(rec + src);
        }
    };
    auto put = [&](ScanLds::Rec &r, const f32x4 (&xs)[kSeg]) __attribute__((always_inline)) {
#pragma unroll
        for (int n = 0; n < kSeg; ++n) {
            const int e = tid + kScanThreads * (n & 1);
            float *dst;
            if (n < 2) dst = &r.qe[e >> 5][4 * (e & 31)];
            else if (n < 4) dst = &r.wn[e >> 5][4 * (e & 31)];
            else if (n < 6) dst = &r.ks[e >> 3][4 * (e & 7)];
            else if (out_wave) dst = &r.pm[t2 >> 3][4 * (t2 & 7)];
            else dst = &r.u[t2 >> 3][4 * (t2 & 7)];
            *(f32x4 *)dst = xs[n];
        }
    };
    f32x4 xs[kSeg];
    fetch(rec_of(0), xs);
    float *state = p.state + (((size_t)m.state_in * p.value_heads + h) * kHeadDv + vq * kVs) * kDk;
    {
        const int v = tid >> 4, d0 = (tid & 15) * 4;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            *(float4 *)&L.s0[v][d0 + 64 * i] = *(const float4 *)(state + (size_t)v * kDk + d0 + 64 * i);
        }
    }
    put(L.r[0], xs);
    if (nchunks > 1) fetch(rec_of(1), xs);
    __syncthreads();
    for (uint32_t c = 0; c < nchunks; ++c) {
        const uint32_t r0 = c * kCk;
        const uint32_t nv = min((uint32_t)kCk, m.rows - r0);
        ScanLds::Rec &R = L.r[c & 1];
        // phase 1, tile (rows 16 tr.., state rows 16 tc..): output waves
        // Qe S0^T, Delta waves U + (-W) S0^T
        Ops<kDk / 16> xa, sb;
        load_ops(xa, out_wave ? &R.qe[16 * tr][0] : &R.wn[16 * tr][0], kPr, lane);
        load_ops(sb, &L.s0[16 * tc][0], kPr, lane);
        f32x4 acc = {0, 0, 0, 0}, acc2 = {0, 0, 0, 0};
        if (!out_wave) {
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = R.u[16 * tr + 4 * sl + i][16 * tc + r16];
        }
#pragma unroll
        for (int st = 0; st < kDk / 16; ++st)
#pragma unroll
            for (int e = 0; e < 4; e += 2) {
                acc = mfma4(xa.v[st][e], sb.v[st][e], acc);
                acc2 = mfma4(xa.v[st][e + 1], sb.v[st][e + 1], acc2);
            }
        acc += acc2;
        if (!out_wave) {
#pragma unroll
            for (int i = 0; i < 4; ++i) L.dt[16 * tc + r16][16 * tr + 4 * sl + i] = acc[i];
        }
        __syncthreads();
        if (out_wave) {
            // o += Pm Delta
            Ops<2> pa, db;
            load_ops(pa, &R.pm[16 * tr][0], kPc, lane);
            load_ops(db, &L.dt[16 * tc][0], kPc, lane);
            mma(acc, pa, db);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t t = 16 * tr + 4 * sl + i;
                if (t < nv) {
                    p.raw_out[((size_t)m.row0 + r0 + t) * p.value_heads * kHeadDv + (size_t)h * kHeadDv +
                              vq * kVs + 16 * tc + r16] = acc[i] * qscale;
                }
            }
        } else {
            // S_C = e^{g_C} S0 + Delta^T Ks^T over state rows 16 tr.., dims 64 tc..
            const float eC = p.chunk_rec[((size_t)(m.chunk0 + c) * p.value_heads + h) * kRecFloats + kRecEc];
            Ops<2> da;
            load_ops(da, &L.dt[16 * tr][0], kPc, lane);
            Ops<2> kb4[4];
#pragma unroll
            for (int n = 0; n < 4; ++n) load_ops(kb4[n], &R.ks[64 * tc + 16 * n][0], kPc, lane);
            float s0v[4][4];
#pragma unroll
            for (int n = 0; n < 4; ++n)
#pragma unroll
                for (int i = 0; i < 4; ++i) s0v[n][i] = L.s0[16 * tr + 4 * sl + i][64 * tc + 16 * n + r16];
            f32x4 s4[4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
#pragma unroll
            for (int st = 0; st < 2; ++st)
#pragma unroll
                for (int e = 0; e < 4; ++e)
#pragma unroll
                    for (int n = 0; n < 4; ++n) s4[n] = mfma4(da.v[st][e], kb4[n].v[st][e], s4[n]);
            // each of these waves rewrites exactly the S0 elements it read
            // into s0v; all other reads of S0 ended before the barrier above
#pragma unroll
            for (int n = 0; n < 4; ++n)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    L.s0[16 * tr + 4 * sl + i][64 * tc + 16 * n + r16] = s4[n][i] + eC * s0v[n][i];
                }
        }
        // the next chunk's record into the other buffer (last read in the
        // previous chunk), and the loads for the one after
        if (c + 1 < nchunks) {
            put(L.r[(c + 1) & 1], xs);
            if (c + 2 < nchunks) fetch(rec_of(c + 2), xs);
        }
        __syncthreads();  // the next chunk reads S0, its record, and rewrites dt
    }
    {
        const int v = tid >> 4, d0 = (tid & 15) * 4;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            *(float4 *)(state + (size_t)v * kDk + d0 + 64 * i) = *(const float4 *)&L.s0[v][d0 + 64 * i];
        }
    }
}

template <class Conv, bool kSplit>
hipError_t launch_chunk_prep(hipStream_t stream, const GdnParams &p, uint32_t max_chunks) {
    // once per instantiation (a thread-safe static initialiser): its LDS is
    // above the default limit
    static const hipError_t configured = hipFuncSetAttribute(
        (const void *)gdn_chunk_prep_kernel<Conv, kSplit>,
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)sizeof(PrepLds<kSplit>));
    if (configured != hipSuccess) return configured;
    SR_LAUNCH("gdn_chunk_prep_kernel", (gdn_chunk_prep_kernel<Conv, kSplit>),
              dim3((kSplit ? 2 : 1) * p.value_heads, max_chunks, p.nseq), dim3(kPrepThreads),
              sizeof(PrepLds<kSplit>), stream, p);
    return hipGetLastError();
}

// records: the launch's (chunk, value head) pairs; the prep takes two
// workgroups per record when that still fits the CUs
hipError_t launch_chunk(hipStream_t stream, const GdnParams &p, uint32_t max_chunks,
                        uint64_t records, int num_cus) {
    const bool split = 2 * records <= (uint64_t)(num_cus > 0 ? num_cus : 1);
    hipError_t e;
    if (p.conv_k == 4) {
        e = split ? launch_chunk_prep<ConvK<4>, true>(stream, p, max_chunks)
                  : launch_chunk_prep<ConvK<4>, false>(stream, p, max_chunks);
    } else {
        e = split ? launch_chunk_prep<ConvChan, true>(stream, p, max_chunks)
                  : launch_chunk_prep<ConvChan, false>(stream, p, max_chunks);
    }
    if (e != hipSuccess) return e;
    const uint32_t pairs = p.nseq * p.value_heads;
    const uint32_t xcd_map = pairs % 8 == 0 ? 1u : 0u;
    static const hipError_t configured = hipFuncSetAttribute(
        (const void *)gdn_chunk_scan_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
        (int)sizeof(ScanLds));
    if (configured != hipSuccess) return configured;
    SR_LAUNCH("gdn_chunk_scan_kernel", gdn_chunk_scan_kernel, dim3(pairs * (kHeadDv / kVs)),
              dim3(kScanThreads), sizeof(ScanLds), stream, p, xcd_map);
    return hipGetLastError();
}

struct NormParams {
    const float *raw;   // [rows][Hv*Dv]
    const void *z;      // [rows][Hv*Dv]
    const float *norm;  // [Dv]
    float *out;
    uint32_t *err_word;
    uint32_t value_heads, value_dim, rows;
    float eps;
    int bf16_in;
    int pairs;          // value_dim 128 and z, norm, out aligned for 2-element accesses
};

// One wave per (row, value head): rms_norm without offset (math.rs:28-50),
// then x * silu(z) (native.rs:737-740).
__global__ void __launch_bounds__(256) gdn_norm_gate_kernel(const NormParams p) {
    const uint32_t wid = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (wid >= p.rows * p.value_heads) return;
    const size_t base = (size_t)wid * p.value_dim;
    if (p.pairs != 0) {
        // two adjacent dims per lane: one 8-byte load per input
        const uint32_t d = 2 * (uint32_t)lane;
        const float2 x = *(const float2 *)(p.raw + base + d);
        const float2 nw = *(const float2 *)(p.norm + d);
        float2 zz;
        if (p.bf16_in != 0) {
            const uint32_t zb = *(const uint32_t *)((const uint16_t *)p.z + base + d);
            zz = float2{__uint_as_float(zb << 16), __uint_as_float(zb & 0xffff0000u)};
        } else {
            zz = *(const float2 *)((const float *)p.z + base + d);
        }
        const float ss = sum64(x.x * x.x + x.y * x.y);
        const float variance = ss / 128.0f;
        if (!isfinite(variance) && lane == 0) atomicOr(p.err_word, kErrNonFiniteVariance);
        const float inv = 1.0f / sqrtf(variance + p.eps);
        *(float2 *)(p.out + base + d) = float2{x.x * inv * nw.x * (zz.x * ref_sigmoid(zz.x)),
                                               x.y * inv * nw.y * (zz.y * ref_sigmoid(zz.y))};
        return;
    }
    if (p.value_dim <= 4 * 64) {
        // every input of the row (raw, z, weights) is requested before the
        // reduction, so the kernel waits for one memory round trip, not two;
        // loads past value_dim read its last element and are not used
        const bool bf16_in = p.bf16_in != 0;
        float x[4], zz[4], nw[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t d = min((uint32_t)lane + 64 * i, p.value_dim - 1);
            x[i] = p.raw[base + d];
            zz[i] = load_act_nb(p.z, base + d, bf16_in);
            nw[i] = p.norm[d];
        }
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if ((uint32_t)lane + 64 * i < p.value_dim) ss += x[i] * x[i];
        }
        ss = sum64(ss);
        const float variance = ss / (float)p.value_dim;
        if (!isfinite(variance) && lane == 0) atomicOr(p.err_word, kErrNonFiniteVariance);
        const float inv = 1.0f / sqrtf(variance + p.eps);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t d = (uint32_t)lane + 64 * i;
            if (d < p.value_dim) p.out[base + d] = x[i] * inv * nw[i] * (zz[i] * ref_sigmoid(zz[i]));
        }
        return;
    }
    float ss = 0.0f;
    for (uint32_t d = lane; d < p.value_dim; d += 64) {
        const float x = p.raw[base + d];
        ss += x * x;
    }
    ss = sum64(ss);
    const float variance = ss / (float)p.value_dim;
    if (!isfinite(variance) && lane == 0) atomicOr(p.err_word, kErrNonFiniteVariance);
    const float inv = 1.0f / sqrtf(variance + p.eps);
    for (uint32_t d = lane; d < p.value_dim; d += 64) {
        const float zz = load_act_nb(p.z, base + d, p.bf16_in != 0);
        p.out[base + d] = p.raw[base + d] * inv * p.norm[d] * (zz * ref_sigmoid(zz));
    }
}

// ---------------------------------------------------------------------------
// gdn_generic_kernel: key and value widths the tuned kernels are not built
// for (key_dim other than 128, value_dim not a multiple of 16; up to
// kGdnMaxDim each).  One workgroup of 256 threads per (value head, sequence),
// token by token as math.rs:190-239: the head's conv channels (q and k of its
// key head, its v) and their history in LDS; the L2 norms of q and k; the
// delta rule with a wave per state row (lanes over the key dims, so every
// state access is a contiguous run of the row) in the order decay, predict,
// correct, read; the raw outputs go to raw_out for gdn_norm_gate_kernel.
// KEEP_ROWS records as gdn_head_kernel writes them.
// ---------------------------------------------------------------------------
constexpr int kGenThreads = 256;
constexpr uint32_t kGenKeysPerLane = kGdnMaxDim / 64;

// Sum over the 256 threads; every thread gets the total.  red holds 4 floats.
__device__ __forceinline__ float block_sum256(float x, float *red) {
    x = sum64(x);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
    __syncthreads();
    const float t = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return t;
}

__global__ void __launch_bounds__(kGenThreads) gdn_generic_kernel(const GdnParams p,
                                                                   uint32_t key_dim) {
    extern __shared__ float gsh[];
    const uint32_t Dk = key_dim, Dv = p.value_dim;
    const uint32_t K = p.conv_k, K1 = K - 1;
    const uint32_t hch = 2 * Dk + Dv;  // q, k and v channels of the head
    float *conv_s = gsh;               // [hch] the row's conv outputs
    float *hist_s = gsh + hch;         // [hch][K-1] raw inputs, oldest first
    __shared__ float red_s[4];
    __shared__ float qk_s[2];
    __shared__ float ab_s[2];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t h = blockIdx.x;
    const GdnMeta m = p.meta[blockIdx.y];
    const uint32_t groups = p.value_heads / p.key_heads;
    const uint32_t kh = h / groups;
    const uint32_t key_width = p.key_heads * Dk;
    const bool bf16_in = p.bf16_in != 0;
    auto chan = [&](uint32_t c) -> uint32_t {
        if (c < Dk) return kh * Dk + c;
        if (c < 2 * Dk) return key_width + kh * Dk + (c - Dk);
        return 2 * key_width + h * Dv + (c - 2 * Dk);
    };
    const size_t hist_slot = ((size_t)m.parity * p.max_slots + m.slot) * p.channels;
    const size_t hist_next = ((size_t)(1 - m.parity) * p.max_slots + m.slot) * p.channels;
    for (uint32_t c = tid; c < hch; c += kGenThreads) {
        for (uint32_t j = 0; j < K1; ++j) hist_s[c * K1 + j] = p.history[(hist_slot + chan(c)) * K1 + j];
    }
    const float a_log_e = expf(p.a_log[h]);
    const float dt = p.dt_bias[h];
    const float qscale = 1.0f / sqrtf((float)Dk);  // math.rs:213
    const float *s_in = p.state + ((size_t)m.state_in * p.value_heads + h) * Dv * Dk;
    float *s_out = p.state + ((size_t)m.state_out * p.value_heads + h) * Dv * Dk;
    const bool keep = p.records != nullptr;
    const uint32_t hv_dv = p.value_heads * Dv;
    const size_t rec_k = p.value_heads + hv_dv;                  // k^ [Hv][Dk]
    const size_t rec_x = rec_k + (size_t)p.value_heads * Dk;     // raw inputs [C]
    const bool owns_qk = (h % groups == 0);
    __syncthreads();

    for (uint32_t r = 0; r < m.rows; ++r) {
        const size_t row = (size_t)m.row0 + r;
        float *rec = keep ? p.records + ((size_t)m.slot * p.keep_rows + r) * p.rec_stride : nullptr;
        // A. causal conv + silu (math.rs:175-185), history shifted in LDS
        for (uint32_t c = tid; c < hch; c += kGenThreads) {
            const uint32_t ch = chan(c);
            const float x = load_act(p.qkv, row * p.channels + ch, bf16_in);
            const float *w = p.conv_w + (size_t)ch * K;
            float acc = 0.0f;
            for (uint32_t j = 0; j < K1; ++j) acc += hist_s[c * K1 + j] * w[j];
            const float value = acc + x * w[K1];
            conv_s[c] = value * ref_sigmoid(value);
            for (uint32_t j = 0; j + 1 < K1; ++j) hist_s[c * K1 + j] = hist_s[c * K1 + j + 1];
            if (K1 > 0) hist_s[c * K1 + K1 - 1] = x;
            if (keep && (c >= 2 * Dk || owns_qk)) rec[rec_x + ch] = x;
        }
        if (tid == 0) {
            // math.rs:220-221
            const float av = load_act(p.a, row * p.value_heads + h, bf16_in);
            const float bv = load_act(p.b, row * p.value_heads + h, bf16_in);
            ab_s[0] = expf(-a_log_e * softplus_ref(av + dt));
            ab_s[1] = ref_sigmoid(bv);
            if (keep) rec[h] = ab_s[0];
        }
        __syncthreads();
        // B. L2 norms of q and k (math.rs:218-219)
        float sq = 0.0f, sk = 0.0f;
        for (uint32_t d = tid; d < Dk; d += kGenThreads) {
            sq += conv_s[d] * conv_s[d];
            sk += conv_s[Dk + d] * conv_s[Dk + d];
        }
        sq = block_sum256(sq, red_s);
        sk = block_sum256(sk, red_s);
        if (tid == 0) {
            qk_s[0] = 1.0f / sqrtf(sq + 1e-6f);
            qk_s[1] = 1.0f / sqrtf(sk + 1e-6f);
        }
        __syncthreads();
        const float qi = qk_s[0], ki = qk_s[1];
        const float alpha = ab_s[0], beta = ab_s[1];
        float kh[kGenKeysPerLane], qh[kGenKeysPerLane];
#pragma unroll
        for (uint32_t i = 0; i < kGenKeysPerLane; ++i) {
            const uint32_t d = lane + 64 * i;
            kh[i] = d < Dk ? conv_s[Dk + d] * ki : 0.0f;
            qh[i] = d < Dk ? conv_s[d] * qi : 0.0f;
            if (keep && wave == 0 && d < Dk) rec[rec_k + (size_t)h * Dk + d] = kh[i];
        }
        // C. delta rule, a wave per state row (math.rs:222-236)
        const float *src = r == 0 ? s_in : s_out;
        for (uint32_t v = wave; v < Dv; v += kGenThreads / 64) {
            const float *srow = src + (size_t)v * Dk;
            float *drow = s_out + (size_t)v * Dk;
            float sv[kGenKeysPerLane];
            float pred = 0.0f;
#pragma unroll
            for (uint32_t i = 0; i < kGenKeysPerLane; ++i) {
                const uint32_t d = lane + 64 * i;
                sv[i] = d < Dk ? srow[d] * alpha : 0.0f;
                pred += sv[i] * kh[i];
            }
            pred = sum64(pred);
            const float corr = beta * (conv_s[2 * Dk + v] - pred);
            if (keep && lane == 0) rec[p.value_heads + (size_t)h * Dv + v] = corr;
            float rd = 0.0f;
#pragma unroll
            for (uint32_t i = 0; i < kGenKeysPerLane; ++i) {
                const uint32_t d = lane + 64 * i;
                sv[i] = fmaf(corr, kh[i], sv[i]);
                rd += sv[i] * qh[i];
                if (d < Dk) drow[d] = sv[i];
            }
            rd = sum64(rd);
            if (lane == 0) p.raw_out[row * hv_dv + (size_t)h * Dv + v] = rd * qscale;
        }
        __syncthreads();  // conv_s is rewritten by the next row
    }
    // next history: v channels here; q/k channels by the first value head of
    // the key group (the others hold the same values)
    for (uint32_t c = tid; c < hch; c += kGenThreads) {
        if (c < 2 * Dk && !owns_qk) continue;
        for (uint32_t j = 0; j < K1; ++j) p.history[(hist_next + chan(c)) * K1 + j] = hist_s[c * K1 + j];
    }
}

// gdn_rollback_kernel for the widths of gdn_generic_kernel: the state after
// row `keep` rebuilt with the forward's own operations (a product by the
// decay, then a fused multiply-add of the correction), a wave per state row.
struct RollbackGenericParams {
    RollbackParams r;
    uint32_t key_dim, value_dim;
};

__global__ void __launch_bounds__(256) gdn_rollback_generic_kernel(const RollbackGenericParams q) {
    const RollbackParams &p = q.r;
    const uint32_t Dk = q.key_dim, Dv = q.value_dim;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t hv_dv = p.value_heads * Dv;
    const size_t rec_k = p.value_heads + hv_dv;
    const size_t rec_x = rec_k + (size_t)p.value_heads * Dk;
    if (blockIdx.x < p.value_heads) {
        const uint32_t h = blockIdx.x;
        for (uint32_t v = wave; v < Dv; v += 4) {
            const float *src = p.state_in + ((size_t)h * Dv + v) * Dk;
            float *dst = p.state_out + ((size_t)h * Dv + v) * Dk;
            float sv[kGenKeysPerLane];
#pragma unroll
            for (uint32_t i = 0; i < kGenKeysPerLane; ++i) {
                const uint32_t d = lane + 64 * i;
                sv[i] = d < Dk ? src[d] : 0.0f;
            }
            for (uint32_t r = 0; r < p.keep; ++r) {
                const float *rec = p.records + (size_t)r * p.rec_stride;
                const float alpha = rec[h];
                const float corr = rec[p.value_heads + (size_t)h * Dv + v];
#pragma unroll
                for (uint32_t i = 0; i < kGenKeysPerLane; ++i) {
                    const uint32_t d = lane + 64 * i;
                    const float khd = d < Dk ? rec[rec_k + (size_t)h * Dk + d] : 0.0f;
                    sv[i] = fmaf(corr, khd, sv[i] * alpha);
                }
            }
#pragma unroll
            for (uint32_t i = 0; i < kGenKeysPerLane; ++i) {
                const uint32_t d = lane + 64 * i;
                if (d < Dk) dst[d] = sv[i];
            }
        }
        return;
    }
    const uint32_t c = (blockIdx.x - p.value_heads) * 256 + tid;
    const uint32_t K1 = p.conv_k - 1;
    if (c >= p.channels || K1 == 0) return;
    for (uint32_t i = 0; i < K1; ++i) {
        const uint32_t t = p.keep + i;
        p.hist_out[(size_t)c * K1 + i] =
            t < K1 ? p.hist_in[(size_t)c * K1 + t]
                   : p.records[(size_t)(t - K1) * p.rec_stride + rec_x + c];
    }
}

// Which kernels a call takes.  Decode-sized calls (at most kHeadKernelRows
// rows per sequence) run one workgroup per (sequence, value head) with the
// norm and gate fused, and so do KEEP_ROWS calls (records of every row).
// Longer calls with Dv = 128 take the chunked MFMA form, which reads the qkv
// rows in 16-byte segments; the rest the token-serial row-block kernel.
enum class GdnRoute { kHead, kChunk, kDelta, kGeneric };

GdnRoute gdn_route(const safetyraise_kernel_gdn_pool *pool, const GdnSeq *seqs, int nseq,
                   bool keep, bool qkv_aligned) {
    uint32_t max_rows = 0;
    for (int i = 0; i < nseq; ++i) max_rows = seqs[i].rows > max_rows ? seqs[i].rows : max_rows;
    if (pool->key_dim != kDk || pool->value_dim % kRows != 0) return GdnRoute::kGeneric;
    if (pool->value_dim == kHeadDv && (max_rows <= kHeadKernelRows || keep)) return GdnRoute::kHead;
    if (pool->value_dim == kHeadDv && qkv_aligned) return GdnRoute::kChunk;
    return GdnRoute::kDelta;
}

}  // namespace

size_t gdn_chunk_rec_bytes(const safetyraise_kernel_gdn_pool *pool, const GdnSeq *seqs, int nseq,
                           bool keep, bool qkv_aligned) {
    if (gdn_route(pool, seqs, nseq, keep, qkv_aligned) != GdnRoute::kChunk) return 0;
    size_t most = 0;
    for (int base = 0; base < nseq; base += kMetaPerLaunch) {
        size_t chunks = 0;
        for (int i = base; i < nseq && i < base + kMetaPerLaunch; ++i) {
            chunks += (seqs[i].rows + kCk - 1) / kCk;
        }
        most = chunks > most ? chunks : most;
    }
    return most * pool->value_heads * kRecFloats * sizeof(float);
}

hipError_t launch_gdn(hipStream_t stream, const GdnLaunch &g, const GdnSeq *seqs, int nseq,
                      uint32_t total_rows) {
    const auto *pool = g.pool;
    const GdnRoute route = gdn_route(pool, seqs, nseq, g.keep, ((uintptr_t)g.qkv & 15) == 0);
    if (g.keep && route != GdnRoute::kHead && route != GdnRoute::kGeneric) {
        return hipErrorInvalidValue;
    }
    const bool head_kernel = route == GdnRoute::kHead;
    const bool chunk_kernel = route == GdnRoute::kChunk;
    if (chunk_kernel && g.chunk_rec == nullptr) return hipErrorInvalidValue;
    for (int base = 0; base < nseq; base += kMetaPerLaunch) {
        const int n = (nseq - base) < kMetaPerLaunch ? (nseq - base) : kMetaPerLaunch;
        GdnParams p;
        p.state = pool->d_state;
        p.history = pool->d_history;
        p.qkv = g.qkv;
        p.a = g.a;
        p.b = g.b;
        p.a_log = g.a_log;
        p.dt_bias = g.dt_bias;
        p.conv_w = g.conv_w;
        p.raw_out = g.raw;
        p.records = g.keep ? g.records : nullptr;
        p.rec_stride = g.rec_stride;
        p.keep_rows = g.keep_rows;
        p.key_heads = pool->key_heads;
        p.value_heads = pool->value_heads;
        p.value_dim = pool->value_dim;
        p.conv_k = pool->conv_kernel;
        p.channels = pool->channels;
        p.max_slots = pool->max_sequences;
        p.bf16_in = g.bf16_in ? 1 : 0;
        p.nseq = (uint32_t)n;
        p.chunk_rec = g.chunk_rec;
        uint32_t chunks = 0, max_chunks = 0;
        for (int i = 0; i < n; ++i) {
            const GdnSeq &q = seqs[base + i];
            p.meta[i] = GdnMeta{q.slot, q.rows, q.row0, q.parity, q.state_in, q.state_out, chunks};
            const uint32_t nc = (q.rows + kCk - 1) / kCk;
            chunks += nc;
            max_chunks = nc > max_chunks ? nc : max_chunks;
        }
        if (head_kernel) {
            const dim3 grid(pool->value_heads, (uint32_t)n);
            if (p.conv_k == 4) {
                SR_LAUNCH("gdn_head_kernel", (gdn_head_kernel<kHeadThreads, ConvK<4>>), grid,
                          dim3(kHeadThreads), 0, stream, p, g.norm, g.z, g.out, g.err_word, g.eps);
            } else {
                SR_LAUNCH("gdn_head_kernel", (gdn_head_kernel<kHeadThreads, ConvChan>), grid,
                          dim3(kHeadThreads), 0, stream, p, g.norm, g.z, g.out, g.err_word, g.eps);
            }
        } else if (route == GdnRoute::kGeneric) {
            const uint32_t hch = 2 * pool->key_dim + pool->value_dim;
            const size_t lds = (size_t)hch * pool->conv_kernel * sizeof(float);
            SR_LAUNCH("gdn_generic_kernel", gdn_generic_kernel, dim3(pool->value_heads, (uint32_t)n),
                      dim3(kGenThreads), lds, stream, p, pool->key_dim);
        } else if (chunk_kernel) {
            const hipError_t e =
                launch_chunk(stream, p, max_chunks, (uint64_t)chunks * pool->value_heads, g.num_cus);
            if (e != hipSuccess) return e;
        } else {
            const uint32_t blocks = (uint32_t)n * pool->value_heads * (pool->value_dim / kRows);
            SR_LAUNCH("gdn_delta_kernel", gdn_delta_kernel, dim3(blocks), dim3(kThreads), 0, stream, p);
        }
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (head_kernel) return hipSuccess;
    NormParams q;
    q.raw = g.raw;
    q.z = g.z;
    q.norm = g.norm;
    q.out = g.out;
    q.err_word = g.err_word;
    q.value_heads = pool->value_heads;
    q.value_dim = pool->value_dim;
    q.rows = total_rows;
    q.eps = g.eps;
    q.bf16_in = g.bf16_in ? 1 : 0;
    const uintptr_t zmask = g.bf16_in ? 3 : 7;
    q.pairs = pool->value_dim == 128 && ((uintptr_t)g.z & zmask) == 0 &&
              (((uintptr_t)g.norm | (uintptr_t)g.out) & 7) == 0;
    const uint32_t waves = total_rows * pool->value_heads;
    SR_LAUNCH("gdn_norm_gate_kernel", gdn_norm_gate_kernel, dim3((waves + 3) / 4), dim3(256), 0,
              stream, q);
    return hipGetLastError();
}

hipError_t launch_gdn_rollback(hipStream_t stream, const GdnRollback &r) {
    RollbackParams p;
    p.state_in = r.state_in;
    p.state_out = r.state_out;
    p.hist_in = r.hist_in;
    p.hist_out = r.hist_out;
    p.records = r.records;
    p.rec_stride = r.rec_stride;
    p.keep = r.keep;
    p.value_heads = r.value_heads;
    p.channels = r.channels;
    p.conv_k = r.conv_k;
    const uint32_t blocks = r.value_heads + (r.channels + 255) / 256;
    if (r.key_dim == kDk && r.value_dim == kHeadDv) {
        SR_LAUNCH("gdn_rollback_kernel", gdn_rollback_kernel, dim3(blocks), dim3(256), 0, stream, p);
    } else {
        const RollbackGenericParams q{p, r.key_dim, r.value_dim};
        SR_LAUNCH("gdn_rollback_generic_kernel", gdn_rollback_generic_kernel, dim3(blocks),
                  dim3(256), 0, stream, q);
    }
    return hipGetLastError();
}

uint32_t gdn_key_dim() { return kDk; }
uint32_t gdn_row_block() { return kRows; }
uint32_t gdn_max_kernel() { return kMaxK; }

}  // namespace sr
