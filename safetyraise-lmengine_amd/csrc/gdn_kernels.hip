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
    uint32_t parity;  // history buffer holding the current history
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
    // silu(sum_{j<K-1} hist[j] * w[j] + x * w[K-1]), then append x
    __device__ __forceinline__ float step(float x, uint32_t K) {
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
        return value * ref_sigmoid(value);
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
    float *srow = p.state + (((size_t)m.slot * p.value_heads + h) * p.value_dim + v_row) * kDk +
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
constexpr int kHeadCh = 2 * kDk + kHeadDv;  // q, k and v channels of one head
constexpr int kHeadThreads = 512;

template <int NTH>
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
    const bool bf16_in = p.bf16_in != 0;

    const uint32_t h = blockIdx.x % p.value_heads;
    const GdnMeta m = p.meta[blockIdx.x / p.value_heads];
    const uint32_t groups = p.value_heads / p.key_heads;
    const uint32_t kh = h / groups;
    const uint32_t key_width = p.key_heads * kDk;
    const uint32_t K1 = p.conv_k - 1;
    const size_t width = (size_t)p.value_heads * kHeadDv;
    auto chan = [&](int c) -> uint32_t {
        if (c < kDk) return kh * kDk + c;
        if (c < 2 * kDk) return key_width + kh * kDk + (c - kDk);
        return 2 * key_width + h * kHeadDv + (c - 2 * kDk);
    };
    // this thread's conv channels: tid (if < 384), and tid + NTH when that is < 384
    const bool one = tid < kHeadCh;
    const bool two = tid + NTH < kHeadCh;
    const uint32_t ch0 = one ? chan(tid) : 0;
    const uint32_t ch1 = two ? chan(tid + NTH) : 0;

    const size_t hist_slot = ((size_t)m.parity * p.max_slots + m.slot) * p.channels;
    const size_t hist_next = ((size_t)(1 - m.parity) * p.max_slots + m.slot) * p.channels;
    // (all loads unconditional: a conditional load ends in a wait for every
    // load in flight; threads without a channel read channel 0 and ignore it)
    ConvChan cv0, cv1;
    cv0.load(p.history + (hist_slot + ch0) * K1, p.conv_w + (size_t)ch0 * p.conv_k, p.conv_k);
    cv1.load(p.history + (hist_slot + ch1) * K1, p.conv_w + (size_t)ch1 * p.conv_k, p.conv_k);
    // inputs of a row: qkv channels, z of this head (dims lane and lane + 64,
    // used by wave 0), a and b
    float x0 = 0.0f, x1 = 0.0f, z0 = 0.0f, z1 = 0.0f, av = 0.0f, bv = 0.0f;
    auto load_row = [&](size_t row) {
        x0 = load_act_nb(p.qkv, row * p.channels + ch0, bf16_in);
        x1 = load_act_nb(p.qkv, row * p.channels + ch1, bf16_in);
        z0 = load_act_nb(z, row * width + h * kHeadDv + lane, bf16_in);
        z1 = load_act_nb(z, row * width + h * kHeadDv + lane + 64, bf16_in);
        av = load_act_nb(p.a, row * p.value_heads + h, bf16_in);
        bv = load_act_nb(p.b, row * p.value_heads + h, bf16_in);
    };
    load_row(m.row0);
    // state rows v = (NTH/16) i + group, dims [8 l16, 8 l16 + 8); requested after
    // the (branchy) conv loads so that nothing waits for them before the
    // delta step itself
    float *sbase = p.state + ((size_t)m.slot * p.value_heads + h) * kHeadDv * kDk + l16 * 8;
    float S[RPG][8];
#pragma unroll
    for (int i = 0; i < RPG; ++i) {
        const float *src = sbase + (size_t)((NTH / 16) * i + group) * kDk;
        const float4 x0 = *(const float4 *)src;
        const float4 x1 = *(const float4 *)(src + 4);
        S[i][0] = x0.x; S[i][1] = x0.y; S[i][2] = x0.z; S[i][3] = x0.w;
        S[i][4] = x1.x; S[i][5] = x1.y; S[i][6] = x1.z; S[i][7] = x1.w;
    }
    const float a_log_e = expf(p.a_log[h]);
    const float dt = p.dt_bias[h];
    const float qscale = 1.0f / sqrtf((float)kDk);  // math.rs:213
    const float nw0 = norm[lane], nw1 = norm[lane + 64];
    __syncthreads();

    for (uint32_t r = 0; r < m.rows; ++r) {
        const size_t row = (size_t)m.row0 + r;
        // A. causal conv + silu (math.rs:175-185), history in registers
        if (one) conv_s[tid] = cv0.step(x0, p.conv_k);
        if (two) conv_s[tid + NTH] = cv1.step(x1, p.conv_k);
        if (tid == 0) {
            // math.rs:220-221
            ab_s[0] = expf(-a_log_e * softplus_ref(av + dt));
            ab_s[1] = ref_sigmoid(bv);
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
            kh8[j] = conv_s[kDk + l16 * 8 + j] * ki;
            qh8[j] = conv_s[l16 * 8 + j] * qi;
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
                float *dst = sbase + (size_t)v * kDk;
                *(float4 *)dst = make_float4(S[i][0], S[i][1], S[i][2], S[i][3]);
                *(float4 *)(dst + 4) = make_float4(S[i][4], S[i][5], S[i][6], S[i][7]);
            }
        }
        __syncthreads();
        // D. RMSNorm without offset (math.rs:28-50), then * silu(z)
        if (wave == 0) {
            const float o0 = out_s[lane], o1 = out_s[lane + 64];
            const float ss = sum64(o0 * o0 + o1 * o1);
            const float variance = ss / (float)kHeadDv;
            if (!isfinite(variance) && lane == 0) atomicOr(err_word, kErrNonFiniteVariance);
            const float inv = 1.0f / sqrtf(variance + eps);
            float *dst = out + row * width + h * kHeadDv;
            dst[lane] = o0 * inv * nw0 * (zc0 * ref_sigmoid(zc0));
            dst[lane + 64] = o1 * inv * nw1 * (zc1 * ref_sigmoid(zc1));
        }
    }

    // next history: v channels here; q/k channels by the first value head of
    // the key group (the others compute the same values)
    const bool owns_qk = (h % groups == 0);
    if (one && (tid >= 2 * kDk || owns_qk)) cv0.store(p.history + (hist_next + ch0) * K1, p.conv_k);
    if (two && (tid + NTH >= 2 * kDk || owns_qk)) cv1.store(p.history + (hist_next + ch1) * K1, p.conv_k);
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
};

// One wave per (row, value head): rms_norm without offset (math.rs:28-50),
// then x * silu(z) (native.rs:737-740).
__global__ void __launch_bounds__(256) gdn_norm_gate_kernel(const NormParams p) {
    const uint32_t wid = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (wid >= p.rows * p.value_heads) return;
    const size_t base = (size_t)wid * p.value_dim;
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

}  // namespace

hipError_t launch_gdn(hipStream_t stream, const GdnLaunch &g, const uint32_t *slots,
                      const uint32_t *rows, const uint32_t *row0, const uint32_t *parity, int nseq,
                      uint32_t total_rows) {
    const auto *pool = g.pool;
    // decode-sized calls (at most kHeadKernelRows rows per sequence) run one
    // workgroup per (sequence, value head) with the norm and gate fused;
    // longer chunks split each head's state rows over workgroups
    uint32_t max_rows = 0;
    for (int i = 0; i < nseq; ++i) max_rows = rows[i] > max_rows ? rows[i] : max_rows;
    const bool head_kernel = pool->value_dim == kHeadDv && max_rows <= kHeadKernelRows;
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
        p.key_heads = pool->key_heads;
        p.value_heads = pool->value_heads;
        p.value_dim = pool->value_dim;
        p.conv_k = pool->conv_kernel;
        p.channels = pool->channels;
        p.max_slots = pool->max_sequences;
        p.bf16_in = g.bf16_in ? 1 : 0;
        p.nseq = (uint32_t)n;
        for (int i = 0; i < n; ++i) {
            p.meta[i] = GdnMeta{slots[base + i], rows[base + i], row0[base + i], parity[base + i]};
        }
        if (head_kernel) {
            const uint32_t blocks = (uint32_t)n * pool->value_heads;
            hipLaunchKernelGGL(gdn_head_kernel<kHeadThreads>, dim3(blocks), dim3(kHeadThreads), 0,
                               stream, p, g.norm, g.z, g.out, g.err_word, g.eps);
        } else {
            const uint32_t blocks = (uint32_t)n * pool->value_heads * (pool->value_dim / kRows);
            hipLaunchKernelGGL(gdn_delta_kernel, dim3(blocks), dim3(kThreads), 0, stream, p);
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
    const uint32_t waves = total_rows * pool->value_heads;
    hipLaunchKernelGGL(gdn_norm_gate_kernel, dim3((waves + 3) / 4), dim3(256), 0, stream, q);
    return hipGetLastError();
}

uint32_t gdn_key_dim() { return kDk; }
uint32_t gdn_row_block() { return kRows; }
uint32_t gdn_max_kernel() { return kMaxK; }

}  // namespace sr
