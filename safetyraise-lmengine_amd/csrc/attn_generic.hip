// Attention for the head widths the tuned kernels are not built for: any
// head_dim other than 64, 128 and 256, up to kGenericMaxHeadDim.  The
// reference takes any width (src/model/math.rs:109-124); this path gives the
// same rows for those shapes on the same paged bf16 cache, in plain f32.
//
// Two kernels per call (Attention::forward's row loop, native.rs:615-645):
//   attn_generic_append_kernel  one wave per (new row, KV head): k RMSNorm
//                               (math.rs:28-50) and RoPE (math.rs:52-99),
//                               k and v rounded to bf16 into the row's page,
//                               non-finite values flagged (state.rs:56-58);
//   attn_generic_kernel         one wave per (new row, query head): q RMSNorm
//                               and RoPE in LDS, then causal_attention
//                               (math.rs:125-152) over the row's visible
//                               keys in tiles of 64 - lane j scores key j of
//                               the tile (a full dot product against the q
//                               row in LDS), online max and sum in f32 with
//                               natural exponentials as the reference uses,
//                               and P.V with a lane per output dim - then
//                               the Qwen3.5 gate and an f32 store.
// Every row is appended before any row attends; row i sees the context and
// rows 0..i, which is what the reference's append-then-attend loop gives.
#include "sr_device.hpp"

namespace sr {

namespace {

constexpr uint32_t kDimsPerLane = kGenericMaxHeadDim / 64;

struct GenericMeta {
    uint32_t slot, ctx, rows, row0;
};

struct GenericParams {
    uint16_t *k_pages;
    uint16_t *v_pages;
    const int32_t *page_table;
    const void *q;
    const void *k;
    const void *v;
    const float *q_norm;
    const float *k_norm;
    const int32_t *positions;
    float *out;
    uint32_t *err_word;
    uint64_t num_pages;
    uint32_t pages_per_seq;
    uint32_t page_tokens;
    uint32_t flags;
    uint32_t heads;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t rotary_dim;
    uint32_t mrope[3];
    float eps;
    uint32_t nseq;
    uint32_t row_base;  // first row of the sequences this launch's grid.y covers
    // theta^(2i/rotary_dim), the host's f32 powf as math.rs:90-91
    float denom[kGenericMaxHeadDim / 2];
    GenericMeta meta[kMetaPerLaunch];
};
static_assert(sizeof(GenericParams) <= 4096, "kernel arguments stay within 4 KiB");

// x (one head's D values in LDS, written by this wave) <- RMSNorm with
// weights w (+ norm_add), then rotate-half RoPE over the first rotary_dim
// values at the row's positions.  The workgroup is this one wave, so the
// barriers only order its own LDS accesses.
__device__ void norm_rope(float *x, const GenericParams &p, const float *w, size_t row,
                          uint32_t lane) {
    const uint32_t D = p.head_dim;
    if ((p.flags & SAFETYRAISE_MI355X_QK_NORM) != 0) {
        const float norm_add = (p.flags & SAFETYRAISE_MI355X_NORM_OFFSET) ? 1.0f : 0.0f;
        float ss = 0.0f;
        for (uint32_t d = lane; d < D; d += 64) ss += x[d] * x[d];
        ss = sum64(ss);
        const float variance = ss / (float)D;
        if (!isfinite(variance) && lane == 0) atomicOr(p.err_word, kErrNonFiniteVariance);
        const float inv = 1.0f / sqrtf(variance + p.eps);
        for (uint32_t d = lane; d < D; d += 64) x[d] = x[d] * inv * (w[d] + norm_add);
    }
    __syncthreads();
    const bool interleaved = (p.flags & SAFETYRAISE_MI355X_MROPE_INTERLEAVED) != 0;
    const int32_t *pos = p.positions + row * 3;
    const uint32_t half = p.rotary_dim / 2;
    for (uint32_t i = lane; i < half; i += 64) {
        const int axis = rope_axis(i, p.mrope, interleaved);
        const float angle = (float)pos[axis] / p.denom[i];
        float sn, cs;
        sincosf(angle, &sn, &cs);
        const float left = x[i];
        const float right = x[i + half];
        x[i] = left * cs - right * sn;
        x[i + half] = right * cs + left * sn;
    }
    __syncthreads();
}

// Element offset of token `tok` of a sequence in KV head kvh's pages.
__device__ __forceinline__ size_t token_base(const GenericParams &p, const int32_t *table,
                                             uint32_t kvh, uint32_t tok) {
    const int32_t page = table[tok / p.page_tokens];
    return (((size_t)kvh * p.num_pages + page) * p.page_tokens + tok % p.page_tokens) *
           p.head_dim;
}

// grid (KV head, row of the sequence, sequence), 64 threads
__global__ void __launch_bounds__(64) attn_generic_append_kernel(const GenericParams p) {
    extern __shared__ float xs[];
    const uint32_t kvh = blockIdx.x, r = p.row_base + blockIdx.y, s = blockIdx.z;
    const GenericMeta m = p.meta[s];
    if (r >= m.rows) return;
    const uint32_t D = p.head_dim, lane = threadIdx.x;
    const bool bf16_in = (p.flags & SAFETYRAISE_MI355X_INPUT_BF16) != 0;
    const size_t row = (size_t)m.row0 + r;
    const size_t kv_row = (row * p.kv_heads + kvh) * D;
    for (uint32_t d = lane; d < D; d += 64) xs[d] = load_act(p.k, kv_row + d, bf16_in);
    __syncthreads();
    norm_rope(xs, p, p.k_norm, row, lane);
    const int32_t *table = p.page_table + (size_t)m.slot * p.pages_per_seq;
    const size_t base = token_base(p, table, kvh, m.ctx + r);
    for (uint32_t d = lane; d < D; d += 64) {
        const float kk = xs[d];
        const float vv = load_act(p.v, kv_row + d, bf16_in);
        if (!isfinite(kk) || !isfinite(vv)) atomicOr(p.err_word, kErrNonFiniteKv);
        p.k_pages[base + d] = f32_to_bf16(kk);
        p.v_pages[base + d] = f32_to_bf16(vv);
    }
}

// grid (query head, row of the sequence, sequence), 64 threads
__global__ void __launch_bounds__(64) attn_generic_kernel(const GenericParams p) {
    extern __shared__ float sh[];
    const uint32_t D = p.head_dim;
    float *qs = sh;      // [D] the normalised, rotated q row
    float *ps = sh + D;  // [64] the tile's probabilities
    const uint32_t head = blockIdx.x, r = p.row_base + blockIdx.y, s = blockIdx.z;
    const GenericMeta m = p.meta[s];
    if (r >= m.rows) return;
    const uint32_t lane = threadIdx.x;
    const bool bf16_in = (p.flags & SAFETYRAISE_MI355X_INPUT_BF16) != 0;
    const bool gated = (p.flags & SAFETYRAISE_MI355X_GATED) != 0;
    const size_t row = (size_t)m.row0 + r;
    const size_t hs = gated ? 2 * (size_t)D : D;  // q values per head (query, then gate)
    const size_t q_off = (row * p.heads + head) * hs;
    for (uint32_t d = lane; d < D; d += 64) qs[d] = load_act(p.q, q_off + d, bf16_in);
    __syncthreads();
    norm_rope(qs, p, p.q_norm, row, lane);

    const float scale = 1.0f / sqrtf((float)D);  // math.rs:126
    const uint32_t kvh = head / (p.heads / p.kv_heads);  // math.rs:129
    const uint32_t n_keys = m.ctx + r + 1;
    const int32_t *table = p.page_table + (size_t)m.slot * p.pages_per_seq;
    float m_run = -INFINITY, l_run = 0.0f;
    float o[kDimsPerLane];
#pragma unroll
    for (uint32_t i = 0; i < kDimsPerLane; ++i) o[i] = 0.0f;
    for (uint32_t t0 = 0; t0 < n_keys; t0 += 64) {
        const uint32_t j = t0 + lane;
        float score = -INFINITY;
        if (j < n_keys) {
            const uint16_t *kr = p.k_pages + token_base(p, table, kvh, j);
            float dot = 0.0f;
            for (uint32_t d = 0; d < D; ++d) dot += qs[d] * bf16_to_f32(kr[d]);
            score = dot * scale;
        }
        const float m_new = fmaxf(m_run, max64(score));
        const float prior = expf(m_run - m_new);  // 0 on the first tile (m_run = -inf)
        const float pj = j < n_keys ? expf(score - m_new) : 0.0f;
        l_run = l_run * prior + sum64(pj);
        ps[lane] = pj;
        __syncthreads();
#pragma unroll
        for (uint32_t i = 0; i < kDimsPerLane; ++i) o[i] *= prior;
        const uint32_t nt = min(64u, n_keys - t0);
        for (uint32_t jj = 0; jj < nt; ++jj) {
            const float pk = ps[jj];
            const uint16_t *vr = p.v_pages + token_base(p, table, kvh, t0 + jj);
#pragma unroll
            for (uint32_t i = 0; i < kDimsPerLane; ++i) {
                const uint32_t d = lane + 64 * i;
                if (d < D) o[i] += pk * bf16_to_f32(vr[d]);
            }
        }
        __syncthreads();  // ps is rewritten by the next tile
        m_run = m_new;
    }
    const float inv_l = 1.0f / l_run;
    float *dst = p.out + (row * p.heads + head) * D;
#pragma unroll
    for (uint32_t i = 0; i < kDimsPerLane; ++i) {
        const uint32_t d = lane + 64 * i;
        if (d >= D) continue;
        float y = o[i] * inv_l;
        if (gated) y *= ref_sigmoid(load_act(p.q, q_off + D + d, bf16_in));  // math.rs sigmoid
        dst[d] = y;
    }
}

}  // namespace

bool generic_head_dim(uint32_t head_dim) {
    return head_dim != 64 && head_dim != 128 && head_dim != 256;
}

hipError_t launch_attn_generic(hipStream_t stream, const AttnLaunch &a, const SeqMeta *seqs,
                               int nseq) {
    if (a.head_dim == 0 || a.head_dim > kGenericMaxHeadDim || a.rope_denom == nullptr ||
        a.rotary_dim > a.head_dim) {
        return hipErrorInvalidValue;
    }
    const auto *pool = a.pool;
    GenericParams p;
    p.k_pages = pool->k_pages;
    p.v_pages = pool->v_pages;
    p.page_table = pool->d_page_table;
    p.q = a.q;
    p.k = a.k;
    p.v = a.v;
    p.q_norm = a.q_norm;
    p.k_norm = a.k_norm;
    p.positions = a.positions;
    p.out = a.out;
    p.err_word = a.err_word;
    p.num_pages = pool->num_pages;
    p.pages_per_seq = pool->pages_per_seq;
    p.page_tokens = pool->page_tokens;
    p.flags = a.flags;
    p.heads = a.heads;
    p.kv_heads = a.kv_heads;
    p.head_dim = a.head_dim;
    p.rotary_dim = a.rotary_dim;
    p.mrope[0] = a.mrope[0];
    p.mrope[1] = a.mrope[1];
    p.mrope[2] = a.mrope[2];
    p.eps = a.eps;
    for (uint32_t i = 0; i < a.rotary_dim / 2; ++i) p.denom[i] = a.rope_denom[i];
    for (int base = 0; base < nseq; base += kMetaPerLaunch) {
        const int n = (nseq - base) < kMetaPerLaunch ? (nseq - base) : kMetaPerLaunch;
        uint32_t max_rows = 0;
        for (int i = 0; i < n; ++i) {
            const SeqMeta &q = seqs[base + i];
            p.meta[i] = GenericMeta{q.slot, q.ctx, q.rows, q.row0};
            max_rows = q.rows > max_rows ? q.rows : max_rows;
        }
        p.nseq = (uint32_t)n;
        // every row's k/v are in the pages before any row attends; grid.y
        // covers at most kRowsPerGrid rows of each sequence per launch
        constexpr uint32_t kRowsPerGrid = 65535;
        for (uint32_t rb = 0; rb < max_rows; rb += kRowsPerGrid) {
            p.row_base = rb;
            const uint32_t nr = max_rows - rb < kRowsPerGrid ? max_rows - rb : kRowsPerGrid;
            SR_LAUNCH("attn_generic_append_kernel", attn_generic_append_kernel,
                      dim3(a.kv_heads, nr, n), dim3(64), a.head_dim * sizeof(float), stream, p);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
        for (uint32_t rb = 0; rb < max_rows; rb += kRowsPerGrid) {
            p.row_base = rb;
            const uint32_t nr = max_rows - rb < kRowsPerGrid ? max_rows - rb : kRowsPerGrid;
            SR_LAUNCH("attn_generic_kernel", attn_generic_kernel, dim3(a.heads, nr, n), dim3(64),
                      (a.head_dim + 64) * sizeof(float), stream, p);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

}  // namespace sr
