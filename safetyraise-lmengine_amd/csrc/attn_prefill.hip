// Chunked-prefill attention for gfx950 on MFMA (fp16 operands, fp32
// accumulate, online softmax in fp32) over the bf16 KV cache.
//
// Replaces, for a batch of sequences that each append many rows, the
// Attention::forward row loop of the reference (src/model/native.rs:627-643):
// QK-RMSNorm and RoPE of every new row (math.rs:28-99), append of the rows'
// K/V to the paged cache (state.rs:52-84), causal_attention of row i over the
// context plus rows 0..i (math.rs:102-155), and the Qwen3.5 output gate.
//
// Two kernels per launch:
//   kv_append_rows_kernel  K RMSNorm + RoPE and V of every new row, rounded
//                          to bf16 into the pages (the reference appends
//                          before it attends, so every row's keys must be in
//                          the cache before any row attends);
//   attn_prefill_kernel    one workgroup per (sequence, KV head, block of 32
//                          new rows); its G waves are the G query heads of
//                          the GQA group and share every K/V tile.
//
// Per 64-key tile a wave computes S^T = K Q^T (keys x rows) and
// O^T += V^T P^T (head_dim x rows) with v_mfma_f32_32x32x16_f16.  In the
// accumulator layout of that instruction a lane holds one column, so with the
// transposed products every lane owns one query row: the row max needs a
// single exchange between the two 32-lane halves (v_permlane32_swap), the row
// sum stays lane-local until the end and rescaling O needs no shuffles.
// Operand precision.  The MFMAs run on fp16 operands: K and V tiles are the
// cache's bf16 values converted exactly to fp16 while they are staged into
// LDS (bf16 has fewer mantissa bits; every bf16 value of magnitude in
// [2^-14, 65504] is an fp16 value), and q (normalised, rotated and scaled by
// log2(e)/sqrt(D) in f32) and the probabilities P are rounded to fp16 once.
// fp16 keeps 3 more mantissa bits than bf16 for q and P, which is what holds
// rows with few visible keys inside the bf16-path tolerance.  A K, V or q
// value beyond the fp16 range becomes infinite and makes that row's output
// non-finite; the row is then flagged (kErrPrefillRange) for the host, which
// recomputes the call on the f32 split-K path.
#include <algorithm>

#include "sr_device.hpp"

namespace sr {

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kRowTile = 32;   // query rows per wave (the MFMA N dimension)
constexpr int kKeyTile = 64;   // keys per LDS stage

struct PrefillMeta {
    uint32_t slot;  // page-table row
    uint32_t ctx;   // tokens cached before this call's rows
    uint32_t rows;  // new rows
    uint32_t row0;  // first row in the call's q/k/v/out/positions
    uint32_t nblk;  // row blocks of this sequence
};

struct PrefillParams {
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
    uint32_t log2_page_tokens;
    uint32_t flags;
    uint32_t heads;
    uint32_t kv_heads;
    uint32_t rotary_dim;
    uint32_t mrope[3];
    float eps;
    uint32_t nseq;
    uint32_t max_blk;
    RopeTable rope;
    PrefillMeta meta[kMetaPerLaunch];
};

// Max of x over lanes l and l^32 (both halves get the same value).
__device__ __forceinline__ float xhalf_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false,
                                                    false);
    return fmaxf(__int_as_float(r[0]), __int_as_float(r[1]));
}
__device__ __forceinline__ float xhalf_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false,
                                                    false);
    return __int_as_float(r[0]) + __int_as_float(r[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Two f32 values to a packed fp16 pair (round to nearest even, v_cvt_pk_f16_f32).
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, f16x2));
}
// Element e of 8 packed bf16 values, widened to f32 (exact).
__device__ __forceinline__ float bf16_elem(const u32x4 &w, int e) {
    return (e & 1) ? bf16hi(w[e >> 1]) : bf16lo(w[e >> 1]);
}

// ---------------------------------------------------------------------------
// K/V append of every new row: one wave per (row, KV head).
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void kv_append_rows_kernel(const PrefillParams p) {
    constexpr int EPL = D / 64;
    __shared__ float rowbuf[4][D];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const PrefillMeta m = p.meta[blockIdx.y];
    const uint32_t item = blockIdx.x * 4 + wave;
    const bool valid = item < m.rows * p.kv_heads;
    const uint32_t r = valid ? item / p.kv_heads : 0;
    const uint32_t kvh = valid ? item % p.kv_heads : 0;
    const bool bf16_in = (p.flags & SAFETYRAISE_MI355X_INPUT_BF16) != 0;
    const bool qk_norm = (p.flags & SAFETYRAISE_MI355X_QK_NORM) != 0;
    const bool interleaved = (p.flags & SAFETYRAISE_MI355X_MROPE_INTERLEAVED) != 0;
    const float norm_add = (p.flags & SAFETYRAISE_MI355X_NORM_OFFSET) ? 1.0f : 0.0f;
    const size_t src = ((size_t)(m.row0 + r) * p.kv_heads + kvh) * D;

    float x[EPL], vv[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        x[i] = valid ? load_act(p.k, src + lane + 64 * i, bf16_in) : 0.0f;
        vv[i] = valid ? load_act(p.v, src + lane + 64 * i, bf16_in) : 0.0f;
    }
    if (qk_norm) {
        // rms_norm (math.rs:28-50): x * (1/sqrt(mean(x^2)+eps)) * (w + offset)
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < EPL; ++i) ss += x[i] * x[i];
        ss = sum64(ss);
        const float variance = ss / (float)D;
        if (valid && !isfinite(variance) && lane == 0) {
            atomicOr(p.err_word, kErrNonFiniteVariance);
        }
        const float inv = 1.0f / sqrtf(variance + p.eps);
#pragma unroll
        for (int i = 0; i < EPL; ++i) x[i] = x[i] * inv * (p.k_norm[lane + 64 * i] + norm_add);
    }
#pragma unroll
    for (int i = 0; i < EPL; ++i) rowbuf[wave][lane + 64 * i] = x[i];
    __syncthreads();

    // RoPE, rotate-half over the first rotary_dim dims (math.rs:52-99)
    const uint32_t half = p.rotary_dim / 2;
    const int32_t *pos3 = p.positions + (size_t)(m.row0 + r) * 3;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        const uint32_t e = lane + 64 * i;
        if (e < p.rotary_dim) {
            const uint32_t pi = e < half ? e : e - half;
            const int axis = rope_axis(pi, p.mrope, interleaved);
            const float angle = (float)pos3[axis] / p.rope.denom[pi];
            float sn, cs;
            sincosf(angle, &sn, &cs);
            const float left = rowbuf[wave][pi];
            const float right = rowbuf[wave][pi + half];
            x[i] = e < half ? left * cs - right * sn : right * cs + left * sn;
        }
    }
    if (!valid) return;
    const uint32_t tok = m.ctx + r;
    const int32_t page = p.page_table[(size_t)m.slot * p.pages_per_seq + (tok >> p.log2_page_tokens)];
    const uint32_t pt_mask = (1u << p.log2_page_tokens) - 1;
    const size_t dst = ((((size_t)kvh * p.num_pages + page) << p.log2_page_tokens) + (tok & pt_mask)) * D;
    bool finite = true;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        finite = finite && isfinite(x[i]) && isfinite(vv[i]);
        p.k_pages[dst + lane + 64 * i] = f32_to_bf16(x[i]);
        p.v_pages[dst + lane + 64 * i] = f32_to_bf16(vv[i]);
    }
    if (!finite) atomicOr(p.err_word, kErrNonFiniteKv);
}

// ---------------------------------------------------------------------------
// Attention.  LDS per stage: K tile [64 keys][D] and V^T tile [D][64 keys],
// both bf16, 16-byte units XOR-swizzled so that MFMA operand reads (eight
// lanes on eight consecutive rows) and tile writes hit distinct banks.
//
// V^T column order.  The accumulator of S^T gives lane l (half h = l/32) the
// keys 8a + 4h + b (a, b < 4) of each 32-key half tile.  The PV product takes
// its B operand (8 keys per lane) straight from those registers, so V^T
// column 16s + 8h + j holds key 16s + 4h + 8(j/4) + (j%4): the A operand of
// step s is then one contiguous 16-byte read.
// ---------------------------------------------------------------------------
template <int D>
struct PrefillLds {
    static constexpr size_t kBytes = (size_t)kKeyTile * D * 2;  // one K or V^T tile
    static constexpr size_t kStage = 2 * kBytes;
    static constexpr size_t kTotal = 2 * kStage;  // double buffered
};

__device__ __forceinline__ uint32_t vt_swz(uint32_t d) { return (d & 7) ^ ((d >> 3) & 7); }

// Two workgroups share a CU when the tiles fit twice in LDS (D <= 128): each
// wave then gets at most 256 registers.
template <int D, int G>
__global__ __launch_bounds__(64 * G * ((G >= 4) ? 1 : (4 + G - 1) / G))
__attribute__((amdgpu_waves_per_eu(D <= 128 ? 2 : 1))) void attn_prefill_kernel(
    const PrefillParams p) {
    constexpr int R = (G >= 4) ? 1 : (4 + G - 1) / G;  // 32-row sub-blocks per workgroup
    constexpr int NW = G * R;
    constexpr int NTHR = 64 * NW;
    constexpr int NS = D / 16;   // QK k-steps
    constexpr int NT = D / 32;   // PV output tiles
    constexpr int KCH = D / 8;   // 16-byte chunks per K row
    constexpr int KL = (kKeyTile * KCH + NTHR - 1) / NTHR;
    constexpr int VU = (kKeyTile / 4) * KCH;  // (4-key group, chunk) units of a V tile
    constexpr int VL = (VU + NTHR - 1) / NTHR;
    extern __shared__ __align__(16) unsigned char lds[];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int h = lane >> 5;
    const int col = lane & 31;

    // blocks: KV head fastest (the 8 XCDs take consecutive blocks, so one KV
    // head's blocks share an L2), then sequence, then row block, last first
    const uint32_t b = blockIdx.x;
    const uint32_t kvh = b % p.kv_heads;
    const uint32_t t2 = b / p.kv_heads;
    const uint32_t s = t2 % p.nseq;
    const PrefillMeta m = p.meta[s];
    const uint32_t qb = p.max_blk - 1 - t2 / p.nseq;
    if (qb >= m.nblk) return;
    const uint32_t blk_row0 = qb * kRowTile * R;
    const uint32_t blk_last = min(blk_row0 + kRowTile * R, m.rows) - 1;
    const uint32_t n_keys = m.ctx + blk_last + 1;
    const uint32_t n_tiles = (n_keys + kKeyTile - 1) / kKeyTile;

    const uint32_t head = kvh * G + (wave % G);
    const uint32_t wrow0 = blk_row0 + kRowTile * (wave / G);
    const uint32_t my_row = min(wrow0 + col, m.rows - 1);
    const uint32_t key_limit = m.ctx + my_row;  // last visible key of this lane's row

    const bool bf16_in = (p.flags & SAFETYRAISE_MI355X_INPUT_BF16) != 0;
    const bool gated = (p.flags & SAFETYRAISE_MI355X_GATED) != 0;
    const bool qk_norm = (p.flags & SAFETYRAISE_MI355X_QK_NORM) != 0;
    const bool interleaved = (p.flags & SAFETYRAISE_MI355X_MROPE_INTERLEAVED) != 0;
    const float norm_add = (p.flags & SAFETYRAISE_MI355X_NORM_OFFSET) ? 1.0f : 0.0f;

    const int32_t *table = p.page_table + (size_t)m.slot * p.pages_per_seq;
    const uint32_t lpt = p.log2_page_tokens;
    const uint32_t pt_mask = (1u << lpt) - 1;
    const size_t head_base = (size_t)kvh * p.num_pages;

    auto tok_addr = [&](uint32_t tok) -> size_t {
        tok = min(tok, n_keys - 1);  // keys past the block's last row are masked
        return (((head_base + (uint32_t)table[tok >> lpt]) << lpt) + (tok & pt_mask)) * D;
    };

    u32x4 kreg[KL];
    u32x4 vreg[VL][4];
    auto load_tile = [&](u32x4(&kreg)[KL], u32x4(&vreg)[VL][4], uint32_t t) {
        const uint32_t key0 = t * kKeyTile;
#pragma unroll
        for (int i = 0; i < KL; ++i) {
            const int c = tid + i * NTHR;
            if ((KL * NTHR == kKeyTile * KCH) || c < kKeyTile * KCH) {
                const int key = c / KCH, ch = c % KCH;
                kreg[i] = *(const u32x4 *)(p.k_pages + tok_addr(key0 + key) + ch * 8);
            }
        }
#pragma unroll
        for (int i = 0; i < VL; ++i) {
            const int u = tid + i * NTHR;
            if ((VL * NTHR == VU) || u < VU) {
                const int ch = u % KCH, g = u / KCH;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    vreg[i][j] = *(const u32x4 *)(p.v_pages + tok_addr(key0 + 4 * g + j) + ch * 8);
                }
            }
        }
    };
    auto store_tile = [&](const u32x4(&kreg)[KL], const u32x4(&vreg)[VL][4], int buf) {
        unsigned char *kt = lds + buf * PrefillLds<D>::kStage;
        unsigned char *vt = kt + PrefillLds<D>::kBytes;
#pragma unroll
        for (int i = 0; i < KL; ++i) {
            const int c = tid + i * NTHR;
            if ((KL * NTHR == kKeyTile * KCH) || c < kKeyTile * KCH) {
                const int key = c / KCH, ch = c % KCH;
                const u32x4 w = kreg[i];
                u32x4 f;
#pragma unroll
                for (int j = 0; j < 4; ++j) f[j] = pack_f16x2(bf16lo(w[j]), bf16hi(w[j]));
                *(u32x4 *)(kt + key * (D * 2) + ((ch ^ (key & 7)) * 16)) = f;
            }
        }
#pragma unroll
        for (int i = 0; i < VL; ++i) {
            const int u = tid + i * NTHR;
            if ((VL * NTHR == VU) || u < VU) {
                const int ch = u % KCH, g = u / KCH;
                const int sblk = g >> 2, q = g & 3;
                const uint32_t unit = 2 * sblk + (q & 1);
                const uint32_t byte_in = 8 * (q >> 1);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    // dim ch*8 + e of the 4 keys, as two fp16 pairs
                    const uint32_t lo =
                        pack_f16x2(bf16_elem(vreg[i][0], e), bf16_elem(vreg[i][1], e));
                    const uint32_t hi =
                        pack_f16x2(bf16_elem(vreg[i][2], e), bf16_elem(vreg[i][3], e));
                    const uint32_t d = ch * 8 + e;
                    *(uint2 *)(vt + d * (kKeyTile * 2) + ((unit ^ vt_swz(d)) * 16) + byte_in) =
                        make_uint2(lo, hi);
                }
            }
        }
    };

    // tile 0 is requested before the q prologue so its latency overlaps it
    load_tile(kreg, vreg, 0);

    // ---- q: RMSNorm, RoPE, scale, fp16 (lane holds dims 16s + 8h + j) ----
    const uint32_t hs = gated ? 2 * D : D;
    const size_t qbase = (size_t)(m.row0 + my_row) * p.heads * hs + (size_t)head * hs;
    float x[NS][8];
#pragma unroll
    for (int st = 0; st < NS; ++st) {
        const size_t off = qbase + 16 * st + 8 * h;
        if (bf16_in) {
            const uint4 w = *(const uint4 *)((const uint16_t *)p.q + off);
            const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                x[st][2 * j] = bf16lo(ww[j]);
                x[st][2 * j + 1] = bf16hi(ww[j]);
            }
        } else {
            const float4 a = *(const float4 *)((const float *)p.q + off);
            const float4 c = *(const float4 *)((const float *)p.q + off + 4);
            x[st][0] = a.x; x[st][1] = a.y; x[st][2] = a.z; x[st][3] = a.w;
            x[st][4] = c.x; x[st][5] = c.y; x[st][6] = c.z; x[st][7] = c.w;
        }
    }
    if (qk_norm) {
        float ss = 0.0f;
#pragma unroll
        for (int st = 0; st < NS; ++st)
#pragma unroll
            for (int j = 0; j < 8; ++j) ss += x[st][j] * x[st][j];
        ss = xhalf_sum(ss);
        const float variance = ss / (float)D;
        if (!isfinite(variance) && lane == 0) {
            atomicOr(p.err_word, kErrNonFiniteVariance);
        }
        const float inv = 1.0f / sqrtf(variance + p.eps);
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            const float4 wa = *(const float4 *)(p.q_norm + 16 * st + 8 * h);
            const float4 wb = *(const float4 *)(p.q_norm + 16 * st + 8 * h + 4);
            const float wv[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
#pragma unroll
            for (int j = 0; j < 8; ++j) x[st][j] = x[st][j] * inv * (wv[j] + norm_add);
        }
    }
    {
        // pairs (i, i + rotary_dim/2); the host routes only rotary_dim/2 that
        // is a multiple of 16 here, so both halves of a pair sit in this lane
        const uint32_t hsteps = p.rotary_dim / 32;
        const int32_t *pos3 = p.positions + (size_t)(m.row0 + my_row) * 3;
        const int32_t pos0 = pos3[0], pos1 = pos3[1], pos2 = pos3[2];
        // (the partner step st + hsteps is selected with compile-time indices
        // so that x stays in registers)
#pragma unroll
        for (int st = 0; st < NS / 2; ++st) {
            if ((uint32_t)st < hsteps) {
                float right[8];
#pragma unroll
                for (int k = 1; k <= NS / 2; ++k) {
                    if ((uint32_t)k == hsteps) {
#pragma unroll
                        for (int j = 0; j < 8; ++j) right[j] = x[st + k][j];
                    }
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint32_t i = 16 * st + 8 * h + j;
                    const int axis = rope_axis(i, p.mrope, interleaved);
                    const int32_t pa = axis == 0 ? pos0 : (axis == 1 ? pos1 : pos2);
                    const float angle = (float)pa / p.rope.denom[i];
                    float sn, cs;
                    sincosf(angle, &sn, &cs);
                    const float left = x[st][j];
                    x[st][j] = left * cs - right[j] * sn;
                    right[j] = right[j] * cs + left * sn;
                }
#pragma unroll
                for (int k = 1; k <= NS / 2; ++k) {
                    if ((uint32_t)k == hsteps) {
#pragma unroll
                        for (int j = 0; j < 8; ++j) x[st + k][j] = right[j];
                    }
                }
            }
        }
    }
    const float qscale = (1.0f / sqrtf((float)D)) * kLog2e;
    f16x8 qop[NS];
#pragma unroll
    for (int st = 0; st < NS; ++st) {
        f32x8 v;
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = x[st][j] * qscale;
        qop[st] = __builtin_convertvector(v, f16x8);
    }

    // ---- main loop over 64-key tiles ----
    f32x16 oacc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) oacc[t] = f32x16{};
    float m_run = -INFINITY;
    float l_run = 0.0f;
    const uint32_t first_row_limit = m.ctx + blk_row0;  // smallest key limit in the block

    for (uint32_t t = 0; t < n_tiles; ++t) {
        const int buf = t & 1;
        store_tile(kreg, vreg, buf);
        __syncthreads();
        if (t + 1 < n_tiles) load_tile(kreg, vreg, t + 1);
        const unsigned char *kt = lds + buf * PrefillLds<D>::kStage;
        const unsigned char *vt = kt + PrefillLds<D>::kBytes;

        // S^T = K Q^T for keys [32u, 32u + 32) of the tile
        f32x16 sacc[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            sacc[u] = f32x16{};
            const int key = 32 * u + col;
#pragma unroll
            for (int st = 0; st < NS; ++st) {
                const f16x8 a =
                    *(const f16x8 *)(kt + key * (D * 2) + (((2 * st + h) ^ (key & 7)) * 16));
                sacc[u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qop[st], sacc[u], 0, 0, 0);
            }
        }
        const uint32_t key0 = t * kKeyTile;
        if (key0 + kKeyTile - 1 > first_row_limit) {
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const uint32_t key = key0 + 32 * u + 8 * (i >> 2) + 4 * h + (i & 3);
                    if (key > key_limit) sacc[u][i] = -INFINITY;
                }
        }
        float mx = sacc[0][0];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sacc[u][i]);
        mx = xhalf_max(mx);
        const float m_new = fmaxf(m_run, mx);
        const float alpha = fast_exp2(m_run - m_new);
        m_run = m_new;
        float psum = 0.0f;
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float pv = fast_exp2(sacc[u][i] - m_new);
                sacc[u][i] = pv;
                psum += pv;
            }
        l_run = l_run * alpha + psum;
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
            for (int tt = 0; tt < NT; ++tt)
#pragma unroll
                for (int i = 0; i < 16; ++i) oacc[tt][i] *= alpha;
        }
        f16x8 pop[4];
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            f32x8 v;
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = sacc[st >> 1][8 * (st & 1) + j];
            pop[st] = __builtin_convertvector(v, f16x8);
        }
        // O^T += V^T P^T
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) {
            const uint32_t d = 32 * tt + col;
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const f16x8 a = *(const f16x8 *)(vt + d * (kKeyTile * 2) +
                                                   (((2 * st + h) ^ vt_swz(d)) * 16));
                oacc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pop[st], oacc[tt], 0, 0, 0);
            }
        }
    }

    // ---- epilogue: o / l, Qwen3.5 gate, f32 store ----
    const uint32_t row = wrow0 + col;
    if (row >= m.rows) return;
    const float inv_l = 1.0f / xhalf_sum(l_run);
    float *dst = p.out + (size_t)(m.row0 + row) * p.heads * D + (size_t)head * D;
    bool finite = true;
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            const uint32_t d0 = 32 * tt + 8 * a + 4 * h;
            float o[4];
#pragma unroll
            for (int bb = 0; bb < 4; ++bb) {
                o[bb] = oacc[tt][4 * a + bb] * inv_l;
                finite = finite && isfinite(o[bb]);
            }
            if (gated) {
#pragma unroll
                for (int bb = 0; bb < 4; ++bb) {
                    o[bb] *= ref_sigmoid(load_act(p.q, qbase + D + d0 + bb, bf16_in));
                }
            }
            *(float4 *)(dst + d0) = make_float4(o[0], o[1], o[2], o[3]);
        }
    }
    if (!finite) atomicOr(p.err_word, kErrPrefillRange);
}

template <int D, int G>
hipError_t launch_dg(hipStream_t stream, const PrefillParams &p, uint32_t append_blocks_x) {
    constexpr int R = (G >= 4) ? 1 : (4 + G - 1) / G;
    hipLaunchKernelGGL(kv_append_rows_kernel<D>, dim3(append_blocks_x, p.nseq), dim3(256), 0,
                       stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    static bool configured = false;
    const size_t lds = PrefillLds<D>::kTotal;
    if (!configured) {
        e = hipFuncSetAttribute((const void *)attn_prefill_kernel<D, G>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        configured = true;
    }
    const uint32_t blocks = p.max_blk * p.nseq * p.kv_heads;
    hipLaunchKernelGGL((attn_prefill_kernel<D, G>), dim3(blocks), dim3(64 * G * R), lds, stream,
                       p);
    return hipGetLastError();
}

template <int D>
hipError_t launch_d(hipStream_t stream, const PrefillParams &p, uint32_t g, uint32_t ax) {
    switch (g) {
        case 1: return launch_dg<D, 1>(stream, p, ax);
        case 2: return launch_dg<D, 2>(stream, p, ax);
        case 3: return launch_dg<D, 3>(stream, p, ax);
        case 4: return launch_dg<D, 4>(stream, p, ax);
        case 5: return launch_dg<D, 5>(stream, p, ax);
        case 6: return launch_dg<D, 6>(stream, p, ax);
        case 7: return launch_dg<D, 7>(stream, p, ax);
        case 8: return launch_dg<D, 8>(stream, p, ax);
        default: return hipErrorInvalidValue;
    }
}

uint32_t rows_per_block(uint32_t g) { return kRowTile * ((g >= 4) ? 1 : (4 + g - 1) / g); }

}  // namespace

bool prefill_supported(const AttnLaunch &a) {
    const uint32_t g = a.heads / a.kv_heads;
    return (a.head_dim == 64 || a.head_dim == 128 || a.head_dim == 256) && g >= 1 && g <= 8 &&
           a.rotary_dim % 32 == 0;
}

hipError_t launch_attn_prefill(hipStream_t stream, const AttnLaunch &a, const SeqMeta *seqs,
                               int nseq) {
    if (nseq <= 0 || nseq > kMetaPerLaunch || !prefill_supported(a)) return hipErrorInvalidValue;
    const auto *pool = a.pool;
    const uint32_t g = a.heads / a.kv_heads;
    const uint32_t rpb = rows_per_block(g);
    PrefillParams p{};
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
    p.log2_page_tokens = (uint32_t)__builtin_ctz(pool->page_tokens);
    p.flags = a.flags;
    p.heads = a.heads;
    p.kv_heads = a.kv_heads;
    p.rotary_dim = a.rotary_dim;
    p.mrope[0] = a.mrope[0];
    p.mrope[1] = a.mrope[1];
    p.mrope[2] = a.mrope[2];
    p.eps = a.eps;
    p.nseq = (uint32_t)nseq;
    p.rope = *a.rope;
    uint32_t max_blk = 0, max_rows = 0;
    for (int i = 0; i < nseq; ++i) {
        PrefillMeta &m = p.meta[i];
        m.slot = seqs[i].slot;
        m.ctx = seqs[i].ctx;
        m.rows = seqs[i].rows;
        m.row0 = seqs[i].row0;
        m.nblk = (m.rows + rpb - 1) / rpb;
        max_blk = std::max(max_blk, m.nblk);
        max_rows = std::max(max_rows, m.rows);
    }
    p.max_blk = max_blk;
    const uint32_t append_x = (uint32_t)(((uint64_t)max_rows * a.kv_heads + 3) / 4);
    switch (a.head_dim) {
        case 64: return launch_d<64>(stream, p, g, append_x);
        case 128: return launch_d<128>(stream, p, g, append_x);
        case 256: return launch_d<256>(stream, p, g, append_x);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace sr
