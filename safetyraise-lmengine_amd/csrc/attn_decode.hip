// Split-K decode attention for gfx950 (one new row per sequence).
//
// Replaces, for a batch of sequences, one pass of the Attention::forward row
// loop (reference src/model/native.rs:627-643): QK-RMSNorm and RoPE of the new
// row, append of its K/V to the paged cache, causal_attention over every
// cached token (src/model/math.rs:102-155), and the Qwen3.5 output gate.
//
// Work decomposition.  For each KV head the launch sees one token space: the
// sequences' visible tokens (context + the new row) laid end to end.  It is
// cut into `parts` equal slices and the grid has exactly parts * kv_heads
// workgroups, as many as the GPU keeps resident, so every workgroup streams
// the same number of bytes and they all finish together (no tail of a
// half-empty GPU).  A slice that crosses sequence boundaries is processed as
// one segment per sequence.  Each segment leaves one (max, sum, output)
// record per query head; a sequence covered by a single segment writes its
// output directly, the others are merged by attn_combine_kernel.
//
// Inside a segment: 256 threads = 16 groups of 16 lanes; a group owns one
// token per pass, a lane owns D/16 consecutive dims, so one K or V row
// (D bf16) is one 16-lane 128-bit-per-lane load and a wave reads 4 whole rows
// per instruction.  All G = heads/kv_heads query heads of the GQA group share
// each K/V load.  Scores are reduced over the 16 lanes with DPP; PV needs no
// cross-lane traffic.  Each group keeps an online-softmax state per head in
// the log2 domain; groups and waves are merged at the end of the segment.
// No MFMA: the step is HBM-bound (4 flop per byte).
#include <algorithm>

#include "sr_device.hpp"

namespace sr {

namespace {

constexpr int kThreads = 256;
constexpr int kChunk = 64;          // tokens per loop iteration (4 passes x 16 groups)
constexpr int kMaxSplitPages = 256; // page ids of one sub-range staged in LDS

struct DecodeMeta {
    uint32_t slot;    // page-table row
    uint32_t ctx;     // tokens cached before the new row
    uint32_t row0;    // row in q/k/v/out/positions
    uint32_t rec0;    // first record index of this sequence
    uint32_t nrec;    // records (segments) of this sequence
    uint32_t start;   // offset of the sequence in the launch's token space
};

struct DecodeParams {
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
    float *partials;
    uint32_t *err_word;
    uint64_t num_pages;
    uint32_t pages_per_seq;
    uint32_t page_tokens;
    uint32_t flags;
    uint32_t heads;
    uint32_t kv_heads;  // KV heads as the grid sees them: the cache's times kv_rep
    uint32_t kv_rep;    // query-head groups per cache KV head (groups of more
                        // than 8 heads run as kv_rep groups of heads/kv_heads)
    uint32_t rotary_dim;
    uint32_t mrope[3];
    float eps;
    uint32_t part_tokens;   // tokens per slice
    uint32_t total_tokens;  // size of the token space
    uint32_t sub_chunks;    // chunks per sub-range whose page ids fit in LDS
    uint32_t log2_page_tokens;
    uint32_t nseq;
    RopeTable rope;
    DecodeMeta meta[kMetaPerLaunch];
};

// D/16 bf16 values of one K or V row owned by a lane.
template <int DPL>
struct Frag {
    uint32_t w[DPL / 2];
};

// Cache pages are streamed once per call: the loads are nontemporal (the
// lines are not kept for reuse), which measured ~8 % more read bandwidth on
// MI355X than ordinary loads in a plain streaming kernel (5.9-6.0 vs
// 5.4-5.7 TB/s).
typedef uint32_t nt_u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t nt_u32x4 __attribute__((ext_vector_type(4)));

template <int DPL>
__device__ __forceinline__ Frag<DPL> load_frag(const uint16_t *p) {
    Frag<DPL> f;
    if constexpr (DPL == 4) {
        const nt_u32x2 x = __builtin_nontemporal_load((const nt_u32x2 *)p);
        f.w[0] = x.x;
        f.w[1] = x.y;
    } else {
#pragma unroll
        for (int i = 0; i < DPL / 8; ++i) {
            const nt_u32x4 x = __builtin_nontemporal_load((const nt_u32x4 *)p + i);
            f.w[4 * i + 0] = x.x;
            f.w[4 * i + 1] = x.y;
            f.w[4 * i + 2] = x.z;
            f.w[4 * i + 3] = x.w;
        }
    }
    return f;
}

template <int DPL>
__device__ __forceinline__ float frag_at(const Frag<DPL> &f, int j) {
    return (j & 1) ? bf16hi(f.w[j >> 1]) : bf16lo(f.w[j >> 1]);
}

template <int D, int G>
struct DecodeShared {
    float vec[G + 1][D];  // q heads of the group, then the new k
    int32_t pages[kMaxSplitPages];
    float red_m[4][G];
    float red_l[4][G];
    float red_o[4][G][D];
    // per (wave, 16-lane group): the chunk's 4G probabilities, then G rescales
    float pbuf[4][4][5 * G];
};

// One reduce-scatter stage over the 16 lanes of a group: the lanes whose bit
// `hi` is clear keep the low half of `in`, the others the high half, and each
// adds its partner's copy of the half it keeps.  CTRL is a DPP pattern that
// pairs every lane with one whose bit differs (row mirror for bit 3, half-row
// mirror for bit 2, quad swaps for bits 1 and 0).
template <int CTRL, int M>
__device__ __forceinline__ void rs_stage(const float (&in)[M], float (&out)[M / 2], bool hi) {
#pragma unroll
    for (int k = 0; k < M / 2; ++k) {
        const float keep = hi ? in[M / 2 + k] : in[k];
        const float send = hi ? in[k] : in[M / 2 + k];
        out[k] = keep + dpp<CTRL>(send);
    }
}

// One segment: tokens [t0, t1) of sequence s for KV head kvh; writes record
// `rec` (or the final output when the sequence has a single record).
// kPageHoldsChunk: page_tokens >= 64, so a 64-token chunk never crosses a page.
template <int D, int G, bool kPageHoldsChunk>
__device__ void decode_segment(const DecodeParams &p, DecodeShared<D, G> &sh, int s, uint32_t kvh,
                               uint32_t t0, uint32_t t1, uint32_t rec) {
    constexpr int DPL = D / 16;  // dims per lane in the main loop
    constexpr int EPL = D / 64;  // elements per lane while normalising
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int group = tid >> 4;
    const int l16 = tid & 15;

    const uint32_t slot = p.meta[s].slot;
    const uint32_t ctx = p.meta[s].ctx;
    const uint32_t row = p.meta[s].row0;
    const uint32_t nrec = p.meta[s].nrec;
    const uint32_t total = ctx + 1;
    const bool owns_new = (t1 == total);

    const bool bf16_in = (p.flags & SAFETYRAISE_MI355X_INPUT_BF16) != 0;
    const bool gated = (p.flags & SAFETYRAISE_MI355X_GATED) != 0;
    const bool qk_norm = (p.flags & SAFETYRAISE_MI355X_QK_NORM) != 0;
    const bool interleaved = (p.flags & SAFETYRAISE_MI355X_MROPE_INTERLEAVED) != 0;
    const float norm_add = (p.flags & SAFETYRAISE_MI355X_NORM_OFFSET) ? 1.0f : 0.0f;
    const uint32_t hs = gated ? 2 * D : D;  // q elements per head
    const size_t q_row = (size_t)row * p.heads * hs;
    // the cache's KV head of this (virtual) one, and the cache's head count
    const uint32_t kvp = kvh / p.kv_rep;
    const size_t kv_row = ((size_t)row * (p.kv_heads / p.kv_rep) + kvp) * D;
    const uint32_t PT = p.page_tokens;
    const int32_t *table = p.page_table + (size_t)slot * p.pages_per_seq;

    __syncthreads();  // the previous segment is done with the shared arrays

    // 0. K/V streaming set-up.  Chunks are the 64-token blocks [64c, 64c+64)
    //    of the sequence, streamed in sub-ranges whose page ids fit in LDS.
    //    The first two chunks are requested before the q prologue so the
    //    prologue overlaps their latency, unless they could hold the new
    //    token, which the prologue writes.
    const uint32_t lpt = p.log2_page_tokens;
    const uint32_t c_lo = t0 / kChunk;
    const uint32_t c_hi = (t1 + kChunk - 1) / kChunk;
    const uint32_t last_pg = (t1 - 1) >> lpt;  // pages past the segment may not exist
    uint32_t s0 = c_lo;
    uint32_t s1 = min(s0 + p.sub_chunks, c_hi);
    uint32_t pg0 = 0, pg1 = 0;
    auto setup_sub = [&]() {
        pg0 = (s0 * kChunk) >> lpt;
        pg1 = min(((s1 * kChunk) - 1) >> lpt, last_pg);
        for (uint32_t i = tid; i <= pg1 - pg0; i += kThreads) {
            sh.pages[i] = table[pg0 + i];
        }
        __syncthreads();
    };
    auto load_chunk = [&](Frag<DPL>(&kb)[4], Frag<DPL>(&vb)[4], uint32_t c) {
        const uint32_t cc = min(c, s1 - 1);
        if constexpr (kPageHoldsChunk) {
            // the whole chunk sits in one page: one lookup, then fixed strides
            const uint32_t tb = cc * kChunk;
            const uint32_t pg = min(tb >> lpt, pg1) - pg0;
            const size_t r =
                (((size_t)kvp * p.num_pages + sh.pages[pg]) << lpt) + (tb & ((1u << lpt) - 1));
            const uint16_t *kp = p.k_pages + r * D + group * D + l16 * DPL;
            const uint16_t *vp = p.v_pages + r * D + group * D + l16 * DPL;
#pragma unroll
            for (int ps = 0; ps < 4; ++ps) {
                kb[ps] = load_frag<DPL>(kp + ps * 16 * D);
                vb[ps] = load_frag<DPL>(vp + ps * 16 * D);
            }
        } else {
#pragma unroll
            for (int ps = 0; ps < 4; ++ps) {
                const uint32_t tok = cc * kChunk + ps * 16 + group;
                const uint32_t pg = min(tok >> lpt, pg1) - pg0;
                const size_t r = (((size_t)kvp * p.num_pages + sh.pages[pg]) << lpt) +
                                 (tok & ((1u << lpt) - 1));
                kb[ps] = load_frag<DPL>(p.k_pages + r * D + l16 * DPL);
                vb[ps] = load_frag<DPL>(p.v_pages + r * D + l16 * DPL);
            }
        }
        // keep chunk loads in program order: the wait before a chunk is
        // consumed then counts only the younger chunks still in flight
        __builtin_amdgcn_sched_barrier(0);
    };
    Frag<DPL> ka[4], va[4], kb[4], vb[4], kc[4], vc[4];
    const bool early = !owns_new || c_hi - c_lo > 2;
    setup_sub();
    if (early) {
        load_chunk(ka, va, s0);
        load_chunk(kb, vb, s0 + 1);
    }

    // 1. per-head RMSNorm of the group's q heads (and of the new k)
    //    (src/model/math.rs:28-50 via native.rs:629-634); every global input
    //    of the prologue is requested before any is used
    const int nvec = G + (owns_new ? 1 : 0);
    const int32_t *pos3 = p.positions + (size_t)row * 3;
    const int32_t pos_axis[3] = {pos3[0], pos3[1], pos3[2]};
    const float v_new = (owns_new && tid < D) ? load_act(p.v, kv_row + tid, bf16_in) : 0.0f;
    for (int h = wave; h < nvec; h += 4) {
        float x[EPL], wv[EPL];
        const float *w = (h < G) ? p.q_norm : p.k_norm;
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
            const int e = lane + 64 * i;
            x[i] = (h < G) ? load_act(p.q, q_row + (size_t)(kvh * G + h) * hs + e, bf16_in)
                           : load_act(p.k, kv_row + e, bf16_in);
            wv[i] = qk_norm ? w[e] : 0.0f;
        }
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
            ss += x[i] * x[i];
        }
        if (qk_norm) {
            ss = sum64(ss);
            const float variance = ss / (float)D;
            if (!isfinite(variance) && lane == 0) {
                atomicOr(p.err_word, kErrNonFiniteVariance);
            }
            const float inv = 1.0f / sqrtf(variance + p.eps);
#pragma unroll
            for (int i = 0; i < EPL; ++i) {
                x[i] = x[i] * inv * (wv[i] + norm_add);
            }
        }
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
            sh.vec[h][lane + 64 * i] = x[i];
        }
    }
    __syncthreads();

    // 2. RoPE, rotate-half over the first rotary_dim dims (math.rs:52-99);
    //    angle = pos / theta^(2i/rotary_dim) with an IEEE f32 division
    const uint32_t half = p.rotary_dim / 2;
    for (uint32_t idx = tid; idx < (uint32_t)nvec * half; idx += kThreads) {
        const uint32_t h = idx / half;
        const uint32_t i = idx - h * half;
        const int axis = rope_axis(i, p.mrope, interleaved);
        const float angle = (float)pos_axis[axis] / p.rope.denom[i];
        float sn, cs;
        sincosf(angle, &sn, &cs);
        const float left = sh.vec[h][i];
        const float right = sh.vec[h][i + half];
        sh.vec[h][i] = left * cs - right * sn;
        sh.vec[h][i + half] = right * cs + left * sn;
    }
    __syncthreads();

    // 3. append the new token's k and v (bf16, round to nearest even); it is
    //    the last token of the sequence, so only this segment reads it.  The
    //    kv_rep groups that share a cache head each write it (the same bits,
    //    computed from the same inputs), so each reads back its own write.
    if (owns_new) {
        const uint32_t tok = ctx;
        const int32_t page = table[tok / PT];
        const size_t base = (((size_t)kvp * p.num_pages + page) * PT + tok % PT) * D;
        if (tid < D) {
            const float kk = sh.vec[G][tid];
            if (!isfinite(kk) || !isfinite(v_new)) {
                atomicOr(p.err_word, kErrNonFiniteKv);
            }
            p.k_pages[base + tid] = f32_to_bf16(kk);
            p.v_pages[base + tid] = f32_to_bf16(v_new);
        }
        __syncthreads();
    }

    // 4. q fragments, prescaled by 1/sqrt(D) * log2(e), each split into a
    //    bf16 pair q = hi + lo (about 16 mantissa bits) so that q.k runs as
    //    bf16 dot2 instructions on the raw K words with f32 accumulation
    const float qscale = (1.0f / sqrtf((float)D)) * kLog2e;
    uint32_t qhi[G][DPL / 2], qlo[G][DPL / 2];
#pragma unroll
    for (int h = 0; h < G; ++h) {
#pragma unroll
        for (int w = 0; w < DPL / 2; ++w) {
            const float a = sh.vec[h][l16 * DPL + 2 * w] * qscale;
            const float b = sh.vec[h][l16 * DPL + 2 * w + 1] * qscale;
            qhi[h][w] = pack_bf16x2(a, b);
            qlo[h][w] = pack_bf16x2(a - bf16lo(qhi[h][w]), b - bf16hi(qhi[h][w]));
        }
    }
    if (!early) {
        load_chunk(ka, va, s0);
        load_chunk(kb, vb, s0 + 1);
    }

    // 5. stream the segment's K/V, online softmax per group and head.
    //    Chunks are the 64-token blocks [64c, 64c+64) of the sequence; a pass
    //    (16 tokens) never crosses a page (page_tokens is a power of two
    //    >= 16), so its page base is wave-uniform and each lane only adds a
    //    constant offset.  Three register buffers rotate so that two chunks
    //    are in flight while the third is consumed; loads are unconditional
    //    (chunk indices past the sub-range clamp to its last chunk) so the
    //    compiler waits for exactly the oldest chunk.  Only the first and last
    //    chunks of the segment can hold tokens outside [t0, t1) and are masked.
    float mrun[G], lrun[G], o[G][DPL];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        mrun[h] = -INFINITY;
        lrun[h] = 0.0f;
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
            o[h][j] = 0.0f;
        }
    }

    auto process = [&](const Frag<DPL>(&kb)[4], const Frag<DPL>(&vb)[4], uint32_t c,
                       bool masked) {
        float sc[4][G];
#pragma unroll
        for (int ps = 0; ps < 4; ++ps) {
            const uint32_t tok = c * kChunk + ps * 16 + group;
            const bool valid = !masked || (tok >= t0 && tok < t1);
#pragma unroll
            for (int h = 0; h < G; ++h) {
                float acc = 0.0f;
#pragma unroll
                for (int w = 0; w < DPL / 2; ++w) {
                    acc = dot2_bf16(qhi[h][w], kb[ps].w[w], acc);
                    acc = dot2_bf16(qlo[h][w], kb[ps].w[w], acc);
                }
                acc = sum16(acc);
                sc[ps][h] = valid ? acc : -INFINITY;
            }
        }
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float cm = fmaxf(fmaxf(sc[0][h], sc[1][h]), fmaxf(sc[2][h], sc[3][h]));
            const float mn = fmaxf(mrun[h], cm);
            const float mu = (mn == -INFINITY) ? 0.0f : mn;
            // rescale only when some lane's running max moved (else alpha == 1)
            if (__builtin_amdgcn_ballot_w64(mn > mrun[h]) != 0) {
                const float alpha = __builtin_amdgcn_exp2f(mrun[h] - mu);
                lrun[h] *= alpha;
#pragma unroll
                for (int j = 0; j < DPL; ++j) {
                    o[h][j] *= alpha;
                }
            }
            float pp[4];
#pragma unroll
            for (int ps = 0; ps < 4; ++ps) {
                pp[ps] = __builtin_amdgcn_exp2f(sc[ps][h] - mu);
            }
            lrun[h] += (pp[0] + pp[1]) + (pp[2] + pp[3]);
#pragma unroll
            for (int j = 0; j < DPL; ++j) {
                float acc = o[h][j];
#pragma unroll
                for (int ps = 0; ps < 4; ++ps) {
                    acc += pp[ps] * frag_at<DPL>(vb[ps], j);
                }
                o[h][j] = acc;
            }
            mrun[h] = mn;
        }
    };

    // Transposed softmax (G = 4 or 8).  The group's 4G (token, head) partial
    // dot products are reduce-scattered over its 16 lanes, so each lane owns
    // F = G/4 complete scores, value v = F*l16 + k = head*4 + pass.  The
    // online softmax then runs once per score instead of on every lane, and
    // the probabilities reach the whole group through a small LDS buffer.
    constexpr bool kTransposed = (G == 4 || G == 8);
    constexpr int NV = kTransposed ? 4 * G : 16;  // (array sizes stay valid for other G)
    constexpr int F = NV / 16;
    float mt = -INFINITY, lt = 0.0f;  // running max / sum of this lane's head
    float *pbuf = sh.pbuf[wave][group & 3];
    auto process_t = [&](const Frag<DPL>(&kb)[4], const Frag<DPL>(&vb)[4], uint32_t c,
                         bool masked) {
      if constexpr (kTransposed) {
        float x[NV];
#pragma unroll
        for (int ps = 0; ps < 4; ++ps) {
#pragma unroll
            for (int h = 0; h < G; ++h) {
                float acc = 0.0f;
#pragma unroll
                for (int w = 0; w < DPL / 2; ++w) {
                    acc = dot2_bf16(qhi[h][w], kb[ps].w[w], acc);
                    acc = dot2_bf16(qlo[h][w], kb[ps].w[w], acc);
                }
                x[h * 4 + ps] = acc;
            }
        }
        float y[NV / 2], z[NV / 4], u[NV / 8], sv[F];
        rs_stage<kDppRowMirror>(x, y, (l16 >> 3) & 1);
        rs_stage<kDppRowHalfMirror>(y, z, (l16 >> 2) & 1);
        rs_stage<kDppQuadXor2>(z, u, (l16 >> 1) & 1);
        rs_stage<kDppQuadXor1>(u, sv, l16 & 1);
        float cm = -INFINITY;
#pragma unroll
        for (int k = 0; k < F; ++k) {
            const uint32_t tok = c * kChunk + ((F * l16 + k) & 3) * 16 + group;
            if (masked && !(tok >= t0 && tok < t1)) {
                sv[k] = -INFINITY;
            }
            cm = fmaxf(cm, sv[k]);
        }
        // the lanes holding one head: a quad (F = 1) or a lane pair (F = 2)
        cm = fmaxf(cm, dpp<kDppQuadXor1>(cm));
        if constexpr (F == 1) cm = fmaxf(cm, dpp<kDppQuadXor2>(cm));
        const float mn = fmaxf(mt, cm);
        const float mu = (mn == -INFINITY) ? 0.0f : mn;
        // rescale only when some lane's running max moved (else alpha == 1)
        const bool rescale = __builtin_amdgcn_ballot_w64(mn > mt) != 0;
        float alpha = 1.0f;
        if (rescale) {
            alpha = __builtin_amdgcn_exp2f(mt - mu);
            lt *= alpha;
        }
        float pk[F], psum = 0.0f;
#pragma unroll
        for (int k = 0; k < F; ++k) {
            pk[k] = __builtin_amdgcn_exp2f(sv[k] - mu);
            psum += pk[k];
        }
        psum += dpp<kDppQuadXor1>(psum);
        if constexpr (F == 1) psum += dpp<kDppQuadXor2>(psum);
        lt += psum;
        mt = mn;
#pragma unroll
        for (int k = 0; k < F; ++k) {
            pbuf[F * l16 + k] = pk[k];
        }
        if (rescale && ((F * l16) & 3) == 0) {
            pbuf[NV + ((F * l16) >> 2)] = alpha;
        }
        // LDS operations of one wave execute in order: these reads see the
        // stores above; the fences only keep the compiler from reordering
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float pv[NV];
#pragma unroll
        for (int i = 0; i < NV / 4; ++i) {
            const float4 t4 = *(const float4 *)(pbuf + 4 * i);
            pv[4 * i] = t4.x;
            pv[4 * i + 1] = t4.y;
            pv[4 * i + 2] = t4.z;
            pv[4 * i + 3] = t4.w;
        }
        if (rescale) {
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float a = pbuf[NV + h];
#pragma unroll
                for (int j = 0; j < DPL; ++j) {
                    o[h][j] *= a;
                }
            }
        }
#pragma unroll
        for (int h = 0; h < G; ++h) {
#pragma unroll
            for (int j = 0; j < DPL; ++j) {
                float acc = o[h][j];
#pragma unroll
                for (int ps = 0; ps < 4; ++ps) {
                    acc += pv[h * 4 + ps] * frag_at<DPL>(vb[ps], j);
                }
                o[h][j] = acc;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
    };

    for (bool first = true; s0 < c_hi; first = false) {
        if (!first) {
            __syncthreads();  // previous sub-range done with the page ids
            setup_sub();
            load_chunk(ka, va, s0);
            load_chunk(kb, vb, s0 + 1);
        }
        auto run = [&](const Frag<DPL>(&kb)[4], Frag<DPL>(&vb)[4], uint32_t c) {
            const bool masked = c * kChunk < t0 || c * kChunk + kChunk > t1;
            if (masked) {
                // a masked token's probability is 0, but its V slot may hold
                // any bits (never written, or past a truncation) and 0 * NaN
                // is NaN: its V words are replaced by zeros
#pragma unroll
                for (int ps = 0; ps < 4; ++ps) {
                    const uint32_t tok = c * kChunk + ps * 16 + group;
                    if (tok < t0 || tok >= t1) {
#pragma unroll
                        for (int w = 0; w < DPL / 2; ++w) vb[ps].w[w] = 0u;
                    }
                }
            }
            if constexpr (kTransposed) {
                process_t(kb, vb, c, masked);
            } else {
                process(kb, vb, c, masked);
            }
        };

        for (uint32_t c = s0; c < s1; c += 3) {
            load_chunk(kc, vc, c + 2);
            run(ka, va, c);
            load_chunk(ka, va, c + 3);
            if (c + 1 < s1) {
                run(kb, vb, c + 1);
            }
            load_chunk(kb, vb, c + 4);
            if (c + 2 < s1) {
                run(kc, vc, c + 2);
            }
        }
        s0 = s1;
        s1 = min(s0 + p.sub_chunks, c_hi);
    }

    // 6. merge the four groups of each wave, then the four waves
    if constexpr (kTransposed) {
        // every lane of a head's quad / pair holds the same running state
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const int owner = (lane & ~15) + (4 * h) / F;
            mrun[h] = __shfl(mt, owner);
            lrun[h] = __shfl(lt, owner);
        }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
        float mx = fmaxf(mrun[h], __shfl_xor(mrun[h], 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mu = (mx == -INFINITY) ? 0.0f : mx;
        const float f = __builtin_amdgcn_exp2f(mrun[h] - mu);
        float l = lrun[h] * f;
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
            float v = o[h][j] * f;
            v += __shfl_xor(v, 16);
            v += __shfl_xor(v, 32);
            o[h][j] = v;
        }
        mrun[h] = mx;
        lrun[h] = l;
    }
    if (lane < 16) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
#pragma unroll
            for (int j = 0; j < DPL; ++j) {
                sh.red_o[wave][h][l16 * DPL + j] = o[h][j];
            }
            if (l16 == 0) {
                sh.red_m[wave][h] = mrun[h];
                sh.red_l[wave][h] = lrun[h];
            }
        }
    }
    __syncthreads();

    const size_t out_row = (size_t)row * p.heads * D;
    float *rec_base = p.partials + ((size_t)rec * p.kv_heads + kvh) * G * (D + 2);
    for (int idx = tid; idx < G * D; idx += kThreads) {
        const int h = idx / D;
        const int d = idx - h * D;
        float M = sh.red_m[0][h];
#pragma unroll
        for (int w = 1; w < 4; ++w) M = fmaxf(M, sh.red_m[w][h]);
        const float Mu = (M == -INFINITY) ? 0.0f : M;
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float f = __builtin_amdgcn_exp2f(sh.red_m[w][h] - Mu);
            L += sh.red_l[w][h] * f;
            O += sh.red_o[w][h][d] * f;
        }
        if (nrec == 1) {
            float r = O / L;
            if (gated) {
                r *= ref_sigmoid(load_act(p.q, q_row + (size_t)(kvh * G + h) * hs + D + d, bf16_in));
            }
            p.out[out_row + (size_t)(kvh * G + h) * D + d] = r;
        } else {
            float *r = rec_base + (size_t)h * (D + 2);
            r[2 + d] = O;
            if (d == 0) {
                r[0] = M;
                r[1] = L;
            }
        }
    }
}

template <int D, int G, bool kPageHoldsChunk>
__global__ void __launch_bounds__(kThreads) attn_decode_kernel(const DecodeParams p) {
    __shared__ DecodeShared<D, G> sh;
    const uint32_t kvh = blockIdx.x % p.kv_heads;
    const uint32_t part = blockIdx.x / p.kv_heads;
    uint32_t g0 = part * p.part_tokens;
    const uint32_t g1 = min(g0 + p.part_tokens, p.total_tokens);
    int s = 0;
    while (s + 1 < (int)p.nseq && p.meta[s + 1].start <= g0) {
        ++s;
    }
    while (g0 < g1) {
        const uint32_t start = p.meta[s].start;
        const uint32_t total = p.meta[s].ctx + 1;
        const uint32_t t0 = g0 - start;
        const uint32_t t1 = min(g1, start + total) - start;
        const uint32_t rec = p.meta[s].rec0 + (part - start / p.part_tokens);
        decode_segment<D, G, kPageHoldsChunk>(p, sh, s, kvh, t0, t1, rec);
        g0 = start + total;
        ++s;
    }
}

// Merges the per-segment (max, sum, output) records of every sequence that
// has more than one in one pass with a running rescale, and applies the
// output gate: one workgroup per (sequence, KV head) x query head of the
// group, one thread per output dim, so each thread's record loads are all in
// flight together.  It runs after attn_decode_kernel on the same stream, so
// the kernel boundary orders the records before they are read (no
// device-scope fences).
template <int D, int G>
__global__ void __launch_bounds__(D) attn_combine_kernel(const DecodeParams p) {
    const uint32_t kvh = blockIdx.x % p.kv_heads;
    const uint32_t s = blockIdx.x / p.kv_heads;
    const uint32_t nrec = p.meta[s].nrec;
    if (nrec == 1) {
        return;  // written directly by the decode kernel
    }
    const bool bf16_in = (p.flags & SAFETYRAISE_MI355X_INPUT_BF16) != 0;
    const bool gated = (p.flags & SAFETYRAISE_MI355X_GATED) != 0;
    const uint32_t hs = gated ? 2 * D : D;
    const uint32_t row = p.meta[s].row0;
    const size_t q_row = (size_t)row * p.heads * hs;
    const size_t out_row = (size_t)row * p.heads * D;
    const float *recs = p.partials + ((size_t)p.meta[s].rec0 * p.kv_heads + kvh) * G * (D + 2);
    const size_t rec_stride = (size_t)p.kv_heads * G * (D + 2);  // between records
    constexpr uint32_t kBatch = 8;  // independent loads in flight per thread
    {
        const int h = blockIdx.y;
        const int d = threadIdx.x;
        const float *r0 = recs + (size_t)h * (D + 2);
        float M = -INFINITY, L = 0.0f, O = 0.0f;
        for (uint32_t sp = 0; sp < nrec; sp += kBatch) {
            float mv[kBatch], lv[kBatch], ov[kBatch];
#pragma unroll
            for (uint32_t u = 0; u < kBatch; ++u) {
                const bool in = sp + u < nrec;
                const float *r = r0 + (in ? (sp + u) : 0) * rec_stride;
                mv[u] = in ? r[0] : -INFINITY;
                lv[u] = r[1];
                ov[u] = r[2 + d];
            }
            float bm = M;
#pragma unroll
            for (uint32_t u = 0; u < kBatch; ++u) bm = fmaxf(bm, mv[u]);
            const float scale = __builtin_amdgcn_exp2f(M - bm);  // M = -inf at first: 0
            L *= scale;
            O *= scale;
#pragma unroll
            for (uint32_t u = 0; u < kBatch; ++u) {
                const float f = __builtin_amdgcn_exp2f(mv[u] - bm);
                L += lv[u] * f;
                O += ov[u] * f;
            }
            M = bm;
        }
        float res = O / L;
        if (gated) {
            res *= ref_sigmoid(load_act(p.q, q_row + (size_t)(kvh * G + h) * hs + D + d, bf16_in));
        }
        p.out[out_row + (size_t)(kvh * G + h) * D + d] = res;
    }
}

template <int D, int G, bool kPageHoldsChunk>
int resident_blocks_per_cu() {
    static int n = [] {
        int v = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &v, attn_decode_kernel<D, G, kPageHoldsChunk>, kThreads, 0) != hipSuccess ||
            v < 1) {
            v = 1;
        }
        return v;
    }();
    return n;
}

template <int D, int G, bool kPageHoldsChunk>
hipError_t launch_dgp(hipStream_t stream, DecodeParams &prm, const DecodePlanInput &in) {
    // slices: as many workgroups as stay resident, at least 256 tokens each
    const uint64_t slots = (uint64_t)resident_blocks_per_cu<D, G, kPageHoldsChunk>() * in.num_cus;
    uint64_t parts = std::max<uint64_t>(slots / prm.kv_heads, 1);
    uint64_t part_tokens = (prm.total_tokens + parts - 1) / parts;
    part_tokens = std::max<uint64_t>((part_tokens + kChunk - 1) / kChunk * kChunk, 256);
    parts = (prm.total_tokens + part_tokens - 1) / part_tokens;
    prm.part_tokens = (uint32_t)part_tokens;
    uint32_t recs = 0;
    for (uint32_t i = 0; i < prm.nseq; ++i) {
        const uint32_t first = prm.meta[i].start / prm.part_tokens;
        const uint32_t last = (prm.meta[i].start + prm.meta[i].ctx) / prm.part_tokens;
        prm.meta[i].rec0 = recs;
        prm.meta[i].nrec = last - first + 1;
        recs += prm.meta[i].nrec;
    }
    float *partials = in.reserve_partials((size_t)recs * prm.kv_heads * G * (D + 2) * sizeof(float));
    if (partials == nullptr) {
        return hipErrorOutOfMemory;
    }
    prm.partials = partials;
    SR_LAUNCH("attn_decode_kernel", (attn_decode_kernel<D, G, kPageHoldsChunk>),
              dim3((uint32_t)parts * prm.kv_heads), dim3(kThreads), 0, stream, prm);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || recs == prm.nseq) {
        return e;  // every sequence in one segment: nothing to combine
    }
    SR_LAUNCH("attn_combine_kernel", (attn_combine_kernel<D, G>), dim3(prm.nseq * prm.kv_heads, G),
              dim3(D), 0, stream, prm);
    return hipGetLastError();
}

template <int D, int G>
hipError_t launch_dg(hipStream_t stream, DecodeParams &prm, const DecodePlanInput &in) {
    return prm.log2_page_tokens >= 6 ? launch_dgp<D, G, true>(stream, prm, in)
                                     : launch_dgp<D, G, false>(stream, prm, in);
}

template <int D>
hipError_t launch_d(hipStream_t stream, DecodeParams &prm, const DecodePlanInput &in, uint32_t g) {
    switch (g) {
        case 1: return launch_dg<D, 1>(stream, prm, in);
        case 2: return launch_dg<D, 2>(stream, prm, in);
        case 3: return launch_dg<D, 3>(stream, prm, in);
        case 4: return launch_dg<D, 4>(stream, prm, in);
        case 5: return launch_dg<D, 5>(stream, prm, in);
        case 6: return launch_dg<D, 6>(stream, prm, in);
        case 7: return launch_dg<D, 7>(stream, prm, in);
        case 8: return launch_dg<D, 8>(stream, prm, in);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_attn_decode(hipStream_t stream, const AttnLaunch &a, const SeqMeta *seqs,
                              int nseq, const DecodePlanInput &in) {
    DecodeParams prm;
    prm.k_pages = a.pool->k_pages;
    prm.v_pages = a.pool->v_pages;
    prm.page_table = a.pool->d_page_table;
    prm.q = a.q;
    prm.k = a.k;
    prm.v = a.v;
    prm.q_norm = a.q_norm;
    prm.k_norm = a.k_norm;
    prm.positions = a.positions;
    prm.out = a.out;
    prm.partials = nullptr;
    prm.err_word = a.err_word;
    prm.num_pages = a.pool->num_pages;
    prm.pages_per_seq = a.pool->pages_per_seq;
    prm.page_tokens = a.pool->page_tokens;
    prm.flags = a.flags;
    prm.heads = a.heads;
    prm.kv_heads = a.kv_heads * a.kv_rep;
    prm.kv_rep = a.kv_rep;
    prm.rotary_dim = a.rotary_dim;
    prm.mrope[0] = a.mrope[0];
    prm.mrope[1] = a.mrope[1];
    prm.mrope[2] = a.mrope[2];
    prm.eps = a.eps;
    // page_tokens is a power of two >= 16 (checked when the pool is created)
    prm.log2_page_tokens = (uint32_t)__builtin_ctz(a.pool->page_tokens);
    prm.sub_chunks = (kMaxSplitPages - 2) * a.pool->page_tokens / kChunk;
    prm.nseq = (uint32_t)nseq;
    prm.rope = *a.rope;
    uint64_t total = 0;
    for (int i = 0; i < nseq; ++i) {
        prm.meta[i].slot = seqs[i].slot;
        prm.meta[i].ctx = seqs[i].ctx;
        prm.meta[i].row0 = seqs[i].row0;
        prm.meta[i].start = (uint32_t)total;
        total += (uint64_t)seqs[i].ctx + 1;
    }
    if (total > 0x7fffffffull) {
        return hipErrorInvalidValue;  // the host splits packs below this
    }
    prm.total_tokens = (uint32_t)total;
    const uint32_t g = a.heads / prm.kv_heads;
    switch (a.head_dim) {
        case 64: return launch_d<64>(stream, prm, in, g);
        case 128: return launch_d<128>(stream, prm, in, g);
        case 256: return launch_d<256>(stream, prm, in, g);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace sr
