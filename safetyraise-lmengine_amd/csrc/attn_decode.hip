// Split-K decode attention for gfx950 (one new row per sequence).
//
// Replaces, for a batch of sequences, one pass of the Attention::forward row
// loop (reference src/model/native.rs:627-643): QK-RMSNorm and RoPE of the new
// row, append of its K/V to the paged cache, causal_attention over every
// cached token (src/model/math.rs:102-155), and the Qwen3.5 output gate.
//
// Work decomposition: one workgroup per (sequence, KV head, split of
// split_tokens cached tokens).  All G = heads/kv_heads query heads of the GQA
// group share each K/V load.  256 threads = 16 groups of 16 lanes; a group
// owns one token per pass, a lane owns D/16 consecutive dims, so one K or V
// row (D bf16) is one 16-lane 128-bit-per-lane load and a wave reads 4 whole
// rows per instruction.  Scores are reduced over the 16 lanes with DPP; PV
// needs no cross-lane traffic.  Each group keeps an online-softmax state per
// head in the log2 domain; groups, waves and finally splits are merged with
// the standard (max, sum, weighted output) combine.  The split workgroup that
// arrives last for a (sequence, KV head) combines all splits, so one launch
// does the whole step.  No MFMA: the step is HBM-bound (4 flop per byte).
#include "sr_device.hpp"

namespace sr {

namespace {

constexpr int kThreads = 256;
constexpr int kChunk = 64;          // tokens per loop iteration (4 passes x 16 groups)
constexpr int kMaxSplitPages = 256; // page ids of one split staged in LDS

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
    uint32_t *counters;
    uint32_t *err_word;
    uint32_t pages_per_seq;
    uint32_t page_tokens;
    uint32_t flags;
    uint32_t heads;
    uint32_t kv_heads;
    uint32_t rotary_dim;
    uint32_t mrope[3];
    float eps;
    uint32_t split_tokens;
    uint32_t nseq;
    RopeTable rope;
    MetaPack meta;
};

// D/16 bf16 values of one K or V row owned by a lane.
template <int DPL>
struct Frag {
    uint32_t w[DPL / 2];
};

template <int DPL>
__device__ __forceinline__ Frag<DPL> load_frag(const uint16_t *p) {
    Frag<DPL> f;
    if constexpr (DPL == 4) {
        const uint2 x = *(const uint2 *)p;
        f.w[0] = x.x;
        f.w[1] = x.y;
    } else {
#pragma unroll
        for (int i = 0; i < DPL / 8; ++i) {
            const uint4 x = *((const uint4 *)p + i);
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
__global__ void __launch_bounds__(kThreads) attn_decode_kernel(const DecodeParams p) {
    constexpr int DPL = D / 16;  // dims per lane in the main loop
    constexpr int EPL = D / 64;  // elements per lane while normalising
    __shared__ float vec_s[G + 1][D];  // q heads of the group, then the new k
    __shared__ int32_t page_s[kMaxSplitPages];
    __shared__ float red_m[4][G];
    __shared__ float red_l[4][G];
    __shared__ float red_o[4][G][D];
    __shared__ int last_s;

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int group = tid >> 4;
    const int l16 = tid & 15;

    const uint32_t kvh = blockIdx.x % p.kv_heads;
    const uint32_t gsplit = blockIdx.x / p.kv_heads;
    int s = 0;
    while (s + 1 < (int)p.nseq && p.meta.m[s + 1].split0 <= gsplit) {
        ++s;
    }
    const uint32_t slot = p.meta.m[s].slot;
    const uint32_t ctx = p.meta.m[s].ctx;
    const uint32_t row = p.meta.m[s].row0;
    const uint32_t split = gsplit - p.meta.m[s].split0;
    const uint32_t total = ctx + 1;
    const uint32_t nsplit = (total + p.split_tokens - 1) / p.split_tokens;
    const uint32_t t0 = split * p.split_tokens;
    const uint32_t t1 = min(t0 + p.split_tokens, total);
    const bool owns_new = (t1 == total);

    const bool bf16_in = (p.flags & SAFETYRAISE_MI355X_INPUT_BF16) != 0;
    const bool gated = (p.flags & SAFETYRAISE_MI355X_GATED) != 0;
    const bool qk_norm = (p.flags & SAFETYRAISE_MI355X_QK_NORM) != 0;
    const bool interleaved = (p.flags & SAFETYRAISE_MI355X_MROPE_INTERLEAVED) != 0;
    const float norm_add = (p.flags & SAFETYRAISE_MI355X_NORM_OFFSET) ? 1.0f : 0.0f;
    const uint32_t hs = gated ? 2 * D : D;  // q elements per head
    const size_t q_row = (size_t)row * p.heads * hs;
    const size_t kv_row = ((size_t)row * p.kv_heads + kvh) * D;
    const uint32_t PT = p.page_tokens;

    // 1. page ids covering [t0, t1)
    const uint32_t pg0 = t0 / PT;
    const uint32_t npg = (t1 - 1) / PT - pg0 + 1;
    const int32_t *table = p.page_table + (size_t)slot * p.pages_per_seq;
    for (uint32_t i = tid; i < npg; i += kThreads) {
        page_s[i] = table[pg0 + i];
    }

    // 2. per-head RMSNorm of the group's q heads (and of the new k)
    //    (src/model/math.rs:28-50 via native.rs:629-634)
    const int nvec = G + (owns_new ? 1 : 0);
    for (int h = wave; h < nvec; h += 4) {
        float x[EPL];
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
            const int e = lane + 64 * i;
            x[i] = (h < G) ? load_act(p.q, q_row + (size_t)(kvh * G + h) * hs + e, bf16_in)
                           : load_act(p.k, kv_row + e, bf16_in);
            ss += x[i] * x[i];
        }
        if (qk_norm) {
            ss = sum64(ss);
            const float variance = ss / (float)D;
            if (!isfinite(variance) && lane == 0) {
                atomicOr(p.err_word, kErrNonFiniteVariance);
            }
            const float inv = 1.0f / sqrtf(variance + p.eps);
            const float *w = (h < G) ? p.q_norm : p.k_norm;
#pragma unroll
            for (int i = 0; i < EPL; ++i) {
                x[i] = x[i] * inv * (w[lane + 64 * i] + norm_add);
            }
        }
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
            vec_s[h][lane + 64 * i] = x[i];
        }
    }
    __syncthreads();

    // 3. RoPE, rotate-half over the first rotary_dim dims (math.rs:52-99);
    //    angle = pos / theta^(2i/rotary_dim) with an IEEE f32 division
    const uint32_t half = p.rotary_dim / 2;
    const int32_t *pos3 = p.positions + (size_t)row * 3;
    for (uint32_t idx = tid; idx < (uint32_t)nvec * half; idx += kThreads) {
        const uint32_t h = idx / half;
        const uint32_t i = idx - h * half;
        const int axis = rope_axis(i, p.mrope, interleaved);
        const float angle = (float)pos3[axis] / p.rope.denom[i];
        float sn, cs;
        sincosf(angle, &sn, &cs);
        const float left = vec_s[h][i];
        const float right = vec_s[h][i + half];
        vec_s[h][i] = left * cs - right * sn;
        vec_s[h][i + half] = right * cs + left * sn;
    }
    __syncthreads();

    // 4. append the new token's k and v (bf16, round to nearest even)
    if (owns_new) {
        const uint32_t tok = ctx;
        const int32_t page = page_s[tok / PT - pg0];
        const size_t base = (((size_t)page * p.kv_heads + kvh) * PT + tok % PT) * D;
        for (int e = tid; e < D; e += kThreads) {
            const float kk = vec_s[G][e];
            const float vv = load_act(p.v, kv_row + e, bf16_in);
            if (!isfinite(kk) || !isfinite(vv)) {
                atomicOr(p.err_word, kErrNonFiniteKv);
            }
            p.k_pages[base + e] = f32_to_bf16(kk);
            p.v_pages[base + e] = f32_to_bf16(vv);
        }
        __syncthreads();
    }

    // 5. q fragments, prescaled by 1/sqrt(D) * log2(e)
    const float qscale = (1.0f / sqrtf((float)D)) * kLog2e;
    float qf[G][DPL];
#pragma unroll
    for (int h = 0; h < G; ++h) {
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
            qf[h][j] = vec_s[h][l16 * DPL + j] * qscale;
        }
    }

    // 6. stream the split's K/V, online softmax per group and head
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
    const size_t head_off = (size_t)kvh * PT;
    auto frag_base = [&](uint32_t tok) -> size_t {
        const int32_t page = page_s[tok / PT - pg0];
        return (((size_t)page * p.kv_heads) * PT + head_off + tok % PT) * D + l16 * DPL;
    };

    Frag<DPL> kf[4], vf[4];
    {
#pragma unroll
        for (int ps = 0; ps < 4; ++ps) {
            const uint32_t tok = min(t0 + ps * 16 + group, t1 - 1);
            const size_t b = frag_base(tok);
            kf[ps] = load_frag<DPL>(p.k_pages + b);
            vf[ps] = load_frag<DPL>(p.v_pages + b);
        }
    }
    for (uint32_t cb = t0; cb < t1; cb += kChunk) {
        Frag<DPL> kn[4], vn[4];
        const bool more = cb + kChunk < t1;
        if (more) {
#pragma unroll
            for (int ps = 0; ps < 4; ++ps) {
                const uint32_t tok = min(cb + kChunk + ps * 16 + group, t1 - 1);
                const size_t b = frag_base(tok);
                kn[ps] = load_frag<DPL>(p.k_pages + b);
                vn[ps] = load_frag<DPL>(p.v_pages + b);
            }
        }
        float sc[4][G];
#pragma unroll
        for (int ps = 0; ps < 4; ++ps) {
            const bool valid = cb + ps * 16 + group < t1;
#pragma unroll
            for (int h = 0; h < G; ++h) {
                float acc = 0.0f;
#pragma unroll
                for (int j = 0; j < DPL; ++j) {
                    acc += qf[h][j] * frag_at<DPL>(kf[ps], j);
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
            const float alpha = __builtin_amdgcn_exp2f(mrun[h] - mu);
            float pp[4];
#pragma unroll
            for (int ps = 0; ps < 4; ++ps) {
                pp[ps] = __builtin_amdgcn_exp2f(sc[ps][h] - mu);
            }
            lrun[h] = lrun[h] * alpha + ((pp[0] + pp[1]) + (pp[2] + pp[3]));
#pragma unroll
            for (int j = 0; j < DPL; ++j) {
                float acc = o[h][j] * alpha;
#pragma unroll
                for (int ps = 0; ps < 4; ++ps) {
                    acc += pp[ps] * frag_at<DPL>(vf[ps], j);
                }
                o[h][j] = acc;
            }
            mrun[h] = mn;
        }
        if (more) {
#pragma unroll
            for (int ps = 0; ps < 4; ++ps) {
                kf[ps] = kn[ps];
                vf[ps] = vn[ps];
            }
        }
    }

    // 7. merge the four groups of each wave, then the four waves
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
                red_o[wave][h][l16 * DPL + j] = o[h][j];
            }
            if (l16 == 0) {
                red_m[wave][h] = mrun[h];
                red_l[wave][h] = lrun[h];
            }
        }
    }
    __syncthreads();

    const size_t out_row = (size_t)row * p.heads * D;
    float *rec_base = p.partials + ((size_t)gsplit * p.kv_heads + kvh) * G * (D + 2);
    for (int idx = tid; idx < G * D; idx += kThreads) {
        const int h = idx / D;
        const int d = idx - h * D;
        float M = red_m[0][h];
#pragma unroll
        for (int w = 1; w < 4; ++w) M = fmaxf(M, red_m[w][h]);
        const float Mu = (M == -INFINITY) ? 0.0f : M;
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float f = __builtin_amdgcn_exp2f(red_m[w][h] - Mu);
            L += red_l[w][h] * f;
            O += red_o[w][h][d] * f;
        }
        if (nsplit == 1) {
            float r = O / L;
            if (gated) {
                r *= ref_sigmoid(load_act(p.q, q_row + (size_t)(kvh * G + h) * hs + D + d, bf16_in));
            }
            p.out[out_row + (size_t)(kvh * G + h) * D + d] = r;
        } else {
            float *rec = rec_base + (size_t)h * (D + 2);
            rec[2 + d] = O;
            if (d == 0) {
                rec[0] = M;
                rec[1] = L;
            }
        }
    }
    if (nsplit == 1) {
        return;
    }

    // 8. the last split to arrive for (sequence, KV head) combines all splits
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev = atomicAdd(&p.counters[s * p.kv_heads + kvh], 1u);
        last_s = (prev == nsplit - 1) ? 1 : 0;
    }
    __syncthreads();
    if (last_s == 0) {
        return;
    }
    __threadfence();
    const float *recs = p.partials + ((size_t)p.meta.m[s].split0 * p.kv_heads + kvh) * G * (D + 2);
    const size_t rec_stride = (size_t)p.kv_heads * G * (D + 2);  // between splits
    for (int idx = tid; idx < G * D; idx += kThreads) {
        const int h = idx / D;
        const int d = idx - h * D;
        const float *r0 = recs + (size_t)h * (D + 2);
        float M = -INFINITY;
        for (uint32_t sp = 0; sp < nsplit; ++sp) {
            M = fmaxf(M, r0[sp * rec_stride]);
        }
        float L = 0.0f, O = 0.0f;
        for (uint32_t sp = 0; sp < nsplit; ++sp) {
            const float *r = r0 + sp * rec_stride;
            const float f = __builtin_amdgcn_exp2f(r[0] - M);
            L += r[1] * f;
            O += r[2 + d] * f;
        }
        float res = O / L;
        if (gated) {
            res *= ref_sigmoid(load_act(p.q, q_row + (size_t)(kvh * G + h) * hs + D + d, bf16_in));
        }
        p.out[out_row + (size_t)(kvh * G + h) * D + d] = res;
    }
    if (tid == 0) {
        atomicExch(&p.counters[s * p.kv_heads + kvh], 0u);
    }
}

template <int D, int G>
hipError_t launch_dg(hipStream_t stream, const DecodeParams &prm, uint32_t blocks) {
    hipLaunchKernelGGL((attn_decode_kernel<D, G>), dim3(blocks), dim3(kThreads), 0, stream, prm);
    return hipGetLastError();
}

template <int D>
hipError_t launch_d(hipStream_t stream, const DecodeParams &prm, uint32_t blocks, uint32_t g) {
    switch (g) {
        case 1: return launch_dg<D, 1>(stream, prm, blocks);
        case 2: return launch_dg<D, 2>(stream, prm, blocks);
        case 3: return launch_dg<D, 3>(stream, prm, blocks);
        case 4: return launch_dg<D, 4>(stream, prm, blocks);
        case 5: return launch_dg<D, 5>(stream, prm, blocks);
        case 6: return launch_dg<D, 6>(stream, prm, blocks);
        case 7: return launch_dg<D, 7>(stream, prm, blocks);
        case 8: return launch_dg<D, 8>(stream, prm, blocks);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

uint32_t decode_max_split_pages() { return kMaxSplitPages; }

hipError_t launch_attn_decode(hipStream_t stream, const AttnLaunch &a, const MetaPack &meta,
                              int nseq, uint32_t splits_total, uint32_t split_tokens,
                              float *partials, uint32_t *counters) {
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
    prm.partials = partials;
    prm.counters = counters;
    prm.err_word = a.err_word;
    prm.pages_per_seq = a.pool->pages_per_seq;
    prm.page_tokens = a.pool->page_tokens;
    prm.flags = a.flags;
    prm.heads = a.heads;
    prm.kv_heads = a.kv_heads;
    prm.rotary_dim = a.rotary_dim;
    prm.mrope[0] = a.mrope[0];
    prm.mrope[1] = a.mrope[1];
    prm.mrope[2] = a.mrope[2];
    prm.eps = a.eps;
    prm.split_tokens = split_tokens;
    prm.nseq = (uint32_t)nseq;
    prm.rope = *a.rope;
    prm.meta = meta;
    const uint32_t blocks = splits_total * a.kv_heads;
    const uint32_t g = a.heads / a.kv_heads;
    switch (a.head_dim) {
        case 64: return launch_d<64>(stream, prm, blocks, g);
        case 128: return launch_d<128>(stream, prm, blocks, g);
        case 256: return launch_d<256>(stream, prm, blocks, g);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace sr
