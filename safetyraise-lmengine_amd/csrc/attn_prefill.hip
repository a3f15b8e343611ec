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
//   kv_append_rows_kernel  one wave per new row (four per workgroup): the
//                          row's RoPE cos/sin (once per rotary pair, also
//                          saved for the q side), the call's page-table
//                          entries when they travel in the arguments,
//                          K RMSNorm + RoPE and V of every KV head, rounded
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
//
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
#include <type_traits>

#include "sr_device.hpp"

namespace sr {

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kRowTile = 32;   // query rows per wave (the MFMA N dimension)
constexpr int kKeyTile = 64;   // keys per LDS stage
constexpr float kLazyRescale = 8.0f;

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
    float2 *rope_cs;  // [call rows][rotary_dim/2] (cos, sin), written by the append kernel
    uint32_t *err_word;
    uint64_t num_pages;
    uint32_t pages_per_seq;
    uint32_t log2_page_tokens;
    uint32_t flags;
    uint32_t heads;
    uint32_t kv_heads;        // KV heads as the attention grids see them: the cache's times kv_rep
    uint32_t kv_rep;          // query-head groups per cache KV head (groups of more
                              // than 8 heads run as kv_rep groups of heads/kv_heads)
    uint32_t cache_kv_heads;  // the cache's KV heads (the append kernel's)
    uint32_t rotary_dim;
    uint32_t mrope[3];
    float eps;
    uint32_t nseq;
    uint32_t max_blk;
    RopeTable rope;
    PrefillMeta meta[kMetaPerLaunch];
    // page-table entries the append kernel writes (and uses for its own rows)
    uint32_t tbl_n;
    uint32_t tbl_idx[kInlineTable];
    int32_t tbl_val[kInlineTable];
};

// Max / sum of x over lanes l and l^32 (both halves get the same bits).
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
// Materialises x in registers at this point of the program: register-only
// work that produced x cannot be moved past it (for example across a
// barrier into the next phase).
template <typename T>
__device__ __forceinline__ void pin(T &x) {
    asm volatile("" : "+v"(x));
}
// The same for a wave-uniform value: it must be in scalar registers here, so
// a kernel-argument load completes at this point (loads issued together
// complete together) and is not re-issued later at each use.
template <typename T>
__device__ __forceinline__ void pin_s(T &x) {
    asm volatile("" : "+s"(x));
}

// Sum of the 8 fp16 values of x added to acc in f32 (v_dot2_f32_f16 with 1s).
__device__ __forceinline__ float sum_f16x8(const f16x8 &x, float acc) {
    const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        acc = __builtin_amdgcn_fdot2(f16x2{x[2 * j], x[2 * j + 1]}, one, acc, false);
    }
    return acc;
}

// ---------------------------------------------------------------------------
// K/V append of every new row.  One wave per row: 16 lanes per KV head, D/16
// contiguous elements per lane (one 16-byte load per tensor at D = 128), four
// heads per pass and two passes' loads in flight together; the row's RoPE
// table is computed once.  Rows are independent and short, so the whole
// call's loads are in flight together.
// ---------------------------------------------------------------------------
constexpr int kAppendHeadsPerWave = 4;

// EPL consecutive activations (bf16 or f32) from element i on, widened to f32.
template <int EPL>
__device__ __forceinline__ void load_span(const void *base, size_t i, bool bf16, float (&x)[EPL]) {
    if (bf16) {
        const uint32_t *w = (const uint32_t *)((const uint16_t *)base + i);
        if constexpr (EPL % 8 == 0) {
#pragma unroll
            for (int c = 0; c < EPL / 8; ++c) {
                const u32x4 v = ((const u32x4 *)w)[c];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    x[8 * c + 2 * j] = bf16lo(v[j]);
                    x[8 * c + 2 * j + 1] = bf16hi(v[j]);
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < EPL / 2; ++j) {
                const uint32_t v = w[j];
                x[2 * j] = bf16lo(v);
                x[2 * j + 1] = bf16hi(v);
            }
        }
    } else {
        const float4 *f = (const float4 *)((const float *)base + i);
#pragma unroll
        for (int c = 0; c < EPL / 4; ++c) {
            const float4 v = f[c];
            x[4 * c] = v.x;
            x[4 * c + 1] = v.y;
            x[4 * c + 2] = v.z;
            x[4 * c + 3] = v.w;
        }
    }
}

// EPL f32 values rounded to bf16 and stored from element i on.
template <int EPL>
__device__ __forceinline__ void store_span_bf16(uint16_t *base, size_t i, const float (&x)[EPL]) {
    uint32_t w[EPL / 2];
#pragma unroll
    for (int j = 0; j < EPL / 2; ++j) w[j] = pack_bf16x2(x[2 * j], x[2 * j + 1]);
    if constexpr (EPL % 8 == 0) {
#pragma unroll
        for (int c = 0; c < EPL / 8; ++c) {
            ((u32x4 *)(base + i))[c] = u32x4{w[4 * c], w[4 * c + 1], w[4 * c + 2], w[4 * c + 3]};
        }
    } else {
#pragma unroll
        for (int j = 0; j < EPL / 2; ++j) ((uint32_t *)(base + i))[j] = w[j];
    }
}

template <int D, bool kBf16In>
__global__ __launch_bounds__(256) void kv_append_rows_kernel(const PrefillParams p) {
    constexpr int EPL = D / 16;
    constexpr int HW = kAppendHeadsPerWave;
    __shared__ float cs_s[4][D / 2];
    __shared__ float sn_s[4][D / 2];
    // normalised K of two head quads, for the rotate-half partners
    __shared__ __align__(16) float xs[4][2][HW][D];
    const int tid = threadIdx.x;
    const int wave = wave_index();
    const int lane = tid & 63;
    const int slot = lane >> 4;  // head of the quad this lane works on
    const int l16 = lane & 15;
    const PrefillMeta m = p.meta[blockIdx.y];
    // the kernel arguments used below, read in one batch and waited for once
    // (left to itself the compiler reads each just before its first use,
    // several dependent scalar round trips ahead of the first vector load)
    uint64_t bk = (uint64_t)p.k, bv = (uint64_t)p.v, bkn = (uint64_t)p.k_norm,
             bpt = (uint64_t)p.page_table, bpos = (uint64_t)p.positions, bcs = (uint64_t)p.rope_cs,
             berr = (uint64_t)p.err_word, bkp = (uint64_t)p.k_pages, bvp = (uint64_t)p.v_pages;
    uint32_t kv_heads = p.cache_kv_heads, flags = p.flags, pages_per_seq = p.pages_per_seq,
             lpt = p.log2_page_tokens, rotary_dim = p.rotary_dim, num_pages = p.num_pages,
             tbl_n = p.tbl_n, m_slot = m.slot, m_ctx = m.ctx, m_rows = m.rows, m_row0 = m.row0;
    uint32_t mrope[3] = {p.mrope[0], p.mrope[1], p.mrope[2]};
    float eps = p.eps;
    asm volatile("" : "+s"(bk), "+s"(bv), "+s"(bkn), "+s"(bpt), "+s"(bpos), "+s"(bcs), "+s"(berr),
                 "+s"(bkp), "+s"(bvp), "+s"(kv_heads), "+s"(flags), "+s"(pages_per_seq), "+s"(lpt),
                 "+s"(rotary_dim), "+s"(num_pages), "+s"(eps), "+s"(tbl_n), "+s"(m_slot),
                 "+s"(m_ctx), "+s"(m_rows), "+s"(m_row0), "+s"(mrope[0]), "+s"(mrope[1]),
                 "+s"(mrope[2]));
    const void *k_in = global_from_bits<const void>(bk);
    const void *v_in = global_from_bits<const void>(bv);
    const float *k_norm = global_from_bits<const float>(bkn);
    const int32_t *page_table = global_from_bits<const int32_t>(bpt);
    const int32_t *positions = global_from_bits<const int32_t>(bpos);
    float2 *rope_cs = global_from_bits<float2>(bcs);
    uint32_t *err_word = global_from_bits<uint32_t>(berr);
    uint16_t *k_pages = global_from_bits<uint16_t>(bkp);
    uint16_t *v_pages = global_from_bits<uint16_t>(bvp);
    // entries of this call's page-table update: block (0,0) writes them for
    // the kernels that follow; every row takes its own page from the list
    // (the table itself may not hold it yet)
    if (blockIdx.x == 0 && blockIdx.y == 0) {
        for (uint32_t i = tid; i < tbl_n; i += 256) {
            ((int32_t *)page_table)[p.tbl_idx[i]] = p.tbl_val[i];
        }
    }
    // one wave per row (all its KV heads); no barrier below, so a wave past
    // the rows just ends
    const uint32_t r = blockIdx.x * 4 + wave;
    if (r >= m_rows) return;
    const uint32_t row = m_row0 + r;
    // the input type is a template parameter: a run-time branch around the
    // span loads would end each in a wait for every load in flight
    constexpr bool bf16_in = kBf16In;
    const bool qk_norm = (flags & SAFETYRAISE_MI355X_QK_NORM) != 0;
    const bool interleaved = (flags & SAFETYRAISE_MI355X_MROPE_INTERLEAVED) != 0;
    const float norm_add = (flags & SAFETYRAISE_MI355X_NORM_OFFSET) ? 1.0f : 0.0f;
    const uint32_t quads = (kv_heads + HW - 1) / HW;
    const uint32_t e0 = l16 * EPL;  // first element of this lane

    // the RoPE table's inputs (the row's three position axes, this lane's
    // frequency denominators) and the row's page are requested first, then
    // the K/V of two head quads at a time (the second repeats the last head
    // when the row has fewer), with no wait in between: the table is computed
    // while the K/V loads are in flight
    const uint32_t half = rotary_dim / 2;
    constexpr int NTAB = (D / 2 + 63) / 64;  // table entries per lane
    const int32_t *pos3 = positions + (size_t)row * 3;
    const int32_t pz0 = pos3[0], pz1 = pos3[1], pz2 = pos3[2];
    float den[NTAB];
#pragma unroll
    for (int k = 0; k < NTAB; ++k) den[k] = p.rope.denom[min((uint32_t)lane + 64 * k, half - 1)];
    const uint32_t tok = m_ctx + r;
    const uint32_t tidx = m_slot * pages_per_seq + (tok >> lpt);
    int32_t page = page_table[tidx];
    const uint32_t ti = p.tbl_idx[min((uint32_t)lane, kInlineTable - 1)];
    float x[2][EPL], vv[2][EPL];
    uint32_t kvh[2];
    bool head_ok[2];
    auto load_quads = [&](uint32_t q0) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t kvh_raw = (q0 + j) * HW + slot;
            head_ok[j] = kvh_raw < kv_heads;
            kvh[j] = min(kvh_raw, kv_heads - 1);
            const size_t src = ((size_t)row * kv_heads + kvh[j]) * D + e0;
            load_span<EPL>(k_in, src, bf16_in, x[j]);
            load_span<EPL>(v_in, src, bf16_in, vv[j]);
        }
    };
    load_quads(0);
    float wk[EPL];
    load_span<EPL>(k_norm, e0, false, wk);  // readable without QK-norm too
    {
        const uint64_t mask = __builtin_amdgcn_ballot_w64((uint32_t)lane < tbl_n && ti == tidx);
        if (mask != 0) page = p.tbl_val[__builtin_ctzll(mask)];
    }
    const uint32_t pt_mask = (1u << lpt) - 1;
    const size_t dst_tok = (((size_t)page << lpt) + (tok & pt_mask)) * D + e0;
    const size_t head_stride = ((size_t)num_pages << lpt) * D;

    // RoPE angle of pair i: pos[axis(i)] / theta^(2i/rotary_dim) with an IEEE
    // f32 division (math.rs:90-91); the row's table, saved for the q side at
    // the end (a store issued here would hold up the wait for the K/V loads)
    float tab_cs[NTAB], tab_sn[NTAB];
#pragma unroll
    for (int k = 0; k < NTAB; ++k) {
        const uint32_t i = lane + 64 * k;
        if (i < half) {
            const int axis = rope_axis(i, mrope, interleaved);
            const int32_t pos = axis == 0 ? pz0 : axis == 1 ? pz1 : pz2;
            const float angle = (float)pos / den[k];
            sincosf(angle, &tab_sn[k], &tab_cs[k]);
            cs_s[wave][i] = tab_cs[k];
            sn_s[wave][i] = tab_sn[k];
        }
    }
    bool finite = true;
    for (uint32_t q0 = 0;;) {
        if (qk_norm) {
            // rms_norm (math.rs:28-50): x * (1/sqrt(mean(x^2)+eps)) * (w + offset)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                float ss = 0.0f;
#pragma unroll
                for (int i = 0; i < EPL; ++i) ss += x[j][i] * x[j][i];
                ss = sum16(ss);
                const float variance = ss / (float)D;
                if (!isfinite(variance) && l16 == 0 && head_ok[j]) {
                    atomicOr(err_word, kErrNonFiniteVariance);
                }
                const float inv = 1.0f / sqrtf(variance + eps);
#pragma unroll
                for (int i = 0; i < EPL; ++i) x[j][i] = x[j][i] * inv * (wk[i] + norm_add);
            }
        }
        // rotate-half over the first rotary_dim dims (math.rs:52-99): element
        // e pairs with e +- half, held by another lane of the same head; the
        // partners go through this wave's LDS (LDS operations of one wave are
        // performed in order, so no barrier is needed).  Every read is issued
        // (indices clamped into the arrays) before the one wait, and the
        // unrotated dims keep x.
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int c = 0; c < EPL / 4; ++c) {
                *(float4 *)&xs[wave][j][slot][e0 + 4 * c] =
                    make_float4(x[j][4 * c], x[j][4 * c + 1], x[j][4 * c + 2], x[j][4 * c + 3]);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float y[2][EPL];
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
            const uint32_t e = e0 + i;
            const bool lo = e < half;
            const uint32_t pi = min(lo ? e : e - half, (uint32_t)(D / 2 - 1));
            const uint32_t pe = min(lo ? e + half : e - half, (uint32_t)(D - 1));
            const float cs = cs_s[wave][pi], sn = sn_s[wave][pi];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const float partner = xs[wave][j][slot][pe];
                const float rot = lo ? x[j][i] * cs - partner * sn : x[j][i] * cs + partner * sn;
                y[j][i] = e < rotary_dim ? rot : x[j][i];
            }
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            bool ok = true;
#pragma unroll
            for (int i = 0; i < EPL; ++i) ok = ok && isfinite(y[j][i]) && isfinite(vv[j][i]);
            finite = finite && (ok || !head_ok[j]);
            if (head_ok[j]) {
                const size_t dst = kvh[j] * head_stride + dst_tok;
                store_span_bf16<EPL>(k_pages, dst, y[j]);
                store_span_bf16<EPL>(v_pages, dst, vv[j]);
            }
        }
        q0 += 2;
        if (q0 >= quads) break;
        load_quads(q0);
    }
#pragma unroll
    for (int k = 0; k < NTAB; ++k) {
        const uint32_t i = lane + 64 * k;
        if (i < half) rope_cs[(size_t)row * half + i] = make_float2(tab_cs[k], tab_sn[k]);
    }
    if (__builtin_amdgcn_ballot_w64(!finite) != 0 && lane == 0) {
        atomicOr(err_word, kErrNonFiniteKv);
    }
}

// One call's append: one wave per row, four per workgroup.
template <int D>
void launch_append(hipStream_t stream, const PrefillParams &p, uint32_t max_rows) {
    const dim3 grid((max_rows + 3) / 4, p.nseq);
    if (p.flags & SAFETYRAISE_MI355X_INPUT_BF16) {
        SR_LAUNCH("kv_append_rows_kernel", (kv_append_rows_kernel<D, true>), grid, dim3(256), 0, stream, p);
    } else {
        SR_LAUNCH("kv_append_rows_kernel", (kv_append_rows_kernel<D, false>), grid, dim3(256), 0, stream, p);
    }
}

// ---------------------------------------------------------------------------
// Attention.  LDS per stage: K tile [64 keys][D] and V^T tile [D][64 keys],
// both fp16, in 16-byte units XOR-swizzled so that MFMA operand reads (16
// lanes on 16 consecutive rows) and tile writes spread over the banks with
// 32 as well as with 64 four-byte banks.
//
// V^T column order.  The accumulator of S^T gives lane l (half h = l/32) the
// keys 8a + 4h + b (a, b < 4) of each 32-key half tile.  The PV product takes
// its B operand (8 keys per lane) straight from those registers, so V^T
// column 16s + 8h + j holds key 16s + 4h + 8(j/4) + (j%4): the A operand of
// step s is then one contiguous 16-byte read.
// ---------------------------------------------------------------------------
template <int D>
constexpr size_t kTileBytes = (size_t)kKeyTile * D * 2;  // one K or V^T tile

// 16-byte unit swizzles: K rows have D/8 units, V^T rows (64 keys) have 8.
template <int D>
__device__ __forceinline__ uint32_t k_swz(uint32_t key) {
    return (D >= 128) ? (key & 15) : (key & 7);
}
__device__ __forceinline__ uint32_t vt_swz(uint32_t d) {
    return ((d >> 1) & 7) ^ ((d & 1) << 2) ^ ((d >> 4) & 7);
}
// Row-major V tiles ([64 keys][D] fp16, like K) read by transposing loads:
// unit c of key row r sits at unit c ^ ((r & 3) << 2), so that one
// transposing read (8 rows x 4 units, 16 lanes per 4 rows x 2 units) meets
// every bank once per half wave.
__device__ __forceinline__ uint32_t v_swz(uint32_t key) { return (key & 3u) << 2; }

// Where one workgroup's rows are: (sequence, KV head, row block) from the
// block index, with the KV head fastest (the 8 XCDs take consecutive blocks,
// so one KV head's blocks share an L2), then the sequence, then the row block
// with the last (longest) blocks first.
struct BlockPos {
    PrefillMeta m;
    uint32_t kvh;
    uint32_t row0;    // first row of the block in the sequence
    uint32_t n_keys;  // keys visible to the block's last row
    uint32_t n_tiles;
    bool active;
};
__device__ __forceinline__ BlockPos block_pos(const PrefillParams &p, uint32_t rows_per_block) {
    BlockPos b;
    const uint32_t t2 = blockIdx.x / p.kv_heads;
    b.kvh = blockIdx.x % p.kv_heads;
    b.m = p.meta[t2 % p.nseq];
    const uint32_t qb = p.max_blk - 1 - t2 / p.nseq;
    b.active = qb < b.m.nblk;
    b.row0 = qb * rows_per_block;
    const uint32_t last = min(b.row0 + rows_per_block, b.m.rows) - 1;
    b.n_keys = b.m.ctx + last + 1;
    b.n_tiles = (b.n_keys + kKeyTile - 1) / kKeyTile;
    return b;
}

// Global -> register -> LDS movement of K and V tiles for a group of NTHR
// threads (gt = thread index in the group).  K goes to LDS as fp16 [key][D]
// (16-byte chunks), V as fp16 V^T (a thread owns 4 consecutive keys x 8 dims
// and transposes them with the fp16 conversion).
template <int D, int NTHR, bool kTilePage>
struct TileIo {
    static constexpr int KCH = D / 8;  // 16-byte chunks per K row
    static constexpr int KL = (kKeyTile * KCH + NTHR - 1) / NTHR;
    static constexpr int VU = (kKeyTile / 4) * KCH;  // (4-key group, chunk) units of a V tile
    static constexpr int VL = (VU + NTHR - 1) / NTHR;
    uint32_t k_goff[KL], k_loff[KL], v_goff[VL];
    uint32_t v_loff[VL][8];
    bool k_on[KL], v_on[VL];
    const uint16_t *k_pages;
    const uint16_t *v_pages;
    const int32_t *table;  // page ids; entry i is page table_first + i
    size_t head_base;
    uint32_t lpt, pt_mask, n_keys, n_tiles, table_first;

    __device__ __forceinline__ void init(int gt, const PrefillParams &p, const BlockPos &b) {
        k_pages = p.k_pages;
        v_pages = p.v_pages;
        table = p.page_table + (size_t)b.m.slot * p.pages_per_seq;
        table_first = 0;
        head_base = (size_t)(b.kvh / p.kv_rep) * p.num_pages;  // the cache's head
        lpt = p.log2_page_tokens;
        pt_mask = (1u << lpt) - 1;
        n_keys = b.n_keys;
        n_tiles = b.n_tiles;
#pragma unroll
        for (int i = 0; i < KL; ++i) {
            const int c = gt + i * NTHR;
            k_on[i] = (KL * NTHR == kKeyTile * KCH) || c < kKeyTile * KCH;
            const int key = k_on[i] ? c / KCH : 0, ch = c % KCH;
            k_goff[i] = key * D + ch * 8;
            k_loff[i] = key * (D * 2) + ((ch ^ k_swz<D>(key)) * 16);
        }
#pragma unroll
        for (int i = 0; i < VL; ++i) {
            const int u = gt + i * NTHR;
            v_on[i] = (VL * NTHR == VU) || u < VU;
            const int ch = u % KCH, g = v_on[i] ? u / KCH : 0;
            const int sblk = g >> 2, q = g & 3;
            const uint32_t unit = 2 * sblk + (q & 1);
            v_goff[i] = 4 * g * D + ch * 8;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t d = ch * 8 + e;
                v_loff[i][e] = d * (kKeyTile * 2) + ((unit ^ vt_swz(d)) * 16) + 8 * (q >> 1);
            }
        }
    }
    // page id of tile t (tiles past the block clamp to its last tile)
    __device__ __forceinline__ uint32_t page_of(uint32_t t) const {
        return kTilePage ? (uint32_t)table[(min(t, n_tiles - 1) * kKeyTile) >> lpt] : 0u;
    }
    __device__ __forceinline__ size_t tok_addr(uint32_t tok) const {
        tok = min(tok, n_keys - 1);  // keys past the block's last row are masked
        return (((head_base + (uint32_t)table[(tok >> lpt) - table_first]) << lpt) +
                (tok & pt_mask)) * D;
    }
    __device__ __forceinline__ size_t tile_base(uint32_t t, uint32_t pg) const {
        return (((head_base + pg) << lpt) + ((t * kKeyTile) & pt_mask)) * D;
    }
    template <int N>
    __device__ __forceinline__ void load_k(u32x4 (&r)[N], uint32_t t, uint32_t pg) const {
        static_assert(N >= KL, "staging registers");
        const uint16_t *kb = k_pages + tile_base(t, pg);
#pragma unroll
        for (int i = 0; i < KL; ++i) {
            if (!k_on[i]) continue;
            if constexpr (kTilePage) {
                r[i] = *(const u32x4 *)(kb + k_goff[i]);
            } else {
                r[i] = *(const u32x4 *)(k_pages + tok_addr(t * kKeyTile + k_goff[i] / D) +
                                        k_goff[i] % D);
            }
        }
    }
    template <int N>
    __device__ __forceinline__ void load_v(u32x4 (&r)[N], uint32_t t, uint32_t pg) const {
        static_assert(N >= 4 * VL, "staging registers");
        const uint16_t *vb = v_pages + tile_base(t, pg);
#pragma unroll
        for (int i = 0; i < VL; ++i) {
            if (!v_on[i]) continue;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (kTilePage) {
                    r[4 * i + j] = *(const u32x4 *)(vb + v_goff[i] + j * D);
                } else {
                    r[4 * i + j] = *(const u32x4 *)(
                        v_pages + tok_addr(t * kKeyTile + v_goff[i] / D + j) + v_goff[i] % D);
                }
            }
        }
    }
    template <int N>
    __device__ __forceinline__ void store_k(const u32x4 (&r)[N], unsigned char *kt) const {
#pragma unroll
        for (int i = 0; i < KL; ++i) {
            if (!k_on[i]) continue;
            u32x4 f;
#pragma unroll
            for (int j = 0; j < 4; ++j) f[j] = pack_f16x2(bf16lo(r[i][j]), bf16hi(r[i][j]));
            *(u32x4 *)(kt + k_loff[i]) = f;
        }
    }
    // valid_keys: keys of the tile that exist; the rest may hold any bits
    // (pages are reused), and although their P is 0, 0 * NaN is not, so in
    // the last tile they become 0.
    template <int N>
    __device__ __forceinline__ void store_v(const u32x4 (&r)[N], unsigned char *vt,
                                            uint32_t valid_keys) const {
#pragma unroll
        for (int i = 0; i < VL; ++i) {
            if (!v_on[i]) continue;
            u32x4 w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = r[4 * i + j];
            if (valid_keys < (uint32_t)kKeyTile) {
                const uint32_t key = v_goff[i] / D;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (key + j >= valid_keys) w[j] = u32x4{0, 0, 0, 0};
                }
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                // dim ch*8 + e of the 4 keys, as two fp16 pairs
                const uint32_t lo = pack_f16x2(bf16_elem(w[0], e), bf16_elem(w[1], e));
                const uint32_t hi = pack_f16x2(bf16_elem(w[2], e), bf16_elem(w[3], e));
                *(uint2 *)(vt + v_loff[i][e]) = make_uint2(lo, hi);
            }
        }
    }
};

// The same tile images as TileIo (K rows with k_swz, V^T with vt_swz), but
// every per-thread offset is recomputed from the thread's index gt at each
// use instead of being held in registers for the whole kernel (callers pass
// a freshly pinned copy of gt, so the compiler cannot hoist the offsets).
template <int D, int NTHR, bool kTilePage>
struct LeanIo {
    static constexpr int KCH = D / 8;                    // 16-byte chunks per row
    static constexpr int KSTEP = NTHR / KCH;             // keys per pass of the threads
    static constexpr int KL = kKeyTile / KSTEP;          // K chunks per thread
    static constexpr int VU = (kKeyTile / 4) * KCH;      // (4-key group, chunk) units
    static constexpr int VL = (VU + NTHR - 1) / NTHR;
    static_assert(NTHR % KCH == 0 && kKeyTile % KSTEP == 0, "thread layout");
    const uint16_t *k_pages;
    const uint16_t *v_pages;
    const int32_t *table;
    size_t head_base;
    uint32_t lpt, pt_mask, n_keys, n_tiles;

    __device__ __forceinline__ void init(const PrefillParams &p, const BlockPos &b) {
        k_pages = p.k_pages;
        v_pages = p.v_pages;
        table = p.page_table + (size_t)b.m.slot * p.pages_per_seq;
        head_base = (size_t)(b.kvh / p.kv_rep) * p.num_pages;  // the cache's head
        lpt = p.log2_page_tokens;
        pt_mask = (1u << lpt) - 1;
        n_keys = b.n_keys;
        n_tiles = b.n_tiles;
    }
    __device__ __forceinline__ uint32_t page_of(uint32_t t) const {
        return kTilePage ? (uint32_t)table[(min(t, n_tiles - 1) * kKeyTile) >> lpt] : 0u;
    }
    // element offset of tile t's first key in its page (kTilePage; pg = page_of(t))
    __device__ __forceinline__ size_t tile_base(uint32_t t, uint32_t pg) const {
        return kTilePage ? (((head_base + pg) << lpt) + ((t * kKeyTile) & pt_mask)) * D : 0;
    }
    __device__ __forceinline__ size_t row(uint32_t t, size_t base, uint32_t key) const {
        if constexpr (kTilePage) {
            return base + (size_t)key * D;
        } else {
            const uint32_t tok = min(t * kKeyTile + key, n_keys - 1);
            return (((head_base + (uint32_t)table[tok >> lpt]) << lpt) + (tok & pt_mask)) * D;
        }
    }
    // kTilePage: the thread's rows of a tile as byte offsets from the tile's
    // first key (the same for every tile, so computed once), and the tile's
    // first byte from a wave-uniform page id.  With the page id in a scalar
    // register the tile pointer is scalar too, and each row load is one
    // global load with a 32-bit vector offset: no 64-bit address arithmetic
    // in the vector unit per tile.
    __device__ __forceinline__ void tile_offsets(uint32_t gt, uint32_t (&off)[KL]) const {
        const uint32_t ch = gt % KCH, k0 = gt / KCH;
#pragma unroll
        for (int i = 0; i < KL; ++i) off[i] = ((k0 + i * KSTEP) * D + ch * 8) * 2;
    }
    __device__ __forceinline__ const unsigned char *tile_ptr(const uint16_t *src, uint32_t t,
                                                             uint32_t pg) const {
        return (const unsigned char *)(src + (((head_base + pg) << lpt) +
                                              ((t * kKeyTile) & pt_mask)) * D);
    }
    template <int N>
    __device__ __forceinline__ void load_rows(u32x4 (&r)[N], const unsigned char *tile,
                                              const uint32_t (&off)[KL]) const {
        static_assert(N >= KL, "staging registers");
#pragma unroll
        for (int i = 0; i < KL; ++i) {
            // the 32-bit offset is materialised here, so the address stays
            // (scalar pointer + zero-extended vector offset), the form of a
            // global load with a scalar base, instead of a hoisted 64-bit
            // vector value added per load
            uint32_t o = off[i];
            pin(o);
            r[i] = *(const u32x4 *)(tile + o);
        }
    }
    // LDS byte offsets of the thread's rows in the K image (is_v false) or
    // the row-major V image (is_v true); computed once
    __device__ __forceinline__ void lds_offsets(uint32_t gt, bool is_v, uint32_t (&off)[KL]) const {
        const uint32_t ch = gt % KCH, k0 = gt / KCH;
#pragma unroll
        for (int i = 0; i < KL; ++i) {
            const uint32_t key = k0 + i * KSTEP;
            off[i] = key * (D * 2) + ((ch ^ (is_v ? v_swz(k0) : k_swz<D>(key))) * 16);
        }
    }
    // store_k / store_v_rows with the offsets of lds_offsets; rows from
    // valid_keys on (V only, a partial last tile) become 0
    template <int N>
    __device__ __forceinline__ void store_rows(const u32x4 (&r)[N], unsigned char *buf,
                                               const uint32_t (&off)[KL], uint32_t k0,
                                               uint32_t valid_keys) const {
        const bool partial = valid_keys < (uint32_t)kKeyTile;  // uniform
#pragma unroll
        for (int i = 0; i < KL; ++i) {
            u32x4 f;
#pragma unroll
            for (int j = 0; j < 4; ++j) f[j] = pack_f16x2(bf16lo(r[i][j]), bf16hi(r[i][j]));
            if (partial && k0 + i * KSTEP >= valid_keys) f = u32x4{0, 0, 0, 0};
            *(u32x4 *)(buf + off[i]) = f;
        }
    }
    template <int N>
    __device__ __forceinline__ void load_k(u32x4 (&r)[N], uint32_t t, size_t base, uint32_t gt) const {
        static_assert(N >= KL, "staging registers");
        const uint32_t ch = gt % KCH, k0 = gt / KCH;
#pragma unroll
        for (int i = 0; i < KL; ++i) r[i] = *(const u32x4 *)(k_pages + row(t, base, k0 + i * KSTEP) + ch * 8);
    }
    template <int N>
    __device__ __forceinline__ void load_v(u32x4 (&r)[N], uint32_t t, size_t base, uint32_t gt) const {
        static_assert(N >= 4 * VL, "staging registers");
        const uint32_t ch = gt % KCH;
#pragma unroll
        for (int i = 0; i < VL; ++i) {
            const uint32_t u = min(gt + i * NTHR, (uint32_t)VU - 1);  // (threads past VU repeat a unit)
            const uint32_t g = u / KCH;
#pragma unroll
            for (int j = 0; j < 4; ++j) r[4 * i + j] = *(const u32x4 *)(v_pages + row(t, base, 4 * g + j) + ch * 8);
        }
    }
    // K (is_v false) or V (is_v true) rows of tile t in the K layout of
    // load_k, as one instruction stream: only the source differs, so there is
    // no branch whose two sides would load into the same registers (the
    // compiler then waits for every load in flight where the sides meet)
    template <int N>
    __device__ __forceinline__ void load_kv(u32x4 (&r)[N], uint32_t t, size_t base, uint32_t gt,
                                            bool is_v) const {
        static_assert(N >= KL, "staging registers");
        const uint32_t ch = gt % KCH, k0 = gt / KCH;
        const uint16_t *src = is_v ? v_pages : k_pages;
#pragma unroll
        for (int i = 0; i < KL; ++i) r[i] = *(const u32x4 *)(src + row(t, base, k0 + i * KSTEP) + ch * 8);
    }
    // V rows loaded by load_kv as the row-major fp16 image (v_swz).  Rows
    // from valid_keys on (past the last key: their probabilities are 0, but
    // the page may hold non-finite leftovers) become 0; only a partial tile
    // pays for that.
    template <int N>
    __device__ __forceinline__ void store_v_rows(const u32x4 (&r)[N], unsigned char *vt,
                                                 uint32_t valid_keys, uint32_t gt) const {
        const uint32_t ch = gt % KCH, k0 = gt / KCH;
        const bool partial = valid_keys < (uint32_t)kKeyTile;  // uniform
#pragma unroll
        for (int i = 0; i < KL; ++i) {
            const uint32_t key = k0 + i * KSTEP;  // key & 3 == k0 & 3
            u32x4 f;
#pragma unroll
            for (int j = 0; j < 4; ++j) f[j] = pack_f16x2(bf16lo(r[i][j]), bf16hi(r[i][j]));
            if (partial && key >= valid_keys) f = u32x4{0, 0, 0, 0};
            *(u32x4 *)(vt + key * (D * 2) + ((ch ^ v_swz(k0)) * 16)) = f;
        }
    }
    template <int N>
    __device__ __forceinline__ void store_k(const u32x4 (&r)[N], unsigned char *kt, uint32_t gt) const {
        const uint32_t ch = gt % KCH, k0 = gt / KCH;
#pragma unroll
        for (int i = 0; i < KL; ++i) {
            const uint32_t key = k0 + i * KSTEP;
            u32x4 f;
#pragma unroll
            for (int j = 0; j < 4; ++j) f[j] = pack_f16x2(bf16lo(r[i][j]), bf16hi(r[i][j]));
            *(u32x4 *)(kt + key * (D * 2) + ((ch ^ k_swz<D>(key)) * 16)) = f;
        }
    }
    // valid_keys: keys of the tile that exist; V rows past them become 0
    template <int N>
    __device__ __forceinline__ void store_v(const u32x4 (&r)[N], unsigned char *vt, uint32_t valid_keys,
                                            uint32_t gt) const {
        const uint32_t ch = gt % KCH;
#pragma unroll
        for (int i = 0; i < VL; ++i) {
            const uint32_t u = gt + i * NTHR;
            if ((VL * NTHR != VU) && u >= (uint32_t)VU) continue;
            const uint32_t g = u / KCH;
            u32x4 w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = (4 * g + j < valid_keys) ? r[4 * i + j] : u32x4{0, 0, 0, 0};
            const uint32_t unit = 2 * (g >> 2) + (g & 1);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t d = ch * 8 + e;
                const uint32_t lo = pack_f16x2(bf16_elem(w[0], e), bf16_elem(w[1], e));
                const uint32_t hi = pack_f16x2(bf16_elem(w[2], e), bf16_elem(w[3], e));
                *(uint2 *)(vt + d * (kKeyTile * 2) + ((unit ^ vt_swz(d)) * 16) + 8 * ((g & 3) >> 1)) =
                    make_uint2(lo, hi);
            }
        }
    }
};

// One wave's query rows: q RMSNorm (math.rs:28-50), RoPE with the row's
// cos/sin from the append kernel, scale by log2(e)/sqrt(D), fp16.  The lane
// holds row (row0 + col) and dims 16s + 8h + j (the B operand of S^T).
// Scalar inputs of q_operands, read from the kernel arguments once at kernel
// entry (q_args), so the prologue does not wait for one argument load after
// another.
struct QArgs {
    const void *q;
    const float *q_norm;
    const float2 *rope_cs;
    uint32_t *err_word;
    uint32_t flags;
    uint32_t rotary_dim;
    float eps;
};

__device__ __forceinline__ QArgs q_args(const PrefillParams &p) {
    QArgs a{p.q, p.q_norm, p.rope_cs, p.err_word, p.flags, p.rotary_dim, p.eps};
    a.q = pin_global(a.q);
    a.q_norm = pin_global(a.q_norm);
    a.rope_cs = pin_global(a.rope_cs);
    a.err_word = pin_global(a.err_word);
    pin_s(a.flags);
    pin_s(a.rotary_dim);
    pin_s(a.eps);
    return a;
}

// The row's RoPE (cos, sin) pairs read from global memory (rope_cs), or from
// a copy of the workgroup's rows in LDS (LdsRope).
struct GlobalRope {
    const float2 *row;
    __device__ __forceinline__ f32x4 pairs(uint32_t i) const { return *(const f32x4 *)(row + i); }
};
struct LdsRope {
    const __attribute__((address_space(3))) float2 *row;
    __device__ __forceinline__ f32x4 pairs(uint32_t i) const {
        return *(const __attribute__((address_space(3))) f32x4 *)(row + i);
    }
};

// q_operands at D = 256: a lane's 128 q values, its 128 norm weights and
// 128 RoPE values held at once would exceed the 256 registers of a wave that
// shares its SIMD.  Pass 1 streams q in for the sum of squares (the same
// partial sums in the same order as q_operands); pass 2 reads each 8-dim
// step again with its RoPE partner (dims i and i + rotary_dim/2 sit in the
// same lane, steps st and st + rotary_dim/32) and the pair's weights and
// (cos, sin), by address, so that no register array is indexed at run time.
// Every output is the same expression on the same values as in q_operands.
template <int D, class Rope>
__device__ __forceinline__ void q_operands_two_pass(const QArgs &p, size_t qbase, uint32_t call_row,
                                                    int h, f16x8 (&qop)[D / 16],
                                                    const Rope *rope) {
    constexpr int NS = D / 16;
    const bool bf16_in = (p.flags & SAFETYRAISE_MI355X_INPUT_BF16) != 0;
    const bool qk_norm = (p.flags & SAFETYRAISE_MI355X_QK_NORM) != 0;
    const float norm_add = (p.flags & SAFETYRAISE_MI355X_NORM_OFFSET) ? 1.0f : 0.0f;
    const uint32_t half = p.rotary_dim / 2;
    const uint32_t hsteps = p.rotary_dim / 32;
    Rope cs;
    if constexpr (std::is_same<Rope, GlobalRope>::value) cs.row = p.rope_cs + (size_t)call_row * half;
    else cs = *rope;
    auto load8 = [&](uint32_t st, float (&x)[8]) __attribute__((always_inline)) {
        if (bf16_in) {
            const u32x4 w = *(const u32x4 *)((const uint16_t *)p.q + qbase + 16 * st + 8 * h);
#pragma unroll
            for (int j = 0; j < 8; ++j) x[j] = bf16_elem(w, j);
        } else {
            const size_t off = qbase + 16 * st + 8 * h;
            const float4 a = *(const float4 *)((const float *)p.q + off);
            const float4 c = *(const float4 *)((const float *)p.q + off + 4);
            x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
            x[4] = c.x; x[5] = c.y; x[6] = c.z; x[7] = c.w;
        }
    };
    float inv = 1.0f;
    if (qk_norm) {
        float part[8];
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            float x[8];
            load8(st, x);
#pragma unroll
            for (int j = 0; j < 8; ++j) part[j] = st == 0 ? x[j] * x[j] : part[j] + x[j] * x[j];
        }
        float ss = ((part[0] + part[1]) + (part[2] + part[3])) + ((part[4] + part[5]) + (part[6] + part[7]));
        ss = xhalf_sum(ss);
        const float variance = ss / (float)D;
        if (!isfinite(variance) && (threadIdx.x & 63) == 0) {
            atomicOr(p.err_word, kErrNonFiniteVariance);
        }
        inv = 1.0f / sqrtf(variance + p.eps);
    }
    // x of step st, normalised as q_operands does it
    auto normed8 = [&](uint32_t st, float (&x)[8]) __attribute__((always_inline)) {
        load8(st, x);
        if (qk_norm) {
            const f32x4 w0 = *(const f32x4 *)(p.q_norm + 16 * st + 8 * h);
            const f32x4 w1 = *(const f32x4 *)(p.q_norm + 16 * st + 8 * h + 4);
#pragma unroll
            for (int j = 0; j < 8; ++j) x[j] = x[j] * inv * ((j < 4 ? w0[j] : w1[j - 4]) + norm_add);
        }
    };
    const float qscale = (1.0f / sqrtf((float)D)) * kLog2e;
#pragma unroll
    for (int st = 0; st < NS; ++st) {
        float x[8];
        normed8(st, x);
        const uint32_t ust = (uint32_t)st;
        if (ust < 2 * hsteps) {
            // rotated: left half (st < hsteps) or right half of a pair
            const bool left = ust < hsteps;
            const uint32_t pst = left ? ust + hsteps : ust - hsteps;  // the partner step
            const uint32_t lst = left ? ust : pst;                     // the pair's (cos, sin) step
            float y[8];
            normed8(pst, y);
#pragma unroll
            for (int j2 = 0; j2 < 4; ++j2) {
                const f32x4 cc = cs.pairs(16 * lst + 8 * h + 2 * j2);
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const int j = 2 * j2 + k;
                    const float c = k ? cc.z : cc.x;
                    const float sn = k ? cc.w : cc.y;
                    // left:  x[st] * cos - x[st + hsteps] * sin
                    // right: x[st] * cos + x[st - hsteps] * sin
                    x[j] = left ? x[j] * c - y[j] * sn : x[j] * c + y[j] * sn;
                }
            }
        }
        f32x8 v;
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = x[j] * qscale;
        qop[st] = __builtin_convertvector(v, f16x8);
    }
}

template <int D, class Rope = GlobalRope>
__device__ __forceinline__ void q_operands(const QArgs &p, size_t qbase, uint32_t call_row,
                                           int h, int lane, f16x8 (&qop)[D / 16],
                                           const Rope *rope = nullptr) {
    constexpr int NS = D / 16;
    if constexpr (D > 128) {
        q_operands_two_pass<D>(p, qbase, call_row, h, qop, rope);
        return;
    }
    const bool bf16_in = (p.flags & SAFETYRAISE_MI355X_INPUT_BF16) != 0;
    const bool qk_norm = (p.flags & SAFETYRAISE_MI355X_QK_NORM) != 0;
    const float norm_add = (p.flags & SAFETYRAISE_MI355X_NORM_OFFSET) ? 1.0f : 0.0f;
    // Every global input is requested before any is used, so that the
    // prologue waits for one round trip: the norm weights (q_norm is always
    // readable: the host passes a zero buffer when there is no QK-norm), the
    // row's RoPE (cos, sin) pairs (the host routes only rotary_dim >= 32, a
    // multiple of 32, here) and q itself.
    const uint32_t half = p.rotary_dim / 2;
    const uint32_t hsteps = p.rotary_dim / 32;
    Rope cs;
    if constexpr (std::is_same<Rope, GlobalRope>::value) cs.row = p.rope_cs + (size_t)call_row * half;
    else cs = *rope;
    f32x4 gw[NS][2];
#pragma unroll
    for (int st = 0; st < NS; ++st) {
        gw[st][0] = *(const f32x4 *)(p.q_norm + 16 * st + 8 * h);
        gw[st][1] = *(const f32x4 *)(p.q_norm + 16 * st + 8 * h + 4);
    }
    f32x4 csv[NS / 2][4];
#pragma unroll
    for (int st = 0; st < NS / 2; ++st) {
        const uint32_t c0 = 16 * min((uint32_t)st, hsteps - 1) + 8 * h;
#pragma unroll
        for (int j2 = 0; j2 < 4; ++j2) csv[st][j2] = cs.pairs(c0 + 2 * j2);  // pairs 2 j2, 2 j2 + 1
    }
    float x[NS][8];
    if (bf16_in) {
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            const u32x4 w = *(const u32x4 *)((const uint16_t *)p.q + qbase + 16 * st + 8 * h);
#pragma unroll
            for (int j = 0; j < 8; ++j) x[st][j] = bf16_elem(w, j);
        }
    } else {
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            const size_t off = qbase + 16 * st + 8 * h;
            const float4 a = *(const float4 *)((const float *)p.q + off);
            const float4 c = *(const float4 *)((const float *)p.q + off + 4);
            x[st][0] = a.x; x[st][1] = a.y; x[st][2] = a.z; x[st][3] = a.w;
            x[st][4] = c.x; x[st][5] = c.y; x[st][6] = c.z; x[st][7] = c.w;
        }
    }
    if (qk_norm) {
        // eight partial sums: a chain of 64 dependent FMAs would sit on the
        // prologue's critical path
        float part[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) part[j] = x[0][j] * x[0][j];
#pragma unroll
        for (int st = 1; st < NS; ++st)
#pragma unroll
            for (int j = 0; j < 8; ++j) part[j] += x[st][j] * x[st][j];
        float ss = ((part[0] + part[1]) + (part[2] + part[3])) + ((part[4] + part[5]) + (part[6] + part[7]));
        ss = xhalf_sum(ss);
        const float variance = ss / (float)D;
        if (!isfinite(variance) && lane == 0) {
            atomicOr(p.err_word, kErrNonFiniteVariance);
        }
        const float inv = 1.0f / sqrtf(variance + p.eps);
#pragma unroll
        for (int st = 0; st < NS; ++st) {
#pragma unroll
            for (int j = 0; j < 8; ++j) x[st][j] = x[st][j] * inv * (gw[st][j >> 2][j & 3] + norm_add);
        }
    }
    // pairs (i, i + rotary_dim/2): both halves of a pair sit in this lane
    // (the partner step st + hsteps is selected with compile-time indices so
    // that x stays in registers; full rotary, the common case, has its own
    // straight-line copy)
    if (hsteps == (uint32_t)(NS / 2)) {
#pragma unroll
        for (int st = 0; st < NS / 2; ++st) {
#pragma unroll
            for (int j2 = 0; j2 < 4; ++j2) {
                const f32x4 cc = csv[st][j2];
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const int j = 2 * j2 + k;
                    const float cs = k ? cc.z : cc.x;
                    const float sn = k ? cc.w : cc.y;
                    const float left = x[st][j], right = x[st + NS / 2][j];
                    x[st][j] = left * cs - right * sn;
                    x[st + NS / 2][j] = right * cs + left * sn;
                }
            }
        }
    } else {
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
            for (int j2 = 0; j2 < 4; ++j2) {
                const f32x4 cc = csv[st][j2];
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const int j = 2 * j2 + k;
                    const float cs = k ? cc.z : cc.x;
                    const float sn = k ? cc.w : cc.y;
                    const float left = x[st][j];
                    x[st][j] = left * cs - right[j] * sn;
                    right[j] = right[j] * cs + left * sn;
                }
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
#pragma unroll
    for (int st = 0; st < NS; ++st) {
        f32x8 v;
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = x[st][j] * qscale;
        qop[st] = __builtin_convertvector(v, f16x8);
    }
}

// S^T = K Q^T + c0 for the 64 keys of a tile (two 32-key accumulators that
// start from c0, operands read two k-steps ahead of their MFMA).
template <int D>
__device__ __forceinline__ void s_tile(const unsigned char *kt, const f16x8 (&qop)[D / 16], int h,
                                       int col, f32x16 (&sacc)[2], const f32x16 &c0) {
    constexpr int NS = D / 16;
    auto k_frag = [&](int u, int st) -> f16x8 {
        const int key = 32 * u + col;
        return *(const f16x8 *)(kt + key * (D * 2) + (((2 * st + h) ^ k_swz<D>(key)) * 16));
    };
    f16x8 ka[2][2] = {{k_frag(0, 0), k_frag(1, 0)}, {k_frag(0, 1), k_frag(1, 1)}};
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int st = 0; st < NS; ++st) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            sacc[u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[st & 1][u], qop[st],
                                                             st == 0 ? c0 : sacc[u], 0, 0, 0);
            if (st + 2 < NS) ka[st & 1][u] = k_frag(u, st + 2);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}
template <int D>
__device__ __forceinline__ void s_tile(const unsigned char *kt, const f16x8 (&qop)[D / 16], int h,
                                       int col, f32x16 (&sacc)[2]) {
    s_tile<D>(kt, qop, h, col, sacc, f32x16{});
}

// O^T += V^T P^T (operands read one k-step ahead of their MFMA).
template <int D>
__device__ __forceinline__ void pv_tile(const unsigned char *vt, const f16x8 (&pop)[4], int h,
                                        int col, f32x16 (&oacc)[D / 32]) {
    constexpr int NT = D / 32;
    auto v_frag = [&](int tt, int st) -> f16x8 {
        const uint32_t d = 32 * tt + col;
        return *(const f16x8 *)(vt + d * (kKeyTile * 2) + (((2 * st + h) ^ vt_swz(d)) * 16));
    };
    f16x8 va[2][NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) va[0][tt] = v_frag(tt, 0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int st = 0; st < 4; ++st) {
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) {
            if (st + 1 < 4) va[(st + 1) & 1][tt] = v_frag(tt, st + 1);
            oacc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[st & 1][tt], pop[st], oacc[tt], 0,
                                                              0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// The same product from a row-major V tile (v_swz): the A operand of lane
// (d = col, half h) for k-step st is V[keys 16 st + 4 h + {0..3, 8..11}][d],
// two transposing reads.  In each 16-lane group (g = lane / 16) lane s points
// at row 4 (s / 4) + ... and columns 4 (s % 4) .. + 3 of the group's 16
// columns; the read hands lane i of the group column i of those 4 rows.
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));

// Byte offset of lane's transposing reads in a V tile, per 32-column tile
// (k-step 0, first read; the other reads add 16 st and 8 rows): column tiles
// tile0 .. tile0 + NT - 1 of a row-major [64 keys][D] tile (D = 128: 16
// units of 16 bytes per row, 4 column tiles; D = 256: 32 units, 8 column
// tiles, read NT = 4 at a time by the two halves of the output dims).  The
// stored unit of logical unit c of key row r is c ^ ((r & 3) << 2) (v_swz),
// and the 4 rows a lane reads have r & 3 = s / 4, so the XOR stays inside the
// lane's column tile's four units.
template <int D, int NT = D / 32>
__device__ __forceinline__ void pv_rows_offsets(int lane, uint32_t (&off)[NT], uint32_t tile0 = 0) {
    static_assert(D == 128 || D == 256, "row-major V tiles of 128 or 256 dims");
    const uint32_t s = lane & 15, g = lane >> 4;
    const uint32_t row = 4 * (g >> 1) + (s >> 2);
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
        const uint32_t unit = (((tile0 + (uint32_t)tt) ^ (s >> 2)) << 2) | ((g & 1) << 1) |
                              ((s >> 1) & 1);
        off[tt] = row * (D * 2) + unit * 16 + (s & 1) * 8;
    }
}

template <int D, int NT = D / 32>
__device__ __forceinline__ void pv_tile_rows(const unsigned char *vt, const uint32_t (&off)[NT],
                                             const f16x8 (&pop)[4], f32x16 (&oacc)[NT]) {
    typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
    auto v_frag = [&](int tt, int st) __attribute__((always_inline)) -> f16x8 {
        const unsigned char *b = vt + off[tt] + st * 16 * (D * 2);
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(b));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(b + 8 * (D * 2)));
        return __builtin_bit_cast(f16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    };
    f16x8 va[2][NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) va[0][tt] = v_frag(tt, 0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int st = 0; st < 4; ++st) {
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) {
            if (st + 1 < 4) va[(st + 1) & 1][tt] = v_frag(tt, st + 1);
            oacc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[st & 1][tt], pop[st], oacc[tt], 0,
                                                              0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// max(a, b, c) as one v_max3_f32, without the quieting of signalling NaNs
// that fmaxf adds per operand (the scores come from MFMAs; a NaN score makes
// the row non-finite either way)
__device__ __forceinline__ float max3_raw(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// Online softmax of one tile (math.rs:133-148 in the log2 domain): causal
// mask, row max across the two lane halves, P = 2^(s - m) in fp16, row sum of
// those fp16 values, lazy rescale of O (only when some row's max moved).
template <int D>
__device__ __forceinline__ void softmax_tile(f32x16 (&sacc)[2], uint32_t key0, bool masked,
                                             uint32_t key_limit, int h, float &m_run, float &l_run,
                                             f32x16 (&oacc)[D / 32], f16x8 (&pop)[4]) {
    constexpr int NT = D / 32;
    if (masked) {
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t key = key0 + 32 * u + 8 * (i >> 2) + 4 * h + (i & 3);
                if (key > key_limit) sacc[u][i] = -INFINITY;
            }
    }
    // row max as a tree: 16 v_max3 at depth 4 instead of a chain of 16
    float m11[11];
#pragma unroll
    for (int j = 0; j < 10; ++j) {
        const int e = 3 * j;
        m11[j] = max3_raw(sacc[e >> 4][e & 15], sacc[(e + 1) >> 4][(e + 1) & 15],
                          sacc[(e + 2) >> 4][(e + 2) & 15]);
    }
    m11[10] = max3_raw(sacc[1][14], sacc[1][15], sacc[1][15]);
    const float m4a = max3_raw(m11[0], m11[1], m11[2]);
    const float m4b = max3_raw(m11[3], m11[4], m11[5]);
    const float m4c = max3_raw(m11[6], m11[7], m11[8]);
    const float m4d = max3_raw(m11[9], m11[10], m11[10]);
    float mx = max3_raw(max3_raw(m4a, m4b, m4c), m4d, m4d);
    mx = xhalf_max(mx);
    // the reference max is only raised when it grows by more than
    // kLazyRescale (log2 units): P stays <= 2^kLazyRescale (exact range for
    // fp16) and O is rescaled rarely; o / l is the same for any common shift
    const float m_new = (mx > m_run + kLazyRescale) ? mx : m_run;
    const float alpha = fast_exp2(m_run - m_new);
    m_run = m_new;
#pragma unroll
    for (int st = 0; st < 4; ++st) {
        f32x8 v;
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = fast_exp2(sacc[st >> 1][8 * (st & 1) + j] - m_new);
        pop[st] = __builtin_convertvector(v, f16x8);
    }
    // the row sum uses the fp16 probabilities the PV product uses
    const float lt =
        sum_f16x8(pop[0], sum_f16x8(pop[2], 0.0f)) + sum_f16x8(pop[1], sum_f16x8(pop[3], 0.0f));
    l_run = l_run * alpha + lt;
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
        for (int tt = 0; tt < NT; ++tt)
#pragma unroll
            for (int i = 0; i < 16; ++i) oacc[tt][i] *= alpha;
    }
}

// A lane's partial row sum of one tile's fp16 probabilities at or below this
// bound proves each of them finite (every p <= the sum < fp16's largest).
constexpr float kPSumMax = 32768.0f;

// Online softmax of one tile against a reference maximum m that moves rarely
// (math.rs:133-148 in the log2 domain).  The S MFMAs start from -m (negm),
// so sacc holds s - m and p = 2^(s - m) takes one exp per score; softmax is
// shift-invariant, so o = sum p v / sum p does not depend on m as long as
// every p is finite in fp16 and the largest is not far below 1.  m is the
// row maximum of the block's first tile (it holds key 0, which every row
// sees); it is raised, with l and O rescaled and the tile's p recomputed,
// only when a lane's partial sum exceeds kPSumMax: one wave-uniform branch,
// taken on the first tile and then only for a score ~15 (log2) above m.
// kMasked: the causal mask applies (the diagonal tiles only).
template <int D, bool kMasked>
__device__ __forceinline__ void softmax_tile_ref(f32x16 (&sacc)[2], uint32_t key0, uint32_t key_limit,
                                                 int h, bool first, float &m_run, f32x16 &negm,
                                                 float &l_run, f32x16 (&oacc)[D / 32],
                                                 f16x8 (&pop)[4]) {
    constexpr int NT = D / 32;
    if constexpr (kMasked) {
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t key = key0 + 32 * u + 8 * (i >> 2) + 4 * h + (i & 3);
                if (key > key_limit) sacc[u][i] = -INFINITY;
            }
    }
    // p = 2^(sacc - shift) in fp16, and the lane's sum of those fp16 values
    // (the row sum uses the probabilities the PV product uses); four
    // independent sums keep the dependency chains short
    auto probs = [&](float shift) __attribute__((always_inline)) {
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            f32x8 v;
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = fast_exp2(sacc[st >> 1][8 * (st & 1) + j] - shift);
            pop[st] = __builtin_convertvector(v, f16x8);
        }
        return (sum_f16x8(pop[0], 0.0f) + sum_f16x8(pop[1], 0.0f)) +
               (sum_f16x8(pop[2], 0.0f) + sum_f16x8(pop[3], 0.0f));
    };
    float lt = probs(0.0f);
    if (__builtin_amdgcn_ballot_w64(first || !(lt <= kPSumMax)) != 0) {
        // a side effect the compiler may not speculate: the branch stays a
        // branch instead of being if-converted into every tile's work
        asm volatile("; softmax reference maximum moves" ::: "memory");
        float m11[11];
#pragma unroll
        for (int j = 0; j < 10; ++j) {
            const int e = 3 * j;
            m11[j] = max3_raw(sacc[e >> 4][e & 15], sacc[(e + 1) >> 4][(e + 1) & 15],
                              sacc[(e + 2) >> 4][(e + 2) & 15]);
        }
        m11[10] = max3_raw(sacc[1][14], sacc[1][15], sacc[1][15]);
        const float m4a = max3_raw(m11[0], m11[1], m11[2]);
        const float m4b = max3_raw(m11[3], m11[4], m11[5]);
        const float m4c = max3_raw(m11[6], m11[7], m11[8]);
        const float m4d = max3_raw(m11[9], m11[10], m11[10]);
        const float mx = xhalf_max(max3_raw(max3_raw(m4a, m4b, m4c), m4d, m4d));
        // a row whose scores here are all masked has mx = -inf: no shift
        const float shift = first ? mx : fmaxf(mx, 0.0f);
        m_run += shift;
#pragma unroll
        for (int i = 0; i < 16; ++i) negm[i] = -m_run;
        // (l and O are still 0 on the first tile, whose shift may be any size)
        const float alpha = first ? 1.0f : fast_exp2(-shift);
        l_run *= alpha;
#pragma unroll
        for (int tt = 0; tt < NT; ++tt)
#pragma unroll
            for (int i = 0; i < 16; ++i) oacc[tt][i] *= alpha;
        lt = probs(shift);
    }
    l_run += lt;
}

// o / l, Qwen3.5 gate (math.rs sigmoid), f32 store; flags non-finite rows.
template <int D>
__device__ __forceinline__ void store_rows(const PrefillParams &p, uint32_t call_row, uint32_t head,
                                           size_t qbase, int h, float l_run,
                                           const f32x16 (&oacc)[D / 32]) {
    constexpr int NT = D / 32;
    const bool bf16_in = (p.flags & SAFETYRAISE_MI355X_INPUT_BF16) != 0;
    const bool gated = (p.flags & SAFETYRAISE_MI355X_GATED) != 0;
    const float inv_l = 1.0f / l_run;
    float *dst = p.out + (size_t)call_row * p.heads * D + (size_t)head * D;
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
            __builtin_nontemporal_store(f32x4{o[0], o[1], o[2], o[3]}, (f32x4 *)(dst + d0));
        }
    }
    if (!finite) atomicOr(p.err_word, kErrPrefillRange);
}

// store_rows for a wave's 32 rows through a 4 KB slice of LDS, 32 dims at a
// time: the lanes write their accumulator values (row col, dims 8a + 4h ..)
// to the slice and read them back row-major, so each store instruction
// writes whole 128-byte lines (8 rows x 32 dims) instead of 32 bytes of each
// of 32 rows.  Same values, gate and finite check as store_rows; rows from
// `valid` on are not stored.  Both write the output with nontemporal stores:
// the kernel never reads it back, and streaming it out took 2.2 us off a
// 512-row call at head_dim 128.
template <int D>
__device__ __forceinline__ void store_rows_lds(const PrefillParams &p, uint32_t call_row0,
                                               int valid, uint32_t head, int h, int col,
                                               int lane, float l_run,
                                               const f32x16 (&oacc)[D / 32],
                                               __attribute__((address_space(3))) f32x4 *slice) {
    constexpr int NT = D / 32;
    const bool bf16_in = (p.flags & SAFETYRAISE_MI355X_INPUT_BF16) != 0;
    const bool gated = (p.flags & SAFETYRAISE_MI355X_GATED) != 0;
    const uint32_t hs = gated ? 2 * D : D;
    const float inv_l = 1.0f / l_run;
    bool finite = true;
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            f32x4 o;
#pragma unroll
            for (int bb = 0; bb < 4; ++bb) {
                o[bb] = oacc[tt][4 * a + bb] * inv_l;
                finite = finite && (col >= valid || isfinite(o[bb]));
            }
            slice[col * 8 + ((2 * a + h) ^ (col & 7))] = o;
        }
        // LDS operations of one wave are performed in order; the fences keep
        // the compiler from moving the reads above the writes
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 8 * i + (lane >> 3), k = lane & 7;
            f32x4 o = slice[r * 8 + (k ^ (r & 7))];
            const uint32_t d0 = 32 * tt + 4 * k;
            if (r < valid) {
                const size_t row = (size_t)(call_row0 + r);
                if (gated) {
                    const size_t gbase = row * p.heads * hs + (size_t)head * hs + D + d0;
#pragma unroll
                    for (int bb = 0; bb < 4; ++bb) o[bb] *= ref_sigmoid(load_act(p.q, gbase + bb, bf16_in));
                }
                __builtin_nontemporal_store(o, (f32x4 *)(p.out + row * p.heads * D + (size_t)head * D + d0));
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    if (!finite) atomicOr(p.err_word, kErrPrefillRange);
}

// ---------------------------------------------------------------------------
// attn_prefill_kernel: all waves of a workgroup process every tile in step
// (one barrier per tile).  One workgroup = the G heads of a KV group x R
// blocks of 32 rows; two workgroups share a CU when the tiles fit twice in
// LDS (D <= 128), each wave then gets at most 256 registers.  Used where the
// ping-pong kernel below does not apply.
// kTilePage: page_tokens >= 64, so a 64-key tile lies in one page and its
// address is one wave-uniform page lookup plus per-thread constants.
// ---------------------------------------------------------------------------
template <int G>
constexpr int kLockstepRows = (G >= 4) ? 1 : (4 + G - 1) / G;

template <int D, int G, bool kTilePage>
__global__ __launch_bounds__(64 * G * kLockstepRows<G>)
__attribute__((amdgpu_waves_per_eu(D <= 128 ? 2 : 1))) void attn_prefill_kernel(
    const PrefillParams p) {
    constexpr int R = kLockstepRows<G>;
    constexpr int NTHR = 64 * G * R;
    constexpr int NS = D / 16;
    constexpr int NT = D / 32;
    using Io = TileIo<D, NTHR, kTilePage>;
    extern __shared__ __align__(16) unsigned char lds[];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int h = lane >> 5;
    const int col = lane & 31;
    const QArgs qa = q_args(p);
    const BlockPos b = block_pos(p, kRowTile * R);
    if (!b.active) return;
    const uint32_t head = b.kvh * G + (wave % G);
    const uint32_t wrow0 = b.row0 + kRowTile * (wave / G);
    const uint32_t my_row = min(wrow0 + col, b.m.rows - 1);
    const uint32_t key_limit = b.m.ctx + my_row;  // last visible key of this lane's row
    const uint32_t first_row_limit = b.m.ctx + b.row0;
    const uint32_t hs = (p.flags & SAFETYRAISE_MI355X_GATED) ? 2 * D : D;
    const size_t qbase = (size_t)(b.m.row0 + my_row) * p.heads * hs + (size_t)head * hs;

    Io io;
    io.init(tid, p, b);
    u32x4 kreg[Io::KL];
    u32x4 vreg[4 * Io::VL];
    uint32_t pg_next = io.page_of(1);
    {
        const uint32_t pg0 = io.page_of(0);
        io.load_k(kreg, 0, pg0);  // before the q prologue, so their latency overlaps it
        io.load_v(vreg, 0, pg0);
    }
    f16x8 qop[NS];
    q_operands<D>(qa, qbase, b.m.row0 + my_row, h, lane, qop);

    f32x16 oacc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) oacc[t] = f32x16{};
    float m_run = -INFINITY;
    float l_run = 0.0f;
    for (uint32_t t = 0; t < b.n_tiles; ++t) {
        unsigned char *kt = lds + (t & 1) * 2 * kTileBytes<D>;
        unsigned char *vt = kt + kTileBytes<D>;
        const uint32_t key0 = t * kKeyTile;
        io.store_k(kreg, kt);
        io.store_v(vreg, vt, b.n_keys - key0);
        __syncthreads();
        if (t + 1 < b.n_tiles) {
            const uint32_t pg = pg_next;
            pg_next = io.page_of(t + 2);  // read two tiles ahead
            io.load_k(kreg, t + 1, pg);
            io.load_v(vreg, t + 1, pg);
        }
        f32x16 sacc[2];
        s_tile<D>(kt, qop, h, col, sacc);
        f16x8 pop[4];
        softmax_tile<D>(sacc, key0, key0 + kKeyTile - 1 > first_row_limit, key_limit, h, m_run,
                        l_run, oacc, pop);
        pv_tile<D>(vt, pop, h, col, oacc);
    }
    const uint32_t row = wrow0 + col;
    const float l = xhalf_sum(l_run);
    if (row < b.m.rows) store_rows<D>(p, b.m.row0 + row, head, qbase, h, l, oacc);
}

// ---------------------------------------------------------------------------
// attn_prefill_pp_kernel: two groups of 4 waves, one wave of each on every
// SIMD, run half an iteration apart ("ping-pong").  The barriers of the
// workgroup split time into phases; in each phase one group issues MFMAs
// (PV of tile t-1 and S of tile t) while the other runs VALU work (softmax
// of its tile t and the staging of the next tile), so each SIMD's matrix
// unit is fed by one wave while its vector unit is busy with the other.
//
//   phase    2t        2t+1        2t+2
//   group 0  M(t)      V(t)        M(t+1)
//   group 1  V(t-1)    M(t)        V(t)
//
// Group 0 converts and stores K tiles, group 1 V tiles, both as row-major
// fp16 images (the PV product reads V with transposing loads); each group
// loads its next tile into registers one step ahead.  Step t stores tile t+1:
// K(t+1) in phase 2t+1, V(t+1) in phase 2t+2.  K(t) is read in phases 2t and
// 2t+1, V(t) in phases 2t+2 and 2t+3, so the tile a store replaces (two
// tiles back) is no longer read: two buffers of each, tile j in buffer j & 1,
// and the loop's two halves address them with constant offsets.
// Every wave passes the same number of barriers (group 1 one extra at the
// start, group 0 one extra at the end).
// One workgroup = 2 x 4 waves = (G heads x 4/G blocks of 32 rows) per group.
// ---------------------------------------------------------------------------
template <int D>
constexpr size_t kPingPongLds = 4 * kTileBytes<D>;  // K x 2, V x 2

// The workgroup's rows' RoPE (cos, sin) pairs, staged once in LDS behind the
// tiles for the q prologue: each row's table is read by the G waves of its
// heads, and read from global memory each lane's 32 pairs cost 16 loads that
// touch 32 rows each.  Rows are padded by 16 bytes so that the 32 rows of a
// read spread over the banks.  With G = 1 a workgroup has 256 rows, too many
// to stage: its waves read global memory.
template <int D, int G>
constexpr bool kStageRope = G >= 2;
template <int D>
constexpr uint32_t kRopePitch = D / 2 + 2;  // float2 per staged row
template <int D, int G>
constexpr size_t kRopeStageBytes = kStageRope<D, G> ? (size_t)2 * kRowTile * (4 / G) * kRopePitch<D> * 8 : 0;
// the epilogue's 4 KB per wave (store_rows_lds), in the same area: the
// RoPE rows are read only in the prologue
constexpr size_t kOutStageBytes = 8 * 4096;
template <int D, int G>
constexpr size_t kPpExtraLds = kRopeStageBytes<D, G> > kOutStageBytes ? kRopeStageBytes<D, G> : kOutStageBytes;

template <int D, int G, bool kTilePage>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void
attn_prefill_pp_kernel(const PrefillParams p) {
    constexpr int RG = 4 / G;  // row blocks per group
    constexpr int NS = D / 16;
    constexpr int NT = D / 32;
    using Io = LeanIo<D, 256, kTilePage>;
    constexpr int SL = Io::KL;
    extern __shared__ __align__(16) unsigned char lds[];
    unsigned char *kbuf = lds;                         // 2 K tiles
    unsigned char *vbuf = lds + 2 * kTileBytes<D>;     // 2 V tiles

    const int tid = threadIdx.x;
    const int wave = wave_index();
    const int lane = tid & 63;
    const int h = lane >> 5;
    const int col = lane & 31;
    const int grp = wave >> 2;  // waves w and w + 4 share a SIMD
    const int gw = wave & 3;
    const QArgs qa = q_args(p);
    const BlockPos b = block_pos(p, 2 * kRowTile * RG);
    if (!b.active) return;
    const uint32_t head = b.kvh * G + (gw % G);
    const uint32_t wrow0 = b.row0 + kRowTile * (grp * RG + gw / G);
    const uint32_t my_row = min(wrow0 + col, b.m.rows - 1);
    const uint32_t key_limit = b.m.ctx + my_row;
    const uint32_t first_row_limit = b.m.ctx + b.row0;
    const uint32_t hs = (p.flags & SAFETYRAISE_MI355X_GATED) ? 2 * D : D;
    const size_t qbase = (size_t)(b.m.row0 + my_row) * p.heads * hs + (size_t)head * hs;
    const uint32_t n = b.n_tiles;

    Io io;
    io.init(p, b);
    const uint32_t gt0 = tid & 255;
    // kTilePage: this thread's row offsets in a global tile and in its
    // group's LDS image (K for group 0, V for group 1), computed once; the
    // group's source pages and LDS image are wave-uniform
    uint32_t goff[SL] = {}, loff[SL] = {};
    const uint32_t k0 = gt0 / Io::KCH;
    if constexpr (kTilePage) {
        io.tile_offsets(gt0, goff);
        io.lds_offsets(gt0, grp != 0, loff);
    }
    const uint16_t *src_pages = grp != 0 ? p.v_pages : p.k_pages;
    unsigned char *img = grp != 0 ? vbuf : kbuf;
    // tile t's first byte from its page id, in scalar registers at this point
    auto tile_at = [&](uint32_t t, uint32_t pg) __attribute__((always_inline)) {
        uint64_t tp = (uint64_t)io.tile_ptr(src_pages, t, __builtin_amdgcn_readfirstlane(pg));
        pin_s(tp);
        return global_from_bits<const unsigned char>(tp);
    };
    // staging registers, two sets: tile j's data lives in stage[j & 1], so a
    // load never waits for the LDS stores that read the other set
    u32x4 stage0[SL] = {}, stage1[SL] = {};
    // tiles 0 and 1 (K by group 0, V by group 1) and tile 2's page id are
    // requested before the q prologue, so their latency overlaps it.  The
    // page id goes first: in the loop it is consumed with one tile's loads
    // issued after it, and a wait that must also cover this path can then
    // still leave those loads in flight.
    uint32_t pg_next = io.page_of(2);
    if constexpr (kTilePage) {
        const uint32_t pg0 = io.page_of(0), pg1 = io.page_of(1);
        io.load_rows(stage0, tile_at(0, pg0), goff);
        io.load_rows(stage1, tile_at(min(1u, n - 1), pg1), goff);
    } else {
        const uint32_t pg0 = io.page_of(0), pg1 = io.page_of(1);
        const size_t tb0 = io.tile_base(0, pg0), tb1 = io.tile_base(min(1u, n - 1), pg1);
        io.load_kv(stage0, 0, tb0, gt0, grp != 0);
        io.load_kv(stage1, min(1u, n - 1), tb1, gt0, grp != 0);
    }
    f16x8 qop[NS];
    if constexpr (kStageRope<D, G>) {
        // every load of the copy is issued before any store (indices clamped
        // into the table; rows past the call's repeat its last row)
        typedef __attribute__((address_space(3))) float2 lds_float2;
        lds_float2 *rs = (lds_float2 *)(lds + kPingPongLds<D>);
        constexpr uint32_t kRows = 2 * kRowTile * RG;
        constexpr uint32_t kChunks = kRows * (D / 4);  // 16-byte chunks at full rotary
        constexpr uint32_t kPer = kChunks / 512;
        static_assert(kChunks % 512 == 0, "chunks per thread");
        const uint32_t cpr = qa.rotary_dim / 4;  // chunks per row
        f32x4 cv[kPer];
#pragma unroll
        for (uint32_t u = 0; u < kPer; ++u) {
            const uint32_t c = min((uint32_t)tid + 512 * u, kRows * cpr - 1);
            const uint32_t rr = c / cpr, k = c - rr * cpr;
            const uint32_t call_row = b.m.row0 + min(b.row0 + rr, b.m.rows - 1);
            cv[u] = *(const f32x4 *)(qa.rope_cs + (size_t)call_row * (qa.rotary_dim / 2) + 2 * k);
        }
#pragma unroll
        for (uint32_t u = 0; u < kPer; ++u) {
            const uint32_t c = tid + 512 * u;
            if (c < kRows * cpr) {
                const uint32_t rr = c / cpr, k = c - rr * cpr;
                *(__attribute__((address_space(3))) f32x4 *)(rs + rr * kRopePitch<D> + 2 * k) = cv[u];
            }
        }
        __syncthreads();
        const LdsRope rope{rs + (my_row - b.row0) * kRopePitch<D>};
        q_operands<D>(qa, qbase, b.m.row0 + my_row, h, lane, qop, &rope);
    } else {
        q_operands<D>(qa, qbase, b.m.row0 + my_row, h, lane, qop);
    }
    if constexpr (kTilePage) {
        io.store_rows(stage0, img, loff, k0, grp != 0 ? b.n_keys : (uint32_t)kKeyTile);
    } else {
        if (grp == 0) io.store_k(stage0, kbuf, gt0);
        else io.store_v_rows(stage0, vbuf, b.n_keys, gt0);
    }
    uint32_t voff[NT];
    pv_rows_offsets<D>(lane, voff);
    f32x16 oacc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) oacc[t] = f32x16{};
    float m_run = 0.0f;  // the reference maximum, set by the first tile
    f32x16 negm = {};    // -m_run in every element: the S accumulators' start
    float l_run = 0.0f;
    f16x8 pop[4];
    __syncthreads();
    if (grp == 1) __syncthreads();  // group 1 starts one phase later

    // one iteration for tile t (t & 1 == PAR): `cur` holds tile t+1 (stored
    // now), `nxt` receives tile t+2.  Unmasked steps (MASKED false) need no
    // causal mask for tile t and store a whole tile t+1 (not the last).
    auto step = [&](uint32_t t, auto par, auto masked, u32x4 (&cur)[SL], u32x4 (&nxt)[SL])
                    __attribute__((always_inline)) {
        constexpr uint32_t PAR = decltype(par)::value;
        constexpr bool MASKED = decltype(masked)::value;
        // ---- M phase: PV(t-1), S(t) ----
        if (t > 0) pv_tile_rows<D>(vbuf + (PAR ^ 1) * kTileBytes<D>, voff, pop, oacc);
        f32x16 sacc[2];
        s_tile<D>(kbuf + PAR * kTileBytes<D>, qop, h, col, sacc, negm);
        __syncthreads();
        // ---- V phase: softmax(t), stage the group's tile t+1, load t+2 ----
        // The page id of tile t+2 (requested one phase earlier) is consumed
        // here, before this phase's LDS stores are issued, so that its wait
        // does not also wait for them.  Then tile t+3's is requested.
        const uint32_t t_next = min(t + 2, n - 1);
        const unsigned char *tile_next = nullptr;
        size_t tb_next = 0;
        if constexpr (kTilePage) {
            tile_next = tile_at(t_next, pg_next);
        } else {
            tb_next = io.tile_base(t_next, pg_next);
            pin(tb_next);
        }
        pg_next = io.page_of(t + 3);
        const uint32_t key0 = t * kKeyTile;
        softmax_tile_ref<D, MASKED>(sacc, key0, key_limit, h, t == 0, m_run, negm, l_run, oacc,
                                    pop);
        if constexpr (kTilePage) {
            if (t + 1 < n) {
                io.store_rows(cur, img + (PAR ^ 1) * kTileBytes<D>, loff, k0,
                              (MASKED && grp != 0) ? b.n_keys - key0 - kKeyTile
                                                   : (uint32_t)kKeyTile);
            }
            // issued on every path (past the end, the last tile again): a
            // load skipped on some path would make the next wait for an older
            // load (the page id) wait for every load in flight
            io.load_rows(nxt, tile_next, goff);
        } else {
            uint32_t gt = gt0;
            pin(gt);
            if (t + 1 < n) {
                if (grp == 0) io.store_k(cur, kbuf + (PAR ^ 1) * kTileBytes<D>, gt);
                else io.store_v_rows(cur, vbuf + (PAR ^ 1) * kTileBytes<D>,
                                     MASKED ? b.n_keys - key0 - kKeyTile : (uint32_t)kKeyTile, gt);
            }
            io.load_kv(nxt, t_next, tb_next, gt, grp != 0);
        }
        // the softmax results stay in this phase
#pragma unroll
        for (int st = 0; st < 4; ++st) pin(pop[st]);
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) pin(oacc[tt]);
        __syncthreads();
    };
    // both halves on every trip round the loop, the odd tile after it: a
    // path that skipped the second half and went round again would reach
    // the first half with that half's own loads still in flight
    uint32_t t = 0;
    using Even = std::integral_constant<uint32_t, 0>;
    using Odd = std::integral_constant<uint32_t, 1>;
    using Whole = std::false_type;
    using Masked = std::true_type;
    // tiles every row of the block sees whole and whose successor is not
    // the last (possibly partial) tile take the unmasked steps; the same
    // count for both groups, so their barriers still pair up
    const uint32_t t_main = min((first_row_limit + 1) / kKeyTile, n >= 2 ? n - 2 : 0u);
    for (; t + 1 < t_main; t += 2) {
        step(t, Even{}, Whole{}, stage1, stage0);
        step(t + 1, Odd{}, Whole{}, stage0, stage1);
    }
    for (; t + 1 < n; t += 2) {
        step(t, Even{}, Masked{}, stage1, stage0);
        step(t + 1, Odd{}, Masked{}, stage0, stage1);
    }
    if (t < n) step(t, Even{}, Masked{}, stage1, stage0);
    pv_tile_rows<D>(vbuf + ((n - 1) & 1) * kTileBytes<D>, voff, pop, oacc);
    if (grp == 0) __syncthreads();  // matches group 1's extra barrier

    const float l = xhalf_sum(l_run);
    const int valid = min((int)b.m.rows - (int)wrow0, kRowTile);
    store_rows_lds<D>(p, b.m.row0 + wrow0, valid, head, h, col, lane, l, oacc,
                      (__attribute__((address_space(3))) f32x4 *)(lds + kPingPongLds<D>) + wave * 256);
}

// softmax_tile_ref in parts, so that a caller can issue the common part
// between MFMAs of its own: softmax_mask1 (the causal mask of a diagonal
// tile), softmax_probs1 (p = 2^(s - shift) in fp16 and the lane's sum of
// those values) and softmax_fixup1 (the wave-uniform ballot and the rare
// branch that moves the reference maximum).
template <bool kMasked>
__device__ __forceinline__ void softmax_mask1(f32x16 (&sacc)[2], uint32_t key0,
                                              uint32_t key_limit, int h) {
    if constexpr (kMasked) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t key = key0 + 32 * kb + 8 * (i >> 2) + 4 * h + (i & 3);
                if (key > key_limit) sacc[kb][i] = -INFINITY;
            }
    }
}
// p = 2^(sacc - shift) in fp16 (k-step st's 8 values packed in pop[st]), and
// the lane's sum of those values
__device__ __forceinline__ float softmax_probs1(const f32x16 (&sacc)[2], float shift,
                                                u32x4 (&pop)[4]) {
#pragma unroll
    for (int st = 0; st < 4; ++st) {
        f32x8 v;
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = fast_exp2(sacc[st >> 1][8 * (st & 1) + j] - shift);
        pop[st] = __builtin_bit_cast(u32x4, __builtin_convertvector(v, f16x8));
    }
    return (sum_f16x8(__builtin_bit_cast(f16x8, pop[0]), 0.0f) +
            sum_f16x8(__builtin_bit_cast(f16x8, pop[1]), 0.0f)) +
           (sum_f16x8(__builtin_bit_cast(f16x8, pop[2]), 0.0f) +
            sum_f16x8(__builtin_bit_cast(f16x8, pop[3]), 0.0f));
}
// the rare branch of softmax_tile_ref: taken on the first tile and when a
// lane's partial sum exceeds kPSumMax
template <int D>
__device__ __forceinline__ void softmax_fixup1(const f32x16 (&sacc)[2], bool first, float lt,
                                               float &m_run, f32x16 &negm, float &l_run,
                                               f32x16 (&oacc)[D / 32], u32x4 (&pop)[4]) {
    constexpr int NT = D / 32;
    if (__builtin_amdgcn_ballot_w64(first || !(lt <= kPSumMax)) != 0) {
        asm volatile("; softmax reference maximum moves" ::: "memory");
        float m11[11];
#pragma unroll
        for (int j = 0; j < 10; ++j) {
            const int e = 3 * j;
            m11[j] = max3_raw(sacc[e >> 4][e & 15], sacc[(e + 1) >> 4][(e + 1) & 15],
                              sacc[(e + 2) >> 4][(e + 2) & 15]);
        }
        m11[10] = max3_raw(sacc[1][14], sacc[1][15], sacc[1][15]);
        const float m4a = max3_raw(m11[0], m11[1], m11[2]);
        const float m4b = max3_raw(m11[3], m11[4], m11[5]);
        const float m4c = max3_raw(m11[6], m11[7], m11[8]);
        const float m4d = max3_raw(m11[9], m11[10], m11[10]);
        const float mx = xhalf_max(max3_raw(max3_raw(m4a, m4b, m4c), m4d, m4d));
        // a row whose scores here are all masked has mx = -inf: no shift
        const float shift = first ? mx : fmaxf(mx, 0.0f);
        m_run += shift;
#pragma unroll
        for (int i = 0; i < 16; ++i) negm[i] = -m_run;
        // (l and O are still 0 on the first tile, whose shift may be any size)
        const float alpha = first ? 1.0f : fast_exp2(-shift);
        l_run *= alpha;
#pragma unroll
        for (int tt = 0; tt < NT; ++tt)
#pragma unroll
            for (int i = 0; i < 16; ++i) oacc[tt][i] *= alpha;
        lt = softmax_probs1(sacc, shift, pop);
    }
    l_run += lt;
}

// ---------------------------------------------------------------------------
// attn_prefill_pipe_kernel (D = 128, G = 2, 4 or 8, page_tokens >= 64): 8
// waves, two per SIMD, each one unit of (query head, 32 rows); G heads x
// 8/G row blocks per workgroup.  Every wave overlaps its own MFMAs with its
// own vector work, software-pipelined over the tiles, with one barrier per
// tile:
//
//   step t   S(t) = K(t) Q^T              convert + store a share of K(t+1)
//                                           and V(t); load its share of
//                                           K(t+2) and V(t+1)
//            O += V(t-1) P(t-1)           softmax(t) -> P(t)
//            barrier
//
// Each chunk between two sched_barriers is one MFMA and the vector work
// issued in its shadow: three VALU of the staging after each S MFMA, one
// pair of probabilities (two exps, a pack, a dot2 into the row sum) after
// each P V MFMA.  The two waves of a SIMD interleave at the hardware's
// choice.  All MFMAs keep their accumulators in VGPRs (at most 256
// registers per wave): an MFMA with AGPR accumulators holds its wave's
// issue about twice as long.
//
// K(t) lives in K buffer t & 1 and V(t) in V buffer t & 1: step t writes K
// buffer (t+1) & 1, last read by S(t-1), and V buffer t & 1, last read by
// the P V product of step t-1, both before the previous barrier.  P is
// double-buffered in registers; a rescale of O (the softmax's rare branch)
// comes after the step's P V product.
//
// LDS images, fp16, read with 16-byte loads only: K rows of 128 dims at a
// pitch of 272 bytes, V^T rows (one per dim, 64 keys in the column order of
// the S^T accumulator, as TileIo::store_v) at 144 bytes.  The pitches put the
// 16 lanes of a read, which hit 16 consecutive rows, on 16 distinct 4-bank
// groups, so every operand address is one base register plus an immediate.
// ---------------------------------------------------------------------------
constexpr uint32_t kPipeKPitch = 272;
constexpr uint32_t kPipeVPitch = 144;
constexpr uint32_t kPipeKTile = kKeyTile * kPipeKPitch;  // 17408
constexpr uint32_t kPipeVTile = 128 * kPipeVPitch;       // 18432
constexpr uint32_t kPipeV0 = 2 * kPipeKTile;
constexpr uint32_t kPipeX0 = kPipeV0 + 2 * kPipeVTile;   // RoPE rows, then output slices
template <int G>
constexpr int kPipeRowBlocks = 8 / G;
template <int G>
constexpr uint32_t kPipeRopeBytes = (uint32_t)kRowTile * kPipeRowBlocks<G> * kRopePitch<128> * 8;
template <int G>
constexpr uint32_t kPipeLds = kPipeX0 + (kPipeRopeBytes<G> > 8 * 4096 ? kPipeRopeBytes<G> : 8 * 4096);

typedef __attribute__((address_space(3))) f16x8 lds_f16x8;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) u32x2 lds_u32x2;

template <int G>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void
attn_prefill_pipe_kernel(const PrefillParams p) {
    constexpr int D = 128;
    constexpr int RB = kPipeRowBlocks<G>;
    constexpr int NT = D / 32;
    constexpr int NS = D / 16;
    static_assert(G == 2 || G == 4 || G == 8, "pipe kernel group sizes");
    static_assert(kPipeLds<G> <= 160 * 1024, "LDS");
    extern __shared__ __align__(16) unsigned char lds[];
    auto lds_at = [&](uint32_t off) __attribute__((always_inline)) {
        return (__attribute__((address_space(3))) unsigned char *)(lds) + off;
    };

    const int tid = threadIdx.x;
    const int wave = wave_index();
    const int lane = tid & 63;
    const int h = lane >> 5;
    const int col = lane & 31;
    const QArgs qa = q_args(p);
    const BlockPos b = block_pos(p, kRowTile * RB);
    if (!b.active) return;
    const uint32_t head = b.kvh * G + (wave % G);
    const uint32_t wrow0 = b.row0 + kRowTile * (wave / G);
    const uint32_t my_row = min(wrow0 + col, b.m.rows - 1);
    const uint32_t key_limit = b.m.ctx + my_row;
    const uint32_t first_row_limit = b.m.ctx + b.row0;
    const uint32_t hs = (p.flags & SAFETYRAISE_MI355X_GATED) ? 2 * D : D;
    const size_t qbase = (size_t)(b.m.row0 + my_row) * p.heads * hs + (size_t)head * hs;
    const uint32_t n = b.n_tiles;

    // tile t of the sequence: one page (page_tokens >= 64), wave-uniform
    const int32_t *table = p.page_table + (size_t)b.m.slot * p.pages_per_seq;
    const size_t head_base = (size_t)(b.kvh / p.kv_rep) * p.num_pages;
    const uint32_t lpt = p.log2_page_tokens;
    const uint32_t pt_mask = (1u << lpt) - 1;
    auto page_of = [&](uint32_t t) __attribute__((always_inline)) {
        return (uint32_t)table[(min(t, n - 1) * kKeyTile) >> lpt];
    };
    auto tile_ptr = [&](const uint16_t *src, uint32_t t, uint32_t pg) __attribute__((always_inline)) {
        const uint32_t tc = min(t, n - 1);
        uint64_t tp = (uint64_t)(src + (((head_base + __builtin_amdgcn_readfirstlane(pg)) << lpt) +
                                        ((tc * kKeyTile) & pt_mask)) * D);
        pin_s(tp);
        return global_from_bits<const unsigned char>(tp);
    };
    // Per-thread offsets, recomputed where used from a lane id read with
    // mbcnt in a volatile asm (not hoisted or merged), so that none of them is
    // live across the q prologue's register peak.
    //   staging (512 threads): K rows 2 r, 2 r + 1 (r = tid / 16), 16-byte
    //   chunk tid % 16 of each; V keys 4 g .. 4 g + 3 (g = tid % 16), dims
    //   4 c .. 4 c + 3 (c = tid / 16), as 8-byte pieces
    //   operand reads: K row col (+32 for the second key half), V^T row col
    //   (+32 per dim tile); k-step st adds 32 bytes
    struct Offs {
        uint32_t k_goff, v_goff, k_loff, v_loff, kr, vr;
    };
    auto offs = [&]() __attribute__((always_inline)) {
        uint32_t l;
        asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
        const uint32_t lo = l & 15, hi = (uint32_t)wave * 4 + (l >> 4);
        const uint32_t c = l & 31, hh = l >> 5;
        Offs o;
        o.k_goff = hi * 2 * (D * 2) + lo * 16;
        o.v_goff = lo * 4 * (D * 2) + hi * 8;
        o.k_loff = hi * 2 * kPipeKPitch + lo * 16;
        o.v_loff = hi * 4 * kPipeVPitch + 32 * (lo >> 2) + 16 * (lo & 1) + 8 * ((lo >> 1) & 1);
        o.kr = c * kPipeKPitch + hh * 16;
        o.vr = c * kPipeVPitch + hh * 16;
        return o;
    };
    const uint32_t vg = tid & 15;  // the thread's V key group (masking)
    auto load_k = [&](u32x4 (&r)[2], const unsigned char *tile, uint32_t goff)
                      __attribute__((always_inline)) {
        uint32_t o = goff;
        pin(o);
#pragma unroll
        for (int i = 0; i < 2; ++i) r[i] = *(const u32x4 *)(tile + o + i * (D * 2));
    };
    auto load_v = [&](u32x2 (&r)[4], const unsigned char *tile, uint32_t goff)
                      __attribute__((always_inline)) {
        uint32_t o = goff;
        pin(o);
#pragma unroll
        for (int j = 0; j < 4; ++j) r[j] = *(const u32x2 *)(tile + o + j * (D * 2));
    };

    u32x4 sk[2];  // K(t+1) at the start of step t
    u32x2 sv[4];  // V(t)
    f16x8 qop[NS];
    {
        u32x4 s0[2];
        const uint32_t pg0 = page_of(0), pg1 = page_of(1);
        const Offs o0 = offs();
        load_k(s0, tile_ptr(p.k_pages, 0, pg0), o0.k_goff);
        load_k(sk, tile_ptr(p.k_pages, 1, pg1), o0.k_goff);
        load_v(sv, tile_ptr(p.v_pages, 0, pg0), o0.v_goff);
        // RoPE (cos, sin) rows of the workgroup in LDS for the q prologue
        // (every load issued before any store)
        typedef __attribute__((address_space(3))) float2 lds_float2;
        lds_float2 *rs = (lds_float2 *)lds_at(kPipeX0);
        constexpr uint32_t kRows = kRowTile * RB;
        constexpr uint32_t kChunks = kRows * (D / 4);
        constexpr uint32_t kPer = kChunks / 512;
        static_assert(kChunks % 512 == 0, "chunks per thread");
        const uint32_t cpr = qa.rotary_dim / 4;
        f32x4 cv[kPer];
#pragma unroll
        for (uint32_t u = 0; u < kPer; ++u) {
            const uint32_t c = min((uint32_t)tid + 512 * u, kRows * cpr - 1);
            const uint32_t rr = c / cpr, k = c - rr * cpr;
            const uint32_t call_row = b.m.row0 + min(b.row0 + rr, b.m.rows - 1);
            cv[u] = *(const f32x4 *)(qa.rope_cs + (size_t)call_row * (qa.rotary_dim / 2) + 2 * k);
        }
#pragma unroll
        for (uint32_t u = 0; u < kPer; ++u) {
            const uint32_t c = tid + 512 * u;
            if (c < kRows * cpr) {
                const uint32_t rr = c / cpr, k = c - rr * cpr;
                *(__attribute__((address_space(3))) f32x4 *)(rs + rr * kRopePitch<D> + 2 * k) = cv[u];
            }
        }
        __syncthreads();
        const LdsRope rope{rs + (my_row - b.row0) * kRopePitch<D>};
        q_operands<D>(qa, qbase, b.m.row0 + my_row, h, lane, qop, &rope);
        const Offs o1 = offs();
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            u32x4 f;
#pragma unroll
            for (int j = 0; j < 4; ++j) f[j] = pack_f16x2(bf16lo(s0[i][j]), bf16hi(s0[i][j]));
            *(lds_u32x4 *)lds_at(o1.k_loff + i * kPipeKPitch) = f;
        }
        __syncthreads();
    }

    f32x16 oacc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) oacc[t] = f32x16{};
    float m_run = 0.0f, l_run = 0.0f;
    f32x16 negm = {};  // -m_run in every element: the S accumulators' start
    u32x4 popA[4], popB[4];
    uint32_t pg_k = page_of(2), pg_v = page_of(1);  // K(t+2) and V(t+1), loaded in step t
    const Offs o = offs();  // (after the prologue's register peak)

    auto step = [&](uint32_t t, auto par, auto masked, auto has_pv, u32x4 (&pprev)[4],
                    u32x4 (&pcur)[4]) __attribute__((always_inline)) {
        constexpr uint32_t PAR = decltype(par)::value;
        constexpr bool MASKED = decltype(masked)::value;
        constexpr bool HAS_PV = decltype(has_pv)::value;
        const uint32_t pgk = pg_k, pgv = pg_v;
        pg_v = pg_k;
        pg_k = page_of(t + 3);
        const uint32_t kbase = PAR * kPipeKTile + o.kr;
        const uint32_t kdst = (PAR ^ 1) * kPipeKTile + o.k_loff;
        const uint32_t vdst = kPipeV0 + PAR * kPipeVTile + o.v_loff;
        const uint32_t valid = MASKED ? min((uint32_t)kKeyTile, b.n_keys - t * kKeyTile)
                                      : (uint32_t)kKeyTile;
        // staging job j (three VALU): j < 8 converts K word j & 3 of row
        // j / 4 and stores the row's chunk after its last word; j >= 8
        // converts the low (keys 4 g, 4 g + 1) or high pair of V^T dim
        // 4 c + (j - 8) / 2 and stores the dim's piece after its high pair;
        // a register set is refilled right after its last conversion
        u32x4 kw;
        uint32_t vlo = 0;
        // Each job in two halves, so that no instruction waits on the one
        // before it: stage_unpack(j) widens the job's two bf16 values to f32
        // (and refills a register set once its last values are out),
        // stage_pack(j) (one MFMA later) rounds them to an fp16 pair and
        // stores the chunk or piece the pair completes.
        float uf[16][2];
        auto stage_unpack = [&](int j) __attribute__((always_inline)) {
            if (j < 8) {
                const int i = j >> 2, w = j & 3;
                uf[j][0] = bf16lo(sk[i][w]);
                uf[j][1] = bf16hi(sk[i][w]);
                if (j == 7) load_k(sk, tile_ptr(p.k_pages, t + 2, pgk), o.k_goff);
            } else {
                const int jj = j - 8, e = jj >> 1, hi = jj & 1;
                if (MASKED && jj == 0) {
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        if (4 * vg + q >= valid) sv[q] = u32x2{0, 0};
                }
                const uint32_t w0 = sv[2 * hi][e >> 1], w1 = sv[2 * hi + 1][e >> 1];
                uf[j][0] = (e & 1) ? bf16hi(w0) : bf16lo(w0);
                uf[j][1] = (e & 1) ? bf16hi(w1) : bf16lo(w1);
                if (j == 15) load_v(sv, tile_ptr(p.v_pages, t + 1, pgv), o.v_goff);
            }
        };
        auto stage_pack = [&](int j) __attribute__((always_inline)) {
            const uint32_t pr = pack_f16x2(uf[j][0], uf[j][1]);
            if (j < 8) {
                const int i = j >> 2, w = j & 3;
                kw[w] = pr;
                if (w == 3) *(lds_u32x4 *)lds_at(kdst + i * kPipeKPitch) = kw;
            } else {
                const int jj = j - 8, e = jj >> 1, hi = jj & 1;
                if (!hi) vlo = pr;
                else *(lds_u32x2 *)lds_at(vdst + e * kPipeVPitch) = u32x2{vlo, pr};
            }
        };
        f16x8 kf[NS][2];
        auto read_k = [&](int st) __attribute__((always_inline)) {
            kf[st][0] = *(const lds_f16x8 *)lds_at(kbase + st * 32);
            kf[st][1] = *(const lds_f16x8 *)lds_at(kbase + 32 * kPipeKPitch + st * 32);
        };
        f32x16 sacc[2];
        // V^T fragments of the P V product, read kVAhead MFMAs ahead of
        // their use; the first ones during the S product's last k-steps
        constexpr int kVAhead = 4;
        const uint32_t vbase = kPipeV0 + (PAR ^ 1) * kPipeVTile + o.vr;
        auto vfrag = [&](int i) __attribute__((always_inline)) {
            const int st = i >> 2, tt = i & 3;
            return *(const lds_f16x8 *)lds_at(vbase + tt * 32 * kPipeVPitch + st * 32);
        };
        f16x8 va[16];
        // K fragments read two k-steps (four MFMAs) ahead of their use
        read_k(0);
        read_k(1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            if (st + 2 < NS) read_k(st + 2);
            if (HAS_PV && st == NS - 2) {
#pragma unroll
                for (int i = 0; i < kVAhead; ++i) va[i] = vfrag(i);
            }
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[st][kb], qop[st],
                                                                  st ? sacc[kb] : negm, 0, 0, 0);
                stage_unpack(2 * st + kb);
                if (st + kb > 0) stage_pack(2 * st + kb - 1);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        stage_pack(15);
        softmax_mask1<MASKED>(sacc, t * kKeyTile, key_limit, h);
        // probability job j: the pair j & 3 of k-step j / 4
        // probability pair j (the pair j & 3 of k-step j / 4) in two halves,
        // so that no instruction waits on the one before it: exp_job(j) takes
        // the two exps, pack_job(j) (one MFMA later) packs them and adds the
        // pair to the row sum
        float ls[4] = {};
        float ex[16][2];
        auto exp_job = [&](int j) __attribute__((always_inline)) {
            const int st = j >> 2, pr = j & 3;
            const int e = 8 * (st & 1) + 2 * pr;
            ex[j][0] = fast_exp2(sacc[st >> 1][e]);
            ex[j][1] = fast_exp2(sacc[st >> 1][e + 1]);
        };
        auto pack_job = [&](int j) __attribute__((always_inline)) {
            const int st = j >> 2, pr = j & 3;
            const uint32_t w = pack_f16x2(ex[j][0], ex[j][1]);
            pcur[st][pr] = w;
            const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
            ls[st] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), one, ls[st], false);
        };
        if constexpr (HAS_PV) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int st = i >> 2, tt = i & 3;
                if (i + kVAhead < 16) va[i + kVAhead] = vfrag(i + kVAhead);
                oacc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                    va[i], __builtin_bit_cast(f16x8, pprev[st]), oacc[tt], 0, 0, 0);
                exp_job(i);
                if (i > 0) pack_job(i - 1);
                __builtin_amdgcn_sched_barrier(0);
            }
            pack_job(15);
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                exp_job(j);
                pack_job(j);
            }
        }
        const float lt = (ls[0] + ls[1]) + (ls[2] + ls[3]);
        softmax_fixup1<D>(sacc, t == 0, lt, m_run, negm, l_run, oacc, pcur);
        __syncthreads();
    };
    auto pv_last = [&](uint32_t vbuf, const u32x4 (&pop)[4]) __attribute__((always_inline)) {
        const uint32_t vbase = vbuf + o.vr;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
#pragma unroll
            for (int tt = 0; tt < NT; ++tt) {
                const f16x8 a = *(const lds_f16x8 *)lds_at(vbase + tt * 32 * kPipeVPitch + st * 32);
                oacc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                    a, __builtin_bit_cast(f16x8, pop[st]), oacc[tt], 0, 0, 0);
            }
        }
    };
    using Even = std::integral_constant<uint32_t, 0>;
    using Odd = std::integral_constant<uint32_t, 1>;
    using Whole = std::false_type;
    using Masked = std::true_type;
    using NoPv = std::false_type;
    using Pv = std::true_type;
    // steps t < t_main: every row sees all of tile t, and V(t) is whole
    const uint32_t t_main = min((first_row_limit + 1) / kKeyTile, n - 1);
    if (t_main > 0) step(0, Even{}, Whole{}, NoPv{}, popB, popA);
    else step(0, Even{}, Masked{}, NoPv{}, popB, popA);
    uint32_t t = 1;
    for (; t + 1 < t_main; t += 2) {
        step(t, Odd{}, Whole{}, Pv{}, popA, popB);
        step(t + 1, Even{}, Whole{}, Pv{}, popB, popA);
    }
    for (; t + 1 < n; t += 2) {
        step(t, Odd{}, Masked{}, Pv{}, popA, popB);
        step(t + 1, Even{}, Masked{}, Pv{}, popB, popA);
    }
    if (t < n) {
        step(t, Odd{}, Masked{}, Pv{}, popA, popB);
        pv_last(kPipeV0 + kPipeVTile, popB);
    } else {
        pv_last(kPipeV0, popA);
    }

    // the output slices share the RoPE rows' area, read only in the prologue
    const int valid = min((int)b.m.rows - (int)wrow0, kRowTile);
    store_rows_lds<D>(p, b.m.row0 + wrow0, valid, head, h, col, lane, xhalf_sum(l_run), oacc,
                      (__attribute__((address_space(3))) f32x4 *)lds_at(kPipeX0) + wave * 256);
}

template <int D, int G>
constexpr bool kUsePingPong = (D == 128) && (G == 1 || G == 2 || G == 4);

// the pipelined kernel takes D = 128 at G = 2, 4 or 8 with tiles inside one
// page; the ping-pong kernel the other D = 128 cases with G = 1, 2 or 4;
// the lock-step kernel the rest
template <int D, int G>
constexpr bool kHasPipe = (D == 128) && (G == 2 || G == 4 || G == 8);

template <int D, int G>
bool use_pipe(const PrefillParams &p) {
    if constexpr (kHasPipe<D, G>) return p.log2_page_tokens >= 6;
    return false;
}

template <int D, int G>
uint32_t rows_per_block_dg(bool pipe) {
    if constexpr (kHasPipe<D, G>) {
        if (pipe) return kRowTile * kPipeRowBlocks<G>;
    }
    return kUsePingPong<D, G> ? 2 * kRowTile * (4 / G) : kRowTile * kLockstepRows<G>;
}

template <int D, int G, bool kTilePage>
hipError_t launch_attn(hipStream_t stream, const PrefillParams &p, uint32_t blocks) {
    // the LDS limits are raised once per instantiation (thread-safe static
    // initialisers): the kernels take more than the default
    if constexpr (kUsePingPong<D, G>) {
        const size_t lds = kPingPongLds<D> + kPpExtraLds<D, G>;
        static const hipError_t configured =
            hipFuncSetAttribute((const void *)attn_prefill_pp_kernel<D, G, kTilePage>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (configured != hipSuccess) return configured;
        SR_LAUNCH("attn_prefill_pp_kernel", (attn_prefill_pp_kernel<D, G, kTilePage>), dim3(blocks),
                  dim3(512), lds, stream, p);
    } else {
        const size_t lds = 4 * kTileBytes<D>;  // K and V^T, double buffered
        static const hipError_t configured =
            hipFuncSetAttribute((const void *)attn_prefill_kernel<D, G, kTilePage>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (configured != hipSuccess) return configured;
        SR_LAUNCH("attn_prefill_kernel", (attn_prefill_kernel<D, G, kTilePage>), dim3(blocks),
                  dim3(64 * G * kLockstepRows<G>), lds, stream, p);
    }
    return hipGetLastError();
}

template <int G>
hipError_t launch_pipe(hipStream_t stream, const PrefillParams &p, uint32_t blocks) {
    static const hipError_t configured =
        hipFuncSetAttribute((const void *)attn_prefill_pipe_kernel<G>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)kPipeLds<G>);
    if (configured != hipSuccess) return configured;
    SR_LAUNCH("attn_prefill_pipe_kernel", (attn_prefill_pipe_kernel<G>), dim3(blocks), dim3(512),
              kPipeLds<G>, stream, p);
    return hipGetLastError();
}

template <int D, int G>
hipError_t launch_dg(hipStream_t stream, PrefillParams &p, const SeqMeta *seqs, int nseq) {
    const bool pipe = use_pipe<D, G>(p);
    const uint32_t rpb = rows_per_block_dg<D, G>(pipe);
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
    launch_append<D>(stream, p, max_rows);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const uint32_t blocks = p.max_blk * p.nseq * p.kv_heads;
    if constexpr (kHasPipe<D, G>) {
        if (pipe) return launch_pipe<G>(stream, p, blocks);
    }
    if (p.log2_page_tokens >= 6) return launch_attn<D, G, true>(stream, p, blocks);
    return launch_attn<D, G, false>(stream, p, blocks);
}

template <int D>
hipError_t launch_d(hipStream_t stream, PrefillParams &p, uint32_t g, const SeqMeta *seqs,
                    int nseq) {
    switch (g) {
        case 1: return launch_dg<D, 1>(stream, p, seqs, nseq);
        case 2: return launch_dg<D, 2>(stream, p, seqs, nseq);
        case 3: return launch_dg<D, 3>(stream, p, seqs, nseq);
        case 4: return launch_dg<D, 4>(stream, p, seqs, nseq);
        case 5: return launch_dg<D, 5>(stream, p, seqs, nseq);
        case 6: return launch_dg<D, 6>(stream, p, seqs, nseq);
        case 7: return launch_dg<D, 7>(stream, p, seqs, nseq);
        case 8: return launch_dg<D, 8>(stream, p, seqs, nseq);
        default: return hipErrorInvalidValue;
    }
}


// ---------------------------------------------------------------------------
// Multi-row verify (MTP drafts): split-K flash decoding with MFMA inner
// products.  A call appends R (2..15) rows per sequence; row r sees the
// context plus rows 0..r.  The R x G query vectors of a KV head (row r, head
// g: vector r*G + g) fill the N dimension of the MFMA tiles, 32 per wave, so
// each K/V tile of the cache is read once for all rows and heads.  The keys
// of a sequence are cut into partitions of part_keys (a multiple of 64); one
// workgroup per (partition, KV head) runs the online softmax over its keys
// and leaves a (max, sum, o[D]) record per query vector, which
// attn_verify_combine_kernel merges (math.rs:133-152 split over the keys).
// A workgroup holds at most 64 query vectors (two consumer waves of 32):
// with more (e.g. 1 + 8 drafts at G = 8), the rows are cut into slices of
// floor(64 / G) rows, one workgroup per (partition, KV head, slice); the
// slices of a partition are dispatched to one XCD at about the same time,
// so the second reads the partition's pages largely from its L2 and the
// Infinity Cache.  Each (row, head) record is written by one slice.
// ---------------------------------------------------------------------------
struct VerifyParams {
    PrefillParams p;       // meta[s].nblk = records per (row, head) of sequence s
    float *partials;       // records of kRecordStride floats
    uint32_t part_keys;
    uint32_t units;           // (partition, KV head) pairs of the launch
    uint32_t slices;          // row slices per unit (each <= 64 query vectors)
    uint32_t rows_per_slice;  // floor(64 / G)
    uint32_t blk0[kMetaPerLaunch];  // first partition of each sequence (prefix)
    uint32_t rec0[kMetaPerLaunch];  // first record of each sequence
};
static_assert(sizeof(VerifyParams) <= 4096, "kernel arguments stay within 4 KiB");


template <int D>
constexpr int kRecordStride = D + 4;  // m, l, 2 unused, o[D] (16-byte aligned)

// LDS entries for the page ids of one partition (the host caps part_keys so
// that a partition never spans more pages)
constexpr uint32_t kVerifyPageSlots = 2048;

// Tile staging of the verify producers (NL lanes per tile, lane gt: 128 at
// D <= 128, where a step stages two tiles, 256 at D = 256, one tile per
// step): fp16 K rows with k_swz; V as fp16 rows with v_swz (kRowV: D = 128
// and 256, read back with transposing LDS loads, so V shares K's page ids
// and row addresses and staging it costs no more than staging K) or as V^T
// with vt_swz (D = 64).  Every offset is recomputed from gt at each use, so
// that only the tiles in flight occupy registers.  Page ids come from the
// partition's LDS copy.  kShared: the partition's tiles are read by more
// than one workgroup (row slices, dispatched together on one XCD), so the
// loads are ordinary ones that leave the lines in L2 for the sibling slices;
// otherwise every tile is read once and the loads are nontemporal.
template <int D, bool kShared = false>
struct VerifyIo {
    static constexpr bool kRowV = D >= 128;
    static constexpr int NL = D <= 128 ? 128 : 256;         // lanes staging one tile
    static constexpr int KCH = D / 8;                       // 16-byte chunks per row
    static constexpr int KSTEP = NL / KCH;                  // keys per pass of the lanes
    static constexpr int KL = kKeyTile / KSTEP;             // K chunks per lane
    static constexpr int VL = kKeyTile / 4 / KSTEP;         // 4-key V units per lane
    const unsigned char *k_head;  // page 0 of this KV head in the K pool
    const unsigned char *v_head;
    const int32_t *pids;  // page ids from page `first` on (LDS)
    uint32_t page_bytes;  // page_tokens * D * 2
    uint32_t lpt, pt_mask, first, last_tok;

    // byte address of 16-byte chunk ch of token tok's row on page pg
    __device__ __forceinline__ const u32x4 *row_ptr(const unsigned char *head, uint32_t pg,
                                                   uint32_t tok, uint32_t ch) const {
        return (const u32x4 *)(head + ((uint64_t)pg * page_bytes +
                                       ((tok & pt_mask) * (uint32_t)(D * 2) + ch * 16)));
    }
    __device__ __forceinline__ void load(u32x4 (&kr)[KL], u32x4 (&vr)[4 * VL], uint32_t t,
                                         uint32_t gt) const {
        const uint32_t ch = gt % KCH, k0 = gt / KCH;
        const uint32_t key0 = t * kKeyTile;
        // keys past the sequence's last are masked: they read its last row.
        // A 4-key V group never straddles a page, and neither does its clamp.
        uint32_t tk[KL], tv[VL], pk[KL], pv[VL];
#pragma unroll
        for (int i = 0; i < KL; ++i) tk[i] = min(key0 + k0 + i * KSTEP, last_tok);
        if constexpr (!kRowV) {
#pragma unroll
            for (int i = 0; i < VL; ++i) tv[i] = min(key0 + 4 * (k0 + i * KSTEP), last_tok);
        }
        // every page id is requested before any is used: one LDS round trip
        // per tile instead of one per load (row-major V shares K's rows)
#pragma unroll
        for (int i = 0; i < KL; ++i) pk[i] = (uint32_t)pids[(tk[i] >> lpt) - first];
        if constexpr (!kRowV) {
#pragma unroll
            for (int i = 0; i < VL; ++i) pv[i] = (uint32_t)pids[(tv[i] >> lpt) - first];
        }
        __builtin_amdgcn_sched_barrier(0);
        // a tile read by one workgroup once: nontemporal loads (streaming
        // reads measured ~8 % faster than ordinary loads)
        auto ld = [](const u32x4 *a) __attribute__((always_inline)) {
            if constexpr (kShared) return *a;
            else return __builtin_nontemporal_load(a);
        };
#pragma unroll
        for (int i = 0; i < KL; ++i) kr[i] = ld(row_ptr(k_head, pk[i], tk[i], ch));
        if constexpr (kRowV) {
            static_assert(4 * VL == KL, "V rows in the K slots' registers");
#pragma unroll
            for (int i = 0; i < KL; ++i) vr[i] = ld(row_ptr(v_head, pk[i], tk[i], ch));
        } else {
#pragma unroll
            for (int i = 0; i < VL; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t tok = min(key0 + 4 * (k0 + i * KSTEP) + j, last_tok);
                    vr[4 * i + j] = ld(row_ptr(v_head, pv[i], tok, ch));
                }
        }
    }
    // Keys past the sequence's last were loaded as copies of its last row
    // (load clamps them), so their V rows are finite and need no zeroing: the
    // consumers mask their scores, and P = 0 times a finite value adds 0.
    __device__ __forceinline__ void store(const u32x4 (&kr)[KL], const u32x4 (&vr)[4 * VL],
                                          unsigned char *kt, unsigned char *vt,
                                          uint32_t gt) const {
        const uint32_t ch = gt % KCH, k0 = gt / KCH;
#pragma unroll
        for (int i = 0; i < KL; ++i) {
            const uint32_t key = k0 + i * KSTEP;
            u32x4 f;
#pragma unroll
            for (int j = 0; j < 4; ++j) f[j] = pack_f16x2(bf16lo(kr[i][j]), bf16hi(kr[i][j]));
            *(u32x4 *)(kt + key * (D * 2) + ((ch ^ k_swz<D>(key)) * 16)) = f;
        }
        if constexpr (kRowV) {
#pragma unroll
            for (int i = 0; i < KL; ++i) {
                const uint32_t key = k0 + i * KSTEP;  // key & 3 == k0 & 3
                u32x4 f;
#pragma unroll
                for (int j = 0; j < 4; ++j) f[j] = pack_f16x2(bf16lo(vr[i][j]), bf16hi(vr[i][j]));
                *(u32x4 *)(vt + key * (D * 2) + ((ch ^ v_swz(k0)) * 16)) = f;
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < VL; ++i) {
            const uint32_t g = k0 + i * KSTEP;
            const u32x4 *w = vr + 4 * i;
            const uint32_t unit = 2 * (g >> 2) + (g & 1);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t d = ch * 8 + e;
                const uint32_t lo = pack_f16x2(bf16_elem(w[0], e), bf16_elem(w[1], e));
                const uint32_t hi = pack_f16x2(bf16_elem(w[2], e), bf16_elem(w[3], e));
                *(uint2 *)(vt + d * (kKeyTile * 2) + ((unit ^ vt_swz(d)) * 16) +
                           8 * ((g & 3) >> 1)) = make_uint2(lo, hi);
            }
        }
    }
};

// One workgroup of 8 waves per (partition, KV head, row slice), one
// workgroup per CU.  Waves 4..7 stream the partition's K/V tiles:
// kVerifyDepth steps are in flight in their registers while they convert
// the oldest into one of two LDS buffer sets.  Waves 0..3 consume, one wave
// per SIMD:
//   D <= 128: two tiles per step (lanes 0..127 of the producers stage the
//     even tile, 128..255 the odd one); consumer pair 0 takes the even
//     tiles, pair 1 the odd ones, each wave of a pair 32 of the query
//     vectors.  Each pair leaves its own record, so a partition has two.
//   D = 256: one tile per step (all 256 producer lanes); consumer wave
//     (half, group) takes 32 query vectors and half of the output dims: the
//     two waves of a vector group compute the same scores and softmax (the
//     same operations on the same tile), each its 128 dims of P V.  One
//     record per partition.
// One barrier per step: after barrier k, the tiles of step k are in LDS and
// the buffers of step k-1 are free.
// steps in flight in the producers' registers: 3 at D <= 128 (measured 2-3 %
// faster than 2, 4 slower); 2 at D = 256, whose steps hold twice the bytes
template <int D>
constexpr int kVerifyDepth = D <= 128 ? 3 : 2;
constexpr int kVerifyThreads = 512;
template <int D>
constexpr uint32_t kVerifyTilesPerStep = D <= 128 ? 2 : 1;
template <int D>
constexpr size_t kVerifyTileLds = 2 * kVerifyTilesPerStep<D> * 2 * kTileBytes<D>;

// kAllTiles (D <= 128 only): each of the four consumer waves takes 32 query
// vectors and both tiles of every step (up to 128 vectors per workgroup, one
// record per partition), for calls with more than 64 vectors per KV head.
template <int D, bool kAllTiles, bool kShared>
__global__ __launch_bounds__(kVerifyThreads) __attribute__((amdgpu_waves_per_eu(2))) void
attn_verify_kernel(const VerifyParams vp) {
    static_assert(!kAllTiles || D <= 128, "D = 256 splits the output dims instead");
    constexpr int NS = D / 16;
    constexpr uint32_t TPS = kVerifyTilesPerStep<D>;
    // records per partition (one per consumer that saw part of its tiles)
    constexpr uint32_t kRecPerPart = kAllTiles ? 1 : TPS;
    constexpr int NTW = D <= 128 ? D / 32 : 4;  // output tiles of a consumer wave
    extern __shared__ __align__(16) unsigned char lds[];
    const PrefillParams &p = vp.p;

    const int tid = threadIdx.x;
    const int wave = wave_index();
    const int lane = tid & 63;
    // block -> (unit, slice): the slices of a unit are 8 blocks apart, so
    // they land on the same XCD (block i runs on XCD i % 8) at about the
    // same time; blocks past the last unit leave at once (whole workgroup)
    const uint32_t grp8 = blockIdx.x / (8 * vp.slices);
    const uint32_t slice = (blockIdx.x / 8) % vp.slices;
    const uint32_t unit = grp8 * 8 + blockIdx.x % 8;
    if (unit >= vp.units) return;
    const uint32_t kvh = unit % p.kv_heads;
    const uint32_t j = unit / p.kv_heads;
    uint32_t s = 0;
    while (s + 1 < p.nseq && vp.blk0[s + 1] <= j) ++s;
    const PrefillMeta m = p.meta[s];
    const uint32_t row_begin = slice * vp.rows_per_slice;
    if (row_begin >= m.rows) return;  // this sequence has fewer slices (whole workgroup)
    const QArgs qa = q_args(p);
    const uint32_t part = j - vp.blk0[s];
    const uint32_t total = m.ctx + m.rows;
    const uint32_t key_begin = part * vp.part_keys;
    const uint32_t key_end = min(key_begin + vp.part_keys, total);
    const uint32_t t0 = key_begin / kKeyTile;
    const uint32_t t1 = (key_end + kKeyTile - 1) / kKeyTile;
    // both roles run the same padded number of steps (one barrier each)
    const uint32_t steps = (t1 - t0 + TPS - 1) / TPS;
    const uint32_t k_pad = (steps + kVerifyDepth<D> - 1) / kVerifyDepth<D> * kVerifyDepth<D>;
    // buffer (step parity b, tile q of the step): K tile, then V tile
    auto tile_lds = [&](uint32_t k, uint32_t q) {
        return lds + ((k & 1) * TPS + q) * 2 * kTileBytes<D>;
    };

    if (wave >= 4) {
        // ---- producers ----
        const uint32_t pt = tid - 256;                 // 0..255
        const uint32_t q = TPS == 2 ? pt >> 7 : 0u;    // which tile of the step
        const uint32_t gt0 = TPS == 2 ? pt & 127 : pt;
        VerifyIo<D, kShared> io;
        io.lpt = p.log2_page_tokens;
        io.pt_mask = (1u << io.lpt) - 1;
        io.page_bytes = (D * 2) << io.lpt;
        const size_t head_bytes = (size_t)(kvh / p.kv_rep) * p.num_pages * io.page_bytes;
        io.k_head = (const unsigned char *)p.k_pages + head_bytes;
        io.v_head = (const unsigned char *)p.v_pages + head_bytes;
        io.last_tok = total - 1;
        // the page ids of the partition's keys go to LDS once, so that no
        // tile load waits on a page-table read
        int32_t *pids = (int32_t *)(lds + kVerifyTileLds<D>);
        const int32_t *table = p.page_table + (size_t)m.slot * p.pages_per_seq;
        io.first = key_begin >> io.lpt;
        const uint32_t n = ((key_end - 1) >> io.lpt) - io.first + 1;
        // all of a lane's table reads are in flight before the first LDS
        // store (past n, the last entry again: in bounds, never stored)
        int32_t pw[kVerifyPageSlots / 256];
#pragma unroll
        for (uint32_t u = 0; u < kVerifyPageSlots / 256; ++u) {
            pw[u] = table[io.first + min(pt + 256 * u, n - 1)];
        }
#pragma unroll
        for (uint32_t u = 0; u < kVerifyPageSlots / 256; ++u) {
            if (pt + 256 * u < n) pids[pt + 256 * u] = pw[u];
        }
        io.pids = pids;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_s_barrier();  // (A) the producers share pids
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        u32x4 kreg[kVerifyDepth<D>][VerifyIo<D>::KL];
        u32x4 vreg[kVerifyDepth<D>][4 * VerifyIo<D>::VL];
#pragma unroll
        for (int u = 0; u < kVerifyDepth<D>; ++u) {
            io.load(kreg[u], vreg[u], min(t0 + TPS * u + q, t1 - 1), gt0);
            __builtin_amdgcn_sched_barrier(0);
        }
        for (uint32_t kb = 0; kb < k_pad; kb += kVerifyDepth<D>) {
#pragma unroll
            for (int u = 0; u < kVerifyDepth<D>; ++u) {
                // offsets are recomputed from a fresh copy of the lane id
                // each step instead of being held live across the loop
                uint32_t gt = gt0;
                pin(gt);
                const uint32_t k = kb + u;
                unsigned char *kt = tile_lds(k, q);
                // tiles past t1 store a repeat of the last tile nobody reads
                io.store(kreg[u], vreg[u], kt, kt + kTileBytes<D>, gt);
                __syncthreads();  // (B) the tiles of step k are in LDS
                io.load(kreg[u], vreg[u], min(t0 + TPS * (k + kVerifyDepth<D>) + q, t1 - 1), gt);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        return;
    }

    // ---- consumers ----
    // tile of the step (pair mode), output dims (D = 256), 32-vector group
    const uint32_t pair = (TPS == 2 && !kAllTiles) ? (uint32_t)wave >> 1 : 0u;
    const uint32_t half = TPS == 2 ? 0u : (uint32_t)wave >> 1;
    const int cw = kAllTiles ? wave : (wave & 1);
    const int h = lane >> 5;
    const int col = lane & 31;
    const uint32_t G = p.heads / p.kv_heads;
    const uint32_t nvec = min(vp.rows_per_slice, m.rows - row_begin) * G;
    const bool computes = 32u * cw < nvec;               // wave-uniform
    const uint32_t vec = min(32u * cw + col, nvec - 1);  // this lane's query vector
    const uint32_t r = row_begin + vec / G;
    const uint32_t head = kvh * G + vec % G;
    const uint32_t key_limit = m.ctx + r;
    const uint32_t hs = (p.flags & SAFETYRAISE_MI355X_GATED) ? 2 * D : D;
    const size_t qbase = (size_t)(m.row0 + r) * p.heads * hs + (size_t)head * hs;
    f16x8 qop[NS];
    if (computes) q_operands<D>(qa, qbase, m.row0 + r, h, lane, qop);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_barrier();  // (A)
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");

    f32x16 oacc[NTW];
#pragma unroll
    for (int t = 0; t < NTW; ++t) oacc[t] = f32x16{};
    uint32_t voff[NTW];
    if constexpr (VerifyIo<D>::kRowV) pv_rows_offsets<D, NTW>(lane, voff, NTW * half);
    float m_run = -INFINITY;
    float l_run = 0.0f;
    // one tile of step k: scores, softmax, P V
    auto consume = [&](uint32_t k, uint32_t tq, uint32_t t) __attribute__((always_inline)) {
        const unsigned char *kt = tile_lds(k, tq);
        const unsigned char *vt = kt + kTileBytes<D>;
        const uint32_t key0 = t * kKeyTile;
        f32x16 sacc[2];
        s_tile<D>(kt, qop, h, col, sacc);
        // keys past the partition end (the last tile of the sequence) and
        // past a row's own position are masked
        const bool edge = key0 + kKeyTile > min(key_end, m.ctx + 1);
        if (edge) {
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const uint32_t key = key0 + 32 * u + 8 * (i >> 2) + 4 * h + (i & 3);
                    if (key >= key_end) sacc[u][i] = -INFINITY;
                }
        }
        f16x8 pop[4];
        // (the softmax's D only sizes the O tiles it rescales: NTW of them)
        softmax_tile<32 * NTW>(sacc, key0, edge, key_limit, h, m_run, l_run, oacc, pop);
        if constexpr (VerifyIo<D>::kRowV) pv_tile_rows<D, NTW>(vt, voff, pop, oacc);
        else pv_tile<D>(vt, pop, h, col, oacc);
    };
    for (uint32_t k = 0; k < k_pad; ++k) {
        __syncthreads();  // (B)
        if constexpr (kAllTiles) {
            const uint32_t t = t0 + TPS * k;
            if (!computes || t >= t1) continue;
            consume(k, 0, t);
            if (t + 1 >= t1) continue;
            consume(k, 1, t + 1);
        } else {
            const uint32_t t = t0 + TPS * k + pair;
            if (!computes || t >= t1) continue;
            consume(k, pair, t);
        }
    }
    const float l = xhalf_sum(l_run);
    if (32u * cw + col >= nvec) return;
    // record (sequence s, row r, head, partition, pair): o unnormalised
    const uint32_t nrec = m.nblk;  // records per (row, head): kRecPerPart per partition
    float *rec = vp.partials + ((size_t)vp.rec0[s] + ((size_t)r * p.heads + head) * nrec +
                                kRecPerPart * part + pair) *
                                   kRecordStride<D>;
    if (h == 0 && half == 0) {
        // a pair that saw no key of this row's range has l = 0
        *(float2 *)rec = make_float2(l > 0.0f ? m_run : -INFINITY, l);
    }
#pragma unroll
    for (int tt = 0; tt < NTW; ++tt)
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            const uint32_t d0 = 128 * half + 32 * tt + 8 * a + 4 * h;
            *(float4 *)(rec + 4 + d0) = make_float4(oacc[tt][4 * a], oacc[tt][4 * a + 1],
                                                    oacc[tt][4 * a + 2], oacc[tt][4 * a + 3]);
        }
}

// One workgroup of four waves per (sequence, row, head): merges the
// partition records in the log2 domain, divides by the sum, applies the
// Qwen3.5 gate and stores.  Wave w takes records w, w + 4, ...; every record
// load of a batch is in flight at once, and the four partial sums meet in LDS.
constexpr int kCombineWaves = 4;

template <int D>
__global__ __launch_bounds__(64 * kCombineWaves) void attn_verify_combine_kernel(const VerifyParams vp) {
    constexpr int EPL = D / 64;
    constexpr int kUnroll = 8;  // records per batch of loads
    __shared__ float part_s[kCombineWaves][D + 1];
    __shared__ float max_s[kCombineWaves];
    const PrefillParams &p = vp.p;
    const uint32_t w = blockIdx.x;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    uint32_t s = 0, base = 0;
    for (; s < p.nseq; ++s) {
        const uint32_t n = p.meta[s].rows * p.heads;
        if (w < base + n) break;
        base += n;
    }
    if (s >= p.nseq) return;  // whole workgroup: no barrier is skipped by part of it
    const PrefillMeta m = p.meta[s];
    const uint32_t r = (w - base) / p.heads;
    const uint32_t head = (w - base) % p.heads;
    const uint32_t nparts = m.nblk;
    const float *rec = vp.partials +
                       ((size_t)vp.rec0[s] + ((size_t)r * p.heads + head) * nparts) * kRecordStride<D>;
    // maximum over the partition maxima, all threads of the workgroup
    float mx = -INFINITY;
    for (uint32_t q = threadIdx.x; q < nparts; q += 64 * kCombineWaves) {
        mx = fmaxf(mx, rec[(size_t)q * kRecordStride<D>]);
    }
    mx = max64(mx);
    if (lane == 0) max_s[wave] = mx;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kCombineWaves; ++i) mx = fmaxf(mx, max_s[i]);
    // this wave's records: weight 2^(m - max) (0 for a record with no
    // visible key, m = -inf, whose o is never used), sum and output
    float l = 0.0f;
    float o[EPL] = {};
    for (uint32_t q0 = wave; q0 < nparts; q0 += kCombineWaves * kUnroll) {
        float2 ml[kUnroll];
        float x[kUnroll][EPL];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            // past the last record: the last one again, with weight 0
            const uint32_t q = min(q0 + (uint32_t)(kCombineWaves * u), nparts - 1);
            const float *rq = rec + (size_t)q * kRecordStride<D>;
            ml[u] = *(const float2 *)rq;
#pragma unroll
            for (int i = 0; i < EPL; ++i) x[u][i] = rq[4 + lane + 64 * i];
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const bool live = q0 + (uint32_t)(kCombineWaves * u) < nparts && ml[u].x != -INFINITY;
            const float sc = live ? fast_exp2(ml[u].x - mx) : 0.0f;
            l += live ? ml[u].y * sc : 0.0f;
#pragma unroll
            for (int i = 0; i < EPL; ++i) o[i] += live ? x[u][i] * sc : 0.0f;
        }
    }
#pragma unroll
    for (int i = 0; i < EPL; ++i) part_s[wave][lane + 64 * i] = o[i];
    if (lane == 0) part_s[wave][D] = l;
    __syncthreads();
    if (wave != 0) return;
    l = 0.0f;
#pragma unroll
    for (int k = 0; k < kCombineWaves; ++k) l += part_s[k][D];
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        o[i] = 0.0f;
#pragma unroll
        for (int k = 0; k < kCombineWaves; ++k) o[i] += part_s[k][lane + 64 * i];
    }
    const bool bf16_in = (p.flags & SAFETYRAISE_MI355X_INPUT_BF16) != 0;
    const bool gated = (p.flags & SAFETYRAISE_MI355X_GATED) != 0;
    const uint32_t hs = gated ? 2 * D : D;
    const size_t qbase = (size_t)(m.row0 + r) * p.heads * hs + (size_t)head * hs;
    float *dst = p.out + (size_t)(m.row0 + r) * p.heads * D + (size_t)head * D;
    const float inv = 1.0f / l;
    bool finite = true;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        float y = o[i] * inv;
        finite = finite && isfinite(y);
        if (gated) y *= ref_sigmoid(load_act(p.q, qbase + D + lane + 64 * i, bf16_in));
        dst[lane + 64 * i] = y;
    }
    if (!finite) atomicOr(p.err_word, kErrPrefillRange);
}

template <int D, bool kAllTiles, bool kShared = false>
hipError_t launch_verify_d(hipStream_t stream, const VerifyParams &vp, uint32_t blocks,
                           uint32_t combine_rows) {
    const size_t lds = kVerifyTileLds<D> + kVerifyPageSlots * sizeof(int32_t);
    static_assert(kVerifyTileLds<D> + kVerifyPageSlots * sizeof(int32_t) <= 160 * 1024,
                  "verify LDS");
    static const hipError_t configured =
        hipFuncSetAttribute((const void *)attn_verify_kernel<D, kAllTiles, kShared>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (configured != hipSuccess) return configured;
    SR_LAUNCH("attn_verify_kernel", (attn_verify_kernel<D, kAllTiles, kShared>), dim3(blocks),
              dim3(kVerifyThreads), lds, stream, vp);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    SR_LAUNCH("attn_verify_combine_kernel", attn_verify_combine_kernel<D>, dim3(combine_rows),
              dim3(64 * kCombineWaves), 0, stream, vp);
    return hipGetLastError();
}

PrefillParams fill_params(const AttnLaunch &a, int nseq, void *rope_scratch) {
    const auto *pool = a.pool;
    PrefillParams p{};
    p.k_pages = pool->k_pages;
    p.v_pages = pool->v_pages;
    p.page_table = pool->d_page_table;
    p.q = a.q;
    p.k = a.k;
    p.v = a.v;
    // without QK-norm the kernels still read a norm vector (unused): the
    // context's zeroed error-word block is readable and large enough
    p.q_norm = a.q_norm != nullptr ? a.q_norm : (const float *)a.err_word;
    p.k_norm = a.k_norm != nullptr ? a.k_norm : (const float *)a.err_word;
    p.positions = a.positions;
    p.out = a.out;
    p.rope_cs = (float2 *)rope_scratch;
    p.err_word = a.err_word;
    p.num_pages = pool->num_pages;
    p.pages_per_seq = pool->pages_per_seq;
    p.log2_page_tokens = (uint32_t)__builtin_ctz(pool->page_tokens);
    p.flags = a.flags;
    p.heads = a.heads;
    p.kv_heads = a.kv_heads * a.kv_rep;
    p.kv_rep = a.kv_rep;
    p.cache_kv_heads = a.kv_heads;
    p.rotary_dim = a.rotary_dim;
    p.mrope[0] = a.mrope[0];
    p.mrope[1] = a.mrope[1];
    p.mrope[2] = a.mrope[2];
    p.eps = a.eps;
    p.nseq = (uint32_t)nseq;
    p.rope = *a.rope;
    p.tbl_n = a.tbl_n;
    for (uint32_t i = 0; i < a.tbl_n; ++i) {
        p.tbl_idx[i] = a.tbl_idx[i];
        p.tbl_val[i] = a.tbl_val[i];
    }
    return p;
}

}  // namespace

bool prefill_supported(const AttnLaunch &a) {
    const uint32_t g = a.heads / (a.kv_heads * a.kv_rep);
    return (a.head_dim == 64 || a.head_dim == 128 || a.head_dim == 256) && g >= 1 && g <= 8 &&
           a.rotary_dim >= 32 && a.rotary_dim % 32 == 0;
}

size_t prefill_rope_bytes(const AttnLaunch &a, uint64_t total_rows) {
    return (size_t)total_rows * (a.rotary_dim / 2) * sizeof(float2);
}

hipError_t launch_attn_prefill(hipStream_t stream, const AttnLaunch &a, const SeqMeta *seqs,
                               int nseq, void *rope_scratch) {
    if (nseq <= 0 || nseq > kMetaPerLaunch || !prefill_supported(a) || rope_scratch == nullptr) {
        return hipErrorInvalidValue;
    }
    const uint32_t g = a.heads / (a.kv_heads * a.kv_rep);
    PrefillParams p = fill_params(a, nseq, rope_scratch);
    switch (a.head_dim) {
        case 64: return launch_d<64>(stream, p, g, seqs, nseq);
        case 128: return launch_d<128>(stream, p, g, seqs, nseq);
        case 256: return launch_d<256>(stream, p, g, seqs, nseq);
        default: return hipErrorInvalidValue;
    }
}

bool verify_supported(const AttnLaunch &a, uint32_t rows) {
    // any rows (the router sends 2..15): more than 64 query vectors per KV
    // head run as row slices
    return prefill_supported(a) && rows >= 2;
}

hipError_t launch_attn_verify(hipStream_t stream, const AttnLaunch &a, const SeqMeta *seqs,
                              int nseq, void *rope_scratch, const DecodePlanInput &in) {
    if (nseq <= 0 || nseq > kMetaPerLaunch || rope_scratch == nullptr) return hipErrorInvalidValue;
    const uint32_t kvv = a.kv_heads * a.kv_rep;  // KV heads of the grid
    const uint32_t g = a.heads / kvv;
    VerifyParams vp{};
    vp.p = fill_params(a, nseq, rope_scratch);
    PrefillParams &p = vp.p;
    // partition size: one workgroup per CU over the whole call, at least
    // 256 keys, a multiple of the 64-key tile
    uint64_t keys = 0;
    uint32_t max_rows = 0;
    for (int i = 0; i < nseq; ++i) {
        if (!verify_supported(a, seqs[i].rows)) return hipErrorInvalidValue;
        keys += (uint64_t)seqs[i].ctx + seqs[i].rows;
        max_rows = std::max(max_rows, seqs[i].rows);
    }
    // query vectors per workgroup: 64 in the pair mode; at D <= 128 a call
    // with more runs every consumer wave over both tiles of a step (128);
    // rows beyond run as further slices of the rows
    const bool all_tiles = a.head_dim <= 128 && max_rows * g > 64;
    vp.rows_per_slice = (all_tiles ? 128 : 64) / g;
    vp.slices = (max_rows + vp.rows_per_slice - 1) / vp.rows_per_slice;
    const uint64_t target = (uint64_t)std::max(in.num_cus, 1);
    uint64_t part = (keys * kvv * vp.slices + target - 1) / target;
    part = std::max<uint64_t>(256, (part + kKeyTile - 1) / kKeyTile * kKeyTile);
    // a partition starting mid-page touches at most part/page_tokens + 2 pages
    const uint64_t max_part =
        ((uint64_t)(kVerifyPageSlots - 2) * a.pool->page_tokens) / kKeyTile * kKeyTile;
    vp.part_keys = (uint32_t)std::min<uint64_t>(std::min(part, max_part), 1u << 30);
    const uint32_t tps = (a.head_dim <= 128 && !all_tiles) ? 2 : 1;  // records per partition
    uint32_t blocks = 0, records = 0, waves = 0;
    for (int i = 0; i < nseq; ++i) {
        PrefillMeta &m = p.meta[i];
        m.slot = seqs[i].slot;
        m.ctx = seqs[i].ctx;
        m.rows = seqs[i].rows;
        m.row0 = seqs[i].row0;
        const uint32_t parts = (m.ctx + m.rows + vp.part_keys - 1) / vp.part_keys;
        m.nblk = tps * parts;  // records per (row, head): one per tile of a step
        vp.blk0[i] = blocks;
        vp.rec0[i] = records;
        blocks += parts;
        records += m.nblk * m.rows * a.heads;
        waves += m.rows * a.heads;
    }
    p.max_blk = 0;
    const size_t stride = a.head_dim == 64    ? kRecordStride<64>
                          : a.head_dim == 128 ? kRecordStride<128>
                                              : kRecordStride<256>;
    vp.partials = in.reserve_partials((size_t)records * stride * sizeof(float));
    if (vp.partials == nullptr) return hipErrorOutOfMemory;
    // K/V of the new rows and their RoPE cos/sin first (append kernel)
    if (a.head_dim == 64) launch_append<64>(stream, p, max_rows);
    else if (a.head_dim == 128) launch_append<128>(stream, p, max_rows);
    else launch_append<256>(stream, p, max_rows);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    vp.units = blocks * kvv;
    // (unit, slice) blocks: groups of 8 units, each group's slices 8 apart
    const uint32_t grid = (vp.units + 7) / 8 * 8 * vp.slices;
    if (a.head_dim == 64) {
        return all_tiles ? launch_verify_d<64, true>(stream, vp, grid, waves)
                         : launch_verify_d<64, false>(stream, vp, grid, waves);
    }
    if (a.head_dim == 128) {
        return all_tiles ? launch_verify_d<128, true>(stream, vp, grid, waves)
                         : launch_verify_d<128, false>(stream, vp, grid, waves);
    }
    // several row slices read each partition's tiles: ordinary loads keep
    // them in L2 for the sibling slices (D <= 128 calls fit one slice)
    return vp.slices > 1 ? launch_verify_d<256, false, true>(stream, vp, grid, waves)
                         : launch_verify_d<256, false>(stream, vp, grid, waves);
}

}  // namespace sr
