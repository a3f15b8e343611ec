/*
 * sr_oracle — CPU restatement of the rsinfer attention / gated-delta-net math.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * plugin and the timed CPU baseline.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it; the plugin never links or calls it.
 *
 * Every function restates one reference function (file:line under the
 * reference repository) with the same operation order: sequential f32 sums,
 * no FMA contraction (built with -ffp-contract=off), glibc libm for exp, log1p,
 * pow, sin and cos, exactly as Rust's f32 methods lower on Linux.
 *
 * Return value of every int function: 0 = OK, 1 = invalid argument (the
 * reference's RsinferError::DimensionError cases), 4 = out of memory.
 */
#ifndef SR_ORACLE_H
#define SR_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

float sro_sigmoid(float x);  /* src/model/math.rs:11-18 */
float sro_silu(float x);     /* src/model/math.rs:20-22 */
float sro_softplus(float x); /* src/model/math.rs:24-26 */
float sro_bf16_round(float x); /* round-to-nearest-even to bf16, widened back */

/* src/model/math.rs:28-50 */
int sro_rms_norm(const float *input, size_t n, const float *weight, size_t wn,
                 float eps, int offset, float *output);

/* src/model/math.rs:52-99.  position[3] are the three MRoPE axes; a NULL
 * mrope_section means None. */
int sro_apply_rope(float *values, size_t n, size_t head_dim, const int64_t position[3],
                   float theta, size_t rotary_dim, const int64_t *mrope_section,
                   int interleaved);

/* src/engine/state.rs:19-127 (PagedKvCache).  Token rows are kept in one
 * contiguous array; pages only decide allocation granularity in the
 * reference, never values.  bf16_storage != 0 rounds appended K/V to bf16
 * (the plugin's storage format), otherwise f32 as in the reference. */
typedef struct sro_kv sro_kv;
sro_kv *sro_kv_new(size_t width, size_t max_tokens, size_t page_tokens, int bf16_storage);
void sro_kv_free(sro_kv *kv);
sro_kv *sro_kv_clone(const sro_kv *kv); /* SequenceState::checkpoint, state.rs:222-224 */
size_t sro_kv_len(const sro_kv *kv);
int sro_kv_append(sro_kv *kv, const float *key, const float *value);            /* :52-84 */
int sro_kv_append_many(sro_kv *kv, const float *keys, const float *values, size_t n);
int sro_kv_get(const sro_kv *kv, size_t token, float *key, float *value);        /* :86-96 */
int sro_kv_truncate(sro_kv *kv, size_t len);                                      /* :99-119 */

/* src/model/math.rs:102-155 */
int sro_causal_attention(const float *query, const sro_kv *cache, size_t heads,
                         size_t kv_heads, size_t dim, float *output);
/* Same arithmetic per head, heads split over nthreads POSIX threads
 * (the "all host cores" CPU baseline; per-head results are identical). */
int sro_causal_attention_mt(const float *query, const sro_kv *cache, size_t heads,
                            size_t kv_heads, size_t dim, float *output, int nthreads);

/* src/model/math.rs:158-187 */
int sro_causal_conv_silu(const float *input, size_t channels, const float *weight,
                         size_t kernel, float *history, float *output);

/* src/model/math.rs:190-239.  state is [Hv][Dv][Dk]. */
int sro_gated_delta_step(const float *qkv, const float *a, const float *b,
                         const float *a_log, const float *dt_bias, size_t key_heads,
                         size_t value_heads, size_t key_dim, size_t value_dim,
                         float *state, float *output);

/* Attention::forward row loop without the projections,
 * src/model/native.rs:615-645.  q_raw rows are heads*dim wide, or
 * heads*2*dim with per-head [q(dim), gate(dim)] when gated != 0.
 * q_norm/k_norm NULL = no QK-norm (Qwen2).  Norm offset = gated (Qwen3.5).
 * positions: rows*3.  out: rows*heads*dim. */
int sro_attention_rows(const float *q_raw, const float *k_raw, const float *v_raw,
                       size_t rows, const int64_t *positions, size_t heads,
                       size_t kv_heads, size_t dim, int gated, const float *q_norm,
                       const float *k_norm, float eps, float theta, size_t rotary_dim,
                       const int64_t *mrope_section, int interleaved, sro_kv *cache,
                       float *out, int nthreads);

/* Gdn::forward row loop without the projections, src/model/native.rs:720-742.
 * qkv: rows*C with C = 2*Hk*Dk + Hv*Dv; z: rows*Hv*Dv; a, b: rows*Hv;
 * conv_weight: C*kernel; history: C*(kernel-1); state: Hv*Dv*Dk;
 * norm: Dv; out: rows*Hv*Dv. */
int sro_gdn_rows(const float *qkv, const float *z, const float *a, const float *b,
                 size_t rows, const float *a_log, const float *dt_bias,
                 const float *conv_weight, size_t kernel, const float *norm, float eps,
                 size_t key_heads, size_t value_heads, size_t key_dim, size_t value_dim,
                 float *history, float *state, float *out);

/* sro_gdn_rows with value heads split over nthreads threads; bit-identical
 * results (test infrastructure: the CPU baseline's all-cores figure). */
int sro_gdn_rows_mt(const float *qkv, const float *z, const float *a, const float *b,
                    size_t rows, const float *a_log, const float *dt_bias,
                    const float *conv_weight, size_t kernel, const float *norm, float eps,
                    size_t key_heads, size_t value_heads, size_t key_dim, size_t value_dim,
                    float *history, float *state, float *out, int nthreads);

/* ABI v1 linear (native/cpu/safetyraise_cpu.c:203-239): output[r][o] =
 * sum over c, in order, of input[r][c] * weight[o][c] in f32, with the weight
 * widened exactly from its dtype (1 = f32, 2 = f16 as :47-78, 3 = bf16 by
 * shift).  Returns 1 for a non-finite input (:221-226) or an unknown dtype. */
/* src/model/native.rs:550-552 (Block::forward, the MLP): out[i] =
 * silu(gate[i]) * up[i], with math.rs:20-22's silu. */
void sro_silu_mul(const float *gate, const float *up, size_t n, float *out);

int sro_linear(const float *input, size_t rows, size_t cols, const void *weight,
               uint32_t dtype, size_t out_features, float *output);

#ifdef __cplusplus
}
#endif

#endif
