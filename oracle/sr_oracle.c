/*
 * sr_oracle.c — TEST INFRASTRUCTURE ONLY (see sr_oracle.h).
 *
 * CPU restatement of the reference's hot-path math, used as the parity
 * checker for the HIP plugin and as the timed CPU baseline.  Citations are
 * file:line in the reference repository.  Build flags matter for fidelity:
 * -O2 -ffp-contract=off (Rust never contracts a*b+c into an FMA, and its
 * iterator sums are strictly left-to-right).
 */
#include "sr_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define SRO_OK 0
#define SRO_INVALID 1
#define SRO_NOMEM 4

/* src/model/math.rs:11-18 — branchy stable sigmoid. */
float sro_sigmoid(float x) {
    if (x >= 0.0f) {
        return 1.0f / (1.0f + expf(-x));
    }
    float e = expf(x);
    return e / (1.0f + e);
}

/* src/model/math.rs:20-22 */
float sro_silu(float x) { return x * sro_sigmoid(x); }

/* src/model/math.rs:24-26 — x.max(0) + exp(-|x|).ln_1p().  Rust's f32::max
 * returns the non-NaN operand, as fmaxf does. */
float sro_softplus(float x) { return fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x))); }

float sro_bf16_round(float x) {
    uint32_t bits;
    memcpy(&bits, &x, sizeof bits);
    if ((bits & 0x7f800000u) == 0x7f800000u && (bits & 0x007fffffu) != 0u) {
        bits = (bits | 0x00400000u) & 0xffff0000u; /* quiet NaN */
    } else {
        bits = (bits + 0x7fffu + ((bits >> 16) & 1u)) & 0xffff0000u;
    }
    float out;
    memcpy(&out, &bits, sizeof out);
    return out;
}

/* Sequential f32 dot product: iter().zip().map(|(a,b)| a*b).sum::<f32>(). */
static float dot_f32(const float *a, const float *b, size_t n) {
    float acc = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        acc += a[i] * b[i];
    }
    return acc;
}

/* src/model/math.rs:28-50 */
int sro_rms_norm(const float *input, size_t n, const float *weight, size_t wn, float eps,
                 int offset, float *output) {
    if (wn == 0 || n % wn != 0 || !isfinite(eps) || eps <= 0.0f) {
        return SRO_INVALID; /* :29-35 */
    }
    const float add = offset ? 1.0f : 0.0f;
    for (size_t row = 0; row < n / wn; ++row) {
        const float *x = input + row * wn;
        float sumsq = 0.0f;
        for (size_t i = 0; i < wn; ++i) {
            sumsq += x[i] * x[i]; /* :38 */
        }
        float variance = sumsq / (float)wn;
        if (!isfinite(variance)) {
            return SRO_INVALID; /* :39-41 */
        }
        float inv = 1.0f / sqrtf(variance + eps); /* :42 */
        for (size_t i = 0; i < wn; ++i) {
            output[row * wn + i] = x[i] * inv * (weight[i] + add); /* :46 */
        }
    }
    return SRO_OK;
}

/* src/model/math.rs:52-99 */
int sro_apply_rope(float *values, size_t n, size_t head_dim, const int64_t position[3],
                   float theta, size_t rotary_dim, const int64_t *mrope_section,
                   int interleaved) {
    if (head_dim == 0 || n % head_dim != 0 || rotary_dim == 0 || rotary_dim > head_dim ||
        rotary_dim % 2 != 0) {
        return SRO_INVALID; /* :58-65 */
    }
    const size_t half = rotary_dim / 2;
    for (size_t h = 0; h < n / head_dim; ++h) {
        float *head = values + h * head_dim;
        for (size_t i = 0; i < half; ++i) {
            size_t axis = 0; /* :69-89 */
            if (mrope_section != NULL) {
                const size_t s0 = (size_t)mrope_section[0];
                const size_t s1 = (size_t)mrope_section[1];
                const size_t s2 = (size_t)mrope_section[2];
                if (interleaved) {
                    if (i % 3 == 1 && i < s1 * 3) {
                        axis = 1;
                    } else if (i % 3 == 2 && i < s2 * 3) {
                        axis = 2;
                    } else {
                        axis = 0;
                    }
                } else {
                    axis = i < s0 ? 0 : (i < s0 + s1 ? 1 : 2);
                }
            }
            /* :90-91 — angle = pos as f32 / theta.powf(2i as f32 / rotary_dim as f32) */
            const float exponent = (float)(2 * i) / (float)rotary_dim;
            const float angle = (float)position[axis] / powf(theta, exponent);
            const float s = sinf(angle); /* :92 sin_cos */
            const float c = cosf(angle);
            const float left = head[i];
            const float right = head[i + half];
            head[i] = left * c - right * s;        /* :94 */
            head[i + half] = right * c + left * s; /* :95 */
        }
    }
    return SRO_OK;
}

/* ---------------- PagedKvCache (src/engine/state.rs:19-127) ---------------- */

struct sro_kv {
    float *keys;
    float *values;
    size_t width;
    size_t max_tokens;
    size_t page_tokens;
    size_t len;
    size_t capacity; /* tokens allocated */
    int bf16_storage;
};

sro_kv *sro_kv_new(size_t width, size_t max_tokens, size_t page_tokens, int bf16_storage) {
    if (width == 0 || max_tokens == 0 || page_tokens == 0) {
        return NULL; /* state.rs:29-31 */
    }
    sro_kv *kv = (sro_kv *)calloc(1, sizeof *kv);
    if (kv == NULL) {
        return NULL;
    }
    kv->width = width;
    kv->max_tokens = max_tokens;
    kv->page_tokens = page_tokens;
    kv->bf16_storage = bf16_storage;
    return kv;
}

void sro_kv_free(sro_kv *kv) {
    if (kv != NULL) {
        free(kv->keys);
        free(kv->values);
        free(kv);
    }
}

static int kv_reserve(sro_kv *kv, size_t tokens) {
    if (tokens <= kv->capacity) {
        return SRO_OK;
    }
    /* grow by whole pages, never past max_tokens (state.rs:59-80) */
    size_t cap = kv->capacity == 0 ? kv->page_tokens : kv->capacity;
    while (cap < tokens) {
        cap *= 2;
    }
    if (cap > kv->max_tokens) {
        cap = kv->max_tokens;
    }
    float *k = (float *)realloc(kv->keys, cap * kv->width * sizeof(float));
    if (k == NULL) {
        return SRO_NOMEM;
    }
    kv->keys = k;
    float *v = (float *)realloc(kv->values, cap * kv->width * sizeof(float));
    if (v == NULL) {
        return SRO_NOMEM;
    }
    kv->values = v;
    kv->capacity = cap;
    return SRO_OK;
}

sro_kv *sro_kv_clone(const sro_kv *kv) {
    sro_kv *copy = sro_kv_new(kv->width, kv->max_tokens, kv->page_tokens, kv->bf16_storage);
    if (copy == NULL) {
        return NULL;
    }
    if (kv->len > 0) {
        if (kv_reserve(copy, kv->len) != SRO_OK) {
            sro_kv_free(copy);
            return NULL;
        }
        memcpy(copy->keys, kv->keys, kv->len * kv->width * sizeof(float));
        memcpy(copy->values, kv->values, kv->len * kv->width * sizeof(float));
    }
    copy->len = kv->len;
    return copy;
}

size_t sro_kv_len(const sro_kv *kv) { return kv->len; }

/* state.rs:52-84 */
int sro_kv_append(sro_kv *kv, const float *key, const float *value) {
    if (kv->len == kv->max_tokens) {
        return SRO_INVALID; /* :53-55 */
    }
    for (size_t i = 0; i < kv->width; ++i) {
        if (!isfinite(key[i]) || !isfinite(value[i])) {
            return SRO_INVALID; /* :56-58 */
        }
    }
    int status = kv_reserve(kv, kv->len + 1);
    if (status != SRO_OK) {
        return status;
    }
    float *k = kv->keys + kv->len * kv->width;
    float *v = kv->values + kv->len * kv->width;
    for (size_t i = 0; i < kv->width; ++i) {
        k[i] = kv->bf16_storage ? sro_bf16_round(key[i]) : key[i];
        v[i] = kv->bf16_storage ? sro_bf16_round(value[i]) : value[i];
    }
    kv->len += 1;
    return SRO_OK;
}

int sro_kv_append_many(sro_kv *kv, const float *keys, const float *values, size_t n) {
    int status = kv_reserve(kv, kv->len + n < kv->max_tokens ? kv->len + n : kv->max_tokens);
    if (status != SRO_OK) {
        return status;
    }
    for (size_t t = 0; t < n; ++t) {
        status = sro_kv_append(kv, keys + t * kv->width, values + t * kv->width);
        if (status != SRO_OK) {
            return status;
        }
    }
    return SRO_OK;
}

/* state.rs:86-96 */
int sro_kv_get(const sro_kv *kv, size_t token, float *key, float *value) {
    if (token >= kv->len) {
        return SRO_INVALID;
    }
    memcpy(key, kv->keys + token * kv->width, kv->width * sizeof(float));
    memcpy(value, kv->values + token * kv->width, kv->width * sizeof(float));
    return SRO_OK;
}

/* state.rs:99-119 */
int sro_kv_truncate(sro_kv *kv, size_t len) {
    if (len > kv->len) {
        return SRO_INVALID;
    }
    kv->len = len;
    return SRO_OK;
}

/* ---------------- causal_attention (src/model/math.rs:102-155) ---------------- */

static void attention_heads(const float *query, const sro_kv *cache, size_t heads,
                            size_t kv_heads, size_t dim, float *output, size_t h0, size_t h1) {
    const float scale = 1.0f / sqrtf((float)dim); /* :126 */
    for (size_t h = h0; h < h1; ++h) {
        const float *q = query + h * dim;
        const size_t kv_offset = h / (heads / kv_heads) * dim; /* :129 */
        float *out = output + h * dim;
        for (size_t i = 0; i < dim; ++i) {
            out[i] = 0.0f;
        }
        float maximum = -INFINITY;
        float normalizer = 0.0f;
        for (size_t token = 0; token < cache->len; ++token) {
            const float *key = cache->keys + token * cache->width + kv_offset;
            const float *value = cache->values + token * cache->width + kv_offset;
            const float score = dot_f32(q, key, dim) * scale; /* :135-140 */
            const float next_max = fmaxf(maximum, score);      /* :141 */
            const float prior = expf(maximum - next_max);      /* :142 */
            const float current = expf(score - next_max);      /* :143 */
            normalizer = normalizer * prior + current;         /* :144 */
            for (size_t i = 0; i < dim; ++i) {
                out[i] = out[i] * prior + value[i] * current; /* :145-147 */
            }
            maximum = next_max;
        }
        for (size_t i = 0; i < dim; ++i) {
            out[i] /= normalizer; /* :150-152 */
        }
    }
}

static int attention_geometry_ok(const float *query, const sro_kv *cache, size_t heads,
                                 size_t kv_heads, size_t dim) {
    (void)query;
    return !(heads == 0 || kv_heads == 0 || dim == 0 || heads % kv_heads != 0 ||
             cache->width != kv_heads * dim || cache->len == 0); /* :109-124 */
}

int sro_causal_attention(const float *query, const sro_kv *cache, size_t heads,
                         size_t kv_heads, size_t dim, float *output) {
    if (!attention_geometry_ok(query, cache, heads, kv_heads, dim)) {
        return SRO_INVALID;
    }
    attention_heads(query, cache, heads, kv_heads, dim, output, 0, heads);
    return SRO_OK;
}

typedef struct {
    const float *query;
    const sro_kv *cache;
    size_t heads, kv_heads, dim, h0, h1;
    float *output;
} attn_job;

static void *attn_worker(void *arg) {
    attn_job *job = (attn_job *)arg;
    attention_heads(job->query, job->cache, job->heads, job->kv_heads, job->dim, job->output,
                    job->h0, job->h1);
    return NULL;
}

int sro_causal_attention_mt(const float *query, const sro_kv *cache, size_t heads,
                            size_t kv_heads, size_t dim, float *output, int nthreads) {
    if (!attention_geometry_ok(query, cache, heads, kv_heads, dim)) {
        return SRO_INVALID;
    }
    if (nthreads <= 1 || heads == 1) {
        attention_heads(query, cache, heads, kv_heads, dim, output, 0, heads);
        return SRO_OK;
    }
    if ((size_t)nthreads > heads) {
        nthreads = (int)heads;
    }
    pthread_t threads[256];
    attn_job jobs[256];
    if (nthreads > 256) {
        nthreads = 256;
    }
    for (int t = 0; t < nthreads; ++t) {
        jobs[t] = (attn_job){query,
                             cache,
                             heads,
                             kv_heads,
                             dim,
                             heads * (size_t)t / (size_t)nthreads,
                             heads * (size_t)(t + 1) / (size_t)nthreads,
                             output};
        if (pthread_create(&threads[t], NULL, attn_worker, &jobs[t]) != 0) {
            attn_worker(&jobs[t]);
            threads[t] = 0;
        }
    }
    for (int t = 0; t < nthreads; ++t) {
        if (threads[t] != 0) {
            pthread_join(threads[t], NULL);
        }
    }
    return SRO_OK;
}

/* ---------------- causal_conv_silu (src/model/math.rs:158-187) ---------------- */

int sro_causal_conv_silu(const float *input, size_t channels, const float *weight,
                         size_t kernel, float *history, float *output) {
    if (kernel == 0) {
        return SRO_INVALID; /* :164-173 */
    }
    for (size_t c = 0; c < channels; ++c) {
        const float *w = weight + c * kernel;
        float *prior = history + c * (kernel - 1);
        const float x = input[c];
        const float value = dot_f32(prior, w, kernel - 1) + x * w[kernel - 1]; /* :179 */
        output[c] = sro_silu(value);                                            /* :180 */
        if (kernel > 1) {                                                       /* :181-184 */
            for (size_t j = 0; j + 1 < kernel - 1; ++j) {
                prior[j] = prior[j + 1];
            }
            prior[kernel - 2] = x;
        }
    }
    return SRO_OK;
}

/* ---------------- gated_delta_step (src/model/math.rs:190-239) ---------------- */

/* value heads h0..h1-1 of one gated_delta_step: every head's arithmetic
 * depends only on its own state rows and the row's q/k of its key head */
static void delta_heads(const float *qkv, const float *a, const float *b, const float *a_log,
                        const float *dt_bias, size_t key_heads, size_t value_heads,
                        size_t key_dim, size_t value_dim, size_t h0, size_t h1, float *state,
                        float *output) {
    const size_t key_width = key_heads * key_dim;
    const size_t key_groups = value_heads / key_heads;
    const float query_scale = 1.0f / sqrtf((float)key_dim); /* :213 */
    for (size_t h = h0; h < h1; ++h) {
        const size_t start = h / key_groups * key_dim; /* :215 */
        const float *q = qkv + start;
        const float *k = qkv + key_width + start;
        const float qi = 1.0f / sqrtf(dot_f32(q, q, key_dim) + 1e-6f); /* :218 */
        const float ki = 1.0f / sqrtf(dot_f32(k, k, key_dim) + 1e-6f); /* :219 */
        const float alpha = expf(-expf(a_log[h]) * sro_softplus(a[h] + dt_bias[h])); /* :220 */
        const float beta = sro_sigmoid(b[h]);                                        /* :221 */
        for (size_t v = 0; v < value_dim; ++v) {
            float *row = state + (h * value_dim + v) * key_dim; /* :223-224 */
            for (size_t i = 0; i < key_dim; ++i) {
                row[i] *= alpha; /* :226-228 decay first */
            }
            float prediction = 0.0f;
            for (size_t i = 0; i < key_dim; ++i) {
                prediction += row[i] * k[i] * ki; /* :229 */
            }
            const float correction =
                beta * (qkv[2 * key_width + h * value_dim + v] - prediction); /* :230 */
            for (size_t i = 0; i < key_dim; ++i) {
                row[i] += correction * k[i] * ki; /* :231-233 */
            }
            float read = 0.0f;
            for (size_t i = 0; i < key_dim; ++i) {
                read += row[i] * q[i] * qi; /* :234-235 */
            }
            output[h * value_dim + v] = read * query_scale;
        }
    }
}

int sro_gated_delta_step(const float *qkv, const float *a, const float *b,
                         const float *a_log, const float *dt_bias, size_t key_heads,
                         size_t value_heads, size_t key_dim, size_t value_dim, float *state,
                         float *output) {
    if (key_heads == 0 || value_heads % key_heads != 0) {
        return SRO_INVALID; /* :201-210 */
    }
    delta_heads(qkv, a, b, a_log, dt_bias, key_heads, value_heads, key_dim, value_dim, 0,
                value_heads, state, output);
    return SRO_OK;
}

/* ---------------- Attention::forward rows (src/model/native.rs:615-645) ---------------- */

int sro_attention_rows(const float *q_raw, const float *k_raw, const float *v_raw, size_t rows,
                       const int64_t *positions, size_t heads, size_t kv_heads, size_t dim,
                       int gated, const float *q_norm, const float *k_norm, float eps,
                       float theta, size_t rotary_dim, const int64_t *mrope_section,
                       int interleaved, sro_kv *cache, float *out, int nthreads) {
    const size_t q_width = heads * dim;
    const size_t kv_width = kv_heads * dim;
    float *query = (float *)malloc(q_width * sizeof(float));
    float *gate = (float *)malloc(q_width * sizeof(float));
    float *key = (float *)malloc(kv_width * sizeof(float));
    float *tmp = (float *)malloc((q_width > kv_width ? q_width : kv_width) * sizeof(float));
    int status = SRO_OK;
    if (query == NULL || gate == NULL || key == NULL || tmp == NULL) {
        status = SRO_NOMEM;
        goto done;
    }
    for (size_t row = 0; row < rows && status == SRO_OK; ++row) {
        if (gated) { /* :618-624 — per-head interleaved [q, gate] */
            const float *src = q_raw + row * q_width * 2;
            for (size_t h = 0; h < heads; ++h) {
                memcpy(query + h * dim, src + h * 2 * dim, dim * sizeof(float));
                memcpy(gate + h * dim, src + h * 2 * dim + dim, dim * sizeof(float));
            }
        } else {
            memcpy(query, q_raw + row * q_width, q_width * sizeof(float));
        }
        memcpy(key, k_raw + row * kv_width, kv_width * sizeof(float));
        if (q_norm != NULL) { /* :629-631 */
            status = sro_rms_norm(query, q_width, q_norm, dim, eps, gated, tmp);
            if (status != SRO_OK) break;
            memcpy(query, tmp, q_width * sizeof(float));
        }
        if (k_norm != NULL) { /* :632-634 */
            status = sro_rms_norm(key, kv_width, k_norm, dim, eps, gated, tmp);
            if (status != SRO_OK) break;
            memcpy(key, tmp, kv_width * sizeof(float));
        }
        const int64_t *pos = positions + row * 3;
        status = sro_apply_rope(query, q_width, dim, pos, theta, rotary_dim, mrope_section,
                                interleaved); /* :635 */
        if (status != SRO_OK) break;
        status = sro_apply_rope(key, kv_width, dim, pos, theta, rotary_dim, mrope_section,
                                interleaved); /* :636 */
        if (status != SRO_OK) break;
        status = sro_kv_append(cache, key, v_raw + row * kv_width); /* :637 */
        if (status != SRO_OK) break;
        float *o = out + row * q_width;
        status = sro_causal_attention_mt(query, cache, heads, kv_heads, dim, o, nthreads); /* :638 */
        if (status != SRO_OK) break;
        if (gated) { /* :639-643 */
            for (size_t i = 0; i < q_width; ++i) {
                o[i] *= sro_sigmoid(gate[i]);
            }
        }
    }
done:
    free(query);
    free(gate);
    free(key);
    free(tmp);
    return status;
}

/* ---------------- Gdn::forward rows (src/model/native.rs:720-742) ---------------- */

int sro_gdn_rows(const float *qkv, const float *z, const float *a, const float *b, size_t rows,
                 const float *a_log, const float *dt_bias, const float *conv_weight,
                 size_t kernel, const float *norm, float eps, size_t key_heads,
                 size_t value_heads, size_t key_dim, size_t value_dim, float *history,
                 float *state, float *out) {
    const size_t channels = 2 * key_heads * key_dim + value_heads * value_dim;
    const size_t width = value_heads * value_dim;
    float *conv = (float *)malloc(channels * sizeof(float));
    float *recurrent = (float *)malloc(width * sizeof(float));
    int status = SRO_OK;
    if (conv == NULL || recurrent == NULL) {
        status = SRO_NOMEM;
        goto done;
    }
    for (size_t row = 0; row < rows; ++row) {
        status = sro_causal_conv_silu(qkv + row * channels, channels, conv_weight, kernel,
                                      history, conv); /* :721-726 */
        if (status != SRO_OK) break;
        status = sro_gated_delta_step(conv, a + row * value_heads, b + row * value_heads, a_log,
                                      dt_bias, key_heads, value_heads, key_dim, value_dim, state,
                                      recurrent); /* :727-736 */
        if (status != SRO_OK) break;
        float *o = out + row * width;
        status = sro_rms_norm(recurrent, width, norm, value_dim, eps, 0, o); /* :737 */
        if (status != SRO_OK) break;
        for (size_t i = 0; i < width; ++i) {
            o[i] *= sro_silu(z[row * width + i]); /* :738-740 */
        }
    }
done:
    free(conv);
    free(recurrent);
    return status;
}

/* sro_gdn_rows with the value heads split over threads (the CPU baseline's
 * all-cores figure).  The conv of every row runs first (it reads no state);
 * then each thread runs the delta rule, norm and gate of its heads over all
 * rows.  Every head's operations and their order are those of sro_gdn_rows,
 * so the results are identical to it bit for bit. */
typedef struct {
    const float *conv, *z, *a, *b, *a_log, *dt_bias, *norm;
    size_t rows, channels, key_heads, value_heads, key_dim, value_dim, h0, h1;
    float eps;
    float *state, *recurrent, *out;
    int status;
} gdn_job;

static void *gdn_worker(void *arg) {
    gdn_job *j = (gdn_job *)arg;
    const size_t width = j->value_heads * j->value_dim;
    for (size_t row = 0; row < j->rows; ++row) {
        float *rec = j->recurrent + row * width;
        delta_heads(j->conv + row * j->channels, j->a + row * j->value_heads,
                    j->b + row * j->value_heads, j->a_log, j->dt_bias, j->key_heads,
                    j->value_heads, j->key_dim, j->value_dim, j->h0, j->h1, j->state, rec);
        const size_t off = j->h0 * j->value_dim, n = (j->h1 - j->h0) * j->value_dim;
        float *o = j->out + row * width + off;
        const int st = sro_rms_norm(rec + off, n, j->norm, j->value_dim, j->eps, 0, o);
        if (st != SRO_OK) {
            j->status = st;
            return NULL;
        }
        for (size_t i = 0; i < n; ++i) {
            o[i] *= sro_silu(j->z[row * width + off + i]);
        }
    }
    return NULL;
}

int sro_gdn_rows_mt(const float *qkv, const float *z, const float *a, const float *b,
                    size_t rows, const float *a_log, const float *dt_bias,
                    const float *conv_weight, size_t kernel, const float *norm, float eps,
                    size_t key_heads, size_t value_heads, size_t key_dim, size_t value_dim,
                    float *history, float *state, float *out, int nthreads) {
    if (key_heads == 0 || value_heads % key_heads != 0) {
        return SRO_INVALID;
    }
    if (nthreads <= 1) {
        return sro_gdn_rows(qkv, z, a, b, rows, a_log, dt_bias, conv_weight, kernel, norm, eps,
                            key_heads, value_heads, key_dim, value_dim, history, state, out);
    }
    if ((size_t)nthreads > value_heads) nthreads = (int)value_heads;
    if (nthreads > 256) nthreads = 256;
    const size_t channels = 2 * key_heads * key_dim + value_heads * value_dim;
    const size_t width = value_heads * value_dim;
    float *conv = (float *)malloc(rows * channels * sizeof(float) + 1);
    float *recurrent = (float *)malloc(rows * width * sizeof(float) + 1);
    int status = SRO_OK;
    if (conv == NULL || recurrent == NULL) {
        status = SRO_NOMEM;
        goto done;
    }
    for (size_t row = 0; row < rows; ++row) {
        status = sro_causal_conv_silu(qkv + row * channels, channels, conv_weight, kernel,
                                      history, conv + row * channels);
        if (status != SRO_OK) goto done;
    }
    {
        pthread_t threads[256];
        gdn_job jobs[256];
        for (int t = 0; t < nthreads; ++t) {
            gdn_job j = {conv, z, a, b, a_log, dt_bias, norm, rows, channels, key_heads,
                         value_heads, key_dim, value_dim,
                         value_heads * (size_t)t / (size_t)nthreads,
                         value_heads * (size_t)(t + 1) / (size_t)nthreads, eps, state,
                         recurrent, out, SRO_OK};
            jobs[t] = j;
            if (pthread_create(&threads[t], NULL, gdn_worker, &jobs[t]) != 0) {
                gdn_worker(&jobs[t]);
                threads[t] = 0;
            }
        }
        for (int t = 0; t < nthreads; ++t) {
            if (threads[t] != 0) pthread_join(threads[t], NULL);
            if (jobs[t].status != SRO_OK) status = jobs[t].status;
        }
    }
done:
    free(conv);
    free(recurrent);
    return status;
}

/* ---- ABI v1 linear (native/cpu/safetyraise_cpu.c:47-89, :203-239) ---- */

/* IEEE binary16 -> binary32, exact for every input (normal, subnormal,
 * zero, infinity and NaN payloads). */
static float sro_half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exponent = (h >> 10) & 0x1fu;
    uint32_t fraction = h & 0x3ffu;
    uint32_t bits;
    if (exponent == 0u) {
        if (fraction == 0u) {
            bits = sign;
        } else {
            int e = -14;
            while ((fraction & 0x400u) == 0u) {
                fraction <<= 1;
                --e;
            }
            bits = sign | ((uint32_t)(e + 127) << 23) | ((fraction & 0x3ffu) << 13);
        }
    } else if (exponent == 0x1fu) {
        bits = sign | 0x7f800000u | (fraction << 13);
    } else {
        bits = sign | ((exponent + 112u) << 23) | (fraction << 13);
    }
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

static float sro_weight_value(const void *weight, uint32_t dtype, size_t index) {
    if (dtype == 1u) {
        return ((const float *)weight)[index];
    }
    const uint16_t bits = ((const uint16_t *)weight)[index];
    if (dtype == 2u) {
        return sro_half_to_float(bits);
    }
    const uint32_t wide = (uint32_t)bits << 16;
    float f;
    memcpy(&f, &wide, sizeof f);
    return f;
}

void sro_silu_mul(const float *gate, const float *up, size_t n, float *out) {
    for (size_t i = 0; i < n; ++i) {
        out[i] = sro_silu(gate[i]) * up[i]; /* native.rs:551 */
    }
}

int sro_linear(const float *input, size_t rows, size_t cols, const void *weight,
               uint32_t dtype, size_t out_features, float *output) {
    if (dtype < 1u || dtype > 3u) {
        return 1;
    }
    for (size_t i = 0; i < rows * cols; ++i) {
        if (!isfinite(input[i])) {
            return 1;
        }
    }
    for (size_t r = 0; r < rows; ++r) {
        for (size_t o = 0; o < out_features; ++o) {
            float sum = 0.0f;
            for (size_t c = 0; c < cols; ++c) {
                sum += input[r * cols + c] * sro_weight_value(weight, dtype, o * cols + c);
            }
            output[r * out_features + o] = sum;
        }
    }
    return 0;
}
