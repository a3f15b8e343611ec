// Paged KV cache data movement: page-table updates, raw row append (scatter)
// and row read-back (gather) in the reference's token-major row layout.
//
// Pool layout in HBM: [kv_head][page][page_tokens][head_dim] bf16 (head
// major), so a head's pages are adjacent.  A reference row (one token,
// [kv_head][head_dim], src/engine/state.rs:90-95) is spread over kv_heads
// runs of head_dim values, one per head region.
#include "sr_device.hpp"

namespace sr {

namespace {

constexpr int kTableBatch = 224;

struct TableUpdate {
    int32_t *table;
    int n;
    uint32_t idx[kTableBatch];
    int32_t val[kTableBatch];
};

__global__ void page_table_set_kernel(const TableUpdate u) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < u.n) {
        u.table[u.idx[i]] = u.val[i];
    }
}

struct ScatterParams {
    uint16_t *k_pages;
    uint16_t *v_pages;
    const int32_t *table;  // row of the sequence
    const void *keys;
    const void *values;
    uint32_t *err_word;
    uint64_t start;
    uint64_t tokens;
    uint64_t num_pages;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t page_tokens;
    int bf16_in;
};

// One thread per 8 consecutive values of one (token, head).
__global__ void kv_scatter_kernel(const ScatterParams p) {
    const uint32_t per_head = p.head_dim / 8;
    const uint64_t n = p.tokens * p.kv_heads * per_head;
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t c = (uint32_t)(i % per_head);
        const uint64_t th = i / per_head;
        const uint32_t h = (uint32_t)(th % p.kv_heads);
        const uint64_t t = th / p.kv_heads;
        const uint64_t tok = p.start + t;
        const int32_t page = p.table[tok / p.page_tokens];
        const size_t dst = (((size_t)h * p.num_pages + page) * p.page_tokens + tok % p.page_tokens) *
                               p.head_dim + (size_t)c * 8;
        const size_t src = (t * p.kv_heads + h) * (size_t)p.head_dim + (size_t)c * 8;
        uint4 kw, vw;
        bool finite = true;
        if (p.bf16_in) {
            kw = *(const uint4 *)((const uint16_t *)p.keys + src);
            vw = *(const uint4 *)((const uint16_t *)p.values + src);
            const uint32_t *kk = (const uint32_t *)&kw;
            const uint32_t *vv = (const uint32_t *)&vw;
            for (int j = 0; j < 4; ++j) {
                finite = finite && isfinite(bf16lo(kk[j])) && isfinite(bf16hi(kk[j])) &&
                         isfinite(bf16lo(vv[j])) && isfinite(bf16hi(vv[j]));
            }
        } else {
            const float4 *kf = (const float4 *)((const float *)p.keys + src);
            const float4 *vf = (const float4 *)((const float *)p.values + src);
            const float4 k0 = kf[0], k1 = kf[1], v0 = vf[0], v1 = vf[1];
            const float kx[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
            const float vx[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
            uint32_t *kk = (uint32_t *)&kw;
            uint32_t *vv = (uint32_t *)&vw;
            for (int j = 0; j < 4; ++j) {
                kk[j] = pack_bf16x2(kx[2 * j], kx[2 * j + 1]);
                vv[j] = pack_bf16x2(vx[2 * j], vx[2 * j + 1]);
            }
            for (int j = 0; j < 8; ++j) {
                finite = finite && isfinite(kx[j]) && isfinite(vx[j]);
            }
        }
        if (!finite) {
            atomicOr(p.err_word, kErrNonFiniteKv);
        }
        *(uint4 *)(p.k_pages + dst) = kw;
        *(uint4 *)(p.v_pages + dst) = vw;
    }
}

// One thread per value: head widths that are not a multiple of 8 (a run of
// 8 values would straddle two heads or start off a 16-byte boundary).
__global__ void kv_scatter_elem_kernel(const ScatterParams p) {
    const uint64_t width = (uint64_t)p.kv_heads * p.head_dim;
    const uint64_t n = p.tokens * width;
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t t = i / width;
        const uint32_t r = (uint32_t)(i % width);
        const uint32_t h = r / p.head_dim;
        const uint32_t d = r % p.head_dim;
        const uint64_t tok = p.start + t;
        const int32_t page = p.table[tok / p.page_tokens];
        const size_t dst =
            (((size_t)h * p.num_pages + page) * p.page_tokens + tok % p.page_tokens) * p.head_dim + d;
        const float k = load_act(p.keys, i, p.bf16_in != 0);
        const float v = load_act(p.values, i, p.bf16_in != 0);
        if (!isfinite(k) || !isfinite(v)) atomicOr(p.err_word, kErrNonFiniteKv);
        p.k_pages[dst] = f32_to_bf16(k);
        p.v_pages[dst] = f32_to_bf16(v);
    }
}

struct GatherParams {
    const uint16_t *k_pages;
    const uint16_t *v_pages;
    const int32_t *table;
    float *keys;
    float *values;
    uint64_t start;
    uint64_t tokens;
    uint64_t num_pages;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t page_tokens;
};

__global__ void kv_gather_kernel(const GatherParams p) {
    const uint64_t width = (uint64_t)p.kv_heads * p.head_dim;
    const uint64_t n = p.tokens * width;
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t t = i / width;
        const uint32_t r = (uint32_t)(i % width);
        const uint32_t h = r / p.head_dim;
        const uint32_t d = r % p.head_dim;
        const uint64_t tok = p.start + t;
        const int32_t page = p.table[tok / p.page_tokens];
        const size_t src =
            (((size_t)h * p.num_pages + page) * p.page_tokens + tok % p.page_tokens) * p.head_dim + d;
        p.keys[i] = bf16_to_f32(p.k_pages[src]);
        p.values[i] = bf16_to_f32(p.v_pages[src]);
    }
}

uint32_t grid_for(uint64_t work, uint32_t threads) {
    const uint64_t blocks = (work + threads - 1) / threads;
    return (uint32_t)(blocks < 65536 ? (blocks == 0 ? 1 : blocks) : 65536);
}

}  // namespace

hipError_t launch_page_table_set(hipStream_t s, int32_t *table, const uint32_t *idx,
                                 const int32_t *val, int n) {
    for (int base = 0; base < n; base += kTableBatch) {
        TableUpdate u;
        u.table = table;
        u.n = (n - base) < kTableBatch ? (n - base) : kTableBatch;
        for (int i = 0; i < u.n; ++i) {
            u.idx[i] = idx[base + i];
            u.val[i] = val[base + i];
        }
        SR_LAUNCH("page_table_set_kernel", page_table_set_kernel, dim3(1), dim3(256), 0, s, u);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_kv_scatter(hipStream_t s, const safetyraise_kernel_kv_pool *pool, uint32_t slot,
                             uint64_t start, uint64_t tokens, const void *keys, const void *values,
                             bool bf16_in, uint32_t *err_word) {
    if (tokens == 0) return hipSuccess;
    ScatterParams p;
    p.k_pages = pool->k_pages;
    p.v_pages = pool->v_pages;
    p.table = pool->d_page_table + (size_t)slot * pool->pages_per_seq;
    p.keys = keys;
    p.values = values;
    p.err_word = err_word;
    p.start = start;
    p.tokens = tokens;
    p.num_pages = pool->num_pages;
    p.kv_heads = pool->kv_heads;
    p.head_dim = pool->head_dim;
    p.page_tokens = pool->page_tokens;
    p.bf16_in = bf16_in ? 1 : 0;
    // (the callers pass 16-byte aligned rows: kv_append checks device
    // pointers, host inputs are staged at 256-byte offsets)
    if (pool->head_dim % 8 == 0) {
        const uint64_t work = tokens * pool->kv_heads * (pool->head_dim / 8);
        SR_LAUNCH("kv_scatter_kernel", kv_scatter_kernel, dim3(grid_for(work, 256)), dim3(256), 0,
                  s, p);
    } else {
        const uint64_t work = tokens * pool->kv_heads * pool->head_dim;
        SR_LAUNCH("kv_scatter_elem_kernel", kv_scatter_elem_kernel, dim3(grid_for(work, 256)),
                  dim3(256), 0, s, p);
    }
    return hipGetLastError();
}

hipError_t launch_kv_gather(hipStream_t s, const safetyraise_kernel_kv_pool *pool, uint32_t slot,
                            uint64_t start, uint64_t tokens, float *keys, float *values) {
    if (tokens == 0) return hipSuccess;
    GatherParams p;
    p.k_pages = pool->k_pages;
    p.v_pages = pool->v_pages;
    p.table = pool->d_page_table + (size_t)slot * pool->pages_per_seq;
    p.keys = keys;
    p.values = values;
    p.start = start;
    p.tokens = tokens;
    p.num_pages = pool->num_pages;
    p.kv_heads = pool->kv_heads;
    p.head_dim = pool->head_dim;
    p.page_tokens = pool->page_tokens;
    const uint64_t work = tokens * pool->kv_heads * pool->head_dim;
    SR_LAUNCH("kv_gather_kernel", kv_gather_kernel, dim3(grid_for(work, 256)), dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_page_copy(hipStream_t s, const safetyraise_kernel_kv_pool *pool, int32_t dst,
                            int32_t src) {
    // one PT x D block per head, the heads head_stride() elements apart
    const size_t width = pool->head_page_elems() * sizeof(uint16_t);
    const size_t pitch = pool->head_stride() * sizeof(uint16_t);
    const size_t d_off = (size_t)dst * pool->head_page_elems();
    const size_t s_off = (size_t)src * pool->head_page_elems();
    hipError_t e = hipMemcpy2DAsync(pool->k_pages + d_off, pitch, pool->k_pages + s_off, pitch,
                                    width, pool->kv_heads, hipMemcpyDeviceToDevice, s);
    if (e != hipSuccess) return e;
    return hipMemcpy2DAsync(pool->v_pages + d_off, pitch, pool->v_pages + s_off, pitch, width,
                            pool->kv_heads, hipMemcpyDeviceToDevice, s);
}

}  // namespace sr
