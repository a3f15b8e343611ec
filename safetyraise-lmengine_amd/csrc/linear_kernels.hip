// ABI v1 linear on the matrix cores: y[M][N] = x[M][K] . W[N][K]^T with f32
// inputs and outputs and an f32, f16 or bf16 weight that stays on the device
// (native/cpu/safetyraise_cpu.c:203-239 is the reference: an f32 sum over the
// columns of each weight row, the weight widened exactly to f32).
//
// The weight is widened exactly here too and the products run on
// v_mfma_f32_16x16x4f32, so every product is an f32 product and only the
// order of the sum differs from the reference (f32 tolerance, not bf16).
//
// Work split.  A workgroup owns 16 rows x 16 outputs and a contiguous range
// of K; its four waves take quarters of that range and meet in LDS.
// Decode-sized calls (M <= 16) thus stream every weight row once, which is
// the HBM-bound regime the ABI's projections live in; each k-step loads 16
// bytes of x and 8 weight elements per lane and feeds 8 MFMAs.  A call with
// fewer tiles than kLinWgPerCu workgroups per CU splits K over up to
// kLinMaxSplits workgroups per tile (grid z): those write partial sums and
// a second kernel adds them in split order, so results do not depend on
// timing.
//
// Operand order.  For MFMA t of a 32-wide k block, lane (r = lane % 16,
// g = lane / 16) feeds A = x[row r][k0 + 8g + t] and B = W[output r][same k]:
// the eight MFMAs cover the block's 32 k values with each lane reading 8
// consecutive ones (any order of k gives the same sum; A and B share it), so
// the four lanes of a row read 128 contiguous bytes of x and 64 of a bf16
// weight row per block.  The accumulator then holds y[row 4g + i][output r]
// in element i.

#include <algorithm>

#include "sr_internal.hpp"
#include "sr_device.hpp"

namespace sr {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kLinTile = 16;   // rows and outputs per workgroup
constexpr int kLinWaves = 4;   // waves splitting K
constexpr uint32_t kLinWgPerCu = 1;    // workgroups per CU a call aims for
constexpr uint32_t kLinMaxSplits = 8;  // K splits per tile at most
constexpr uint32_t kLinBlock = 32;      // k per block (8 MFMAs)
constexpr uint32_t kLinMinSplitK = 512;  // K per split at least (4 blocks per wave)

template <int DT>
__device__ __forceinline__ float widen(const void *w, size_t i) {
    if constexpr (DT == SAFETYRAISE_KERNEL_DTYPE_F32) {
        return ((const float *)w)[i];
    } else if constexpr (DT == SAFETYRAISE_KERNEL_DTYPE_F16) {
        return (float)((const _Float16 *)w)[i];
    } else {
        return __uint_as_float((uint32_t)((const uint16_t *)w)[i] << 16);
    }
}

// Elements k .. k+7 of a row starting at element `row`, those from `lim` on
// replaced by 0.  The reads themselves are clamped into the row (K >= 1;
// kVec: K a multiple of 8, so k and lim are too), and the zeros are selected
// after the load: a load behind a branch would make later waits wait for
// every load in flight.  kVec: the row start is 32-byte aligned for f32
// (16-byte for 16-bit weights).
template <int DT, bool kVec>
__device__ __forceinline__ f32x8 load8(const void *base, size_t row, uint32_t k, uint32_t K,
                                       uint32_t lim) {
    f32x8 v;
    if constexpr (kVec) {
        const size_t i = row + min(k, K - 8);
        if constexpr (DT == SAFETYRAISE_KERNEL_DTYPE_F32) {
            const f32x4 lo = *(const f32x4 *)((const float *)base + i);
            const f32x4 hi = *(const f32x4 *)((const float *)base + i + 4);
            v = f32x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        } else if constexpr (DT == SAFETYRAISE_KERNEL_DTYPE_F16) {
            v = __builtin_convertvector(*(const f16x8 *)((const _Float16 *)base + i), f32x8);
        } else {
            const uint4 u = *(const uint4 *)((const uint16_t *)base + i);
            v = f32x8{__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                      __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u),
                      __uint_as_float(u.z << 16), __uint_as_float(u.z & 0xffff0000u),
                      __uint_as_float(u.w << 16), __uint_as_float(u.w & 0xffff0000u)};
        }
        const bool live = k < lim;
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = live ? v[j] : 0.0f;
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float e = widen<DT>(base, row + min(k + j, K - 1));
            v[j] = k + j < lim ? e : 0.0f;
        }
    }
    return v;
}

// y: the output, or (grid z > 1) partial sums [grid z][M][N].  kGroup: k
// blocks per register set (4; 2 for calls with many workgroups per CU, which
// then hold more waves per SIMD).
template <int DT, bool kVec, int kGroup>
__global__ __launch_bounds__(64 * kLinWaves) void linear_kernel(const float *x, const void *w,
                                                                 float *y, uint32_t M, uint32_t N,
                                                                 uint32_t K) {
    __shared__ f32x4 red[kLinWaves - 1][64];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const uint32_t r = lane & 15, g = lane >> 4;
    const uint32_t n0 = blockIdx.x * kLinTile, m0 = blockIdx.y * kLinTile;
    // rows past M / N read the last row and their results are not stored
    if (K == 0) {  // empty sums (uniform): zeros
        if (wave == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t m = m0 + 4 * g + i, n = n0 + r;
                if (m < M && n < N) y[(size_t)m * N + n] = 0.0f;
            }
        }
        return;
    }
    const size_t xrow = (size_t)min(m0 + r, M - 1) * K;
    const size_t wrow = (size_t)min(n0 + r, N - 1) * K;
    y += (size_t)blockIdx.z * M * N;
    const uint32_t nblk = (K + kLinBlock - 1) / kLinBlock;
    const uint32_t s0 = (uint32_t)((uint64_t)nblk * blockIdx.z / gridDim.z);
    const uint32_t s1 = (uint32_t)((uint64_t)nblk * (blockIdx.z + 1) / gridDim.z);
    const uint32_t b0 = s0 + (uint32_t)((uint64_t)(s1 - s0) * wave / kLinWaves);
    const uint32_t b1 = s0 + (uint32_t)((uint64_t)(s1 - s0) * (wave + 1) / kLinWaves);
    // this wave's k range ends at kend: loads past it read zeros, so a group
    // that runs past the range adds nothing (and no block is counted twice)
    const uint32_t kend = min(kLinBlock * b1, K);
    // groups of kGroup blocks in two register sets: while the MFMAs of one
    // set run, the loads of the other are in flight (the sets alternate
    // explicitly, so the compiler cannot merge them into one and wait for
    // loads it has just issued)
    f32x8 xa[kGroup], wa[kGroup], xb[kGroup], wb[kGroup];
    auto load_group = [&](uint32_t b, f32x8 (&xv)[kGroup], f32x8 (&wv)[kGroup])
                          __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < kGroup; ++j) {
            const uint32_t k = kLinBlock * (b + j) + 8 * g;
            xv[j] = load8<SAFETYRAISE_KERNEL_DTYPE_F32, kVec>(x, xrow, k, K, kend);
            wv[j] = load8<DT, kVec>(w, wrow, k, K, kend);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // four accumulation chains (MFMA t of a block feeds chain t % 4), so
    // consecutive MFMAs do not wait for each other's results
    constexpr int kChains = 4;
    f32x4 acc4[kChains];
#pragma unroll
    for (int c = 0; c < kChains; ++c) acc4[c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    auto mfma_group = [&](const f32x8 (&xv)[kGroup], const f32x8 (&wv)[kGroup])
                          __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < kGroup; ++j) {
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                f32x4 &a = acc4[t % kChains];
                a = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[j][t], wv[j][t], a, 0, 0, 0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // groups past the range load zeros (clamped reads) and add nothing
    load_group(b0, xa, wa);
    for (uint32_t b = b0; b < b1; b += 2 * kGroup) {
        load_group(b + kGroup, xb, wb);
        mfma_group(xa, wa);
        load_group(b + 2 * kGroup, xa, wa);
        mfma_group(xb, wb);
    }
    const f32x4 acc = (acc4[0] + acc4[1]) + (acc4[2] + acc4[3]);
    if (wave > 0) red[wave - 1][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    f32x4 sum = acc;
#pragma unroll
    for (int j = 0; j < kLinWaves - 1; ++j) sum += red[j][lane];
    const uint32_t n = n0 + r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t m = m0 + 4 * g + i;
        if (m < M && n < N) y[(size_t)m * N + n] = sum[i];
    }
}

// y[i] = sum over z < splits of part[z][i], added in z order (splits <=
// kLinMaxSplits; all loads are issued before the first add)
__global__ __launch_bounds__(256) void linear_split_sum_kernel(const float *part, float *y,
                                                               uint32_t count, uint32_t splits) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= count) return;
    float v[kLinMaxSplits];
#pragma unroll
    for (uint32_t z = 0; z < kLinMaxSplits; ++z) v[z] = part[(size_t)min(z, splits - 1) * count + i];
    float s = v[0];
#pragma unroll
    for (uint32_t z = 1; z < kLinMaxSplits; ++z) s = z < splits ? s + v[z] : s;
    y[i] = s;
}

template <int DT, int kGroup>
void launch_dt(hipStream_t stream, const float *x, const void *w, float *y, uint32_t M, uint32_t N,
               uint32_t K, uint32_t splits) {
    const dim3 grid((N + kLinTile - 1) / kLinTile, (M + kLinTile - 1) / kLinTile, splits);
    // 16-byte loads need 16-byte aligned rows: K a multiple of 8 and x itself
    // aligned (a device caller may pass a view that starts mid-vector; the
    // weight is the plugin's own allocation)
    if ((K & 7u) == 0 && ((uintptr_t)x & 15u) == 0) {
        SR_LAUNCH("linear_kernel", (linear_kernel<DT, true, kGroup>), grid, dim3(64 * kLinWaves), 0,
                  stream, x, w, y, M, N, K);
    } else {
        SR_LAUNCH("linear_kernel", (linear_kernel<DT, false, kGroup>), grid, dim3(64 * kLinWaves), 0,
                  stream, x, w, y, M, N, K);
    }
}

template <int DT>
void launch_dt_groups(hipStream_t stream, const float *x, const void *w, float *y, uint32_t M,
                      uint32_t N, uint32_t K, uint32_t splits, int num_cus) {
    const uint64_t wgs = (uint64_t)((N + kLinTile - 1) / kLinTile) * ((M + kLinTile - 1) / kLinTile) *
                         splits;
    if (wgs >= 2 * (uint64_t)(num_cus > 0 ? num_cus : 1)) {
        launch_dt<DT, 2>(stream, x, w, y, M, N, K, splits);
    } else {
        launch_dt<DT, 4>(stream, x, w, y, M, N, K, splits);
    }
}

}  // namespace

uint32_t linear_splits(uint32_t M, uint32_t N, uint32_t K, int num_cus) {
    const uint64_t tiles = (uint64_t)((N + kLinTile - 1) / kLinTile) * ((M + kLinTile - 1) / kLinTile);
    const uint64_t target = (uint64_t)kLinWgPerCu * (uint64_t)(num_cus > 0 ? num_cus : 1);
    if (tiles == 0 || tiles >= target) return 1;
    uint64_t s = (target + tiles - 1) / tiles;
    s = std::min<uint64_t>(s, K / kLinMinSplitK);
    s = std::min<uint64_t>(s, kLinMaxSplits);
    return s < 1 ? 1u : (uint32_t)s;
}

size_t linear_scratch_bytes(uint32_t M, uint32_t N, uint32_t K, int num_cus) {
    const uint32_t s = linear_splits(M, N, K, num_cus);
    return s > 1 ? (size_t)s * M * N * sizeof(float) : 0;
}

hipError_t launch_linear(hipStream_t stream, const float *x, const void *w, uint32_t dtype,
                         float *y, uint32_t M, uint32_t N, uint32_t K, float *scratch,
                         int num_cus) {
    if (M == 0 || N == 0) return hipSuccess;
    constexpr uint32_t kMaxRows = 65535u * kLinTile;  // grid y limit of one launch
    if (M > kMaxRows) {
        // equal blocks of rows, one launch each: every block has at least
        // kMaxRows / 2 rows, so enough tiles that none splits K and the
        // scratch (sized 0 for such M) is not used
        const uint32_t nb = (M + kMaxRows - 1) / kMaxRows;
        const uint32_t per = ((M + nb - 1) / nb + kLinTile - 1) / kLinTile * kLinTile;
        for (uint32_t r0 = 0; r0 < M; r0 += per) {
            const uint32_t m = std::min(per, M - r0);
            const hipError_t e = launch_linear(stream, x + (size_t)r0 * K, w, dtype,
                                               y + (size_t)r0 * N, m, N, K, nullptr, num_cus);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    const uint32_t splits = linear_splits(M, N, K, num_cus);
    if (splits > 1 && scratch == nullptr) return hipErrorInvalidValue;
    float *dst = splits > 1 ? scratch : y;
    switch (dtype) {
        case SAFETYRAISE_KERNEL_DTYPE_F32:
            launch_dt_groups<SAFETYRAISE_KERNEL_DTYPE_F32>(stream, x, w, dst, M, N, K, splits, num_cus);
            break;
        case SAFETYRAISE_KERNEL_DTYPE_F16:
            launch_dt_groups<SAFETYRAISE_KERNEL_DTYPE_F16>(stream, x, w, dst, M, N, K, splits, num_cus);
            break;
        case SAFETYRAISE_KERNEL_DTYPE_BF16:
            launch_dt_groups<SAFETYRAISE_KERNEL_DTYPE_BF16>(stream, x, w, dst, M, N, K, splits, num_cus);
            break;
        default:
            return hipErrorInvalidValue;
    }
    if (splits > 1) {
        // splits > 1 only when tiles < kLinWgPerCu * CUs, so M * N is small
        const uint32_t count = M * N;
        SR_LAUNCH("linear_split_sum_kernel", linear_split_sum_kernel, dim3((count + 255) / 256),
                  dim3(256), 0, stream, scratch, y, count, splits);
    }
    return hipGetLastError();
}

}  // namespace sr
