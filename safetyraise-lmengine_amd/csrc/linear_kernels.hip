// ABI v1 linear on the matrix cores: y[M][N] = x[M][K] . W[N][K]^T with f32
// inputs and outputs and an f32, f16 or bf16 weight that stays on the device
// (native/cpu/safetyraise_cpu.c:203-239 is the reference: an f32 sum over the
// columns of each weight row, the weight widened exactly to f32).
//
// Every product is an exact f32 product and only the order of the sum differs
// from the reference (f32 tolerance, not bf16): f32 and f16 weights are
// widened exactly and run on v_mfma_f32_16x16x4f32; for bf16 weights x is
// split exactly into three bf16 parts (split3) that each multiply the stored
// weight on v_mfma_f32_16x16x32_bf16, 3 MFMAs per 32-k block and tile instead
// of 8 at a quarter of the rate.
//
// Weight layout.  F32 and F16 weights stay row-major as given.  A BF16 weight
// is repacked once, when its handle is created (linear_pack_bf16), into
// 1 KB tiles: for output tile t (16 rows) and k block b (32 columns) the 512
// elements from (t * nblk + b) * 512 on hold, at 8 (16 g + r), W[16 t + r]
// [32 b + 8 g .. + 8], with zeros past N and K.  Lane (r, g) then loads its
// operand as 16 contiguous bytes, one load instruction reads 1 KB of
// contiguous memory instead of 64 bytes of 16 rows, and every call reads
// aligned whole blocks whatever its shape.
//
// Work split.  A workgroup owns 16 rows x 16 T outputs (T tiles per wave)
// and a contiguous range of K; its W waves take equal parts of that range
// and meet in LDS.  Decode-sized calls (M <= 16) stream every weight row
// once, the HBM-bound regime the ABI's projections live in; each k block
// loads 32 bytes of x per lane, used by T tiles, and 8 weight elements per
// tile.  x is the larger share of the bytes a lane loads, so T > 1 keeps the
// load pipeline (texture address unit) from being the limit.  A call whose
// tiles do not cover the CUs splits K over up to kLinMaxSplits workgroups per
// tile (grid z): those write partial sums and a second kernel adds them in
// split order, so results do not depend on timing (linear_plan chooses).
//
// Operand order.  For a 32-wide k block, lane (r = lane % 16, g = lane / 16)
// holds x[row r][k0 + 8g .. + 8] and W[output r][same k] (any order of k
// gives the same sum; A and B share it): the f32 MFMA t takes element t of
// each, the bf16 MFMA all eight.  The four lanes of a row read 128
// contiguous bytes of x per block.  The accumulator then holds
// y[row 4g + i][output r] in element i.

#include <algorithm>
#include <type_traits>

#include "sr_internal.hpp"
#include "sr_device.hpp"

namespace sr {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kLinTile = 16;   // rows and outputs per workgroup
constexpr int kLinWaves = 4;   // waves splitting K
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

// Elements i .. i+7 (16-byte aligned for 16-bit types, 32-byte for f32),
// widened exactly to f32.
template <int DT>
__device__ __forceinline__ f32x8 load8_at(const void *base, size_t i) {
    if constexpr (DT == SAFETYRAISE_KERNEL_DTYPE_F32) {
        const f32x4 lo = *(const f32x4 *)((const float *)base + i);
        const f32x4 hi = *(const f32x4 *)((const float *)base + i + 4);
        return f32x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    } else if constexpr (DT == SAFETYRAISE_KERNEL_DTYPE_F16) {
        return __builtin_convertvector(*(const f16x8 *)((const _Float16 *)base + i), f32x8);
    } else {
        const uint4 u = *(const uint4 *)((const uint16_t *)base + i);
        return f32x8{__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                     __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u),
                     __uint_as_float(u.z << 16), __uint_as_float(u.z & 0xffff0000u),
                     __uint_as_float(u.w << 16), __uint_as_float(u.w & 0xffff0000u)};
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
        v = load8_at<DT>(base, row + min(k, K - 8));
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

// bf16's largest finite value, 0x7F7F
constexpr float kBf16Max = 3.38953139e38f;

// x as hi + mid + lo in bf16, each the round-to-nearest-even of what the
// parts before it leave: exact for every finite x with |x| >= 2^-110 (below,
// bits under 2^-133 are lost).  hi is taken from x clamped to bf16's finite
// range (one v_med3_f32), so a finite x above bf16's largest value still
// splits exactly (x - hi is then exact and below 2^121).  With a bf16 weight
// the three products are exact f32 products and their sum is w x up to f32
// rounding.  An infinite x gives a NaN part, so a product with a non-finite
// input is non-finite as the reference's is (the ABI call rejects such
// inputs before any kernel runs, as native/cpu/safetyraise_cpu.c:221-226 does).
__device__ __forceinline__ void split3(const f32x8 &x, bf16x8 &hi, bf16x8 &mid, bf16x8 &lo) {
    f32x8 xc;
#pragma unroll
    for (int j = 0; j < 8; ++j) xc[j] = __builtin_amdgcn_fmed3f(x[j], -kBf16Max, kBf16Max);
    hi = __builtin_convertvector(xc, bf16x8);
    const f32x8 r1 = x - __builtin_convertvector(hi, f32x8);
    mid = __builtin_convertvector(r1, bf16x8);
    const f32x8 r2 = r1 - __builtin_convertvector(mid, f32x8);
    lo = __builtin_convertvector(r2, bf16x8);
}

// y: the output, or (grid z > 1) partial sums [grid z][M][N].  T: output tiles per wave (the workgroup owns 16 T
// outputs; each x fragment a lane loads feeds T MFMAs, so x is read once
// per 16 T outputs).  W: waves per workgroup, splitting its k range.  kGroup: k
// blocks per register set (4; 2 for calls with many workgroups per CU, which
// then hold more waves per SIMD).  kExact: every wave's k range is a whole
// number of pairs of groups of whole blocks (the host checks), so no load
// reaches past it, nothing is masked and the last pair prefetches nothing.
template <int DT, bool kVec, int T, int W, int kGroup, bool kExact>
__global__ __launch_bounds__(64 * W) void linear_kernel(const float *x, const void *w, float *y,
                                                        uint32_t M, uint32_t N, uint32_t K) {
    static_assert(!kExact || kVec, "exact ranges use the vector loads");
    __shared__ f32x4 red[W - 1][T][64];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const uint32_t r = lane & 15, g = lane >> 4;
    const uint32_t n0 = blockIdx.x * kLinTile * T, m0 = blockIdx.y * kLinTile;
    // rows past M / N read the last row and their results are not stored
    if (K == 0) {  // empty sums (uniform): zeros
        if (wave == 0) {
#pragma unroll
            for (int u = 0; u < T; ++u)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t m = m0 + 4 * g + i, n = n0 + kLinTile * u + r;
                    if (m < M && n < N) y[(size_t)m * N + n] = 0.0f;
                }
        }
        return;
    }
    // kTiled (bf16 weights): the weight is in 1 KB tiles; x is split in
    // three bf16 parts, so a 32-k block takes 3 v_mfma_f32_16x16x32_bf16 per
    // tile instead of 8 v_mfma_f32_16x16x4f32
    constexpr bool kTiled = DT == SAFETYRAISE_KERNEL_DTYPE_BF16;
    const uint32_t nblk = (K + kLinBlock - 1) / kLinBlock;
    const size_t xrow = (size_t)min(m0 + r, M - 1) * K;
    // row-major weights: the row of output r of each tile; tiled: this
    // lane's 16 bytes in block 0 of each tile (tiles past N read the last)
    size_t wrow[T];
#pragma unroll
    for (int u = 0; u < T; ++u) {
        if constexpr (kTiled) {
            const uint32_t tile = min(n0 / kLinTile + u, (N - 1) / kLinTile);
            wrow[u] = (size_t)tile * nblk * 512 + (size_t)lane * 8;
        } else {
            wrow[u] = (size_t)min(n0 + kLinTile * u + r, N - 1) * K;
        }
    }
    y += (size_t)blockIdx.z * M * N;
    const uint32_t s0 = (uint32_t)((uint64_t)nblk * blockIdx.z / gridDim.z);
    const uint32_t s1 = (uint32_t)((uint64_t)nblk * (blockIdx.z + 1) / gridDim.z);
    const uint32_t b0 = s0 + (uint32_t)((uint64_t)(s1 - s0) * wave / W);
    const uint32_t b1 = s0 + (uint32_t)((uint64_t)(s1 - s0) * (wave + 1) / W);
    // this wave's k range ends at kend: loads past it read zeros, so a group
    // that runs past the range adds nothing (and no block is counted twice)
    const uint32_t kend = min(kLinBlock * b1, K);
    // groups of kGroup blocks in two register sets: while the MFMAs of one
    // set run, the loads of the other are in flight (the sets alternate
    // explicitly, so the compiler cannot merge them into one and wait for
    // loads it has just issued)
    using WV = std::conditional_t<kTiled, bf16x8, f32x8>;
    f32x8 xa[kGroup], xb[kGroup];
    WV wa[kGroup][T], wb[kGroup][T];
    auto load_group = [&](uint32_t b, f32x8 (&xv)[kGroup], WV (&wv)[kGroup][T])
                          __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < kGroup; ++j) {
            const uint32_t k = kLinBlock * (b + j) + 8 * g;
            if constexpr (kExact) {
                xv[j] = load8_at<SAFETYRAISE_KERNEL_DTYPE_F32>(x, xrow + k);
            } else {
                xv[j] = load8<SAFETYRAISE_KERNEL_DTYPE_F32, kVec>(x, xrow, k, K, kend);
            }
#pragma unroll
            for (int u = 0; u < T; ++u) {
                if constexpr (kTiled && kExact) {
                    wv[j][u] = *(const bf16x8 *)((const uint16_t *)w + wrow[u] +
                                                 (size_t)(b + j) * 512);
                } else if constexpr (kTiled) {
                    // blocks past this wave's range: read the last block of
                    // the tile, add zeros (selected after the load)
                    uint4 v = *(const uint4 *)((const uint16_t *)w + wrow[u] +
                                               (size_t)min(b + j, nblk - 1) * 512);
                    if (!(b + j < b1)) v = uint4{0, 0, 0, 0};
                    wv[j][u] = __builtin_bit_cast(bf16x8, v);
                } else if constexpr (kExact) {
                    wv[j][u] = load8_at<DT>(w, wrow[u] + k);
                } else {
                    wv[j][u] = load8<DT, kVec>(w, wrow[u], k, K, kend);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // kChains accumulation chains per tile (MFMA t of a block feeds chain
    // t % kChains, or one chain per part of x), so consecutive MFMAs do not
    // wait for each other's results
    constexpr int kChains = kTiled ? 3 : (T == 1 ? 4 : 2);
    f32x4 acc4[T][kChains];
#pragma unroll
    for (int u = 0; u < T; ++u)
#pragma unroll
        for (int c = 0; c < kChains; ++c) acc4[u][c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    auto mfma_group = [&](const f32x8 (&xv)[kGroup], const WV (&wv)[kGroup][T])
                          __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < kGroup; ++j) {
            if constexpr (kTiled) {
                bf16x8 part[3];
                split3(xv[j], part[0], part[1], part[2]);
#pragma unroll
                for (int c = 0; c < 3; ++c)
#pragma unroll
                    for (int u = 0; u < T; ++u)
                        acc4[u][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(part[c], wv[j][u],
                                                                             acc4[u][c], 0, 0, 0);
            } else {
#pragma unroll
                for (int t = 0; t < 8; ++t) {
#pragma unroll
                    for (int u = 0; u < T; ++u) {
                        f32x4 &a = acc4[u][t % kChains];
                        a = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[j][t], wv[j][u][t], a, 0, 0, 0);
                    }
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    load_group(b0, xa, wa);
    if constexpr (kExact) {
        // b1 - b0 is a positive multiple of 2 kGroup: the last pair loads
        // nothing past b1
        uint32_t b = b0;
        for (; b + 2 * kGroup < b1; b += 2 * kGroup) {
            load_group(b + kGroup, xb, wb);
            mfma_group(xa, wa);
            load_group(b + 2 * kGroup, xa, wa);
            mfma_group(xb, wb);
        }
        load_group(b + kGroup, xb, wb);
        mfma_group(xa, wa);
        mfma_group(xb, wb);
    } else {
        // groups past the range load zeros (clamped reads) and add nothing
        for (uint32_t b = b0; b < b1; b += 2 * kGroup) {
            load_group(b + kGroup, xb, wb);
            mfma_group(xa, wa);
            load_group(b + 2 * kGroup, xa, wa);
            mfma_group(xb, wb);
        }
    }
    // the chains summed last to first (with split x: lo + mid, then hi)
    f32x4 acc[T];
#pragma unroll
    for (int u = 0; u < T; ++u) {
        acc[u] = acc4[u][kChains - 1];
#pragma unroll
        for (int c = kChains - 2; c >= 0; --c) acc[u] += acc4[u][c];
    }
    if (wave > 0) {
#pragma unroll
        for (int u = 0; u < T; ++u) red[wave - 1][u][lane] = acc[u];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int u = 0; u < T; ++u) {
        f32x4 sum = acc[u];
#pragma unroll
        for (int j = 0; j < W - 1; ++j) sum += red[j][u][lane];
        const uint32_t n = n0 + kLinTile * u + r;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t m = m0 + 4 * g + i;
            if (m < M && n < N) y[(size_t)m * N + n] = sum[i];
        }
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

// ---------------------------------------------------------------------------
// Calls with many rows (prefill chunks) on bf16 weights: a tiled product.
// linear_split_x_kernel first writes x once as its three bf16 parts (split3)
// in MFMA lane order: for row tile t (16 rows), k block b (32 columns) and
// part c, the 1 KB at ((t * nblk + b) * 3 + c) KB holds, at lane 16 g + r,
// x[16 t + r][32 b + 8 g .. + 8].  linear_gemm_kernel then owns 128 rows x
// 128 outputs per workgroup; its 8 waves are 4 (rows) x 2 (outputs), each
// computing 32 rows x 64 outputs (2 x 4 tiles of 16 x 16).  Per stage of 64 k
// (two 32-k blocks) the workgroup copies its 48 KB of split x straight from
// memory into LDS (global_load_lds: no registers, no VALU), double-buffered;
// a wave reads its row tiles' parts with ds_read_b128 and its 4 weight tiles
// straight from the tile layout (16 bytes per lane, prefetched one stage
// ahead).  So x is read once per 128 outputs and the weight once per 128
// rows, and the loop is loads and MFMAs only.  Two accumulation chains per
// tile: the hi part's products, and the mid and lo parts' (three chains of 8
// tiles would not fit the registers of two waves per SIMD).  Requires K % 64
// == 0; rows past M and tiles past N read clamped copies whose results are
// not stored.
// ---------------------------------------------------------------------------
constexpr int kGemmWM = 4, kGemmWN = 2;  // waves over rows, over outputs
constexpr int kGemmRT = 2, kGemmCT = 4;  // 16 x 16 tiles per wave: rows, outputs
constexpr int kGemmBM = 16 * kGemmRT * kGemmWM;  // 128 rows per workgroup
constexpr int kGemmBN = 16 * kGemmCT * kGemmWN;  // 128 outputs per workgroup
constexpr int kGemmKB = 2;                       // 32-k blocks per stage
constexpr uint32_t kGemmK = kGemmKB * kLinBlock;  // 64 k per stage
constexpr uint32_t kGemmMinRows = 64;             // rows from which calls take this kernel
// one stage of split x in LDS: [k block][part][row tile][lane] x 16 bytes
constexpr int kGemmStageBytes = kGemmKB * 3 * (kGemmBM / 16) * 64 * 16;
constexpr int kGemmStageBlocks = kGemmStageBytes / 1024;  // 1 KB blocks per stage (48)

// Thread c: lane c % 64 of (row tile, k block) c / 64, its 8 values split.
template <bool kVec>
__global__ __launch_bounds__(256) void linear_split_x_kernel(const float *x, uint16_t *xs,
                                                            uint32_t M, uint32_t K,
                                                            uint64_t chunks) {
    const uint64_t c = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= chunks) return;
    const uint32_t nblk = K / kLinBlock;
    const uint32_t lane = (uint32_t)(c & 63);
    const uint64_t tb = c >> 6;
    const uint32_t t = (uint32_t)(tb / nblk), b = (uint32_t)(tb % nblk);
    const uint32_t row = min(kLinTile * t + (lane & 15), M - 1);
    const size_t off = (size_t)row * K + kLinBlock * b + 8 * (lane >> 4);
    f32x8 v;
    if constexpr (kVec) {
        v = load8_at<SAFETYRAISE_KERNEL_DTYPE_F32>(x, off);
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = x[off + j];
    }
    bf16x8 part[3];
    split3(v, part[0], part[1], part[2]);
    typedef uint32_t u32x4s __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int p = 0; p < 3; ++p) {
        *(u32x4s *)(xs + ((tb * 3 + p) * 64 + lane) * 8) = __builtin_bit_cast(u32x4s, part[p]);
    }
}

__global__ __launch_bounds__(512) void linear_gemm_kernel(const uint16_t *xs, const void *w,
                                                         float *y, uint32_t M, uint32_t N,
                                                         uint32_t K) {
    extern __shared__ __align__(16) unsigned char gemm_lds[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave % kGemmWM, wn = wave / kGemmWM;
    const uint32_t m0 = blockIdx.y * kGemmBM, n0 = blockIdx.x * kGemmBN;
    const uint32_t nblk = K / kLinBlock;
    const uint32_t stages = K / kGemmK;
    const uint32_t last_tile = (N - 1) / kLinTile;
    const uint32_t last_row_tile = (M - 1) / kLinTile;

    // the split-x blocks this wave copies per stage: blocks q = 6 wave .. +6
    // of the stage's 48, block q = (k block, part, row tile) in LDS order
    const uint16_t *xsrc[kGemmStageBlocks / 8];
    uint32_t xdst[kGemmStageBlocks / 8];
#pragma unroll
    for (int i = 0; i < kGemmStageBlocks / 8; ++i) {
        const uint32_t q = (uint32_t)wave * (kGemmStageBlocks / 8) + i;
        const uint32_t rt = q % (kGemmBM / 16), part = (q / (kGemmBM / 16)) % 3,
                       kb = q / (3 * (kGemmBM / 16));
        const uint32_t t = min(m0 / kLinTile + rt, last_row_tile);
        xsrc[i] = xs + (((size_t)t * nblk + kb) * 3 + part) * 512 + (size_t)lane * 8;
        xdst[i] = q * 1024;
    }
    // this wave's weight tiles: 16 bytes of block 0 per lane (tiles past N
    // read the last one)
    const uint16_t *wt[kGemmCT];
#pragma unroll
    for (int j = 0; j < kGemmCT; ++j) {
        const uint32_t tile = min(n0 / kLinTile + kGemmCT * wn + j, last_tile);
        wt[j] = (const uint16_t *)w + (size_t)tile * nblk * 512 + (size_t)lane * 8;
    }
    typedef uint32_t u32x4g __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) unsigned char lds_byte;
    lds_byte *lds = (lds_byte *)gemm_lds;
    auto copy_x = [&](uint32_t s, uint32_t buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < kGemmStageBlocks / 8; ++i) {
            // a stage's two k blocks: block s of the call's stages is k
            // blocks 2 s, 2 s + 1, i.e. (2 s) * 3 * 512 elements past block 0
            __builtin_amdgcn_global_load_lds(xsrc[i] + (size_t)s * kGemmKB * 3 * 512,
                                             lds + buf * kGemmStageBytes + xdst[i], 16, 0, 0);
        }
    };
    auto load_w = [&](uint32_t s, bf16x8 (&wv)[kGemmKB][kGemmCT]) __attribute__((always_inline)) {
#pragma unroll
        for (int kb = 0; kb < kGemmKB; ++kb)
#pragma unroll
            for (int j = 0; j < kGemmCT; ++j)
                wv[kb][j] = *(const bf16x8 *)(wt[j] + (size_t)(kGemmKB * s + kb) * 512);
    };

    f32x4 acc[kGemmRT][kGemmCT][2];
#pragma unroll
    for (int i = 0; i < kGemmRT; ++i)
#pragma unroll
        for (int j = 0; j < kGemmCT; ++j)
#pragma unroll
            for (int c = 0; c < 2; ++c) acc[i][j][c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    bf16x8 wa[kGemmKB][kGemmCT], wb[kGemmKB][kGemmCT];
    copy_x(0, 0);
    load_w(0, wa);
    __syncthreads();
    auto compute = [&](uint32_t buf, const bf16x8 (&wv)[kGemmKB][kGemmCT]) __attribute__((always_inline)) {
#pragma unroll
        for (int kb = 0; kb < kGemmKB; ++kb) {
            bf16x8 a[kGemmRT][3];
#pragma unroll
            for (int i = 0; i < kGemmRT; ++i)
#pragma unroll
                for (int c = 0; c < 3; ++c) {
                    const uint32_t chunk = ((kb * 3 + c) * (kGemmBM / 16) + kGemmRT * wm + i) * 64 + lane;
                    a[i][c] = __builtin_bit_cast(
                        bf16x8, *(const __attribute__((address_space(3))) u32x4g *)(
                                    lds + buf * kGemmStageBytes + chunk * 16));
                }
#pragma unroll
            for (int c = 0; c < 3; ++c)
#pragma unroll
                for (int i = 0; i < kGemmRT; ++i)
#pragma unroll
                    for (int j = 0; j < kGemmCT; ++j) {
                        f32x4 &ac = acc[i][j][c == 0 ? 0 : 1];
                        ac = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i][c], wv[kb][j], ac, 0, 0, 0);
                    }
        }
    };
    // stages in pairs, so that the two weight register sets alternate by
    // name; the copy of stage s + 1 into the other buffer is in flight while
    // stage s computes, and the barrier after it waits for the copy
    uint32_t s = 0;
    for (; s + 2 <= stages; s += 2) {
        const bool more1 = s + 1 < stages;
        if (more1) {
            copy_x(s + 1, (s + 1) & 1);
            load_w(s + 1, wb);
        }
        compute(s & 1, wa);
        __syncthreads();
        const bool more2 = s + 2 < stages;
        if (more2) {
            copy_x(s + 2, s & 1);
            load_w(s + 2, wa);
        }
        compute((s + 1) & 1, wb);
        __syncthreads();
    }
    if (s < stages) compute(s & 1, wa);

    // the mid + lo chain, then hi; lane (r, g) holds y[row 4g + e][output
    // r] of each tile in element e
    const uint32_t r = lane & 15, g = lane >> 4;
#pragma unroll
    for (int i = 0; i < kGemmRT; ++i)
#pragma unroll
        for (int j = 0; j < kGemmCT; ++j) {
            const f32x4 sum = acc[i][j][1] + acc[i][j][0];
            const uint32_t n = n0 + kLinTile * (kGemmCT * wn + j) + r;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t m = m0 + kLinTile * (kGemmRT * wm + i) + 4 * g + e;
                if (m < M && n < N) y[(size_t)m * N + n] = sum[e];
            }
        }
}

// The form for calls with many outputs (at least kWideMinOutputs): 4 waves
// per 128 x 128 tile, each owning 64 rows x 64 outputs (4 x 4 tiles), two
// workgroups per CU.  Per 32-k block a wave reads 12 A fragments from LDS and
// 4 weight fragments from memory for 48 MFMAs: half the weight bytes per
// MFMA of linear_gemm_kernel's 32 x 64 wave tiles, and a 24 KB stage (one
// k block), so that two workgroups fit a CU and each one's barriers are
// covered by the other.  Measured on the Qwen3-8B layer at 2048 rows: 2.19
// ms per layer against 2.61 with linear_gemm_kernel for every call; 64 x 128
// wave tiles (256 accumulators, one workgroup per CU) measured 2.70 ms, the
// compiler moving accumulators between register files, and this form for
// the 1024-output k/v calls too 2.26 ms (half the CUs idle).
constexpr int kWideWM = 2, kWideWN = 2;           // waves over rows, over outputs
constexpr int kWideRT = 4, kWideCT = 4;           // 16 x 16 tiles per wave
constexpr int kWideBM = 16 * kWideRT * kWideWM;   // 128 rows per workgroup
constexpr int kWideBN = 16 * kWideCT * kWideWN;   // 128 outputs per workgroup
constexpr int kWideStageBytes = 3 * (kWideBM / 16) * 1024;  // [part][row tile] 1 KB blocks
constexpr int kWideStageBlocks = kWideStageBytes / 1024;    // 24
constexpr int kWideThreads = 64 * kWideWM * kWideWN;
constexpr uint32_t kWideMinOutputs = 2048;

__global__ __launch_bounds__(kWideThreads, 2) void linear_gemm_wide_kernel(const uint16_t *xs,
                                                                         const void *w, float *y,
                                                                         uint32_t M, uint32_t N,
                                                                         uint32_t K) {
    extern __shared__ __align__(16) unsigned char gemm_lds[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave % kWideWM, wn = wave / kWideWM;
    const uint32_t m0 = blockIdx.y * kWideBM, n0 = blockIdx.x * kWideBN;
    const uint32_t nblk = K / kLinBlock;
    const uint32_t last_tile = (N - 1) / kLinTile;
    const uint32_t last_row_tile = (M - 1) / kLinTile;

    // the split-x blocks this wave copies per stage: q = 6 wave .. + 6 of the
    // stage's 24, block q = (part, row tile) in LDS order
    constexpr int kCopies = kWideStageBlocks / (kWideThreads / 64);
    const uint16_t *xsrc[kCopies];
    uint32_t xdst[kCopies];
#pragma unroll
    for (int i = 0; i < kCopies; ++i) {
        const uint32_t q = (uint32_t)wave * kCopies + i;
        const uint32_t rt = q % (kWideBM / 16), part = q / (kWideBM / 16);
        const uint32_t t = min(m0 / kLinTile + rt, last_row_tile);
        xsrc[i] = xs + ((size_t)t * nblk * 3 + part) * 512 + (size_t)lane * 8;
        xdst[i] = q * 1024;
    }
    const uint16_t *wt[kWideCT];
#pragma unroll
    for (int j = 0; j < kWideCT; ++j) {
        const uint32_t tile = min(n0 / kLinTile + kWideCT * wn + j, last_tile);
        wt[j] = (const uint16_t *)w + (size_t)tile * nblk * 512 + (size_t)lane * 8;
    }
    typedef uint32_t u32x4g __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) unsigned char lds_byte;
    lds_byte *lds = (lds_byte *)gemm_lds;
    auto copy_x = [&](uint32_t s, uint32_t buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < kCopies; ++i) {
            // k block s is s * 3 * 512 elements past block 0
            __builtin_amdgcn_global_load_lds(xsrc[i] + (size_t)s * 3 * 512,
                                             lds + buf * kWideStageBytes + xdst[i], 16, 0, 0);
        }
    };
    auto load_w = [&](uint32_t s, bf16x8 (&wv)[kWideCT]) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < kWideCT; ++j) wv[j] = *(const bf16x8 *)(wt[j] + (size_t)s * 512);
    };

    f32x4 acc[kWideRT][kWideCT];
#pragma unroll
    for (int i = 0; i < kWideRT; ++i)
#pragma unroll
        for (int j = 0; j < kWideCT; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // one part of x at a time: 4 A fragments live, read just before their
    // 32 MFMAs
    auto compute = [&](uint32_t buf, const bf16x8 (&wv)[kWideCT]) __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            bf16x8 a[kWideRT];
#pragma unroll
            for (int i = 0; i < kWideRT; ++i) {
                const uint32_t chunk = (c * (kWideBM / 16) + kWideRT * wm + i) * 64 + lane;
                a[i] = __builtin_bit_cast(
                    bf16x8, *(const __attribute__((address_space(3))) u32x4g *)(
                                lds + buf * kWideStageBytes + chunk * 16));
            }
#pragma unroll
            for (int i = 0; i < kWideRT; ++i)
#pragma unroll
                for (int j = 0; j < kWideCT; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], wv[j], acc[i][j], 0, 0, 0);
                }
        }
    };
    bf16x8 wa[kWideCT], wb[kWideCT];
    copy_x(0, 0);
    load_w(0, wa);
    __syncthreads();
    // stages in pairs (K is a multiple of 64, so their number is even), so
    // that the two weight register sets alternate by name; the copy of stage
    // s + 1 into the other buffer is in flight while stage s computes, and
    // the barrier after it waits for the copy.  No branch around a compute:
    // the last pair reloads the last stage into the buffer nobody reads
    // again (a branch made the accumulators move between register files).
    const uint32_t stages = nblk;
    for (uint32_t s = 0; s < stages; s += 2) {
        copy_x(s + 1, 1);
        load_w(s + 1, wb);
        compute(0, wa);
        __syncthreads();
        const uint32_t s2 = min(s + 2, stages - 1);
        copy_x(s2, 0);
        load_w(s2, wa);
        compute(1, wb);
        __syncthreads();
    }

    // lane (r, g) holds y[row 4g + e][output r] of each tile in element e
    const uint32_t r = lane & 15, g = lane >> 4;
#pragma unroll
    for (int i = 0; i < kWideRT; ++i)
#pragma unroll
        for (int j = 0; j < kWideCT; ++j) {
            const f32x4 sum = acc[i][j];
            const uint32_t n = n0 + kLinTile * (kWideCT * wn + j) + r;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t m = m0 + kLinTile * (kWideRT * wm + i) + 4 * g + e;
                if (m < M && n < N) y[(size_t)m * N + n] = sum[e];
            }
        }
}

// The bf16 tile layout from a row-major [N][K] weight: thread c writes the
// 16 bytes lane c % 64 loads from tile block c / 64 (blocks in tile-major
// order, nblk per tile), zeros past N and K.
__global__ __launch_bounds__(256) void linear_pack_bf16_kernel(const uint16_t *src, uint16_t *dst,
                                                               uint64_t N, uint64_t K, uint64_t nblk,
                                                               uint64_t chunks) {
    const uint64_t c = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= chunks) return;
    const uint64_t lane = c & 63, tb = c >> 6;
    const uint64_t n = kLinTile * (tb / nblk) + (lane & 15);
    const uint64_t k0 = kLinBlock * (tb % nblk) + 8 * (lane >> 4);
    uint32_t p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint64_t ka = k0 + 2 * i;
        const uint32_t lo = n < N && ka < K ? src[n * K + ka] : 0u;
        const uint32_t hi = n < N && ka + 1 < K ? src[n * K + ka + 1] : 0u;
        p[i] = lo | (hi << 16);
    }
    *(uint4 *)(dst + c * 8) = uint4{p[0], p[1], p[2], p[3]};
}

// How a call is cut: T output tiles per wave, W waves per workgroup and K
// split over `splits` workgroups per tile (their partial sums are added by
// a second kernel, in split order), never more workgroups than CUs (one
// 8-wave workgroup fills a CU: one more would take a second round).  T = 3
// or, for bf16 weights, 4 (x read once per 48 or 64 outputs, 8 waves: two
// per SIMD; wider weights take more registers than a wave has) when its
// workgroups cover 7/8 of the CUs without a split, or with one when the
// weight is large enough (kLinSplitTElems) that the second kernel's few
// microseconds are small against the stream; otherwise one tile per wave
// and 4 waves, K split until the CUs are covered.
constexpr uint64_t kLinSplitTElems = (uint64_t)32 << 20;
struct LinPlan {
    uint32_t T, W, splits;
};
LinPlan linear_plan(uint32_t M, uint32_t N, uint32_t K, uint32_t dtype, int num_cus) {
    const uint64_t cus = (uint64_t)(num_cus > 0 ? num_cus : 1);
    const uint64_t mt = (M + kLinTile - 1) / kLinTile;
    auto splits_for = [&](uint64_t tiles) -> uint32_t {
        if (tiles == 0 || tiles >= cus) return 1;
        uint64_t s = cus / tiles;
        s = std::min<uint64_t>(s, K / kLinMinSplitK);
        s = std::min<uint64_t>(s, kLinMaxSplits);
        return s < 1 ? 1u : (uint32_t)s;
    };
    const uint32_t t_max = dtype == SAFETYRAISE_KERNEL_DTYPE_BF16 ? 4 : 3;
    for (uint32_t T = 3; T <= t_max; ++T) {
        const uint64_t t = (uint64_t)((N + T * kLinTile - 1) / (T * kLinTile)) * mt;
        const uint32_t s = splits_for(t);
        if (t * s * 8 >= cus * 7 && (s == 1 || (uint64_t)N * K >= kLinSplitTElems)) {
            return {T, 8, s};
        }
    }
    const uint64_t t1 = (uint64_t)((N + kLinTile - 1) / kLinTile) * mt;
    return {1, kLinWaves, splits_for(t1)};
}

template <int DT, int T, int W, int kGroup>
void launch_dt(hipStream_t stream, const float *x, const void *w, float *y, uint32_t M, uint32_t N,
               uint32_t K, uint32_t splits) {
    const dim3 grid((N + kLinTile * T - 1) / (kLinTile * T), (M + kLinTile - 1) / kLinTile, splits);
    // the kernel timer's label names the plan (tiles per wave, K split)
    const char *name = T == 3   ? "linear_kernel_t3"
                       : T == 4 ? "linear_kernel_t4"
                                : (splits > 1 ? "linear_kernel_t1_split" : "linear_kernel_t1");
    // 16-byte loads need 16-byte aligned rows: K a multiple of 8 and x itself
    // aligned (a device caller may pass a view that starts mid-vector; the
    // weight is the plugin's own allocation)
    if ((K & 7u) == 0 && ((uintptr_t)x & 15u) == 0) {
        // every wave gets the same whole number of pairs of groups
        const bool exact = K % kLinBlock == 0 &&
                           (K / kLinBlock) % (splits * (uint32_t)W * 2u * (uint32_t)kGroup) == 0;
        if (exact) {
            SR_LAUNCH(name, (linear_kernel<DT, true, T, W, kGroup, true>), grid, dim3(64 * W), 0,
                      stream, x, w, y, M, N, K);
        } else {
            SR_LAUNCH(name, (linear_kernel<DT, true, T, W, kGroup, false>), grid, dim3(64 * W), 0,
                      stream, x, w, y, M, N, K);
        }
    } else {
        SR_LAUNCH(name, (linear_kernel<DT, false, T, W, kGroup, false>), grid, dim3(64 * W), 0,
                  stream, x, w, y, M, N, K);
    }
}

template <int DT>
void launch_dt_plan(hipStream_t stream, const float *x, const void *w, float *y, uint32_t M,
                    uint32_t N, uint32_t K, const LinPlan &plan, int num_cus) {
    if (plan.T == 3) {
        launch_dt<DT, 3, 8, 2>(stream, x, w, y, M, N, K, plan.splits);
        return;
    }
    if constexpr (DT == SAFETYRAISE_KERNEL_DTYPE_BF16) {
        if (plan.T == 4) {
            launch_dt<DT, 4, 8, 2>(stream, x, w, y, M, N, K, plan.splits);
            return;
        }
    }
    const uint64_t wgs = (uint64_t)((N + kLinTile - 1) / kLinTile) * ((M + kLinTile - 1) / kLinTile) *
                         plan.splits;
    if (wgs >= 2 * (uint64_t)(num_cus > 0 ? num_cus : 1)) {
        launch_dt<DT, 1, kLinWaves, 2>(stream, x, w, y, M, N, K, plan.splits);
    } else {
        launch_dt<DT, 1, kLinWaves, 4>(stream, x, w, y, M, N, K, plan.splits);
    }
}

}  // namespace

size_t linear_weight_bytes(uint64_t rows, uint64_t cols, uint32_t dtype) {
    uint64_t n = 0, bytes = 0;
    if (dtype == SAFETYRAISE_KERNEL_DTYPE_BF16) {
        // whole tiles of 16 rows x 32 columns
        const uint64_t tiles = (rows + kLinTile - 1) / kLinTile;
        const uint64_t blocks = (cols + kLinBlock - 1) / kLinBlock;
        if (__builtin_mul_overflow(tiles, blocks, &n) || __builtin_mul_overflow(n, 1024u, &bytes)) {
            return SIZE_MAX;
        }
        return (size_t)bytes;
    }
    const uint64_t element = dtype == SAFETYRAISE_KERNEL_DTYPE_F32 ? 4 : 2;
    if (__builtin_mul_overflow(rows, cols, &n) || __builtin_mul_overflow(n, element, &bytes)) {
        return SIZE_MAX;
    }
    return (size_t)bytes;
}

hipError_t linear_pack_bf16(hipStream_t stream, const void *src, void *dst, uint64_t rows,
                            uint64_t cols) {
    const uint64_t nblk = (cols + kLinBlock - 1) / kLinBlock;
    const uint64_t chunks = (rows + kLinTile - 1) / kLinTile * nblk * 64;
    if (chunks == 0) return hipSuccess;
    const uint64_t blocks = (chunks + 255) / 256;
    if (blocks > 0x7fffffffu) return hipErrorInvalidValue;
    SR_LAUNCH("linear_pack_bf16_kernel", linear_pack_bf16_kernel, dim3((uint32_t)blocks),
              dim3(256), 0, stream, (const uint16_t *)src, (uint16_t *)dst, rows, cols, nblk,
              chunks);
    return hipGetLastError();
}

namespace {
constexpr uint32_t kMaxRows = 65535u * kLinTile;  // grid y limit of one row-tile launch

// Whether a call takes the tiled product: bf16 weight, 64+ rows, K a multiple
// of 64, and 128 x 128 tiles for at least half the CUs (fewer, and the
// row-tile kernel's weight stream is faster).  Calls above kMaxRows rows run
// as row blocks without scratch.
bool gemm_applies(uint32_t M, uint32_t N, uint32_t K, uint32_t dtype, int num_cus) {
    if (dtype != SAFETYRAISE_KERNEL_DTYPE_BF16 || M < kGemmMinRows || M > kMaxRows || K == 0 ||
        K % kGemmK != 0) {
        return false;
    }
    const uint64_t tiles = (uint64_t)((M + kGemmBM - 1) / kGemmBM) * ((N + kGemmBN - 1) / kGemmBN);
    return 2 * tiles >= (uint64_t)(num_cus > 0 ? num_cus : 1);
}
// split x of a tiled-product call: whole row tiles x K x 3 bf16 parts
size_t gemm_split_bytes(uint32_t M, uint32_t K) {
    return (size_t)((M + kLinTile - 1) / kLinTile) * kLinTile * K * 3 * sizeof(uint16_t);
}
}  // namespace

size_t linear_scratch_bytes(uint32_t M, uint32_t N, uint32_t K, uint32_t dtype, int num_cus) {
    if (gemm_applies(M, N, K, dtype, num_cus)) return gemm_split_bytes(M, K);
    const uint32_t s = linear_plan(M, N, K, dtype, num_cus).splits;
    return s > 1 ? (size_t)s * M * N * sizeof(float) : 0;
}

// y = 0 for calls with no inputs per output (K = 0): the sum over an empty
// row, as the reference's loop leaves it (a kernel, not a memset, so that a
// captured stream records no memset node)
__global__ __launch_bounds__(256) void linear_zero_kernel(float *y, uint64_t count) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < count) y[i] = 0.0f;
}

hipError_t launch_linear(hipStream_t stream, const float *x, const void *w, uint32_t dtype,
                         float *y, uint32_t M, uint32_t N, uint32_t K, float *scratch,
                         int num_cus) {
    if (M == 0 || N == 0) return hipSuccess;
    if (K == 0) {
        const uint64_t count = (uint64_t)M * N;
        SR_LAUNCH("linear_zero_kernel", linear_zero_kernel, dim3((uint32_t)((count + 255) / 256)),
                  dim3(256), 0, stream, y, count);
        return hipGetLastError();
    }
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
    if (scratch != nullptr && gemm_applies(M, N, K, dtype, num_cus)) {
        // x split once into scratch, then the tiled product; its two x
        // stages take 96 KB of LDS, above the default limit
        static const hipError_t configured = hipFuncSetAttribute(
            (const void *)linear_gemm_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
            2 * kGemmStageBytes);
        if (configured != hipSuccess) return configured;
        uint16_t *xs = (uint16_t *)scratch;
        const uint64_t chunks = (uint64_t)((M + kLinTile - 1) / kLinTile) * (K / kLinBlock) * 64;
        const dim3 sgrid((uint32_t)((chunks + 255) / 256));
        if (((uintptr_t)x & 15u) == 0) {
            SR_LAUNCH("linear_split_x_kernel", linear_split_x_kernel<true>, sgrid, dim3(256), 0,
                      stream, x, xs, M, K, chunks);
        } else {
            SR_LAUNCH("linear_split_x_kernel", linear_split_x_kernel<false>, sgrid, dim3(256), 0,
                      stream, x, xs, M, K, chunks);
        }
        const uint64_t wide_tiles =
            (uint64_t)((M + kWideBM - 1) / kWideBM) * ((N + kWideBN - 1) / kWideBN);
        if (N >= kWideMinOutputs && 2 * wide_tiles >= (uint64_t)(num_cus > 0 ? num_cus : 1)) {
            const dim3 grid((N + kWideBN - 1) / kWideBN, (M + kWideBM - 1) / kWideBM);
            SR_LAUNCH("linear_gemm_wide_kernel", linear_gemm_wide_kernel, grid, dim3(kWideThreads),
                      2 * kWideStageBytes, stream, xs, w, y, M, N, K);
            return hipGetLastError();
        }
        const dim3 grid((N + kGemmBN - 1) / kGemmBN, (M + kGemmBM - 1) / kGemmBM);
        SR_LAUNCH("linear_gemm_kernel", linear_gemm_kernel, grid, dim3(64 * kGemmWM * kGemmWN),
                  2 * kGemmStageBytes, stream, xs, w, y, M, N, K);
        return hipGetLastError();
    }
    const LinPlan plan = linear_plan(M, N, K, dtype, num_cus);
    const uint32_t splits = plan.splits;
    if (splits > 1 && scratch == nullptr) return hipErrorInvalidValue;
    float *dst = splits > 1 ? scratch : y;
    switch (dtype) {
        case SAFETYRAISE_KERNEL_DTYPE_F32:
            launch_dt_plan<SAFETYRAISE_KERNEL_DTYPE_F32>(stream, x, w, dst, M, N, K, plan, num_cus);
            break;
        case SAFETYRAISE_KERNEL_DTYPE_F16:
            launch_dt_plan<SAFETYRAISE_KERNEL_DTYPE_F16>(stream, x, w, dst, M, N, K, plan, num_cus);
            break;
        case SAFETYRAISE_KERNEL_DTYPE_BF16:
            launch_dt_plan<SAFETYRAISE_KERNEL_DTYPE_BF16>(stream, x, w, dst, M, N, K, plan, num_cus);
            break;
        default:
            return hipErrorInvalidValue;
    }
    if (splits > 1) {
        // splits > 1 only when the tiles do not cover the CUs, so M * N is small
        const uint32_t count = M * N;
        SR_LAUNCH("linear_split_sum_kernel", linear_split_sum_kernel, dim3((count + 255) / 256),
                  dim3(256), 0, stream, scratch, y, count, splits);
    }
    return hipGetLastError();
}

}  // namespace sr
