// ABI v1 linear on the matrix cores: y[M][N] = x[M][K] . W[N][K]^T with f32
// inputs and outputs and an f32, f16 or bf16 weight that stays on the device
// (native/cpu/safetyraise_cpu.c:203-239 is the reference: an f32 sum over the
// columns of each weight row, the weight widened exactly to f32).
//
// The weight is widened exactly here too and the products run on
// v_mfma_f32_16x16x4f32, so every product is an f32 product and only the
// order of the sum differs from the reference (f32 tolerance, not bf16).
//
// Work split.  A workgroup owns 16 rows x 16 outputs; its four waves take
// contiguous quarters of K and meet in LDS.  Decode-sized calls (M <= 16)
// thus launch N/16 workgroups that each stream their 16 weight rows once,
// which is the HBM-bound regime the ABI's projections live in; each k-step
// loads 16 bytes of x and 4 weight elements per lane and feeds 4 MFMAs.
//
// Operand order.  For MFMA t of a 16-wide k block, lane (r = lane % 16,
// g = lane / 16) feeds A = x[row r][k0 + 4g + t] and B = W[output r][same k]:
// the four MFMAs cover the block's 16 k values with each lane reading 4
// consecutive ones (any order of k gives the same sum; A and B share it).
// The accumulator then holds y[row 4g + i][output r] in element i.

#include "sr_internal.hpp"
#include "sr_device.hpp"

namespace sr {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

constexpr int kLinTile = 16;   // rows and outputs per workgroup
constexpr int kLinWaves = 4;   // waves splitting K

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

// Elements k .. k+3 of a row starting at element `row` (zeros past K).
// kVec: K % 4 == 0, so a block start k < K has all four in range and the
// row start is 16-byte aligned for f32 (8-byte for 16-bit weights).
template <int DT, bool kVec>
__device__ __forceinline__ f32x4 load4(const void *base, size_t row, uint32_t k, uint32_t K) {
    f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (kVec) {
        if (k < K) {
            if constexpr (DT == SAFETYRAISE_KERNEL_DTYPE_F32) {
                v = *(const f32x4 *)((const float *)base + row + k);
            } else if constexpr (DT == SAFETYRAISE_KERNEL_DTYPE_F16) {
                v = __builtin_convertvector(*(const f16x4 *)((const _Float16 *)base + row + k), f32x4);
            } else {
                const uint2 u = *(const uint2 *)((const uint16_t *)base + row + k);
                v = f32x4{__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                          __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u)};
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (k + j < K) v[j] = widen<DT>(base, row + k + j);
        }
    }
    return v;
}

template <int DT, bool kVec>
__global__ __launch_bounds__(64 * kLinWaves) void linear_kernel(const float *x, const void *w,
                                                                 float *y, uint32_t M, uint32_t N,
                                                                 uint32_t K) {
    __shared__ f32x4 red[kLinWaves - 1][64];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const uint32_t r = lane & 15, g = lane >> 4;
    const uint32_t n0 = blockIdx.x * kLinTile, m0 = blockIdx.y * kLinTile;
    // rows past M / N read the last row and their results are not stored
    const size_t xrow = (size_t)min(m0 + r, M - 1) * K;
    const size_t wrow = (size_t)min(n0 + r, N - 1) * K;
    const uint32_t nblk = (K + 15) / 16;
    const uint32_t b0 = (uint32_t)((uint64_t)nblk * wave / kLinWaves);
    const uint32_t b1 = (uint32_t)((uint64_t)nblk * (wave + 1) / kLinWaves);
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t b = b0; b < b1; ++b) {
        const uint32_t k = 16 * b + 4 * g;
        const f32x4 a = load4<SAFETYRAISE_KERNEL_DTYPE_F32, kVec>(x, xrow, k, K);
        const f32x4 c = load4<DT, kVec>(w, wrow, k, K);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, c.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, c.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, c.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, c.w, acc, 0, 0, 0);
    }
    if (wave > 0) red[wave - 1][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int j = 0; j < kLinWaves - 1; ++j) acc += red[j][lane];
    const uint32_t n = n0 + r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t m = m0 + 4 * g + i;
        if (m < M && n < N) y[(size_t)m * N + n] = acc[i];
    }
}

template <int DT>
void launch_dt(hipStream_t stream, const float *x, const void *w, float *y, uint32_t M, uint32_t N,
               uint32_t K) {
    const dim3 grid((N + kLinTile - 1) / kLinTile, (M + kLinTile - 1) / kLinTile);
    if ((K & 3u) == 0) {
        hipLaunchKernelGGL((linear_kernel<DT, true>), grid, dim3(64 * kLinWaves), 0, stream, x, w, y,
                           M, N, K);
    } else {
        hipLaunchKernelGGL((linear_kernel<DT, false>), grid, dim3(64 * kLinWaves), 0, stream, x, w,
                           y, M, N, K);
    }
}

}  // namespace

hipError_t launch_linear(hipStream_t stream, const float *x, const void *w, uint32_t dtype,
                         float *y, uint32_t M, uint32_t N, uint32_t K) {
    if (M == 0 || N == 0) return hipSuccess;
    if (M > 65535u * kLinTile) return hipErrorInvalidValue;  // grid y limit
    switch (dtype) {
        case SAFETYRAISE_KERNEL_DTYPE_F32:
            launch_dt<SAFETYRAISE_KERNEL_DTYPE_F32>(stream, x, w, y, M, N, K);
            break;
        case SAFETYRAISE_KERNEL_DTYPE_F16:
            launch_dt<SAFETYRAISE_KERNEL_DTYPE_F16>(stream, x, w, y, M, N, K);
            break;
        case SAFETYRAISE_KERNEL_DTYPE_BF16:
            launch_dt<SAFETYRAISE_KERNEL_DTYPE_BF16>(stream, x, w, y, M, N, K);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace sr
