// Device helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdint>

#include "sr_internal.hpp"

// hipLaunchKernelGGL with the kernel timer's events for this launch (null
// events, an ordinary launch, when timing is off).
#define SR_LAUNCH(name, kernel, grid, block, lds, stream, ...)                              \
    do {                                                                                    \
        const ::sr::LaunchEvents _ev = ::sr::timed_launch(name);                            \
        hipExtLaunchKernelGGL(kernel, grid, block, lds, stream, _ev.start, _ev.stop, 0,     \
                              __VA_ARGS__);                                                 \
    } while (0)

namespace sr {

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float((uint32_t)h << 16);
}
__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// f32 to bf16, rounded to nearest even (one v_cvt_pk_bf16_f32 per pair;
// f32 denormals are kept, a NaN stays a NaN).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// acc + a.lo*b.lo + a.hi*b.hi for packed bf16 pairs, f32 accumulation
// (the products of two bf16 values are exact in f32).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), acc, false);
}

// Reads element i of an f32 or bf16 activation tensor.
__device__ __forceinline__ float load_act(const void *p, size_t i, bool bf16) {
    return bf16 ? bf16_to_f32(((const uint16_t *)p)[i]) : ((const float *)p)[i];
}

// The same without a branch: one 32-bit load of the aligned word that holds
// element i (the element itself for f32), then a select.  Loads behind a
// branch end in a wait for every load in flight; these stay in flight.
__device__ __forceinline__ float load_act_nb(const void *p, size_t i, bool bf16) {
    const uint32_t *w = (const uint32_t *)p + (bf16 ? (i >> 1) : i);
    const uint32_t x = *w;
    const uint32_t bits = bf16 ? ((i & 1) ? (x & 0xffff0000u) : (x << 16)) : x;
    return __uint_as_float(bits);
}

// Index of the calling wave in its workgroup, in a scalar register: branches
// on it are scalar branches, so a wave runs only its own side of an
// if/else instead of both under an exec mask (where registers one side loads
// into and the other reuses would cost a wait for every load in flight).
__device__ __forceinline__ int wave_index() {
    return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

// Pins a kernel-argument pointer in scalar registers at this point (its read
// is issued with the other argument reads and waited for once, not at each
// first use) and hands it back as a pointer still known to address global
// memory: a pointer pinned as is becomes generic, and loads through it flat
// loads, which also count against the LDS wait counter.
template <typename T>
__device__ __forceinline__ T *pin_global(T *p) {
    uint64_t v = (uint64_t)p;
    asm volatile("" : "+s"(v));
    return (T *)(__attribute__((address_space(1))) T *)v;
}

// A pointer held as an integer (for example pinned together with other
// values in one asm statement), back as a pointer known to address global
// memory.
template <typename T>
__device__ __forceinline__ T *global_from_bits(uint64_t v) {
    return (T *)(__attribute__((address_space(1))) T *)v;
}

// DPP controls (gfx9 encoding): quad permutes, half-row and row mirrors.
constexpr int kDppQuadXor1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}

// Sum / max over each aligned group of 16 lanes; every lane of the group ends
// with the same bits (each step combines a commutative pair).
__device__ __forceinline__ float sum16(float x) {
    x += dpp<kDppQuadXor1>(x);
    x += dpp<kDppQuadXor2>(x);
    x += dpp<kDppRowHalfMirror>(x);
    x += dpp<kDppRowMirror>(x);
    return x;
}
__device__ __forceinline__ float max16(float x) {
    x = fmaxf(x, dpp<kDppQuadXor1>(x));
    x = fmaxf(x, dpp<kDppQuadXor2>(x));
    x = fmaxf(x, dpp<kDppRowHalfMirror>(x));
    x = fmaxf(x, dpp<kDppRowMirror>(x));
    return x;
}
// Over the whole 64-lane wave.
__device__ __forceinline__ float sum64(float x) {
    x = sum16(x);
    x += __shfl_xor(x, 16);
    x += __shfl_xor(x, 32);
    return x;
}
__device__ __forceinline__ float max64(float x) {
    x = max16(x);
    x = fmaxf(x, __shfl_xor(x, 16));
    x = fmaxf(x, __shfl_xor(x, 32));
    return x;
}

// MRoPE axis of rotary pair i (src/model/math.rs:69-89).
__device__ __forceinline__ int rope_axis(uint32_t i, const uint32_t mrope[3], bool interleaved) {
    if (mrope[0] == 0 && mrope[1] == 0 && mrope[2] == 0) {
        return 0;
    }
    if (interleaved) {
        if (i % 3 == 1 && i < mrope[1] * 3) return 1;
        if (i % 3 == 2 && i < mrope[2] * 3) return 2;
        return 0;
    }
    if (i < mrope[0]) return 0;
    if (i < mrope[0] + mrope[1]) return 1;
    return 2;
}

// Reference sigmoid (src/model/math.rs:11-18): 1 / (1 + e^-x) for x >= 0,
// e^x / (1 + e^x) otherwise.  Both branches share e = e^{-|x|}, so one exp
// and one division give the same values without divergence.
__device__ __forceinline__ float ref_sigmoid(float x) {
    const float e = expf(-fabsf(x));
    return (x >= 0.0f ? 1.0f : e) / (1.0f + e);
}

}  // namespace sr
