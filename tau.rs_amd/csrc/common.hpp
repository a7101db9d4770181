// Shared device helpers for the MI355X (gfx950, CDNA4) MoE expert-FFN path.
//
// Conventions used by every kernel in this library:
//  * activations and expert weights are BF16, accumulation is FP32;
//  * wavefronts are 64 lanes; MFMA tiles are v_mfma_f32_32x32x16_bf16 (LDS-tiled
//    prefill) and v_mfma_f32_16x16x32_bf16 (weight-streaming decode);
//  * launches never allocate, synchronise or read back; they are ordered on the
//    caller's stream and return 0 on successful enqueue, hipErrorInvalidValue (1)
//    for rejected arguments, otherwise hipGetLastError().
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tau_moe.h"

namespace tau_amd {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr int kXcds = 8;  // MI355X: 8 XCDs, blocks dispatched round-robin over them

// Invalid-argument status, identical in value to hipErrorInvalidValue and the
// reference's cudaErrorInvalidValue.
constexpr int kInvalid = (int)hipErrorInvalidValue;

__device__ __forceinline__ float bf16_bits_to_float(uint16_t b) {
    return __uint_as_float(((uint32_t)b) << 16);
}

// Round-to-nearest-even FP32 -> BF16 (NaN stays NaN); lowers to v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint16_t float_to_bf16_bits(float v) {
    __bf16 h = (__bf16)v;
    return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float round_bf16(float v) {
    return bf16_bits_to_float(float_to_bf16_bits(v));
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return (uint32_t)float_to_bf16_bits(lo) | ((uint32_t)float_to_bf16_bits(hi) << 16);
}

// SiLU in FP32: v / (1 + exp(-v)) (silu_and_mul.cu:71-74 of the reference).
__device__ __forceinline__ float silu(float v) {
    return v / (1.0f + expf(-v));
}

__device__ __forceinline__ float sigmoid(float v) {
    return 1.0f / (1.0f + expf(-v));
}

// Block-index remap so that consecutive work items land on the same XCD
// (block b runs on XCD b % 8).  `per_xcd` = ceil(total / 8); returns an item
// index in [0, 8 * per_xcd), or -1 for blocks past 8 * per_xcd (grids are
// sized from capacity, so the tail blocks must not alias live items).
// Callers also drop indices >= total.
__device__ __forceinline__ int xcd_remap(int block, int per_xcd) {
    if (block >= kXcds * per_xcd) return -1;
    return (block % kXcds) * per_xcd + block / kXcds;
}

// Wave-wide lane mask of lanes below this one.
__device__ __forceinline__ uint64_t lanemask_lt() {
    const int lane = threadIdx.x & 63;
    return lane ? (~0ull >> (64 - lane)) : 0ull;
}

}  // namespace tau_amd
