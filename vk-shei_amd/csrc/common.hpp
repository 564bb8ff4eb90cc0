// Shared device helpers for the gfx950 attention path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mslim {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef float floatx16_t __attribute__((ext_vector_type(16)));

constexpr float kLog2e = 1.4426950408889634f;

// BF16 decode: the bit pattern is the high half of an f32 (gpu_llm.cl:7-9).
__device__ __forceinline__ float bf16_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t pair) { return __uint_as_float(pair & 0xffff0000u); }
__device__ __forceinline__ float read_bf16(uint16_t bits) { return __uint_as_float(((uint32_t)bits) << 16); }

// BF16 encode with the reference's exact rule (gpu_llm.cl:10-21): NaN keeps
// sign and upper payload with the quiet bit forced; everything else rounds to
// nearest even.  Used for every value a kernel writes out.
__device__ __forceinline__ uint16_t write_bf16(float value) {
    uint32_t bits = __float_as_uint(value);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((bits >> 16) | 0x0040u);
    bits += 0x7fffu + ((bits >> 16) & 1u);
    return (uint16_t)(bits >> 16);
}

__device__ __forceinline__ float round_bf16(float value) { return read_bf16(write_bf16(value)); }

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return (uint32_t)write_bf16(lo) | ((uint32_t)write_bf16(hi) << 16);
}

// Butterfly reductions across the 64-lane wavefront.
__device__ __forceinline__ float wave_xor_max(float v, int mask) {
    return fmaxf(v, __shfl_xor(v, mask, 64));
}
__device__ __forceinline__ float wave_xor_sum(float v, int mask) {
    return v + __shfl_xor(v, mask, 64);
}

}  // namespace mslim
