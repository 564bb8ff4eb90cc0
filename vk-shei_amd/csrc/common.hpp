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

// IEEE binary16 -> f32, exact for every encoding (subnormals, inf, NaN
// payloads) through the hardware conversion.
__device__ __forceinline__ float half_to_float(uint16_t bits) {
    return (float)__builtin_bit_cast(_Float16, bits);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return (uint32_t)write_bf16(lo) | ((uint32_t)write_bf16(hi) << 16);
}

typedef short short4_t __attribute__((ext_vector_type(4)));
typedef short short8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// HBM -> LDS copy of 16 bytes per lane (global_load_lds_dwordx4): lane l's
// bytes land at lds_base + 16*l; lds_base must be wavefront-uniform.
__device__ __forceinline__ void dma16(const void *global, void *lds_base) {
    __builtin_amdgcn_global_load_lds(global, lds_base, 16, 0, 0);
}

// ds_read_b64_tr_b16: within each 16-lane quarter wave, lane i receives
// element i%4 of the 8 bytes read by lanes i/4, 4+i/4, 8+i/4, 12+i/4.
__device__ __forceinline__ short4_t lds_read_tr16(const uint16_t *lds) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) short4_t *)(lds));
}

__device__ __forceinline__ bool wave_any(bool pred) {
    return __builtin_amdgcn_ballot_w64(pred) != 0;
}

// Sum of a BF16 pair into an fp32 accumulator (v_dot2_f32_bf16 with ones).
__device__ __forceinline__ float add_bf16_pair(bf16x2_t pair, float acc) {
    bf16x2_t ones;
    ones[0] = (__bf16)1.0f;
    ones[1] = (__bf16)1.0f;
    return __builtin_amdgcn_fdot2_f32_bf16(pair, ones, acc, false);
}

// Butterfly reductions across the 64-lane wavefront.
__device__ __forceinline__ float wave_xor_max(float v, int mask) {
    return fmaxf(v, __shfl_xor(v, mask, 64));
}
__device__ __forceinline__ float wave_xor_sum(float v, int mask) {
    return v + __shfl_xor(v, mask, 64);
}

}  // namespace mslim
