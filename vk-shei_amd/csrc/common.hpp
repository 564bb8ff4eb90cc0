// Shared device helpers for the gfx950 attention path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// Device code is written for gfx950 (MI355X) only.  Besides the MFMA shapes,
// LDS transpose reads and DMA forms it uses, the split merges of decode and
// prefill publish partials across XCDs with relaxed agent-scope atomics whose
// order is gfx950's implementation (write-through stores, L2-bypassing
// loads), so any other target is refused at compile time.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "mslim_attn device code targets gfx950 only"
#endif

namespace mslim {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef float floatx16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;

// BF16 decode: the bit pattern is the high half of an f32 (gpu_llm.cl:7-9).
__device__ __forceinline__ float bf16_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t pair) { return __uint_as_float(pair & 0xffff0000u); }
__device__ __forceinline__ float read_bf16(uint16_t bits) { return __uint_as_float(((uint32_t)bits) << 16); }

// BF16 encode with the reference's exact rule (gpu_llm.cl:10-21): NaN keeps
// sign and upper payload with the quiet bit forced; everything else rounds to
// nearest even.  write_bf16_rule states the rule in integer steps;
// write_bf16, used for every value a kernel writes out, is gfx950's
// conversion instruction (a scalar cast, v_cvt_pk_bf16_f32 with the value in
// the low half), one instruction instead of seven.  The two agree on every
// one of the 2^32 f32 encodings, NaNs and subnormals included:
// mslim_attn_check_bf16_encoding compares them over all of them on the
// device.  (The two-value form through __builtin_convertvector gave wrong
// high halves in the same comparison and is not used.)
__device__ __forceinline__ uint16_t write_bf16_rule(float value) {
    uint32_t bits = __float_as_uint(value);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((bits >> 16) | 0x0040u);
    bits += 0x7fffu + ((bits >> 16) & 1u);
    return (uint16_t)(bits >> 16);
}

__device__ __forceinline__ uint16_t write_bf16(float value) { return __builtin_bit_cast(uint16_t, (__bf16)value); }

__device__ __forceinline__ float round_bf16(float value) { return read_bf16(write_bf16(value)); }

// Row (in head_dim units) of logical token `token`, kv head `head`, in a pool
// of pages [page][kv_heads][1 << shift][head_dim] under page-table row `table`.
__device__ __forceinline__ int64_t page_row(const int32_t *table, int shift, int kv_heads, int head,
                                           int64_t token) {
    const int64_t page = table[token >> shift];
    return ((page * kv_heads + head) << shift) + (token & ((1 << shift) - 1));
}

// llm_swiglu's arithmetic (gpu_llm.cl:225-237) on BF16 gate and up values:
// BF16(BF16(g / (1 + e^-g)) * u), e^-g evaluated in double and rounded once,
// every other step correctly rounded in f32.  The first stage depends on the
// 16 gate bits only, so kernels with many outputs read it from a 65,536-entry
// table of swiglu_act_bf16 (built once per context) instead.
__device__ __forceinline__ uint16_t swiglu_act_bf16(uint16_t gate) {
    const float g = read_bf16(gate);
    const float e = (float)exp(-(double)g);
    return write_bf16(__fdiv_rn(g, __fadd_rn(1.0f, e)));
}
__device__ __forceinline__ uint16_t swiglu_mul_bf16(uint16_t activated, uint16_t up) {
    return write_bf16(__fmul_rn(read_bf16(activated), read_bf16(up)));
}
__device__ __forceinline__ uint16_t swiglu_bf16(uint16_t gate, uint16_t up) {
    return swiglu_mul_bf16(swiglu_act_bf16(gate), up);
}

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

// A pointer that is the same in every lane, kept in SGPRs (the compiler
// cannot always prove uniformity; scalar-base copies need it).
template <typename T>
__device__ __forceinline__ T *uniform_ptr(T *p) {
    const uint64_t v = reinterpret_cast<uintptr_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<T *>((uintptr_t)(((uint64_t)hi << 32) | lo));
}

// LDS offset (wave-uniform, in an SGPR) of a __shared__ address.
__device__ __forceinline__ uint32_t lds_offset(const void *lds) {
    return __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)lds);
}

// The same copy as dma16 from a wavefront-uniform base (an SGPR pair) plus
// a per-lane 32-bit byte offset, issued through inline assembly so that the
// compiler does not order later LDS reads behind it (it cannot tell which
// LDS stage an in-flight copy targets and would wait for all of them).  The
// caller waits for it explicitly: s_waitcnt vmcnt, then a barrier, before any
// wavefront reads the destination.  A loop over tiles advances only the
// scalar base, so a copy costs no per-lane address arithmetic.
// M0 is reserved by the compiler, so the asm saves and restores it.
__device__ __forceinline__ void dma16_async(const void *base, uint32_t offset, uint32_t lds_base) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %3\n\t"
        "global_load_lds_dwordx4 %1, %2\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(offset), "s"(base), "s"(lds_base)
        : "memory");
}

// ds_read_b64_tr_b16: within each 16-lane quarter wave, lane i receives
// element i%4 of the 8 bytes read by lanes i/4, 4+i/4, 8+i/4, 12+i/4.
__device__ __forceinline__ short4_t lds_read_tr16(const uint16_t *lds) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) short4_t *)(lds));
}

// The same two reads from a 32-bit LDS byte address.
__device__ __forceinline__ short4_t lds_read_tr16_at(uint32_t addr) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4_t *)(uintptr_t)addr);
}
__device__ __forceinline__ bf16x8_t lds_read_b128(uint32_t addr) {
    return *(const __attribute__((address_space(3))) bf16x8_t *)(uintptr_t)addr;
}

// s_waitcnt immediate that waits until at most n vector-memory operations
// are outstanding and leaves the LDS/scalar and export counters alone.
constexpr int vmcnt_imm(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }
// The same with every LDS read of this wavefront complete (lgkmcnt 0).
constexpr int vmcnt_lds_imm(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4); }
// The same with at most l LDS reads outstanding (lgkmcnt l).  LDS reads
// complete in issue order when no scalar memory load is in flight, so the
// last l reads may still be pending and every earlier one has completed.
constexpr int vmcnt_lds_last_imm(int n, int l) { return vmcnt_lds_imm(n) | (l << 8); }

// Workgroup barrier without the memory fence of __syncthreads(): with LDS
// DMA in flight that fence would wait for every outstanding DMA (vmcnt 0).
// Callers order LDS themselves with vmcnt_lds_imm waits before it.
__device__ __forceinline__ void raw_barrier() { __builtin_amdgcn_s_barrier(); }

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

// Maximum of a lane's value and its partner's in the other 32-lane half.
// v_permlane32_swap on two copies of x leaves, in every lane, x itself in one
// result and the partner's x in the other, so their maximum is the answer.
__device__ __forceinline__ float half_pair_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __builtin_fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Keeps a value's computation at this point of the program: an empty asm
// that reads and writes it cannot be moved, so the value must be ready here
// (used to hold VALU work between the MFMAs it is meant to overlap).
__device__ __forceinline__ void pin_value(uint32_t &x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void pin_value(float &x) { asm volatile("" : "+v"(x)); }

// Butterfly reductions across the 64-lane wavefront.
__device__ __forceinline__ float wave_xor_max(float v, int mask) {
    return fmaxf(v, __shfl_xor(v, mask, 64));
}
__device__ __forceinline__ float wave_xor_sum(float v, int mask) {
    return v + __shfl_xor(v, mask, 64);
}

}  // namespace mslim
