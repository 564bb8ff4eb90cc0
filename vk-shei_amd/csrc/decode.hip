// Single-token GQA decode over a BF16 K/V cache, dense or ColdStore-paged.
//
// Replaces llm_attention_qk / softmax / pv (gpu_llm.cl:150-212),
// llm_exact_hot_fused_attention (:975-1025), the ColdStore-V PV stage
// (:280-322) and the split-KV mode of mslim_attention_tiled / _merge
// (tiled_attention.cl:9-155).
//
// Decode reads every K and V byte once, so it is an HBM stream.  One
// workgroup of four wavefronts owns one (sequence, kv head, split)
// partition of `split_tokens` logical tokens and serves all G query heads of
// the GQA group from the same K/V bytes:
//   * the four wavefronts take interleaved 32-token tiles, so together they
//     stream one contiguous region;
//   * each wavefront keeps a ring of DEPTH tiles of K and V in registers, so
//     DEPTH-1 tiles stay in flight while one is computed;
//   * Q.K^T for the group runs on v_mfma_f32_16x16x32_bf16 with the 16 tokens
//     of a block as M and the (zero padded) G heads as N.  Each lane loads 64
//     contiguous bytes of one K row as its A operand, so no K byte passes
//     through LDS;
//   * the online softmax max / sum run on 64-lane butterflies;
//   * P.V runs on the same MFMA: V arrives in 128-bit loads (16 lanes per
//     256-byte row for D = 128) and is staged transposed through a per-
//     wavefront LDS slab as the B operand, with P taken straight from the
//     S^T accumulator as the A operand;
//   * the four wavefronts merge in LDS; the partitions of one (sequence, kv
//     head) are merged in fixed partition order by the workgroup that
//     finishes last (or, when the context asks for it, by a second launch;
//     both orders give the same bits);
//   * launches of more partitions than two per CU run them as 512 host-
//     packed lists, one workgroup per list (the LIST kernel), so that every
//     CU gets the same work; which workgroup computes a partition does not
//     change its bits.
// Partitions are fixed by logical token index, and the paged and dense
// variants differ only in how a 16-token block's base address is formed, so
// both produce bit-identical outputs (the reference's dense == ColdStore
// invariant, gpu_llm/mod.rs:2993-3048).
#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <mutex>
#include <utility>
#include <vector>
#include <cstdint>
#include <type_traits>

namespace mslim {

namespace {

// Four wavefronts per workgroup and a ring of two tiles per wavefront: eight
// wavefronts, a three-deep ring and 2,048-token splits were each measured
// slower at cfg4 (rotating layer caches).
constexpr int kWaves = 4;
constexpr int kDepth = 2;
constexpr int kTile = 32;
// List mode: two lists per CU (two workgroups fit), at most kMaxListItems
// partitions in all.
constexpr int kListBins = 512;
constexpr int kMaxListItems = 896;

// Launch tables.  32-bit words: seq_len[batch] | split_begin[batch + 1] |
// full_begin[batch + 1]; 16-bit halves: last_order[batch] |
// bin_start[list_bins + 1] | list[items].  Launches of up to kInlineBatch
// sequences carry them in the kernel arguments (words / halves); larger ones
// read a device copy made on the stream before the launch (ext_words /
// ext_halves non-zero).  Either way the kernel reads them with scalar loads.
constexpr int kInlineWords = 3 * kInlineBatch + 2;
constexpr int kInlineHalves = (kInlineBatch + kListBins + 1 + kMaxListItems + 1) / 2 * 2;

struct DeviceArgs {
    const uint16_t *q, *k, *v;
    uint16_t *out;
    float *partial_ml;
    float *partial_acc;
    int *counters;  // [batch][kv_heads] splits finished, zero between launches
    const int32_t *page_table;
    int64_t seq_stride_tokens;
    int pages_per_seq, page_shift;
    int batch, q_heads, kv_heads;
    int split_tokens;
    float scale_log2e;
    // List mode (list_bins > 0, the LIST kernel): workgroup w runs the
    // partitions list[i], bin_start[w] <= i < bin_start[w + 1], one after
    // another, each given by its launch index (what blockIdx.x is in the
    // one-partition-per-workgroup kernel).
    int list_bins;
    uint64_t ext_words, ext_halves;
    // Launch order of the partitions: every sequence's partitions but its
    // last, in sequence order (full_begin: prefix counts), then the last
    // partitions, longest first (last_order: sequence indices).
    int32_t words[kInlineWords];
    uint16_t halves[kInlineHalves];
};

typedef const __attribute__((address_space(4))) uint32_t ConstantU32;

// The launch tables as the kernel reads them (constant address space, so a
// uniform index becomes a scalar load; halves are read as their aligned
// dword).
struct Tables {
    ConstantU32 *w, *h;
    int batch, bins;
    __device__ int half(int i) const { return (int)((h[i >> 1] >> ((i & 1) * 16)) & 0xFFFFu); }
    __device__ int seq_len(int b) const { return (int)w[b]; }
    __device__ int split_begin(int b) const { return (int)w[batch + b]; }
    __device__ int full_begin(int b) const { return (int)w[2 * batch + 1 + b]; }
    __device__ int last_order(int i) const { return half(i); }
    __device__ int bin_start(int i) const { return half(batch + i); }
    __device__ int list(int i) const { return half(batch + bins + 1 + i); }
};

// Every kernel here takes the DeviceArgs as its first argument, at offset 0
// of the kernel-argument segment.
__device__ __forceinline__ Tables tables_of(const DeviceArgs &a) {
    Tables t;
    if (a.ext_words) {
        t.w = reinterpret_cast<ConstantU32 *>(a.ext_words);
        t.h = reinterpret_cast<ConstantU32 *>(a.ext_halves);
    } else {
        const auto base = (const __attribute__((address_space(4))) char *)__builtin_amdgcn_kernarg_segment_ptr();
        t.w = reinterpret_cast<ConstantU32 *>(base + offsetof(DeviceArgs, words));
        t.h = reinterpret_cast<ConstantU32 *>(base + offsetof(DeviceArgs, halves));
    }
    t.batch = a.batch;
    t.bins = a.list_bins;
    return t;
}

// Base of the 16-token block starting at logical token t0 (a multiple of 16).
template <int D, bool PAGED>
__device__ __forceinline__ const uint16_t *block_base(const DeviceArgs &a, const uint16_t *cache,
                                                      int b, int kvh, int t0) {
    if constexpr (PAGED) {
        const int shift = a.page_shift;
        const int page = a.page_table[(int64_t)b * a.pages_per_seq + (t0 >> shift)];
        const int64_t row = (((int64_t)page * a.kv_heads + kvh) << shift) + (t0 & ((1 << shift) - 1));
        return cache + row * D;
    } else {
        return cache + (((int64_t)b * a.seq_stride_tokens + t0) * a.kv_heads + kvh) * D;
    }
}

// Element stride between consecutive token rows inside a 16-token block.
template <int D, bool PAGED>
__device__ __forceinline__ int row_stride(const DeviceArgs &a) {
    if constexpr (PAGED) return D;
    else return a.kv_heads * D;
}

// Ordering point for LDS traffic inside one wavefront: a wavefront's LDS
// operations execute in order, so only the compiler must not move them.
__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int D>
struct TileRegs {
    static constexpr int KS = D / 32;
    static constexpr int NV = D / 16;  // 128-bit V loads per 32-token tile
    bf16x8_t k[2][KS];
    uint4 v[NV];
};

// Byte pick for v_perm_b32: low half = bf16 `e` of `lo_src`, high half =
// bf16 `e` of `hi_src` (e = 0 or 1 inside the dword).
__device__ __forceinline__ uint32_t pair_bf16(uint32_t hi_src, uint32_t lo_src, int e) {
    // v_perm_b32 numbering: bytes 0-3 come from the second operand, 4-7 from
    // the first.
    const uint32_t sel = e ? 0x07060302u : 0x05040100u;
    return __builtin_amdgcn_perm(hi_src, lo_src, sel);
}

// K and V bytes are read exactly once per call.  A call that streams at least
// the 256 MB Infinity Cache loads them non-temporally (NT), so the stream
// does not allocate in L2 or the Infinity Cache; smaller calls use ordinary
// loads.  Measured over distinct caches cycled call after call (nothing
// reusable between calls), non-temporal against ordinary: 537 MB (cfg4)
// 87.9 vs 96.0 us, 268 MB 48.0 vs 51.4 us, 134-138 MB equal or up to 1.7 us
// slower (the cfg5 decoder's 8 x 4,224 tokens), 67 MB 0.5 us slower.
constexpr int64_t kNonTemporalBytes = 256ll << 20;
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
template <bool NT>
__device__ __forceinline__ bf16x8_t kv_load8(const uint16_t *p) {
    if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const bf16x8_t *>(p));
    else return *reinterpret_cast<const bf16x8_t *>(p);
}
template <bool NT>
__device__ __forceinline__ uint4 kv_load4(const uint16_t *p) {
    if constexpr (NT) {
        const u32x4_t t = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
        return make_uint4(t.x, t.y, t.z, t.w);
    } else {
        return *reinterpret_cast<const uint4 *>(p);
    }
}

// Relaxed agent-scope atomics on float pairs (8-byte aligned): coherent
// across the XCDs' L2 caches.
__device__ __forceinline__ void store_coherent2(float *p, float x, float y) {
    const uint64_t w = (uint64_t)__float_as_uint(x) | ((uint64_t)__float_as_uint(y) << 32);
    __hip_atomic_store(reinterpret_cast<uint64_t *>(p), w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 load_coherent2(const float *p) {
    const uint64_t w = __hip_atomic_load(reinterpret_cast<const uint64_t *>(p), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    return make_float2(__uint_as_float((uint32_t)w), __uint_as_float((uint32_t)(w >> 32)));
}

template <int D, int G>
__device__ __forceinline__ void merge_splits(const DeviceArgs &a, int b, int kvh, int tid, int nthreads,
                                             bool coherent);

template <int D, int G, bool PAGED, bool FUSED, bool NT, bool LIST>
__global__ __launch_bounds__(64 * kWaves, 2) void decode_kernel(DeviceArgs a) {
    constexpr int DEPTH = kDepth;
    constexpr int KS = D / 32;        // Q.K MFMA k-steps per 16-token block
    constexpr int LPR = D / 8;        // lanes per V row (8 BF16 per lane)
    constexpr int RPI = 64 / LPR;     // V rows per load instruction
    constexpr int NV = kTile / RPI;   // V loads per tile = consecutive rows per lane
    constexpr int NS = D / 16;        // P.V MFMA output slices of 16 dims
    constexpr int VT = kTile + 8;     // transposed V row (one dim), in elements
    static_assert(G <= 16, "one MFMA N tile covers the GQA group");

    __shared__ __align__(16) uint16_t vt_lds[kWaves][D * VT];
    __shared__ float comb_ml[kWaves][G][2];
    __shared__ float comb_acc[kWaves][G][D];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int row16 = lane & 15;
    const int grp = lane >> 4;
    const Tables tab = tables_of(a);
    // One partition, given by its launch index (kv head fastest).
    auto partition = [&](const int launch_index) __attribute__((always_inline)) {
    const int kvh = launch_index % a.kv_heads;
    const int sg = launch_index / a.kv_heads;
    // Full partitions launch first and the shorter last partitions after
    // them, longest first: when a launch has more workgroups than fit at
    // once, the dispatcher hands the short ones to the CUs that free up.
    // The partition's logical index (split_begin[b] + split) is unchanged.
    int b = 0, split = 0;
    const int full_total = tab.full_begin(a.batch);
    if (sg < full_total) {
        // the last sequence whose full partitions begin at or before sg
        // (full_begin does not decrease and starts at 0)
        int hi = a.batch - 1;
        while (b < hi) {
            const int mid = (b + hi + 1) >> 1;
            if (tab.full_begin(mid) <= sg) b = mid;
            else hi = mid - 1;
        }
        split = sg - tab.full_begin(b);
    } else {
        b = tab.last_order(sg - full_total);
        split = tab.split_begin(b + 1) - tab.split_begin(b) - 1;
    }
    const int nsplit = tab.split_begin(b + 1) - tab.split_begin(b);
    const int seq_len = tab.seq_len(b);
    const int begin = split * a.split_tokens;
    const int end = min(seq_len, begin + a.split_tokens);
    const int ntiles = (end - begin + kTile - 1) / kTile;
    const int qh0 = kvh * G;
    const float c = a.scale_log2e;
    const int rs = row_stride<D, PAGED>(a);
    uint16_t *vt = vt_lds[wave];

    // Q as the B operand of S^T = K.Q^T: lane holds head row16, dims
    // j*32 + grp*8 .. +8 (heads >= G are zero).
    bf16x8_t qf[KS];
#pragma unroll
    for (int j = 0; j < KS; ++j) {
        if (row16 < G)
            qf[j] = *reinterpret_cast<const bf16x8_t *>(
                a.q + ((int64_t)b * a.q_heads + qh0 + row16) * D + j * 32 + grp * 8);
        else
            qf[j] = bf16x8_t{};
    }

    // Loads of a tile never branch: rows past the last valid token are
    // clamped to it (their scores are masked to -inf), so every call issues
    // the same loads and the wait counts stay exact.
    //   K: MFMA A layout, lane = (token row16 of a 16-token block, dims grp*8
    //      + 32j), 64 contiguous bytes of one row per lane.
    //   V: lane (vh = lane / LPR, vc = lane % LPR) loads dims vc*8..+8 of the
    //      NV consecutive rows vh*NV .. vh*NV+NV-1; each load instruction
    //      covers RPI whole rows.
    const int last = end - 1;
    const int vh = lane / LPR;
    const int vc = lane % LPR;
    auto load_tile = [&](TileRegs<D> &r, int tile) {
        const int t0 = begin + tile * kTile;
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            const int bt = min(t0 + blk * 16, last & ~15);
            const int row = min(t0 + blk * 16 + row16, last) - bt;
            const uint16_t *p = block_base<D, PAGED>(a, a.k, b, kvh, bt) + row * rs + grp * 8;
#pragma unroll
            for (int j = 0; j < KS; ++j) r.k[blk][j] = kv_load8<NT>(p + j * 32);
        }
        const uint16_t *vb0 = block_base<D, PAGED>(a, a.v, b, kvh, min(t0, last & ~15));
        const uint16_t *vb1 = block_base<D, PAGED>(a, a.v, b, kvh, min(t0 + 16, last & ~15));
        const int blk = (vh * NV) >> 4;  // rows of one lane never straddle a block
        const int bt = min(t0 + blk * 16, last & ~15);
        const uint16_t *vb = blk ? vb1 : vb0;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int row = min(t0 + vh * NV + i, last) - bt;
            r.v[i] = kv_load4<NT>(vb + row * rs + vc * 8);
        }
    };

    float m_run = -INFINITY;
    float l_run = 0.0f;
    floatx4_t o[NS];  // O[head 4*grp+i][dim 16*slice + row16]
#pragma unroll
    for (int sl = 0; sl < NS; ++sl) o[sl] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};

    auto compute_tile = [&](const TileRegs<D> &r, int tile) {
        const int t0 = begin + tile * kTile;
        // Stage V transposed: vt[dim][token].  A lane owns NV consecutive
        // tokens of 8 dims, i.e. NV*2 contiguous bytes of 8 rows of vt.
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            uint32_t w[NV / 2];
#pragma unroll
            for (int k = 0; k < NV / 2; ++k) {
                const uint32_t lo = (&r.v[2 * k].x)[e >> 1];
                const uint32_t hi = (&r.v[2 * k + 1].x)[e >> 1];
                w[k] = pair_bf16(hi, lo, e & 1);
            }
            uint16_t *dst = vt + (vc * 8 + e) * VT + vh * NV;
            if constexpr (NV == 8) {
                *reinterpret_cast<uint4 *>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
            } else if constexpr (NV == 4) {
                *reinterpret_cast<uint2 *>(dst) = make_uint2(w[0], w[1]);
            }
        }

        // S^T block = K (16 tokens x D) . Q^T (D x 16 heads).
        floatx4_t s[2];
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            s[blk] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < KS; ++j)
                s[blk] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(r.k[blk][j], qf[j], s[blk], 0, 0, 0);
        }
        // Lane holds head row16, tokens t0 + blk*16 + grp*4 + i.
        if (t0 + kTile > end) {
#pragma unroll
            for (int blk = 0; blk < 2; ++blk)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (t0 + blk * 16 + grp * 4 + i >= end) s[blk][i] = -INFINITY;
        }
        float mx = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                         fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
        mx = wave_xor_max(mx, 16);
        mx = wave_xor_max(mx, 32);
        const float m_new = fmaxf(m_run, mx);
        const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * c);
        const float mc = m_new * c;
        // P as the A operand of O = P.V: row = head row16, k-slot j of lane
        // group grp = token (j < 4 ? 4*grp + j : 16 + 4*grp + j - 4), which is
        // exactly where the S^T accumulator left it.
        // The row sum adds the same BF16-rounded p that the P.V MFMA
        // multiplies, so O / l is a convex combination of V rows.
        bf16x8_t pa;
        float psum = 0.0f;
#pragma unroll
        for (int blk = 0; blk < 2; ++blk)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const __bf16 p = (__bf16)__builtin_amdgcn_exp2f(fmaf(s[blk][i], c, -mc));
                psum += (float)p;
                pa[blk * 4 + i] = p;
            }
        l_run = l_run * alpha + psum;
        m_run = m_new;
        // Rows of the O accumulator are heads 4*grp + i: fetch their alphas.
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float ai = __shfl(alpha, 4 * grp + i, 64);
#pragma unroll
            for (int sl = 0; sl < NS; ++sl) o[sl][i] *= ai;
        }
        wave_lds_fence();
        // V as the B operand: col = dim 16*slice + row16, k-slots of lane
        // group grp = the same tokens as P's.
#pragma unroll
        for (int sl = 0; sl < NS; ++sl) {
            const uint16_t *src = vt + (sl * 16 + row16) * VT + 4 * grp;
            const uint2 lo = *reinterpret_cast<const uint2 *>(src);
            const uint2 hi = *reinterpret_cast<const uint2 *>(src + 16);
            const bf16x8_t vb = __builtin_bit_cast(bf16x8_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
            o[sl] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, vb, o[sl], 0, 0, 0);
        }
        wave_lds_fence();
    };

    // Ring of DEPTH tile buffers over this wavefront's tiles wave, wave+4,
    // ...; the loop is unrolled by DEPTH so every buffer index is a
    // compile-time constant, and DEPTH-1 tiles are in flight during compute.
    const int my_tiles = ntiles > wave ? (ntiles - wave + kWaves - 1) / kWaves : 0;
    auto tile_of = [&](int i) { return wave + kWaves * min(i, my_tiles - 1); };
    TileRegs<D> ring[DEPTH];
    if (my_tiles > 0) {
#pragma unroll
        for (int d = 0; d < DEPTH - 1; ++d) load_tile(ring[d], tile_of(d));
    }
    for (int base = 0; base < my_tiles; base += DEPTH) {
#pragma unroll
        for (int s = 0; s < DEPTH; ++s) {
            const int i = base + s;
            if (i >= my_tiles) break;
            load_tile(ring[(s + DEPTH - 1) % DEPTH], tile_of(i + DEPTH - 1));
            __builtin_amdgcn_sched_barrier(0);
            compute_tile(ring[s], tile_of(i));
        }
    }

    // Per wavefront: l over the four lane groups of each head; O rows are
    // heads 4*grp + i, dims 16*slice + row16.
    l_run = wave_xor_sum(l_run, 16);
    l_run = wave_xor_sum(l_run, 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int h = 4 * grp + i;
        if (h < G) {
#pragma unroll
            for (int sl = 0; sl < NS; ++sl) comb_acc[wave][h][sl * 16 + row16] = o[sl][i];
        }
    }
    if (lane < G) {
        comb_ml[wave][lane][0] = m_run;  // -inf for a wavefront without tiles
        comb_ml[wave][lane][1] = l_run;
    }
    __syncthreads();

    // Combine the four wavefronts in fixed order: thread -> (head, 4 dims).
    constexpr int ITEMS = G * D / 4;
    const bool final_write = nsplit == 1;
    // Partials are stored by logical partition index, the order the merge
    // reads them in, whatever the launch order.
    const int64_t part = ((int64_t)(tab.split_begin(b) + split) * a.kv_heads + kvh) * G;
    for (int it = tid; it < ITEMS; it += 64 * kWaves) {
        const int g = it / (D / 4);
        const int d = (it % (D / 4)) * 4;
        float m = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) m = fmaxf(m, comb_ml[w][g][0]);
        float l = 0.0f;
        float4 ov = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float wt = __builtin_amdgcn_exp2f((comb_ml[w][g][0] - m) * c);
            l = fmaf(comb_ml[w][g][1], wt, l);
            const float4 x = *reinterpret_cast<const float4 *>(&comb_acc[w][g][d]);
            ov.x = fmaf(x.x, wt, ov.x); ov.y = fmaf(x.y, wt, ov.y);
            ov.z = fmaf(x.z, wt, ov.z); ov.w = fmaf(x.w, wt, ov.w);
        }
        if (final_write) {
            uint2 packed;
            packed.x = pack_bf16x2(ov.x / l, ov.y / l);
            packed.y = pack_bf16x2(ov.z / l, ov.w / l);
            *reinterpret_cast<uint2 *>(a.out + ((int64_t)b * a.q_heads + qh0 + g) * D + d) = packed;
        } else if constexpr (FUSED) {
            // Agent-scope atomic stores: the merging workgroup may run on
            // another XCD.
            float *pa = a.partial_acc + (part + g) * D + d;
            store_coherent2(pa, ov.x, ov.y);
            store_coherent2(pa + 2, ov.z, ov.w);
            if (d == 0) store_coherent2(a.partial_ml + (part + g) * 2, m, l);
        } else {
            *reinterpret_cast<float4 *>(a.partial_acc + (part + g) * D + d) = ov;
            if (d == 0) *reinterpret_cast<float2 *>(a.partial_ml + (part + g) * 2) = make_float2(m, l);
        }
    }
    if constexpr (FUSED) {
        if (final_write) return;
        // Publication of the partials, ordered at the ISA level: the
        // partials were written with agent-scope atomic stores, which gfx950
        // issues write-through to the device coherence point (sc1), and every
        // thread waits for its own stores to complete (s_waitcnt vmcnt(0))
        // before the barrier, so they are visible to every XCD before thread
        // 0 counts the split.  The merging workgroup reads them with
        // agent-scope atomic loads, which bypass the XCD-local L2 (sc1).  The
        // language-level release / acquire on the counter gives the same
        // order but adds an L2 write-back and invalidate per workgroup:
        // measured on cfg4 / cfg3 / the cfg5 decoder shape, 98.8 / 149 / 40
        // us with release / acquire on thread 0's RMW, 119 / 254 / 60 us with
        // a release fence in every thread, against 90.0 / 124 / 34 us here.
        // The separate merge launch (MSLIM_ATTN_OPT_DECODE_MERGE), ordered by
        // the kernel boundary, measured 92.4 / 122 / 36 us and gives the same
        // bits.  The workgroup that takes the count to nsplit - 1 merges the
        // partitions in fixed order, as decode_merge_kernel does, and resets
        // the counter for the next call.
        __builtin_amdgcn_s_waitcnt(0);
        __shared__ int last;
        __syncthreads();
        if (tid == 0) {
            int *ctr = a.counters + (int64_t)b * a.kv_heads + kvh;
            const int done = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last = done == nsplit - 1;
            if (last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!last) return;
        merge_splits<D, G>(a, b, kvh, tid, 64 * kWaves, true);
    }
    };
    if constexpr (LIST) {
        const int i0 = tab.bin_start(blockIdx.x), i1 = tab.bin_start(blockIdx.x + 1);
        for (int i = i0; i < i1; ++i) {
            if (i > i0) __syncthreads();  // the previous partition's LDS is free
            partition(tab.list(i));
        }
    } else {
        partition((int)blockIdx.x);
    }
}

// Fixed-order log-sum-exp merge of the split partials of one (sequence, kv
// head): thread -> (head, 4 dims), one online pass over the partitions (the
// deterministic counterpart of mslim_attention_merge,
// tiled_attention.cl:131-155).  Run either by the last split workgroup of
// the decode kernel (partials read with coherent loads) or as a launch of its
// own after it.
template <int D, int G>
__device__ __forceinline__ void merge_splits(const DeviceArgs &a, int b, int kvh, int tid, int nthreads,
                                             bool coherent) {
    const Tables tab = tables_of(a);
    const int nsplit = tab.split_begin(b + 1) - tab.split_begin(b);
    const int s0 = tab.split_begin(b);
    const float c = a.scale_log2e;
    const int qh0 = kvh * G;
    for (int it = tid; it < G * D / 4; it += nthreads) {
        const int g = it / (D / 4);
        const int d = (it % (D / 4)) * 4;
        float m = -INFINITY, l = 0.0f;
        float4 ov = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        auto fold = [&](float2 ml, float4 x) {
            const float m_new = fmaxf(m, ml.x);
            const float wo = __builtin_amdgcn_exp2f((m - m_new) * c);
            const float wn = __builtin_amdgcn_exp2f((ml.x - m_new) * c);
            l = fmaf(l, wo, ml.y * wn);
            ov.x = fmaf(ov.x, wo, x.x * wn); ov.y = fmaf(ov.y, wo, x.y * wn);
            ov.z = fmaf(ov.z, wo, x.z * wn); ov.w = fmaf(ov.w, wo, x.w * wn);
            m = m_new;
        };
        auto index = [&](int s) { return ((int64_t)(s0 + s) * a.kv_heads + kvh) * G + g; };
        if (coherent) {
            // The merge ends the call, so all loads of a batch of K
            // partitions go out before its first fold (3K pair loads, one
            // round trip); indices past the last partition repeat it and are
            // not folded.
            auto batches = [&](auto kb) {
                constexpr int K = decltype(kb)::value;
                for (int sb = 0; sb < nsplit; sb += K) {
                    float2 ml[K], x0[K], x1[K];
#pragma unroll
                    for (int j = 0; j < K; ++j) {
                        const int64_t idx = index(min(sb + j, nsplit - 1));
                        const float *pa = a.partial_acc + idx * D + d;
                        ml[j] = load_coherent2(a.partial_ml + idx * 2);
                        x0[j] = load_coherent2(pa);
                        x1[j] = load_coherent2(pa + 2);
                    }
#pragma unroll
                    for (int j = 0; j < K; ++j) {
                        if (sb + j < nsplit) fold(ml[j], make_float4(x0[j].x, x0[j].y, x1[j].x, x1[j].y));
                    }
                }
            };
            if (nsplit <= 8) batches(std::integral_constant<int, 8>{});
            else batches(std::integral_constant<int, 16>{});
        } else {
#pragma unroll 8
            for (int s = 0; s < nsplit; ++s) {
                const int64_t idx = index(s);
                fold(*reinterpret_cast<const float2 *>(a.partial_ml + idx * 2),
                     *reinterpret_cast<const float4 *>(a.partial_acc + idx * D + d));
            }
        }
        uint2 packed;
        packed.x = pack_bf16x2(ov.x / l, ov.y / l);
        packed.y = pack_bf16x2(ov.z / l, ov.w / l);
        *reinterpret_cast<uint2 *>(a.out + ((int64_t)b * a.q_heads + qh0 + g) * D + d) = packed;
    }
}

template <int D, int G>
__global__ __launch_bounds__(256) void decode_merge_kernel(DeviceArgs a) {
    const int kvh = blockIdx.x % a.kv_heads;
    const int b = blockIdx.x / a.kv_heads;
    const Tables tab = tables_of(a);
    if (tab.split_begin(b + 1) - tab.split_begin(b) <= 1) return;
    merge_splits<D, G>(a, b, kvh, threadIdx.x, 256, false);
}

// Any-geometry fallback (head_dim not 64/128, or groups outside 1/2/4/8):
// one wavefront per (sequence, query head), 64-token tiles, one token per
// lane for Q.K, dims across lanes for P.V.  Same addressing rule as the fast
// kernel, so dense and paged stay bit-identical here too.
template <bool PAGED>
__global__ __launch_bounds__(64) void decode_generic_kernel(DeviceArgs a, int D) {
    __shared__ float p_lds[64];
    const int lane = threadIdx.x;
    const int b = blockIdx.x / a.q_heads;
    const int qh = blockIdx.x % a.q_heads;
    const int group = a.q_heads / a.kv_heads;
    const int kvh = qh / group;
    const int seq_len = tables_of(a).seq_len(b);
    const float c = a.scale_log2e;
    const uint16_t *q = a.q + ((int64_t)b * a.q_heads + qh) * D;
    auto row_ptr = [&](const uint16_t *cache, int t) -> const uint16_t * {
        if constexpr (PAGED) {
            const int shift = a.page_shift;
            const int page = a.page_table[(int64_t)b * a.pages_per_seq + (t >> shift)];
            return cache + ((((int64_t)page * a.kv_heads + kvh) << shift) + (t & ((1 << shift) - 1))) * D;
        } else {
            return cache + (((int64_t)b * a.seq_stride_tokens + t) * a.kv_heads + kvh) * D;
        }
    };
    float m_run = -INFINITY, l_run = 0.0f;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // dims lane + 64*i, D <= 256
    for (int t0 = 0; t0 < seq_len; t0 += 64) {
        const int t = t0 + lane;
        float s = -INFINITY;
        if (t < seq_len) {
            const uint16_t *kp = row_ptr(a.k, t);
            float dot = 0.0f;
            for (int d = 0; d < D; ++d) dot = fmaf(read_bf16(q[d]), read_bf16(kp[d]), dot);
            s = dot;
        }
        float mx = s;
        for (int mask = 1; mask < 64; mask <<= 1) mx = wave_xor_max(mx, mask);
        const float m_new = fmaxf(m_run, mx);
        const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * c);
        const float p = __builtin_amdgcn_exp2f(fmaf(s, c, -m_new * c));
        float ps = p;
        for (int mask = 1; mask < 64; mask <<= 1) ps = wave_xor_sum(ps, mask);
        l_run = l_run * alpha + ps;
        m_run = m_new;
        p_lds[lane] = p;
        __syncthreads();
        const int n = min(64, seq_len - t0);
        for (int i = 0; i < 4; ++i) acc[i] *= alpha;
        for (int j = 0; j < n; ++j) {
            const uint16_t *vp = row_ptr(a.v, t0 + j);
            const float pj = p_lds[j];
            for (int i = 0; i < 4; ++i) {
                const int d = lane + 64 * i;
                if (d < D) acc[i] = fmaf(pj, read_bf16(vp[d]), acc[i]);
            }
        }
        __syncthreads();
    }
    for (int i = 0; i < 4; ++i) {
        const int d = lane + 64 * i;
        if (d < D) a.out[((int64_t)b * a.q_heads + qh) * D + d] = write_bf16(acc[i] / l_run);
    }
}

template <int D, int G, bool FUSED, bool LIST>
void launch_variant(const DeviceArgs &a, bool paged, bool nt, dim3 grid, hipStream_t stream) {
    const dim3 block(64 * kWaves);
    if (paged && nt)
        hipLaunchKernelGGL((decode_kernel<D, G, true, FUSED, true, LIST>), grid, block, 0, stream, a);
    else if (paged)
        hipLaunchKernelGGL((decode_kernel<D, G, true, FUSED, false, LIST>), grid, block, 0, stream, a);
    else if (nt)
        hipLaunchKernelGGL((decode_kernel<D, G, false, FUSED, true, LIST>), grid, block, 0, stream, a);
    else
        hipLaunchKernelGGL((decode_kernel<D, G, false, FUSED, false, LIST>), grid, block, 0, stream, a);
}

// fused: the last split workgroup of each (sequence, kv head) merges; else a
// decode_merge_kernel launch follows when any sequence has several splits.
template <int D, int G>
hipError_t launch_fast(const DeviceArgs &a, bool paged, bool nt, int total_splits, bool merge, bool fused,
                       hipStream_t stream) {
    // Lists are built for the fused merge only (launch_decode).
    if (fused && a.list_bins)
        launch_variant<D, G, true, true>(a, paged, nt, dim3((unsigned)a.list_bins), stream);
    else if (fused)
        launch_variant<D, G, true, false>(a, paged, nt, dim3((unsigned)(total_splits * a.kv_heads)), stream);
    else
        launch_variant<D, G, false, false>(a, paged, nt, dim3((unsigned)(total_splits * a.kv_heads)), stream);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess || !merge || fused) return err;
    hipLaunchKernelGGL((decode_merge_kernel<D, G>), dim3((unsigned)(a.batch * a.kv_heads)), dim3(256), 0,
                       stream, a);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void zero_i32_kernel(int *p, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0;
}

// Split partials of the allocation-free decode entry point (16 MiB, the
// reference's decode scratch bound, attention_kernel.rs:124-139).  Host code
// never passes `scratch` itself to a kernel: its device address comes from
// hipGetSymbolAddress, per device.
static __device__ __align__(256) unsigned char scratch[kDecodeStaticBytes];

}  // namespace

hipError_t decode_static_scratch(int device, float **ptr) {
    static std::mutex lock;
    static void *address[kMaxDevices] = {};
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> guard(lock);
    if (!address[device]) {
        void *p = nullptr;
        const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess) return err;
        if (!p) return hipErrorInvalidSymbol;
        address[device] = p;
    }
    *ptr = static_cast<float *>(address[device]);
    return hipSuccess;
}

hipError_t launch_zero_i32(int *p, int n, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(zero_i32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, p, n);
    return hipGetLastError();
}

size_t decode_partial_bytes(const DecodeLaunch &l) {
    int64_t splits = 0;
    for (int i = 0; i < l.batch; ++i) splits += decode_splits(l.seq_len[i], l.split_tokens);
    const int group = l.q_heads / l.kv_heads;
    return (size_t)splits * l.kv_heads * group * (l.head_dim + 2) * sizeof(float);
}

int decode_auto_split_tokens(const int32_t *seq_lens, int batch, int kv_heads) {
    // S1 = tokens * kv_heads / 256, a multiple of 256 in [256, 16384] (128
    // for batches too small to fill the CUs): about one workgroup per CU (256
    // on MI355X).  For equal lengths that is the
    // measured best (4,096 tokens for 4 x 32k x 8 kv heads, 1,280 for
    // 8 x 4,224), and it is returned as is.
    //
    // Ragged lengths leave short last partitions beside full ones.  The
    // kernel launches the full partitions first and the last ones longest
    // first; workgroups i and i + 256 start together on one CU, and each later
    // workgroup starts on the CU that frees a slot first.  Two workgroups on a
    // CU measured no faster together than one, so a CU finishes when its
    // total work is done.  Each candidate split from S1 down to S1 / 4 (at
    // most 2,048 workgroups) is scored by the busiest CU under that dispatch
    // (greedy: each later workgroup to the least-loaded CU), counting
    // kWorkgroupCost tokens of fixed cost per workgroup; the lowest score
    // wins, ties keep the larger split.  On five measured batch shapes
    // (ragged and equal) this picks the fastest split of the sweep.
    constexpr int kCus = 256;
    constexpr int64_t kWorkgroupCost = 256;
    constexpr int64_t kMaxWorkgroups = 2048;
    int64_t total = 0;
    bool uniform = true;
    for (int i = 0; i < batch; ++i) {
        total += seq_lens[i];
        uniform &= seq_lens[i] == seq_lens[0];
    }
    int64_t per = (total * kv_heads + kCus - 1) / kCus;
    // A batch too small to give every CU 256 tokens (under 64k tokens x kv
    // heads) takes 128-token splits: one tile per wavefront, 0.9 us faster
    // than 256 at cfg1 (B = 1, T = 1,024, 8 kv heads), while 64-token splits
    // leave half of each workgroup idle and measured slower.
    if (per <= 128) return 128;
    per = (per + 255) / 256 * 256;
    const int s1 = (int)std::min<int64_t>(16384, std::max<int64_t>(256, per));
    if (uniform) return s1;
    const int step = std::max(256, s1 / 16 / 256 * 256);
    int best_split = s1;
    int64_t best_load = INT64_MAX;
    int64_t load[kCus];
    int last_len[kMaxBatch];
    for (int s = s1; s >= std::max(256, s1 / 4); s -= step) {
        int64_t workgroups = 0;
        for (int b = 0; b < batch; ++b) workgroups += (int64_t)decode_splits(seq_lens[b], s) * kv_heads;
        if (workgroups > kMaxWorkgroups && s != s1) continue;
        for (int b = 0; b < batch; ++b) last_len[b] = seq_lens[b] - (decode_splits(seq_lens[b], s) - 1) * s;
        std::sort(last_len, last_len + batch, [](int x, int y) { return x > y; });
        std::fill(load, load + kCus, (int64_t)0);
        // Min-heap of (load, CU) in a fixed array: the choice allocates
        // nothing, so the allocation-free entry point can make it too.
        std::pair<int64_t, int> free_first[kCus];
        const auto later = std::greater<std::pair<int64_t, int>>();
        int64_t wg = 0;
        auto place = [&](int64_t tokens) {
            const int64_t work = tokens + kWorkgroupCost;
            if (wg < 2 * kCus) {
                load[wg % kCus] += work;
                if (wg == 2 * kCus - 1) {
                    for (int c = 0; c < kCus; ++c) free_first[c] = {load[c], c};
                    std::make_heap(free_first, free_first + kCus, later);
                }
            } else {
                std::pop_heap(free_first, free_first + kCus, later);
                auto &top = free_first[kCus - 1];
                load[top.second] = top.first + work;
                top.first = load[top.second];
                std::push_heap(free_first, free_first + kCus, later);
            }
            ++wg;
        };
        for (int b = 0; b < batch; ++b)
            for (int sp = 0; sp + 1 < decode_splits(seq_lens[b], s); ++sp)
                for (int h = 0; h < kv_heads; ++h) place(s);
        for (int b = 0; b < batch; ++b)
            for (int h = 0; h < kv_heads; ++h) place(last_len[b]);
        const int64_t busiest = *std::max_element(load, load + kCus);
        if (busiest < best_load) {
            best_load = busiest;
            best_split = s;
        }
    }
    return best_split;
}

// List mode, for fused-merge launches of more partitions than fit at once
// (two workgroups per CU: 512) and at most kMaxListItems: the partitions,
// longest first (ties in launch order), each go to the list with the least
// work so far (tokens plus kListItemCost per partition for its first loads,
// combine and publication; ties to the lower list), and the launch runs 512
// workgroups, one per list.  With one partition per workgroup, a CU gets the
// next workgroup whenever one of its two slots frees, and which partitions
// share a CU follows from that order: the measured per-CU work of cfg3
// (640 partitions) spread from 121 to 175 32-token tiles around a mean of
// 144, and the call ended with the busiest CUs.  Packed lists give every
// pair of lists on a CU nearly the same work.  Fixed-size arrays: the
// allocation-free entry point plans too.
constexpr int64_t kListItemCost = 256;

// Host view of the launch tables, in the layout of DeviceArgs::words and
// DeviceArgs::halves (or of their device copy).
struct TableWriter {
    int32_t *w;
    uint16_t *h;
    int batch, bins;
    int32_t &seq_len(int b) { return w[b]; }
    int32_t &split_begin(int b) { return w[batch + b]; }
    int32_t &full_begin(int b) { return w[2 * batch + 1 + b]; }
    uint16_t &last_order(int i) { return h[i]; }
    uint16_t &bin_start(int i) { return h[batch + i]; }
    uint16_t &list(int i) { return h[batch + bins + 1 + i]; }
};

void plan_lists(TableWriter &t, int total, int kvh, int split_tokens) {
    const int items = total * kvh;
    const int full = t.full_begin(t.batch);
    std::pair<int, int> order[kMaxListItems];  // (tokens, launch index)
    for (int i = 0; i < items; ++i) {
        const int sg = i / kvh;
        int tokens = split_tokens;
        if (sg >= full) {
            const int b = t.last_order(sg - full);
            tokens = t.seq_len(b) - (t.split_begin(b + 1) - t.split_begin(b) - 1) * split_tokens;
        }
        order[i] = {tokens, i};
    }
    // Longest first, ties in launch order (the order a stable sort keeps);
    // std::sort with the index as tie-break allocates nothing, as the
    // allocation-free entry point needs.
    std::sort(order, order + items, [](const std::pair<int, int> &x, const std::pair<int, int> &y) {
        return x.first != y.first ? x.first > y.first : x.second < y.second;
    });
    std::pair<int64_t, int> heap[kListBins];  // (work, list): least work on top
    for (int w = 0; w < kListBins; ++w) heap[w] = {0, w};
    const auto later = std::greater<std::pair<int64_t, int>>();
    int16_t bin_of[kMaxListItems];
    int count[kListBins] = {};
    for (int i = 0; i < items; ++i) {
        std::pop_heap(heap, heap + kListBins, later);
        auto &top = heap[kListBins - 1];
        bin_of[i] = (int16_t)top.second;
        ++count[top.second];
        top.first += order[i].first + kListItemCost;
        std::push_heap(heap, heap + kListBins, later);
    }
    int cursor[kListBins];
    t.bin_start(0) = 0;
    for (int w = 0; w < kListBins; ++w) {
        cursor[w] = t.bin_start(w);
        t.bin_start(w + 1) = (uint16_t)(t.bin_start(w) + count[w]);
    }
    for (int i = 0; i < items; ++i) t.list(cursor[bin_of[i]]++) = (uint16_t)order[i].second;
}

// Layout of a launch's tables: partitions in all, list mode, and where they
// go (the kernel arguments, or a device copy of word_bytes of words followed
// by half_bytes of halves).
struct TablePlan {
    int total = 0;
    bool lists = false;
    bool inline_args = true;
    size_t word_bytes = 0, half_bytes = 0;
};

TablePlan table_plan(const DecodeLaunch &l) {
    TablePlan p;
    for (int i = 0; i < l.batch; ++i) p.total += decode_splits(l.seq_len[i], l.split_tokens);
    const int64_t items = (int64_t)p.total * l.kv_heads;
    p.lists = decode_fast_path(l.head_dim, l.q_heads / l.kv_heads) && !l.separate_merge && items > kListBins &&
              items <= kMaxListItems;
    const int64_t halves = l.batch + (p.lists ? kListBins + 1 + items : 0);
    p.inline_args = l.batch <= kInlineBatch && halves <= kInlineHalves;
    p.word_bytes = ((size_t)(3 * l.batch + 2) * 4 + 255) & ~(size_t)255;
    p.half_bytes = ((size_t)halves * 2 + 3) & ~(size_t)3;
    return p;
}

size_t decode_table_bytes(const DecodeLaunch &l) {
    const TablePlan p = table_plan(l);
    return p.inline_args ? 0 : p.word_bytes + p.half_bytes;
}

bool decode_fast_path(int head_dim, int group) {
    return (head_dim == 64 || head_dim == 128) &&
           (group == 1 || group == 2 || group == 4 || group == 8 || group == 16);
}

namespace {

hipError_t launch_kernels(const DeviceArgs &a, const DecodeLaunch &l, int total, bool merge, int64_t kv_tokens,
                          hipStream_t stream) {
    const int group = l.q_heads / l.kv_heads;
    const bool nt = kv_tokens * l.kv_heads * l.head_dim * 2 * 2 >= kNonTemporalBytes;
    if (!decode_fast_path(l.head_dim, group)) {
        const dim3 grid((unsigned)(l.batch * l.q_heads));
        if (l.paged)
            hipLaunchKernelGGL((decode_generic_kernel<true>), grid, dim3(64), 0, stream, a, l.head_dim);
        else
            hipLaunchKernelGGL((decode_generic_kernel<false>), grid, dim3(64), 0, stream, a, l.head_dim);
        return hipGetLastError();
    }
#define MSLIM_DECODE_CASE(DD, GG) \
    if (l.head_dim == DD && group == GG) \
        return launch_fast<DD, GG>(a, l.paged, nt, total, merge, !l.separate_merge, stream);
    MSLIM_DECODE_CASE(128, 16)
    MSLIM_DECODE_CASE(128, 8)
    MSLIM_DECODE_CASE(128, 4)
    MSLIM_DECODE_CASE(128, 2)
    MSLIM_DECODE_CASE(128, 1)
    MSLIM_DECODE_CASE(64, 16)
    MSLIM_DECODE_CASE(64, 8)
    MSLIM_DECODE_CASE(64, 4)
    MSLIM_DECODE_CASE(64, 2)
    MSLIM_DECODE_CASE(64, 1)
#undef MSLIM_DECODE_CASE
    return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_decode(const DecodeLaunch &l, hipStream_t stream) {
    DeviceArgs a{};
    a.q = l.q; a.k = l.k; a.v = l.v; a.out = l.out;
    a.partial_ml = l.partial_ml; a.partial_acc = l.partial_acc;
    a.counters = l.counters;
    a.page_table = l.page_table;
    a.seq_stride_tokens = l.seq_stride_tokens;
    a.pages_per_seq = l.pages_per_seq;
    a.page_shift = 0;
    if (l.paged) {
        while ((1 << a.page_shift) < l.page_tokens) ++a.page_shift;
    }
    a.batch = l.batch; a.q_heads = l.q_heads; a.kv_heads = l.kv_heads;
    a.split_tokens = l.split_tokens;
    a.scale_log2e = l.scale * kLog2e;
    const TablePlan plan = table_plan(l);
    TableWriter t{a.words, a.halves, l.batch, plan.lists ? kListBins : 0};
    if (!plan.inline_args) {
        if (!l.tables || l.tables->bytes < plan.word_bytes + plan.half_bytes) return hipErrorInvalidValue;
        t.w = static_cast<int32_t *>(l.tables->host);
        t.h = reinterpret_cast<uint16_t *>(static_cast<char *>(l.tables->host) + plan.word_bytes);
    }
    int total = 0;
    bool merge = false;
    int64_t kv_tokens = 0;
    for (int i = 0; i < l.batch; ++i) {
        kv_tokens += l.seq_len[i];
        t.seq_len(i) = l.seq_len[i];
        t.split_begin(i) = total;
        const int n = decode_splits(l.seq_len[i], l.split_tokens);
        merge |= n > 1;
        total += n;
    }
    t.split_begin(l.batch) = total;
    int full = 0;
    for (int i = 0; i < l.batch; ++i) {
        t.full_begin(i) = full;
        full += t.split_begin(i + 1) - t.split_begin(i) - 1;
        t.last_order(i) = (uint16_t)i;
    }
    t.full_begin(l.batch) = full;
    auto last_len = [&](int i) {
        return l.seq_len[i] - (t.split_begin(i + 1) - t.split_begin(i) - 1) * l.split_tokens;
    };
    // Longest last partition first, ties in sequence order; no allocation
    // (std::stable_sort may take a temporary buffer from the heap).
    std::sort(t.h, t.h + l.batch, [&](uint16_t x, uint16_t y) {
        const int lx = last_len(x), ly = last_len(y);
        return lx != ly ? lx > ly : x < y;
    });
    if (plan.lists) {
        plan_lists(t, total, l.kv_heads, l.split_tokens);
        a.list_bins = kListBins;
    }
    if (!plan.inline_args) {
        const hipError_t err = hipMemcpyAsync(l.tables->device, l.tables->host, plan.word_bytes + plan.half_bytes,
                                              hipMemcpyHostToDevice, stream);
        if (err != hipSuccess) return err;
        a.ext_words = (uint64_t)reinterpret_cast<uintptr_t>(l.tables->device);
        a.ext_halves = a.ext_words + plan.word_bytes;
    }
    const hipError_t err = launch_kernels(a, l, total, merge, kv_tokens, stream);
    // The host and device copies of the tables are free again once the
    // launches are done.
    if (err == hipSuccess && !plan.inline_args) return hipEventRecord(l.tables->done, stream);
    return err;
}

}  // namespace mslim
