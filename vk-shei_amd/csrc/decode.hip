// Single-token GQA decode over a BF16 K/V cache, dense or ColdStore-paged.
//
// Replaces llm_attention_qk / softmax / pv (gpu_llm.cl:150-212),
// llm_exact_hot_fused_attention (:975-1025), the ColdStore-V PV stage
// (:280-322) and the split-KV mode of mslim_attention_tiled / _merge
// (tiled_attention.cl:9-155).
//
// Decode reads every K and V byte once, so it is an HBM stream.  One
// wavefront owns one (sequence, kv head, split) partition of `split_tokens`
// logical tokens and serves all G query heads of the GQA group from the same
// K/V bytes:
//   * Q.K^T for the group runs on v_mfma_f32_16x16x32_bf16 with the 16 tokens
//     of a block as M and the (zero padded) G heads as N.  Each lane loads
//     64 contiguous bytes of one K row as its A operand, so a 16-token block
//     is four 128-bit loads per lane and no K byte passes through LDS.
//   * the online softmax max / sum run on 64-lane butterflies;
//   * P.V accumulates in fp32 on the VALU from 128-bit V loads (16 lanes per
//     256-byte row for D = 128), with P broadcast through a 2 KB LDS tile;
//   * the next 32-token tile's K and V are in flight while the current one is
//     computed.
// Partitions are fixed by logical token index, and the paged and dense
// variants differ only in how a 16-token block's base address is formed, so
// both produce bit-identical outputs (the reference's dense == ColdStore
// invariant, gpu_llm/mod.rs:2993-3048).
#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>

namespace mslim {

namespace {

struct DeviceArgs {
    const uint16_t *q, *k, *v;
    uint16_t *out;
    float *partial_ml;
    float *partial_acc;
    const int32_t *page_table;
    int64_t seq_stride_tokens;
    int pages_per_seq, page_shift;
    int batch, q_heads, kv_heads;
    int split_tokens;
    float scale_log2e;
    int seq_len[kMaxBatch];
    int split_begin[kMaxBatch + 1];
};

// Base of the 16-token block starting at logical token t0 (a multiple of 16)
// and the element stride between its rows.
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

template <int D, bool PAGED>
__device__ __forceinline__ int64_t row_stride(const DeviceArgs &a) {
    if constexpr (PAGED) return D;
    else return (int64_t)a.kv_heads * D;
}

// Sequence owning global split index sg (uniform scalar search).
__device__ __forceinline__ int sequence_of(const DeviceArgs &a, int sg) {
    int b = 0;
    while (b + 1 < a.batch && a.split_begin[b + 1] <= sg) ++b;
    return b;
}

template <int D, int G, bool PAGED>
__global__ __launch_bounds__(64) void decode_split_kernel(DeviceArgs a) {
    constexpr int KS = D / 32;        // MFMA k-steps per 16-token block
    constexpr int LPR = D / 8;        // lanes per V row (8 BF16 per lane)
    constexpr int RPI = 64 / LPR;     // V rows per load instruction
    constexpr int NV = 32 / RPI;      // V loads per 32-token tile
    constexpr int GP = G < 4 ? 4 : G; // LDS row of P, float4 aligned

    __shared__ float p_lds[2][32][GP];
    __shared__ float alpha_lds[2][GP];

    const int lane = threadIdx.x;
    const int row16 = lane & 15;
    const int grp = lane >> 4;
    const int kvh = blockIdx.x % a.kv_heads;
    const int sg = blockIdx.x / a.kv_heads;
    const int b = sequence_of(a, sg);
    const int split = sg - a.split_begin[b];
    const int nsplit = a.split_begin[b + 1] - a.split_begin[b];
    const int seq_len = a.seq_len[b];
    const int begin = split * a.split_tokens;
    const int end = min(seq_len, begin + a.split_tokens);
    const int qh0 = kvh * G;
    const float c = a.scale_log2e;
    const int64_t rs = row_stride<D, PAGED>(a);

    // Q as the B operand: lane holds head row16, dims j*32 + grp*8 .. +8.
    bf16x8_t qf[KS];
#pragma unroll
    for (int j = 0; j < KS; ++j) {
        if (row16 < G) {
            qf[j] = *reinterpret_cast<const bf16x8_t *>(
                a.q + ((int64_t)b * a.q_heads + qh0 + row16) * D + j * 32 + grp * 8);
        } else {
            qf[j] = bf16x8_t{};
        }
    }

    // Tile registers: K in MFMA A layout, V in VALU layout.
    bf16x8_t kr[2][KS];
    uint4 vr[NV];

    auto load_tile = [&](int t0, bf16x8_t (&kd)[2][KS], uint4 (&vd)[NV]) {
        const bool tail = t0 + 32 > end;
        const int last = end - 1;
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            int bt = t0 + blk * 16;
            int row = row16;
            if (tail) {
                const int bt_c = min(bt, last & ~15);
                row = min(bt + row16, last) - bt_c;
                bt = bt_c;
            }
            const uint16_t *p = block_base<D, PAGED>(a, a.k, b, kvh, bt) + row * rs + grp * 8;
#pragma unroll
            for (int j = 0; j < KS; ++j) kd[blk][j] = *reinterpret_cast<const bf16x8_t *>(p + j * 32);
        }
#pragma unroll
        for (int r = 0; r < NV; ++r) {
            const int trow = r * RPI + lane / LPR;  // 0..31 within the tile
            int bt = t0 + (trow & 16);
            int row = trow & 15;
            if (tail) {
                const int bt_c = min(bt, last & ~15);
                row = min(bt + row, last) - bt_c;
                bt = bt_c;
            }
            const uint16_t *p = block_base<D, PAGED>(a, a.v, b, kvh, bt) + row * rs + (lane % LPR) * 8;
            vd[r] = *reinterpret_cast<const uint4 *>(p);
        }
    };

    float m_run = -INFINITY;
    float l_run = 0.0f;
    float acc[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] = 0.0f;

    const int ntiles = (end - begin + 31) >> 5;
    load_tile(begin, kr, vr);
    for (int it = 0; it < ntiles; ++it) {
        const int t0 = begin + it * 32;
        const int buf = it & 1;
        bf16x8_t kn[2][KS];
        uint4 vn[NV];
        if (it + 1 < ntiles) load_tile(t0 + 32, kn, vn);

        // S^T block = K (16 tokens x D) . Q^T (D x 16 heads).
        floatx4_t s[2];
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            s[blk] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < KS; ++j)
                s[blk] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kr[blk][j], qf[j], s[blk], 0, 0, 0);
        }
        // Lane holds head row16, tokens t0 + blk*16 + grp*4 + i.
        if (t0 + 32 > end) {
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
        float psum = 0.0f;
#pragma unroll
        for (int blk = 0; blk < 2; ++blk)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float p = __builtin_amdgcn_exp2f(fmaf(s[blk][i], c, -mc));
                psum += p;
                if (row16 < G) p_lds[buf][blk * 16 + grp * 4 + i][row16] = p;
            }
        l_run = l_run * alpha + psum;
        m_run = m_new;
        if (grp == 0 && row16 < G) alpha_lds[buf][row16] = alpha;
        __syncthreads();

        float al[GP];
#pragma unroll
        for (int g4 = 0; g4 < GP; g4 += 4) {
            const float4 t = *reinterpret_cast<const float4 *>(&alpha_lds[buf][g4]);
            al[g4] = t.x; al[g4 + 1] = t.y; al[g4 + 2] = t.z; al[g4 + 3] = t.w;
        }
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[g][e] *= al[g];

#pragma unroll
        for (int r = 0; r < NV; ++r) {
            const int trow = r * RPI + lane / LPR;
            float p[GP];
#pragma unroll
            for (int g4 = 0; g4 < GP; g4 += 4) {
                const float4 t = *reinterpret_cast<const float4 *>(&p_lds[buf][trow][g4]);
                p[g4] = t.x; p[g4 + 1] = t.y; p[g4 + 2] = t.z; p[g4 + 3] = t.w;
            }
            const uint4 w = vr[r];
            const float v[8] = {bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y),
                                bf16_lo(w.z), bf16_hi(w.z), bf16_lo(w.w), bf16_hi(w.w)};
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(p[g], v[e], acc[g][e]);
        }

#pragma unroll
        for (int blk = 0; blk < 2; ++blk)
#pragma unroll
            for (int j = 0; j < KS; ++j) kr[blk][j] = kn[blk][j];
#pragma unroll
        for (int r = 0; r < NV; ++r) vr[r] = vn[r];
    }

    // Combine the four lane groups: l over groups of the same head, acc over
    // lanes holding the same 8 dims of different token rows.
    l_run = wave_xor_sum(l_run, 16);
    l_run = wave_xor_sum(l_run, 32);
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
#pragma unroll
            for (int mask = LPR; mask < 64; mask <<= 1) acc[g][e] = wave_xor_sum(acc[g][e], mask);
        }

    const int chunk = lane % LPR;
    const int slot = lane / LPR;
    if (nsplit == 1) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float l = __shfl(l_run, g, 64);
            if (slot == g % RPI) {
                uint4 o;
                o.x = pack_bf16x2(acc[g][0] / l, acc[g][1] / l);
                o.y = pack_bf16x2(acc[g][2] / l, acc[g][3] / l);
                o.z = pack_bf16x2(acc[g][4] / l, acc[g][5] / l);
                o.w = pack_bf16x2(acc[g][6] / l, acc[g][7] / l);
                *reinterpret_cast<uint4 *>(a.out + ((int64_t)b * a.q_heads + qh0 + g) * D + chunk * 8) = o;
            }
        }
    } else {
        const int64_t base = ((int64_t)sg * a.kv_heads + kvh) * G;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            if (slot == g % RPI) {
                float *dst = a.partial_acc + (base + g) * D + chunk * 8;
                *reinterpret_cast<float4 *>(dst) = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
                *reinterpret_cast<float4 *>(dst + 4) = make_float4(acc[g][4], acc[g][5], acc[g][6], acc[g][7]);
            }
        }
        if (lane < G) {
            *reinterpret_cast<float2 *>(a.partial_ml + (base + lane) * 2) = make_float2(m_run, l_run);
        }
    }
}

// Fixed-order log-sum-exp merge of split partials (the deterministic
// counterpart of mslim_attention_merge, tiled_attention.cl:131-155).
template <int D>
__global__ __launch_bounds__(64) void decode_merge_kernel(DeviceArgs a) {
    const int b = blockIdx.x / a.q_heads;
    const int qh = blockIdx.x % a.q_heads;
    const int nsplit = a.split_begin[b + 1] - a.split_begin[b];
    if (nsplit <= 1) return;
    const int group = a.q_heads / a.kv_heads;
    const int kvh = qh / group, g = qh % group;
    const float c = a.scale_log2e;
    const int s0 = a.split_begin[b];
    auto idx = [&](int s) { return ((int64_t)(s0 + s) * a.kv_heads + kvh) * group + g; };
    float m = -INFINITY;
    for (int s = 0; s < nsplit; ++s) m = fmaxf(m, a.partial_ml[idx(s) * 2]);
    float l = 0.0f;
    for (int s = 0; s < nsplit; ++s) {
        const float w = __builtin_amdgcn_exp2f((a.partial_ml[idx(s) * 2] - m) * c);
        l = fmaf(a.partial_ml[idx(s) * 2 + 1], w, l);
    }
    for (int d = threadIdx.x; d < D; d += 64) {
        float o = 0.0f;
        for (int s = 0; s < nsplit; ++s) {
            const float w = __builtin_amdgcn_exp2f((a.partial_ml[idx(s) * 2] - m) * c);
            o = fmaf(a.partial_acc[idx(s) * D + d], w, o);
        }
        a.out[((int64_t)b * a.q_heads + qh) * D + d] = write_bf16(o / l);
    }
}

// Any-geometry fallback (head_dim not a multiple of 32, or groups above 8):
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
    const int seq_len = a.seq_len[b];
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

template <int D, int G>
hipError_t launch_fast(const DeviceArgs &a, bool paged, int total_splits, bool merge,
                       hipStream_t stream) {
    const dim3 grid((unsigned)(total_splits * a.kv_heads));
    if (paged) {
        hipLaunchKernelGGL((decode_split_kernel<D, G, true>), grid, dim3(64), 0, stream, a);
    } else {
        hipLaunchKernelGGL((decode_split_kernel<D, G, false>), grid, dim3(64), 0, stream, a);
    }
    hipError_t err = hipGetLastError();
    if (err != hipSuccess || !merge) return err;
    hipLaunchKernelGGL((decode_merge_kernel<D>), dim3((unsigned)(a.batch * a.q_heads)), dim3(64), 0,
                       stream, a);
    return hipGetLastError();
}

}  // namespace

int decode_auto_split_tokens(const int32_t *seq_lens, int batch, int kv_heads) {
    int64_t total = 0;
    for (int i = 0; i < batch; ++i) total += seq_lens[i];
    int64_t per = (total * kv_heads + 2047) / 2048;
    per = (per + 63) / 64 * 64;
    return (int)std::min<int64_t>(4096, std::max<int64_t>(64, per));
}

bool decode_fast_path(int head_dim, int group) {
    return (head_dim == 64 || head_dim == 128) &&
           (group == 1 || group == 2 || group == 4 || group == 8);
}

hipError_t launch_decode(const DecodeLaunch &l, hipStream_t stream) {
    DeviceArgs a{};
    a.q = l.q; a.k = l.k; a.v = l.v; a.out = l.out;
    a.partial_ml = l.partial_ml; a.partial_acc = l.partial_acc;
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
    int total = 0;
    bool merge = false;
    for (int i = 0; i < l.batch; ++i) {
        a.seq_len[i] = l.seq_len[i];
        a.split_begin[i] = total;
        const int s = decode_splits(l.seq_len[i], l.split_tokens);
        merge |= s > 1;
        total += s;
    }
    a.split_begin[l.batch] = total;
    const int group = l.q_heads / l.kv_heads;
    if (!decode_fast_path(l.head_dim, group)) {
        const dim3 grid((unsigned)(l.batch * l.q_heads));
        if (l.paged)
            hipLaunchKernelGGL((decode_generic_kernel<true>), grid, dim3(64), 0, stream, a, l.head_dim);
        else
            hipLaunchKernelGGL((decode_generic_kernel<false>), grid, dim3(64), 0, stream, a, l.head_dim);
        return hipGetLastError();
    }
#define MSLIM_DECODE_CASE(DD, GG) \
    if (l.head_dim == DD && group == GG) return launch_fast<DD, GG>(a, l.paged, total, merge, stream);
    MSLIM_DECODE_CASE(128, 8)
    MSLIM_DECODE_CASE(128, 4)
    MSLIM_DECODE_CASE(128, 2)
    MSLIM_DECODE_CASE(128, 1)
    MSLIM_DECODE_CASE(64, 8)
    MSLIM_DECODE_CASE(64, 4)
    MSLIM_DECODE_CASE(64, 2)
    MSLIM_DECODE_CASE(64, 1)
#undef MSLIM_DECODE_CASE
    return hipErrorInvalidValue;
}

}  // namespace mslim
