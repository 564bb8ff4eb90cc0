// Causal GQA prefill attention (queries >= 1 after `prior` cached tokens).
//
// Replaces llm_prefill_qk / softmax / pv (gpu_llm.cl:462-541) and the tiled
// kernel's multi-query modes (tiled_attention.cl:9-129) with a flash-style
// kernel on gfx950 MFMA:
//   * a workgroup of 4 wavefronts owns 32 query rows for 4 query heads of one
//     GQA group (or 64 rows x 2 heads, 128 rows x 1 head for groups 2 and 1),
//     so every K/V tile staged in LDS is reused by all its heads;
//   * each wavefront computes S^T = K . Q^T with v_mfma_f32_32x32x16_bf16
//     (keys as M, its 32 query rows as N).  The S^T accumulator already has
//     one query row per lane, which is exactly the P^T operand layout of
//     O^T = V^T . P^T, so P never leaves registers and the row softmax, the
//     rescale of O and the causal mask are per-lane operations;
//   * V is staged transposed ([dim][key]) in LDS so its MFMA operand is two
//     8-byte LDS reads per lane;
//   * key tiles above a wavefront's diagonal are skipped, and workgroups
//     start from the longest (last) row blocks.
#include "common.hpp"
#include "kernels.hpp"

namespace mslim {

namespace {

struct PrefillArgs {
    const uint16_t *q, *k, *v;
    uint16_t *out;
    int queries, prior, history;
    int q_heads, kv_heads;
    float scale_log2e;
};

constexpr int kBN = 64;  // keys per LDS tile

template <int D>
struct PrefillLds {
    static constexpr int KSTR = D + 8;    // K tile row stride (elements)
    static constexpr int VSTR = kBN + 8;  // transposed V row stride (elements)
    uint16_t k[kBN * KSTR];
    uint16_t vt[D * VSTR];
};

// HW = query heads per workgroup; the 4 wavefronts cover HW heads x (4/HW)
// row blocks of 32 rows.
template <int D, int HW>
__global__ __launch_bounds__(256, 2) void prefill_mfma_kernel(PrefillArgs a) {
    constexpr int KS = D / 16;           // QK k-steps (16 dims each)
    constexpr int MT = D / 32;           // O^T row tiles (32 dims each)
    constexpr int RW = 32 * (4 / HW);    // query rows per workgroup
    constexpr int KCH = kBN * D / 8 / 256;  // 16-byte K chunks per thread
    constexpr int VCH = (kBN / 2) * (D / 8) / 256;  // V key-pair items per thread
    using L = PrefillLds<D>;
    __shared__ L lds;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int col = lane & 31;  // query row within the wavefront's block
    const int half = lane >> 5;

    const int group = a.q_heads / a.kv_heads;
    const int subgroups = group / HW;
    const int kvh = blockIdx.y / subgroups;
    const int head = kvh * group + (blockIdx.y % subgroups) * HW + wave % HW;
    const int nrb = (a.queries + RW - 1) / RW;
    const int r0 = (nrb - 1 - (int)blockIdx.x) * RW;   // longest rows first
    const int rw0 = r0 + (wave / HW) * 32;              // this wavefront's first row
    const int row = rw0 + col;
    const int row_abs = a.prior + row;
    const float c = a.scale_log2e;

    // Q^T as the B operand: lane holds row `col`, dims j*16 + half*8 .. +8.
    bf16x8_t qf[KS];
    {
        const int qrow = min(row, a.queries - 1);
        const uint16_t *qp = a.q + ((int64_t)qrow * a.q_heads + head) * D + half * 8;
#pragma unroll
        for (int j = 0; j < KS; ++j) qf[j] = *reinterpret_cast<const bf16x8_t *>(qp + j * 16);
    }

    const int key_end = min(a.history, a.prior + r0 + RW);  // keys this workgroup needs
    const int nkt = (key_end + kBN - 1) / kBN;
    const int wave_last_key = a.prior + rw0 + 31;

    // Global -> register prefetch of one K/V tile.
    uint4 kreg[KCH];
    uint4 vreg[VCH][2];
    auto fetch = [&](int kt) {
#pragma unroll
        for (int i = 0; i < KCH; ++i) {
            const int chunk = tid + 256 * i;
            const int key = kt * kBN + chunk / (D / 8);
            const int dc = chunk % (D / 8);
            kreg[i] = key < a.history
                          ? *reinterpret_cast<const uint4 *>(
                                a.k + ((int64_t)key * a.kv_heads + kvh) * D + dc * 8)
                          : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < VCH; ++i) {
            const int item = tid + 256 * i;
            const int pair = item % (kBN / 2);
            const int dc = item / (kBN / 2);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int key = kt * kBN + 2 * pair + h;
                vreg[i][h] = key < a.history
                                 ? *reinterpret_cast<const uint4 *>(
                                       a.v + ((int64_t)key * a.kv_heads + kvh) * D + dc * 8)
                                 : make_uint4(0, 0, 0, 0);
            }
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int i = 0; i < KCH; ++i) {
            const int chunk = tid + 256 * i;
            const int key = chunk / (D / 8);
            const int dc = chunk % (D / 8);
            *reinterpret_cast<uint4 *>(&lds.k[key * L::KSTR + dc * 8]) = kreg[i];
        }
#pragma unroll
        for (int i = 0; i < VCH; ++i) {
            const int item = tid + 256 * i;
            const int pair = item % (kBN / 2);
            const int dc = item / (kBN / 2);
            const uint32_t a0[4] = {vreg[i][0].x, vreg[i][0].y, vreg[i][0].z, vreg[i][0].w};
            const uint32_t a1[4] = {vreg[i][1].x, vreg[i][1].y, vreg[i][1].z, vreg[i][1].w};
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                // dims 2w and 2w+1 of keys 2*pair and 2*pair+1
                const uint32_t lo = (a0[w] & 0xffffu) | (a1[w] << 16);
                const uint32_t hi = (a0[w] >> 16) | (a1[w] & 0xffff0000u);
                const int d = dc * 8 + 2 * w;
                *reinterpret_cast<uint32_t *>(&lds.vt[d * L::VSTR + 2 * pair]) = lo;
                *reinterpret_cast<uint32_t *>(&lds.vt[(d + 1) * L::VSTR + 2 * pair]) = hi;
            }
        }
    };

    floatx16_t o[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[mt][r] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;

    fetch(0);
    for (int kt = 0; kt < nkt; ++kt) {
        __syncthreads();
        stage();
        __syncthreads();
        if (kt + 1 < nkt) fetch(kt + 1);
        if (kt * kBN > wave_last_key) continue;  // tile entirely above this wavefront's rows

        // S^T = K (keys x D) . Q^T (D x rows), two 32-key blocks.
        floatx16_t s[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (int r = 0; r < 16; ++r) s[kb][r] = 0.0f;
            const uint16_t *kp = &lds.k[(kb * 32 + col) * L::KSTR + half * 8];
#pragma unroll
            for (int j = 0; j < KS; ++j) {
                const bf16x8_t af = *reinterpret_cast<const bf16x8_t *>(kp + j * 16);
                s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, qf[j], s[kb], 0, 0, 0);
            }
        }
        // s[kb][r] is the score of row `row` against key
        // kt*64 + kb*32 + (r/4)*8 + half*4 + r%4.
        if (kt * kBN + kBN - 1 > a.prior + rw0) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = kt * kBN + kb * 32 + (r >> 2) * 8 + half * 4 + (r & 3);
                    if (key > row_abs) s[kb][r] = -INFINITY;
                }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
        mx = wave_xor_max(mx, 32);
        const float m_new = fmaxf(m_run, mx);
        const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * c);
        const float mc = m_new * c;
        float psum = 0.0f;
        bf16x8_t pf[2][2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = __builtin_amdgcn_exp2f(fmaf(s[kb][r], c, -mc));
                psum += p;
                pf[kb][r >> 3][r & 7] = (__bf16)p;
            }
        l_run = l_run * alpha + psum;
        m_run = m_new;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[mt][r] *= alpha;

        // O^T (dims x rows) += V^T (dims x keys) . P^T (keys x rows).
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const uint16_t *vp = &lds.vt[(mt * 32 + col) * L::VSTR + half * 4];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const uint2 lo = *reinterpret_cast<const uint2 *>(vp + kb * 32 + 16 * t);
                    const uint2 hi = *reinterpret_cast<const uint2 *>(vp + kb * 32 + 16 * t + 8);
                    const uint4 packed = make_uint4(lo.x, lo.y, hi.x, hi.y);
                    const bf16x8_t af = __builtin_bit_cast(bf16x8_t, packed);
                    o[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, pf[kb][t], o[mt], 0, 0, 0);
                }
        }
    }

    const float l = l_run + __shfl_xor(l_run, 32, 64);
    if (row < a.queries) {
        uint16_t *op = a.out + ((int64_t)row * a.q_heads + head) * D;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const int d = mt * 32 + r4 * 8 + half * 4;
                uint2 w;
                w.x = pack_bf16x2(o[mt][r4 * 4 + 0] / l, o[mt][r4 * 4 + 1] / l);
                w.y = pack_bf16x2(o[mt][r4 * 4 + 2] / l, o[mt][r4 * 4 + 3] / l);
                *reinterpret_cast<uint2 *>(op + d) = w;
            }
    }
}

// Any-geometry fallback: one wavefront per (query row, head), 64-key tiles.
__global__ __launch_bounds__(64) void prefill_generic_kernel(PrefillArgs a, int D) {
    __shared__ float p_lds[64];
    const int lane = threadIdx.x;
    const int row = blockIdx.x / a.q_heads;
    const int qh = blockIdx.x % a.q_heads;
    const int kvh = qh / (a.q_heads / a.kv_heads);
    const int valid = a.prior + row + 1;
    const float c = a.scale_log2e;
    const uint16_t *q = a.q + ((int64_t)row * a.q_heads + qh) * D;
    float m_run = -INFINITY, l_run = 0.0f;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int t0 = 0; t0 < valid; t0 += 64) {
        const int t = t0 + lane;
        float s = -INFINITY;
        if (t < valid) {
            const uint16_t *kp = a.k + ((int64_t)t * a.kv_heads + kvh) * D;
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
        const int n = min(64, valid - t0);
        for (int i = 0; i < 4; ++i) acc[i] *= alpha;
        for (int j = 0; j < n; ++j) {
            const uint16_t *vp = a.v + ((int64_t)(t0 + j) * a.kv_heads + kvh) * D;
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
        if (d < D) a.out[((int64_t)row * a.q_heads + qh) * D + d] = write_bf16(acc[i] / l_run);
    }
}

template <int D, int HW>
hipError_t launch_mfma(const PrefillArgs &a, hipStream_t stream) {
    constexpr int RW = 32 * (4 / HW);
    const int group = a.q_heads / a.kv_heads;
    const dim3 grid((unsigned)((a.queries + RW - 1) / RW), (unsigned)(a.kv_heads * (group / HW)));
    hipLaunchKernelGGL((prefill_mfma_kernel<D, HW>), grid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace

bool prefill_fast_path(int head_dim, int group) {
    return (head_dim == 64 || head_dim == 128) && (group == 1 || group == 2 || group % 4 == 0);
}

hipError_t launch_prefill(const PrefillLaunch &l, hipStream_t stream) {
    PrefillArgs a{};
    a.q = l.q; a.k = l.k; a.v = l.v; a.out = l.out;
    a.queries = l.queries; a.prior = l.prior; a.history = l.prior + l.queries;
    a.q_heads = l.q_heads; a.kv_heads = l.kv_heads;
    a.scale_log2e = l.scale * kLog2e;
    const int group = l.q_heads / l.kv_heads;
    if (!prefill_fast_path(l.head_dim, group)) {
        hipLaunchKernelGGL(prefill_generic_kernel, dim3((unsigned)(l.queries * l.q_heads)), dim3(64), 0,
                           stream, a, l.head_dim);
        return hipGetLastError();
    }
    const int hw = group >= 4 ? 4 : group;
    if (l.head_dim == 128) {
        if (hw == 4) return launch_mfma<128, 4>(a, stream);
        if (hw == 2) return launch_mfma<128, 2>(a, stream);
        return launch_mfma<128, 1>(a, stream);
    }
    if (hw == 4) return launch_mfma<64, 4>(a, stream);
    if (hw == 2) return launch_mfma<64, 2>(a, stream);
    return launch_mfma<64, 1>(a, stream);
}

}  // namespace mslim
