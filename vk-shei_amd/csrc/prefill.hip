// Causal GQA prefill attention (queries >= 1 after `prior` cached tokens).
//
// Replaces llm_prefill_qk / softmax / pv (gpu_llm.cl:462-541) and the tiled
// kernel's multi-query modes (tiled_attention.cl:9-129) with a flash-style
// kernel on gfx950 MFMA:
//   * a workgroup of 8 wavefronts owns 32 query rows for 8 query heads of one
//     GQA group (or 64 rows x 4 heads, 128 x 2, 256 x 1 for smaller groups),
//     so every 64-key K/V tile staged in LDS serves all its heads;
//   * K and V tiles move HBM -> LDS with global_load_lds_dwordx4 (no VGPR
//     staging) into a two-stage ring, one barrier per tile.  Each lane picks
//     its source chunk so that rows land XOR-swizzled in LDS;
//   * each wavefront computes S^T = K . Q^T on v_mfma_f32_32x32x16_bf16 (keys
//     as M, its 32 query rows as N).  The S^T accumulator has one query row
//     per lane, which is the P^T operand layout of O^T = V^T . P^T, so P
//     never leaves registers and the row softmax, the O rescale and the
//     causal mask are per-lane operations;
//   * the V^T operand is read from the row-major V tile with
//     ds_read_b64_tr_b16 (two per MFMA);
//   * O is rescaled only when a row maximum grows by more than 8 in log2
//     units (exact: the final O / l uses the same stale maximum), row sums
//     use v_dot2 on the BF16 P that feeds the MFMA;
//   * key tiles above a wavefront's diagonal are skipped; workgroups are
//     mapped so that each XCD works through whole kv heads, longest row
//     blocks first, keeping those heads' K/V resident in its L2.
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

constexpr int kBN = 64;          // keys per LDS tile
constexpr int kXcds = 8;         // MI355X accelerator complex dies
constexpr float kLazyLog2 = 8.0f;  // rescale O only past 2^8 growth

template <int D>
struct Swz {
    static constexpr int NSLOT = D / 8;              // 16-byte slots per row
    static constexpr int RPC = 1024 / (2 * D);       // rows per 1 KB DMA chunk
    static constexpr int CHUNKS = kBN * D * 2 / 1024; // DMA chunks per tile
    // K: slot ^ (row % NSLOT) keeps 16 consecutive rows' reads of one slot on
    // distinct banks.  V: slot ^ 2*(row % (NSLOT/2)) keeps the four rows and
    // two slots of a transpose read on distinct banks.
    __device__ static int k(int row, int slot) { return slot ^ (row & (NSLOT - 1)); }
    __device__ static int v(int row, int slot) { return slot ^ ((2 * row) & (NSLOT - 1)); }
};

// s_waitcnt immediate that waits until at most n vector-memory operations
// are outstanding and leaves the LDS/scalar and export counters alone.
[[maybe_unused]] constexpr int vmcnt_imm(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }

// WAVES wavefronts per workgroup cover HW heads x (WAVES/HW) row blocks of
// 32 rows; STAGES K/V tiles live in LDS (STAGES-1 in flight).
template <int D, int HW, int WAVES, int STAGES>
__global__ __launch_bounds__(64 * WAVES, 2) void prefill_mfma_kernel(PrefillArgs a) {
    constexpr int KS = D / 16;           // QK k-steps (16 dims each)
    constexpr int MT = D / 32;           // O^T row tiles (32 dims each)
    constexpr int RW = 32 * (WAVES / HW);  // query rows per workgroup
    using S = Swz<D>;
    constexpr int TILE = kBN * D;        // elements per K or V tile
    constexpr int DMA_PER_WAVE = 2 * (S::CHUNKS / WAVES);  // K + V instructions per tile
    static_assert(STAGES == 2 || STAGES == 3, "two or three LDS stages");
    __shared__ __align__(16) uint16_t k0[TILE], v0[TILE], k1[TILE], v1[TILE];
    __shared__ __align__(16) uint16_t k2[STAGES == 3 ? TILE : 8], v2[STAGES == 3 ? TILE : 8];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 31;  // query row within the wavefront's block
    const int half = lane >> 5;

    // XCD-aware work mapping.  Workgroup L is dispatched to XCD L % 8; give
    // every XCD a contiguous slice of the work list ordered (kv head, row
    // block longest first, head subgroup), so an XCD streams the K/V of as
    // few kv heads as possible and they stay in its L2.
    const int group = a.q_heads / a.kv_heads;
    const int subgroups = group / HW;
    const int nrb = (a.queries + RW - 1) / RW;
    const int total = nrb * a.kv_heads * subgroups;
    const int per_xcd = (total + kXcds - 1) / kXcds;
    const int item = (int)(blockIdx.x % kXcds) * per_xcd + (int)(blockIdx.x / kXcds);
    if (item >= total) return;
    const int per_head = nrb * subgroups;
    const int kvh = item / per_head;
    const int rank = (item % per_head) / subgroups;      // 0 = longest rows
    const int sub = item % subgroups;
    const int head = kvh * group + sub * HW + wave % HW;
    const int r0 = (nrb - 1 - rank) * RW;
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
    const int last_key = a.history - 1;

    // DMA of one K/V tile: wavefront w moves chunks w, w+WAVES, ...; lane l of
    // chunk ch lands at row RPC*ch + l/NSLOT, physical slot l % NSLOT and
    // fetches the logical slot that the swizzle maps there.  Keys past the
    // history are clamped to the last key (they are masked).
    auto dma_tile = [&](uint16_t *kd, uint16_t *vd, int kt) {
#pragma unroll
        for (int i = 0; i < S::CHUNKS / WAVES; ++i) {
            const int ch = wave + WAVES * i;
            const int r = S::RPC * ch + lane / S::NSLOT;
            const int p = lane % S::NSLOT;
            const int key = min(kt * kBN + r, last_key);
            const int64_t base = ((int64_t)key * a.kv_heads + kvh) * D;
            dma16(a.k + base + S::k(r, p) * 8, kd + ch * 512);
            dma16(a.v + base + S::v(r, p) * 8, vd + ch * 512);
        }
    };

    floatx16_t o[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[mt][r] = 0.0f;
    float m_used = -INFINITY, l_run = 0.0f;

    auto compute_tile = [&](const uint16_t *kl, const uint16_t *vl, int kt) {
        if (kt * kBN > wave_last_key) return;  // tile entirely above this wavefront's rows
        // S^T = K (keys x D) . Q^T (D x rows), two 32-key blocks.
        floatx16_t s[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) s[kb][r] = 0.0f;
        // K fragments are read one k-step ahead of the MFMAs that use them.
        auto kfrag = [&](int j, int kb) {
            const int kr = kb * 32 + col;
            return *reinterpret_cast<const bf16x8_t *>(kl + kr * D + S::k(kr, 2 * j + half) * 8);
        };
        bf16x8_t kcur[2] = {kfrag(0, 0), kfrag(0, 1)};
#pragma unroll
        for (int j = 0; j < KS; ++j) {
            bf16x8_t knext[2];
            if (j + 1 < KS) {
                knext[0] = kfrag(j + 1, 0);
                knext[1] = kfrag(j + 1, 1);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
                s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kcur[kb], qf[j], s[kb], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (j + 1 < KS) {
                kcur[0] = knext[0];
                kcur[1] = knext[1];
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
        float mx = s[0][0];
#pragma unroll
        for (int r = 1; r < 31; r += 2) {
            const float x = r < 16 ? s[0][r] : s[1][r - 16];
            const float y = r + 1 < 16 ? s[0][r + 1] : s[1][r + 1 - 16];
            mx = __builtin_fmaxf(__builtin_fmaxf(mx, x), y);
        }
        mx = fmaxf(mx, s[1][15]);
        mx = wave_xor_max(mx, 32);
        // Lazy rescale: keep the old maximum while the tile stays within 2^8.
        if (wave_any(mx * c > m_used * c + kLazyLog2)) {
            const float m_new = fmaxf(m_used, mx);
            const float alpha = __builtin_amdgcn_exp2f((m_used - m_new) * c);
            l_run *= alpha;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[mt][r] *= alpha;
            m_used = m_new;
        }
        const float mc = m_used * c;
        bf16x8_t pf[2][2];
        float psum = 0.0f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                const float p0 = __builtin_amdgcn_exp2f(fmaf(s[kb][r], c, -mc));
                const float p1 = __builtin_amdgcn_exp2f(fmaf(s[kb][r + 1], c, -mc));
                bf16x2_t pp;
                pp[0] = (__bf16)p0;
                pp[1] = (__bf16)p1;
                pf[kb][r >> 3][r & 7] = pp[0];
                pf[kb][r >> 3][(r & 7) + 1] = pp[1];
                psum = add_bf16_pair(pp, psum);
            }
        l_run += psum;

        // O^T (dims x rows) += V^T (dims x keys) . P^T (keys x rows).  The
        // V^T operand of lane (q = lane/16, i = lane%16) holds dims
        // mt*32 + 16*(q%2) + i of keys kb*32 + 16t + 4*(q/2) + {0..3} and
        // kb*32 + 16t + 8 + 4*(q/2) + {0..3}; a transpose read gives four of
        // them when source lane 4r+j of the quarter wave reads row T_r,
        // dims c0 + 4j .. +3.  MFMAs run mt fastest so consecutive ones
        // update different accumulators.
        const int q4 = lane >> 4;
        const int rr = (lane & 15) >> 2;
        const int jj = lane & 3;
        // V^T fragment of MFMA number n = (kb*2 + t)*MT + mt, read two MFMAs
        // ahead of its use.
        auto vfrag = [&](int n) {
            const int mt = n % MT, t = (n / MT) % 2, kb = n / (2 * MT);
            const int t0 = kb * 32 + 16 * t + 4 * (q4 >> 1) + rr;  // row of the first read
            const int t1 = t0 + 8;
            const int e = mt * 32 + 16 * (q4 & 1) + 4 * jj;       // first dim this lane reads
            const int slot = e >> 3, off = e & 7;
            const short4_t lo = lds_read_tr16(vl + t0 * D + S::v(t0, slot) * 8 + off);
            const short4_t hi = lds_read_tr16(vl + t1 * D + S::v(t1, slot) * 8 + off);
            const short8_t both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            return __builtin_bit_cast(bf16x8_t, both);
        };
        constexpr int NPV = 4 * MT;
        bf16x8_t vq[3];
        vq[0] = vfrag(0);
        vq[1] = vfrag(1);
#pragma unroll
        for (int n = 0; n < NPV; ++n) {
            if (n + 2 < NPV) vq[(n + 2) % 3] = vfrag(n + 2);
            __builtin_amdgcn_sched_barrier(0);
            const int mt = n % MT, t = (n / MT) % 2, kb = n / (2 * MT);
            o[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vq[n % 3], pf[kb][t], o[mt], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Ring of STAGES tiles: stage buffers are distinct LDS objects and the
    // loop is unrolled by STAGES, so the compiler can tell the in-flight DMA
    // targets from the buffer being read.  Before computing tile kt a
    // wavefront waits for its own DMA of kt (the STAGES-2 newer tiles may stay
    // in flight), then the barrier makes every wavefront's part visible and
    // frees the stage that the next DMA overwrites.
    if constexpr (STAGES == 2) {
        dma_tile(k0, v0, 0);
        for (int kt = 0; kt < nkt; kt += 2) {
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (kt + 1 < nkt) dma_tile(k1, v1, kt + 1);
            compute_tile(k0, v0, kt);
            if (kt + 1 >= nkt) break;
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (kt + 2 < nkt) dma_tile(k0, v0, kt + 2);
            compute_tile(k1, v1, kt + 1);
        }
    } else {
        // DMAs are issued for every stage slot (clamped to the last tile) so
        // the outstanding count is always exact.
        dma_tile(k0, v0, 0);
        dma_tile(k1, v1, min(1, nkt - 1));
        for (int kt = 0; kt < nkt; kt += 3) {
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(DMA_PER_WAVE));
            __syncthreads();
            dma_tile(k2, v2, min(kt + 2, nkt - 1));
            compute_tile(k0, v0, kt);
            if (kt + 1 >= nkt) break;
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(DMA_PER_WAVE));
            __syncthreads();
            dma_tile(k0, v0, min(kt + 3, nkt - 1));
            compute_tile(k1, v1, kt + 1);
            if (kt + 2 >= nkt) break;
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(DMA_PER_WAVE));
            __syncthreads();
            dma_tile(k1, v1, min(kt + 4, nkt - 1));
            compute_tile(k2, v2, kt + 2);
        }
        __builtin_amdgcn_s_waitcnt(0);  // no DMA may still target LDS at exit
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

#ifndef MSLIM_PREFILL_WAVES
#define MSLIM_PREFILL_WAVES 8
#endif
#ifndef MSLIM_PREFILL_STAGES
#define MSLIM_PREFILL_STAGES 2
#endif

template <int D, int HW>
hipError_t launch_mfma(const PrefillArgs &a, hipStream_t stream) {
    constexpr int WAVES = MSLIM_PREFILL_WAVES;
    constexpr int HWW = HW > WAVES ? WAVES : HW;
    constexpr int RW = 32 * (WAVES / HWW);
    const int group = a.q_heads / a.kv_heads;
    const int total = ((a.queries + RW - 1) / RW) * a.kv_heads * (group / HWW);
    const int per_xcd = (total + kXcds - 1) / kXcds;
    hipLaunchKernelGGL((prefill_mfma_kernel<D, HWW, WAVES, MSLIM_PREFILL_STAGES>),
                       dim3((unsigned)(per_xcd * kXcds)), dim3(64 * WAVES), 0, stream, a);
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
    // Heads per workgroup: the largest of 8, 4, 2, 1 that divides the group.
    const int hw = group % 8 == 0 ? 8 : group % 4 == 0 ? 4 : group;
    if (l.head_dim == 128) {
        if (hw == 8) return launch_mfma<128, 8>(a, stream);
        if (hw == 4) return launch_mfma<128, 4>(a, stream);
        if (hw == 2) return launch_mfma<128, 2>(a, stream);
        return launch_mfma<128, 1>(a, stream);
    }
    if (hw == 8) return launch_mfma<64, 8>(a, stream);
    if (hw == 4) return launch_mfma<64, 4>(a, stream);
    if (hw == 2) return launch_mfma<64, 2>(a, stream);
    return launch_mfma<64, 1>(a, stream);
}

}  // namespace mslim
