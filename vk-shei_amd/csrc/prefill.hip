// Causal GQA prefill attention (queries >= 1 after `prior` cached tokens).
//
// Replaces llm_prefill_qk / softmax / pv (gpu_llm.cl:462-541) and the tiled
// kernel's multi-query modes (tiled_attention.cl:9-129) with a flash-style
// kernel on gfx950 MFMA:
//   * a workgroup of 8 wavefronts owns 32 query rows for 8 query heads of one
//     GQA group (or 64 rows x 4 heads, 128 x 2, 256 x 1 for smaller groups),
//     so every 64-key K/V tile staged in LDS serves all its heads;
//   * K and V tiles move HBM -> LDS with global_load_lds_dwordx4 (no VGPR
//     staging) into a four-stage ring, two tiles ahead of use, one barrier
//     per tile.  Each lane picks its source chunk so that rows land
//     XOR-swizzled in LDS;
//   * each wavefront computes S^T = K . Q^T on v_mfma_f32_32x32x16_bf16 (keys
//     as M, its 32 query rows as N).  The S^T accumulator has one query row
//     per lane, which is the P^T operand layout of O^T = V^T . P^T, so P
//     never leaves registers and the row softmax, the O rescale and the
//     causal mask are per-lane operations;
//   * the V^T operand is read from the row-major V tile with
//     ds_read_b64_tr_b16 (two per MFMA);
//   * on gfx950 ordinary VALU work hides under MFMAs only when the same
//     wavefront interleaves the two, so each wavefront software-pipelines its
//     own tiles: the softmax of tile j runs in the MFMA slots of P.V of tile
//     j-1;
//   * O is rescaled only when a row maximum grows by more than 8 in log2
//     units (exact: the final O / l uses the same stale maximum), row sums
//     use v_dot2 on the BF16 P that feeds the MFMA;
//   * workgroups are mapped so that each XCD works through whole kv heads,
//     longest row blocks first, keeping those heads' K/V resident in its L2.
#include <type_traits>

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
    // distinct banks.  V: a transpose read serves 32 lanes per cycle from
    // four consecutive rows and four consecutive slots (8 bytes each half);
    // the XOR must spread those 16 (row, slot) pairs over all 16 slot
    // positions of a 256-byte row (D = 128: slot ^ 4*(row % 4)), or over the
    // two row parities x 8 slots of a 128-byte row (D = 64: slot ^ 2*row).
    __device__ static int k(int row, int slot) { return slot ^ (row & (NSLOT - 1)); }
    __device__ static int v(int row, int slot) {
        return NSLOT == 16 ? slot ^ (4 * (row & 3)) : slot ^ ((2 * row) & (NSLOT - 1));
    }
};

// s_waitcnt immediate that waits until at most n vector-memory operations
// are outstanding and leaves the LDS/scalar and export counters alone.
constexpr int vmcnt_imm(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }
// The same with every LDS read of this wavefront complete (lgkmcnt 0).
constexpr int vmcnt_lds_imm(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4); }

// Workgroup barrier without the memory fence of __syncthreads(): with LDS
// DMA in flight that fence would wait for every outstanding DMA (vmcnt 0).
// Callers order LDS themselves with vmcnt_lds_imm waits before it.
__device__ __forceinline__ void raw_barrier() { __builtin_amdgcn_s_barrier(); }

// Iteration j of a wavefront issues the QK MFMAs of tile j, then the P.V
// MFMAs of tile j-1 with the softmax of tile j spread over their slots (row
// maximum in the first two slots, exp2 / BF16 pack / row sums in the rest).
// A rescale of O decided by the softmax of tile j is applied at the start of
// iteration j+1, after P.V of tile j-1 and before P.V of tile j.  Four LDS
// stages hold V(j-1), K(j) and the copies of tiles j+1 and j+2; the copies
// are issued by inline assembly and waited for explicitly ahead of a
// fence-free barrier.  HW heads x (8/HW) row blocks of 32 rows per
// workgroup.
template <int D, int HW>
__global__ __launch_bounds__(512, 1) void prefill_mfma_kernel(PrefillArgs a) {
    constexpr int ST = 4;  // LDS stages
    constexpr int WAVES = 8;
    constexpr int KS = D / 16;
    constexpr int MT = D / 32;
    constexpr int RW = 32 * (WAVES / HW);
    constexpr int NS = 4 * MT;  // P.V MFMA slots per tile
    static_assert(NS >= 8, "slot plan needs at least eight P.V slots");
    using S = Swz<D>;
    constexpr int TILE = kBN * D;
    __shared__ __align__(16) uint16_t k0[TILE], v0[TILE], k1[TILE], v1[TILE];
    __shared__ __align__(16) uint16_t k2[TILE], v2[TILE], k3[TILE], v3[TILE];
    constexpr int CPW = S::CHUNKS / WAVES;  // 1 KB chunks of K (and of V) per wavefront

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 31;
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
    const int rank = (item % per_head) / subgroups;
    const int sub = item % subgroups;
    const int head = kvh * group + sub * HW + wave % HW;
    const int r0 = (nrb - 1 - rank) * RW;
    const int rw0 = r0 + (wave / HW) * 32;
    const int row = rw0 + col;
    const int row_abs = a.prior + row;
    const float c = a.scale_log2e;

    bf16x8_t qf[KS];
    {
        const int qrow = min(row, a.queries - 1);
        const uint16_t *qp = a.q + ((int64_t)qrow * a.q_heads + head) * D + half * 8;
#pragma unroll
        for (int j = 0; j < KS; ++j) qf[j] = *reinterpret_cast<const bf16x8_t *>(qp + j * 16);
    }
    // Q has landed before any K/V copy is issued (no wait inside the loop
    // may hold back copies in flight).
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

    const int key_end = min(a.history, a.prior + r0 + RW);
    const int nkt = (key_end + kBN - 1) / kBN;
    const int last_key = a.history - 1;

    // Copy of one K/V tile: wavefront w moves chunks w, w+8, ...; lane l of
    // chunk ch lands at row RPC*ch + l/NSLOT, physical slot l % NSLOT and
    // fetches the logical slot that the swizzle maps there.  Keys past the
    // history are clamped to the last key (they are masked).
    auto dma_tile = [&](uint16_t *kd, uint16_t *vd, int kt) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < CPW; ++i) {
            const int ch = wave + WAVES * i;
            const int r = S::RPC * ch + lane / S::NSLOT;
            const int p = lane % S::NSLOT;
            const int key = min(kt * kBN + r, last_key);
            const int64_t base = ((int64_t)key * a.kv_heads + kvh) * D;
            dma16_async(a.k + base + S::k(r, p) * 8, lds_offset(kd + ch * 512));
            dma16_async(a.v + base + S::v(r, p) * 8, lds_offset(vd + ch * 512));
        }
    };

    floatx16_t o[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[mt][r] = 0.0f;
    float m_used = -INFINITY, l_run = 0.0f;
    float alpha_pending = 1.0f;
    bool rescale_pending = false;
    floatx16_t s[2];
    bf16x8_t pprev[2][2];  // P of the previous tile, [key block][16-key half]

    const int q4 = lane >> 4;
    const int rr = (lane & 15) >> 2;
    const int jj = lane & 3;

    auto qk = [&](const uint16_t *kl) __attribute__((always_inline)) {
        auto kfrag = [&](int ks, int kb) __attribute__((always_inline)) {
            const int kr = kb * 32 + col;
            return *reinterpret_cast<const bf16x8_t *>(kl + kr * D + S::k(kr, 2 * ks + half) * 8);
        };
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) s[kb][r] = 0.0f;
        bf16x8_t kq[3];
        kq[0] = kfrag(0, 0);
        kq[1] = kfrag(0, 1);
#pragma unroll
        for (int n = 0; n < 2 * KS; ++n) {
            if (n + 2 < 2 * KS) kq[(n + 2) % 3] = kfrag((n + 2) / 2, (n + 2) % 2);
            __builtin_amdgcn_sched_barrier(0);
            s[n % 2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kq[n % 3], qf[n / 2], s[n % 2], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    auto mask_tile = [&](int kt) __attribute__((always_inline)) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = kt * kBN + kb * 32 + (r >> 2) * 8 + half * 4 + (r & 3);
                if (key > row_abs) s[kb][r] = -INFINITY;
            }
    };

    // P.V of the previous tile (V stage vp, when do_pv) with the softmax of
    // the current scores (when do_sm) spread over the MFMA slots.
    auto pv_softmax = [&](const uint16_t *vp, auto pv_tag, auto sm_tag) __attribute__((always_inline)) {
        constexpr bool do_pv = decltype(pv_tag)::value;
        constexpr bool do_sm = decltype(sm_tag)::value;
        auto vfrag = [&](int n) __attribute__((always_inline)) {
            const int mt = n % MT, t = (n / MT) % 2, kb = n / (2 * MT);
            const int t0 = kb * 32 + 16 * t + 4 * (q4 >> 1) + rr;
            const int t1 = t0 + 8;
            const int e = mt * 32 + 16 * (q4 & 1) + 4 * jj;
            const int slot = e >> 3, off = e & 7;
            const short4_t lo = lds_read_tr16(vp + t0 * D + S::v(t0, slot) * 8 + off);
            const short4_t hi = lds_read_tr16(vp + t1 * D + S::v(t1, slot) * 8 + off);
            const short8_t both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            return __builtin_bit_cast(bf16x8_t, both);
        };
        bf16x8_t vq[3];
        if constexpr (do_pv) {
            vq[0] = vfrag(0);
            vq[1] = vfrag(1);
        }
        float mx = 0.0f, mc = 0.0f, psum = 0.0f;
        uint32_t pw[2][8];
#pragma unroll
        for (int n = 0; n < NS; ++n) {
            if constexpr (do_pv) {
                if (n + 2 < NS) vq[(n + 2) % 3] = vfrag(n + 2);
            }
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (do_pv) {
                const int mt = n % MT, t = (n / MT) % 2, kb = n / (2 * MT);
                o[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vq[n % 3], pprev[kb][t], o[mt], 0, 0, 0);
            }
            if constexpr (do_sm) {
                if (n == 0) {  // row maximum, first key block
                    mx = __builtin_fmaxf(s[0][0], s[0][1]);
#pragma unroll
                    for (int r = 2; r < 16; r += 2) mx = __builtin_fmaxf(__builtin_fmaxf(mx, s[0][r]), s[0][r + 1]);
                } else if (n == 1) {  // second key block, both halves, lazy decision
#pragma unroll
                    for (int r = 0; r < 16; r += 2) mx = __builtin_fmaxf(__builtin_fmaxf(mx, s[1][r]), s[1][r + 1]);
                    mx = half_pair_max(mx);
                    const bool grow = wave_any(mx * c > m_used * c + kLazyLog2);
                    const float m_new = grow ? fmaxf(m_used, mx) : m_used;
                    const float alpha = __builtin_amdgcn_exp2f((m_used - m_new) * c);
                    l_run *= alpha;
                    alpha_pending = alpha;
                    rescale_pending = grow;
                    m_used = m_new;
                    mc = m_used * c;
                } else {
                    // pairs of scores, spread over slots 2 .. NS-1
#pragma unroll
                    for (int pidx = 0; pidx < 16; ++pidx) {
                        if (2 + (pidx * (NS - 2)) / 16 != n) continue;
                        const int kb = pidx / 8, r = (pidx % 8) * 2;
                        bf16x2_t pp;
                        pp[0] = (__bf16)__builtin_amdgcn_exp2f(fmaf(s[kb][r], c, -mc));
                        pp[1] = (__bf16)__builtin_amdgcn_exp2f(fmaf(s[kb][r + 1], c, -mc));
                        pw[kb][r >> 1] = __builtin_bit_cast(uint32_t, pp);
                        psum = add_bf16_pair(pp, psum);
                        pin_value(pw[kb][r >> 1]);
                    }
                    pin_value(psum);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (do_sm) {
            l_run += psum;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const uint4 u = {pw[kb][4 * t], pw[kb][4 * t + 1], pw[kb][4 * t + 2], pw[kb][4 * t + 3]};
                    pprev[kb][t] = __builtin_bit_cast(bf16x8_t, u);
                }
        }
    };

    using Yes = std::true_type;
    using No = std::false_type;
    auto apply_rescale = [&]() __attribute__((always_inline)) {
        if (rescale_pending) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[mt][r] *= alpha_pending;
            rescale_pending = false;
        }
    };
    // One iteration j (1 <= j < nkt): kc = K(j), vp = V(j-1); the stage of
    // tile j-2 (kd, vd) receives tile j+2.  Tiles entirely above a
    // wavefront's rows are computed too: their scores are all masked, so
    // they add exactly zero.  Every iteration issues one copy batch (the
    // last tile is repeated past the end) so the wait below is exact.
    auto iteration = [&](int j, const uint16_t *kc, const uint16_t *vp, uint16_t *kd, uint16_t *vd)
        __attribute__((always_inline)) {
        // This wavefront's copy of tile j has landed (that of tile j+1 may
        // still be in flight); the barrier publishes tile j and tells that
        // every wavefront is past iteration j-1, which freed stage j-2.
        __builtin_amdgcn_s_waitcnt(vmcnt_lds_imm(2 * CPW));
        raw_barrier();
        dma_tile(kd, vd, min(j + 2, nkt - 1));
        apply_rescale();
        qk(kc);
        if (j * kBN + kBN - 1 > a.prior + rw0) mask_tile(j);
        pv_softmax(vp, Yes{}, Yes{});
    };

    // Prologue: tiles 0, 1, 2 in flight (repeats of the last tile past the
    // end), tile 0 scored and turned into P.  Stage i holds tile j with
    // j % 4 == i; the loop is unrolled by four so every stage is a distinct
    // LDS object.
    dma_tile(k0, v0, 0);
    dma_tile(k1, v1, min(1, nkt - 1));
    dma_tile(k2, v2, min(2, nkt - 1));
    __builtin_amdgcn_s_waitcnt(vmcnt_lds_imm(2 * 2 * CPW));
    raw_barrier();
    qk(k0);
    if (kBN - 1 > a.prior + rw0) mask_tile(0);
    pv_softmax(v0, No{}, Yes{});
    for (int j = 1; j < nkt; j += ST) {
        iteration(j, k1, v0, k3, v3);
        if (j + 1 >= nkt) break;
        iteration(j + 1, k2, v1, k0, v0);
        if (j + 2 >= nkt) break;
        iteration(j + 2, k3, v2, k1, v1);
        if (j + 3 >= nkt) break;
        iteration(j + 3, k0, v3, k2, v2);
    }
    // P.V of the last tile, from the stage that holds it.
    __builtin_amdgcn_s_waitcnt(vmcnt_lds_imm(0));
    apply_rescale();
    const int last_stage = (nkt - 1) % ST;
    if (last_stage == 0) pv_softmax(v0, Yes{}, No{});
    else if (last_stage == 1) pv_softmax(v1, Yes{}, No{});
    else if (last_stage == 2) pv_softmax(v2, Yes{}, No{});
    else pv_softmax(v3, Yes{}, No{});
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // no DMA may still target LDS at exit

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
    constexpr int RW = 32 * (8 / HW);
    const int group = a.q_heads / a.kv_heads;
    const int total = ((a.queries + RW - 1) / RW) * a.kv_heads * (group / HW);
    const int per_xcd = (total + kXcds - 1) / kXcds;
    hipLaunchKernelGGL((prefill_mfma_kernel<D, HW>), dim3((unsigned)(per_xcd * kXcds)), dim3(512), 0, stream, a);
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
