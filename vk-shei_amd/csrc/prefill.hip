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
//     j-1.  The first two P.V MFMAs of tile j-1 run ahead of the QK MFMAs of
//     tile j (their V fragments read before the barrier), and the copy of a
//     later tile is issued behind the first QK MFMAs, so the SIMD has MFMA
//     work while the tile's first K fragments are in flight;
//   * Q enters the QK MFMAs pre-multiplied by scale * log2(e) (rounded to
//     BF16) and the S accumulator starts from -m (the row's reference
//     maximum), so each score leaves the MFMA as the exp2 argument: the
//     softmax costs exp2, a BF16 pack and a row-sum step per score, no
//     multiply;
//   * O is rescaled only when a tile's row sum under the current maximum
//     exceeds 2^8 (exact: the final O / l uses the same stale maximum), row
//     sums use v_dot2 on the BF16 P that feeds the MFMA;
//   * workgroups are mapped so that each XCD works through whole kv heads,
//     longest row blocks first, keeping those heads' K/V resident in its L2;
//     the shortest row blocks of every XCD form a pool taken at run time, so
//     XCDs of different clocks finish together;
//   * a launch too small to keep every CU busy for the length of its longest
//     row block (cfg2's 2,048 tokens: 256 workgroups of 1 to 32 key tiles;
//     the decoder's 512-token prompt chunks: 64 workgroups) splits long row
//     blocks into chunks of key tiles and dispatches all chunks longest
//     first.  Chunks are counted back from the causal diagonal, so every
//     chunk but the last sees only unmasked keys; the last workgroup of a
//     split row block to finish merges the chunks' (m, l, O) partials in
//     fixed chunk order, so the result does not depend on timing.
#include <algorithm>
#include <mutex>
#include <map>
#include <array>
#include <queue>
#include <type_traits>
#include <vector>

#include "common.hpp"
#include "kernels.hpp"

namespace mslim {

namespace {

// Split-mode work items in the kernel arguments: row block | chunk << 10 |
// head group << 16, longest first; at most kMaxChunks chunks per row block.
constexpr int kMaxSplitItems = 768;
constexpr int kMaxChunks = 8;
constexpr uint32_t kNoItem = 0xFFFFFFFFu;  // padding slot of the item table

struct PrefillArgs {
    const uint16_t *q, *k, *v;
    uint16_t *out;
    int queries, prior, history;
    int q_heads, kv_heads;
    float scale_log2e;
    // chunk_tiles > 0: split mode.  partial holds [row block key][max_chunks]
    // [wave][MT * 8 + 1][64] float pairs (O, then (m, l)), counters one int
    // per row block key (kv head group x row blocks), zero between launches.
    int chunk_tiles, max_chunks, items;
    float *partial;
    int *counters;
    // Unsplit launches: the last pool_items entries of every XCD's slice of
    // the work list go to a shared pool; each XCD runs pool_items +
    // kPoolSpare workgroups that take pool entries through pool_counter.
    int pool_items;
    int *pool_counter;
    uint32_t item[kMaxSplitItems];
};

constexpr int kBN = 64;          // keys per LDS tile
constexpr int kCus = 256;        // MI355X compute units
constexpr int kXcds = 8;         // MI355X accelerator complex dies
// Run-time pool of an unsplit launch: at most kPoolMax row blocks per XCD,
// kPoolSpare extra workgroups per XCD to take them.
constexpr int kPoolMax = 64;
constexpr int kPoolSpare = 8;
// Lazy rescale: the reference maximum moves only when a tile's row sum under
// it exceeds 2^8 (so every p stays within 2^8 of the reference).
constexpr float kLazyBound = 256.0f;
// QK MFMA of a tile after which the copy of a later tile is issued.
constexpr int kCopySlot = 3;
// P.V slots of a tile issued ahead of the next tile's QK MFMAs.
constexpr int kHead = 2;

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
    static_assert(2 * kHead <= 15 && kHead + 2 <= NS, "head reads must fit the lgkmcnt field");
    using S = Swz<D>;
    constexpr int TILE = kBN * D;
    // The four K stages, then the four V stages: each set spans 64 KiB, so
    // one per-lane fragment address serves every stage through the LDS
    // instructions' 16-bit immediate offset.
    __shared__ __align__(16) uint16_t kv_lds[2 * ST][TILE];
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
    //
    // XCDs run at different clocks (measured up to 5% apart on one device),
    // so equal slices finish at different times.  With a pool, the shortest
    // pool_items entries of every slice are instead taken at run time, one
    // atomic increment per workgroup, in the order (entry, XCD): a faster
    // XCD reaches its pool workgroups sooner and takes more of them.  The
    // pool has pool_items + kPoolSpare workgroups per XCD; those that find
    // it empty exit, and the last of them to draw resets the counter.
    const int group = a.q_heads / a.kv_heads;
    const int subgroups = group / HW;
    const int nrb = (a.queries + RW - 1) / RW;
    int kvh, sub, rb, chunk = 0;
    if (a.chunk_tiles) {
        if ((int)blockIdx.x >= a.items || a.item[blockIdx.x] == kNoItem) return;
        const uint32_t u = a.item[blockIdx.x];
        rb = (int)(u & 1023u);
        chunk = (int)((u >> 10) & 63u);
        const int hg = (int)(u >> 16);
        kvh = hg / subgroups;
        sub = hg % subgroups;
    } else {
        const int total = nrb * a.kv_heads * subgroups;
        const int per_xcd = (total + kXcds - 1) / kXcds;
        const int xcd = (int)(blockIdx.x % kXcds), slot = (int)(blockIdx.x / kXcds);
        int item;
        if (slot < per_xcd - a.pool_items) {
            item = xcd * per_xcd + slot;
        } else {
            __shared__ int drawn;
            if (tid == 0) {
                const int g = __hip_atomic_fetch_add(a.pool_counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (g == kXcds * (a.pool_items + kPoolSpare) - 1)
                    __hip_atomic_store(a.pool_counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                drawn = g;
            }
            __syncthreads();
            const int g = __builtin_amdgcn_readfirstlane(drawn);
            if (g >= kXcds * a.pool_items) return;
            item = (g % kXcds) * per_xcd + per_xcd - a.pool_items + g / kXcds;
        }
        if (item >= total) return;
        // Uniform by construction; the compiler cannot prove it across the
        // pool branch, and the K/V copies need the tile bases in SGPRs.
        item = __builtin_amdgcn_readfirstlane(item);
        const int per_head = nrb * subgroups;
        kvh = item / per_head;
        rb = nrb - 1 - (item % per_head) / subgroups;
        sub = item % subgroups;
    }
    const int head = kvh * group + sub * HW + wave % HW;
    const int r0 = rb * RW;
    const int rw0 = r0 + (wave / HW) * 32;
    const int row = rw0 + col;
    const int row_abs = a.prior + row;
    const float c = a.scale_log2e;

    // Q enters the MFMAs pre-multiplied by scale * log2(e) and rounded to
    // BF16 (RNE), so every score comes out of the QK MFMAs in log2 units and
    // the softmax needs no multiply per score.
    bf16x8_t qf[KS];
    {
        const int qrow = min(row, a.queries - 1);
        const uint16_t *qp = a.q + ((int64_t)qrow * a.q_heads + head) * D + half * 8;
#pragma unroll
        for (int j = 0; j < KS; ++j) qf[j] = *reinterpret_cast<const bf16x8_t *>(qp + j * 16);
#pragma unroll
        for (int j = 0; j < KS; ++j)
#pragma unroll
            for (int e = 0; e < 8; ++e) qf[j][e] = (__bf16)((float)qf[j][e] * c);
    }
    // Q has landed before any K/V copy is issued (no wait inside the loop
    // may hold back copies in flight).
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

    const int key_end = min(a.history, a.prior + r0 + RW);
    const int nkt = (key_end + kBN - 1) / kBN;
    const int last_key = a.history - 1;
    // Tiles [tb, te) of this workgroup: chunk c of nchunks, counted back from
    // the last tile (chunk 0 takes the remainder).
    int nchunks = 1, tb = 0, te = nkt;
    if (a.chunk_tiles) {
        nchunks = (nkt + a.chunk_tiles - 1) / a.chunk_tiles;
        te = nkt - (nchunks - 1 - chunk) * a.chunk_tiles;
        tb = max(0, te - a.chunk_tiles);
    }
    const int ntl = te - tb;

    // Copy of one K/V tile: wavefront w moves chunks w, w+8, ...; lane l of
    // chunk ch lands at row RPC*ch + l/NSLOT, physical slot l % NSLOT and
    // fetches the logical slot that the swizzle maps there.  Keys past the
    // history are clamped to the last key (they are masked); only the tile
    // that holds the last key has such rows, and its copies move those lanes'
    // offsets back to the last key's row.  Offsets are bytes from the tile's first row, so a copy
    // needs only the scalar tile base (no per-lane 64-bit address arithmetic
    // per tile).
    const uint32_t row_bytes = (uint32_t)a.kv_heads * D * 2;
    const int tile_last = last_key / kBN;
    const int last_row = last_key - tile_last * kBN;
    uint32_t koff[CPW], voff[CPW];
#pragma unroll
    for (int i = 0; i < CPW; ++i) {
        const int ch = wave + WAVES * i;
        const int r = S::RPC * ch + lane / S::NSLOT;
        const int p = lane % S::NSLOT;
        const uint32_t head_bytes = (uint32_t)kvh * D * 2;
        koff[i] = (uint32_t)r * row_bytes + head_bytes + S::k(r, p) * 16;
        voff[i] = (uint32_t)r * row_bytes + head_bytes + S::v(r, p) * 16;
    }
    // LDS byte address of this wavefront's first chunk in every stage.
    const uint32_t kst_lds[ST] = {lds_offset(kv_lds[0] + wave * 512), lds_offset(kv_lds[1] + wave * 512),
                                  lds_offset(kv_lds[2] + wave * 512), lds_offset(kv_lds[3] + wave * 512)};
    const uint32_t vst_lds[ST] = {lds_offset(kv_lds[4] + wave * 512), lds_offset(kv_lds[5] + wave * 512),
                                  lds_offset(kv_lds[6] + wave * 512), lds_offset(kv_lds[7] + wave * 512)};
    auto dma_tile = [&](int st, int kt) __attribute__((always_inline)) {
        const int64_t base = (int64_t)kt * kBN * row_bytes;
        const char *kb = reinterpret_cast<const char *>(a.k) + base;
        const char *vb = reinterpret_cast<const char *>(a.v) + base;
        if (kt != tile_last) {
#pragma unroll
            for (int i = 0; i < CPW; ++i) {
                dma16_async(kb, koff[i], kst_lds[st] + i * WAVES * 1024);
                dma16_async(vb, voff[i], vst_lds[st] + i * WAVES * 1024);
            }
        } else {
            // Rows past the last key fetch the last key's row (the same
            // logical slot): the offset moves back by whole rows.
#pragma unroll
            for (int i = 0; i < CPW; ++i) {
                const int r = S::RPC * (wave + WAVES * i) + lane / S::NSLOT;
                const uint32_t back = (uint32_t)max(r - last_row, 0) * row_bytes;
                dma16_async(kb, koff[i] - back, kst_lds[st] + i * WAVES * 1024);
                dma16_async(vb, voff[i] - back, vst_lds[st] + i * WAVES * 1024);
            }
        }
    };

    floatx16_t o[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[mt][r] = 0.0f;
    // m_used: the row's reference maximum in log2 units; seed holds -m_used
    // in every element and is the QK accumulator's initial value, so the
    // MFMAs return scores relative to the reference.
    float m_used = -INFINITY, l_run = 0.0f;
    floatx16_t seed;
    float alpha_pending = 1.0f;
    bool rescale_pending = false;
    floatx16_t s[2];
    bf16x8_t pprev[2][2];  // P of the previous tile, [key block][16-key half]

    const int q4 = lane >> 4;
    const int rr = (lane & 15) >> 2;
    const int jj = lane & 3;

    // Per-lane LDS byte addresses of the fragment reads in stage 0.  The
    // swizzles depend on a row only through row % 16 (K) and row % 4 (V),
    // which the row steps below (kb * 32 rows, 16 and 8 rows of V) keep, so
    // a stage (TILE * 2 bytes), a key block and a V row step are immediate
    // offsets of the same address; the bases are opaque scalars, so the
    // compiler folds every such step into the instruction.
    constexpr uint32_t STAGE = TILE * 2;
    uint32_t kaddr[KS], vaddr[MT];
    {
        const uint32_t kbase = lds_offset(kv_lds[0]), vbase = lds_offset(kv_lds[ST]);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            kaddr[ks] = kbase + (uint32_t)(col * D * 2 + S::k(col, 2 * ks + half) * 16);
        const int t0 = 4 * (q4 >> 1) + rr;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int e = mt * 32 + 16 * (q4 & 1) + 4 * jj;
            vaddr[mt] = vbase + (uint32_t)(t0 * D * 2 + S::v(t0, e >> 3) * 16 + (e & 7) * 2);
        }
    }

    // S^T of one tile from K stage kst; seeded: relative to the reference
    // (first tile of the workgroup: absolute, the reference is not known yet).
    auto qk = [&](int kst, auto seeded_tag, auto &&mid) __attribute__((always_inline)) {
        constexpr bool seeded = decltype(seeded_tag)::value;
        auto kfrag = [&](int ks, int kb) __attribute__((always_inline)) {
            return lds_read_b128(kaddr[ks] + kst * STAGE + kb * 32 * D * 2);
        };
        bf16x8_t kq[3];
        kq[0] = kfrag(0, 0);
        kq[1] = kfrag(0, 1);
#pragma unroll
        for (int n = 0; n < 2 * KS; ++n) {
            if (n + 2 < 2 * KS) kq[(n + 2) % 3] = kfrag((n + 2) / 2, (n + 2) % 2);
            __builtin_amdgcn_sched_barrier(0);
            if (n < 2) {
                floatx16_t init;
                if constexpr (seeded) {
                    init = seed;
                } else {
#pragma unroll
                    for (int r = 0; r < 16; ++r) init[r] = 0.0f;
                }
                s[n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kq[n], qf[0], init, 0, 0, 0);
            } else {
                s[n % 2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kq[n % 3], qf[n / 2], s[n % 2], 0, 0, 0);
            }
            if (n == kCopySlot) mid();
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Key kt * kBN + kb * 32 + (r >> 2) * 8 + half * 4 + (r & 3) of element
    // (kb, r) is masked when it passes the row: one lane threshold, then a
    // compare with a constant per element.
    auto mask_tile = [&](int kt) __attribute__((always_inline)) {
        const int thr = row_abs - kt * kBN - half * 4;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                if (kb * 32 + (r >> 2) * 8 + (r & 3) > thr) s[kb][r] = -INFINITY;
    };

    using Yes = std::true_type;
    using No = std::false_type;
    // Pair pidx of the current scores (key block pidx / 8, rows 2 (pidx % 8)
    // and the next): exp2 of the score less `sub` (none for scores already
    // relative to the reference), BF16 pack, and the row sum of the packed P
    // that feeds the MFMA.
    auto score_pair = [&](int pidx, uint32_t (&pw)[2][8], float &psum, auto sub_tag, float sub)
        __attribute__((always_inline)) {
        constexpr bool do_sub = decltype(sub_tag)::value;
        const int kb = pidx / 8, r = (pidx % 8) * 2;
        bf16x2_t pp;
        if constexpr (do_sub) {
            pp[0] = (__bf16)__builtin_amdgcn_exp2f(s[kb][r] - sub);
            pp[1] = (__bf16)__builtin_amdgcn_exp2f(s[kb][r + 1] - sub);
        } else {
            pp[0] = (__bf16)__builtin_amdgcn_exp2f(s[kb][r]);
            pp[1] = (__bf16)__builtin_amdgcn_exp2f(s[kb][r + 1]);
        }
        pw[kb][r >> 1] = __builtin_bit_cast(uint32_t, pp);
        psum = add_bf16_pair(pp, psum);
        pin_value(pw[kb][r >> 1]);
    };

    // V^T fragment of P.V slot n from V stage vst.
    auto vfrag = [&](int vst, int n) __attribute__((always_inline)) {
        const int mt = n % MT, t = (n / MT) % 2, kb = n / (2 * MT);
        const uint32_t a0 = vaddr[mt] + vst * STAGE + (kb * 32 + 16 * t) * D * 2;
        const short4_t lo = lds_read_tr16_at(a0);
        const short4_t hi = lds_read_tr16_at(a0 + 8 * D * 2);
        const short8_t both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        return __builtin_bit_cast(bf16x8_t, both);
    };
    // The first kHead P.V slots of a tile run ahead of the next tile's QK
    // MFMAs, from fragments read before the barrier: the SIMD has MFMA work
    // while the next tile's first K fragments are in flight.
    bf16x8_t vhead[kHead];
    auto read_head = [&](int vst) __attribute__((always_inline)) {
#pragma unroll
        for (int n = 0; n < kHead; ++n) vhead[n] = vfrag(vst, n);
    };
    auto pv_head = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int n = 0; n < kHead; ++n) {
            const int mt = n % MT, t = (n / MT) % 2, kb = n / (2 * MT);
            __builtin_amdgcn_sched_barrier(0);
            o[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vhead[n], pprev[kb][t], o[mt], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // P.V slots kHead .. NS-1 of the previous tile (V stage vst, when do_pv)
    // with the softmax of the current scores (when do_sm) spread over them
    // (over all NS slots when there is no P.V).
    auto pv_softmax = [&](int vst, auto pv_tag, auto sm_tag, auto first_tag)
        __attribute__((always_inline)) {
        constexpr bool do_pv = decltype(pv_tag)::value;
        constexpr bool do_sm = decltype(sm_tag)::value;
        constexpr bool first = decltype(first_tag)::value;
        constexpr int N0 = do_pv ? kHead : 0;  // first slot
        constexpr int NL = NS - N0;             // slots here
        bf16x8_t vq[3];
        if constexpr (do_pv) {
            vq[0] = vfrag(vst, N0);
            vq[1] = vfrag(vst, N0 + 1);
        }
        float mx = 0.0f, psum = 0.0f;
        uint32_t pw[2][8];
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int n = N0 + i;
            if constexpr (do_pv) {
                if (n + 2 < NS) vq[(i + 2) % 3] = vfrag(vst, n + 2);
            }
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (do_pv) {
                const int mt = n % MT, t = (n / MT) % 2, kb = n / (2 * MT);
                o[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vq[i % 3], pprev[kb][t], o[mt], 0, 0, 0);
            }
            if constexpr (do_sm && first) {
                // The workgroup's first tile: the reference is still -inf, so
                // take the row maximum first (slots 0 and 1), then the pairs
                // less it.
                if (i == 0) {
                    mx = s[0][0];
#pragma unroll
                    for (int r = 1; r < 15; r += 2) mx = __builtin_fmaxf(__builtin_fmaxf(mx, s[0][r]), s[0][r + 1]);
                } else if (i == 1) {
                    mx = __builtin_fmaxf(__builtin_fmaxf(mx, s[0][15]), s[1][0]);
#pragma unroll
                    for (int r = 1; r < 15; r += 2) mx = __builtin_fmaxf(__builtin_fmaxf(mx, s[1][r]), s[1][r + 1]);
                    m_used = half_pair_max(__builtin_fmaxf(mx, s[1][15]));
                } else {
#pragma unroll
                    for (int pidx = 0; pidx < 16; ++pidx)
                        if (2 + (pidx * (NL - 2)) / 16 == i) score_pair(pidx, pw, psum, Yes{}, m_used);
                    pin_value(psum);
                }
            } else if constexpr (do_sm) {
                // Every later tile: the pairs (scores already relative to the
                // reference) in all slots but the last, then the lazy-rescale
                // test in the last slot.
#pragma unroll
                for (int pidx = 0; pidx < 16; ++pidx)
                    if ((pidx * (NL - 1)) / 16 == i) score_pair(pidx, pw, psum, No{}, 0.0f);
                pin_value(psum);
                // Every p of the tile is at most its row sum, so the reference
                // need not move while each row sum stays within 2^8 (exact: the
                // final O / l uses the same reference).  Otherwise (rare after
                // the first tile; also when a p overflowed) take the tile's row
                // maximum, move the reference for the rows that exceed it, and
                // recompute the tile's P under the new one.
                if (i == NL - 1 && wave_any(psum > kLazyBound)) {
                    mx = s[0][0];
#pragma unroll
                    for (int r = 1; r < 15; r += 2) mx = __builtin_fmaxf(__builtin_fmaxf(mx, s[0][r]), s[0][r + 1]);
                    mx = __builtin_fmaxf(__builtin_fmaxf(mx, s[0][15]), s[1][0]);
#pragma unroll
                    for (int r = 1; r < 15; r += 2) mx = __builtin_fmaxf(__builtin_fmaxf(mx, s[1][r]), s[1][r + 1]);
                    mx = half_pair_max(__builtin_fmaxf(mx, s[1][15]));
                    // The row's maximum above the reference (0: it stays).
                    const float shift = fmaxf(mx, 0.0f);
                    const float alpha = __builtin_amdgcn_exp2f(-shift);
                    l_run *= alpha;
                    alpha_pending = alpha;
                    rescale_pending = true;
                    m_used += shift;
#pragma unroll
                    for (int r = 0; r < 16; ++r) seed[r] = -m_used;
                    psum = 0.0f;
#pragma unroll
                    for (int pidx = 0; pidx < 16; ++pidx) score_pair(pidx, pw, psum, Yes{}, shift);
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

    auto apply_rescale = [&]() __attribute__((always_inline)) {
        if (rescale_pending) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[mt][r] *= alpha_pending;
            rescale_pending = false;
        }
    };
    // One iteration j (1 <= j < nkt): K stage kst holds tile j, V stage vst
    // tile j-1; stage sd
    // (that of tile j-2) receives tile j+2.  Tiles entirely above a
    // wavefront's rows are computed too: their scores are all masked, so
    // they add exactly zero.  Every iteration issues one copy batch (the
    // last tile is repeated past the end) so the wait below is exact.
    // j counts this workgroup's tiles from 0; its key tile is tb + j.
    auto iteration = [&](int j, int kst, int vst, int sd) __attribute__((always_inline)) {
        // This wavefront's copy of tile j has landed (that of tile j+1 may
        // still be in flight); the barrier publishes tile j and tells that
        // every wavefront is past iteration j-1, which freed stage j-2.
        // This wavefront's reads of stage j-2 are complete before the
        // barrier frees it; the head reads (of stage j-1) may still be in
        // flight.
        read_head(vst);
        __builtin_amdgcn_s_waitcnt(vmcnt_lds_last_imm(2 * CPW, 2 * kHead));
        raw_barrier();
        apply_rescale();
        pv_head();
        // The next copy goes out behind the first QK MFMAs, so the fragment
        // reads and MFMAs of this tile start right after the barrier.
        qk(kst, Yes{}, [&]() __attribute__((always_inline)) { dma_tile(sd, tb + min(j + 2, ntl - 1)); });
        if ((tb + j) * kBN + kBN - 1 > a.prior + rw0) mask_tile(tb + j);
        pv_softmax(vst, Yes{}, Yes{}, No{});
    };

    // Prologue: tiles 0, 1, 2 in flight (repeats of the last tile past the
    // end), tile 0 scored and turned into P.  Stage i holds tile j with
    // j % 4 == i; the loop is unrolled by four so every stage is a distinct
    // LDS object.
    dma_tile(0, tb);
    dma_tile(1, tb + min(1, ntl - 1));
    dma_tile(2, tb + min(2, ntl - 1));
    __builtin_amdgcn_s_waitcnt(vmcnt_lds_imm(2 * 2 * CPW));
    raw_barrier();
    qk(0, No{}, []() {});
    if (tb * kBN + kBN - 1 > a.prior + rw0) mask_tile(tb);
    pv_softmax(0, No{}, Yes{}, Yes{});
    // The first maximum always moves the reference from -inf; O is still
    // zero then, so there is nothing to rescale.
    rescale_pending = false;
#pragma unroll
    for (int r = 0; r < 16; ++r) seed[r] = -m_used;
    for (int j = 1; j < ntl; j += ST) {
        iteration(j, 1, 0, 3);
        if (j + 1 >= ntl) break;
        iteration(j + 1, 2, 1, 0);
        if (j + 2 >= ntl) break;
        iteration(j + 2, 3, 2, 1);
        if (j + 3 >= ntl) break;
        iteration(j + 3, 0, 3, 2);
    }
    // P.V of the last tile, from the stage that holds it.
    const int last_stage = (ntl - 1) % ST;
    read_head(last_stage);
    __builtin_amdgcn_s_waitcnt(vmcnt_lds_imm(0));
    apply_rescale();
    pv_head();
    if (last_stage == 0) pv_softmax(0, Yes{}, No{}, No{});
    else if (last_stage == 1) pv_softmax(1, Yes{}, No{}, No{});
    else if (last_stage == 2) pv_softmax(2, Yes{}, No{}, No{});
    else pv_softmax(3, Yes{}, No{}, No{});
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // no DMA may still target LDS at exit

    const float l = l_run + __shfl_xor(l_run, 32, 64);
    // O / l as O * (1 / l): one correctly rounded reciprocal per row instead
    // of D divisions (within one f32 ulp of the quotient before the BF16
    // rounding).
    auto write_out = [&](const floatx16_t *acc, float lsum) __attribute__((always_inline)) {
        if (row >= a.queries) return;
        uint16_t *op = a.out + ((int64_t)row * a.q_heads + head) * D;
        const float inv = 1.0f / lsum;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const int d = mt * 32 + r4 * 8 + half * 4;
                uint2 w;
                w.x = pack_bf16x2(acc[mt][r4 * 4 + 0] * inv, acc[mt][r4 * 4 + 1] * inv);
                w.y = pack_bf16x2(acc[mt][r4 * 4 + 2] * inv, acc[mt][r4 * 4 + 3] * inv);
                *reinterpret_cast<uint2 *>(op + d) = w;
            }
    };
    if (nchunks == 1) {
        write_out(o, l);
        return;
    }

    // Split row block: publish this chunk's partial as float pairs in
    // [pair][lane] order (O, then (m, l)), so every store and load covers a
    // contiguous 512-byte run.  The stores are agent-scope atomic pairs
    // (written through to the device coherence point), each thread waits for
    // its own, and only then does thread 0 count the chunk; the merging
    // workgroup reads the others with agent-scope atomic loads (the decode
    // merge's ordering).  This order rests on how gfx950 implements those
    // relaxed agent-scope operations (sc1 write-through stores, loads that
    // bypass the XCD's L2), not on the language memory model; common.hpp
    // refuses any other build target.  Release / acquire on thread 0's count
    // gives the same bits but costs an L2 write-back and invalidate per
    // workgroup: cfg2 48.7 against 44.9 us, a 512-query chunk after 3,584
    // tokens 46.2 against 44.2 us, 1,000 queries after 777 tokens 41.1
    // against 37.5 us (medians of eight interleaved rounds).
    constexpr int PAIRS = MT * 8 + 1;
    const int rbk = (kvh * subgroups + sub) * nrb + rb;
    auto chunk_base = [&](int ch) __attribute__((always_inline)) {
        return a.partial + ((((int64_t)rbk * a.max_chunks + ch) * WAVES + wave) * PAIRS * 64 + lane) * 2;
    };
    auto put2 = [](float *p, float x, float y) __attribute__((always_inline)) {
        const uint64_t w = (uint64_t)__float_as_uint(x) | ((uint64_t)__float_as_uint(y) << 32);
        __hip_atomic_store(reinterpret_cast<uint64_t *>(p), w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    auto get2 = [](const float *p) __attribute__((always_inline)) {
        const uint64_t w = __hip_atomic_load(reinterpret_cast<const uint64_t *>(p), __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
        return make_float2(__uint_as_float((uint32_t)w), __uint_as_float((uint32_t)(w >> 32)));
    };
    {
        float *mine = chunk_base(chunk);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 16; r += 2) put2(mine + (mt * 8 + r / 2) * 128, o[mt][r], o[mt][r + 1]);
        put2(mine + (MT * 8) * 128, m_used, l);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __shared__ int last;
    __syncthreads();
    if (tid == 0) {
        int *ctr = a.counters + rbk;
        const int done = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = done == nchunks - 1;
        if (last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last) return;
    // Merge in chunk order: M = the largest chunk maximum (log2 units), then
    // O = sum_c O_c 2^(m_c - M) and l likewise, chunk 0 first; this
    // workgroup's own chunk enters from registers at its place in the order.
    // The O of the first other chunk and the (m, l) pairs of all chunks go
    // out as one batch of uncached loads (one round trip); every further
    // chunk's O is one more batch.
    const int first_other = chunk == 0 ? 1 : 0;
    float2 x[MT * 8];
#pragma unroll
    for (int e = 0; e < MT * 8; ++e) x[e] = get2(chunk_base(first_other) + e * 128);
    float2 ml[kMaxChunks];
#pragma unroll
    for (int ch = 0; ch < kMaxChunks; ++ch)
        if (ch < nchunks) ml[ch] = ch == chunk ? make_float2(m_used, l) : get2(chunk_base(ch) + (MT * 8) * 128);
    float mmax = m_used, lsum = 0.0f;
#pragma unroll
    for (int ch = 0; ch < kMaxChunks; ++ch)
        if (ch < nchunks) mmax = fmaxf(mmax, ml[ch].x);
#pragma unroll
    for (int ch = 0; ch < kMaxChunks; ++ch)
        if (ch < nchunks) lsum = fmaf(ml[ch].y, __builtin_amdgcn_exp2f(ml[ch].x - mmax), lsum);
    floatx16_t acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[mt][r] = 0.0f;
#pragma unroll
    for (int ch = 0; ch < kMaxChunks; ++ch) {
        if (ch >= nchunks) break;
        if (ch == chunk) {
            const float w = __builtin_amdgcn_exp2f(m_used - mmax);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[mt][r] = fmaf(o[mt][r], w, acc[mt][r]);
            continue;
        }
        if (ch != first_other) {
#pragma unroll
            for (int e = 0; e < MT * 8; ++e) x[e] = get2(chunk_base(ch) + e * 128);
        }
        const float w = __builtin_amdgcn_exp2f(ml[ch].x - mmax);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                acc[mt][2 * r] = fmaf(x[mt * 8 + r].x, w, acc[mt][2 * r]);
                acc[mt][2 * r + 1] = fmaf(x[mt * 8 + r].y, w, acc[mt][2 * r + 1]);
            }
    }
    write_out(acc, lsum);
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
    const int spare = a.pool_items ? kPoolSpare : 0;
    const unsigned grid = a.chunk_tiles ? (unsigned)a.items : (unsigned)((per_xcd + spare) * kXcds);
    hipLaunchKernelGGL((prefill_mfma_kernel<D, HW>), dim3(grid), dim3(512), 0, stream, a);
    return hipGetLastError();
}

// Heads per workgroup: the largest of 8, 4, 2, 1 that divides the group.
int heads_per_workgroup(int group) { return group % 8 == 0 ? 8 : group % 4 == 0 ? 4 : group; }

// Key tiles of row block rb.
int row_block_tiles(const PrefillLaunch &l, int rows_per_block, int rb) {
    const int key_end = std::min(l.prior + l.queries, l.prior + (rb + 1) * rows_per_block);
    return (key_end + kBN - 1) / kBN;
}

}  // namespace

bool prefill_fast_path(int head_dim, int group) {
    return (head_dim == 64 || head_dim == 128) && (group == 1 || group == 2 || group % 4 == 0);
}

namespace {

// Predicted span, in 64-key tiles, of a launch whose row blocks split into
// chunks of tc tiles (tc >= the longest row block: no split).  The items go,
// longest first, to the CU of their XCD that frees first (each XCD takes its
// own kv heads when they divide evenly over the XCDs, as launch_prefill deals
// them; otherwise all CUs share one list); an item costs its tiles plus
// kItemFixedTiles (Q, the first copies, the partial or output write), and a
// row block split into n chunks ends (n - 1) * kMergeChunkTiles after its last
// chunk (the merge loads every other chunk's O as one uncached batch).  Fitted
// to every chunk length measured on 28 launches of 256 to 3,072 queries after
// 0 to 3,584 tokens, 4 to 8 heads per kv head: the chunk it picks is the
// fastest measured or within 3.5% of it.
constexpr double kItemFixedTiles = 7.0;
constexpr double kMergeChunkTiles = 4.0;

double split_span(const PrefillLaunch &l, int rows, int nrb, int groups, int subgroups, int tc) {
    const bool by_head = l.kv_heads % kXcds == 0;
    const int lists = by_head ? kXcds : 1;
    const int cus = by_head ? kCus / kXcds : kCus;
    double span = 0.0;
    std::vector<std::pair<int, int>> items;  // (tiles, row block key)
    std::vector<double> row_end((size_t)groups * nrb);
    for (int x = 0; x < lists; ++x) {
        items.clear();
        for (int hg = 0; hg < groups; ++hg) {
            if (by_head && ((hg / subgroups) / (l.kv_heads / kXcds)) % kXcds != x) continue;
            for (int rb = 0; rb < nrb; ++rb) {
                const int nkt = row_block_tiles(l, rows, rb);
                const int nc = (nkt + tc - 1) / tc;
                for (int c = 0; c < nc; ++c) items.push_back({c ? tc : nkt - (nc - 1) * tc, hg * nrb + rb});
            }
        }
        std::stable_sort(items.begin(), items.end(),
                         [](const std::pair<int, int> &a, const std::pair<int, int> &b) { return a.first > b.first; });
        std::vector<double> free_at(cus, 0.0);
        std::priority_queue<std::pair<double, int>, std::vector<std::pair<double, int>>,
                            std::greater<std::pair<double, int>>> cu;
        for (int c = 0; c < cus; ++c) cu.push({0.0, c});
        for (const auto &it : items) {
            auto top = cu.top();
            cu.pop();
            const double end = top.first + kItemFixedTiles + it.first;
            cu.push({end, top.second});
            row_end[(size_t)it.second] = std::max(row_end[(size_t)it.second], end);
            span = std::max(span, end);
        }
    }
    if (tc < (int)1e9) {
        for (int hg = 0; hg < groups; ++hg)
            for (int rb = 0; rb < nrb; ++rb) {
                const int nc = (row_block_tiles(l, rows, rb) + tc - 1) / tc;
                if (nc > 1) span = std::max(span, row_end[(size_t)hg * nrb + rb] + (nc - 1) * kMergeChunkTiles);
            }
    }
    return span;
}

PrefillSplit plan_split(const PrefillLaunch &l);

}  // namespace

// The plan depends on the shape only and costs up to a few hundred us of
// host time, so plans are kept per shape (a decoder repeats a few prompt-chunk
// shapes over every layer and sequence).
PrefillSplit prefill_split_plan(const PrefillLaunch &l) {
    const int group = l.q_heads / l.kv_heads;
    if (!l.split_allowed || !prefill_fast_path(l.head_dim, group)) return PrefillSplit{};
    const std::array<int, 5> key = {l.queries, l.prior, l.q_heads, l.kv_heads, l.head_dim};
    static std::mutex lock;
    static std::map<std::array<int, 5>, PrefillSplit> plans;
    {
        std::lock_guard<std::mutex> guard(lock);
        const auto it = plans.find(key);
        if (it != plans.end()) return it->second;
    }
    const PrefillSplit p = plan_split(l);
    std::lock_guard<std::mutex> guard(lock);
    if (plans.size() >= 4096) plans.clear();
    plans.emplace(key, p);
    return p;
}

namespace {

PrefillSplit plan_split(const PrefillLaunch &l) {
    PrefillSplit p;
    const int group = l.q_heads / l.kv_heads;
    const int hw = heads_per_workgroup(group);
    const int rows = 32 * (8 / hw);
    const int nrb = (l.queries + rows - 1) / rows;
    const int groups = l.kv_heads * (group / hw);
    if (nrb > 1024 || groups > 65535) return p;
    int64_t work = 0;
    int longest = 0;
    for (int rb = 0; rb < nrb; ++rb) {
        const int t = row_block_tiles(l, rows, rb);
        work += t;
        longest = std::max(longest, t);
    }
    work *= groups;
    // One workgroup per CU (128 KiB of LDS each): a launch is balanced when
    // its longest workgroup is close to the mean work per CU.
    const int64_t target = (work + kCus - 1) / kCus;
    // Every chunk but the last must end below the diagonal of its row block,
    // whose rows span rows / 64 + 1 key tiles; a chunk also costs a prologue
    // of three tile copies, so chunks are at least 4 tiles.
    const int min_chunk = std::max(4, rows / kBN + 2);
    if (longest <= target + target / 4 || longest <= min_chunk) return p;
    // Chunk lengths from a quarter below the mean work per CU to twice it
    // (those the item table and the merge hold), and no split at all, scored
    // by split_span; the shortest span wins, ties to the shorter chunk.
    const int subgroups = group / hw;
    const int lo = (int)std::max<int64_t>(min_chunk, target - target / 4);
    const int hi = (int)std::min<int64_t>(longest - 1, 2 * target);
    int best = 0;
    int64_t best_items = 0;
    double best_span = split_span(l, rows, nrb, groups, subgroups, (int)1e9);
    for (int tc = lo; tc <= hi; ++tc) {
        int64_t items = 0;
        for (int rb = 0; rb < nrb; ++rb) items += (row_block_tiles(l, rows, rb) + tc - 1) / tc;
        items *= groups;
        if (items > kMaxSplitItems || (longest + tc - 1) / tc > kMaxChunks) continue;
        const double span = split_span(l, rows, nrb, groups, subgroups, tc);
        if (span < best_span) {
            best_span = span;
            best = tc;
            best_items = items;
        }
    }
    if (!best) return p;
    p.chunk_tiles = best;
    p.items = (int)best_items;
    p.max_chunks = (longest + best - 1) / best;
    p.counters = groups * nrb;
    const int pairs = (l.head_dim / 32) * 8 + 1;
    p.partial_bytes = (size_t)groups * nrb * p.max_chunks * 8 * pairs * 64 * 2 * sizeof(float);
    return p;
}

}  // namespace

int prefill_pool_items(const PrefillLaunch &l) {
    const int group = l.q_heads / l.kv_heads;
    if (!l.pool_allowed || !prefill_fast_path(l.head_dim, group) || prefill_split_plan(l).chunk_tiles) return 0;
    const int hw = heads_per_workgroup(group);
    const int rows = 32 * (8 / hw);
    const int64_t total = (int64_t)((l.queries + rows - 1) / rows) * l.kv_heads * (group / hw);
    const int64_t per_xcd = (total + kXcds - 1) / kXcds;
    // Only launches with at least two row blocks per CU queue any; then the
    // shortest quarter of every slice, at most kPoolMax.  At cfg4's 256 row
    // blocks per XCD, 64 and 96 measured equally fast and 32 slower; every
    // pooled row block that another XCD takes reads its kv head's K/V from
    // beyond that XCD's L2 (fetched per call: 281 MB without a pool, 344 MB
    // with 64, 448 MB with 96, 526 MB with 128).
    if (per_xcd < 2 * (kCus / kXcds)) return 0;
    return (int)std::min<int64_t>(kPoolMax, per_xcd / 4);
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
    const int hw = heads_per_workgroup(group);
    const PrefillSplit plan = prefill_split_plan(l);
    if (plan.chunk_tiles) {
        if (!l.partial || !l.counters) return hipErrorInvalidValue;
        // Items (row block, chunk, head group), longest first; the chunks of
        // a row block are counted back from its last tile, chunk 0 taking the
        // remainder (the kernel recomputes the same ranges).
        const int rows = 32 * (8 / hw);
        const int nrb = (l.queries + rows - 1) / rows;
        const int groups = l.kv_heads * (group / hw);
        //
        // Workgroup L runs on XCD L % 8.  When the kv heads split evenly over
        // the XCDs, each XCD gets the items of its own kv heads, longest
        // first, so its L2 holds few heads' K/V (as the unsplit mapping
        // does); otherwise one longest-first list is dealt round-robin.
        std::vector<std::vector<std::pair<int, uint32_t>>> buckets(kXcds);
        const bool by_head = l.kv_heads % kXcds == 0;
        for (int hg = 0; hg < groups; ++hg)
            for (int rb = nrb - 1; rb >= 0; --rb) {
                const int nkt = row_block_tiles(l, rows, rb);
                const int nc = (nkt + plan.chunk_tiles - 1) / plan.chunk_tiles;
                for (int c = 0; c < nc; ++c) {
                    const int size = c ? plan.chunk_tiles : nkt - (nc - 1) * plan.chunk_tiles;
                    const int kvh = hg / (group / hw);
                    buckets[by_head ? (kvh / (l.kv_heads / kXcds)) % kXcds : 0].push_back(
                        {size, (uint32_t)rb | ((uint32_t)c << 10) | ((uint32_t)hg << 16)});
                }
            }
        auto longest_first = [](const std::pair<int, uint32_t> &x, const std::pair<int, uint32_t> &y) {
            return x.first > y.first;
        };
        size_t slots = 0;
        if (by_head) {
            size_t most = 0;
            for (auto &b : buckets) {
                std::stable_sort(b.begin(), b.end(), longest_first);
                most = std::max(most, b.size());
            }
            slots = most * kXcds;
            if (slots > (size_t)kMaxSplitItems) return hipErrorInvalidValue;
            for (size_t j = 0; j < most; ++j)
                for (int x = 0; x < kXcds; ++x)
                    a.item[j * kXcds + x] = j < buckets[x].size() ? buckets[x][j].second : kNoItem;
        } else {
            std::stable_sort(buckets[0].begin(), buckets[0].end(), longest_first);
            slots = buckets[0].size();
            for (size_t i = 0; i < slots; ++i) a.item[i] = buckets[0][i].second;
        }
        a.chunk_tiles = plan.chunk_tiles;
        a.max_chunks = plan.max_chunks;
        a.items = (int)slots;
        a.partial = l.partial;
        a.counters = l.counters;
    } else if (const int pool = prefill_pool_items(l)) {
        if (!l.pool_counter) return hipErrorInvalidValue;
        a.pool_items = pool;
        a.pool_counter = l.pool_counter;
    }
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
