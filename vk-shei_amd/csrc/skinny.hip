// BF16 projections of decode batches (tokens <= 16) on MFMA:
//   out[t][r] = BF16(sum_k x[t][k] * w[r][k]),  fp32 accumulation.
// The decode projections of the reference (llm_fused_qkv_bf16,
// llm_fused_swiglu_bf16 and the reuse-8 GEMV, gpu_llm.cl:553-596, :740-834;
// with its HIP backend the same products go to hipBLASLt, gpu_resources.rs:
// 366-378) stream every weight once per step, so the work is HBM-bound on the
// weights; the token vectors are a few hundred KiB and stay in L2.
//
// Workgroups of 8 wavefronts work through tiles of 16 weight rows (a grid
// of a few workgroups per CU, each taking every grid-th tile).  A tile's sum
// over the inner dimension is cut into 16 partial sums: partial j folds the
// 128-input blocks j, j + 16, ... in order, four v_mfma_f32_16x16x32_bf16
// steps per block with the weights as A (16 rows x 32 inputs, one 16-byte
// load per lane) and the tokens as B (32 inputs x 16 tokens, padded with
// zeros); wavefront w keeps partials w and w + 8, and the 16 partial 16x16
// tiles are added in LDS in order 0 .. 15.  That order depends on the inner
// dimension only, so a product gives the same bits in every entry point,
// fused form and launch shape.  Each wavefront keeps a ring of two (or
// four) load batches in flight, and the next tile's first batches go out
// before a tile's partials are summed.
//
// When the token rows fit (<= 8 tokens of <= 4096 inputs) the workgroup
// stages them in LDS once for all its tiles, by DMA while its first weight
// batches are in flight (the per-k-step B loads cost a quarter of the
// streaming rate when they go to L2), and can apply the
// RMSNorm that precedes the product there: the reference's llm_rmsnorm
// (gpu_llm.cl:72-98) with its 128-lane strided sums, 64..1 tree and BF16
// stages, bit-identical to mslim_attn_rmsnorm followed by the product.
// Epilogues:
//   plain   out = BF16(acc)
//   add     out = BF16(resid + BF16(acc))           (llm_add after the product)
//   swiglu  out = SwiGLU(BF16(acc_gate), BF16(acc_up))   (llm_swiglu after both;
//           its first stage read from the context's table of every gate value).
//           A tile is 8 outputs: rows 0-7 of the A operand are their gate
//           rows and rows 8-15 their up rows, so the two sums of an output
//           meet in lanes l and l + 32 (14,336 outputs make 1,792 tiles, 7
//           per CU, where 16 gate plus 16 up rows per tile left 3.5)
// which equal the unfused product followed by the elementwise kernel bit for
// bit.  Up to three matrices with separate outputs share one launch (Q, K, V).
#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <type_traits>

namespace mslim {

namespace {

constexpr int kTileRows = 16;
// The k range of a tile is cut into blocks of kBlock inputs; partial sum j
// (of kSlots) folds blocks j, j + kSlots, ... in ascending order, four MFMA
// steps per block, and the tile's result is the partials added in order
// 0 .. kSlots-1.  That order depends on the inner dimension only, so every
// launch shape and entry point gives the same bits for the same product.
constexpr int kSlots = 16;
constexpr int kUnroll = 4;   // MFMA steps (16-byte weight loads per lane) per block
constexpr int kBlock = 32 * kUnroll;
constexpr int kMaxSegments = 3;
constexpr int kCus = 256;

// kQkvRope: Q, K and V with RoPE and the K/V append in the epilogue.
enum Epilogue { kPlain = 0, kAdd = 1, kSwiglu = 2, kQkvRope = 3 };

struct SkinnyArgs {
    const uint16_t *w[kMaxSegments];
    uint16_t *out[kMaxSegments];
    int rows[kMaxSegments];
    int first_tile[kMaxSegments];
    int segments;
    int tiles;
    const uint16_t *x;       // [tokens][inner]
    const uint16_t *w_up;    // swiglu: up weights beside w[0] (gate)
    const uint16_t *resid;   // add: [tokens][rows[0]], may equal out[0]
    const uint16_t *norm_w;  // staged rows only: RMSNorm weights [inner], or null
    const uint16_t *act_table;  // swiglu: swiglu_act_bf16 of every BF16 gate value
    float eps;
    int inner, tokens;
    // kQkvRope: segments Q, K, V; token t at positions[t] in page-table row t
    const int32_t *positions, *page_table;
    uint16_t *k_pool, *v_pool;
    int pages_per_seq, shift, kv_heads, head_dim;
    RopeCosSin cossin;
};

// The inverse-frequency table rides in the kernel arguments of the RoPE
// variant only.
struct NoRope {};
template <int EPI>
using RopeArg = typename std::conditional<EPI == kQkvRope, RopeTable, NoRope>::type;

__device__ __forceinline__ bf16x8_t load8(const uint16_t *p) { return *reinterpret_cast<const bf16x8_t *>(p); }

// Token vectors staged in LDS (XLDS): up to kStageTokens rows of up to
// kStageInner inputs, 8 KiB per row, with 16-byte chunk c of row r stored at
// chunk c ^ (r & 7), so that the eight rows of a B fragment read (same c)
// fall in different banks.
constexpr int kStageTokens = 8;
constexpr int kStageInner = 4096;
constexpr int kStageBytes = kStageTokens * kStageInner * 2;
constexpr int kPartialBytes = kSlots * 64 * 16;  // one matrix's partial tiles
// RMSNorm weights staged in the partial space, after the norm scratch.
constexpr uint32_t kNormWeightOffset = 4096;
static_assert(kNormWeightOffset + kStageInner * 2 <= kPartialBytes, "RMSNorm weights fit the partial space");

__device__ __forceinline__ int stage_index(int row, int col) {
    return row * kStageInner + ((((col >> 3) ^ row) & 7) | ((col >> 3) & ~7)) * 8 + (col & 7);
}

template <int EPI, bool XLDS, bool NORM, int WAVES, int DEPTH>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(4))) void skinny_kernel(
    SkinnyArgs a, RopeArg<EPI> rope) {
    // Partial slots per wavefront, MFMA steps per load batch and batches per
    // block.
    constexpr int NS = kSlots / WAVES;
    constexpr int UB = kUnroll;
    constexpr int PB = kUnroll / UB;
    constexpr int kTileOut = EPI == kSwiglu ? kTileRows / 2 : kTileRows;  // outputs per tile
    // Batches per loop iteration: a multiple of the ring depth and of the
    // slot cycle (powers of two), so that every batch's ring entry and
    // accumulator are known at compile time.
    constexpr int PERIOD = PB * NS > DEPTH ? PB * NS : DEPTH;
    constexpr int kThreads = WAVES * 64;
    // LDS: the staged rows, then the partial tiles; the RMSNorm scratch
    // lives in the partial space before the first tile ends.
    __shared__ __align__(16) unsigned char lds[(XLDS ? kStageBytes : 0) + kPartialBytes];
    uint16_t *xs = reinterpret_cast<uint16_t *>(lds);
    auto partial = reinterpret_cast<floatx4_t(*)[64]>(lds + (XLDS ? kStageBytes : 0));
    // wave is uniform: the k range of a batch and its bounds tests are
    // scalar, so a step's B read is branched on, not masked lane by lane
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kq = (lane >> 4) * 8;
    const int tok = lane & 15;
    const bool live = tok < a.tokens;
    // Column j of an MFMA result depends on column j of B only, and the
    // columns of tokens past the batch are never written: their lanes read a
    // staged row that exists (whatever it holds) instead of being masked.
    const int xrow = min(tok, kStageTokens - 1);
    const bf16x8_t zero = {};

    // The tile's weights: lane l holds row r0 + l % 16, inputs 8 (l / 16) ..
    // +7 of each 32-input step; rows past the end re-read the last row and
    // are not written.
    // With RoPE, a Q or K tile takes 8 rows of the first half of a head
    // and their 8 rotate-half partners (rows 8 .. 15 of the tile); a SwiGLU
    // tile takes the gate rows of 8 outputs and then their up rows.  Either
    // way each pair meets in lanes l and l + 32 of the output, and which rows
    // a tile reads changes nothing in how each output is summed.
    struct Tile {
        const uint16_t *wp;
        uint16_t *out;
        int rows, r0, seg;
    };
    auto rope_row = [&](int r0, int i) __attribute__((always_inline)) {
        const int tph = a.head_dim / 16;  // tiles per head
        const int tl = r0 / kTileRows;
        return (tl / tph) * a.head_dim + (tl % tph) * 8 + (i < 8 ? i : a.head_dim / 2 + i - 8);
    };
    auto tile_of = [&](int tile) __attribute__((always_inline)) {
        int seg = 0;
        if (a.segments > 1 && tile >= a.first_tile[1]) seg = 1;
        if (a.segments > 2 && tile >= a.first_tile[2]) seg = 2;
        Tile t;
        t.rows = a.rows[seg];
        t.seg = seg;
        t.r0 = (tile - a.first_tile[seg]) * kTileOut;
        if constexpr (EPI == kSwiglu) {
            const int row = min(t.r0 + (lane & 7), t.rows - 1);
            t.wp = ((lane & 15) < 8 ? a.w[seg] : a.w_up) + (int64_t)row * a.inner + kq;
        } else {
            const int row =
                EPI == kQkvRope && seg < 2 ? rope_row(t.r0, lane & 15) : min(t.r0 + (lane & 15), t.rows - 1);
            t.wp = a.w[seg] + (int64_t)row * a.inner + kq;
        }
        t.out = a.out[seg];
        return t;
    };
    struct Batch {
        bf16x8_t wa[UB], xb[UB];
    };
    const uint16_t *xp = a.x + (int64_t)(live ? tok : 0) * a.inner + kq;
    // inner % 32 == 0: a step that starts inside the row ends inside it.
    auto load_batch = [&](Batch &bt, const Tile &t, int k0) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < UB; ++u) {
            const int k = k0 + u * 32;
            const bool in = k < a.inner;
            bt.wa[u] = in ? load8(t.wp + k) : zero;
            if (!XLDS) bt.xb[u] = in && live ? load8(xp + k) : zero;
        }
    };
    // The same with every load issued (addresses clamped into the row,
    // values past it replaced by zeros): a fixed count of vector memory
    // instructions, kRingLoads for a whole ring.
    auto load_batch_all = [&](Batch &bt, const Tile &t, int k0) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < UB; ++u) {
            const int k = k0 + u * 32;
            const int kc = min(k, a.inner - 32);
            const bf16x8_t w = load8(t.wp + kc);
            bt.wa[u] = k < a.inner ? w : zero;
        }
    };
    constexpr int kRingLoads = DEPTH * UB;
    floatx4_t acc[NS];
    auto use_batch = [&](const Batch &bt, int k0, int m) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < UB; ++u) {
            const int k = k0 + u * 32;
            bf16x8_t xb;
            if (XLDS) xb = k < a.inner ? *reinterpret_cast<const bf16x8_t *>(xs + stage_index(xrow, k + kq)) : zero;
            else xb = bt.xb[u];
            acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bt.wa[u], xb, acc[m], 0, 0, 0);
        }
    };
    // Batch i of a wavefront: block wave + (i / PB) * WAVES, part i % PB.
    auto k_of = [&](int kb0, int u) __attribute__((always_inline)) {
        return kb0 + (u / PB) * WAVES * kBlock + (u % PB) * 32 * UB;
    };
    const int kfirst = wave * kBlock;

    // kQkvRope: the lane's token position, the pool row of kv head 0 at it
    // (-1: nothing to append) and the c and s of its four output rows, loaded
    // after the tile's k loop, behind the next tile's first weight batches,
    // so that they arrive while the partial tiles are exchanged.
    struct RopeIn {
        int pos, row;
        float cs[4], sn[4];
    };
    auto rope_fetch = [&](const Tile &cur) __attribute__((always_inline)) {
        RopeIn in{};
        in.row = -1;
        if constexpr (EPI == kQkvRope) {
            in.pos = a.positions[tok];
            if (in.pos >= 0 && (int64_t)in.pos < ((int64_t)a.pages_per_seq << a.shift)) {
                const int page = a.page_table[(int64_t)tok * a.pages_per_seq + (in.pos >> a.shift)];
                in.row = ((page * a.kv_heads) << a.shift) + (in.pos & ((1 << a.shift) - 1));
            }
            if (cur.seg < 2) {
                const int half = a.head_dim / 2;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int f = rope_row(cur.r0, 4 * (lane >> 4) + j) % a.head_dim % half;
                    rope_cs(a.cossin, in.pos, f, half, rope.inv[f], in.cs[j], in.sn[j]);
                }
            }
        }
        return in;
    };

    // kQkvRope output (wave 0, live lanes): BF16 of each sum as the plain
    // product writes it, then for Q and K the rotation of rope_append
    // (x c + (-+partner) s, each product rounded, BF16 sum), Q to out[0] and
    // K and V into the page pools at the token's position; positions outside
    // the page table append nothing, as rope_append.
    auto rope_epilogue = [&](const Tile &cur, const floatx4_t &sum, const RopeIn &in) __attribute__((always_inline)) {
        if constexpr (EPI == kQkvRope) {
            const int rp_row = in.row;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int i = 4 * (lane >> 4) + j;
                const uint16_t y = write_bf16(sum[j]);
                if (cur.seg == 2) {
                    const int r = cur.r0 + i;
                    if (rp_row >= 0 && r < cur.rows)
                        a.v_pool[((int64_t)rp_row + ((int64_t)(r / a.head_dim) << a.shift)) * a.head_dim +
                                 r % a.head_dim] = y;
                    continue;
                }
                const uint16_t partner = (uint16_t)__shfl_xor((int)y, 32, 64);
                const int r = rope_row(cur.r0, i);
                const int head = r / a.head_dim, d = r % a.head_dim;
                const float p = read_bf16(partner);
                const float left = round_bf16(__fmul_rn(read_bf16(y), in.cs[j]));
                const float right = round_bf16(__fmul_rn(i < 8 ? -p : p, in.sn[j]));
                const uint16_t o = write_bf16(__fadd_rn(left, right));
                if (cur.seg == 0) cur.out[(int64_t)tok * cur.rows + r] = o;
                else if (rp_row >= 0)
                    a.k_pool[((int64_t)rp_row + ((int64_t)head << a.shift)) * a.head_dim + d] = o;
            }
        }
    };

    // kAdd: wave 0's residual values of a tile (lane l: token l % 16, rows
    // r0 + 4 (l / 16) + j) are loaded before the tile's first weight batches,
    // so their latency passes under the k loop instead of after the fold;
    // being older than every batch, they change none of the waits for the
    // batches.  A tile reads only its own rows, so out == resid is safe.
    uint16_t res_next[4] = {}, res_cur[4] = {};
    auto resid_fetch = [&](const Tile &tt) __attribute__((always_inline)) {
        if constexpr (EPI == kAdd) {
            if (wave == 0 && live) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int r = tt.r0 + 4 * (lane >> 4) + j;
                    if (r < tt.rows) res_next[j] = a.resid[(int64_t)tok * tt.rows + r];
                }
            }
        }
    };

    int tile = blockIdx.x;
    Batch ring[DEPTH];
    Tile t = tile_of(tile);
    resid_fetch(t);
    if constexpr (!XLDS) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d)
            if (k_of(kfirst, d) < a.inner) load_batch(ring[d], t, k_of(kfirst, d));
    } else {
        // The B operand (token rows) is the same for every row tile: it goes
        // to LDS once per workgroup, by DMA (global_load_lds_dwordx4, no
        // registers held), ahead of the first DEPTH weight batches, which
        // then stay in flight through the staging and the RMSNorm: the wait
        // below leaves exactly the kRingLoads weight loads outstanding.
        // Wave instruction j fills LDS chunks 64 j .. 64 j + 63, i.e. row
        // j / 8; lane l takes the row's logical chunk (64 (j % 8) + l) ^
        // (row & 7).
        const int chunks = a.inner / 8;
        const uint32_t xs_lds = lds_offset(xs);
        for (int j = wave; j < a.tokens * (kStageInner / 8 / 64); j += WAVES) {
            const int r = j >> 3;
            const int c = ((j & 7) * 64 + lane) ^ (r & 7);
            if (c < chunks) dma16_async(a.x, (uint32_t)(r * a.inner + c * 8) * 2u, xs_lds + (uint32_t)j * 1024u);
        }
        if constexpr (NORM) {
            // the RMSNorm weights into the partial space, after its scratch
            for (int j = wave; j * 64 < chunks; j += WAVES)
                if (j * 64 + lane < chunks)
                    dma16_async(a.norm_w, (uint32_t)(j * 64 + lane) * 16u,
                                lds_offset(partial) + kNormWeightOffset + (uint32_t)j * 1024u);
        }
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) load_batch_all(ring[d], t, k_of(kfirst, d));
        // The DMA is not tracked by the compiler: wait for it by count.
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(kRingLoads));
        __syncthreads();
        if constexpr (NORM) {
            // RMSNorm of each staged row (gpu_llm.cl:72-98) as
            // mslim_attn_rmsnorm computes it: 128 lanes per row, lane g sums
            // elements g, g + 128, ... in order; the tree adds pairs
            // (g, g + 64) through LDS, then 32 .. 1 by shuffles.  A group of
            // 128 lanes takes rows grp, grp + kGroups, ...
            constexpr int kGroups = kThreads / 128;
            constexpr int kRowsPerGroup = kStageTokens / kGroups;
            float *norm_part = reinterpret_cast<float *>(partial);    // [kStageTokens][64]
            float *norm_factor = norm_part + kStageTokens * 64;      // [kStageTokens]
            const uint16_t *norm_w = reinterpret_cast<const uint16_t *>(
                reinterpret_cast<const unsigned char *>(partial) + kNormWeightOffset);
            const int grp = threadIdx.x >> 7, g = threadIdx.x & 127;
            float s[kRowsPerGroup];
#pragma unroll
            for (int rr = 0; rr < kRowsPerGroup; ++rr) {
                const int r = grp + rr * kGroups;
                s[rr] = 0.0f;
                if (r < a.tokens) {
                    // Element g + 128 k of the row sits 128 k elements after
                    // element g (the swizzle permutes chunks within groups
                    // of 64 elements), so one base address with immediate
                    // offsets serves every read.  Eight reads go ahead of
                    // their FMAs, in element order; elements past the row's
                    // end would add exact zeros (the sum is never -0) and
                    // are left out.
                    const uint16_t *rowp = xs + stage_index(r, g);
                    const int steps = a.inner / 128;
                    int k = 0;
                    for (; k + 8 <= steps; k += 8) {
                        float e[8];
#pragma unroll
                        for (int j = 0; j < 8; ++j) e[j] = read_bf16(rowp[128 * (k + j)]);
#pragma unroll
                        for (int j = 0; j < 8; ++j) s[rr] = __fmaf_rn(e[j], e[j], s[rr]);
                    }
                    for (; k < steps; ++k) {
                        const float v = read_bf16(rowp[128 * k]);
                        s[rr] = __fmaf_rn(v, v, s[rr]);
                    }
                    if (g + 128 * steps < a.inner) {
                        const float v = read_bf16(rowp[128 * steps]);
                        s[rr] = __fmaf_rn(v, v, s[rr]);
                    }
                    if (g >= 64) norm_part[r * 64 + g - 64] = s[rr];
                }
            }
            __syncthreads();
#pragma unroll
            for (int rr = 0; rr < kRowsPerGroup; ++rr) {
                const int r = grp + rr * kGroups;
                if (r < a.tokens && g < 64) {
                    float sum = __fadd_rn(s[rr], norm_part[r * 64 + g]);
#pragma unroll
                    for (int stride = 32; stride > 0; stride >>= 1)
                        sum = __fadd_rn(sum, __shfl_down(sum, stride, 64));
                    if (g == 0) {
                        const float mean = __fdiv_rn(sum, (float)a.inner);
                        norm_factor[r] = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(mean, a.eps)));
                    }
                }
            }
            __syncthreads();
            // BF16(BF16(x * factor) * w), eight elements per chunk, in place:
            // thread t takes chunk t % kRowChunks of rows t / kRowChunks,
            // + kThreads / kRowChunks, ..., so its weights are read and
            // widened once.
            constexpr int kRowChunks = kStageInner / 8;
            const int c = (int)threadIdx.x % kRowChunks;
            if (c < chunks) {
                const bf16x8_t wv = *reinterpret_cast<const bf16x8_t *>(norm_w + c * 8);
                float wf[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) wf[e] = (float)wv[e];
                for (int r = (int)threadIdx.x / kRowChunks; r < a.tokens; r += kThreads / kRowChunks) {
                    bf16x8_t *p = reinterpret_cast<bf16x8_t *>(xs + stage_index(r, c * 8));
                    const bf16x8_t xv = *p;
                    const float f = norm_factor[r];
                    bf16x8_t y;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const __bf16 n = (__bf16)__fmul_rn((float)xv[e], f);
                        y[e] = (__bf16)__fmul_rn((float)n, wf[e]);
                    }
                    *p = y;
                }
            }
            __syncthreads();
        }
    }


    while (true) {
#pragma unroll
        for (int m = 0; m < NS; ++m) acc[m] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
        // A ring of DEPTH batches: batch i + DEPTH loads into batch i's
        // registers once batch i is used.
        for (int kb0 = kfirst; kb0 < a.inner; kb0 += (PERIOD / PB) * WAVES * kBlock) {
#pragma unroll
            for (int u = 0; u < PERIOD; ++u) {
                Batch &b = ring[u % DEPTH];
                const int k = k_of(kb0, u);
                if (k < a.inner) {
                    use_batch(b, k, (u / PB) % NS);
                    const int kn = k_of(kb0, u + DEPTH);
                    if (kn < a.inner) load_batch(b, t, kn);
                }
            }
        }
        // The next tile's first batches go out before this tile's partials
        // are summed.
        const Tile cur = t;
#pragma unroll
        for (int j = 0; j < 4; ++j) res_cur[j] = res_next[j];
        const int next = tile + (int)gridDim.x;
        if (next < a.tiles) {
            t = tile_of(next);
            resid_fetch(t);
#pragma unroll
            for (int d = 0; d < DEPTH; ++d)
                if (k_of(kfirst, d) < a.inner) load_batch(ring[d], t, k_of(kfirst, d));
        }
        RopeIn rin{};
        if (EPI == kQkvRope && wave == 0 && live) rin = rope_fetch(cur);
        floatx4_t sum;
#pragma unroll
        for (int m = 0; m < NS; ++m) partial[wave + m * WAVES][lane] = acc[m];
        __syncthreads();
        if (wave == 0) {
            sum = partial[0][lane];
            for (int j = 1; j < kSlots; ++j) sum += partial[j][lane];
        }
        __syncthreads();  // the partials are read before they are written again
        if constexpr (EPI == kQkvRope) {
            if (wave == 0 && live) rope_epilogue(cur, sum, rin);
        } else if constexpr (EPI == kSwiglu) {
            if (wave == 0 && live) {
                // lane l < 32 holds the gate sums of outputs r0 + 4 (l / 16)
                // + j, lane l + 32 the up sums of the same outputs
                float up[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) up[j] = __shfl_xor(sum[j], 32, 64);
                if (lane < 32) {
                    uint16_t *out = cur.out + (int64_t)tok * cur.rows;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int r = cur.r0 + 4 * (lane >> 4) + j;
                        if (r < cur.rows) out[r] = swiglu_mul_bf16(a.act_table[write_bf16(sum[j])], write_bf16(up[j]));
                    }
                }
            }
        } else if (wave == 0 && live) {
            // D layout: lane l holds rows 4*(l/16) + j, token l%16.
            uint16_t *out = cur.out + (int64_t)tok * cur.rows;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int r = cur.r0 + 4 * (lane >> 4) + j;
                if (r >= cur.rows) continue;
                const uint16_t y = write_bf16(sum[j]);
                if (EPI == kPlain) out[r] = y;
                else out[r] = write_bf16(__fadd_rn(read_bf16(res_cur[j]), read_bf16(y)));
            }
        }
        if (next >= a.tiles) break;
        tile = next;
    }
}

// Tiles of a matrix of `rows` outputs: 16 rows each, or 8 gate/up pairs.
int tiles_of(int epi, int rows) {
    const int per = epi == kSwiglu ? kTileRows / 2 : kTileRows;
    return (rows + per - 1) / per;
}

// Launch shape, measured at the cfg5 decode shapes (1 and 8 tokens, weights
// cycled through more memory than the last-level cache): workgroups of 8
// wavefronts, at most two per CU (a grid of at most 512, each workgroup
// taking every grid-th tile), ahead of 16 wavefronts with one (QKV's 384
// tiles then all run at once, and one workgroup's reduction overlaps the
// other's loads), and a two-deep ring of load batches (four gained nothing
// and spills when the token rows are not staged).  The paired SwiGLU tiles
// run best on the same grid (at 8 tokens, RMSNorm + gate/up 46.1 us against
// 49.1 with four workgroups per CU, 55.5 with one and 58.8 with one per
// tile), with a four-deep ring when the token rows are staged (45.2 against
// 46.1 us; the same at 1 token and without the RMSNorm).
constexpr int kPerCu = 2;

template <int EPI, bool XLDS, bool NORM>
hipError_t launch_with(SkinnyArgs &a, hipStream_t stream, const RopeArg<EPI> &rope = {}) {
    int tiles = 0;
    for (int s = 0; s < a.segments; ++s) {
        a.first_tile[s] = tiles;
        tiles += tiles_of(EPI, a.rows[s]);
    }
    a.tiles = tiles;
    const unsigned grid = (unsigned)std::min(tiles, kPerCu * kCus);
    if constexpr (EPI == kSwiglu && XLDS)
        hipLaunchKernelGGL((skinny_kernel<EPI, XLDS, NORM, 8, 4>), dim3(grid), dim3(8 * 64), 0, stream, a, rope);
    else
        hipLaunchKernelGGL((skinny_kernel<EPI, XLDS, NORM, 8, 2>), dim3(grid), dim3(8 * 64), 0, stream, a, rope);
    return hipGetLastError();
}

template <int EPI>
hipError_t launch(SkinnyArgs &a, hipStream_t stream) {
    if (a.tokens <= kStageTokens && a.inner <= kStageInner) {
        if (a.norm_w) return launch_with<EPI, true, true>(a, stream);
        return launch_with<EPI, true, false>(a, stream);
    }
    if (a.norm_w) return hipErrorInvalidValue;  // the caller normalises first
    return launch_with<EPI, false, false>(a, stream);
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

bool skinny_supported(int inner, int tokens, const void *x, const void *w0, const void *w1, const void *w2) {
    return tokens >= 1 && tokens <= kSkinnyMaxTokens && inner >= 32 && inner % 32 == 0 && aligned16(x) &&
           aligned16(w0) && aligned16(w1) && aligned16(w2);
}

bool skinny_norm_supported(int inner, int tokens, const void *norm_w) {
    return tokens <= kStageTokens && inner <= kStageInner && aligned16(norm_w);
}

hipError_t launch_skinny_gemm(const SkinnyMatrix *m, int count, const uint16_t *x, int inner, int tokens,
                              hipStream_t stream, const uint16_t *norm_w, float eps) {
    SkinnyArgs a{};
    for (int s = 0; s < count; ++s) {
        a.w[s] = m[s].w;
        a.out[s] = m[s].out;
        a.rows[s] = m[s].rows;
    }
    a.segments = count;
    a.x = x;
    a.inner = inner;
    a.tokens = tokens;
    a.norm_w = norm_w;
    a.eps = eps;
    return launch<kPlain>(a, stream);
}

bool skinny_rope_supported(int inner, int tokens, int head_dim, const void *x, const void *wq, const void *wk,
                           const void *wv, const void *norm_w) {
    return skinny_supported(inner, tokens, x, wq, wk, wv) && tokens <= kStageTokens && inner <= kStageInner &&
           aligned16(norm_w) && head_dim % 16 == 0 && head_dim >= 16 && head_dim <= 2 * kRopeTable;
}

hipError_t launch_skinny_qkv_rope(const SkinnyMatrix *m, const uint16_t *x, int inner, int tokens,
                                  const uint16_t *norm_w, float eps, const SkinnyRope &r, hipStream_t stream) {
    SkinnyArgs a{};
    for (int s = 0; s < 3; ++s) {
        a.w[s] = m[s].w;
        a.out[s] = m[s].out;
        a.rows[s] = m[s].rows;
    }
    a.segments = 3;
    a.x = x;
    a.inner = inner;
    a.tokens = tokens;
    a.norm_w = norm_w;
    a.eps = eps;
    a.positions = r.positions;
    a.page_table = r.page_table;
    a.k_pool = r.k_pool;
    a.v_pool = r.v_pool;
    a.pages_per_seq = r.pages_per_seq;
    a.shift = r.shift;
    a.kv_heads = r.kv_heads;
    a.head_dim = r.head_dim;
    a.cossin = r.cossin;
    const RopeTable &table =
        rope_inverse_table(r.head_dim, r.theta, r.llama3, r.factor, r.low, r.high, r.original_max);
    if (!norm_w) return launch_with<kQkvRope, true, false>(a, stream, table);
    return launch_with<kQkvRope, true, true>(a, stream, table);
}

hipError_t launch_skinny_gemm_add(const SkinnyMatrix &m, const uint16_t *resid, const uint16_t *x, int inner,
                                  int tokens, hipStream_t stream) {
    SkinnyArgs a{};
    a.w[0] = m.w;
    a.out[0] = m.out;
    a.rows[0] = m.rows;
    a.segments = 1;
    a.resid = resid;
    a.x = x;
    a.inner = inner;
    a.tokens = tokens;
    return launch<kAdd>(a, stream);
}

hipError_t launch_skinny_swiglu(const uint16_t *w_gate, const uint16_t *w_up, uint16_t *out, int rows,
                                const uint16_t *x, int inner, int tokens, const uint16_t *act_table,
                                hipStream_t stream, const uint16_t *norm_w, float eps) {
    SkinnyArgs a{};
    a.w[0] = w_gate;
    a.w_up = w_up;
    a.out[0] = out;
    a.rows[0] = rows;
    a.segments = 1;
    a.x = x;
    a.inner = inner;
    a.tokens = tokens;
    a.norm_w = norm_w;
    a.eps = eps;
    a.act_table = act_table;
    return launch<kSwiglu>(a, stream);
}

}  // namespace mslim
