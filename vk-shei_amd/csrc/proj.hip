// BF16 projections of prompt chunks on MFMA (more than 16 token rows):
//   out[t][r] = BF16(sum_k x[t][k] * w[r][k]),  fp32 accumulation, rounded once.
// The prefill products of the reference (llm_prefill_gemv_reuse8/16/32,
// llm_prefill_fused_qkv_reuse8 and llm_prefill_fused_swiglu_reuse8,
// gpu_llm.cl:553-683, :1253-1383, driven from gpu_llm/prefill.rs:132-290;
// tv_hip_matrix_multiply, hipblaslt_bridge.cpp:203-233, under its HIP
// backend) as one hand-written gfx950 kernel:
//   * a workgroup of four wavefronts (one per SIMD) owns 128 weight rows x BN
//     token rows of the output; each wavefront WM x 64 (WM = 32, BN = 64 for
//     launches of few tiles; WM = 64, BN = 128 otherwise), as blocks of
//     v_mfma_f32_32x32x16_bf16 with the weights as A (rows = M) and the token
//     rows as B (N), so a lane ends up with 4 consecutive output rows of one
//     token per 4 accumulators;
//   * both operands are K-contiguous; 64-element k-steps of both move HBM ->
//     LDS with global_load_lds_dwordx4 into a three-stage ring (128-byte rows,
//     16-byte slots XOR-swizzled by (row / 2) % 8, so every 16 rows of a
//     fragment read fall in distinct banks), one barrier per k-step;
//   * the last sub-step's MFMAs of a k-step run after the next barrier, behind
//     the next stage's first fragment reads;
//   * tiles are dealt to XCDs in contiguous slices with the token tiles of a
//     weight slice adjacent, so each weight row is read from HBM by one XCD;
//   * epilogues: plain, residual add (out = BF16(resid + BF16(acc)), llm_add
//     after the product), SwiGLU of a gate and an up product computed in the
//     same tile (llm_swiglu after both), and up to three matrices with their
//     own outputs in one launch (Q, K, V), each equal bit for bit to the
//     plain product followed by the elementwise kernel.
// Every output is summed by one wavefront in fixed k order, so results do not
// depend on the tiling or on timing: a fused launch equals the separate ones.
// Shapes outside the fast path (inner not a multiple of 64, unaligned
// pointers) run proj_generic_kernel: one wavefront per output, lane-strided
// partial sums and a fixed reduction tree.
#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>

namespace mslim {

namespace {

constexpr int kBM = 128;   // weight rows per workgroup tile
constexpr int kBK = 64;    // inputs per k-step
constexpr int kStages = 3; // LDS ring stages
constexpr int kKAlign = kBK;  // inner must be a multiple of this for the tiled kernel
constexpr int kXcds = 8;
constexpr int kMaxSeg = 3;

enum Epi { kPlain = 0, kAdd = 1, kSwiglu = 2 };

struct ProjArgs {
    const uint16_t *w[kMaxSeg];
    uint16_t *out[kMaxSeg];
    int rows[kMaxSeg];
    int first_tile[kMaxSeg + 1];  // row tiles before segment s; [segments] = all
    int segments;
    const uint16_t *w_up;   // SwiGLU: up weights beside w[0] (gate)
    const uint16_t *act_table;  // SwiGLU: swiglu_act_bf16 of every gate value
    const uint16_t *resid;  // add: [tokens][rows[0]], may equal out[0]
    const uint16_t *x;      // [tokens][inner]
    int inner, tokens;
    int n_tiles;            // token tiles
    // ksplit > 1: workgroup (tile, s) sums k-steps [s nk / ksplit,
    // (s + 1) nk / ksplit) into partial[s][product][out], fp32, where out
    // runs over every segment's [tokens][rows] in segment order (out_base)
    // and product is the gate (0) or up (1) sum of SwiGLU; a second launch
    // adds the partials in split order and applies the epilogue.
    int ksplit;
    float *partial;
    int64_t out_base[kMaxSeg + 1];  // [segments] = all outputs
};

// Swizzle of a row of NSL 16-byte slots: the slot XOR this.  64 banks of 4
// bytes hold two 128-byte rows, so the 16 rows one LDS cycle serves are
// conflict-free when the 8 rows of each parity take 8 distinct slots; a
// 256-byte row fills the banks alone and needs 16 distinct slots.
template <int NSL>
__device__ __forceinline__ int proj_swz(int row) {
    return NSL == 8 ? (row >> 1) & 7 : row & (NSL - 1);
}

// LDS of a configuration: ST stages of the weight tile(s) and the token tile;
// the SwiGLU epilogue reuses it for the 128 KiB activation table.
constexpr int kTableBytes = kSwigluTableEntries * 2;
constexpr int proj_lds_bytes(int wm, int bk, int st, int epi) {
    const int stages = st * ((epi == kSwiglu ? 2 : 1) * kBM + 64 * (4 / (kBM / wm))) * bk * 2;
    return epi == kSwiglu && stages < kTableBytes ? kTableBytes : stages;
}

template <int WM, int BK, int ST, int EPI>
__global__ __launch_bounds__(256) void proj_kernel(ProjArgs a) {
    constexpr int kStages = ST;
    constexpr int kBK = BK;
    constexpr int ROWB = BK * 2;      // bytes of one row of a stage
    constexpr int NSL = BK / 8;       // 16-byte slots per row
    constexpr int RPC = 1024 / ROWB;  // rows per 1 KiB copy chunk
    constexpr int SUB = BK / 16;      // MFMA k-steps per stage
    constexpr int WAVES = 4;
    constexpr int WR = kBM / WM;       // wavefronts along the rows
    constexpr int WN = WAVES / WR;     // and along the tokens, 64 each
    constexpr int BN = 64 * WN;
    constexpr int MI = WM / 32;        // 32-row MFMA blocks per wavefront
    constexpr int NA = EPI == kSwiglu ? 2 : 1;
    constexpr int A_BYTES = kBM * kBK * 2;  // one weight stage: 16 KiB
    constexpr int B_BYTES = BN * kBK * 2;
    constexpr int A_CH = kBM / RPC / WAVES;   // 1 KiB copy chunks per wavefront
    constexpr int B_CH = BN / RPC / WAVES;
    constexpr int PER_STAGE = NA * A_CH + B_CH;  // copies per wavefront per k-step
    static_assert(A_CH >= 1 && B_CH >= 1 && PER_STAGE * (kStages - 2) <= 63, "copy plan");
    static_assert((kStages - 1) * A_BYTES + kBM * ROWB <= 65536 && (kStages - 1) * B_BYTES + BN * ROWB <= 65536,
                  "fragment reads reach every stage by immediate offsets");
    __shared__ __align__(16) unsigned char lds[proj_lds_bytes(WM, BK, ST, EPI)];
    unsigned char *const a_lds = lds;                                  // [kStages][A_BYTES]
    unsigned char *const u_lds = lds + kStages * A_BYTES;              // SwiGLU up: [kStages][A_BYTES]
    unsigned char *const b_lds = lds + kStages * NA * A_BYTES;         // [kStages][B_BYTES]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr = wave % WR, wc = wave / WR;
    const int h = lane >> 5;

    // XCD-aware tile: workgroup L runs on XCD L % 8; each XCD takes a
    // contiguous slice of the tiles, ordered (row tile, token tile).
    const int items = a.first_tile[a.segments] * a.n_tiles * a.ksplit;
    const int per_xcd = (items + kXcds - 1) / kXcds;
    const int w_index = (int)(blockIdx.x % kXcds) * per_xcd + (int)(blockIdx.x / kXcds);
    if (w_index >= items) return;
    const int t_index = w_index / a.ksplit, split = w_index % a.ksplit;
    const int mt = t_index / a.n_tiles, nt = t_index % a.n_tiles;
    // The segment's matrix, by uniform selects (a dynamic index into the
    // kernel arguments would not stay scalar).
    const bool s1 = a.segments > 1 && mt >= a.first_tile[1], s2 = a.segments > 2 && mt >= a.first_tile[2];
    const int rows = s2 ? a.rows[2] : s1 ? a.rows[1] : a.rows[0];
    const int m0 = (mt - (s2 ? a.first_tile[2] : s1 ? a.first_tile[1] : 0)) * kBM;
    const uint16_t *const wseg = s2 ? a.w[2] : s1 ? a.w[1] : a.w[0];
    uint16_t *const out = s2 ? a.out[2] : s1 ? a.out[1] : a.out[0];
    const int n0 = nt * BN;
    const int inner = a.inner;
    const int nk_all = inner / kBK;
    const int kb = split * nk_all / a.ksplit;
    const int nk = (split + 1) * nk_all / a.ksplit - kb;

    // Copy offsets: chunk c of a stage is RPC rows; lane l lands in row
    // RPC c + l / NSL, physical slot l % NSL, and fetches the logical slot
    // (l % NSL) ^ proj_swz(row) of that row.  Rows past the matrix re-read
    // its last row (their outputs are not written).
    const uint32_t row_bytes = (uint32_t)inner * 2;
    uint32_t aoff[A_CH], boff[B_CH];
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
        const int r = RPC * (wave + WAVES * i) + lane / NSL;
        aoff[i] = (uint32_t)(min(m0 + r, rows - 1) - m0) * row_bytes +
                  (uint32_t)(((lane % NSL) ^ proj_swz<NSL>(r)) * 16);
    }
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
        const int r = RPC * (wave + WAVES * i) + lane / NSL;
        boff[i] = (uint32_t)(min(n0 + r, a.tokens - 1) - n0) * row_bytes +
                  (uint32_t)(((lane % NSL) ^ proj_swz<NSL>(r)) * 16);
    }
    const int64_t k_first = (int64_t)kb * kBK;
    const char *const wbase = uniform_ptr(reinterpret_cast<const char *>(wseg + (int64_t)m0 * inner + k_first));
    const char *const ubase =
        EPI == kSwiglu ? uniform_ptr(reinterpret_cast<const char *>(a.w_up + (int64_t)m0 * inner + k_first))
                       : nullptr;
    const char *const xbase = uniform_ptr(reinterpret_cast<const char *>(a.x + (int64_t)n0 * inner + k_first));
    uint32_t a_dst[kStages], u_dst[kStages], b_dst[kStages];
#pragma unroll
    for (int st = 0; st < kStages; ++st) {
        a_dst[st] = lds_offset(a_lds + st * A_BYTES + wave * 1024);
        u_dst[st] = EPI == kSwiglu ? lds_offset(u_lds + st * A_BYTES + wave * 1024) : 0;
        b_dst[st] = lds_offset(b_lds + st * B_BYTES + wave * 1024);
    }
    auto copy_step = [&](int st, int kt) __attribute__((always_inline)) {
        const int64_t k = (int64_t)kt * kBK * 2;
#pragma unroll
        for (int i = 0; i < A_CH; ++i) {
            dma16_async(wbase + k, aoff[i], a_dst[st] + i * WAVES * 1024);
            if (EPI == kSwiglu) dma16_async(ubase + k, aoff[i], u_dst[st] + i * WAVES * 1024);
        }
#pragma unroll
        for (int i = 0; i < B_CH; ++i) dma16_async(xbase + k, boff[i], b_dst[st] + i * WAVES * 1024);
    };

    // Fragment addresses in stage 0: row WM wr + l % 32 (weights) or 64 wc +
    // l % 32 (tokens), logical slot 2 s + l / 32 of sub-step s, physical slot
    // that ^ proj_swz(row) = (2 s + h) ^ proj_swz(l % 32).  A 32-row block and
    // a stage are immediate offsets (the swizzle depends on row % 32 only).
    uint32_t fa[SUB], fu[SUB], fb[SUB];
    {
        const uint32_t abase = lds_offset(a_lds), ubase_l = lds_offset(u_lds), bbase = lds_offset(b_lds);
#pragma unroll
        for (int s = 0; s < SUB; ++s) {
            const uint32_t sw = (uint32_t)(((2 * s + h) ^ proj_swz<NSL>(lane & 31)) * 16);
            fa[s] = abase + (uint32_t)(WM * wr + (lane & 31)) * ROWB + sw;
            fu[s] = ubase_l + (uint32_t)(WM * wr + (lane & 31)) * ROWB + sw;
            fb[s] = bbase + (uint32_t)(64 * wc + (lane & 31)) * ROWB + sw;
        }
    }

    floatx16_t acc[MI][2], accu[MI][2];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                acc[i][j][r] = 0.0f;
                if (EPI == kSwiglu) accu[i][j][r] = 0.0f;
            }

    struct Frag {
        bf16x8_t a[MI], u[MI], b[2];
    };
    auto read_frag = [&](Frag &f, int st, int s) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            f.a[i] = lds_read_b128(fa[s] + st * A_BYTES + i * 32 * ROWB);
            if (EPI == kSwiglu) f.u[i] = lds_read_b128(fu[s] + st * A_BYTES + i * 32 * ROWB);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) f.b[j] = lds_read_b128(fb[s] + st * B_BYTES + j * 32 * ROWB);
    };
    auto mfma = [&](const Frag &f) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
                if (EPI == kSwiglu)
                    accu[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.u[i], f.b[j], accu[i][j], 0, 0, 0);
            }
    };

    // K loop.  Iteration kt: this wavefront's copy of k-step kt has landed
    // (later ones may be in flight), the barrier publishes it and frees the
    // stage of kt-1, which receives k-step kt + kStages - 1 (the last k-step
    // is repeated past the end so the wait counts stay exact).  The fragments
    // of kt-1's last sub-step were read before the barrier; their MFMAs run
    // while the first fragments of kt are in flight.
    Frag cur, nxt;
#pragma unroll
    for (int st = 0; st < kStages - 1; ++st) copy_step(st, min(st, nk - 1));
    auto iteration = [&](int kt, int st, int sd, auto first_tag) __attribute__((always_inline)) {
        constexpr bool first = decltype(first_tag)::value;
        __builtin_amdgcn_s_waitcnt(vmcnt_lds_imm((kStages - 2) * PER_STAGE));
        raw_barrier();
        read_frag(nxt, st, 0);
        if constexpr (!first) mfma(cur);
        copy_step(sd, min(kt + kStages - 1, nk - 1));
#pragma unroll
        for (int s = 0; s < SUB; ++s) {
            __builtin_amdgcn_sched_barrier(0);
            cur = nxt;
            if (s + 1 < SUB) read_frag(nxt, st, s + 1);
            if (s + 1 < SUB) mfma(cur);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    using Yes = std::true_type;
    using No = std::false_type;
    // Stage of k-step kt is kt % kStages; the loop is unrolled by kStages so
    // every stage index is a constant.
    iteration(0, 0, kStages - 1, Yes{});
    for (int kt = 1; kt < nk; kt += kStages) {
#pragma unroll
        for (int u = 0; u < kStages; ++u) {
            if (kt + u >= nk) break;
            iteration(kt + u, (1 + u) % kStages, u % kStages, No{});
        }
    }
    mfma(cur);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // no copy may still target LDS at exit

    // SwiGLU: the activation table replaces the stages in LDS (one 128 KiB
    // copy per workgroup, from L2), after every wavefront's last fragment
    // read.
    const uint16_t *table = nullptr;
    if constexpr (EPI == kSwiglu) {
        __syncthreads();
        const char *tb = uniform_ptr(reinterpret_cast<const char *>(a.act_table));
        const uint32_t dst = lds_offset(lds + wave * 1024);
#pragma unroll
        for (int i = 0; i < kTableBytes / 1024 / WAVES; ++i)
            dma16_async(tb + (int64_t)(wave + WAVES * i) * 1024, (uint32_t)lane * 16, dst + i * WAVES * 1024);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        __syncthreads();
        table = reinterpret_cast<const uint16_t *>(lds);
    }

    // Epilogue: lane l holds token 64 wc + 32 j + l % 32 and, per group g of
    // four accumulators, rows WM wr + 32 i + 8 g + 4 h .. +3.
    if (a.ksplit > 1) {
        const int64_t obase = s2 ? a.out_base[2] : s1 ? a.out_base[1] : 0;
        float *const part = a.partial + (int64_t)split * NA * a.out_base[a.segments] + obase;
        float *const part_up = part + a.out_base[a.segments];
        const bool vecf = (rows & 3) == 0 && (obase & 3) == 0;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int t = n0 + 64 * wc + 32 * j + (lane & 31);
            if (t >= a.tokens) continue;
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int r = m0 + WM * wr + 32 * i + 8 * g + 4 * h;
                    if (r >= rows) continue;
                    const int64_t o = (int64_t)t * rows + r;
                    if (vecf && r + 3 < rows) {
                        const floatx4_t v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                                             acc[i][j][4 * g + 3]};
                        *reinterpret_cast<floatx4_t *>(part + o) = v;
                        if (EPI == kSwiglu) {
                            const floatx4_t u = {accu[i][j][4 * g], accu[i][j][4 * g + 1], accu[i][j][4 * g + 2],
                                                 accu[i][j][4 * g + 3]};
                            *reinterpret_cast<floatx4_t *>(part_up + o) = u;
                        }
                    } else {
                        for (int e = 0; e < 4 && r + e < rows; ++e) {
                            part[o + e] = acc[i][j][4 * g + e];
                            if (EPI == kSwiglu) part_up[o + e] = accu[i][j][4 * g + e];
                        }
                    }
                }
        }
        return;
    }
    const bool vec = (rows & 3) == 0 && (reinterpret_cast<uintptr_t>(out) & 7) == 0 &&
                     (EPI != kAdd || (reinterpret_cast<uintptr_t>(a.resid) & 7) == 0);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int t = n0 + 64 * wc + 32 * j + (lane & 31);
        if (t >= a.tokens) continue;
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int r = m0 + WM * wr + 32 * i + 8 * g + 4 * h;
                if (r >= rows) continue;
                uint16_t y[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint16_t p = write_bf16(acc[i][j][4 * g + e]);
                    if (EPI == kSwiglu) y[e] = swiglu_mul_bf16(table[p], write_bf16(accu[i][j][4 * g + e]));
                    else y[e] = p;
                }
                const int64_t o = (int64_t)t * rows + r;
                if (vec && r + 3 < rows) {
                    if (EPI == kAdd) {
                        const uint2 rv = *reinterpret_cast<const uint2 *>(a.resid + o);
                        const uint16_t rs[4] = {(uint16_t)rv.x, (uint16_t)(rv.x >> 16), (uint16_t)rv.y,
                                                (uint16_t)(rv.y >> 16)};
#pragma unroll
                        for (int e = 0; e < 4; ++e) y[e] = write_bf16(__fadd_rn(read_bf16(rs[e]), read_bf16(y[e])));
                    }
                    uint2 w;
                    w.x = (uint32_t)y[0] | ((uint32_t)y[1] << 16);
                    w.y = (uint32_t)y[2] | ((uint32_t)y[3] << 16);
                    *reinterpret_cast<uint2 *>(out + o) = w;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if (r + e >= rows) break;
                        uint16_t v = y[e];
                        if (EPI == kAdd) v = write_bf16(__fadd_rn(read_bf16(a.resid[o + e]), read_bf16(v)));
                        out[o + e] = v;
                    }
                }
            }
    }
}

// Split launches: out = epilogue(BF16(partial[0] + partial[1] + ...)), the
// partials added in split order, four outputs per thread.
template <int EPI>
__global__ __launch_bounds__(256) void proj_merge_kernel(ProjArgs a) {
    constexpr int NA = EPI == kSwiglu ? 2 : 1;
    const int64_t n = a.out_base[a.segments];
    const int64_t i0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i0 >= n) return;
    // Four outputs of one segment with 16-byte partials and 8-byte outputs
    // (and residual): one vector access each; otherwise element by element.
    // The arithmetic per element is the same either way.
    const int seg0 = (a.segments > 2 && i0 >= a.out_base[2]) ? 2 : (a.segments > 1 && i0 >= a.out_base[1]) ? 1 : 0;
    const int64_t li0 = i0 - a.out_base[seg0];
    const bool vec = i0 + 3 < a.out_base[seg0 + 1] && (li0 & 3) == 0 &&
                     ((reinterpret_cast<uintptr_t>(a.partial) | reinterpret_cast<uintptr_t>(a.out[seg0]) |
                       (EPI == kAdd ? reinterpret_cast<uintptr_t>(a.resid) : 0)) & 15) == 0;
    if (vec) {
        float4 v = *reinterpret_cast<const float4 *>(a.partial + i0);
        float4 vu = EPI == kSwiglu ? *reinterpret_cast<const float4 *>(a.partial + n + i0) : float4{};
        for (int s = 1; s < a.ksplit; ++s) {
            const float4 w = *reinterpret_cast<const float4 *>(a.partial + (int64_t)s * NA * n + i0);
            v = float4{__fadd_rn(v.x, w.x), __fadd_rn(v.y, w.y), __fadd_rn(v.z, w.z), __fadd_rn(v.w, w.w)};
            if (EPI == kSwiglu) {
                const float4 wu = *reinterpret_cast<const float4 *>(a.partial + ((int64_t)s * NA + 1) * n + i0);
                vu = float4{__fadd_rn(vu.x, wu.x), __fadd_rn(vu.y, wu.y), __fadd_rn(vu.z, wu.z), __fadd_rn(vu.w, wu.w)};
            }
        }
        const float vs[4] = {v.x, v.y, v.z, v.w}, us[4] = {vu.x, vu.y, vu.z, vu.w};
        uint16_t rs[4] = {0, 0, 0, 0};
        if (EPI == kAdd) {
            const uint2 r = *reinterpret_cast<const uint2 *>(a.resid + li0);
            rs[0] = (uint16_t)r.x; rs[1] = (uint16_t)(r.x >> 16); rs[2] = (uint16_t)r.y; rs[3] = (uint16_t)(r.y >> 16);
        }
        uint16_t ys[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            uint16_t y = write_bf16(vs[e]);
            if (EPI == kSwiglu) y = swiglu_mul_bf16(a.act_table[y], write_bf16(us[e]));
            if (EPI == kAdd) y = write_bf16(__fadd_rn(read_bf16(rs[e]), read_bf16(y)));
            ys[e] = y;
        }
        *reinterpret_cast<uint2 *>(a.out[seg0] + li0) =
            uint2{(uint32_t)ys[0] | ((uint32_t)ys[1] << 16), (uint32_t)ys[2] | ((uint32_t)ys[3] << 16)};
        return;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int64_t i = i0 + e;
        if (i >= n) break;
        float v = a.partial[i], vu = EPI == kSwiglu ? a.partial[n + i] : 0.0f;
        for (int s = 1; s < a.ksplit; ++s) {
            v = __fadd_rn(v, a.partial[(int64_t)s * NA * n + i]);
            if (EPI == kSwiglu) vu = __fadd_rn(vu, a.partial[((int64_t)s * NA + 1) * n + i]);
        }
        const int seg = (a.segments > 2 && i >= a.out_base[2]) ? 2 : (a.segments > 1 && i >= a.out_base[1]) ? 1 : 0;
        const int64_t li = i - a.out_base[seg];
        uint16_t y = write_bf16(v);
        if (EPI == kSwiglu) y = swiglu_mul_bf16(a.act_table[y], write_bf16(vu));
        if (EPI == kAdd) y = write_bf16(__fadd_rn(read_bf16(a.resid[li]), read_bf16(y)));
        a.out[seg][li] = y;
    }
}

// Any shape: one wavefront per output element.  Lane l sums k = l, l + 64,
// ... in order, then the 64 partial sums meet in a fixed butterfly, so the
// fp32 error stays near (K / 64 + 6) roundings of the magnitudes.
template <int EPI>
__global__ __launch_bounds__(256) void proj_generic_kernel(ProjArgs a) {
    const int lane = threadIdx.x & 63;
    const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    int64_t total = 0;
    for (int s = 0; s < a.segments; ++s) total += (int64_t)a.rows[s] * a.tokens;
    if (item >= total) return;
    int seg = 0;
    int64_t rest = item;
    while (rest >= (int64_t)a.rows[seg] * a.tokens) {
        rest -= (int64_t)a.rows[seg] * a.tokens;
        ++seg;
    }
    const int rows = a.rows[seg];
    const int t = (int)(rest / rows), r = (int)(rest % rows);
    const uint16_t *w = a.w[seg] + (int64_t)r * a.inner;
    const uint16_t *u = EPI == kSwiglu ? a.w_up + (int64_t)r * a.inner : nullptr;
    const uint16_t *x = a.x + (int64_t)t * a.inner;
    float s = 0.0f, su = 0.0f;
    for (int k = lane; k < a.inner; k += 64) {
        const float xv = read_bf16(x[k]);
        s = __fmaf_rn(read_bf16(w[k]), xv, s);
        if (EPI == kSwiglu) su = __fmaf_rn(read_bf16(u[k]), xv, su);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        s = __fadd_rn(s, __shfl_xor(s, m, 64));
        if (EPI == kSwiglu) su = __fadd_rn(su, __shfl_xor(su, m, 64));
    }
    if (lane != 0) return;
    const int64_t o = (int64_t)t * rows + r;
    uint16_t y = write_bf16(s);
    if (EPI == kSwiglu) y = swiglu_bf16(y, write_bf16(su));
    if (EPI == kAdd) y = write_bf16(__fadd_rn(read_bf16(a.resid[o]), read_bf16(y)));
    a.out[seg][o] = y;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

// A long inner dimension (the down projection's 14,336) leaves too few
// 128 x 128 output tiles to fill the CUs at prompt-chunk sizes; its k range is
// split in two, with a merge launch.  The choice depends on inner only, so
// every entry point (one matrix or several, fused epilogue or not) sums a
// given product in the same order.
int proj_ksplit(int inner) { return inner >= 8192 && inner % (2 * kKAlign) == 0 ? 2 : 1; }

namespace {

template <int EPI>
hipError_t launch(ProjArgs &a, hipStream_t stream) {
    a.first_tile[0] = 0;
    for (int s = 0; s < a.segments; ++s) a.first_tile[s + 1] = a.first_tile[s] + (a.rows[s] + kBM - 1) / kBM;
    for (int s = a.segments + 1; s <= kMaxSeg; ++s) a.first_tile[s] = a.first_tile[a.segments];
    bool fast = a.inner % kKAlign == 0 && aligned16(a.x) && (EPI != kSwiglu || aligned16(a.w_up));
    for (int s = 0; s < a.segments; ++s) fast = fast && aligned16(a.w[s]);
    if (!fast) {
        a.ksplit = 1;
        int64_t total = 0;
        for (int s = 0; s < a.segments; ++s) total += (int64_t)a.rows[s] * a.tokens;
        hipLaunchKernelGGL((proj_generic_kernel<EPI>), dim3((unsigned)((total + 3) / 4)), dim3(256), 0, stream, a);
        return hipGetLastError();
    }
    // 128 x 128 tiles (64 x 64 per wavefront) when the launch has at least
    // three of them per four CUs, 128 x 64 (32 x 64 per wavefront) below.
    // Measured on the cfg5 shapes at 512 tokens (us, 128 x 128 / 128 x 64):
    // Q, K, V 33.4 / 36.7; O 36.9 / 26.0; gate and up 151 / 215; down 137 /
    // 107 (a k-step of 128 with two stages was slower for every shape).
    const int64_t m_tiles = a.first_tile[a.segments];
    a.ksplit = proj_ksplit(a.inner);
    if (a.ksplit > 1 && !a.partial) return hipErrorInvalidValue;
    a.out_base[0] = 0;
    for (int s = 0; s < a.segments; ++s) a.out_base[s + 1] = a.out_base[s] + (int64_t)a.rows[s] * a.tokens;
    for (int s = a.segments + 1; s <= kMaxSeg; ++s) a.out_base[s] = a.out_base[a.segments];
    const bool wide = (a.ksplit > 1 || m_tiles * ((a.tokens + 127) / 128) >= 192) &&
                      proj_lds_bytes(64, kBK, kStages, EPI) <= 163840;
    const int bn = wide ? 128 : 64;
    a.n_tiles = (a.tokens + bn - 1) / bn;
    const int64_t tiles = m_tiles * a.n_tiles * a.ksplit;
    const unsigned grid = (unsigned)(((tiles + kXcds - 1) / kXcds) * kXcds);
    if constexpr (proj_lds_bytes(64, kBK, kStages, EPI) <= 163840) {
        if (wide) {
            hipLaunchKernelGGL((proj_kernel<64, kBK, kStages, EPI>), dim3(grid), dim3(256), 0, stream, a);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((proj_kernel<32, kBK, kStages, EPI>), dim3(grid), dim3(256), 0, stream, a);
    return hipGetLastError();
}

template <int EPI>
hipError_t launch_split(ProjArgs &a, hipStream_t stream) {
    if (hipError_t e = launch<EPI>(a, stream)) return e;
    if (a.ksplit < 2) return hipSuccess;
    const int64_t n = a.out_base[a.segments];
    hipLaunchKernelGGL((proj_merge_kernel<EPI>), dim3((unsigned)((n + 1023) / 1024)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_proj(const SkinnyMatrix *m, int count, const uint16_t *x, int inner, int tokens, float *partial,
                       hipStream_t stream) {
    ProjArgs a{};
    for (int s = 0; s < count; ++s) {
        a.w[s] = m[s].w;
        a.out[s] = m[s].out;
        a.rows[s] = m[s].rows;
    }
    a.segments = count;
    a.x = x;
    a.inner = inner;
    a.tokens = tokens;
    a.partial = partial;
    return launch_split<kPlain>(a, stream);
}

hipError_t launch_proj_add(const SkinnyMatrix &m, const uint16_t *resid, const uint16_t *x, int inner, int tokens,
                           float *partial, hipStream_t stream) {
    ProjArgs a{};
    a.w[0] = m.w;
    a.out[0] = m.out;
    a.rows[0] = m.rows;
    a.segments = 1;
    a.resid = resid;
    a.x = x;
    a.inner = inner;
    a.tokens = tokens;
    a.partial = partial;
    return launch_split<kAdd>(a, stream);
}

hipError_t launch_proj_swiglu(const uint16_t *w_gate, const uint16_t *w_up, uint16_t *out, int rows,
                              const uint16_t *x, int inner, int tokens, const uint16_t *act_table, float *partial,
                              hipStream_t stream) {
    ProjArgs a{};
    a.w[0] = w_gate;
    a.w_up = w_up;
    a.act_table = act_table;
    a.out[0] = out;
    a.rows[0] = rows;
    a.segments = 1;
    a.x = x;
    a.inner = inner;
    a.tokens = tokens;
    a.partial = partial;
    return launch_split<kSwiglu>(a, stream);
}

}  // namespace mslim
