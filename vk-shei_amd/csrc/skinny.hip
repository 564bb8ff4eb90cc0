// BF16 projections of decode batches (tokens <= 16) on MFMA:
//   out[t][r] = BF16(sum_k x[t][k] * w[r][k]),  fp32 accumulation.
// The decode projections of the reference (llm_fused_qkv_bf16,
// llm_fused_swiglu_bf16 and the reuse-8 GEMV, gpu_llm.cl:553-596, :740-834;
// with its HIP backend the same products go to hipBLASLt, gpu_resources.rs:
// 366-378) stream every weight once per step, so the work is HBM-bound on the
// weights; the token vectors are a few hundred KiB and stay in L2.
//
// A workgroup owns 16 output rows and all tokens.  Each wavefront takes every
// WAVES-th block of 32*kUnroll inputs and runs v_mfma_f32_16x16x32_bf16 with
// the weights as A (16 rows x 32 inputs, one 16-byte load per lane) and the
// tokens as B (32 inputs x 16 tokens, padded with zeros), kUnroll loads in
// flight per operand.  When the token rows fit (<= 8 tokens of <= 4096
// inputs) the workgroup stages them in LDS first: the per-k-step B loads cost
// a quarter of the streaming rate when they go to L2.  The WAVES partial 16x16 tiles are summed in LDS in
// fixed wave order, so results do not depend on timing.  Epilogues:
//   plain   out = BF16(acc)
//   add     out = BF16(resid + BF16(acc))           (llm_add after the product)
//   swiglu  out = SwiGLU(BF16(acc_gate), BF16(acc_up))   (llm_swiglu after both)
// which equal the unfused product followed by the elementwise kernel bit for
// bit.  Up to three matrices with separate outputs share one launch (Q, K, V).
#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>

namespace mslim {

namespace {

constexpr int kTileRows = 16;
// MFMA steps per load batch: kUnroll 16-byte weight loads in flight per lane
// before the first MFMA of the batch.  Unroll 8, a two-deep register ring of
// batches, a persistent grid and non-temporal weight loads each measured no
// faster (non-temporal loads cost 10-30%).
constexpr int kUnroll = 4;
constexpr int kMaxSegments = 3;

enum Epilogue { kPlain = 0, kAdd = 1, kSwiglu = 2 };

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
    int inner, tokens;
};

__device__ __forceinline__ bf16x8_t load8(const uint16_t *p) { return *reinterpret_cast<const bf16x8_t *>(p); }


// Token vectors staged in LDS (XLDS): up to kStageTokens rows of up to
// kStageInner inputs, each row padded by 16 bytes so that the 16 token rows
// of a B fragment read fall in different banks.
constexpr int kStageTokens = 8;
constexpr int kStageInner = 4096;
constexpr int kStageStride = kStageInner + 8;

template <int WAVES, int EPI, bool XLDS>
__global__ __launch_bounds__(WAVES * 64) void skinny_kernel(SkinnyArgs a) {
    // One LDS region holds the staged token rows during the k loop and the
    // wavefronts' partial tiles after it, so two workgroups fit on a CU.
    constexpr int kPartialBytes = (EPI == kSwiglu ? 2 : 1) * WAVES * 64 * 16;
    constexpr int kStageBytes = XLDS ? kStageTokens * kStageStride * 2 : 0;
    __shared__ __align__(16) unsigned char lds[kPartialBytes > kStageBytes ? kPartialBytes : kStageBytes];
    auto partial = reinterpret_cast<floatx4_t(*)[WAVES][64]>(lds);
    uint16_t *xs = reinterpret_cast<uint16_t *>(lds);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int tile = blockIdx.x;  // one workgroup per 16-row tile
    if (XLDS) {
        // The B operand (token rows) is the same for every row tile: read it
        // once per workgroup with 16-byte loads instead of once per k-step
        // per wavefront.
        // All of a thread's loads go out before its first LDS write (a
        // load-wait-write loop costs one L2 round trip per 16 bytes); past
        // the last chunk the index is clamped in bounds and not written.
        constexpr int kPerThread = kStageTokens * kStageInner / 8 / (WAVES * 64);
        const int chunks = a.inner / 8;
        const int total = a.tokens * chunks;
        bf16x8_t v[kPerThread];
#pragma unroll
        for (int k = 0; k < kPerThread; ++k) {
            const int i = min((int)threadIdx.x + k * WAVES * 64, total - 1);
            v[k] = load8(a.x + (int64_t)(i / chunks) * a.inner + (i % chunks) * 8);
        }
        __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the writes
#pragma unroll
        for (int k = 0; k < kPerThread; ++k) {
            const int i = (int)threadIdx.x + k * WAVES * 64;
            if (i < total) *reinterpret_cast<bf16x8_t *>(xs + (i / chunks) * kStageStride + (i % chunks) * 8) = v[k];
        }
        __syncthreads();
    }
    int seg = 0;
    if (a.segments > 1 && tile >= a.first_tile[1]) seg = 1;
    if (a.segments > 2 && tile >= a.first_tile[2]) seg = 2;
    const int rows = a.rows[seg];
    const int r0 = (tile - a.first_tile[seg]) * kTileRows;
    // A operand: lane l holds row r0 + l%16, inputs 8*(l/16) .. +7 of each
    // 32-input block; B operand: token l%16, the same inputs.  Rows past the
    // end re-read the last row and are not written.
    const int row = min(r0 + (lane & 15), rows - 1);
    const int kq = (lane >> 4) * 8;
    const int tok = lane & 15;
    const bool live = tok < a.tokens;
    const uint16_t *wp = a.w[seg] + (int64_t)row * a.inner + kq;
    const uint16_t *up = EPI == kSwiglu ? a.w_up + (int64_t)row * a.inner + kq : nullptr;
    const uint16_t *xp = a.x + (int64_t)(live ? tok : 0) * a.inner + kq;
    const uint16_t *xl = xs + (live ? tok : 0) * kStageStride + kq;
    floatx4_t acc = {0.0f, 0.0f, 0.0f, 0.0f}, acc_up = {0.0f, 0.0f, 0.0f, 0.0f};
    const bf16x8_t zero = {};
    // inner % 32 == 0: a block that starts inside the row ends inside it.
    struct Batch {
        bf16x8_t wa[kUnroll], wu[kUnroll], xb[kUnroll];
    };
    auto load_batch = [&](Batch &bt, int k0) {
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int k = k0 + u * 32;
            const bool in = k < a.inner;
            bt.wa[u] = in ? load8(wp + k) : zero;
            if (EPI == kSwiglu) bt.wu[u] = in ? load8(up + k) : zero;
            if (XLDS) bt.xb[u] = in && live ? *reinterpret_cast<const bf16x8_t *>(xl + k) : zero;
            else bt.xb[u] = in && live ? load8(xp + k) : zero;
        }
    };
    auto use_batch = [&](const Batch &bt) {
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bt.wa[u], bt.xb[u], acc, 0, 0, 0);
            if (EPI == kSwiglu) acc_up = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bt.wu[u], bt.xb[u], acc_up, 0, 0, 0);
        }
    };
    const int step = WAVES * 32 * kUnroll;
    for (int k0 = wave * 32 * kUnroll; k0 < a.inner; k0 += step) {
        Batch bt;
        load_batch(bt, k0);
        use_batch(bt);
    }
    if (XLDS) __syncthreads();  // every wavefront is done with the staged rows
    partial[0][wave][lane] = acc;
    if (EPI == kSwiglu) partial[EPI == kSwiglu ? 1 : 0][wave][lane] = acc_up;
    __syncthreads();
    if (wave != 0) return;
    floatx4_t sum = partial[0][0][lane], sum_up = partial[EPI == kSwiglu ? 1 : 0][0][lane];
    for (int w = 1; w < WAVES; ++w) {
        sum += partial[0][w][lane];
        if (EPI == kSwiglu) sum_up += partial[EPI == kSwiglu ? 1 : 0][w][lane];
    }
    // D layout: lane l holds rows 4*(l/16) + j, token l%16.
    if (!live) return;
    uint16_t *out = a.out[seg] + (int64_t)tok * rows;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = r0 + 4 * (lane >> 4) + j;
        if (r >= rows) continue;
        const uint16_t y = write_bf16(sum[j]);
        if (EPI == kPlain) {
            out[r] = y;
        } else if (EPI == kAdd) {
            out[r] = write_bf16(__fadd_rn(read_bf16(a.resid[(int64_t)tok * rows + r]), read_bf16(y)));
        } else {
            out[r] = swiglu_bf16(y, write_bf16(sum_up[j]));
        }
    }
}

int tiles_of(int rows) { return (rows + kTileRows - 1) / kTileRows; }

template <int EPI, bool XLDS>
hipError_t launch_with(SkinnyArgs &a, hipStream_t stream) {
    int tiles = 0;
    for (int s = 0; s < a.segments; ++s) {
        a.first_tile[s] = tiles;
        tiles += tiles_of(a.rows[s]);
    }
    // Few row tiles get more wavefronts each, so that enough weight loads are
    // in flight to cover HBM latency.
    a.tiles = tiles;
    // Measured per shape at 8 tokens (weights cycled through more memory
    // than the Infinity Cache holds): 8 wavefronts for the gate/up pair,
    // for inputs too wide to stage and for many row tiles; 16 for the rest.
    const int waves = (EPI == kSwiglu || a.inner > kStageInner || tiles >= 1024) ? 8 : 16;
    const unsigned grid = (unsigned)tiles;
    if (waves == 16)
        hipLaunchKernelGGL((skinny_kernel<16, EPI, XLDS>), dim3(grid), dim3(16 * 64), 0, stream, a);
    else
        hipLaunchKernelGGL((skinny_kernel<8, EPI, XLDS>), dim3(grid), dim3(8 * 64), 0, stream, a);
    return hipGetLastError();
}

template <int EPI>
hipError_t launch(SkinnyArgs &a, hipStream_t stream) {
    if (a.tokens <= kStageTokens && a.inner <= kStageInner) return launch_with<EPI, true>(a, stream);
    return launch_with<EPI, false>(a, stream);
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

bool skinny_supported(int inner, int tokens, const void *x, const void *w0, const void *w1, const void *w2) {
    return tokens >= 1 && tokens <= kSkinnyMaxTokens && inner >= 32 && inner % 32 == 0 && aligned16(x) &&
           aligned16(w0) && aligned16(w1) && aligned16(w2);
}

hipError_t launch_skinny_gemm(const SkinnyMatrix *m, int count, const uint16_t *x, int inner, int tokens,
                              hipStream_t stream) {
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
    return launch<kPlain>(a, stream);
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
                                const uint16_t *x, int inner, int tokens, hipStream_t stream) {
    SkinnyArgs a{};
    a.w[0] = w_gate;
    a.w_up = w_up;
    a.out[0] = out;
    a.rows[0] = rows;
    a.segments = 1;
    a.x = x;
    a.inner = inner;
    a.tokens = tokens;
    return launch<kSwiglu>(a, stream);
}

}  // namespace mslim
