// RMSNorm, RoPE and SwiGLU feeding the attention path.
//
// These keep the reference's BF16 stage roundings and reduction order exactly
// (gpu_llm.cl:72-146, :225-237, :378-456), so for identical inputs they are
// bit-identical to the C restatement used as the checker.  Two choices make
// that possible and are the only departures from the OpenCL text:
//   * 1/sqrt is the correctly rounded square root followed by a correctly
//     rounded division (OpenCL's rsqrt has no fixed rounding);
//   * exp, log, sin and cos are evaluated in double precision and rounded
//     once to float.
// No multiply-add is contracted: every stage rounds as written.
#include <cmath>

#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>

#pragma clang fp contract(off)

namespace mslim {

namespace {

// Tree over the 128 lane sums of an RMSNorm row, pairs (t, t + stride) for
// stride 64 .. 1 (gpu_llm.cl:72-98): the first level crosses the two
// wavefronts through LDS, the rest are shuffles inside wavefront 0, whose lane
// 0 ends with the same sum and leaves it in partials[0].
__device__ __forceinline__ void rms_tree(float *partials, float s, int tid) {
    if (tid >= 64) partials[tid] = s;
    __syncthreads();
    if (tid < 64) {
        float t = __fadd_rn(s, partials[tid + 64]);
#pragma unroll
        for (int stride = 32; stride > 0; stride >>= 1) t = __fadd_rn(t, __shfl_down(t, stride, 64));
        if (tid == 0) partials[0] = t;
    }
    __syncthreads();
}

// llm_rmsnorm / llm_prefill_norm (gpu_llm.cl:72-98, :378-408): one workgroup
// of 128 lanes per token, strided FMA sum of squares, 64..1 tree.
__global__ __launch_bounds__(128) void rmsnorm_kernel(const uint16_t *in, const uint16_t *w,
                                                      uint16_t *out, int hidden, float eps) {
    __shared__ float partials[128];
    const int tid = threadIdx.x;
    const uint16_t *row = in + (int64_t)blockIdx.x * hidden;
    uint16_t *dst = out + (int64_t)blockIdx.x * hidden;
    float s = 0.0f;
    for (int i = tid; i < hidden; i += 128) {
        const float v = read_bf16(row[i]);
        s = __fmaf_rn(v, v, s);
    }
    rms_tree(partials, s, tid);
    const float mean = __fdiv_rn(partials[0], (float)hidden);
    const float factor = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(mean, eps)));
    for (int i = tid; i < hidden; i += 128) {
        const uint16_t normalized = write_bf16(__fmul_rn(read_bf16(row[i]), factor));
        dst[i] = write_bf16(__fmul_rn(read_bf16(normalized), read_bf16(w[i])));
    }
}

// The same RMSNorm with the row and the weights staged in LDS by 16-byte
// loads, all issued before the first wait, and the output written back by
// 16-byte stores.  Lane `tid` still sums elements tid, tid+128, ... in order
// and the tree is unchanged, so the result is bit-identical to rmsnorm_kernel;
// what changes is that the row no longer arrives as 32 dependent 2-byte loads
// per lane.  hidden % (128 * kRmsBatch) == 0 and hidden <= kRmsStagedMax;
// dynamic LDS 4 * hidden bytes.
constexpr int kRmsStagedMax = 8192;  // 32 KiB of dynamic LDS
constexpr int kRmsBatch = 8;

__global__ __launch_bounds__(128) void rmsnorm_staged_kernel(const uint16_t *in, const uint16_t *w,
                                                             uint16_t *out, int hidden, float eps) {
    extern __shared__ uint4 staged[];
    __shared__ float partials[128];
    uint16_t *row = reinterpret_cast<uint16_t *>(staged);
    const uint16_t *wt = row + hidden;
    const int tid = threadIdx.x;
    const int chunks = hidden / 8;
    const uint4 *src = reinterpret_cast<const uint4 *>(in + (int64_t)blockIdx.x * hidden);
    const uint4 *wsrc = reinterpret_cast<const uint4 *>(w);
    // Every load of the lane goes out before its first LDS write (the
    // compiler otherwise pairs each load with its write and waits between
    // them); chunks past the row are clamped in bounds and not written.
    constexpr int kPer = kRmsStagedMax / 8 / 128;
    bf16x8_t xa[kPer], wa[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int c = min(tid + 128 * k, chunks - 1);
        xa[k] = *reinterpret_cast<const bf16x8_t *>(src + c);
        wa[k] = *reinterpret_cast<const bf16x8_t *>(wsrc + c);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int c = tid + 128 * k;
        if (c < chunks) {
            reinterpret_cast<bf16x8_t *>(staged)[c] = xa[k];
            reinterpret_cast<bf16x8_t *>(staged)[chunks + c] = wa[k];
        }
    }
    __syncthreads();
    // hidden % (128 * kBatch) == 0: each lane's elements are read from LDS
    // eight at a time, with no bounds test between the reads, ahead of the
    // FMA chain, which still runs over them in ascending order.
    float s = 0.0f;
    for (int base = tid; base < hidden; base += 128 * kRmsBatch) {
        float v[kRmsBatch];
#pragma unroll
        for (int u = 0; u < kRmsBatch; ++u) v[u] = read_bf16(row[base + 128 * u]);
#pragma unroll
        for (int u = 0; u < kRmsBatch; ++u) s = __fmaf_rn(v[u], v[u], s);
    }
    rms_tree(partials, s, tid);
    const float mean = __fdiv_rn(partials[0], (float)hidden);
    const float factor = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(mean, eps)));
    // each lane rewrites only the elements it read, so in place is safe
    for (int base = tid; base < hidden; base += 128 * kRmsBatch) {
        uint16_t xv[kRmsBatch], wv[kRmsBatch];
#pragma unroll
        for (int u = 0; u < kRmsBatch; ++u) {
            xv[u] = row[base + 128 * u];
            wv[u] = wt[base + 128 * u];
        }
#pragma unroll
        for (int u = 0; u < kRmsBatch; ++u) {
            const uint16_t normalized = write_bf16(__fmul_rn(read_bf16(xv[u]), factor));
            row[base + 128 * u] = write_bf16(__fmul_rn(read_bf16(normalized), read_bf16(wv[u])));
        }
    }
    __syncthreads();
    uint4 *dst = reinterpret_cast<uint4 *>(out + (int64_t)blockIdx.x * hidden);
    for (int c = tid; c < chunks; c += 128) dst[c] = staged[c];
}

// Inverse frequency of rotary dimension pair `fd` (kernels.rs:51-66,
// gpu_llm.cl:123-138), f32 arithmetic with once-rounded log and exp.
__device__ float rope_inverse_frequency(int fd, int head_dim, float theta, int llama3, float factor,
                                        float low, float high, float original_max) {
    const float log_theta = (float)log((double)theta);
    const float exponent = __fdiv_rn(__fmul_rn(-(float)fd, log_theta), (float)head_dim);
    float inv = (float)exp((double)exponent);
    if (llama3) {
        const float wavelength = __fdiv_rn(6.28318530717958647692f, inv);
        const float low_wavelength = __fdiv_rn(original_max, low);
        const float high_wavelength = __fdiv_rn(original_max, high);
        if (wavelength > low_wavelength) {
            inv = __fdiv_rn(inv, factor);
        } else if (wavelength >= high_wavelength) {
            const float smooth = __fdiv_rn(__fsub_rn(__fdiv_rn(original_max, wavelength), low),
                                           __fsub_rn(high, low));
            inv = __fadd_rn(__fmul_rn(__fsub_rn(1.0f, smooth), __fdiv_rn(inv, factor)),
                            __fmul_rn(smooth, inv));
        }
    }
    return inv;
}

// One rotated element of llm_rope / llm_prefill_rope (gpu_llm.cl:102-146,
// :412-456): element d of head `head` of a token row [heads][head_dim] at
// `position`, rotate-half partner, c and s rounded to BF16; `inv` is the
// inverse frequency of pair d % (head_dim / 2).
__device__ __forceinline__ uint16_t rope_element_cs(const uint16_t *token_row, int head, int d, int head_dim,
                                                    float cs, float sn) {
    const int half = head_dim / 2;
    const uint16_t *h = token_row + (int64_t)head * head_dim;
    const float partner = read_bf16(h[d < half ? d + half : d - half]);
    const float rotated = d < half ? -partner : partner;
    const float left = round_bf16(__fmul_rn(read_bf16(h[d]), cs));
    const float right = round_bf16(__fmul_rn(rotated, sn));
    return write_bf16(__fadd_rn(left, right));
}

__device__ __forceinline__ uint16_t rope_element(const uint16_t *token_row, int head, int d, int head_dim,
                                                 int64_t position, float inv) {
    float cs, sn;
    rope_trig(position, inv, cs, sn);
    return rope_element_cs(token_row, head, d, head_dim, cs, sn);
}

// One lane per element.  Row t sits at position start + t, or at
// positions[t] when a position array is given (one decode row per sequence
// of a batch).
__global__ __launch_bounds__(256) void rope_kernel(const uint16_t *in, uint16_t *out, int64_t total,
                                                   int heads, int head_dim, int start,
                                                   const int32_t *positions, float theta,
                                                   int llama3, float factor, float low, float high,
                                                   float original_max) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int64_t elements = (int64_t)heads * head_dim;
    const int64_t token = i / elements;
    const int in_token = (int)(i % elements);
    const int64_t position = positions ? (int64_t)positions[token] : start + token;
    const int d = in_token % head_dim;
    const float inv = rope_inverse_frequency((d % (head_dim / 2)) * 2, head_dim, theta, llama3, factor, low, high,
                                             original_max);
    out[i] = rope_element(in + token * elements, in_token / head_dim, d, head_dim, position, inv);
}

// The same rotation with one workgroup per token row: the row's c and s
// (one pair per rotary dimension pair, head_dim / 2 <= 256) are computed once
// into LDS and shared by all heads, instead of once per element, from the
// launch's inverse-frequency table.  Each value is computed exactly as
// rope_element computes it, so the output is bit-identical.
__global__ __launch_bounds__(256) void rope_token_kernel(const uint16_t *in, uint16_t *out, int heads,
                                                         int head_dim, int start, const int32_t *positions,
                                                         RopeTable table, RopeCosSin cossin) {
    __shared__ float cs[256], sn[256];
    const int64_t token = blockIdx.x;
    const int half = head_dim / 2;
    const int64_t position = positions ? (int64_t)positions[token] : start + token;
    // Lanes [0, half) compute c and lanes [half, 2 * half) compute s, so the
    // table costs one trigonometric evaluation per lane, not two.
    if (position < cossin.positions) {
        for (int f = threadIdx.x; f < half; f += blockDim.x) rope_cs(cossin, position, f, half, 0.0f, cs[f], sn[f]);
    } else {
        for (int t = threadIdx.x; t < 2 * half; t += blockDim.x) {
            const int f = t % half;
            const float phase = __fmul_rn((float)position, table.inv[f]);
            if (t < half) cs[f] = round_bf16((float)cos((double)phase));
            else sn[f] = round_bf16((float)sin((double)phase));
        }
    }
    __syncthreads();
    const int elements = heads * head_dim;
    const uint16_t *row = in + token * elements;
    uint16_t *dst = out + token * elements;
    auto rotate = [&](float x, float partner, int d) {
        const float rotated = d < half ? -partner : partner;
        const int f = d % half;
        const float left = round_bf16(__fmul_rn(x, cs[f]));
        const float right = round_bf16(__fmul_rn(rotated, sn[f]));
        return write_bf16(__fadd_rn(left, right));
    };
    if (head_dim % 16 == 0 && (((uintptr_t)row | (uintptr_t)dst) & 15) == 0) {
        // 16-byte chunks of 8 elements (half % 8 == 0: a chunk and its
        // rotate-half partner chunk each lie in one half of a head); every
        // lane's loads of a batch go out before its first use.
        constexpr int kBatch = 4;
        const int chunks = elements / 8;
        for (int c0 = threadIdx.x; c0 < chunks; c0 += kBatch * blockDim.x) {
            uint4 x[kBatch], p[kBatch];
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                const int e = min(c0 + k * (int)blockDim.x, chunks - 1) * 8;
                const int d = e % head_dim;
                x[k] = *reinterpret_cast<const uint4 *>(row + e);
                p[k] = *reinterpret_cast<const uint4 *>(row + e - d + (d < half ? d + half : d - half));
            }
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                const int c = c0 + k * (int)blockDim.x;
                if (c >= chunks) continue;
                const int d = (c * 8) % head_dim;
                const uint16_t *xs = reinterpret_cast<const uint16_t *>(&x[k]);
                const uint16_t *ps = reinterpret_cast<const uint16_t *>(&p[k]);
                uint16_t r[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) r[j] = rotate(read_bf16(xs[j]), read_bf16(ps[j]), d + j);
                *reinterpret_cast<uint4 *>(dst + c * 8) = *reinterpret_cast<const uint4 *>(r);
            }
        }
        return;
    }
    for (int e = threadIdx.x; e < elements; e += blockDim.x) {
        const int d = e % head_dim;
        const int h0 = e - d;
        dst[e] = rotate(read_bf16(row[e]), read_bf16(row[h0 + (d < half ? d + half : d - half)]), d);
    }
}

// Q and K of a prompt chunk in one launch: a workgroup takes kRopeRows-or-
// fewer consecutive token rows, and its lanes rotate (d, d + half) pairs of
// 8-element chunks, the chunk and its rotate-half partner loaded once and
// both outputs written, over the rows' Q heads then K heads.  Every load of
// a lane goes out before the rows' c and s are gathered into LDS (from the
// context's table, or one trigonometric evaluation per lane per row where
// the table does not reach), shared by Q and K.  Each output is
// rope_element's value for its position, bit-identical to rope_token_kernel
// on Q and on K.
// head_dim % 16 == 0 and 16-byte aligned rows.  PAIRS pair units per lane
// (each unit 8 rotate-half pairs); the launcher picks it (rope_qk_shape).
constexpr int kRopeRows = 8;
constexpr int kRopePairsPerLane = 4;  // the most a launch uses: its capacity
template <int PAIRS>
__global__ __launch_bounds__(256) void rope_qk_kernel(const uint16_t *q, uint16_t *q_out, const uint16_t *k,
                                                      uint16_t *k_out, int tokens, int rows_per_group,
                                                      int q_heads, int kv_heads, int head_dim, int start,
                                                      RopeTable table, RopeCosSin cossin) {
    __shared__ float cs[kRopeRows][kRopeTable], sn[kRopeRows][kRopeTable];
    const int half = head_dim / 2;
    const int hchunks = half / 8;                       // pair units per head
    const int units = (q_heads + kv_heads) * hchunks;  // pair units per row
    const int row0 = blockIdx.x * rows_per_group;
    const int rows = min(rows_per_group, tokens - row0);
    const int work = rows * units;
    uint4 x[PAIRS], p[PAIRS];
#pragma unroll
    for (int j = 0; j < PAIRS; ++j) {
        const int i = min((int)threadIdx.x + j * 256, work - 1);
        const int r = i / units, u = i % units, head = u / hchunks, c = (u % hchunks) * 8;
        const uint16_t *src = head < q_heads ? q + ((int64_t)(row0 + r) * q_heads + head) * head_dim
                                             : k + ((int64_t)(row0 + r) * kv_heads + head - q_heads) * head_dim;
        x[j] = *reinterpret_cast<const uint4 *>(src + c);
        p[j] = *reinterpret_cast<const uint4 *>(src + c + half);
    }
    if (start + row0 + rows <= cossin.positions) {
        // the rows' c and s from the context's table
        for (int t = threadIdx.x; t < rows * half; t += 256)
            rope_cs(cossin, start + row0 + t / half, t % half, half, 0.0f, cs[t / half][t % half],
                    sn[t / half][t % half]);
    } else {
        for (int t = threadIdx.x; t < rows * 2 * half; t += 256) {
            const int r = t / (2 * half), f = t % (2 * half) % half;
            const float phase = __fmul_rn((float)(start + row0 + r), table.inv[f]);
            if (t % (2 * half) < half) cs[r][f] = round_bf16((float)cos((double)phase));
            else sn[r][f] = round_bf16((float)sin((double)phase));
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < PAIRS; ++j) {
        const int i = (int)threadIdx.x + j * 256;
        if (i >= work) break;
        const int r = i / units, u = i % units, head = u / hchunks, c = (u % hchunks) * 8;
        uint16_t *dst = head < q_heads ? q_out + ((int64_t)(row0 + r) * q_heads + head) * head_dim
                                       : k_out + ((int64_t)(row0 + r) * kv_heads + head - q_heads) * head_dim;
        const uint16_t *xs = reinterpret_cast<const uint16_t *>(&x[j]);
        const uint16_t *ps = reinterpret_cast<const uint16_t *>(&p[j]);
        uint16_t lo[8], hi[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int f = c + e;
            const float a = read_bf16(xs[e]), b = read_bf16(ps[e]);
            // first half: x * c + (-partner) * s; second half: x * c + partner * s
            lo[e] = write_bf16(__fadd_rn(round_bf16(__fmul_rn(a, cs[r][f])), round_bf16(__fmul_rn(-b, sn[r][f]))));
            hi[e] = write_bf16(__fadd_rn(round_bf16(__fmul_rn(b, cs[r][f])), round_bf16(__fmul_rn(a, sn[r][f]))));
        }
        *reinterpret_cast<uint4 *>(dst + c) = *reinterpret_cast<const uint4 *>(lo);
        *reinterpret_cast<uint4 *>(dst + c + half) = *reinterpret_cast<const uint4 *>(hi);
    }
}

// A decode step's RoPE and K/V append in one launch, each sequence b at
// positions[b]: rotated Q rows to q_out; rotated K and the V rows straight
// into the page pool through page-table row b.  Lanes [0, nq) rotate Q
// elements, [nq, nq + nk) rotate K elements, the rest copy V 16 bytes at a
// time.  Equal to rope_kernel on Q and on K followed by pages_append.
__global__ __launch_bounds__(256) void rope_append_kernel(RopeAppendArgs a, RopeTable table) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t nq = (int64_t)a.batch * a.q_heads * a.head_dim;
    const int64_t nk = (int64_t)a.batch * a.kv_heads * a.head_dim;
    const int64_t nv = nk / 8;
    if (i >= nq + nk + nv) return;
    if (i < nq) {
        const int64_t elements = (int64_t)a.q_heads * a.head_dim;
        const int b = (int)(i / elements), e = (int)(i % elements), d = e % a.head_dim;
        const int half = a.head_dim / 2;
        float cs, sn;
        rope_cs(a.cossin, a.positions[b], d % half, half, table.inv[d % half], cs, sn);
        a.q_out[i] = rope_element_cs(a.q + b * elements, e / a.head_dim, d, a.head_dim, cs, sn);
        return;
    }
    const int64_t kvd = (int64_t)a.kv_heads * a.head_dim;
    const int64_t j = i - nq;
    const int b = (int)((j < nk ? j : (j - nk) * 8) / kvd);
    const int64_t position = a.positions[b];
    if (position < 0 || position >= ((int64_t)a.pages_per_seq << a.shift)) return;
    const int32_t *rows = a.page_table + (int64_t)b * a.pages_per_seq;
    if (j < nk) {
        const int e = (int)(j % kvd), head = e / a.head_dim, d = e % a.head_dim;
        const int half = a.head_dim / 2;
        float cs, sn;
        rope_cs(a.cossin, position, d % half, half, table.inv[d % half], cs, sn);
        a.k_pool[page_row(rows, a.shift, a.kv_heads, head, position) * a.head_dim + d] =
            rope_element_cs(a.k + b * kvd, head, d, a.head_dim, cs, sn);
    } else {
        const int e = (int)(((j - nk) * 8) % kvd), head = e / a.head_dim, d = e % a.head_dim;
        *reinterpret_cast<uint4 *>(a.v_pool + page_row(rows, a.shift, a.kv_heads, head, position) * a.head_dim +
                                   d) = *reinterpret_cast<const uint4 *>(a.v + b * kvd + e);
    }
}

// llm_swiglu (gpu_llm.cl:225-237): BF16(BF16(g / (1 + e^-g)) * u).
__global__ __launch_bounds__(256) void swiglu_kernel(const uint16_t *gate, const uint16_t *up,
                                                     uint16_t *out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    out[i] = swiglu_bf16(gate[i], up[i]);
}

// Residual add with one BF16 rounding (llm_add, gpu_llm.cl:214-222).
__global__ __launch_bounds__(256) void add_kernel(const uint16_t *a, const uint16_t *b, uint16_t *out,
                                                  int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = write_bf16(__fadd_rn(read_bf16(a[i]), read_bf16(b[i])));
}

// Embedding rows of `tokens` ids (llm_embed, gpu_llm.cl:24-33), 16 bytes per
// lane.  Ids out of range write zeros and set *bad when bad is given.
__global__ __launch_bounds__(256) void embed_kernel(const uint16_t *table, const int32_t *ids, int tokens,
                                                    int hidden, int vocab, uint16_t *out, int *bad) {
    const int chunks = hidden / 8;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)tokens * chunks) return;
    const int t = (int)(i / chunks), c = (int)(i % chunks);
    const int id = ids[t];
    uint4 v = make_uint4(0, 0, 0, 0);
    if (id >= 0 && id < vocab) v = *reinterpret_cast<const uint4 *>(table + (int64_t)id * hidden + c * 8);
    else if (c == 0 && bad) *bad = 1;
    *reinterpret_cast<uint4 *>(out + (int64_t)t * hidden + c * 8) = v;
}

// Greedy token of each row of BF16 logits (llm_argmax, gpu_llm.cl:239-270),
// one workgroup of 1024 lanes per row.  Every lane starts from (-inf, index 0)
// and takes a value that is greater, or equal with a lower index: NaN never
// wins, the first index wins ties, and a row with nothing above -inf gives 0.
// That rule makes the result independent of how elements are split over
// lanes, so VEC lanes read 8 logits per 16-byte load (rows 16-byte aligned,
// vocab % 8 == 0), four loads in flight.
constexpr int kArgmaxThreads = 1024;

__device__ __forceinline__ void argmax_take(float x, int i, float &best, int &index) {
    if (x > best || (x == best && i < index)) {
        best = x;
        index = i;
    }
}

template <bool VEC>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const uint16_t *logits, int rows, int vocab,
                                                                int32_t *out) {
    __shared__ float values[kArgmaxThreads];
    __shared__ int indices[kArgmaxThreads];
    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    const uint16_t *l = logits + (int64_t)row * vocab;
    float best = -INFINITY;
    int index = 0;
    if (VEC) {
        const uint4 *l4 = reinterpret_cast<const uint4 *>(l);
        const int chunks = vocab / 8;
        constexpr int U = 4;
        for (int base = tid; base < chunks; base += kArgmaxThreads * U) {
            uint4 v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int c = base + u * kArgmaxThreads;
                if (c < chunks) v[u] = l4[c];
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int c = base + u * kArgmaxThreads;
                if (c >= chunks) break;
                const uint32_t words[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    argmax_take(read_bf16((uint16_t)(words[k] & 0xffffu)), c * 8 + 2 * k, best, index);
                    argmax_take(read_bf16((uint16_t)(words[k] >> 16)), c * 8 + 2 * k + 1, best, index);
                }
            }
        }
    } else {
        for (int i = tid; i < vocab; i += kArgmaxThreads) argmax_take(read_bf16(l[i]), i, best, index);
    }
    values[tid] = best;
    indices[tid] = index;
    __syncthreads();
    for (int stride = kArgmaxThreads / 2; stride > 0; stride >>= 1) {
        if (tid < stride) {
            const float ov = values[tid + stride];
            const int oi = indices[tid + stride];
            if (ov > values[tid] || (ov == values[tid] && oi < indices[tid])) {
                values[tid] = ov;
                indices[tid] = oi;
            }
        }
        __syncthreads();
    }
    if (tid == 0) out[row] = indices[0];
}

}  // namespace

hipError_t launch_rmsnorm(const uint16_t *in, const uint16_t *w, uint16_t *out, int tokens,
                          int hidden, float eps, hipStream_t stream) {
    const bool aligned = ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(w) |
                           reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    if (aligned && hidden % (128 * kRmsBatch) == 0 && hidden <= kRmsStagedMax)
        hipLaunchKernelGGL(rmsnorm_staged_kernel, dim3((unsigned)tokens), dim3(128), (size_t)hidden * 4, stream,
                           in, w, out, hidden, eps);
    else
        hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)tokens), dim3(128), 0, stream, in, w, out, hidden,
                           eps);
    return hipGetLastError();
}

namespace {

// rope_inverse_frequency on the host for pairs 0 .. head_dim/2 - 1: the same
// f32 operations in the same order (no contraction in this file), log and exp
// in f64 rounded once.  The last table is kept per thread, since a decoder
// launches the same one for every layer.
const RopeTable &rope_table(int head_dim, float theta, int llama3, float factor, float low, float high,
                            float original_max) {
    struct Cached {
        bool valid = false;
        int head_dim = 0, llama3 = 0;
        float theta = 0, factor = 0, low = 0, high = 0, original_max = 0;
        RopeTable table;
    };
    thread_local Cached c;
    if (c.valid && c.head_dim == head_dim && c.theta == theta && c.llama3 == llama3 && c.factor == factor &&
        c.low == low && c.high == high && c.original_max == original_max)
        return c.table;
    const float log_theta = (float)std::log((double)theta);
    for (int f = 0; f < head_dim / 2; ++f) {
        const float exponent = (-(float)(2 * f) * log_theta) / (float)head_dim;
        float inv = (float)std::exp((double)exponent);
        if (llama3) {
            const float wavelength = 6.28318530717958647692f / inv;
            const float low_wavelength = original_max / low;
            const float high_wavelength = original_max / high;
            if (wavelength > low_wavelength) {
                inv = inv / factor;
            } else if (wavelength >= high_wavelength) {
                const float smooth = (original_max / wavelength - low) / (high - low);
                inv = (1.0f - smooth) * (inv / factor) + smooth * inv;
            }
        }
        c.table.inv[f] = inv;
    }
    c.valid = true;
    c.head_dim = head_dim;
    c.theta = theta;
    c.llama3 = llama3;
    c.factor = factor;
    c.low = low;
    c.high = high;
    c.original_max = original_max;
    return c.table;
}

}  // namespace

// Table rows of positions 0 .. positions - 1, one lane per (position, pair).
__global__ __launch_bounds__(256) void rope_cossin_kernel(uint16_t *rows, int64_t positions, int half,
                                                          RopeTable table) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= positions * half) return;
    const int64_t p = i / half;
    const int f = (int)(i % half);
    float cs, sn;
    rope_trig(p, table.inv[f], cs, sn);
    rows[p * 2 * half + f] = write_bf16(cs);
    rows[p * 2 * half + half + f] = write_bf16(sn);
}

hipError_t launch_rope_cossin(uint16_t *rows, int64_t positions, int head_dim, float theta, int llama3, float factor,
                              float low, float high, float original_max, hipStream_t stream) {
    if (head_dim > 2 * kRopeTable || head_dim % 2) return hipErrorInvalidValue;
    const RopeTable &table = rope_table(head_dim, theta, llama3, factor, low, high, original_max);
    const int half = head_dim / 2;
    hipLaunchKernelGGL(rope_cossin_kernel, dim3((unsigned)((positions * half + 255) / 256)), dim3(256), 0, stream,
                       rows, positions, half, table);
    return hipGetLastError();
}

const RopeTable &rope_inverse_table(int head_dim, float theta, int llama3, float factor, float low, float high,
                                    float original_max) {
    return rope_table(head_dim, theta, llama3, factor, low, high, original_max);
}

hipError_t launch_rope(const uint16_t *in, uint16_t *out, int tokens, int heads, int head_dim,
                       int start, const int32_t *positions, float theta, int llama3, float factor,
                       float low, float high, float original_max, RopeCosSin cossin, hipStream_t stream) {
    if (head_dim <= 2 * kRopeTable) {
        const RopeTable &table = rope_table(head_dim, theta, llama3, factor, low, high, original_max);
        hipLaunchKernelGGL(rope_token_kernel, dim3((unsigned)tokens), dim3(256), 0, stream, in, out, heads,
                           head_dim, start, positions, table, cossin);
        return hipGetLastError();
    }
    const int64_t total = (int64_t)tokens * heads * head_dim;
    const unsigned blocks = (unsigned)((total + 255) / 256);
    hipLaunchKernelGGL(rope_kernel, dim3(blocks), dim3(256), 0, stream, in, out, total, heads, head_dim,
                       start, positions, theta, llama3, factor, low, high, original_max);
    return hipGetLastError();
}

bool rope_qk_supported(int head_dim, int heads, const void *q, const void *q_out, const void *k, const void *k_out) {
    // a row's pair units (8 rotate-half pairs each) must fit one workgroup's
    // kRopePairsPerLane x 256 lanes
    return head_dim % 16 == 0 && head_dim <= 2 * kRopeTable && heads >= 1 &&
           (int64_t)heads * (head_dim / 16) <= kRopePairsPerLane * 256 &&
           ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(q_out) | reinterpret_cast<uintptr_t>(k) |
             reinterpret_cast<uintptr_t>(k_out)) & 15) == 0;
}

hipError_t launch_rope_qk(const uint16_t *q, uint16_t *q_out, const uint16_t *k, uint16_t *k_out, int tokens,
                          int q_heads, int kv_heads, int head_dim, int start, float theta, int llama3, float factor,
                          float low, float high, float original_max, RopeCosSin cossin, hipStream_t stream) {
    const RopeTable &table = rope_table(head_dim, theta, llama3, factor, low, high, original_max);
    const int units = (q_heads + kv_heads) * (head_dim / 16);
    if (units > kRopePairsPerLane * 256) return hipErrorInvalidValue;
    // About 1,024 workgroups: rows per workgroup from the token count, then
    // the fewest pair units per lane (2 to 4) that hold those rows.  Measured
    // (us; 2 / 3 / 4 pairs per lane): 2,048 rows of 32 + 8 heads of 128 8.83 /
    // 8.37 / 8.91; 512 rows after 3,584 tokens 4.21 / 4.58 / 4.97; 8,192 rows
    // of 64 + 8 heads (one row per workgroup either way) - / 51.3 / 53.2.
    const int want = std::max(1, std::min(kRopeRows, tokens / 1024));
    const int pairs = std::max(2, std::min(kRopePairsPerLane, (want * units + 255) / 256));
    const int rows = std::max(1, std::min(kRopeRows, pairs * 256 / units));
    const int needed = std::max(2, (rows * units + 255) / 256);  // the same rows with fewer pairs
    const dim3 grid((unsigned)((tokens + rows - 1) / rows));
    if (needed <= 2)
        hipLaunchKernelGGL(rope_qk_kernel<2>, grid, dim3(256), 0, stream, q, q_out, k, k_out, tokens, rows, q_heads,
                           kv_heads, head_dim, start, table, cossin);
    else if (needed == 3)
        hipLaunchKernelGGL(rope_qk_kernel<3>, grid, dim3(256), 0, stream, q, q_out, k, k_out, tokens, rows, q_heads,
                           kv_heads, head_dim, start, table, cossin);
    else
        hipLaunchKernelGGL(rope_qk_kernel<4>, grid, dim3(256), 0, stream, q, q_out, k, k_out, tokens, rows, q_heads,
                           kv_heads, head_dim, start, table, cossin);
    return hipGetLastError();
}

hipError_t launch_rope_append(const RopeAppendArgs &a, hipStream_t stream) {
    if (a.head_dim > 2 * kRopeTable) return hipErrorInvalidValue;
    const RopeTable &table = rope_table(a.head_dim, a.theta, a.llama3, a.factor, a.low, a.high, a.original_max);
    const int64_t nk = (int64_t)a.batch * a.kv_heads * a.head_dim;
    const int64_t total = (int64_t)a.batch * a.q_heads * a.head_dim + nk + nk / 8;
    hipLaunchKernelGGL(rope_append_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, a, table);
    return hipGetLastError();
}

// The first SwiGLU stage for every BF16 gate value (kSwigluTableEntries).
__global__ __launch_bounds__(256) void swiglu_table_kernel(uint16_t *table) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    table[i] = swiglu_act_bf16((uint16_t)i);
}

hipError_t launch_swiglu_table(uint16_t *table, hipStream_t stream) {
    hipLaunchKernelGGL(swiglu_table_kernel, dim3(kSwigluTableEntries / 256), dim3(256), 0, stream, table);
    return hipGetLastError();
}

// write_bf16 against write_bf16_rule over every f32 encoding: thread t
// checks encodings t, t + threads, ... and stores its mismatch count.  Each
// step converts two values into one packed pair as kernels that write BF16
// vectors do (the instruction's two-source form, which the compiler uses for
// such pairs): encoding b in the low half and the bijection b * 0x9e3779b1
// (odd, so every encoding appears once) in the high half.
__global__ __launch_bounds__(256) void bf16_encoding_check_kernel(uint32_t *mismatches) {
    const uint32_t tid = blockIdx.x * 256u + threadIdx.x;
    const uint32_t threads = gridDim.x * 256u;
    uint32_t bad = 0;
    for (uint64_t b = tid; b < (1ull << 32); b += threads) {
        const float lo = __uint_as_float((uint32_t)b);
        const float hi = __uint_as_float((uint32_t)b * 0x9e3779b1u);
        bf16x2_t pair;
        pair[0] = __builtin_bit_cast(__bf16, write_bf16(lo));
        pair[1] = __builtin_bit_cast(__bf16, write_bf16(hi));
        const uint32_t got = __builtin_bit_cast(uint32_t, pair);
        bad += (got & 0xffffu) != write_bf16_rule(lo);
        bad += (got >> 16) != write_bf16_rule(hi);
    }
    mismatches[tid] = bad;
}

hipError_t launch_bf16_encoding_check(uint32_t *mismatches, hipStream_t stream) {
    hipLaunchKernelGGL(bf16_encoding_check_kernel, dim3(kEncodingCheckThreads / 256), dim3(256), 0, stream,
                       mismatches);
    return hipGetLastError();
}

hipError_t launch_swiglu(const uint16_t *gate, const uint16_t *up, uint16_t *out, size_t n,
                         hipStream_t stream) {
    const unsigned blocks = (unsigned)((n + 255) / 256);
    hipLaunchKernelGGL(swiglu_kernel, dim3(blocks), dim3(256), 0, stream, gate, up, out, (int64_t)n);
    return hipGetLastError();
}

hipError_t launch_add(const uint16_t *a, const uint16_t *b, uint16_t *out, size_t n, hipStream_t stream) {
    hipLaunchKernelGGL(add_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, a, b, out, (int64_t)n);
    return hipGetLastError();
}

hipError_t launch_embed(const uint16_t *table, const int32_t *ids, int tokens, int hidden, int vocab,
                        uint16_t *out, int *bad, hipStream_t stream) {
    const int64_t work = (int64_t)tokens * (hidden / 8);
    hipLaunchKernelGGL(embed_kernel, dim3((unsigned)((work + 255) / 256)), dim3(256), 0, stream, table, ids, tokens,
                       hidden, vocab, out, bad);
    return hipGetLastError();
}

hipError_t launch_argmax(const uint16_t *logits, int rows, int vocab, int32_t *out, hipStream_t stream) {
    if (vocab % 8 == 0 && (reinterpret_cast<uintptr_t>(logits) & 15) == 0)
        hipLaunchKernelGGL(argmax_kernel<true>, dim3((unsigned)rows), dim3(kArgmaxThreads), 0, stream, logits, rows,
                           vocab, out);
    else
        hipLaunchKernelGGL(argmax_kernel<false>, dim3((unsigned)rows), dim3(kArgmaxThreads), 0, stream, logits, rows,
                           vocab, out);
    return hipGetLastError();
}

}  // namespace mslim
