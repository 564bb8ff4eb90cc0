// Portable-backend decode: one query token over exact K/V frames.
//
// Replaces GpuBackend::decode (gpu_backend.rs:149-377), whose OpenCL kernels
// mslim_qk / mslim_softmax / mslim_pv (gpu_attention.cl:5-82) take an f32
// query [q_heads][D], raw little-endian K/V frames [tokens][kv_heads][D] in
// BF16, F16 or F32 (key and value formats independent) and produce f32
// output [q_heads][D].  Everything here is computed in f32; formats are
// decoded exactly (BF16 and F16 widen to f32 without rounding).
//
// Layout of the work: a workgroup of 256 threads owns one (query head,
// split) pair.  A split walks its tokens in tiles of 256, one token per
// thread for the score, then all threads accumulate P.V with the head
// dimension across threads (V reads coalesced) and the tile's tokens spread
// over thread groups when D < 256.  An online softmax carries (m, l) across
// tiles; splits are combined by a fixed-order merge launch, so the result is
// deterministic for a given split count.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace mslim {

namespace {

constexpr int kThreads = 256;

template <int FMT>
struct Fmt;
template <>
struct Fmt<kFormatBf16> {
    __device__ static float at(const void *p, int64_t i) {
        return read_bf16(static_cast<const uint16_t *>(p)[i]);
    }
    __device__ static void widen8(const uint4 w, float *out) {
        const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            out[2 * j] = bf16_lo(u[j]);
            out[2 * j + 1] = bf16_hi(u[j]);
        }
    }
};
template <>
struct Fmt<kFormatF16> {
    __device__ static float at(const void *p, int64_t i) {
        return half_to_float(static_cast<const uint16_t *>(p)[i]);
    }
    __device__ static void widen8(const uint4 w, float *out) {
        const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            out[2 * j] = half_to_float((uint16_t)(u[j] & 0xffffu));
            out[2 * j + 1] = half_to_float((uint16_t)(u[j] >> 16));
        }
    }
};
template <>
struct Fmt<kFormatF32> {
    __device__ static float at(const void *p, int64_t i) { return static_cast<const float *>(p)[i]; }
};

struct FramesArgs {
    const float *q;
    const void *k, *v;
    float *out;
    float *partial_ml;   // [q_heads][splits][2]
    float *partial_acc;  // [q_heads][splits][D]
    int64_t tokens;
    int q_heads, kv_heads, head_dim;
    int split_tokens, splits;
    float scale;
};

// Block-wide reductions of one float per thread (every thread gets the result).
__device__ float block_max(float v, float *red) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = wave_xor_max(v, m);
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}
__device__ float block_sum(float v, float *red) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = wave_xor_sum(v, m);
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[4 + wave] = v;
    __syncthreads();
    return (red[4] + red[5]) + (red[6] + red[7]);
}

// Dot product of the query (in LDS) with one key row.  VEC reads the row in
// 16-byte pieces; the caller guarantees 16-byte alignment of every row.
template <int KF, bool VEC>
__device__ float key_dot(const float *q_lds, const void *k, int64_t row, int d) {
    float dot = 0.0f;
    if constexpr (VEC && KF != kFormatF32) {
        const uint4 *p = reinterpret_cast<const uint4 *>(static_cast<const char *>(k) + row * 2);
        for (int j = 0; j < d; j += 8) {
            float e[8];
            Fmt<KF>::widen8(p[j / 8], e);
#pragma unroll
            for (int i = 0; i < 8; ++i) dot = fmaf(q_lds[j + i], e[i], dot);
        }
    } else if constexpr (VEC) {
        const float4 *p = reinterpret_cast<const float4 *>(static_cast<const float *>(k) + row);
        for (int j = 0; j < d; j += 4) {
            const float4 e = p[j / 4];
            dot = fmaf(q_lds[j], e.x, dot);
            dot = fmaf(q_lds[j + 1], e.y, dot);
            dot = fmaf(q_lds[j + 2], e.z, dot);
            dot = fmaf(q_lds[j + 3], e.w, dot);
        }
    } else {
        for (int j = 0; j < d; ++j) dot = fmaf(q_lds[j], Fmt<KF>::at(k, row + j), dot);
    }
    return dot;
}

// DG threads share one token's P.V row (DG = the head dimension rounded up to
// a power of two, at most 256); kThreads / DG groups take interleaved tokens.
template <int KF, int VF, bool VEC>
__global__ __launch_bounds__(kThreads) void frames_split_kernel(FramesArgs a) {
    __shared__ float q_lds[kFramesMaxDim];
    __shared__ float p_lds[kThreads];
    __shared__ float red[8];
    __shared__ float acc_lds[kThreads];

    const int tid = threadIdx.x;
    const int qh = blockIdx.y;
    const int split = blockIdx.x;
    const int d = a.head_dim;
    const int kvh = qh / (a.q_heads / a.kv_heads);
    for (int j = tid; j < d; j += kThreads) q_lds[j] = a.q[(int64_t)qh * d + j];

    int dg = 1;
    while (dg < d && dg < kThreads) dg <<= 1;
    const int groups = kThreads / dg;
    const int grp = tid / dg;
    const int lane_d = tid % dg;
    constexpr int kMaxPer = kFramesMaxDim / kThreads;  // dims per thread when D > 256
    float acc[kMaxPer];
#pragma unroll
    for (int i = 0; i < kMaxPer; ++i) acc[i] = 0.0f;

    const int64_t begin = (int64_t)split * a.split_tokens;
    const int64_t end = min(a.tokens, begin + a.split_tokens);
    const int64_t row_stride = (int64_t)a.kv_heads * d;
    float m_run = -INFINITY, l_run = 0.0f;
    __syncthreads();

    for (int64_t t0 = begin; t0 < end; t0 += kThreads) {
        const int64_t t = t0 + tid;
        float s = -INFINITY;
        if (t < end) s = key_dot<KF, VEC>(q_lds, a.k, t * row_stride + (int64_t)kvh * d, d) * a.scale;
        const float m_new = fmaxf(m_run, block_max(s, red));
        const float alpha = expf(m_run - m_new);
        const float p = t < end ? expf(s - m_new) : 0.0f;
        p_lds[tid] = p;
        l_run = l_run * alpha + block_sum(p, red);  // block_sum's barriers publish p_lds
        m_run = m_new;
#pragma unroll
        for (int i = 0; i < kMaxPer; ++i) acc[i] *= alpha;
        const int n = (int)min((int64_t)kThreads, end - t0);
        for (int j = grp; j < n; j += groups) {
            const float pj = p_lds[j];
            const int64_t vrow = (t0 + j) * row_stride + (int64_t)kvh * d;
#pragma unroll
            for (int i = 0; i < kMaxPer; ++i) {
                const int dim = lane_d + i * dg;
                if (dim < d) acc[i] = fmaf(pj, Fmt<VF>::at(a.v, vrow + dim), acc[i]);
            }
        }
        __syncthreads();  // p_lds is rewritten by the next tile
    }

    // Sum the token groups (only when several share the tile: then D <= 128
    // and each thread holds one dimension).
    if (groups > 1) {
        acc_lds[tid] = acc[0];
        __syncthreads();
        if (tid < dg) {
            float sum = 0.0f;
            for (int g = 0; g < groups; ++g) sum += acc_lds[g * dg + tid];
            acc[0] = sum;
        }
    }
    if (grp != 0) return;
    if (a.splits == 1) {
#pragma unroll
        for (int i = 0; i < kMaxPer; ++i) {
            const int dim = lane_d + i * dg;
            if (dim < d) a.out[(int64_t)qh * d + dim] = acc[i] / l_run;
        }
        return;
    }
    const int64_t slot = (int64_t)qh * a.splits + split;
    if (tid == 0) {
        a.partial_ml[slot * 2] = m_run;
        a.partial_ml[slot * 2 + 1] = l_run;
    }
#pragma unroll
    for (int i = 0; i < kMaxPer; ++i) {
        const int dim = lane_d + i * dg;
        if (dim < d) a.partial_acc[slot * d + dim] = acc[i];
    }
}

// Fixed-order log-sum-exp merge of the splits of one query head.
__global__ __launch_bounds__(kThreads) void frames_merge_kernel(FramesArgs a) {
    const int qh = blockIdx.x;
    const float *ml = a.partial_ml + (int64_t)qh * a.splits * 2;
    const float *acc = a.partial_acc + (int64_t)qh * a.splits * a.head_dim;
    float m = -INFINITY;
    for (int s = 0; s < a.splits; ++s) m = fmaxf(m, ml[2 * s]);
    float l = 0.0f;
    for (int s = 0; s < a.splits; ++s) l += expf(ml[2 * s] - m) * ml[2 * s + 1];
    for (int dim = threadIdx.x; dim < a.head_dim; dim += kThreads) {
        float o = 0.0f;
        for (int s = 0; s < a.splits; ++s) o += expf(ml[2 * s] - m) * acc[(int64_t)s * a.head_dim + dim];
        a.out[(int64_t)qh * a.head_dim + dim] = o / l;
    }
}

// Output of an empty cache (gpu_backend.rs:157-159); a kernel rather than a
// memset so that the call stays a plain kernel node under graph capture.
__global__ __launch_bounds__(kThreads) void frames_zero_kernel(float *out, int n) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i < n) out[i] = 0.0f;
}

template <int KF, int VF>
hipError_t launch_formats(const FramesArgs &a, bool vec, hipStream_t stream) {
    const dim3 grid((unsigned)a.splits, (unsigned)a.q_heads);
    if (vec)
        hipLaunchKernelGGL((frames_split_kernel<KF, VF, true>), grid, dim3(kThreads), 0, stream, a);
    else
        hipLaunchKernelGGL((frames_split_kernel<KF, VF, false>), grid, dim3(kThreads), 0, stream, a);
    return hipGetLastError();
}

template <int KF>
hipError_t launch_value_format(const FramesArgs &a, int vf, bool vec, hipStream_t stream) {
    if (vf == kFormatBf16) return launch_formats<KF, kFormatBf16>(a, vec, stream);
    if (vf == kFormatF16) return launch_formats<KF, kFormatF16>(a, vec, stream);
    return launch_formats<KF, kFormatF32>(a, vec, stream);
}

}  // namespace

int frames_split_tokens(int64_t tokens, int q_heads) {
    // About 2,048 workgroups over the whole launch, at least one 256-token
    // tile per split.
    int64_t splits = (2048 + q_heads - 1) / q_heads;
    const int64_t tiles = (tokens + kThreads - 1) / kThreads;
    splits = std::max<int64_t>(1, std::min(splits, tiles));
    const int64_t per = (tokens + splits - 1) / splits;
    return (int)((per + kThreads - 1) / kThreads * kThreads);
}

hipError_t launch_frames_decode(const FramesLaunch &l, hipStream_t stream) {
    if (l.tokens == 0) {
        const int n = l.q_heads * l.head_dim;
        hipLaunchKernelGGL(frames_zero_kernel, dim3((unsigned)((n + kThreads - 1) / kThreads)), dim3(kThreads),
                           0, stream, l.out, n);
        return hipGetLastError();
    }
    FramesArgs a{};
    a.q = l.q; a.k = l.k; a.v = l.v; a.out = l.out;
    a.partial_ml = l.partial_ml; a.partial_acc = l.partial_acc;
    a.tokens = l.tokens;
    a.q_heads = l.q_heads; a.kv_heads = l.kv_heads; a.head_dim = l.head_dim;
    a.split_tokens = l.split_tokens;
    a.splits = (int)((l.tokens + l.split_tokens - 1) / l.split_tokens);
    a.scale = l.scale;
    // 16-byte row pieces when every row start is 16-byte aligned.
    const int kb = l.key_format == kFormatF32 ? 4 : 2;
    const bool vec = ((int64_t)l.head_dim * kb) % 16 == 0 && (reinterpret_cast<uintptr_t>(l.k) & 15) == 0;
    hipError_t e;
    if (l.key_format == kFormatBf16) e = launch_value_format<kFormatBf16>(a, l.value_format, vec, stream);
    else if (l.key_format == kFormatF16) e = launch_value_format<kFormatF16>(a, l.value_format, vec, stream);
    else e = launch_value_format<kFormatF32>(a, l.value_format, vec, stream);
    if (e != hipSuccess || a.splits == 1) return e;
    hipLaunchKernelGGL(frames_merge_kernel, dim3((unsigned)a.q_heads), dim3(kThreads), 0, stream, a);
    return hipGetLastError();
}

}  // namespace mslim
