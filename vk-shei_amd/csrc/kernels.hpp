// Host-side launch interface of the gfx950 kernels (one translation unit per
// kernel family).  Every launcher validates nothing: the C ABI layer checks
// shapes, pointers and limits before calling it.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "common.hpp"

namespace mslim {

// Sequences per decode launch.  Launches of up to kInlineBatch sequences
// carry their launch tables in the kernel arguments; larger ones copy them to
// the device on the stream first (DecodeTables).
constexpr int kMaxBatch = 4096;
constexpr int kInlineBatch = 64;

// A pinned host buffer and a device buffer of `bytes` each for the launch
// tables of a decode launch that does not carry them in its arguments, and
// the event recorded after the launches that read them: the caller waits for
// it before reusing the buffers.
struct DecodeTables {
    void *host;
    void *device;
    size_t bytes;
    hipEvent_t done;
};

struct DecodeLaunch {
    const uint16_t *q;
    const uint16_t *k;  // dense cache base or K page pool
    const uint16_t *v;  // dense cache base or V page pool
    uint16_t *out;
    float *partial_ml;   // [splits_total][kv_heads][G][2]
    float *partial_acc;  // [splits_total][kv_heads][G][D]
    int *counters;       // [batch][kv_heads], all zero between launches
    const int32_t *page_table;  // paged only: [batch][pages_per_seq]
    int64_t seq_stride_tokens;  // dense only
    int pages_per_seq;
    int page_tokens;            // paged only, multiple of 16
    int batch, q_heads, kv_heads, head_dim;
    float scale;
    int split_tokens;           // multiple of 64
    int seq_len[kMaxBatch];
    bool paged;
    // false: the last split workgroup of each (sequence, kv head) merges the
    // partials (counters needed); true: a merge launch follows the decode
    // launch (counters unused).  Both give the same bits.
    bool separate_merge;
    // Launches whose tables do not fit the kernel arguments
    // (decode_table_bytes > 0) need these buffers.
    const DecodeTables *tables;
};

// Number of split partitions of a sequence of `tokens` tokens.
inline int decode_splits(int tokens, int split_tokens) {
    return (tokens + split_tokens - 1) / split_tokens;
}
// Library choice of split_tokens for a batch: about one workgroup per CU for
// equal lengths, smaller for ragged lengths when that evens out the busiest
// CU's load; a multiple of 256 in 256..16384, or 128 for tiny batches.
int decode_auto_split_tokens(const int32_t *seq_lens, int batch, int kv_heads);
// True when the MFMA fast path covers this geometry.
bool decode_fast_path(int head_dim, int group);
hipError_t launch_decode(const DecodeLaunch &a, hipStream_t stream);
// Bytes of the device copy of a launch's tables (0: they fit the kernel
// arguments).  Needs seq_len, split_tokens, the geometry and separate_merge.
size_t decode_table_bytes(const DecodeLaunch &l);
// Split-partial bytes a decode launch of this shape needs.
size_t decode_partial_bytes(const DecodeLaunch &l);
// A file-scope device array of kDecodeStaticBytes that the allocation-free
// decode entry point uses for its split partials.  decode_static_scratch
// returns its address on the current device (hipGetSymbolAddress on the first
// call per device, cached after).  Every call on one device shares it.
constexpr size_t kDecodeStaticBytes = (size_t)16 << 20;
constexpr int kMaxDevices = 64;
hipError_t decode_static_scratch(int device, float **ptr);
// n int32 zeros at p (a fill kernel: safe under graph capture).
hipError_t launch_zero_i32(int *p, int n, hipStream_t stream);

struct PrefillLaunch {
    const uint16_t *q, *k, *v;
    uint16_t *out;
    int queries, prior, q_heads, kv_heads, head_dim;
    float scale;
    bool split_allowed;  // chunk long row blocks when the launch is small
    float *partial;      // split workspace of prefill_split_plan().partial_bytes
    int *counters;       // prefill_split_plan().counters ints, zero between launches
    bool pool_allowed;   // hand the shortest row blocks out at run time (unsplit launches)
    int *pool_counter;   // one int, zero between launches, when prefill_pool_items() > 0
};
bool prefill_fast_path(int head_dim, int group);
// Row blocks per XCD that an unsplit launch hands out at run time (0: none).
int prefill_pool_items(const PrefillLaunch &l);
// How a launch splits its row blocks: chunk_tiles == 0 means no split.
struct PrefillSplit {
    int chunk_tiles = 0, max_chunks = 1, items = 0, counters = 0;
    size_t partial_bytes = 0;
};
PrefillSplit prefill_split_plan(const PrefillLaunch &l);
hipError_t launch_prefill(const PrefillLaunch &a, hipStream_t stream);

// Portable-backend decode: f32 query, raw K/V frames, f32 output.
constexpr int kFormatBf16 = 1, kFormatF16 = 2, kFormatF32 = 3;  // gpu_backend.rs:258-262
constexpr int kFramesMaxDim = 1024;
struct FramesLaunch {
    const float *q;
    const void *k, *v;
    int key_format, value_format;
    float *out;
    float *partial_ml, *partial_acc;  // [q_heads][splits][2], [q_heads][splits][D]
    int64_t tokens;                   // >= 1
    int q_heads, kv_heads, head_dim;
    int split_tokens;                 // multiple of 256
    float scale;
};
// Tokens per split for a launch of `tokens` tokens and q_heads heads.
int frames_split_tokens(int64_t tokens, int q_heads);
hipError_t launch_frames_decode(const FramesLaunch &l, hipStream_t stream);

hipError_t launch_rmsnorm(const uint16_t *in, const uint16_t *w, uint16_t *out, int tokens,
                          int hidden, float eps, hipStream_t stream);
// Cos and sin of every rotary pair by position, as BF16: row p (p <
// positions) holds c[0 .. half) then s[0 .. half), the values the RoPE
// kernels would compute for position p.  Built once per context and RoPE
// configuration by launch_rope_cossin; the launchers below take it
// optionally (rows null: none) and compute positions past it themselves.
struct RopeCosSin {
    const uint16_t *rows = nullptr;
    int64_t positions = 0;
};
// Inverse frequencies of the rotary pairs f = 0 .. head_dim/2 - 1 of one
// launch, computed on the host with the same f32 operations as
// rope_inverse_frequency (llm_rope, gpu_llm.cl:123-138) and the same
// once-rounded f64 log and exp, so the kernels need no f64 log or exp per
// lane.  Covers head_dim <= 2 * kRopeTable.  The host keeps the last one per
// thread.
constexpr int kRopeTable = 256;
struct RopeTable {
    float inv[kRopeTable];
};
const RopeTable &rope_inverse_table(int head_dim, float theta, int llama3, float factor, float low, float high,
                                    float original_max);

// c and s of pair f at `position`: BF16(cos(position * inv)), BF16(sin(...))
// with the phase in f32 and the functions in f64.  No contraction: with it
// the compiler may fold the f32 product into a double-precision FMA of the
// inlined cos, which changes c and s at some positions.
__device__ __forceinline__ void rope_trig(int64_t position, float inv, float &cs, float &sn) {
#pragma clang fp contract(off)
    const float phase = __fmul_rn((float)position, inv);
    cs = round_bf16((float)cos((double)phase));
    sn = round_bf16((float)sin((double)phase));
}

// The same from a RopeCosSin table where it covers the position.
__device__ __forceinline__ void rope_cs(const RopeCosSin &t, int64_t position, int f, int half, float inv,
                                        float &cs, float &sn) {
    if (position >= 0 && position < t.positions) {
        const uint16_t *row = t.rows + position * 2 * half;
        cs = read_bf16(row[f]);
        sn = read_bf16(row[half + f]);
    } else {
        rope_trig(position, inv, cs, sn);
    }
}
hipError_t launch_rope_cossin(uint16_t *rows, int64_t positions, int head_dim, float theta, int llama3, float factor,
                              float low, float high, float original_max, hipStream_t stream);
// Row t at position start + t, or positions[t] (device int32) when not null.
hipError_t launch_rope(const uint16_t *in, uint16_t *out, int tokens, int heads, int head_dim,
                       int start, const int32_t *positions, float theta, int llama3, float factor,
                       float low, float high, float original_max, RopeCosSin cossin, hipStream_t stream);
// RoPE of a prompt chunk's Q ([tokens][q_heads][head_dim]) and K
// ([tokens][kv_heads][head_dim]) rows at positions start + t in one launch,
// bit-identical to launch_rope on each; when rope_qk_supported (head_dim a
// multiple of 16, at most 512; heads = q_heads + kv_heads with heads *
// head_dim <= 16384; 16-byte aligned rows).
bool rope_qk_supported(int head_dim, int heads, const void *q, const void *q_out, const void *k, const void *k_out);
hipError_t launch_rope_qk(const uint16_t *q, uint16_t *q_out, const uint16_t *k, uint16_t *k_out, int tokens,
                          int q_heads, int kv_heads, int head_dim, int start, float theta, int llama3, float factor,
                          float low, float high, float original_max, RopeCosSin cossin, hipStream_t stream);
// A decode step's RoPE of Q and K and the append of rotated K and V to the
// page pool, one token per sequence at positions[b] (device int32).
struct RopeAppendArgs {
    const uint16_t *q, *k, *v;  // [batch][heads][head_dim] rows
    uint16_t *q_out, *k_pool, *v_pool;
    const int32_t *page_table;  // [batch][pages_per_seq]
    const int32_t *positions;   // [batch]
    int pages_per_seq, shift;   // page_tokens = 1 << shift
    int batch, q_heads, kv_heads, head_dim;
    float theta;
    int llama3;
    float factor, low, high, original_max;
    RopeCosSin cossin;
};
hipError_t launch_rope_append(const RopeAppendArgs &a, hipStream_t stream);
// Table of swiglu_act_bf16 for every BF16 gate value (128 KiB).
constexpr int kSwigluTableEntries = 65536;
hipError_t launch_swiglu_table(uint16_t *table, hipStream_t stream);
// Mismatch counts of write_bf16 against write_bf16_rule over all 2^32 f32
// encodings, one uint32 per thread (kEncodingCheckThreads of them).
constexpr int kEncodingCheckThreads = 1 << 20;
hipError_t launch_bf16_encoding_check(uint32_t *mismatches, hipStream_t stream);
hipError_t launch_swiglu(const uint16_t *gate, const uint16_t *up, uint16_t *out, size_t n,
                         hipStream_t stream);
hipError_t launch_add(const uint16_t *a, const uint16_t *b, uint16_t *out, size_t n, hipStream_t stream);
hipError_t launch_embed(const uint16_t *table, const int32_t *ids, int tokens, int hidden, int vocab,
                        uint16_t *out, int *bad, hipStream_t stream);
hipError_t launch_argmax(const uint16_t *logits, int rows, int vocab, int32_t *out, hipStream_t stream);

// ColdStore record frames of pool pages (record header, token-hash tables
// and footer; the payloads stay in the pool).
constexpr int kRecordHeaderBytes = 104;  // cold_store.rs:23
constexpr int kRecordFooterBytes = 56;   // cold_store.rs:24
constexpr uint32_t kRecordVersion = 3;   // cold_store.rs:22
struct RecordDesc {                      // layout of mslim_attn_page_record
    uint64_t page_id;
    uint64_t token_start;
    uint32_t layer;
    uint32_t tokens;
    int32_t pool_page;
    uint32_t first_row;                  // pool-page row of the record's first token
};
static_assert(sizeof(RecordDesc) == 32, "RecordDesc must match mslim_attn_page_record");
struct FramesCodecLaunch {
    const void *k_pool, *v_pool;
    int64_t pool_pages;
    int page_tokens, kv_heads, head_dim;
    uint32_t tile;
    const RecordDesc *records;
    int count;
    void *frames;
    int64_t frame_bytes;
    bool staged;  // payloads in compacted staging slots instead of pool pages
};
int64_t record_frame_bytes(int page_tokens);
hipError_t launch_record_frames(const FramesCodecLaunch &a, hipStream_t stream);
struct PayloadMoveLaunch {
    void *k_pool, *v_pool;
    int64_t pool_pages;
    int page_tokens, kv_heads, head_dim;
    const RecordDesc *records;
    int count;
    void *k_stage, *v_stage;  // [count][kv_heads * page_tokens * head_dim] BF16 slots
};
hipError_t launch_record_payloads(const PayloadMoveLaunch &a, bool to_staging, hipStream_t stream);

// Decode-batch projections on MFMA (tokens <= kSkinnyMaxTokens, inner a
// multiple of 32, x and weights 16-byte aligned): out[t][r] =
// BF16(sum_k x[t][k] w[r][k]) for up to three matrices in one launch, or with
// a residual-add or SwiGLU epilogue equal to the unfused elementwise kernels.
constexpr int kSkinnyMaxTokens = 16;
struct SkinnyMatrix {
    const uint16_t *w;  // [rows][inner]
    uint16_t *out;      // [tokens][rows]
    int rows;
};
bool skinny_supported(int inner, int tokens, const void *x, const void *w0, const void *w1 = nullptr,
                      const void *w2 = nullptr);
// The plain and SwiGLU forms can apply the RMSNorm (weights norm_w, eps) to x
// first when skinny_norm_supported: bit-identical to launch_rmsnorm followed
// by the product.
bool skinny_norm_supported(int inner, int tokens, const void *norm_w);
hipError_t launch_skinny_gemm(const SkinnyMatrix *m, int count, const uint16_t *x, int inner, int tokens,
                              hipStream_t stream, const uint16_t *norm_w = nullptr, float eps = 0.0f);
// Q, K and V of a decode step with the RoPE and K/V append of
// launch_rope_append in the epilogue (m[0..2] = Q, K, V; m[0].out receives
// the rotated Q, K and V go into the pools), optionally after the RMSNorm;
// bit-identical to the product (or RMSNorm + product) followed by
// launch_rope_append.  When skinny_rope_supported.
struct SkinnyRope {
    const int32_t *positions, *page_table;
    uint16_t *k_pool, *v_pool;
    int pages_per_seq, shift, kv_heads, head_dim;
    float theta;
    int llama3;
    float factor, low, high, original_max;
    RopeCosSin cossin;
};
bool skinny_rope_supported(int inner, int tokens, int head_dim, const void *x, const void *wq, const void *wk,
                           const void *wv, const void *norm_w);
hipError_t launch_skinny_qkv_rope(const SkinnyMatrix *m, const uint16_t *x, int inner, int tokens,
                                  const uint16_t *norm_w, float eps, const SkinnyRope &r, hipStream_t stream);
hipError_t launch_skinny_gemm_add(const SkinnyMatrix &m, const uint16_t *resid, const uint16_t *x, int inner,
                                  int tokens, hipStream_t stream);
// act_table: launch_swiglu_table's table (device, 128 KiB).
hipError_t launch_skinny_swiglu(const uint16_t *w_gate, const uint16_t *w_up, uint16_t *out, int rows,
                                const uint16_t *x, int inner, int tokens, const uint16_t *act_table,
                                hipStream_t stream, const uint16_t *norm_w = nullptr, float eps = 0.0f);

// The same products for any number of token rows (csrc/proj.hip): the tiled
// MFMA kernel when inner is a multiple of 64 and x and the weights are
// 16-byte aligned, one wavefront per output otherwise.  Same epilogues.
// Split launches (proj_ksplit(inner) > 1) keep fp32 partials in `partial`:
// proj_ksplit * products * tokens * (sum of the matrices' rows) floats, with
// products 2 for SwiGLU (gate and up) and 1 otherwise.
int proj_ksplit(int inner);
hipError_t launch_proj(const SkinnyMatrix *m, int count, const uint16_t *x, int inner, int tokens, float *partial,
                       hipStream_t stream);
hipError_t launch_proj_add(const SkinnyMatrix &m, const uint16_t *resid, const uint16_t *x, int inner, int tokens,
                           float *partial, hipStream_t stream);
// act_table: launch_swiglu_table's table (device, 128 KiB).
hipError_t launch_proj_swiglu(const uint16_t *w_gate, const uint16_t *w_up, uint16_t *out, int rows,
                              const uint16_t *x, int inner, int tokens, const uint16_t *act_table, float *partial,
                              hipStream_t stream);

hipError_t launch_pages_write(uint16_t *k_pool, uint16_t *v_pool, const int32_t *page_table,
                              int page_tokens, int kv_heads, int head_dim, int64_t first_token,
                              int64_t tokens, const uint16_t *k_rows, const uint16_t *v_rows,
                              hipStream_t stream);
// One token per sequence of a batch: row b goes to position positions[b]
// (device int32) through page-table row b; positions outside
// [0, pages_per_seq * page_tokens) are skipped.
hipError_t launch_pages_append(uint16_t *k_pool, uint16_t *v_pool, const int32_t *page_table,
                               int pages_per_seq, int page_tokens, int kv_heads, int head_dim,
                               int batch, const int32_t *positions, const uint16_t *k_rows,
                               const uint16_t *v_rows, hipStream_t stream);
hipError_t launch_pages_gather(const uint16_t *pool, const int32_t *page_table, int page_tokens,
                               int kv_heads, int head_dim, int64_t first_token, int64_t tokens,
                               uint16_t *rows_out, hipStream_t stream);
// Canonical head-major serialisation of one layer tensor: tokens
// [first, first+count) of kv head `head` into out[count][head_dim]
// (dense token-major source when page_table is null).
hipError_t launch_canonical_rows(const uint16_t *src, const int32_t *page_table, int page_tokens,
                                 int kv_heads, int head_dim, int head, int64_t first,
                                 int64_t count, uint16_t *out, hipStream_t stream);

}  // namespace mslim
