// C ABI of libmslim_attn: context, buffers, argument checks and dispatch.
// Declarations and reference citations live in include/mslim_attn.h.
#include "../../include/mslim_attn.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "kernels.hpp"
#include "sha256.hpp"

namespace {

thread_local std::string g_error;

// hipblaslt_bridge.cpp:26-34 conventions: -1 bad arguments, 100 + hipError_t.
int fail(const std::string &message, int code = -1) {
    g_error = message;
    return code;
}
int check_hip(hipError_t code, const char *what) {
    if (code == hipSuccess) return 0;
    g_error = std::string(what) + ": " + hipGetErrorString(code);
    return 100 + (int)code;
}


struct Context {
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    std::mutex mutex;
    void *workspace = nullptr;      // decode split partials
    uint16_t *swiglu_table = nullptr;  // SwiGLU activation of every BF16 gate value
    void *proj_partial = nullptr;      // fp32 partials of split projections
    size_t proj_partial_bytes = 0;
    void *norm_rows = nullptr;         // normalised rows of the RMSNorm + product entries
    size_t norm_rows_bytes = 0;
    void *qkv_rows = nullptr;          // Q, K, V rows of the unfused RMSNorm + QKV + RoPE + append
    size_t qkv_rows_bytes = 0;
    // RoPE cos/sin by position for the last RoPE configuration used
    uint16_t *rope_rows = nullptr;
    int64_t rope_positions = 0;
    size_t rope_bytes = 0;
    float rope_key[6] = {};    // head_dim, theta, llama3, factor, low, high
    float rope_key_max = 0.0f;  // original_max
    size_t workspace_bytes = 0;
    // Decode launch tables beyond the kernel arguments: a ring of pinned
    // host / device buffer pairs, each free again once its event completes.
    static constexpr int kTableSlots = 4;
    struct TableSlot {
        void *host = nullptr, *device = nullptr;
        size_t host_bytes = 0, device_bytes = 0;
        hipEvent_t done = nullptr;
    } table_slot[kTableSlots];
    int table_next = 0;
    int *counters = nullptr;        // decode split counters, zero between launches
    size_t counter_bytes = 0;
    bool counters_dirty = false;    // a decode launch failed: clear before the next
    bool separate_merge = false;    // MSLIM_ATTN_OPT_DECODE_MERGE
    void *prefill_partial = nullptr;  // split prefill partials
    size_t prefill_partial_bytes = 0;
    void *prefill_counters = nullptr;  // split chunk counters / pool counter, zero between launches
    size_t prefill_counter_bytes = 0;
    bool prefill_counters_dirty = false;
    bool prefill_split = true;        // MSLIM_ATTN_OPT_PREFILL_SPLIT
    bool prefill_pool = true;         // MSLIM_ATTN_OPT_PREFILL_POOL
    void *staging = nullptr;       // device, digest serialisation
    size_t staging_bytes = 0;
    void *host_staging = nullptr;  // pinned host, digest readback
    size_t host_staging_bytes = 0;
    void *backend = nullptr;       // device, backend_decode query/frames/output
    size_t backend_bytes = 0;
    hipEvent_t ev_start = nullptr, ev_end = nullptr;
    void *gemm_in = nullptr, *gemm_out = nullptr;  // device staging of matrix_multiply
    size_t gemm_in_bytes = 0, gemm_out_bytes = 0;

    ~Context() {
        if (stream) (void)hipStreamSynchronize(stream);
        if (gemm_in) (void)hipFree(gemm_in);
        if (gemm_out) (void)hipFree(gemm_out);
        if (workspace) (void)hipFree(workspace);
        if (swiglu_table) (void)hipFree(swiglu_table);
        if (proj_partial) (void)hipFree(proj_partial);
        if (norm_rows) (void)hipFree(norm_rows);
        if (qkv_rows) (void)hipFree(qkv_rows);
        if (rope_rows) (void)hipFree(rope_rows);
        if (prefill_partial) (void)hipFree(prefill_partial);
        if (prefill_counters) (void)hipFree(prefill_counters);
        if (counters) (void)hipFree(counters);
        for (TableSlot &t : table_slot) {
            if (t.host) (void)hipHostFree(t.host);
            if (t.device) (void)hipFree(t.device);
            if (t.done) (void)hipEventDestroy(t.done);
        }
        if (staging) (void)hipFree(staging);
        if (host_staging) (void)hipHostFree(host_staging);
        if (backend) (void)hipFree(backend);
        if (ev_start) (void)hipEventDestroy(ev_start);
        if (ev_end) (void)hipEventDestroy(ev_end);
        if (own_stream) (void)hipStreamDestroy(own_stream);
    }
};

Context *ctx_of(void *handle) { return static_cast<Context *>(handle); }

// Grow a device scratch buffer; the stream is drained first so no queued
// kernel still uses the old allocation.
int grow_device(Context &c, void **mem, size_t *cap, size_t bytes, const char *what) {
    if (*cap >= bytes) return 0;
    if (*mem) {
        if (int rc = check_hip(hipStreamSynchronize(c.stream), what)) return rc;
        if (int rc = check_hip(hipFree(*mem), what)) return rc;
    }
    *mem = nullptr;
    *cap = 0;
    if (int rc = check_hip(hipMalloc(mem, bytes), what)) return rc;
    *cap = bytes;
    return 0;
}

int grow_host(void **mem, size_t *cap, size_t bytes, const char *what) {
    if (*cap >= bytes) return 0;
    if (*mem) (void)hipHostFree(*mem);
    *mem = nullptr;
    *cap = 0;
    if (int rc = check_hip(hipHostMalloc(mem, bytes, hipHostMallocDefault), what)) return rc;
    *cap = bytes;
    return 0;
}

bool valid_geometry(int q_heads, int kv_heads, int head_dim) {
    // portable.rs:420-441 plus the kernels' 16-byte row pieces and D <= 256
    // (attention_kernel.rs:113-118 bounds the tiled kernel the same way).
    return q_heads > 0 && kv_heads > 0 && q_heads % kv_heads == 0 && head_dim > 0 &&
           head_dim <= 256 && head_dim % 8 == 0;
}

bool is_pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

// Serialises calls on a context and makes its device current for the call;
// the calling thread's device is restored on the way out.
struct Lock {
    explicit Lock(Context &c) : guard(c.mutex), device(c.device) {
        if (hipGetDevice(&saved) != hipSuccess) saved = -1;
        if (saved != device) (void)hipSetDevice(device);
    }
    ~Lock() {
        if (saved >= 0 && saved != device) (void)hipSetDevice(saved);
    }
    Lock(const Lock &) = delete;
    Lock &operator=(const Lock &) = delete;
    std::lock_guard<std::mutex> guard;
    int device;
    int saved = -1;
};

static_assert(MSLIM_ATTN_MAX_BATCH == mslim::kMaxBatch, "decode batch limit of the C ABI and the launcher");

// Argument checks and the split choice shared by every decode entry point.
int decode_prepare(mslim::DecodeLaunch &l, const int32_t *seq_lens, int split_tokens) {
    if (l.batch < 1 || l.batch > MSLIM_ATTN_MAX_BATCH || !seq_lens)
        return fail("decode batch must be 1..4096 with host seq_lens");
    if (!valid_geometry(l.q_heads, l.kv_heads, l.head_dim))
        return fail("decode geometry invalid (q_heads % kv_heads, head_dim multiple of 8 <= 256)");
    if (!l.q || !l.k || !l.v || !l.out) return fail("decode needs non-null q, k, v, out");
    if (l.out == l.q || l.out == l.k || l.out == l.v)
        return fail("decode output must not alias read-only Q/K/V");
    if (!(l.scale > 0.0f) || !std::isfinite(l.scale)) return fail("decode scale must be finite and > 0");
    for (int i = 0; i < l.batch; ++i) {
        if (seq_lens[i] < 1) return fail("decode seq_lens must be >= 1");
        l.seq_len[i] = seq_lens[i];
    }
    if (split_tokens < 0 || split_tokens % 64)
        return fail("split_tokens must be 0 or a positive multiple of 64");
    l.split_tokens = split_tokens ? split_tokens
                                  : mslim::decode_auto_split_tokens(seq_lens, l.batch, l.kv_heads);
    return 0;
}

// Partials at `base`: the (m, l) pairs, then the accumulators.
void decode_place_partials(mslim::DecodeLaunch &l, void *base) {
    int64_t splits = 0;
    for (int i = 0; i < l.batch; ++i) splits += mslim::decode_splits(l.seq_len[i], l.split_tokens);
    const size_t ml_bytes = (size_t)splits * l.kv_heads * (l.q_heads / l.kv_heads) * 2 * sizeof(float);
    l.partial_ml = static_cast<float *>(base);
    l.partial_acc = reinterpret_cast<float *>(static_cast<char *>(base) + ml_bytes);
}

int decode_common(Context &c, mslim::DecodeLaunch &l, const int32_t *seq_lens, int split_tokens) {
    if (int rc = decode_prepare(l, seq_lens, split_tokens)) return rc;
    if (int rc = grow_device(c, &c.workspace, &c.workspace_bytes, mslim::decode_partial_bytes(l),
                             "hipMalloc decode split workspace"))
        return rc;
    decode_place_partials(l, c.workspace);
    // One split counter per (sequence, kv head); the kernel leaves them at
    // zero, so they are cleared only when the buffer is (re)allocated.
    const size_t ctr_bytes = (size_t)std::max(l.batch, mslim::kInlineBatch) * l.kv_heads * sizeof(int);
    if (c.counter_bytes < ctr_bytes) {
        void *mem = c.counters;
        if (int rc = grow_device(c, &mem, &c.counter_bytes, ctr_bytes, "hipMalloc decode split counters"))
            return rc;
        c.counters = static_cast<int *>(mem);
        c.counters_dirty = true;
    }
    // A fill kernel, not hipMemsetAsync: the call may be under graph capture.
    if (c.counters_dirty) {
        if (int rc = check_hip(mslim::launch_zero_i32(c.counters, (int)(c.counter_bytes / sizeof(int)), c.stream),
                               "clear split counters"))
            return rc;
        c.counters_dirty = false;
    }
    l.counters = c.counters;
    l.separate_merge = c.separate_merge;
    mslim::DecodeTables tables{};
    if (const size_t bytes = mslim::decode_table_bytes(l)) {
        hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
        if (int rc = check_hip(hipStreamIsCapturing(c.stream, &capture), "hipStreamIsCapturing")) return rc;
        if (capture != hipStreamCaptureStatusNone)
            return fail("decode of more than 64 sequences copies its launch tables host to device and "
                        "cannot be recorded into a graph");
        Context::TableSlot &t = c.table_slot[c.table_next];
        c.table_next = (c.table_next + 1) % Context::kTableSlots;
        // The slot's previous launch has read both buffers once this returns.
        if (!t.done)
            if (int rc = check_hip(hipEventCreateWithFlags(&t.done, hipEventDisableTiming), "hipEventCreate tables"))
                return rc;
        if (int rc = check_hip(hipEventSynchronize(t.done), "decode tables wait")) return rc;
        if (int rc = grow_host(&t.host, &t.host_bytes, bytes, "hipHostMalloc decode tables")) return rc;
        if (int rc = grow_device(c, &t.device, &t.device_bytes, bytes, "hipMalloc decode tables")) return rc;
        tables = mslim::DecodeTables{t.host, t.device, bytes, t.done};
        l.tables = &tables;
    }
    const int rc = check_hip(mslim::launch_decode(l, c.stream), "decode attention launch");
    // A launch that failed may have left counts behind: clear them before
    // the next fused merge relies on them.
    if (rc) c.counters_dirty = true;
    return rc;
}


// Checks shared by both portable-backend entry points (portable.rs:420-441
// geometry rules; the kernel holds the query in LDS, so head_dim <= 1024).
int frames_validate(int key_format, int value_format, int64_t tokens, int q_heads, int kv_heads,
                    int head_dim) {
    auto fmt_ok = [](int f) { return f >= MSLIM_ATTN_FORMAT_BF16 && f <= MSLIM_ATTN_FORMAT_F32; };
    if (!fmt_ok(key_format) || !fmt_ok(value_format))
        return fail("K/V format must be 1 (BF16), 2 (F16) or 3 (F32)");
    if (q_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || q_heads % kv_heads)
        return fail("invalid geometry: heads and dimension must be positive, q_heads divisible by kv_heads");
    if (head_dim > mslim::kFramesMaxDim) return fail("invalid geometry: head_dim above 1024");
    if (tokens < 0 || tokens > ((int64_t)1 << 40) / ((int64_t)kv_heads * head_dim))
        return fail("invalid geometry: token count out of range");
    return 0;
}

size_t format_bytes(int format) { return format == MSLIM_ATTN_FORMAT_F32 ? 4 : 2; }

// Enqueue split + merge on the context stream; returns the scratch bytes used.
int frames_enqueue(Context &c, mslim::FramesLaunch &l, uint64_t *scratch) {
    *scratch = 0;
    l.scale = (float)(1.0 / std::sqrt((double)l.head_dim));
    l.split_tokens = l.tokens > 0 ? mslim::frames_split_tokens(l.tokens, l.q_heads) : 256;
    const int64_t splits = (l.tokens + l.split_tokens - 1) / l.split_tokens;
    if (splits > 1) {
        const size_t ml = (size_t)l.q_heads * splits * 2 * sizeof(float);
        const size_t acc = (size_t)l.q_heads * splits * l.head_dim * sizeof(float);
        if (int rc = grow_device(c, &c.workspace, &c.workspace_bytes, ml + acc,
                                 "hipMalloc frames split workspace"))
            return rc;
        l.partial_ml = static_cast<float *>(c.workspace);
        l.partial_acc = reinterpret_cast<float *>(static_cast<char *>(c.workspace) + ml);
        *scratch = ml + acc;
    }
    return check_hip(mslim::launch_frames_decode(l, c.stream), "frames decode launch");
}

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }
}  // namespace

extern "C" {

const char *mslim_attn_last_error(void) { return g_error.c_str(); }

void *mslim_attn_ctx_new(void) {
    g_error.clear();
    if (const char *ov = std::getenv("HSA_OVERRIDE_GFX_VERSION")) {
        g_error = std::string("HSA_OVERRIDE_GFX_VERSION=") + ov +
                  " is refused: the kernels are built for native gfx950 only";
        return nullptr;
    }
    int count = 0;
    if (check_hip(hipGetDeviceCount(&count), "hipGetDeviceCount")) return nullptr;
    if (count < 1) {
        g_error = "No HIP GPU device";
        return nullptr;
    }
    int device = 0;
    if (check_hip(hipGetDevice(&device), "hipGetDevice")) return nullptr;
    hipDeviceProp_t props{};
    if (check_hip(hipGetDeviceProperties(&props, device), "hipGetDeviceProperties")) return nullptr;
    if (std::strncmp(props.gcnArchName, "gfx950", 6) != 0) {
        g_error = std::string("mslim_attn requires a gfx950 (MI355X) device, found ") + props.gcnArchName;
        return nullptr;
    }
    auto *c = new (std::nothrow) Context;
    if (!c) {
        g_error = "Out of memory for mslim_attn context";
        return nullptr;
    }
    c->device = device;
    if (check_hip(hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking), "hipStreamCreate")) {
        delete c;
        return nullptr;
    }
    c->stream = c->own_stream;
    // The SwiGLU activation of every BF16 gate value, for the fused
    // projection epilogue (128 KiB, built once, ready when this returns).
    if (check_hip(hipMalloc(&c->swiglu_table, (size_t)mslim::kSwigluTableEntries * 2), "hipMalloc SwiGLU table") ||
        check_hip(mslim::launch_swiglu_table(c->swiglu_table, c->own_stream), "SwiGLU table launch") ||
        check_hip(hipStreamSynchronize(c->own_stream), "SwiGLU table")) {
        delete c;
        return nullptr;
    }
    // The allocation-free decode's fixed partials array: its address on this
    // device is taken here, once, so that entry point's first call loads
    // nothing.
    float *scratch = nullptr;
    if (check_hip(mslim::decode_static_scratch(device, &scratch), "hipGetSymbolAddress decode scratch")) {
        delete c;
        return nullptr;
    }
    return c;
}

void mslim_attn_ctx_destroy(void *ctx) { delete ctx_of(ctx); }

int mslim_attn_get_device_info(void *ctx, mslim_attn_device_info *out) {
    g_error.clear();
    if (!ctx || !out) return fail("device info needs a context and an output struct");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    hipDeviceProp_t prop{};
    if (int rc = check_hip(hipGetDeviceProperties(&prop, c.device), "hipGetDeviceProperties")) return rc;
    int driver = 0;
    if (int rc = check_hip(hipDriverGetVersion(&driver), "hipDriverGetVersion")) return rc;
    size_t free_bytes = 0, total_bytes = 0;
    if (int rc = check_hip(hipMemGetInfo(&free_bytes, &total_bytes), "hipMemGetInfo")) return rc;
    std::memset(out, 0, sizeof *out);
    std::snprintf(out->name, sizeof out->name, "%s", prop.name);
    std::snprintf(out->arch, sizeof out->arch, "%s", prop.gcnArchName);
    std::snprintf(out->vendor, sizeof out->vendor, "%s", "Advanced Micro Devices, Inc.");
    out->driver_version = driver;
    out->compute_units = (uint32_t)prop.multiProcessorCount;
    out->global_memory_bytes = (uint64_t)prop.totalGlobalMem;
    out->max_allocation_bytes = (uint64_t)free_bytes;
    out->lds_bytes_per_workgroup = (uint32_t)prop.sharedMemPerBlock;
    out->max_clock_mhz = (uint32_t)(prop.clockRate / 1000);
    out->memory_clock_mhz = (uint32_t)(prop.memoryClockRate / 1000);
    out->memory_bus_bits = (uint32_t)prop.memoryBusWidth;
    return 0;
}

int mslim_attn_check_bf16_encoding(void *ctx, uint64_t *mismatches) {
    g_error.clear();
    if (!ctx || !mismatches) return fail("encoding check needs a context and an output");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    uint32_t *counts = nullptr;
    const size_t bytes = (size_t)mslim::kEncodingCheckThreads * sizeof(uint32_t);
    if (int rc = check_hip(hipMalloc(reinterpret_cast<void **>(&counts), bytes), "hipMalloc encoding check"))
        return rc;
    std::vector<uint32_t> host(mslim::kEncodingCheckThreads);
    int rc = check_hip(mslim::launch_bf16_encoding_check(counts, c.stream), "encoding check launch");
    if (!rc) rc = check_hip(hipMemcpyAsync(host.data(), counts, bytes, hipMemcpyDeviceToHost, c.stream), "D2H");
    if (!rc) rc = check_hip(hipStreamSynchronize(c.stream), "hipStreamSynchronize");
    const int free_rc = check_hip(hipFree(counts), "hipFree encoding check");
    if (rc) return rc;
    if (free_rc) return free_rc;
    uint64_t total = 0;
    for (uint32_t v : host) total += v;
    *mismatches = total;
    return 0;
}

int mslim_attn_ctx_set_stream(void *ctx, void *hip_stream) {
    g_error.clear();
    if (!ctx) return fail("null context");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    // The context's workspace and split counters serve one stream at a time:
    // work queued on the old stream finishes before any call on the new one.
    if (int rc = check_hip(hipStreamSynchronize(c.stream), "hipStreamSynchronize before stream switch"))
        return rc;
    c.stream = static_cast<hipStream_t>(hip_stream);
    return 0;
}

int mslim_attn_ctx_set_option(void *ctx, int option, int64_t value) {
    g_error.clear();
    if (!ctx) return fail("null context");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    switch (option) {
    case MSLIM_ATTN_OPT_DECODE_MERGE:
        if (value != MSLIM_ATTN_DECODE_MERGE_FUSED && value != MSLIM_ATTN_DECODE_MERGE_SEPARATE)
            return fail("decode merge mode must be 0 (fused) or 1 (separate launch)");
        c.separate_merge = value == MSLIM_ATTN_DECODE_MERGE_SEPARATE;
        return 0;
    case MSLIM_ATTN_OPT_PREFILL_SPLIT:
        if (value != 0 && value != 1) return fail("prefill split must be 0 (never) or 1 (automatic)");
        c.prefill_split = value == 1;
        return 0;
    case MSLIM_ATTN_OPT_PREFILL_POOL:
        if (value != 0 && value != 1) return fail("prefill pool must be 0 (static mapping) or 1 (automatic)");
        c.prefill_pool = value == 1;
        return 0;
    default:
        return fail("unknown context option");
    }
}

int mslim_attn_synchronize(void *ctx) {
    g_error.clear();
    if (!ctx) return fail("null context");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    return check_hip(hipStreamSynchronize(c.stream), "hipStreamSynchronize");
}

void *mslim_attn_buf_alloc(void *ctx, size_t bytes) {
    g_error.clear();
    if (!ctx || !bytes) {
        g_error = "invalid buffer allocation";
        return nullptr;
    }
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    void *p = nullptr;
    if (check_hip(hipMalloc(&p, bytes), "hipMalloc buffer")) return nullptr;
    return p;
}

void *mslim_attn_buf_upload(void *ctx, const uint8_t *bytes, size_t byte_length) {
    g_error.clear();
    if (!ctx || !bytes || !byte_length) {
        g_error = "Invalid upload payload";
        return nullptr;
    }
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    void *p = nullptr;
    if (check_hip(hipMalloc(&p, byte_length), "hipMalloc upload")) return nullptr;
    if (check_hip(hipMemcpy(p, bytes, byte_length, hipMemcpyHostToDevice), "hipMemcpy upload")) {
        (void)hipFree(p);
        return nullptr;
    }
    return p;
}

int mslim_attn_buf_free(void *ctx, void *buffer) {
    g_error.clear();
    if (!ctx || !buffer) return fail("invalid buffer handle");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    if (int rc = check_hip(hipStreamSynchronize(c.stream), "hipStreamSynchronize before free")) return rc;
    return check_hip(hipFree(buffer), "hipFree buffer");
}

int mslim_attn_buf_read(void *ctx, const void *buffer, size_t offset, uint8_t *out, size_t size) {
    g_error.clear();
    if (!ctx || !buffer || !out || !size) return fail("invalid buffer readback");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    if (int rc = check_hip(hipMemcpyAsync(out, static_cast<const char *>(buffer) + offset, size,
                                          hipMemcpyDeviceToHost, c.stream),
                           "hipMemcpy readback"))
        return rc;
    return check_hip(hipStreamSynchronize(c.stream), "hipStreamSynchronize readback");
}

int mslim_attn_buf_write(void *ctx, void *buffer, size_t offset, const uint8_t *in, size_t size) {
    g_error.clear();
    if (!ctx || !buffer || !in || !size) return fail("invalid buffer write");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    if (int rc = check_hip(hipMemcpyAsync(static_cast<char *>(buffer) + offset, in, size,
                                          hipMemcpyHostToDevice, c.stream),
                           "hipMemcpy write"))
        return rc;
    return check_hip(hipStreamSynchronize(c.stream), "hipStreamSynchronize write");
}

int mslim_attn_decode_auto_split(const int32_t *seq_lens, int batch, int kv_heads) {
    g_error.clear();
    if (!seq_lens || batch < 1 || batch > MSLIM_ATTN_MAX_BATCH || kv_heads < 1)
        return fail("decode batch must be 1..4096 with host seq_lens and kv_heads >= 1");
    for (int i = 0; i < batch; ++i)
        if (seq_lens[i] < 1) return fail("decode seq_lens must be >= 1");
    return mslim::decode_auto_split_tokens(seq_lens, batch, kv_heads);
}

int mslim_attn_decode_dense(void *ctx, const void *q, const void *k, const void *v, void *out,
                            int batch, const int32_t *seq_lens, int64_t seq_stride_tokens,
                            int q_heads, int kv_heads, int head_dim, float scale,
                            int split_tokens) {
    g_error.clear();
    if (!ctx) return fail("null context");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    mslim::DecodeLaunch l{};
    l.q = static_cast<const uint16_t *>(q);
    l.k = static_cast<const uint16_t *>(k);
    l.v = static_cast<const uint16_t *>(v);
    l.out = static_cast<uint16_t *>(out);
    l.batch = batch; l.q_heads = q_heads; l.kv_heads = kv_heads; l.head_dim = head_dim;
    l.scale = scale;
    l.paged = false;
    l.seq_stride_tokens = seq_stride_tokens;
    if (seq_lens && batch >= 1 && batch <= MSLIM_ATTN_MAX_BATCH) {
        for (int i = 0; i < batch; ++i)
            if (seq_lens[i] > seq_stride_tokens && batch > 1)
                return fail("dense decode: seq_lens exceed seq_stride_tokens");
    }
    if (batch > 1 && seq_stride_tokens < 1) return fail("dense decode: seq_stride_tokens must be >= 1");
    return decode_common(c, l, seq_lens, split_tokens);
}

}  // extern "C"

namespace {
int paged_launch_args(mslim::DecodeLaunch &l, const void *q, const void *k_pool, const void *v_pool, void *out,
                      int batch, const int32_t *seq_lens, const int32_t *page_table, int pages_per_seq,
                      int page_tokens, int q_heads, int kv_heads, int head_dim, float scale) {
    if (!page_table) return fail("paged decode needs a device page table");
    if (!is_pow2(page_tokens) || page_tokens < 16 || page_tokens > 4096)
        return fail("page_tokens must be a power of two in 16..4096");
    if (seq_lens && batch >= 1 && batch <= MSLIM_ATTN_MAX_BATCH) {
        for (int i = 0; i < batch; ++i)
            if ((int64_t)pages_per_seq * page_tokens < seq_lens[i])
                return fail("paged decode: page table row shorter than the sequence");
    }
    l = mslim::DecodeLaunch{};
    l.q = static_cast<const uint16_t *>(q);
    l.k = static_cast<const uint16_t *>(k_pool);
    l.v = static_cast<const uint16_t *>(v_pool);
    l.out = static_cast<uint16_t *>(out);
    l.batch = batch; l.q_heads = q_heads; l.kv_heads = kv_heads; l.head_dim = head_dim;
    l.scale = scale;
    l.paged = true;
    l.page_table = page_table;
    l.pages_per_seq = pages_per_seq;
    l.page_tokens = page_tokens;
    return 0;
}
}  // namespace

extern "C" {

int mslim_attn_decode_paged(void *ctx, const void *q, const void *k_pool, const void *v_pool,
                            void *out, int batch, const int32_t *seq_lens,
                            const int32_t *page_table, int pages_per_seq, int page_tokens,
                            int q_heads, int kv_heads, int head_dim, float scale,
                            int split_tokens) {
    g_error.clear();
    if (!ctx) return fail("null context");
    mslim::DecodeLaunch l;
    if (int rc = paged_launch_args(l, q, k_pool, v_pool, out, batch, seq_lens, page_table, pages_per_seq,
                                   page_tokens, q_heads, kv_heads, head_dim, scale))
        return rc;
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    return decode_common(c, l, seq_lens, split_tokens);
}

int mslim_attn_decode_paged_noalloc(void *ctx, const void *q, const void *k_pool, const void *v_pool,
                                    void *out, int batch, const int32_t *seq_lens,
                                    const int32_t *page_table, int pages_per_seq, int page_tokens,
                                    int q_heads, int kv_heads, int head_dim, float scale,
                                    int split_tokens) {
    g_error.clear();
    if (!ctx) return fail("null context");
    mslim::DecodeLaunch l;
    if (int rc = paged_launch_args(l, q, k_pool, v_pool, out, batch, seq_lens, page_table, pages_per_seq,
                                   page_tokens, q_heads, kv_heads, head_dim, scale))
        return rc;
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    if (int rc = decode_prepare(l, seq_lens, split_tokens)) return rc;
    const size_t need = mslim::decode_partial_bytes(l);
    if (need > mslim::kDecodeStaticBytes)
        return fail("allocation-free decode: split partials need " + std::to_string(need) +
                    " bytes, above the fixed " + std::to_string(mslim::kDecodeStaticBytes) +
                    "-byte scratch; use a larger split_tokens or mslim_attn_decode_paged");
    float *scratch = nullptr;
    if (int rc = check_hip(mslim::decode_static_scratch(c.device, &scratch), "hipGetSymbolAddress decode scratch"))
        return rc;
    decode_place_partials(l, scratch);
    // The merge runs as its own launch, so no counter has to start at zero.
    l.counters = nullptr;
    l.separate_merge = true;
    if (mslim::decode_table_bytes(l))
        return fail("allocation-free decode takes at most 64 sequences (launch tables in the kernel "
                    "arguments); use mslim_attn_decode_paged");
    return check_hip(mslim::launch_decode(l, c.stream), "decode attention launch");
}

int mslim_attn_prefill_split_tiles(int queries, int prior, int q_heads, int kv_heads, int head_dim) {
    g_error.clear();
    if (!valid_geometry(q_heads, kv_heads, head_dim) || queries < 1 || prior < 0 ||
        (int64_t)queries + prior > INT32_MAX - 64)
        return fail("prefill split query needs a valid geometry, queries >= 1 and prior >= 0");
    mslim::PrefillLaunch l{};
    l.queries = queries; l.prior = prior; l.q_heads = q_heads; l.kv_heads = kv_heads; l.head_dim = head_dim;
    l.split_allowed = true;
    return mslim::prefill_split_plan(l).chunk_tiles;
}

int mslim_attn_prefill_pool_items(int queries, int prior, int q_heads, int kv_heads, int head_dim) {
    g_error.clear();
    if (!valid_geometry(q_heads, kv_heads, head_dim) || queries < 1 || prior < 0 ||
        (int64_t)queries + prior > INT32_MAX - 64)
        return fail("prefill pool query needs a valid geometry, queries >= 1 and prior >= 0");
    mslim::PrefillLaunch l{};
    l.queries = queries; l.prior = prior; l.q_heads = q_heads; l.kv_heads = kv_heads; l.head_dim = head_dim;
    l.split_allowed = true;
    l.pool_allowed = true;
    return mslim::prefill_pool_items(l);
}

int mslim_attn_prefill_causal(void *ctx, const void *q, const void *k, const void *v, void *out,
                              int queries, int prior, int q_heads, int kv_heads, int head_dim,
                              float scale) {
    g_error.clear();
    if (!ctx) return fail("null context");
    if (!valid_geometry(q_heads, kv_heads, head_dim)) return fail("prefill geometry invalid");
    if (queries < 1 || prior < 0 || (int64_t)queries + prior > INT32_MAX - 64)
        return fail("prefill needs queries >= 1, prior >= 0 and a 32-bit history");
    if (!q || !k || !v || !out) return fail("prefill needs non-null q, k, v, out");
    if (out == q || out == k || out == v) return fail("prefill output must not alias read-only Q/K/V");
    if (!(scale > 0.0f) || !std::isfinite(scale)) return fail("prefill scale must be finite and > 0");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    mslim::PrefillLaunch l{};
    l.q = static_cast<const uint16_t *>(q);
    l.k = static_cast<const uint16_t *>(k);
    l.v = static_cast<const uint16_t *>(v);
    l.out = static_cast<uint16_t *>(out);
    l.queries = queries; l.prior = prior; l.q_heads = q_heads; l.kv_heads = kv_heads;
    l.head_dim = head_dim; l.scale = scale;
    l.split_allowed = c.prefill_split;
    l.pool_allowed = c.prefill_pool;
    const mslim::PrefillSplit plan = mslim::prefill_split_plan(l);
    const int pool = plan.chunk_tiles ? 0 : mslim::prefill_pool_items(l);
    if (plan.chunk_tiles || pool) {
        if (plan.chunk_tiles) {
            if (int rc = grow_device(c, &c.prefill_partial, &c.prefill_partial_bytes, plan.partial_bytes,
                                     "hipMalloc prefill split partials"))
                return rc;
        }
        // A split launch counts chunks per row block; a pooled one draws
        // from counter 0.  Both leave their counters at zero.
        const size_t ctr_bytes = plan.chunk_tiles ? (size_t)plan.counters * sizeof(int) : sizeof(int);
        if (c.prefill_counter_bytes < ctr_bytes) {
            if (int rc = grow_device(c, &c.prefill_counters, &c.prefill_counter_bytes, ctr_bytes,
                                     "hipMalloc prefill split counters"))
                return rc;
            c.prefill_counters_dirty = true;
        }
        if (c.prefill_counters_dirty) {
            if (int rc = check_hip(mslim::launch_zero_i32(static_cast<int *>(c.prefill_counters),
                                                          (int)(c.prefill_counter_bytes / sizeof(int)), c.stream),
                                   "clear prefill split counters"))
                return rc;
            c.prefill_counters_dirty = false;
        }
        l.partial = static_cast<float *>(c.prefill_partial);
        l.counters = static_cast<int *>(c.prefill_counters);
        l.pool_counter = static_cast<int *>(c.prefill_counters);
    }
    const int rc = check_hip(mslim::launch_prefill(l, c.stream), "prefill attention launch");
    if (rc && (plan.chunk_tiles || pool)) c.prefill_counters_dirty = true;
    return rc;
}

int mslim_attn_frames_decode(void *ctx, const float *query, const void *keys, int key_format,
                             const void *values, int value_format, float *out, int64_t tokens,
                             int q_heads, int kv_heads, int head_dim) {
    g_error.clear();
    if (!ctx) return fail("null context");
    if (int rc = frames_validate(key_format, value_format, tokens, q_heads, kv_heads, head_dim)) return rc;
    if (!query || !out || (tokens > 0 && (!keys || !values)))
        return fail("frames decode needs non-null query, out and (for tokens > 0) keys, values");
    if ((const void *)out == (const void *)query || (const void *)out == keys ||
        (const void *)out == values)
        return fail("frames decode output must not alias read-only query/keys/values");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    mslim::FramesLaunch l{};
    l.q = query; l.k = keys; l.v = values; l.out = out;
    l.key_format = key_format; l.value_format = value_format;
    l.tokens = tokens; l.q_heads = q_heads; l.kv_heads = kv_heads; l.head_dim = head_dim;
    uint64_t scratch = 0;
    return frames_enqueue(c, l, &scratch);
}

int mslim_attn_backend_decode(void *ctx, const float *query, const void *keys, int key_format,
                              const void *values, int value_format, int64_t tokens, int q_heads,
                              int kv_heads, int head_dim, float *out,
                              mslim_attn_timings *timings) {
    g_error.clear();
    const auto start = std::chrono::steady_clock::now();
    if (!ctx) return fail("null context");
    if (int rc = frames_validate(key_format, value_format, tokens, q_heads, kv_heads, head_dim)) return rc;
    if (!query || !out || (tokens > 0 && (!keys || !values)))
        return fail("backend decode needs host query, out and (for tokens > 0) keys, values");
    const size_t qn = (size_t)q_heads * head_dim;
    // gpu_backend.rs:154-159: the query is checked before the empty-cache case.
    for (size_t i = 0; i < qn; ++i)
        if (!std::isfinite(query[i])) return fail("non-finite computation: GPU Q", MSLIM_ATTN_ERR_NONFINITE);
    if (tokens == 0) {
        std::fill(out, out + qn, 0.0f);
        return 0;
    }
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    const size_t row = (size_t)kv_heads * head_dim;
    const size_t kb = (size_t)tokens * row * format_bytes(key_format);
    const size_t vb = (size_t)tokens * row * format_bytes(value_format);
    const size_t q_off = 0, k_off = align256(qn * 4), v_off = k_off + align256(kb);
    const size_t o_off = v_off + align256(vb), total = o_off + align256(qn * 4);
    if (int rc = grow_device(c, &c.backend, &c.backend_bytes, total, "hipMalloc backend buffers")) return rc;
    if (!c.ev_start) {
        if (int rc = check_hip(hipEventCreate(&c.ev_start), "hipEventCreate")) return rc;
        if (int rc = check_hip(hipEventCreate(&c.ev_end), "hipEventCreate")) return rc;
    }
    char *base = static_cast<char *>(c.backend);
    if (int rc = check_hip(hipMemcpyAsync(base + q_off, query, qn * 4, hipMemcpyHostToDevice, c.stream), "write Q"))
        return rc;
    if (int rc = check_hip(hipMemcpyAsync(base + k_off, keys, kb, hipMemcpyHostToDevice, c.stream), "write K"))
        return rc;
    if (int rc = check_hip(hipMemcpyAsync(base + v_off, values, vb, hipMemcpyHostToDevice, c.stream), "write V"))
        return rc;
    mslim::FramesLaunch l{};
    l.q = reinterpret_cast<const float *>(base + q_off);
    l.k = base + k_off; l.v = base + v_off;
    l.out = reinterpret_cast<float *>(base + o_off);
    l.key_format = key_format; l.value_format = value_format;
    l.tokens = tokens; l.q_heads = q_heads; l.kv_heads = kv_heads; l.head_dim = head_dim;
    uint64_t scratch = 0;
    if (int rc = check_hip(hipEventRecord(c.ev_start, c.stream), "hipEventRecord")) return rc;
    if (int rc = frames_enqueue(c, l, &scratch)) return rc;
    if (int rc = check_hip(hipEventRecord(c.ev_end, c.stream), "hipEventRecord")) return rc;
    if (int rc = check_hip(hipMemcpyAsync(out, l.out, qn * 4, hipMemcpyDeviceToHost, c.stream), "GPU output readback"))
        return rc;
    if (int rc = check_hip(hipStreamSynchronize(c.stream), "finish GPU")) return rc;
    float kernel_ms = 0.0f;
    if (int rc = check_hip(hipEventElapsedTime(&kernel_ms, c.ev_start, c.ev_end), "hipEventElapsedTime")) return rc;
    if (timings) {
        timings->dispatch_ms =
            std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - start).count();
        timings->kernel_ms = kernel_ms;
        timings->input_kv_bytes = kb + vb;
        timings->scratch_bytes = scratch;
        timings->output_bytes = qn * 4;
    }
    for (size_t i = 0; i < qn; ++i)
        if (!std::isfinite(out[i])) return fail("non-finite computation: GPU output", MSLIM_ATTN_ERR_NONFINITE);
    return 0;
}

int mslim_attn_rmsnorm(void *ctx, const void *input, const void *weight, void *output, int tokens,
                       int hidden, float epsilon) {
    g_error.clear();
    if (!ctx || !input || !weight || !output || tokens < 1 || hidden < 1 || !std::isfinite(epsilon) ||
        epsilon < 0.0f)
        return fail("invalid RMSNorm arguments");
    if (output == input || output == weight) return fail("RMSNorm output must not alias its inputs");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    return check_hip(mslim::launch_rmsnorm(static_cast<const uint16_t *>(input),
                                           static_cast<const uint16_t *>(weight),
                                           static_cast<uint16_t *>(output), tokens, hidden, epsilon,
                                           c.stream),
                     "RMSNorm launch");
}

// The context's RoPE cos/sin table for this configuration, covering at
// least min(need, the size limit) positions: built (or rebuilt for another
// configuration) on the context stream, behind any RoPE work already queued.
// A table the size limit or the device memory does not allow is simply not
// used: the kernels compute those positions themselves, with the same bits.
constexpr size_t kRopeTableMaxBytes = (size_t)32 << 20;
constexpr int64_t kRopeTableMinPositions = 8192;

static mslim::RopeCosSin rope_cossin(Context &c, int head_dim, float theta, int llama3, float factor, float low,
                                     float high, float original_max, int64_t need) {
    if (head_dim > 512 || head_dim % 2) return {};
    const float key[6] = {(float)head_dim, theta, (float)llama3, llama3 ? factor : 0.0f, llama3 ? low : 0.0f,
                          llama3 ? high : 0.0f};
    const float key_max = llama3 ? original_max : 0.0f;
    const bool same = std::memcmp(key, c.rope_key, sizeof key) == 0 &&
                      std::memcmp(&key_max, &c.rope_key_max, sizeof key_max) == 0 && c.rope_rows;
    const size_t row_bytes = (size_t)head_dim * 2;  // c and s of head_dim / 2 pairs
    const int64_t limit = (int64_t)(kRopeTableMaxBytes / row_bytes);
    int64_t want = std::min(limit, std::max(need, kRopeTableMinPositions));
    want = std::min(limit, (want + 4095) / 4096 * 4096);
    if (same && c.rope_positions >= std::min(want, std::max(need, (int64_t)1))) return {c.rope_rows, c.rope_positions};
    if (same) want = std::max(want, c.rope_positions);
    const size_t bytes = (size_t)want * row_bytes;
    if (bytes > c.rope_bytes) {
        // work queued on the stream may still read the old table
        if (c.rope_rows) {
            if (hipStreamSynchronize(c.stream) != hipSuccess || hipFree(c.rope_rows) != hipSuccess) {
                (void)hipGetLastError();
                c.rope_rows = nullptr;
                c.rope_bytes = 0;
                c.rope_positions = 0;
                return {};
            }
        }
        c.rope_rows = nullptr;
        c.rope_bytes = 0;
        c.rope_positions = 0;
        if (hipMalloc(reinterpret_cast<void **>(&c.rope_rows), bytes) != hipSuccess) {
            (void)hipGetLastError();
            c.rope_rows = nullptr;
            return {};
        }
        c.rope_bytes = bytes;
    }
    if (mslim::launch_rope_cossin(c.rope_rows, want, head_dim, theta, llama3, factor, low, high, original_max,
                                  c.stream) != hipSuccess) {
        (void)hipGetLastError();
        c.rope_positions = 0;
        return {};
    }
    std::memcpy(c.rope_key, key, sizeof key);
    c.rope_key_max = key_max;
    c.rope_positions = want;
    return {c.rope_rows, c.rope_positions};
}

int mslim_attn_rope(void *ctx, const void *input, void *output, int tokens, int heads, int head_dim,
                    int start_position, float theta, int llama3_scaling, float factor,
                    float low_freq_factor, float high_freq_factor, float original_max_position) {
    g_error.clear();
    if (!ctx || !input || !output || tokens < 1 || heads < 1 || head_dim < 2 || head_dim % 2 ||
        start_position < 0 || !(theta > 0.0f) || !std::isfinite(theta))
        return fail("invalid RoPE arguments");
    if (output == input) return fail("RoPE output must not alias its input");
    if (llama3_scaling && (!(factor > 0.0f) || !(high_freq_factor > low_freq_factor) ||
                           !(low_freq_factor > 0.0f) || !(original_max_position > 0.0f)))
        return fail("invalid llama3 RoPE scaling parameters");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    const mslim::RopeCosSin table = rope_cossin(c, head_dim, theta, llama3_scaling, factor, low_freq_factor,
                                                high_freq_factor, original_max_position,
                                                (int64_t)start_position + tokens);
    // The Q + K kernel with no K rows: the same bits, several rows per
    // workgroup.
    if (mslim::rope_qk_supported(head_dim, heads, input, output, input, output))
        return check_hip(mslim::launch_rope_qk(static_cast<const uint16_t *>(input), static_cast<uint16_t *>(output),
                                               nullptr, nullptr, tokens, heads, 0, head_dim, start_position, theta,
                                               llama3_scaling, factor, low_freq_factor, high_freq_factor,
                                               original_max_position, table, c.stream),
                         "RoPE launch");
    return check_hip(mslim::launch_rope(static_cast<const uint16_t *>(input),
                                        static_cast<uint16_t *>(output), tokens, heads, head_dim,
                                        start_position, nullptr, theta, llama3_scaling, factor,
                                        low_freq_factor, high_freq_factor, original_max_position, table,
                                        c.stream),
                     "RoPE launch");
}

int mslim_attn_rope_qk(void *ctx, const void *q, void *q_out, const void *k, void *k_out, int tokens, int q_heads,
                       int kv_heads, int head_dim, int start_position, float theta, int llama3_scaling, float factor,
                       float low_freq_factor, float high_freq_factor, float original_max_position) {
    g_error.clear();
    if (!ctx || !q || !q_out || !k || !k_out || tokens < 1 || q_heads < 1 || kv_heads < 1 || head_dim < 2 ||
        head_dim % 2 || start_position < 0 || !(theta > 0.0f) || !std::isfinite(theta))
        return fail("invalid RoPE arguments");
    if (q_out == q || q_out == k || k_out == q || k_out == k || q_out == k_out)
        return fail("RoPE outputs must not alias the inputs or each other");
    if (llama3_scaling && (!(factor > 0.0f) || !(high_freq_factor > low_freq_factor) ||
                           !(low_freq_factor > 0.0f) || !(original_max_position > 0.0f)))
        return fail("invalid llama3 RoPE scaling parameters");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    const auto *qi = static_cast<const uint16_t *>(q), *ki = static_cast<const uint16_t *>(k);
    auto *qo = static_cast<uint16_t *>(q_out), *ko = static_cast<uint16_t *>(k_out);
    const mslim::RopeCosSin table = rope_cossin(c, head_dim, theta, llama3_scaling, factor, low_freq_factor,
                                                high_freq_factor, original_max_position,
                                                (int64_t)start_position + tokens);
    if (mslim::rope_qk_supported(head_dim, q_heads + kv_heads, q, q_out, k, k_out))
        return check_hip(mslim::launch_rope_qk(qi, qo, ki, ko, tokens, q_heads, kv_heads, head_dim, start_position,
                                               theta, llama3_scaling, factor, low_freq_factor, high_freq_factor,
                                               original_max_position, table, c.stream),
                         "RoPE launch");
    if (int rc = check_hip(mslim::launch_rope(qi, qo, tokens, q_heads, head_dim, start_position, nullptr, theta,
                                              llama3_scaling, factor, low_freq_factor, high_freq_factor,
                                              original_max_position, table, c.stream),
                           "RoPE launch"))
        return rc;
    return check_hip(mslim::launch_rope(ki, ko, tokens, kv_heads, head_dim, start_position, nullptr, theta,
                                        llama3_scaling, factor, low_freq_factor, high_freq_factor,
                                        original_max_position, table, c.stream),
                     "RoPE launch");
}

int mslim_attn_rope_rows(void *ctx, const void *input, void *output, int tokens, int heads, int head_dim,
                         const int32_t *positions, float theta, int llama3_scaling, float factor,
                         float low_freq_factor, float high_freq_factor, float original_max_position) {
    g_error.clear();
    if (!ctx || !input || !output || !positions || tokens < 1 || heads < 1 || head_dim < 2 ||
        head_dim % 2 || !(theta > 0.0f) || !std::isfinite(theta))
        return fail("invalid RoPE arguments");
    if (output == input) return fail("RoPE output must not alias its input");
    if (llama3_scaling && (!(factor > 0.0f) || !(high_freq_factor > low_freq_factor) ||
                           !(low_freq_factor > 0.0f) || !(original_max_position > 0.0f)))
        return fail("invalid llama3 RoPE scaling parameters");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    // positions live on the device: the table covers what it covers
    const mslim::RopeCosSin table = rope_cossin(c, head_dim, theta, llama3_scaling, factor, low_freq_factor,
                                                high_freq_factor, original_max_position, 0);
    return check_hip(mslim::launch_rope(static_cast<const uint16_t *>(input),
                                        static_cast<uint16_t *>(output), tokens, heads, head_dim, 0,
                                        positions, theta, llama3_scaling, factor, low_freq_factor,
                                        high_freq_factor, original_max_position, table, c.stream),
                     "RoPE launch");
}

int mslim_attn_swiglu(void *ctx, const void *gate, const void *up, void *output, size_t n) {
    g_error.clear();
    if (!ctx || !gate || !up || !output || !n) return fail("invalid SwiGLU arguments");
    if (output == gate || output == up) return fail("SwiGLU output must not alias its inputs");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    return check_hip(mslim::launch_swiglu(static_cast<const uint16_t *>(gate),
                                          static_cast<const uint16_t *>(up),
                                          static_cast<uint16_t *>(output), n, c.stream),
                     "SwiGLU launch");
}

int mslim_attn_add(void *ctx, const void *a, const void *b, void *output, size_t n) {
    g_error.clear();
    if (!ctx || !a || !b || !output || !n) return fail("invalid residual add arguments");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    return check_hip(mslim::launch_add(static_cast<const uint16_t *>(a), static_cast<const uint16_t *>(b),
                                       static_cast<uint16_t *>(output), n, c.stream),
                     "residual add launch");
}

int mslim_attn_embed(void *ctx, const void *table, int vocab, int hidden, const int32_t *ids, int tokens,
                     void *output, int *bad) {
    g_error.clear();
    if (!ctx || !table || !ids || !output || vocab < 1 || hidden < 8 || hidden % 8 || tokens < 1)
        return fail("invalid embedding arguments (hidden must be a positive multiple of 8)");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    return check_hip(mslim::launch_embed(static_cast<const uint16_t *>(table), ids, tokens, hidden, vocab,
                                         static_cast<uint16_t *>(output), bad, c.stream),
                     "embedding launch");
}

int mslim_attn_argmax(void *ctx, const void *logits, int rows, int vocab, int32_t *out) {
    g_error.clear();
    if (!ctx || !logits || !out || rows < 1 || vocab < 1) return fail("invalid argmax arguments");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    return check_hip(mslim::launch_argmax(static_cast<const uint16_t *>(logits), rows, vocab, out, c.stream),
                     "argmax launch");
}

int mslim_attn_pages_write(void *ctx, void *k_pool, void *v_pool, const int32_t *page_table,
                           int page_tokens, int kv_heads, int head_dim, int64_t first_token,
                           int64_t tokens, const void *k_rows, const void *v_rows) {
    g_error.clear();
    if (!ctx || !k_pool || !v_pool || !page_table || !k_rows || !v_rows || tokens < 1 ||
        first_token < 0 || kv_heads < 1 || head_dim < 8 || head_dim % 8 || !is_pow2(page_tokens) ||
        page_tokens > (1 << 20))
        return fail("invalid page write arguments");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    return check_hip(mslim::launch_pages_write(
                         static_cast<uint16_t *>(k_pool), static_cast<uint16_t *>(v_pool), page_table,
                         page_tokens, kv_heads, head_dim, first_token, tokens,
                         static_cast<const uint16_t *>(k_rows), static_cast<const uint16_t *>(v_rows),
                         c.stream),
                     "page write launch");
}

int mslim_attn_pages_append(void *ctx, void *k_pool, void *v_pool, const int32_t *page_table,
                            int pages_per_seq, int page_tokens, int kv_heads, int head_dim, int batch,
                            const int32_t *positions, const void *k_rows, const void *v_rows) {
    g_error.clear();
    if (!ctx || !k_pool || !v_pool || !page_table || !positions || !k_rows || !v_rows || batch < 1 ||
        pages_per_seq < 1 || kv_heads < 1 || head_dim < 8 || head_dim % 8 || !is_pow2(page_tokens) ||
        page_tokens > (1 << 20))
        return fail("invalid page append arguments");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    return check_hip(mslim::launch_pages_append(
                         static_cast<uint16_t *>(k_pool), static_cast<uint16_t *>(v_pool), page_table,
                         pages_per_seq, page_tokens, kv_heads, head_dim, batch, positions,
                         static_cast<const uint16_t *>(k_rows), static_cast<const uint16_t *>(v_rows),
                         c.stream),
                     "page append launch");
}

// RoPE of Q and K and the append of K and V on a context already locked,
// arguments checked.
static int rope_append_locked(Context &c, const void *q, const void *k, const void *v, void *q_out, void *k_pool,
                              void *v_pool, const int32_t *page_table, int pages_per_seq, int page_tokens, int batch,
                              const int32_t *positions, int q_heads, int kv_heads, int head_dim, float theta,
                              int llama3_scaling, float factor, float low_freq_factor, float high_freq_factor,
                              float original_max_position) {
    mslim::RopeAppendArgs a{};
    a.q = static_cast<const uint16_t *>(q);
    a.k = static_cast<const uint16_t *>(k);
    a.v = static_cast<const uint16_t *>(v);
    a.q_out = static_cast<uint16_t *>(q_out);
    a.k_pool = static_cast<uint16_t *>(k_pool);
    a.v_pool = static_cast<uint16_t *>(v_pool);
    a.page_table = page_table;
    a.positions = positions;
    a.pages_per_seq = pages_per_seq;
    a.shift = 0;
    while ((1 << a.shift) < page_tokens) ++a.shift;
    a.batch = batch;
    a.q_heads = q_heads;
    a.kv_heads = kv_heads;
    a.head_dim = head_dim;
    a.theta = theta;
    a.llama3 = llama3_scaling;
    a.factor = factor;
    a.low = low_freq_factor;
    a.high = high_freq_factor;
    a.original_max = original_max_position;
    // every position the page table can hold
    a.cossin = rope_cossin(c, head_dim, theta, llama3_scaling, factor, low_freq_factor, high_freq_factor,
                           original_max_position, (int64_t)pages_per_seq << a.shift);
    return check_hip(mslim::launch_rope_append(a, c.stream), "RoPE append launch");
}

int mslim_attn_rope_append(void *ctx, const void *q, const void *k, const void *v, void *q_out, void *k_pool,
                           void *v_pool, const int32_t *page_table, int pages_per_seq, int page_tokens, int batch,
                           const int32_t *positions, int q_heads, int kv_heads, int head_dim, float theta,
                           int llama3_scaling, float factor, float low_freq_factor, float high_freq_factor,
                           float original_max_position) {
    g_error.clear();
    if (!ctx || !q || !k || !v || !q_out || !k_pool || !v_pool || !page_table || !positions || batch < 1 ||
        pages_per_seq < 1 || q_heads < 1 || kv_heads < 1 || head_dim < 8 || head_dim % 8 || head_dim > 512 ||
        !is_pow2(page_tokens) || page_tokens > (1 << 20) || !(theta > 0.0f) || !std::isfinite(theta))
        return fail("invalid RoPE append arguments");
    if (q_out == q) return fail("RoPE output must not alias its input");
    if (llama3_scaling && (!(factor > 0.0f) || !(high_freq_factor > low_freq_factor) ||
                           !(low_freq_factor > 0.0f) || !(original_max_position > 0.0f)))
        return fail("invalid llama3 RoPE scaling parameters");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    return rope_append_locked(c, q, k, v, q_out, k_pool, v_pool, page_table, pages_per_seq, page_tokens, batch,
                              positions, q_heads, kv_heads, head_dim, theta, llama3_scaling, factor, low_freq_factor,
                              high_freq_factor, original_max_position);
}

int mslim_attn_pages_gather(void *ctx, const void *pool, const int32_t *page_table, int page_tokens,
                            int kv_heads, int head_dim, int64_t first_token, int64_t tokens,
                            void *rows_out) {
    g_error.clear();
    if (!ctx || !pool || !page_table || !rows_out || tokens < 1 || first_token < 0 || kv_heads < 1 ||
        head_dim < 8 || head_dim % 8 || !is_pow2(page_tokens) || page_tokens > (1 << 20))
        return fail("invalid page gather arguments");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    return check_hip(mslim::launch_pages_gather(static_cast<const uint16_t *>(pool), page_table,
                                                page_tokens, kv_heads, head_dim, first_token, tokens,
                                                static_cast<uint16_t *>(rows_out), c.stream),
                     "page gather launch");
}

int mslim_attn_logical_kv_sha256(void *ctx, int layers, int64_t tokens, int kv_heads, int head_dim,
                                 const void *const *keys, const void *const *values,
                                 const int32_t *const *page_tables, int page_tokens,
                                 char *hex_out) {
    g_error.clear();
    if (!ctx || layers < 1 || tokens < 0 || kv_heads < 1 || head_dim < 8 || head_dim % 8 || !keys ||
        !values || !hex_out)
        return fail("invalid logical K/V digest arguments");
    if (page_tables && (!is_pow2(page_tokens) || page_tokens > (1 << 20)))
        return fail("paged digest needs page_tokens a power of two");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    mslim::Sha256 sha;
    static const char tag[] = "mslim-dense-kv-state-v1";
    sha.update(tag, sizeof tag - 1);
    uint8_t le[8];
    for (int i = 0; i < 8; ++i) le[i] = (uint8_t)((uint64_t)tokens >> (8 * i));
    sha.update(le, 8);
    const int64_t chunk_tokens = std::max<int64_t>(1, std::min<int64_t>(tokens, (int64_t)1 << 16));
    const size_t chunk_bytes = (size_t)chunk_tokens * head_dim * 2;
    if (tokens > 0) {
        if (int rc = grow_device(c, &c.staging, &c.staging_bytes, chunk_bytes, "hipMalloc digest staging"))
            return rc;
        if (int rc = grow_host(&c.host_staging, &c.host_staging_bytes, chunk_bytes,
                               "hipHostMalloc digest staging"))
            return rc;
    }
    for (int layer = 0; layer < layers && tokens > 0; ++layer) {
        const void *parts[2] = {keys[layer], values[layer]};
        const int32_t *table = page_tables ? page_tables[layer] : nullptr;
        if (!parts[0] || !parts[1] || (page_tables && !table))
            return fail("logical K/V digest: null layer buffer");
        for (int p = 0; p < 2; ++p)
            for (int h = 0; h < kv_heads; ++h)
                for (int64_t t0 = 0; t0 < tokens; t0 += chunk_tokens) {
                    const int64_t n = std::min(chunk_tokens, tokens - t0);
                    if (int rc = check_hip(mslim::launch_canonical_rows(
                                               static_cast<const uint16_t *>(parts[p]), table, page_tokens,
                                               kv_heads, head_dim, h, t0, n,
                                               static_cast<uint16_t *>(c.staging), c.stream),
                                           "digest serialisation launch"))
                        return rc;
                    const size_t bytes = (size_t)n * head_dim * 2;
                    if (int rc = check_hip(hipMemcpyAsync(c.host_staging, c.staging, bytes,
                                                          hipMemcpyDeviceToHost, c.stream),
                                           "digest readback"))
                        return rc;
                    if (int rc = check_hip(hipStreamSynchronize(c.stream), "digest readback sync"))
                        return rc;
                    sha.update(c.host_staging, bytes);
                }
    }
    uint8_t digest[32];
    sha.finish(digest);
    static const char hexd[] = "0123456789abcdef";
    for (int i = 0; i < 32; ++i) {
        hex_out[2 * i] = hexd[digest[i] >> 4];
        hex_out[2 * i + 1] = hexd[digest[i] & 15];
    }
    hex_out[64] = '\0';
    return 0;
}


int64_t mslim_attn_record_frame_bytes(int page_tokens) {
    return page_tokens >= 1 ? mslim::record_frame_bytes(page_tokens) : -1;
}

int mslim_attn_record_frames(void *ctx, const void *k_pool, const void *v_pool, int64_t pool_pages,
                             int page_tokens, int kv_heads, int head_dim, uint32_t tile,
                             const mslim_attn_page_record *records, int count, void *frames) {
    g_error.clear();
    if (!ctx || !k_pool || !v_pool || !records || !frames || count < 0 || pool_pages < 1)
        return fail("invalid record frame arguments");
    if (!is_pow2(page_tokens) || page_tokens > 512 || kv_heads < 1 || head_dim < 8 || head_dim % 8)
        return fail("record frames need page_tokens a power of two <= 512, kv_heads >= 1 and "
                    "head_dim a multiple of 8");
    if (tile == 0 || (uint32_t)head_dim % tile) return fail("head_dim is not a multiple of tile");
    if ((uintptr_t)k_pool % 16 || (uintptr_t)v_pool % 16 || (uintptr_t)frames % 8)
        return fail("record frames need 16-byte aligned pools and an 8-byte aligned frame buffer");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    mslim::FramesCodecLaunch l;
    l.k_pool = k_pool;
    l.v_pool = v_pool;
    l.pool_pages = pool_pages;
    l.page_tokens = page_tokens;
    l.kv_heads = kv_heads;
    l.head_dim = head_dim;
    l.tile = tile;
    l.records = reinterpret_cast<const mslim::RecordDesc *>(records);
    l.count = count;
    l.frames = frames;
    l.frame_bytes = mslim::record_frame_bytes(page_tokens);
    l.staged = false;
    return check_hip(mslim::launch_record_frames(l, c.stream), "record frame launch");
}

int mslim_attn_record_frames_staged(void *ctx, const void *k_stage, const void *v_stage, int page_tokens,
                                    int kv_heads, int head_dim, uint32_t tile,
                                    const mslim_attn_page_record *records, int count, void *frames) {
    g_error.clear();
    if (!ctx || !k_stage || !v_stage || !records || !frames || count < 0)
        return fail("invalid staged record frame arguments");
    if (!is_pow2(page_tokens) || page_tokens > 512 || kv_heads < 1 || head_dim < 8 || head_dim % 8)
        return fail("record frames need page_tokens a power of two <= 512, kv_heads >= 1 and "
                    "head_dim a multiple of 8");
    if (tile == 0 || (uint32_t)head_dim % tile) return fail("head_dim is not a multiple of tile");
    if ((uintptr_t)k_stage % 16 || (uintptr_t)v_stage % 16 || (uintptr_t)frames % 8)
        return fail("record frames need 16-byte aligned staging and an 8-byte aligned frame buffer");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    mslim::FramesCodecLaunch l;
    l.k_pool = k_stage;
    l.v_pool = v_stage;
    l.pool_pages = count;
    l.page_tokens = page_tokens;
    l.kv_heads = kv_heads;
    l.head_dim = head_dim;
    l.tile = tile;
    l.records = reinterpret_cast<const mslim::RecordDesc *>(records);
    l.count = count;
    l.frames = frames;
    l.frame_bytes = mslim::record_frame_bytes(page_tokens);
    l.staged = true;
    return check_hip(mslim::launch_record_frames(l, c.stream), "staged record frame launch");
}

void *mslim_attn_host_alloc(void *ctx, size_t bytes) {
    g_error.clear();
    if (!ctx || !bytes) {
        g_error = "invalid pinned host allocation";
        return nullptr;
    }
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    void *p = nullptr;
    if (check_hip(hipHostMalloc(&p, bytes, hipHostMallocDefault), "hipHostMalloc staging")) return nullptr;
    return p;
}

int mslim_attn_host_free(void *ctx, void *host) {
    g_error.clear();
    if (!ctx || !host) return fail("invalid pinned host buffer");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    if (int rc = check_hip(hipStreamSynchronize(c.stream), "hipStreamSynchronize before host free")) return rc;
    return check_hip(hipHostFree(host), "hipHostFree staging");
}

int mslim_attn_record_payloads(void *ctx, void *k_pool, void *v_pool, int64_t pool_pages, int page_tokens,
                               int kv_heads, int head_dim, const mslim_attn_page_record *records, int count,
                               void *k_stage, void *v_stage, int direction) {
    g_error.clear();
    if (!ctx || !k_pool || !v_pool || !records || !k_stage || !v_stage || count < 0 || pool_pages < 1 ||
        (direction != 0 && direction != 1))
        return fail("invalid record payload arguments");
    if (!is_pow2(page_tokens) || page_tokens > 512 || kv_heads < 1 || head_dim < 8 || head_dim % 8)
        return fail("record payloads need page_tokens a power of two <= 512, kv_heads >= 1 and "
                    "head_dim a multiple of 8");
    if ((uintptr_t)k_pool % 16 || (uintptr_t)v_pool % 16 || (uintptr_t)k_stage % 16 || (uintptr_t)v_stage % 16)
        return fail("record payloads need 16-byte aligned pools and staging");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    mslim::PayloadMoveLaunch l;
    l.k_pool = k_pool;
    l.v_pool = v_pool;
    l.pool_pages = pool_pages;
    l.page_tokens = page_tokens;
    l.kv_heads = kv_heads;
    l.head_dim = head_dim;
    l.records = reinterpret_cast<const mslim::RecordDesc *>(records);
    l.count = count;
    l.k_stage = k_stage;
    l.v_stage = v_stage;
    return check_hip(mslim::launch_record_payloads(l, direction == 0, c.stream), "record payload launch");
}

// The fp32 partials of a split projection (none for other shapes), in a
// context buffer that only grows (stage code 400 if it cannot).
// `outputs`: products x the matrices' total rows (2 x rows for SwiGLU).
static int proj_partials(Context &c, int inner, int64_t outputs, int tokens, float **partial) {
    *partial = nullptr;
    const int split = mslim::proj_ksplit(inner);
    if (split < 2) return 0;
    if (grow_device(c, &c.proj_partial, &c.proj_partial_bytes, (size_t)split * outputs * tokens * sizeof(float),
                    "hipMalloc projection partials"))
        return 400;
    *partial = static_cast<float *>(c.proj_partial);
    return 0;
}

// One product on the context's stream: the MFMA decode kernel for up to 16
// aligned tokens, the tiled MFMA kernel (or its any-shape form) above.  A
// failed launch is stage code 404, as the reference's matmul stage.
static int project(Context &c, const void *weight, const void *input, void *output, int inner, int rows,
                   int tokens) {
    const mslim::SkinnyMatrix m{static_cast<const uint16_t *>(weight), static_cast<uint16_t *>(output), rows};
    const auto *x = static_cast<const uint16_t *>(input);
    if (mslim::skinny_supported(inner, tokens, input, weight))
        return check_hip(mslim::launch_skinny_gemm(&m, 1, x, inner, tokens, c.stream), "decode projection launch")
                   ? 404
                   : 0;
    float *partial = nullptr;
    if (int rc = proj_partials(c, inner, rows, tokens, &partial)) return rc;
    return check_hip(mslim::launch_proj(&m, 1, x, inner, tokens, partial, c.stream), "projection launch") ? 404 : 0;
}

// tv_hip_matrix_multiply's argument limits (hipblaslt_bridge.cpp:207-210).
static bool gemm_args_ok(const void *ctx, const void *w, const void *in, const void *out, int inner, int rows,
                         int tokens) {
    return ctx && w && in && out && inner > 0 && rows > 0 && tokens > 0 && tokens <= 512 && inner <= 32768 &&
           rows <= 500000;
}

int mslim_attn_matrix_multiply(void *ctx, const void *weight, const uint8_t *input, uint8_t *output, int inner,
                               int rows, int tokens) {
    g_error.clear();
    if (!gemm_args_ok(ctx, weight, input, output, inner, rows, tokens))
        return fail("invalid BF16 matrix dimensions/arguments");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    const size_t insize = (size_t)inner * tokens * 2, outsize = (size_t)rows * tokens * 2;
    if (grow_device(c, &c.gemm_in, &c.gemm_in_bytes, insize, "hipMalloc BF16 input")) return 400;
    if (grow_device(c, &c.gemm_out, &c.gemm_out_bytes, outsize, "hipMalloc BF16 output")) return 401;
    if (check_hip(hipMemcpyAsync(c.gemm_in, input, insize, hipMemcpyHostToDevice, c.stream), "BF16 matrix input H2D"))
        return 402;
    if (int rc = project(c, weight, c.gemm_in, c.gemm_out, inner, rows, tokens)) return rc;
    if (check_hip(hipMemcpyAsync(output, c.gemm_out, outsize, hipMemcpyDeviceToHost, c.stream),
                  "BF16 matrix output D2H"))
        return 405;
    return check_hip(hipStreamSynchronize(c.stream), "BF16 matrix output D2H") ? 405 : 0;
}

int mslim_attn_gemm_bf16(void *ctx, const void *weight, const void *input, void *output, int inner, int rows,
                         int tokens) {
    g_error.clear();
    if (!gemm_args_ok(ctx, weight, input, output, inner, rows, tokens))
        return fail("invalid BF16 matrix dimensions/arguments");
    if (output == input || output == weight) return fail("GEMM output must not alias its inputs");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    return project(c, weight, input, output, inner, rows, tokens);
}

int mslim_attn_gemm_bf16_add(void *ctx, const void *weight, const void *input, const void *residual,
                             void *output, int inner, int rows, int tokens) {
    g_error.clear();
    if (!gemm_args_ok(ctx, weight, input, output, inner, rows, tokens) || !residual)
        return fail("invalid BF16 matrix dimensions/arguments");
    if (output == input || output == weight || residual == input)
        return fail("GEMM output must not alias its inputs");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    const auto *w = static_cast<const uint16_t *>(weight);
    const auto *x = static_cast<const uint16_t *>(input);
    if (mslim::skinny_supported(inner, tokens, input, weight)) {
        const mslim::SkinnyMatrix m{w, static_cast<uint16_t *>(output), rows};
        return check_hip(mslim::launch_skinny_gemm_add(m, static_cast<const uint16_t *>(residual), x, inner,
                                                       tokens, c.stream),
                         "decode projection launch")
                   ? 404
                   : 0;
    }
    const mslim::SkinnyMatrix m{w, static_cast<uint16_t *>(output), rows};
    float *partial = nullptr;
    if (int rc = proj_partials(c, inner, rows, tokens, &partial)) return rc;
    return check_hip(mslim::launch_proj_add(m, static_cast<const uint16_t *>(residual), x, inner, tokens, partial,
                                            c.stream),
                     "projection launch")
               ? 404
               : 0;
}

int mslim_attn_gemm_swiglu(void *ctx, const void *gate_weight, const void *up_weight, const void *input,
                           void *output, int inner, int rows, int tokens) {
    g_error.clear();
    if (!gemm_args_ok(ctx, gate_weight, input, output, inner, rows, tokens) || !up_weight)
        return fail("invalid BF16 matrix dimensions/arguments");
    if (output == input || output == gate_weight || output == up_weight)
        return fail("GEMM output must not alias its inputs");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    const auto *x = static_cast<const uint16_t *>(input);
    if (mslim::skinny_supported(inner, tokens, input, gate_weight, up_weight)) {
        return check_hip(mslim::launch_skinny_swiglu(static_cast<const uint16_t *>(gate_weight),
                                                     static_cast<const uint16_t *>(up_weight),
                                                     static_cast<uint16_t *>(output), rows, x, inner, tokens,
                                                     c.swiglu_table, c.stream),
                         "decode projection launch")
                   ? 404
                   : 0;
    }
    float *partial = nullptr;
    if (int rc = proj_partials(c, inner, 2 * (int64_t)rows, tokens, &partial)) return rc;
    return check_hip(mslim::launch_proj_swiglu(static_cast<const uint16_t *>(gate_weight),
                                               static_cast<const uint16_t *>(up_weight),
                                               static_cast<uint16_t *>(output), rows, x, inner, tokens,
                                               c.swiglu_table, partial, c.stream),
                     "projection launch")
               ? 404
               : 0;
}

int mslim_attn_gemm_qkv(void *ctx, const void *q_weight, const void *k_weight, const void *v_weight,
                        const void *input, void *q_out, void *k_out, void *v_out, int inner, int q_rows,
                        int kv_rows, int tokens) {
    g_error.clear();
    if (!gemm_args_ok(ctx, q_weight, input, q_out, inner, q_rows, tokens) ||
        !gemm_args_ok(ctx, k_weight, input, k_out, inner, kv_rows, tokens) ||
        !gemm_args_ok(ctx, v_weight, input, v_out, inner, kv_rows, tokens))
        return fail("invalid BF16 matrix dimensions/arguments");
    if (q_out == input || k_out == input || v_out == input) return fail("GEMM output must not alias its inputs");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    if (mslim::skinny_supported(inner, tokens, input, q_weight, k_weight, v_weight)) {
        const mslim::SkinnyMatrix m[3] = {
            {static_cast<const uint16_t *>(q_weight), static_cast<uint16_t *>(q_out), q_rows},
            {static_cast<const uint16_t *>(k_weight), static_cast<uint16_t *>(k_out), kv_rows},
            {static_cast<const uint16_t *>(v_weight), static_cast<uint16_t *>(v_out), kv_rows}};
        return check_hip(mslim::launch_skinny_gemm(m, 3, static_cast<const uint16_t *>(input), inner, tokens,
                                                   c.stream),
                         "decode projection launch")
                   ? 404
                   : 0;
    }
    const mslim::SkinnyMatrix m[3] = {
        {static_cast<const uint16_t *>(q_weight), static_cast<uint16_t *>(q_out), q_rows},
        {static_cast<const uint16_t *>(k_weight), static_cast<uint16_t *>(k_out), kv_rows},
        {static_cast<const uint16_t *>(v_weight), static_cast<uint16_t *>(v_out), kv_rows}};
    float *partial = nullptr;
    if (int rc = proj_partials(c, inner, (int64_t)q_rows + 2 * (int64_t)kv_rows, tokens, &partial)) return rc;
    return check_hip(mslim::launch_proj(m, 3, static_cast<const uint16_t *>(input), inner, tokens, partial, c.stream),
                     "projection launch")
               ? 404
               : 0;
}

// ---- RMSNorm + projections ----------------------------------------------

// The rows normalised into a context buffer (shapes the projection kernels do
// not normalise themselves): mslim_attn_rmsnorm's kernels.
static int normalise_rows(Context &c, const void *input, const void *norm_weight, float epsilon, int inner,
                          int tokens, const void **rows) {
    if (grow_device(c, &c.norm_rows, &c.norm_rows_bytes, (size_t)inner * tokens * 2, "hipMalloc normalised rows"))
        return 400;
    if (int rc = check_hip(mslim::launch_rmsnorm(static_cast<const uint16_t *>(input),
                                                 static_cast<const uint16_t *>(norm_weight),
                                                 static_cast<uint16_t *>(c.norm_rows), tokens, inner, epsilon,
                                                 c.stream),
                           "RMSNorm launch"))
        return rc;
    *rows = c.norm_rows;
    return 0;
}

static bool norm_args_ok(const void *norm_weight, float epsilon) {
    return norm_weight && std::isfinite(epsilon) && epsilon >= 0.0f;
}

int mslim_attn_rmsnorm_gemm_bf16(void *ctx, const void *norm_weight, float epsilon, const void *weight,
                                 const void *input, void *output, int inner, int rows, int tokens) {
    g_error.clear();
    if (!gemm_args_ok(ctx, weight, input, output, inner, rows, tokens) || !norm_args_ok(norm_weight, epsilon))
        return fail("invalid RMSNorm + BF16 matrix arguments");
    if (output == input || output == weight || output == norm_weight) return fail("GEMM output must not alias its inputs");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    if (mslim::skinny_supported(inner, tokens, input, weight) &&
        mslim::skinny_norm_supported(inner, tokens, norm_weight)) {
        const mslim::SkinnyMatrix m{static_cast<const uint16_t *>(weight), static_cast<uint16_t *>(output), rows};
        return check_hip(mslim::launch_skinny_gemm(&m, 1, static_cast<const uint16_t *>(input), inner, tokens,
                                                   c.stream, static_cast<const uint16_t *>(norm_weight), epsilon),
                         "decode projection launch")
                   ? 404
                   : 0;
    }
    const void *x = nullptr;
    if (int rc = normalise_rows(c, input, norm_weight, epsilon, inner, tokens, &x)) return rc;
    return project(c, weight, x, output, inner, rows, tokens);
}

// RMSNorm + QKV on a context already locked, arguments checked.
static int rmsnorm_gemm_qkv_locked(Context &c, const void *norm_weight, float epsilon, const void *q_weight,
                                   const void *k_weight, const void *v_weight, const void *input, void *q_out,
                                   void *k_out, void *v_out, int inner, int q_rows, int kv_rows, int tokens) {
    const mslim::SkinnyMatrix m[3] = {
        {static_cast<const uint16_t *>(q_weight), static_cast<uint16_t *>(q_out), q_rows},
        {static_cast<const uint16_t *>(k_weight), static_cast<uint16_t *>(k_out), kv_rows},
        {static_cast<const uint16_t *>(v_weight), static_cast<uint16_t *>(v_out), kv_rows}};
    if (mslim::skinny_supported(inner, tokens, input, q_weight, k_weight, v_weight) &&
        mslim::skinny_norm_supported(inner, tokens, norm_weight))
        return check_hip(mslim::launch_skinny_gemm(m, 3, static_cast<const uint16_t *>(input), inner, tokens,
                                                   c.stream, static_cast<const uint16_t *>(norm_weight), epsilon),
                         "decode projection launch")
                   ? 404
                   : 0;
    const void *x = nullptr;
    if (int rc = normalise_rows(c, input, norm_weight, epsilon, inner, tokens, &x)) return rc;
    if (mslim::skinny_supported(inner, tokens, x, q_weight, k_weight, v_weight))
        return check_hip(mslim::launch_skinny_gemm(m, 3, static_cast<const uint16_t *>(x), inner, tokens, c.stream),
                         "decode projection launch")
                   ? 404
                   : 0;
    float *partial = nullptr;
    if (int rc = proj_partials(c, inner, (int64_t)q_rows + 2 * (int64_t)kv_rows, tokens, &partial)) return rc;
    return check_hip(mslim::launch_proj(m, 3, static_cast<const uint16_t *>(x), inner, tokens, partial, c.stream),
                     "projection launch")
               ? 404
               : 0;
}

int mslim_attn_rmsnorm_gemm_qkv(void *ctx, const void *norm_weight, float epsilon, const void *q_weight,
                                const void *k_weight, const void *v_weight, const void *input, void *q_out,
                                void *k_out, void *v_out, int inner, int q_rows, int kv_rows, int tokens) {
    g_error.clear();
    if (!gemm_args_ok(ctx, q_weight, input, q_out, inner, q_rows, tokens) ||
        !gemm_args_ok(ctx, k_weight, input, k_out, inner, kv_rows, tokens) ||
        !gemm_args_ok(ctx, v_weight, input, v_out, inner, kv_rows, tokens) || !norm_args_ok(norm_weight, epsilon))
        return fail("invalid RMSNorm + BF16 matrix arguments");
    if (q_out == input || k_out == input || v_out == input) return fail("GEMM output must not alias its inputs");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    return rmsnorm_gemm_qkv_locked(c, norm_weight, epsilon, q_weight, k_weight, v_weight, input, q_out, k_out, v_out,
                                   inner, q_rows, kv_rows, tokens);
}

int mslim_attn_rmsnorm_gemm_swiglu(void *ctx, const void *norm_weight, float epsilon, const void *gate_weight,
                                   const void *up_weight, const void *input, void *output, int inner, int rows,
                                   int tokens) {
    g_error.clear();
    if (!gemm_args_ok(ctx, gate_weight, input, output, inner, rows, tokens) || !up_weight ||
        !norm_args_ok(norm_weight, epsilon))
        return fail("invalid RMSNorm + BF16 matrix arguments");
    if (output == input || output == gate_weight || output == up_weight)
        return fail("GEMM output must not alias its inputs");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    const auto *gw = static_cast<const uint16_t *>(gate_weight), *uw = static_cast<const uint16_t *>(up_weight);
    if (mslim::skinny_supported(inner, tokens, input, gate_weight, up_weight) &&
        mslim::skinny_norm_supported(inner, tokens, norm_weight))
        return check_hip(mslim::launch_skinny_swiglu(gw, uw, static_cast<uint16_t *>(output), rows,
                                                     static_cast<const uint16_t *>(input), inner, tokens,
                                                     c.swiglu_table, c.stream,
                                                     static_cast<const uint16_t *>(norm_weight), epsilon),
                         "decode projection launch")
                   ? 404
                   : 0;
    const void *x = nullptr;
    if (int rc = normalise_rows(c, input, norm_weight, epsilon, inner, tokens, &x)) return rc;
    if (mslim::skinny_supported(inner, tokens, x, gate_weight, up_weight))
        return check_hip(mslim::launch_skinny_swiglu(gw, uw, static_cast<uint16_t *>(output), rows,
                                                     static_cast<const uint16_t *>(x), inner, tokens,
                                                     c.swiglu_table, c.stream),
                         "decode projection launch")
                   ? 404
                   : 0;
    float *partial = nullptr;
    if (int rc = proj_partials(c, inner, 2 * (int64_t)rows, tokens, &partial)) return rc;
    return check_hip(mslim::launch_proj_swiglu(gw, uw, static_cast<uint16_t *>(output), rows,
                                               static_cast<const uint16_t *>(x), inner, tokens, c.swiglu_table,
                                               partial, c.stream),
                     "projection launch")
               ? 404
               : 0;
}

int mslim_attn_rmsnorm_qkv_rope_append(void *ctx, const void *norm_weight, float epsilon, const void *q_weight,
                                       const void *k_weight, const void *v_weight, const void *input, void *q_out,
                                       void *k_pool, void *v_pool, const int32_t *page_table, int pages_per_seq,
                                       int page_tokens, int batch, const int32_t *positions, int inner, int q_heads,
                                       int kv_heads, int head_dim, float theta, int llama3_scaling, float factor,
                                       float low_freq_factor, float high_freq_factor, float original_max_position) {
    g_error.clear();
    if (!ctx || !norm_args_ok(norm_weight, epsilon) || !q_weight || !k_weight || !v_weight || !input || !q_out ||
        !k_pool || !v_pool || !page_table || !positions || batch < 1 || batch > 512 || inner < 1 ||
        inner > 32768 || pages_per_seq < 1 || q_heads < 1 || kv_heads < 1 || head_dim < 8 || head_dim % 8 ||
        head_dim > 512 || (int64_t)q_heads * head_dim > 500000 || (int64_t)kv_heads * head_dim > 500000 ||
        !is_pow2(page_tokens) || page_tokens > (1 << 20) || !(theta > 0.0f) || !std::isfinite(theta))
        return fail("invalid RMSNorm + QKV + RoPE append arguments");
    const int q_rows = q_heads * head_dim, kv_rows = kv_heads * head_dim;
    if (llama3_scaling && (!(factor > 0.0f) || !(high_freq_factor > low_freq_factor) ||
                           !(low_freq_factor > 0.0f) || !(original_max_position > 0.0f)))
        return fail("invalid llama3 RoPE scaling parameters");
    if (q_out == input || q_out == k_pool || q_out == v_pool) return fail("Q output must not alias the inputs or pools");
    Context &c = *ctx_of(ctx);
    Lock lock(c);
    int shift = 0;
    while ((1 << shift) < page_tokens) ++shift;
    if (mslim::skinny_rope_supported(inner, batch, head_dim, input, q_weight, k_weight, v_weight, norm_weight)) {
        mslim::SkinnyRope r{};
        r.positions = positions;
        r.page_table = page_table;
        r.k_pool = static_cast<uint16_t *>(k_pool);
        r.v_pool = static_cast<uint16_t *>(v_pool);
        r.pages_per_seq = pages_per_seq;
        r.shift = shift;
        r.kv_heads = kv_heads;
        r.head_dim = head_dim;
        r.theta = theta;
        r.llama3 = llama3_scaling;
        r.factor = factor;
        r.low = low_freq_factor;
        r.high = high_freq_factor;
        r.original_max = original_max_position;
        r.cossin = rope_cossin(c, head_dim, theta, llama3_scaling, factor, low_freq_factor, high_freq_factor,
                               original_max_position, (int64_t)pages_per_seq << shift);
        const mslim::SkinnyMatrix m[3] = {
            {static_cast<const uint16_t *>(q_weight), static_cast<uint16_t *>(q_out), q_rows},
            {static_cast<const uint16_t *>(k_weight), nullptr, kv_rows},
            {static_cast<const uint16_t *>(v_weight), nullptr, kv_rows}};
        return check_hip(mslim::launch_skinny_qkv_rope(m, static_cast<const uint16_t *>(input), inner, batch,
                                                       static_cast<const uint16_t *>(norm_weight), epsilon, r,
                                                       c.stream),
                         "decode projection launch")
                   ? 404
                   : 0;
    }
    // Other shapes: the two operations, Q, K and V through a context buffer,
    // under the one lock (another call on the context may not regrow the
    // buffer in between).
    const size_t bytes = (size_t)batch * (q_rows + 2 * (size_t)kv_rows) * 2;
    if (grow_device(c, &c.qkv_rows, &c.qkv_rows_bytes, bytes, "hipMalloc QKV rows")) return 400;
    uint16_t *q = static_cast<uint16_t *>(c.qkv_rows);
    uint16_t *k = q + (size_t)batch * q_rows, *v = k + (size_t)batch * kv_rows;
    if (int rc = rmsnorm_gemm_qkv_locked(c, norm_weight, epsilon, q_weight, k_weight, v_weight, input, q, k, v, inner,
                                         q_rows, kv_rows, batch))
        return rc;
    return rope_append_locked(c, q, k, v, q_out, k_pool, v_pool, page_table, pages_per_seq, page_tokens, batch,
                              positions, q_heads, kv_heads, head_dim, theta, llama3_scaling, factor, low_freq_factor,
                              high_freq_factor, original_max_position);
}

}  // extern "C"
