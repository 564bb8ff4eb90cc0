/*
 * mslim_attn -- MI355X (gfx950) attention hot path of M-SLIM behind a C ABI.
 *
 * Drop-in boundary for the reference's native bridge (native_hip.rs:13-20,
 * :84-134; native/hipblaslt_bridge.cpp:155-233) and for the device launches
 * that gpu_backend.rs / gpu_llm/gpu_resources.rs / gpu_llm/prefill.rs /
 * gpu_llm/tiled_attention.rs issue today through OpenCL.  Plain pointers and
 * sizes only.
 *
 * Conventions (kept from hipblaslt_bridge.cpp:24-39):
 *   * every int-returning entry point returns 0 on success, -1 for invalid
 *     arguments, 100 + hipError_t for a HIP runtime failure and 400..409 for a
 *     failed stage; pointer-returning ones return NULL on failure;
 *   * the message of the last failure on the calling thread is returned by
 *     mslim_attn_last_error();
 *   * a context serialises its calls with its own mutex (hipblaslt_bridge.cpp
 *     :61, :179) and issues all device work in order on one HIP stream, the
 *     equivalent of the reference's single in-order OpenCL queue
 *     (gpu_resources.rs:122-123);
 *   * compute entry points are stream-ordered: they return after enqueueing.
 *     mslim_attn_synchronize() is the queue.finish() equivalent; the buffer
 *     read/write entry points block, like CL_BLOCKING transfers;
 *   * all tensors are BF16 bit patterns (uint16 little-endian) unless stated,
 *     device pointers, and the output must not alias any input
 *     (tiled_attention.rs:204-207).
 *
 * Layouts:
 *   Q        [batch][q_heads][head_dim]                 (decode)
 *            [queries][q_heads][head_dim]               (prefill)
 *   dense K/V token-major [tokens][kv_heads][head_dim] per sequence
 *            (gpu_llm.cl:148-149); sequence b starts at b * seq_stride_tokens
 *            tokens.
 *   paged K/V pool of pages [page][kv_heads][page_tokens][head_dim]: the
 *            head-major ColdStore page payload (cold_store.rs:480-483,
 *            gpu_region_store.rs:386-390); page_table[b][i] is the pool page
 *            holding tokens [i*page_tokens, (i+1)*page_tokens) of sequence b.
 *            The table is device memory and is not validated: every entry a
 *            call reaches must name a page of the pool, as the reference's
 *            region store guarantees for its own table
 *            (gpu_region_store.rs:113-116, :486-489).
 */
#ifndef MSLIM_ATTN_H
#define MSLIM_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Sequences per decode launch.  Launches of up to 64 sequences carry their
 * launch tables in the kernel arguments; larger ones copy the tables (16
 * bytes per sequence) host to device on the context stream before the
 * kernel, so they cannot be recorded into a graph, and the allocation-free
 * entry point takes at most 64. */
#define MSLIM_ATTN_MAX_BATCH 4096

/* ---- Context and errors -------------------------------------------------- */

/* Replaces tv_hip_last_error (hipblaslt_bridge.cpp:157-159, bound at
 * native_hip.rs:13,101).  Thread-local, never NULL. */
const char *mslim_attn_last_error(void);

/* Replaces tv_hip_new (hipblaslt_bridge.cpp:160-169, native_hip.rs:102,111).
 * Gate: device 0 must report gcnArchName "gfx950..." and
 * HSA_OVERRIDE_GFX_VERSION must be unset (hipblaslt_bridge.cpp:69-87).
 * NULL on failure. */
void *mslim_attn_ctx_new(void);

/* Replaces tv_hip_destroy (hipblaslt_bridge.cpp:170-172, native_hip.rs:103). */
void mslim_attn_ctx_destroy(void *ctx);

/* Device report, the GpuDeviceInfo of gpu_backend.rs:21-32 (OpenCL
 * clGetDeviceInfo fields) from hipGetDeviceProperties.  max_allocation_bytes
 * is the memory free at the time of the call (HIP has no per-allocation
 * limit below it). */
typedef struct {
    char name[256];
    char arch[64];   /* gcnArchName, "gfx950:..." */
    char vendor[64];
    int driver_version;
    uint32_t compute_units;
    uint64_t global_memory_bytes;
    uint64_t max_allocation_bytes;
    uint32_t lds_bytes_per_workgroup;
    uint32_t max_clock_mhz;     /* peak engine clock (hipDeviceProp_t::clockRate) */
    uint32_t memory_clock_mhz;  /* peak memory clock (memoryClockRate) */
    uint32_t memory_bus_bits;   /* memory interface width (memoryBusWidth) */
} mslim_attn_device_info;
int mslim_attn_get_device_info(void *ctx, mslim_attn_device_info *out);

/* Device self-check of the BF16 encoder every kernel writes with: gfx950's
 * f32 -> bf16 conversion instruction against the reference's integer rule
 * (round to nearest even; NaN keeps sign and upper payload with the quiet
 * bit forced; gpu_llm.cl:10-21), over all 2^32 f32 encodings.  Stores the
 * number that differ (0 on a conforming device) in *mismatches; takes a few
 * milliseconds and 4 MiB of temporary device memory.  No reference
 * counterpart: it backs the library's use of the instruction. */
int mslim_attn_check_bf16_encoding(void *ctx, uint64_t *mismatches);

/* Route this context's work onto an existing HIP stream; NULL names the HIP
 * null (legacy default) stream.  Until this is called the context uses a
 * stream of its own.  No reference counterpart: the OpenCL engine owns its
 * single queue (gpu_resources.rs:122-123); callers that share a stream with
 * other libraries need to name it. */
int mslim_attn_ctx_set_stream(void *ctx, void *hip_stream);
/* A context's decode workspace and split counters serve one stream at a
 * time: mslim_attn_ctx_set_stream waits for the work queued on the old
 * stream before it switches, and one context must not be driven from two
 * host threads on two streams at once. */

/* Context options.  No reference counterpart (the OpenCL engine has no merge
 * choice); for tests and callers that want the two-launch merge.
 *   MSLIM_ATTN_OPT_DECODE_MERGE: how split-KV decode partials are merged --
 *     MSLIM_ATTN_DECODE_MERGE_FUSED (default): the last workgroup of each
 *     (sequence, kv head) merges them inside the decode launch;
 *     MSLIM_ATTN_DECODE_MERGE_SEPARATE: a merge launch follows the decode
 *     launch.  Both merge in fixed partition order and give the same bits.
 * Returns -1 for an unknown option or value. */
#define MSLIM_ATTN_OPT_DECODE_MERGE 1
#define MSLIM_ATTN_DECODE_MERGE_FUSED 0
#define MSLIM_ATTN_DECODE_MERGE_SEPARATE 1
/*   MSLIM_ATTN_OPT_PREFILL_SPLIT: 1 (default) lets mslim_attn_prefill_causal
 *     split the key range of long row blocks into chunks, merged in fixed
 *     chunk order, when a launch has too few workgroups to keep every CU busy
 *     (same tolerance, deterministic; the output differs from the unsplit
 *     launch in rounding only); 0 never splits. */
#define MSLIM_ATTN_OPT_PREFILL_SPLIT 2
/*   MSLIM_ATTN_OPT_PREFILL_POOL: 1 (default) lets an unsplit
 *     mslim_attn_prefill_causal launch with at least two row blocks per CU
 *     hand its shortest row blocks out at run time (one atomic counter in
 *     the context's device memory), so XCDs running at different clocks
 *     finish together; 0 maps every row block statically.  Each row block
 *     is computed the same way whichever workgroup takes it: the output is
 *     bit-identical either way. */
#define MSLIM_ATTN_OPT_PREFILL_POOL 3
int mslim_attn_ctx_set_option(void *ctx, int option, int64_t value);

/* queue.finish() equivalent (gpu_llm/mod.rs:1998-2001). */
int mslim_attn_synchronize(void *ctx);

/* ---- Device buffers ------------------------------------------------------- */

/* GpuEngine::alloc_u8 (gpu_resources.rs) equivalent; NULL on failure. */
void *mslim_attn_buf_alloc(void *ctx, size_t bytes);
/* Page-locked host memory (hipHostMalloc) for staging that the buffer
 * read/write entry points move by DMA: the seal and restore staging of the
 * ColdStore path, reused across calls.  No reference counterpart (the
 * reference stages through ordinary Vec<u8>).  NULL on failure;
 * mslim_attn_host_free waits for the context's stream first. */
void *mslim_attn_host_alloc(void *ctx, size_t bytes);
int mslim_attn_host_free(void *ctx, void *host);
/* Replaces tv_hip_load_weight (hipblaslt_bridge.cpp:173-187,
 * native_hip.rs:104,146): allocate and copy `bytes` host bytes. */
void *mslim_attn_buf_upload(void *ctx, const uint8_t *bytes, size_t byte_length);
/* Replaces tv_hip_free_weight (hipblaslt_bridge.cpp:188-193). */
int mslim_attn_buf_free(void *ctx, void *buffer);
/* Replaces tv_hip_read_weight (hipblaslt_bridge.cpp:194-202): blocking
 * device->host copy of `size` bytes at `offset`. */
int mslim_attn_buf_read(void *ctx, const void *buffer, size_t offset, uint8_t *out,
                        size_t size);
/* Blocking host->device copy (enqueue_write_buffer CL_BLOCKING,
 * gpu_resources.rs:1010-1016, :1028-1033). */
int mslim_attn_buf_write(void *ctx, void *buffer, size_t offset, const uint8_t *in,
                         size_t size);

/* ---- Attention ------------------------------------------------------------ */

/* Single-token GQA decode over a dense token-major BF16 K/V cache for a
 * ragged batch.  Replaces GpuEngine::attention (gpu_resources.rs:583-643:
 * llm_attention_qk/softmax/pv, gpu_llm.cl:150-212), exact_hot_fused_attention
 * (gpu_resources.rs:783-825, gpu_llm.cl:975-1025) and TiledAttention::run with
 * queries = 1 (tiled_attention.rs:161-293).
 *   seq_lens: host array of `batch` token counts (>= 1), batch <= 64.
 *   scale: softmax scale applied to Q.K (reference: 1/sqrt(head_dim)).
 *   split_tokens: tokens per split-KV partition, a multiple of 64, or 0 to let
 *   the library pick from the shape.  Partitions are defined on logical token
 *   indices only, so the paged entry point with the same split_tokens gives
 *   bit-identical output. */
int mslim_attn_decode_dense(void *ctx, const void *q, const void *k, const void *v,
                            void *out, int batch, const int32_t *seq_lens,
                            int64_t seq_stride_tokens, int q_heads, int kv_heads,
                            int head_dim, float scale, int split_tokens);

/* The split_tokens that split_tokens = 0 picks for this batch: about one
 * workgroup per CU for equal lengths, a smaller split for ragged lengths
 * when that evens out the busiest CU's load; a multiple of 256 in
 * [256, 16384], or 128 for a batch too small to give each of the 256 CUs
 * 256 tokens (tokens x kv_heads <= 32,768).  A function of the lengths and kv_heads only, so the dense
 * and paged entry points pick the same partitions.  Host only (no context,
 * no device work); -1 on invalid arguments.  No counterpart in the
 * reference, whose split count is a config field (attention_kernel.rs:
 * 16-40, splits 1..64). */
int mslim_attn_decode_auto_split(const int32_t *seq_lens, int batch, int kv_heads);

/* The same decode over the ColdStore-exact paged layout.  Replaces
 * attention_gpu_region (gpu_resources.rs:883-1063: llm_attention_qk/softmax +
 * llm_lod_pv_stage/finish, gpu_llm.cl:280-322) at epsilon = 0, with K and V
 * both resident in the device page pool.
 *   page_table: device int32 [batch][pages_per_seq].
 *   page_tokens: tokens per page, a multiple of 16 (16 in the ColdStore-exact
 *   configuration). */
int mslim_attn_decode_paged(void *ctx, const void *q, const void *k_pool,
                            const void *v_pool, void *out, int batch,
                            const int32_t *seq_lens, const int32_t *page_table,
                            int pages_per_seq, int page_tokens, int q_heads,
                            int kv_heads, int head_dim, float scale, int split_tokens);

/* mslim_attn_decode_paged without any allocation.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * split partials live in a fixed 16 MiB device array of the library (one per
 * GPU, held until the process ends) instead of the context workspace, and the
 * partitions are merged by a second launch, so no counter has to start at
 * zero.  Same arguments and the same output bits as mslim_attn_decode_paged
 * with the same split_tokens.  A call whose partials exceed 16 MiB
 * (splits x kv_heads x group x (head_dim + 2) x 4 bytes) fails with -1 and
 * names the size.  Every call on one GPU shares the array, whichever context
 * makes it: calls that overlap on one GPU (two streams or two host threads)
 * race and give wrong results. */
int mslim_attn_decode_paged_noalloc(void *ctx, const void *q, const void *k_pool,
                                    const void *v_pool, void *out, int batch,
                                    const int32_t *seq_lens, const int32_t *page_table,
                                    int pages_per_seq, int page_tokens, int q_heads,
                                    int kv_heads, int head_dim, float scale,
                                    int split_tokens);

/* Causal GQA attention for a chunk of `queries` new tokens after `prior`
 * cached tokens: row i attends keys 0..prior+i.  K/V hold prior+queries
 * tokens, token-major.  Replaces BatchKernels::attention (prefill.rs:363-435:
 * llm_prefill_qk/softmax/pv, gpu_llm.cl:462-541) and TiledAttention::run
 * (tiled_attention.rs:161-293) for queries >= 1, including batched
 * multi-query decode. */
int mslim_attn_prefill_causal(void *ctx, const void *q, const void *k, const void *v,
                              void *out, int queries, int prior, int q_heads,
                              int kv_heads, int head_dim, float scale);

/* Key tiles (64 keys each) per chunk that mslim_attn_prefill_causal splits
 * the longest row blocks of this shape into, or 0 when the launch is not
 * split (enough workgroups to keep every CU busy, or MSLIM_ATTN_OPT_PREFILL_
 * SPLIT off).  A function of the shape only.  Host only (no context, no
 * device work); -1 on invalid arguments.  No reference counterpart. */
int mslim_attn_prefill_split_tiles(int queries, int prior, int q_heads, int kv_heads, int head_dim);

/* Row blocks per XCD that mslim_attn_prefill_causal hands out at run time
 * for this shape (MSLIM_ATTN_OPT_PREFILL_POOL on), or 0 when the launch maps
 * every row block statically (split launches, fewer than two row blocks per
 * CU, the any-geometry fallback).  A function of the shape only.  Host only;
 * -1 on invalid arguments.  No reference counterpart. */
int mslim_attn_prefill_pool_items(int queries, int prior, int q_heads, int kv_heads, int head_dim);

/* ---- Portable backend (exact K/V frames) ------------------------------------ */

/* K/V frame formats: the dtype codes of gpu_backend.rs:258-262. */
#define MSLIM_ATTN_FORMAT_BF16 1
#define MSLIM_ATTN_FORMAT_F16 2
#define MSLIM_ATTN_FORMAT_F32 3
/* Return code for a non-finite query or output (PortableError::NonFinite,
 * portable.rs:43, raised at gpu_backend.rs:154-156 and :363-365). */
#define MSLIM_ATTN_ERR_NONFINITE (-2)

/* Per-call report of mslim_attn_backend_decode; mirrors GpuTimings
 * (gpu_backend.rs:34-44).  The reference's three kernel times become one:
 * QK, softmax and P.V run fused. */
typedef struct {
    double dispatch_ms;       /* whole call: uploads, kernels, readback */
    double kernel_ms;         /* attention kernels (HIP events) */
    uint64_t input_kv_bytes;  /* K + V payload bytes uploaded */
    uint64_t scratch_bytes;   /* split partials in device memory */
    uint64_t output_bytes;
} mslim_attn_timings;

/* Single-token decode over exact K/V frames on device buffers: the work of
 * GpuBackend::decode (gpu_backend.rs:149-377; kernels mslim_qk / mslim_softmax
 * / mslim_pv, gpu_attention.cl:35-82).
 *   query: f32 [q_heads][head_dim].
 *   keys / values: raw little-endian [tokens][kv_heads][head_dim] in
 *   key_format / value_format (MSLIM_ATTN_FORMAT_*), the frames concatenated
 *   in append order as gpu_backend.rs:186-198 concatenates them.
 *   out: f32 [q_heads][head_dim]; scale 1/sqrt(head_dim) (gpu_attention.cl:48).
 *   tokens == 0 writes zeros (gpu_backend.rs:157-159).  head_dim <= 1024.
 * Stream-ordered: non-finite inputs propagate into the output unchecked. */
int mslim_attn_frames_decode(void *ctx, const float *query, const void *keys, int key_format,
                             const void *values, int value_format, float *out, int64_t tokens,
                             int q_heads, int kv_heads, int head_dim);

/* The blocking host-memory form, one call per AttentionBackend::decode
 * (portable.rs:561-565, gpu_backend.rs:370-377): uploads the host query and
 * frames into context-owned device buffers (reused across calls, unlike the
 * reference's per-call allocation), runs mslim_attn_frames_decode, reads the
 * output back and returns MSLIM_ATTN_ERR_NONFINITE for a non-finite query
 * ("GPU Q") or output ("GPU output").  `timings` may be NULL. */
int mslim_attn_backend_decode(void *ctx, const float *query, const void *keys, int key_format,
                              const void *values, int value_format, int64_t tokens, int q_heads,
                              int kv_heads, int head_dim, float *out,
                              mslim_attn_timings *timings);

/* ---- Feeder kernels ------------------------------------------------------- */

/* RMSNorm over `tokens` rows of `hidden` BF16 values: 128-lane strided FMA
 * sum of squares, tree reduction, y = BF16(BF16(x*f)*w).  Replaces
 * GpuEngine::norm (gpu_resources.rs:485-507, llm_rmsnorm gpu_llm.cl:72-98) and
 * the prefill norm (prefill.rs:292-320, llm_prefill_norm gpu_llm.cl:378-408). */
int mslim_attn_rmsnorm(void *ctx, const void *input, const void *weight, void *output,
                       int tokens, int hidden, float epsilon);

/* Rotate-half RoPE on [tokens][heads][head_dim], row t at position
 * start_position + t, optional llama3 frequency scaling.  Replaces
 * GpuEngine::rope (gpu_resources.rs:509-537, llm_rope gpu_llm.cl:102-146) and
 * the prefill RoPE (prefill.rs:322-361, llm_prefill_rope gpu_llm.cl:412-456);
 * arguments mirror RopeKernelConfig (gpu_llm/kernels.rs:15-23). */
int mslim_attn_rope(void *ctx, const void *input, void *output, int tokens, int heads,
                    int head_dim, int start_position, float theta, int llama3_scaling,
                    float factor, float low_freq_factor, float high_freq_factor,
                    float original_max_position);

/* The prefill RoPE of a prompt chunk's Q ([tokens][q_heads][head_dim]) and K
 * ([tokens][kv_heads][head_dim]) in one call: the same bits as
 * mslim_attn_rope on Q and on K at the same start_position (prefill.rs:322-361
 * rotates the two with two llm_prefill_rope launches, gpu_llm.cl:412-456).
 * One launch shares each row's cos/sin between the Q and K heads when
 * head_dim is a multiple of 16 (at most 512), the rows are 16-byte aligned
 * and (q_heads + kv_heads) * head_dim <= 16384; otherwise two. */
int mslim_attn_rope_qk(void *ctx, const void *q, void *q_out, const void *k, void *k_out, int tokens,
                       int q_heads, int kv_heads, int head_dim, int start_position, float theta,
                       int llama3_scaling, float factor, float low_freq_factor, float high_freq_factor,
                       float original_max_position);

/* The same RoPE with row t at position positions[t] (device int32 [tokens],
 * each >= 0): one decode row per sequence of a batch, each sequence at its own
 * position.  The reference rotates one sequence per call (llm_rope's `pos`,
 * gpu_llm.cl:102-146; gpu_resources.rs:509-537). */
int mslim_attn_rope_rows(void *ctx, const void *input, void *output, int tokens, int heads,
                         int head_dim, const int32_t *positions, float theta, int llama3_scaling,
                         float factor, float low_freq_factor, float high_freq_factor,
                         float original_max_position);

/* out = BF16(BF16(silu(gate)) * up) over n elements.  Replaces
 * GpuEngine::swiglu (gpu_resources.rs:561-581, llm_swiglu gpu_llm.cl:225-237). */
int mslim_attn_swiglu(void *ctx, const void *gate, const void *up, void *output, size_t n);

/* output = BF16(a + b) over n elements (llm_add, gpu_llm.cl:214-222): the
 * residual adds of a decoder layer. */
int mslim_attn_add(void *ctx, const void *a, const void *b, void *output, size_t n);

/* Rows `ids[t]` (device int32 [tokens]) of a [vocab][hidden] BF16 table into
 * output [tokens][hidden] (llm_embed, gpu_llm.cl:24-33).  An id outside
 * [0, vocab) gives a zero row and, when `bad` (device int) is not NULL, sets
 * *bad = 1.  hidden must be a multiple of 8. */
int mslim_attn_embed(void *ctx, const void *table, int vocab, int hidden, const int32_t *ids,
                     int tokens, void *output, int *bad);

/* Greedy token of each of `rows` rows of BF16 logits [rows][vocab] into device
 * int32 out[rows], the first index winning ties (llm_argmax,
 * gpu_llm.cl:239-270). */
int mslim_attn_argmax(void *ctx, const void *logits, int rows, int vocab, int32_t *out);

/* ---- ColdStore-exact page pool --------------------------------------------- */

/* The page entry points below (write, append, gather, digest) take any
 * power-of-two page_tokens: 16 is the ColdStore-exact pool the paged decode
 * reads, and 1 makes a pool of token-major rows, i.e. the dense layout
 * addressed through a table (GpuRegionStore uses 1-token pages for decode
 * appends, gpu_region_store.rs:376-384). */

/* Write `tokens` token-major rows of one sequence (K and V, [tokens][kv_heads]
 * [head_dim]) into the page pool at logical positions first_token.. through
 * the device page table row `page_table` (int32 [pages]).  The device
 * counterpart of GpuRegionStore::append_batch's token-major -> head-major page
 * conversion (gpu_region_store.rs:391-520). */
int mslim_attn_pages_write(void *ctx, void *k_pool, void *v_pool, const int32_t *page_table,
                           int page_tokens, int kv_heads, int head_dim, int64_t first_token,
                           int64_t tokens, const void *k_rows, const void *v_rows);

/* Decode-step append of one token to each of `batch` sequences: K/V row b
 * ([batch][kv_heads][head_dim]) goes to logical position positions[b] (device
 * int32) through page-table row b of the device table [batch][pages_per_seq].
 * A position outside [0, pages_per_seq * page_tokens) writes nothing.  The
 * batched form of the per-token KV append of run_layer (gpu_llm/mod.rs:
 * 2103-2136) into the page layout of gpu_region_store.rs:391-520. */
int mslim_attn_pages_append(void *ctx, void *k_pool, void *v_pool, const int32_t *page_table,
                            int pages_per_seq, int page_tokens, int kv_heads, int head_dim,
                            int batch, const int32_t *positions, const void *k_rows,
                            const void *v_rows);

/* One decode step's RoPE and K/V append in a single launch: Q rows
 * ([batch][q_heads][head_dim]) rotated to q_out, K rows rotated and written
 * with the V rows ([batch][kv_heads][head_dim]) to logical position
 * positions[b] of sequence b through page-table row b.  Equal, bit for bit, to
 * mslim_attn_rope_rows on Q and on K followed by mslim_attn_pages_append of
 * the rotated K and V (head_dim a multiple of 8, at most 512).  The reference
 * runs the two llm_rope launches and the K/V copies of run_layer separately
 * (gpu_llm/mod.rs:2094-2136). */
int mslim_attn_rope_append(void *ctx, const void *q, const void *k, const void *v, void *q_out,
                           void *k_pool, void *v_pool, const int32_t *page_table, int pages_per_seq,
                           int page_tokens, int batch, const int32_t *positions, int q_heads,
                           int kv_heads, int head_dim, float theta, int llama3_scaling, float factor,
                           float low_freq_factor, float high_freq_factor,
                           float original_max_position);

/* Gather `tokens` logical positions [first_token, first_token+tokens) of one
 * sequence from a page pool into token-major rows [tokens][kv_heads][head_dim].
 * The device counterpart of GpuRegionStore::read_keys / read_values
 * (gpu_region_store.rs:828-927).  Apply it once to the K pool and once to the
 * V pool. */
int mslim_attn_pages_gather(void *ctx, const void *pool, const int32_t *page_table,
                            int page_tokens, int kv_heads, int head_dim,
                            int64_t first_token, int64_t tokens, void *rows_out);

/* Logical K/V SHA-256 (hex, 65 bytes with NUL) of `layers` layers of one
 * sequence of `tokens` tokens: "mslim-dense-kv-state-v1" || u64 LE tokens ||
 * per layer K then V in [kv_heads][token][head_dim] order.  Replaces
 * GpuLlm::logical_kv_sha256 (gpu_llm/mod.rs:1981-2028) and
 * GpuRegionStore::logical_kv_sha256 (gpu_region_store.rs:341-371).
 *   Dense: keys[l] / values[l] are token-major device buffers, page_tables
 *   NULL.  Paged: keys[l] / values[l] are page pools and page_tables[l] the
 *   device page-table row of layer l (page_tokens > 0).  Blocking. */
int mslim_attn_logical_kv_sha256(void *ctx, int layers, int64_t tokens, int kv_heads,
                                 int head_dim, const void *const *keys,
                                 const void *const *values,
                                 const int32_t *const *page_tables, int page_tokens,
                                 char *hex_out);

/* ---- ColdStore record frames ----------------------------------------------- */

/* One ColdStore record to be made from a pool page: its header fields
 * (cold_store.rs:291-309) and the pool page holding its K and V payloads in
 * rows first_row .. first_row + tokens - 1 of every head (first_row > 0 when
 * a record starts inside a page, for example after a turn that ended there;
 * first_row + tokens <= page_tokens). */
typedef struct {
    uint64_t page_id;
    uint64_t token_start;
    uint32_t layer;
    uint32_t tokens;    /* 1..page_tokens */
    int32_t pool_page;  /* 0..pool_pages-1 */
    uint32_t first_row; /* pool-page row of the first token */
} mslim_attn_page_record;

#define MSLIM_ATTN_RECORD_HEADER_BYTES 104 /* cold_store.rs:23 */
#define MSLIM_ATTN_RECORD_FOOTER_BYTES 56  /* cold_store.rs:24 */

/* Bytes of one frame slot for pools of `page_tokens`-token pages:
 * 104 + 16 * page_tokens + 56. */
int64_t mslim_attn_record_frame_bytes(int page_tokens);

/* Compute, on the device, everything of a ColdStore record except its
 * payloads, for `count` records whose K/V payloads sit in pool pages.  The
 * device counterpart of ColdStore::prepare_page (cold_store.rs:269-349) with
 * token_hashes (:725-742), checksum / checksum_many (:909-922) and the
 * SHA-256 record digest (:924-930); byte-identical to them.
 *   k_pool, v_pool: page pools [pool_pages][kv_heads][page_tokens][head_dim]
 *     BF16 (head_dim * 2 bytes per row).
 *   records: device array [count].
 *   frames: device output [count][mslim_attn_record_frame_bytes(page_tokens)];
 *     slot i holds header (104 B) | K token hashes (8 * tokens_i B) | V token
 *     hashes (8 * tokens_i B) | zeros | footer (56 B, the slot's last bytes).
 * Record i's file bytes are slot[0 .. 104 + 16 * tokens_i) | K payload |
 * V payload | slot footer, the payloads being the head-major
 * [kv_heads][tokens_i][head_dim] rows first_row.. of pool page pool_page.  A
 * record whose tokens, first_row or pool_page is out of range gets an
 * all-zero slot (no header magic).  `tile` must divide head_dim
 * (cold_store.rs:690-692).  Stream-ordered. */
int mslim_attn_record_frames(void *ctx, const void *k_pool, const void *v_pool, int64_t pool_pages,
                             int page_tokens, int kv_heads, int head_dim, uint32_t tile,
                             const mslim_attn_page_record *records, int count, void *frames);

/* The same frames for records whose payloads sit in staging (slot i of
 * k_stage / v_stage holds record i compacted to [kv_heads][tokens_i]
 * [head_dim], the layout of mslim_attn_record_payloads) instead of pool
 * pages; pool_page and first_row are not read.  Lets a restore verify a
 * stored record on the device before any of its bytes reach the pool (the
 * reference verifies each record before its bytes reach the GPU buffer,
 * gpu_llm/mod.rs:1367-1398).  Stream-ordered. */
int mslim_attn_record_frames_staged(void *ctx, const void *k_stage, const void *v_stage, int page_tokens,
                                    int kv_heads, int head_dim, uint32_t tile,
                                    const mslim_attn_page_record *records, int count, void *frames);

/* Move the payloads of `count` records between their pool pages and
 * contiguous staging, so a batch of records crosses PCIe as one copy each
 * way.  Staging slot i (kv_heads * page_tokens * head_dim * 2 bytes in
 * k_stage and in v_stage) holds record i's payload compacted to
 * [kv_heads][tokens_i][head_dim]: exactly the bytes ColdStore stores
 * (cold_store.rs:480-483).  direction 0: pool -> staging (sealing pages into
 * the ColdStore, the device side of GpuRegionStore::append_batch,
 * gpu_region_store.rs:452-472); direction 1: staging -> pool (restoring
 * verified pages, replacing the per-chunk read_values + H2D staging of
 * gpu_resources.rs:1017-1048).  Only rows first_row .. first_row + tokens_i
 * - 1 of each pool page move.  Records out of range are skipped.
 * Stream-ordered. */
int mslim_attn_record_payloads(void *ctx, void *k_pool, void *v_pool, int64_t pool_pages, int page_tokens,
                               int kv_heads, int head_dim, const mslim_attn_page_record *records,
                               int count, void *k_stage, void *v_stage, int direction);

/* ---- Projection GEMM -------------------------------------------------------- */

/* Replaces tv_hip_matrix_multiply (hipblaslt_bridge.cpp:203-233, bound at
 * native_hip.rs:19-20): output[tokens][rows] = BF16(input[tokens][inner] .
 * weight[rows][inner]^T), fp32 accumulation rounded once, on the library's
 * own MFMA kernels (no hipBLASLt).  weight is a device buffer
 * (mslim_attn_buf_upload); input and output are HOST buffers of BF16 bits
 * and the call blocks, as in the reference.  Limits as the reference:
 * 0 < tokens <= 512, 0 < inner <= 32768, 0 < rows <= 500000.  Codes: -1
 * arguments, 100+hipError_t, 400/401 staging allocation, 402 H2D, 404
 * product launch, 405 D2H (the stage codes of hipblaslt_bridge.cpp:217-231;
 * the 200+ library statuses and 403 no longer arise). */
int mslim_attn_matrix_multiply(void *ctx, const void *weight, const uint8_t *input, uint8_t *output,
                               int inner, int rows, int tokens);

/* The same product on device buffers (input [tokens][inner], output
 * [tokens][rows]), stream-ordered: the form the device-resident layer
 * (norm -> QKV -> RoPE -> attention -> O -> SwiGLU -> down) chains without
 * host round trips.  output must not alias input or weight.  Decode batches
 * (tokens <= 16, inner a multiple of 32, input and weight 16-byte aligned)
 * run on the MFMA kernel that streams the weights once, the role of the
 * reference's decode GEMVs (llm_gemv_bf16 / reuse-8, gpu_llm.cl:38-68,
 * :553-596); larger products run on the tiled MFMA kernel of the prompt
 * chunks (llm_prefill_gemv_reuse8/16/32, gpu_llm.cl:553-683), or, for inner
 * not a multiple of 64 or unaligned buffers, a kernel of one wavefront per
 * output.  Each product of a given shape is summed in one fixed order, so
 * every entry point below that fuses an epilogue gives the same bits as this
 * one followed by the elementwise call. */
int mslim_attn_gemm_bf16(void *ctx, const void *weight, const void *input, void *output, int inner,
                         int rows, int tokens);

/* output = BF16(residual + BF16(input . weight^T)): the O and down
 * projections with the residual add of run_layer (gpu_llm/mod.rs:2056-2350;
 * llm_add, gpu_llm.cl:214-222) fused.  Bit-identical to mslim_attn_gemm_bf16
 * followed by mslim_attn_add.  output may equal residual. */
int mslim_attn_gemm_bf16_add(void *ctx, const void *weight, const void *input, const void *residual,
                             void *output, int inner, int rows, int tokens);

/* output = SwiGLU(BF16(input . gate^T), BF16(input . up^T)) over
 * [tokens][rows]: llm_fused_swiglu_bf16 (gpu_llm.cl:797-834,
 * project_swiglu8 prefill.rs:247).  Bit-identical to two mslim_attn_gemm_bf16
 * calls followed by mslim_attn_swiglu. */
int mslim_attn_gemm_swiglu(void *ctx, const void *gate_weight, const void *up_weight, const void *input,
                           void *output, int inner, int rows, int tokens);

/* The Q, K and V projections of one input in one call: llm_fused_qkv_bf16
 * (gpu_llm.cl:740-796, project_fused_qkv gpu_resources.rs:406-440).
 * Bit-identical to three mslim_attn_gemm_bf16 calls. */
int mslim_attn_gemm_qkv(void *ctx, const void *q_weight, const void *k_weight, const void *v_weight,
                        const void *input, void *q_out, void *k_out, void *v_out, int inner, int q_rows,
                        int kv_rows, int tokens);

/* The RMSNorm that precedes a projection in run_layer (llm_rmsnorm,
 * gpu_llm.cl:72-98, then the product; gpu_llm/mod.rs:2056-2350), in one
 * call: bit-identical to mslim_attn_rmsnorm(input, norm_weight, epsilon)
 * followed by mslim_attn_gemm_bf16 / _gemm_qkv / _gemm_swiglu on the
 * normalised rows.  Decode batches of up to 8 rows of up to 4096 inputs
 * normalise inside the projection kernel (no launch and no buffer for the
 * normalised rows); other shapes normalise into a context buffer first. */
int mslim_attn_rmsnorm_gemm_bf16(void *ctx, const void *norm_weight, float epsilon, const void *weight,
                                 const void *input, void *output, int inner, int rows, int tokens);
int mslim_attn_rmsnorm_gemm_qkv(void *ctx, const void *norm_weight, float epsilon, const void *q_weight,
                                const void *k_weight, const void *v_weight, const void *input, void *q_out,
                                void *k_out, void *v_out, int inner, int q_rows, int kv_rows, int tokens);
int mslim_attn_rmsnorm_gemm_swiglu(void *ctx, const void *norm_weight, float epsilon, const void *gate_weight,
                                   const void *up_weight, const void *input, void *output, int inner, int rows,
                                   int tokens);

/* The head of a decode step's layer in one call (run_layer,
 * gpu_llm/mod.rs:2056-2136: input norm, fused QKV, the two RoPEs and the K/V
 * copy into the cache): bit-identical to mslim_attn_rmsnorm_gemm_qkv into
 * [batch][q_heads * head_dim] / [batch][kv_heads * head_dim] rows followed by
 * mslim_attn_rope_append with the same arguments.  q_out receives the rotated
 * Q rows; the rotated K and the V row of sequence b go into the pools at
 * positions[b] through page_table row b (no append for a position outside
 * the table).  Batches of up to 8 rows of up to 4096 inputs with head_dim a
 * multiple of 16 run as one kernel (RoPE and append in the projection's
 * epilogue); other shapes run the two calls through a context buffer. */
int mslim_attn_rmsnorm_qkv_rope_append(void *ctx, const void *norm_weight, float epsilon, const void *q_weight,
                                       const void *k_weight, const void *v_weight, const void *input, void *q_out,
                                       void *k_pool, void *v_pool, const int32_t *page_table, int pages_per_seq,
                                       int page_tokens, int batch, const int32_t *positions, int inner, int q_heads,
                                       int kv_heads, int head_dim, float theta, int llama3_scaling, float factor,
                                       float low_freq_factor, float high_freq_factor, float original_max_position);

#ifdef __cplusplus
}
#endif
#endif /* MSLIM_ATTN_H */
