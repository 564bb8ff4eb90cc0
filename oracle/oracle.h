/*
 * CPU oracle for the M-SLIM attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library restates, in plain C, the reference
 * algorithms of sheilyneural-afk/VK-SHEI that the MI355X kernels replace.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it,
 * and only as the checker.  The product path (libmslim_attn.so) never links or
 * calls it.
 *
 * Every function cites the reference file:line it follows.  Transcendental
 * functions (exp, log, pow, sin, cos) are evaluated in double precision and
 * rounded once to float: the reference's own libm/OpenCL bits for these are not
 * reproducible here, and the once-rounded value is the common target that the
 * HIP feeder kernels evaluate the same way.
 *
 * Pinning status: see the "pin:" note on each function.  Functions whose note
 * reads "parity unpinned" have no golden vector, known answer or closed-form
 * check that would fail on a plausible mistake.
 */
#ifndef MSLIM_ORACLE_H
#define MSLIM_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- BF16 codec --------------------------------------------------------- */
/* gpu_llm.cl:7-9.  pin: exhaustive over all 65,536 encodings
 * (tests/fixed_width_decode.rs:10-21 restated). */
float orc_read_bf16(uint16_t bits);
/* gpu_llm.cl:10-21.  pin: exhaustive over all 2^32 f32 inputs against
 * orc_bf16_round_independent and against the half-2.7.1 branch form. */
uint16_t orc_write_bf16(float value);
/* half 2.7.1 `bf16::from_f32` (used by native_cpu_adapter.rs:179-181): branch
 * form of round-to-nearest-even with NaN quieting. */
uint16_t orc_half_bf16_from_f32(float value);
/* Independent RNE: scale to an integer significand in double, nearbyint(),
 * scale back.  Used only to pin the two forms above. */
uint16_t orc_bf16_round_independent(float value);
/* Counts mismatches of the three encoders over the f32 bit range
 * [start, start+count) (count may be 2^32 with start 0). */
uint64_t orc_bf16_encoder_mismatches(uint64_t start, uint64_t count);
void orc_bf16_to_f32_array(const uint16_t *in, float *out, size_t n);
void orc_f32_to_bf16_array(const float *in, uint16_t *out, size_t n);

/* ---- Attention oracles -------------------------------------------------- */
/* native_cpu_adapter.rs:253-307 `dense_attention_bf16`: f32 products summed
 * sequentially without FMA, f32 softmax (:223-233), scale = 1/sqrt(D) in f32
 * (:235-237), output rounded to BF16 (returned as f32 values).
 * K/V token-major [tokens][kv_heads][head_dim] BF16 bits.  Returns 0 or -1. */
int orc_dense_attention_bf16(int query_heads, int kv_heads, int head_dim,
                             const float *query, const uint16_t *keys,
                             const uint16_t *values, int tokens, float *out);

/* portable.rs:575-646 `CpuReferenceBackend::decode`: f64 online log-sum-exp
 * over K/V of dtype 1=BF16, 2=F16, 3=F32 (raw LE bits, [tokens][kvh][D]).
 * Returns 0, 1 (ShapeMismatch), 2 (NonFinite).  tokens==0 gives zeros.
 * pin: portable.rs:683-710 (zero query -> mapped V), :712-726 (extreme
 * scores -> exactly 3.0), :806-825 (rejections); brute force in f64. */
int orc_cpu_reference_decode(int query_heads, int kv_heads, int head_dim,
                             const float *query, const void *keys,
                             const void *values, int dtype, int tokens,
                             float *out);
/* The same with separate K and V formats: the reference decodes every frame
 * element through its own tensor's dtype (portable.rs:120-145), and the GPU
 * backend takes one key and one value format (gpu_backend.rs:187-199). */
int orc_cpu_reference_decode_formats(int query_heads, int kv_heads, int head_dim,
                                     const float *query, const void *keys, int key_dtype,
                                     const void *values, int value_dtype, int tokens,
                                     float *out);

/* Causal prefill on the CPU path: the reference CPU decoder processes a prompt
 * token by token (native_cpu_adapter.rs:486-534), so query row i attends to
 * keys 0..prior+i with `dense_attention_bf16`.  q: [queries][QH][D] f32,
 * K/V token-major with prior+queries tokens, out: [queries][QH][D]. */
int orc_prefill_causal_cpu(int query_heads, int kv_heads, int head_dim,
                           const float *query, const uint16_t *keys,
                           const uint16_t *values, int queries, int prior,
                           float *out);

/* gpu_llm.cl:150-212 (llm_attention_qk / softmax / pv) and :462-541
 * (llm_prefill_qk / softmax / pv): the reference GPU arithmetic, sequential
 * FMA over d and t, dot * (1/sqrt(D)), f32 exp.  Q BF16 bits, out BF16 bits.
 * queries/prior as in the prefill kernels; decode is queries=1, prior=T-1. */
int orc_gpu_reference_attention(int query_heads, int kv_heads, int head_dim,
                                const uint16_t *query, const uint16_t *keys,
                                const uint16_t *values, int queries, int prior,
                                uint16_t *out);

/* ---- Feeder kernels ----------------------------------------------------- */
/* native_cpu_adapter.rs:194-204 `rms_norm` (f32 sequential sum, no FMA). */
void orc_rms_norm_cpu(const float *x, const float *w, int n, float eps, float *out);
/* gpu_llm.cl:72-98 / :378-408 `llm_rmsnorm` / `llm_prefill_norm`: 128-lane
 * strided FMA sum of squares, 64..1 tree reduction, factor = 1/sqrt(mean+eps),
 * y = BF16(BF16(x*f)*w).  One row of `hidden` elements per token. */
void orc_rmsnorm_gpu(const uint16_t *x, const uint16_t *w, int tokens, int hidden,
                     float eps, uint16_t *out);
/* kernels.rs:51-66 / gpu_llm.cl:123-138 inverse frequency (GPU form, with
 * optional llama3 scaling).  pin: gpu_llm/mod.rs:2849-2877 transformers
 * 4.51.3 table. */
float orc_rope_inverse_frequency(int frequency_dim, int head_dim, float theta,
                                 int llama3, float factor, float low_freq,
                                 float high_freq, float original_max_position);
/* gpu_llm.cl:102-146 / :412-456 `llm_rope` / `llm_prefill_rope`:
 * rotate-half, c,s rounded BF16, out = BF16(BF16(x*c) + BF16(rot*s)).
 * x: [tokens][heads][head_dim] BF16, position of row t = start + t.
 * pin: position 0 is the identity (native_cpu_adapter.rs:996-1001). */
void orc_rope_gpu(const uint16_t *x, uint16_t *out, int tokens, int heads,
                  int head_dim, int start_position, float theta, int llama3,
                  float factor, float low_freq, float high_freq,
                  float original_max_position);
/* native_cpu_adapter.rs:206-221 `apply_rope` (CPU form, angle = pos /
 * theta^(2i/D)), in place on f32 values of one token. */
void orc_rope_cpu(float *values, int heads, int dim, int position, float theta);
/* gpu_llm.cl:225-237 `llm_swiglu` (= native_cpu_adapter.rs:559-566). */
void orc_swiglu(const uint16_t *gate, const uint16_t *up, size_t n, uint16_t *out);
/* native_cpu_adapter.rs:223-233 `softmax` (f32). pin: sums to 1 (:1003-1008) */
void orc_softmax(float *values, int n);

/* gpu_llm.cl:214-222 `llm_add`: out = BF16(a + b).
 * pin: sums of small integers are exact; a + (-a) = +0; ties to even at the
 * BF16 boundary (1 + 2^-8 -> 1, 1 + 3*2^-8 -> 1 + 2^-6). */
void orc_add_bf16(const uint16_t *a, const uint16_t *b, size_t n, uint16_t *out);
/* gpu_llm.cl:239-270 `llm_argmax` over each of `rows` rows: start from
 * (-inf, 0), take a value that is greater or equal with a lower index.
 * pin: numpy.argmax on rows of distinct finite values; first index on ties;
 * NaN never chosen; a row of -inf (or NaN) gives 0. */
void orc_argmax_bf16(const uint16_t *logits, int rows, int vocab, int32_t *out);

/* hipblaslt_bridge.cpp:203-233: out[t][r] = BF16(sum_i in[t][i] * w[r][i]),
 * fp32 accumulation (fma, ascending i), one rounding. */
void orc_matmul_bf16(const uint16_t *w, const uint16_t *in, int inner, int rows, int tokens, uint16_t *out);

/* native_cpu_adapter.rs:129-150 NativeWeightArchive::matvec of the reference
 * CPU decoder: out[r] = BF16(sum_i w[r][i] * x[i]) with every product rounded
 * to f32 and summed left to right from -0.0 (no FMA), x in f32.  Rows are
 * independent (the reference runs them in parallel with rayon), so they are
 * split over OpenMP threads; each row's sum order is unchanged.
 * pin: the sequence order of the sum ([2^25, 1, -2^25, 1] -> 1, not 2 or 0),
 * no FMA (a product that an FMA would keep unrounded), BF16 rounding of the
 * sum, and f64 brute force within one rounding on random rows. */
void orc_matvec_cpu(const uint16_t *w, const float *x, int rows, int cols, float *out);

/* native_cpu_adapter.rs:577-582: the reference CPU decoder's greedy token,
 * `max_by(|a, b| a.total_cmp(b))` over the f32 logits: the LAST index among
 * equal maxima, under IEEE total order (-NaN < -inf < ... < -0 < +0 < ... <
 * +inf < +NaN).  The GPU argmax (orc_argmax_bf16, gpu_llm.cl:239-270) takes
 * the FIRST index on ties and never picks NaN.
 * pin: ties resolve to the last index, -0 < +0, +NaN above +inf, -NaN below
 * -inf; distinct values agree with numpy.argmax. */
int32_t orc_argmax_total_last(const float *logits, int n);

/* ---- Integrity primitives ----------------------------------------------- */
/* cold_store.rs:909-922 FNV-1a-64 over concatenated parts.
 * pin: published vectors ("" -> cbf29ce484222325, "a" -> af63dc4c8601ec8c). */
uint64_t orc_fnv1a64(const uint8_t *bytes, size_t n, uint64_t state);
/* FIPS 180-4 SHA-256 (the sha2 0.11.1 crate, cold_store.rs:924-930).
 * pin: FIPS vectors "abc", "", 448-bit message, 10^6 x 'a'. */
typedef struct { uint32_t h[8]; uint64_t len; uint8_t buf[64]; size_t fill; } orc_sha256_ctx;
void orc_sha256_init(orc_sha256_ctx *c);
void orc_sha256_update(orc_sha256_ctx *c, const uint8_t *data, size_t n);
void orc_sha256_final(orc_sha256_ctx *c, uint8_t out[32]);
void orc_sha256(const uint8_t *data, size_t n, uint8_t out[32]);

/* ---- ColdStore record and region store --------------------------------- */
/* cold_store.rs:725-742 per-token FNV hash over all heads of a head-major
 * payload [heads][tokens][per_head_token bytes]. */
int orc_token_hashes(const uint8_t *payload, size_t len, uint32_t tokens,
                     uint32_t heads, uint64_t *out);
/* cold_store.rs:269-349 `prepare_page`: full record bytes.  Returns the record
 * length (0 on invalid geometry); writes at most `cap` bytes to `record`. */
size_t orc_coldstore_record(uint64_t page_id, uint32_t layer, uint64_t token_start,
                            uint32_t tokens, uint32_t heads, uint32_t head_dim,
                            uint32_t tile, const uint8_t *key, size_t key_len,
                            const uint8_t *value, size_t value_len,
                            uint8_t *record, size_t cap);
/* gpu_region_store.rs:459-472 token-major [n][kvh][D] -> head-major
 * [kvh][n][D] page payload (row_bytes = D*2). */
void orc_token_to_head_major(const uint8_t *token_major, uint32_t n, uint32_t kvh,
                             uint32_t row_bytes, uint8_t *head_major);
/* gpu_region_store.rs:828-878 / :882-927 gather: positions through a
 * token->(page, offset) table into token-major bytes.  `pages` holds
 * head-major payloads of `page_tokens` tokens, `page_of[t]`/`offset_of[t]`
 * the per-token address.  pin: gpu_region_store.rs:991-1040 known answers. */
void orc_gather_token_major(const uint8_t *pool, size_t page_bytes,
                            uint32_t page_tokens, uint32_t kvh, uint32_t row_bytes,
                            const uint32_t *page_of, const uint32_t *offset_of,
                            const uint32_t *positions, size_t count, uint8_t *out);
/* gpu_region_store.rs:341-371 and gpu_llm/mod.rs:1981-2028 logical K/V
 * SHA-256: "mslim-dense-kv-state-v1" || u64 tokens || per layer K then V,
 * each in [kvh][token][D] order, from token-major per-layer buffers. */
void orc_logical_kv_sha256(uint32_t layers, uint64_t tokens, uint32_t kvh,
                           uint32_t row_bytes, const uint8_t *const *keys,
                           const uint8_t *const *values, uint8_t out[32]);

#ifdef __cplusplus
}
#endif
#endif
