/* Decoder runner over libmslim_attn (exported by libmslim_host).
 *
 * The per-layer order of the reference GPU runtime -- run_layer
 * (src/gpu_llm/mod.rs:2056-2350) for decode and run_batch_layer
 * (src/gpu_llm/prefill.rs:897-1061) for prompt chunks -- chained on device
 * buffers through the attention library:
 *   embed -> per layer [RMSNorm -> Q,K,V projections -> RoPE(Q,K) -> K/V into
 *   the ColdStore-exact page pool (16-token pages) -> attention -> O
 *   projection -> residual add -> RMSNorm -> gate, up -> SwiGLU -> down ->
 *   residual add] -> RMSNorm -> LM head -> greedy token (first index on ties).
 * The reference drives one session per GpuLlm; a runner here holds
 * `max_batch` sequence slots whose decode steps run as one batch.
 * Every entry point returns 0 on success and -1 with mslim_model_last_error()
 * set on failure; calls on one runner are serialised by the caller. */
#ifndef MSLIM_MODEL_H
#define MSLIM_MODEL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Weight tensors per layer, in the order of the `weights` array below. */
#define MSLIM_MODEL_LAYER_TENSORS 9

/* K/V layouts (mslim_model_new's kv_layout).  PAGED: the ColdStore-exact pool
 * of 16-token head-major pages read by mslim_attn_decode_paged, as the
 * GPU-region runtime (GpuLlm::load_with_gpu_region_native_hip,
 * src/gpu_llm/mod.rs:299-306).  DENSE: token-major rows per slot read by
 * mslim_attn_decode_dense, as the Workspace cache of load_dense_native_hip
 * (mod.rs:308).  Both give bit-identical tokens, logits and K/V digests
 * (the reference's invariant, mod.rs:2993-3048). */
#define MSLIM_MODEL_KV_PAGED 0
#define MSLIM_MODEL_KV_DENSE 1

/* ModelSpec fields a layer uses (src/model_config.rs:22-42) and the RoPE
 * arguments of RopeKernelConfig (src/gpu_llm/kernels.rs:15-23). */
typedef struct {
    int layers, hidden, q_heads, kv_heads, head_dim, intermediate, vocab;
    float rms_eps, rope_theta;
    int llama3_scaling;
    float rope_factor, rope_low_freq_factor, rope_high_freq_factor, rope_original_max_position;
} mslim_model_spec;

const char *mslim_model_last_error(void);

/* A runner on an attention-library context (mslim_attn_ctx_new), which must
 * outlive it.  `weights` holds 3 + 9 * layers device BF16 pointers:
 *   [0] embedding [vocab][hidden], [1] final norm [hidden],
 *   [2] LM head [vocab][hidden] (the embedding when tied), then per layer
 *   input norm [hidden], q [q_heads*head_dim][hidden], k and v
 *   [kv_heads*head_dim][hidden], o [hidden][q_heads*head_dim], post norm
 *   [hidden], gate and up [intermediate][hidden], down [hidden][intermediate].
 * max_batch <= 64 slots, chunk_tokens <= 512 prompt tokens per causal chunk,
 * max_context tokens per slot, kv_layout MSLIM_MODEL_KV_*.  The runner
 * allocates its K/V pools and activations on the context's device.  Replaces
 * GpuLlm::load_dense_native_hip / load_with_gpu_region_native_hip
 * (src/gpu_llm/mod.rs:299-308) for weights already on the device. */
void *mslim_model_new(void *attn_ctx, const mslim_model_spec *spec, const void *const *weights,
                      int max_batch, int chunk_tokens, int max_context, int kv_layout);
void mslim_model_destroy(void *model);

/* Prompt of slot `seq` from position 0; *next_token = greedy token after the
 * prompt, not appended (GpuLlm::prefill_only, src/gpu_llm/mod.rs:2499-2570). */
int mslim_model_prefill(void *model, int seq, const int32_t *prompt, int tokens,
                        int32_t *next_token);

/* One token for each of slots 0..batch-1 at that slot's position
 * (GpuLlm::forward_token, src/gpu_llm/mod.rs:2457-2484, for a batch). */
int mslim_model_forward_batch(void *model, const int32_t *tokens, int batch,
                              int32_t *next_tokens);

/* Slot 0: prefill, then greedy tokens until max_new or an EOS id; out holds
 * max_new ids (GpuLlm::generate, src/gpu_llm/mod.rs:2571-2700). */
int mslim_model_generate(void *model, const int32_t *prompt, int tokens, int max_new,
                         const int32_t *eos_ids, int eos_count, int32_t *out, int *generated);

/* Tokens held by slot `seq`, or -1 (GpuLlm::position, mod.rs:1314). */
int64_t mslim_model_position(void *model, int seq);
/* Empty slot `seq` (GpuLlm::reset_session, mod.rs:1530-1577).  With a
 * ColdStore attached, deferred tokens are committed first and the slot
 * continues in a fresh store at <parent>/session-<pid>-<nonce> beside the old
 * directory, which keeps the finished session for a later restore. */
int mslim_model_reset(void *model, int seq);
/* BF16 bits of the last logits: 1 row after prefill, one per slot after a
 * batch step (GpuStep::logits, mod.rs:116-118). */
int mslim_model_logits(void *model, uint16_t *out, size_t capacity, int *rows);
/* PrefillSettings JSON (calibration_profile.rs:21-27: batch_tokens,
 * weight_reuse_tokens, attention) of the runner (GpuLlm::prefill_settings,
 * mod.rs:594-600); fails if it does not fit in `capacity` bytes. */
int mslim_model_prefill_settings(void *model, char *json_out, size_t capacity);
/* Validate and install PrefillSettings JSON while every slot is empty
 * (GpuLlm::set_calibration_prefill_settings, mod.rs:602-632): batch_tokens
 * becomes the prompt chunk (1 when null), up to the chunk_tokens the runner
 * was created with; experimental attention modes are rejected. */
int mslim_model_set_prefill_settings(void *model, const char *json);
/* GpuLlm::logical_kv_sha256 (mod.rs:1981-2028) of slot `seq`, hex with NUL. */
int mslim_model_logical_kv_sha256(void *model, int seq, char *hex_out);

/* ---- ColdStore-exact persistence (MSLIM_MODEL_KV_PAGED only) -------------- */

/* Give empty slot `seq` the canonical ColdStore <directory>/pages-exact.kv
 * (created, or opened with its committed records; GpuRegionConfig::
 * cold_directory of the GPU-region runtime, gpu_llm/mod.rs:299-306).  While
 * attached, mslim_model_prefill commits the prompt's K/V at its end
 * (gpu_llm/prefill.rs:760-790), decode steps defer their commit, and
 * mslim_model_flush_cold commits every token past the committed prefix
 * (flush_deferred_cold, gpu_llm/mod.rs:1614-1699).  A prefill into a slot
 * whose store already holds tokens fails: restore it instead. */
int mslim_model_attach_cold_store(void *model, int seq, const char *directory);
int mslim_model_detach_cold_store(void *model, int seq);
int mslim_model_flush_cold(void *model, int seq);
/* Deferred (1, the default) or immediate (0) commit of decode steps, the
 * reference's mslim_deferred_cold_commit switch: in immediate mode every
 * mslim_model_forward_batch commits each attached slot's new token before it
 * returns (gpu_llm/mod.rs:2162-2164); switching to it first commits what is
 * deferred. */
int mslim_model_set_deferred_cold_commit(void *model, int deferred);
/* Load the store's committed prefix of `tokens` tokens (every layer must hold
 * exactly that many) into empty slot `seq`, verifying every record on the
 * device (header, token hashes, checksums, SHA-256) before any byte reaches
 * the page pool; afterwards the slot continues at position `tokens`
 * (restore_session, gpu_llm/mod.rs:1335-1451).  A corrupt or incomplete
 * store fails and leaves the slot empty. */
int mslim_model_restore_session(void *model, int seq, int64_t tokens);
/* GpuRegionStore::logical_kv_sha256 (gpu_region_store.rs:341-371) of the
 * slot's ColdStore, read from the file: equal to mslim_model_logical_kv_
 * sha256 once every token is committed. */
int mslim_model_cold_logical_kv_sha256(void *model, int seq, char *hex_out);

/* Persistence figures of one slot (gpu_llm/mod.rs:192-208). */
typedef struct {
    int attached;
    int64_t committed_tokens;
    double prefill_seal_seconds;          /* last_prefill_cold_seal_seconds */
    double last_commit_seconds;           /* last_deferred_cold_commit_seconds */
    int64_t last_committed_token_layers;  /* last_deferred_cold_committed_token_layers */
    double last_restore_seconds;
} mslim_model_cold_info;
int mslim_model_cold_report(void *model, int seq, mslim_model_cold_info *out);
/* Directory of the slot's ColdStore ("" when none is attached), with NUL;
 * fails if it does not fit in `capacity` bytes. */
int mslim_model_cold_directory(void *model, int seq, char *out, size_t capacity);

/* ---- failure handling ----------------------------------------------------- */

/* Cooperative cancellation (the AtomicBool `cancel` of GpuLlm::prefill_only
 * and generate_cancellable, src/gpu_llm/mod.rs:2499-2700): `flag` points to a
 * caller-owned int32 (nonzero = cancel) that the runner reads, relaxed, at
 * every prompt chunk and layer boundary of a prefill (prefill_batched,
 * src/gpu_llm/prefill.rs:653-680) and at every token boundary of
 * mslim_model_forward_batch and mslim_model_generate.  A cancelled prefill
 * fails with "GPU batch prefill cancelled[ at layer boundary]" and poisons
 * its slot; a cancelled generation seals the turn's decoded prefix in an
 * attached ColdStore (mod.rs:2704-2712) and fails with "GPU generation
 * cancelled by client", leaving the slot usable.  NULL clears the flag. */
int mslim_model_set_cancel_flag(void *model, const int32_t *flag);
/* 1 when slot `seq` is poisoned, 0 when healthy, -1 on error.  A device step
 * that fails after its arguments were accepted (a library error, a failed
 * ColdStore commit, a prefill cancelled mid-prompt) poisons the slots it was
 * writing (every slot of a forward_batch); every later call that would use a
 * poisoned slot fails until mslim_model_reset(seq), which discards the
 * slot's K/V without committing them.  (The reference's poisoned GpuLlm,
 * src/gpu_llm/mod.rs:2462-2483, refuses even the reset; its worker is
 * restarted instead.) */
int mslim_model_poisoned(void *model, int seq);
/* Failure injection for failure-handling tests (no counterpart in the
 * reference): the next device step that reaches layer `layer` fails there,
 * once, with an argument error from the attention library (kind
 * MSLIM_MODEL_INJECT_ARGUMENT_ERROR) or as if the cancel flag had been raised
 * at that layer boundary of a prefill (kind MSLIM_MODEL_INJECT_CANCEL).
 * Kind 0 disarms. */
#define MSLIM_MODEL_INJECT_ARGUMENT_ERROR 1
#define MSLIM_MODEL_INJECT_CANCEL 2
int mslim_model_inject_failure(void *model, int kind, int layer);

#ifdef __cplusplus
}
#endif

#endif /* MSLIM_MODEL_H */
