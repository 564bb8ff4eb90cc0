// Llama-style decoder over the gfx950 library: the per-layer order of the
// reference GPU runtime (run_layer, gpu_llm/mod.rs:2056-2350; run_batch_layer,
// gpu_llm/prefill.rs:897-1061) chained through the C ABI on device buffers:
//   embed -> per layer [RMSNorm -> Q,K,V projections -> RoPE(Q,K) -> K/V into
//   the ColdStore-exact page pool -> attention -> O projection -> add ->
//   RMSNorm -> gate, up -> SwiGLU -> down -> add] -> RMSNorm -> LM head ->
//   greedy token (first index on ties).
// A runner holds `max_batch` sequence slots.  Prefill runs one slot's prompt
// in causal chunks of up to `chunk_tokens` (prefill_batched, mod.rs:2499-2570);
// decode runs one token for each of slots 0..B-1, each at its own position,
// over every layer's K/V in the chosen layout.  Weights are device BF16 buffers owned by
// the caller, row-major [out][in] as tv_hip_matrix_multiply expects.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "attention_kernel.hpp"
#include "native.hpp"
#include "region_store.hpp"

namespace mslim {
namespace model {

// The ModelSpec fields a layer uses (model_config.rs:22-42; RoPE arguments as
// RopeKernelConfig, gpu_llm/kernels.rs:15-23).
struct ModelSpec {
    int layers = 0, hidden = 0, q_heads = 0, kv_heads = 0, head_dim = 0, intermediate = 0, vocab = 0;
    float rms_eps = 1e-5f, rope_theta = 500000.0f;
    int llama3 = 0;
    float rope_factor = 1.0f, rope_low = 1.0f, rope_high = 2.0f, rope_original_max = 1.0f;
    void validate() const;
};

struct LayerWeights {
    const void *input_norm = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr;
    const void *post_norm = nullptr, *gate = nullptr, *up = nullptr, *down = nullptr;
};

struct ModelWeights {
    const void *embed = nullptr;  // [vocab][hidden]
    std::vector<LayerWeights> layers;
    const void *final_norm = nullptr;
    const void *lm_head = nullptr;  // [vocab][hidden]; the embedding when tied
};

// GpuStep (gpu_llm/mod.rs:112-119) without the timing field.
struct Step {
    int32_t argmax_token = 0;
    int64_t position = 0;  // tokens of the slot after this step
};

// Where a runner keeps K/V: the ColdStore-exact pool of 16-token head-major
// pages behind a page table (the GPU-region route, load_with_gpu_region_
// native_hip, gpu_llm/mod.rs:299-306), or dense token-major rows per slot
// (the Workspace cache of load_dense_native_hip, mod.rs:308).  The two give
// bit-identical tokens and logits, the reference's invariant of
// mod.rs:2993-3048.
enum class KvLayout { Paged = 0, Dense = 1 };

// ColdStore persistence of one slot: the reference's last_prefill_cold_seal_
// seconds, last_deferred_cold_commit_seconds and last_deferred_cold_committed_
// token_layers (gpu_llm/mod.rs:192-208, :1696-1697) and the committed
// length.
struct ColdReport {
    bool attached = false;
    int64_t committed_tokens = 0;    // tokens of every layer in the ColdStore
    double prefill_seal_seconds = 0.0;
    double last_commit_seconds = 0.0;
    int64_t last_committed_token_layers = 0;
    double last_restore_seconds = 0.0;
};

// Sequence slots per runner: every decode step's launch tables then travel in
// the kernel arguments (no host-to-device copy inside a step).
constexpr int kMaxSlots = 64;

class DecoderRunner {
public:
    static constexpr int kPageTokens = 16;
    DecoderRunner(std::shared_ptr<NativeContext> ctx, ModelSpec spec, ModelWeights weights, int max_batch,
                  int chunk_tokens, int max_context, KvLayout layout = KvLayout::Paged);
    ~DecoderRunner();
    DecoderRunner(const DecoderRunner &) = delete;
    DecoderRunner &operator=(const DecoderRunner &) = delete;

    // Prompt of slot `seq` from position 0 (prefill_only, mod.rs:2499-2570):
    // the greedy token after the prompt, not appended.
    Step prefill_only(int seq, const std::vector<int32_t> &prompt);
    // One token for each slot 0..tokens.size()-1 at that slot's position
    // (forward_token, mod.rs:2457-2484, for a batch of sessions).
    std::vector<Step> forward_batch(const std::vector<int32_t> &tokens);
    // prefill_only, then greedy steps until max_new tokens or an EOS id
    // (generate_cancellable, mod.rs:2587-2700).  Returns the generated tokens.
    std::vector<int32_t> generate(int seq, const std::vector<int32_t> &prompt, int max_new,
                                  const std::vector<int32_t> &eos_ids);
    // Empty slot `seq`.  With a ColdStore attached, deferred tokens are
    // committed first and the slot continues in a fresh store at
    // <parent>/session-<pid>-<nonce> beside the old directory
    // (reset_session, gpu_llm/mod.rs:1530-1577).
    void reset(int seq);
    // BF16 logits of the last prefill (1 row) or forward_batch (one row per
    // slot), as raw bits.
    std::vector<uint16_t> last_logits() const;
    int64_t position(int seq) const { return positions_.at(seq); }
    int max_batch() const { return max_batch_; }
    // GpuLlm::logical_kv_sha256 (mod.rs:1981-2028) of one slot, read from the
    // K/V pools.
    std::string logical_kv_sha256(int seq) const;
    const ModelSpec &spec() const { return spec_; }
    // GpuLlm::prefill_settings / set_calibration_prefill_settings
    // (gpu_llm/mod.rs:594-632): the prompt chunk is batch_tokens (1 when
    // sequential); new settings are validated and installed only while every
    // slot is empty, and the chunk may not exceed the one the runner was
    // built for.
    PrefillSettings prefill_settings() const { return settings_; }
    void set_calibration_prefill_settings(const PrefillSettings &settings);

    // ColdStore-exact persistence (paged layout only).  attach_cold_store
    // gives slot `seq` a canonical ColdStore at <directory>/pages-exact.kv
    // (the GPU-region runtime's GpuRegionConfig::cold_directory,
    // gpu_llm/mod.rs:299-306), opening the records already there.  With a
    // store attached, prefill_only commits the prompt's K/V at its end (the
    // prefill seal, gpu_llm/prefill.rs:760-790) and decode steps defer their
    // commit; flush_cold commits every token past the committed prefix (the
    // end-of-turn flush_deferred_cold, mod.rs:1614-1699).  restore_session
    // loads a store's committed prefix of `tokens` tokens into an empty slot
    // after verifying every record on the device (restore_session,
    // mod.rs:1335-1451).  The slot's ColdStore digest is
    // cold_logical_kv_sha256 (gpu_region_store.rs:341-371).
    void attach_cold_store(int seq, const std::string &directory);
    void detach_cold_store(int seq);
    void flush_cold(int seq);
    void restore_session(int seq, int64_t tokens);
    std::string cold_logical_kv_sha256(int seq);
    ColdReport cold_report(int seq) const;
    // Directory of the slot's ColdStore; empty when none is attached.
    std::string cold_directory(int seq) const;
    // Deferred (default) or immediate commit of decode steps: the reference's
    // mslim_deferred_cold_commit switch.  Immediate mode commits each step's
    // K/V before forward_batch returns (gpu_llm/mod.rs:2162-2164); switching
    // to it first commits what is deferred.
    void set_deferred_cold_commit(bool deferred);

    // Cooperative cancellation: a caller-owned flag (nonzero = cancel), read
    // at every prompt chunk and layer boundary of a prefill
    // (prefill_batched, gpu_llm/prefill.rs:653-680) and at every token
    // boundary of forward_batch and generate (generate_cancellable,
    // gpu_llm/mod.rs:2587-2700).  nullptr clears it.
    void set_cancel_flag(const int32_t *flag) { cancel_ = flag; }
    // A slot whose device step failed after its arguments were accepted
    // (a library error, a failed commit, or a prefill cancelled mid-prompt)
    // holds K/V written for some layers only.  It is poisoned and every call
    // that would use it fails until reset(seq), which discards its K/V
    // (the reference's poisoned runtime, gpu_llm/mod.rs:2462-2483, refuses
    // even the reset and is restarted instead).  A cancellation at a token
    // boundary leaves the slot consistent and does not poison it.
    bool poisoned(int seq) const;
    // Failure injection for the failure-handling tests: the next device step
    // that reaches layer `layer` fails there, once, with an argument error
    // from the attention library (kInjectArgumentError) or as if the cancel
    // flag had been raised (kInjectCancel).
    static constexpr int kInjectArgumentError = 1, kInjectCancel = 2;
    void inject_failure(int kind, int layer);

private:
    // Throws the prefill cancellation error when the flag is raised (or an
    // injected cancel is due at `layer`).
    void check_cancel(const char *where, int layer);
    void injected_error(int layer);
    void check_healthy(int seq) const;
    void *alloc(size_t bytes);
    void chunk(int seq, const int32_t *ids, int n, int64_t prior);
    // The page pool of every layer (one allocation each for K and V) and the
    // pool pages of slot `seq` per layer, for the ColdStore device paths.
    region::DevicePagePool all_layer_pool() const;
    std::vector<region::LayerBlocks> slot_blocks(int seq) const;
    void seal_slot(int seq, int64_t from, int64_t to);
    void head(const uint16_t *rows_in, int rows);
    void mlp(const LayerWeights &w, int n);
    const int32_t *table_row(int seq) const { return table_ + (int64_t)seq * pages_per_seq_; }
    // Dense layout: token-major rows of slot `seq` in a layer pool.
    const uint16_t *dense_rows(const void *pool, int seq) const {
        return static_cast<const uint16_t *>(pool) + (size_t)seq * max_context_ * spec_.kv_heads * spec_.head_dim;
    }

    std::shared_ptr<NativeContext> ctx_;
    ModelSpec spec_;
    ModelWeights w_;
    KvLayout layout_;
    int max_batch_, chunk_tokens_, max_context_, page_tokens_, pages_per_seq_, rows_cap_;
    float scale_;
    PrefillSettings settings_;
    std::vector<int64_t> positions_;
    std::vector<void *> owned_;
    std::vector<void *> k_pools_, v_pools_;  // layer l: k_base_ + l * layer pool bytes
    void *k_base_ = nullptr, *v_base_ = nullptr;
    std::vector<int32_t> host_table_;          // copy of the device page table
    std::vector<std::unique_ptr<region::RegionStore>> cold_;
    std::vector<ColdReport> cold_report_;
    std::unique_ptr<region::DeviceStaging> staging_;
    bool deferred_cold_ = true;
    const int32_t *cancel_ = nullptr;
    std::vector<char> poisoned_;
    int inject_kind_ = 0, inject_layer_ = -1;
    int32_t *table_ = nullptr, *ids_ = nullptr, *pos_ = nullptr, *next_ = nullptr;
    uint16_t *x_ = nullptr, *q_ = nullptr, *k_ = nullptr, *v_ = nullptr, *qr_ = nullptr,
             *kr_ = nullptr, *attn_ = nullptr, *act_ = nullptr,
             *kd_ = nullptr, *vd_ = nullptr, *logits_ = nullptr;
    int logits_rows_ = 0;
};

}  // namespace model
}  // namespace mslim
