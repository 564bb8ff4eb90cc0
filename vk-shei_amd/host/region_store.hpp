// Exact (epsilon = 0) GPU region store of the reference
// (gpu_region_store.rs:118-928): the per-layer token -> (ColdStore page,
// offset) table over a canonical ColdStore, the token-major <-> head-major
// page conversion, non-finite rejection on append, grouped partial reads and
// the logical K/V SHA-256, with the same argument meaning and error texts.
//
// The device page pool adds two batch paths the reference does through the
// host: seal_device_pages commits pages that live in the pool (the
// end-of-turn deferred commit, gpu_llm/mod.rs:1614-1699) with the record
// frames computed on the device, and restore_to_device loads a layer's
// committed pages into the pool and verifies every byte on the device
// (replacing read_values + per-chunk H2D, gpu_resources.rs:1017-1048).
//
// Not built: the positive-epsilon LOD selection (4-bit LSH axis, mass
// certificates, micro regions); a config with epsilon > 0 is rejected.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <optional>
#include <string>
#include <vector>

#include "cold_store.hpp"
#include "native.hpp"
#include "portable.hpp"

namespace mslim {
namespace region {

// gpu_region_store.rs:34-70
struct RegionConfig {
    double epsilon = 0.0;
    size_t stage_tokens = 64;
    std::optional<std::string> cold_directory;
    void validate() const;
};

// gpu_region_store.rs:72-100, the fields exact mode maintains.
struct RegionStats {
    size_t queries = 0;
    size_t exact_k_scores_computed_on_gpu = 0;
    size_t exact_v_tokens_read_from_cold = 0;
    size_t exact_v_tokens_skipped = 0;
    size_t exact_fallbacks = 0;
    size_t certificates_met = 0;
    double maximum_certified_error_bound = 0.0;
    size_t four_bit_index_payload_bytes = 0;
    uint64_t physical_cold_store_bytes = 0;
    size_t physical_cold_store_pages = 0;
    uint64_t cold_value_read_calls = 0;
    size_t prefill_batched_page_tokens = 0;
    size_t gpu_stage_tokens = 0;
    size_t device_sealed_pages = 0;
    size_t device_restored_pages = 0;
    bool shared_original_cpu_algorithms = true;
};

// gpu_region_store.rs:102-110
struct SelectionResult {
    std::vector<size_t> positions;
    std::vector<float> selected_mass_per_head;
    std::vector<double> bounds;
    size_t candidates_from_original_4bit_lsh = 0;
    size_t omitted = 0;
    double tolerance = 0.0;
};

// A device page pool [pool_pages][kv_heads][page_tokens][head_dim] BF16 for
// K and for V; page_tokens a power of two.
struct DevicePagePool {
    void *k_pool = nullptr;
    void *v_pool = nullptr;
    int64_t pool_pages = 0;
    int page_tokens = 16;
};

class RegionStore {
public:
    // gpu_region_store.rs:137-207: opens (and restores) or creates
    // <cold_directory>/pages-exact.kv, or a private temporary directory.
    RegionStore(portable::AttentionGeometry geometry, size_t layer_count, RegionConfig config);
    ~RegionStore();
    RegionStore(const RegionStore &) = delete;
    RegionStore &operator=(const RegionStore &) = delete;

    const RegionConfig &config() const { return config_; }
    portable::AttentionGeometry geometry() const { return geometry_; }
    size_t stage_tokens() const { return config_.stage_tokens; }
    cold::ColdStoreStats storage_metrics() const { return cold_.stats(); }
    const cold::ColdStore &cold_store() const { return cold_; }
    // Tokens observed for layer 0 (the length of the reference's context
    // axis, which observes layer-0 keys).
    size_t axis_token_len() const { return axis_tokens_; }
    size_t layer_tokens(size_t layer) const;
    const std::vector<double> &value_abs_max(size_t layer) const { return value_abs_max_.at(layer); }

    // gpu_region_store.rs:341-371 (hex digest)
    std::string logical_kv_sha256();
    // gpu_region_store.rs:376-384
    void append(size_t layer, size_t position, const uint8_t *key, const uint8_t *value, size_t token_bytes);
    // gpu_region_store.rs:391-520: token-major [n][kv_heads][head_dim] BF16.
    void append_batch(size_t layer, size_t position, const std::vector<uint8_t> &keys_token_major,
                      const std::vector<uint8_t> &values_token_major, size_t page_tokens);
    // gpu_region_store.rs:642-661
    SelectionResult select_dense_exact(size_t layer);
    // gpu_region_store.rs:828-927: token-major bytes of the given positions.
    std::vector<uint8_t> read_values(size_t layer, const std::vector<size_t> &positions);
    std::vector<uint8_t> read_keys(size_t layer, const std::vector<size_t> &positions);

    // Commit tokens [position, position + count) of `layer` from the device
    // pool as one ColdStore record per pool page.  `blocks[i]` is the pool
    // page of the sequence's logical page position / page_tokens + i.
    // position must equal layer_tokens(layer) and be a multiple of
    // page_tokens.  Values are checked like append_batch (V finite on every
    // layer, K finite on layer 0) before any record is committed.
    void seal_device_pages(NativeContext &ctx, size_t layer, size_t position, const DevicePagePool &pool,
                           const std::vector<int32_t> &blocks, size_t count);
    // Load every committed page of `layer` into the device pool at
    // blocks[token_start / page_tokens] and verify each record on the device
    // against its stored header, token hashes, checksums and SHA-256.  The
    // layer's records must each cover one aligned pool page.  On error the
    // pool pages written by this call hold unverified bytes.
    void restore_to_device(NativeContext &ctx, size_t layer, const DevicePagePool &pool,
                           const std::vector<int32_t> &blocks);

    RegionStats stats;

private:
    struct PageAddress {
        uint64_t page_id;
        size_t offset;
    };
    void restore_catalogue();
    std::vector<uint8_t> read_rows(size_t layer, const std::vector<size_t> &positions, bool key);

    RegionConfig config_;
    portable::AttentionGeometry geometry_;
    std::string temp_dir_;  // non-empty when the store owns a temporary directory
    cold::ColdStore cold_;
    std::vector<std::vector<PageAddress>> pages_;
    std::vector<std::vector<double>> value_abs_max_;
    size_t axis_tokens_ = 0;
};

}  // namespace region
}  // namespace mslim
