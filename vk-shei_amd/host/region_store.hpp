// Exact (epsilon = 0) GPU region store of the reference
// (gpu_region_store.rs:118-928): the per-layer token -> (ColdStore page,
// offset) table over a canonical ColdStore, the token-major <-> head-major
// page conversion, non-finite rejection on append, grouped partial reads and
// the logical K/V SHA-256, with the same argument meaning and error texts.
//
// The device page pool adds two batch paths the reference does through the
// host: seal_device_layers commits pages that live in the pool (the
// end-of-turn deferred commit, gpu_llm/mod.rs:1614-1699, and the prefill
// seal, gpu_llm/prefill.rs:760-790) with the record frames computed on the
// device, and restore_device_layers verifies committed records on the
// device and loads them into the pool (restore_session, gpu_llm/mod.rs:
// 1335-1451, replacing read_values + per-chunk H2D, gpu_resources.rs:
// 1017-1048).
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

// Staging of the device seal and restore paths, reused across calls: device
// buffers for record descriptors, frames and compacted payloads, and
// page-locked host buffers that the copies move by DMA.  Grown on demand,
// freed with the object; the context must outlive it.
class DeviceStaging {
public:
    explicit DeviceStaging(NativeContext &ctx) : ctx_(ctx) {}
    ~DeviceStaging();
    DeviceStaging(const DeviceStaging &) = delete;
    DeviceStaging &operator=(const DeviceStaging &) = delete;
    NativeContext &ctx() { return ctx_; }
    // Room for `records` records of `frame_slot` frame bytes and
    // `payload_bytes` bytes of K (and of V) each.
    void reserve(size_t records, size_t frame_slot, size_t payload_bytes);

    void *d_desc = nullptr, *d_frames = nullptr, *d_k = nullptr, *d_v = nullptr;
    uint8_t *h_desc = nullptr, *h_frames = nullptr, *h_k = nullptr, *h_v = nullptr;

private:
    void grow(size_t &cap, size_t bytes, void **dev, uint8_t **host);
    NativeContext &ctx_;
    size_t desc_cap_ = 0, frames_cap_ = 0, payload_cap_ = 0;
};

// Pool pages of one layer for the multi-layer device paths: blocks[i] is the
// pool page that holds the sequence's logical page i (token i * page_tokens
// onward).
struct LayerBlocks {
    size_t layer;
    std::vector<int32_t> blocks;
};

// Device seals of fewer records than this frame them on the host (see
// RegionStore::seal_device_layers).  Measured on MI355X with 16 host threads,
// 64 KiB records (8 kv heads x 16 tokens x 128 dims), whole seal wall time,
// device framing / host framing: 32 records 5.2 / 1.2 ms, 256: 7.6 / 6.4 ms,
// 512: 11.1 / 12.7 ms, 4096: 59.7 / 105.2 ms.
constexpr size_t kHostFramingRecords = 384;

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
    size_t layer_count() const { return pages_.size(); }
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
    // pool as one ColdStore record per pool page (or part of one).
    // `blocks[i]` is the pool page of the sequence's logical page
    // position / page_tokens + i.  position must equal layer_tokens(layer).
    // Values are checked like append_batch (V finite on every layer, K
    // finite on layer 0) before any record is committed.  One layer of
    // seal_device_layers, with staging of its own.
    void seal_device_pages(NativeContext &ctx, size_t layer, size_t position, const DevicePagePool &pool,
                           const std::vector<int32_t> &blocks, size_t count);
    // Load every committed page of `layer` into the device pool at
    // blocks[token_start / page_tokens] after verifying each record on the
    // device against its stored header, token hashes, checksums and SHA-256;
    // a corrupt record leaves the pool untouched.  One layer of
    // restore_device_layers, with staging of its own.
    void restore_to_device(NativeContext &ctx, size_t layer, const DevicePagePool &pool,
                           const std::vector<int32_t> &blocks);

    // Commit tokens [position, position + count) of every listed layer from
    // the device pool in few launches: the end-of-turn deferred commit
    // (gpu_llm/mod.rs:1614-1699) and the prefill seal (gpu_llm/prefill.rs:
    // 760-790) of a whole model.  position must equal each layer's
    // layer_tokens; it need not be a page boundary (the first record then
    // starts inside its pool page).  One record per pool page or part of
    // one, layers in order, so the file holds the records the reference's
    // per-layer append_batch writes for 16-token pages.  Layers are staged in
    // groups of at most `max_group_bytes` of payload; each group is checked
    // (V finite on every layer, K finite on layer 0) before any of its
    // records is committed, as append_batch checks each layer.
    // A group of fewer than host_framing_below() records is framed on the
    // host (header, token hashes, checksums and SHA-256 of each record from
    // the payloads read back anyway, records on parallel threads, SHA-NI
    // where the CPU has it) instead of by mslim_attn_record_frames, whose
    // serial SHA-256 chain per record gives each launch a floor of about
    // 4 ms; both write the same bytes.
    void seal_device_layers(DeviceStaging &staging, size_t position, size_t count, const DevicePagePool &pool,
                            const std::vector<LayerBlocks> &layers, size_t max_group_bytes = (size_t)256 << 20);
    size_t host_framing_below() const { return host_framing_below_; }
    void set_host_framing_below(size_t records) { host_framing_below_ = records; }
    // Load every committed record of the listed layers into the pool and
    // verify each on the device (header, token hashes, checksums, SHA-256)
    // from its staged copy BEFORE any byte reaches the pool: a corrupt store
    // leaves the pool untouched.  Each record must lie within one pool page.
    // Returns the number of records moved.
    size_t restore_device_layers(DeviceStaging &staging, const DevicePagePool &pool,
                                 const std::vector<LayerBlocks> &layers);

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
    size_t host_framing_below_ = kHostFramingRecords;
    std::string temp_dir_;  // non-empty when the store owns a temporary directory
    cold::ColdStore cold_;
    std::vector<std::vector<PageAddress>> pages_;
    std::vector<std::vector<double>> value_abs_max_;
    size_t axis_tokens_ = 0;
};

}  // namespace region
}  // namespace mslim
