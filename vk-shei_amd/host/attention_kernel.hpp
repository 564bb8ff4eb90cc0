// Bounded attention-kernel configuration (attention_kernel.rs:6-139): the
// same fields, JSON form, validation rules, error texts and identifiers, and
// the mapping of each mode onto the gfx950 kernels of libmslim_attn.
#pragma once

#include <cstddef>
#include <cstdint>
#include <optional>
#include <string>

#include "json.hpp"

namespace mslim {

// attention_kernel.rs:6-15; JSON names are snake_case (serde rename_all).
enum class AttentionKernelMode { Reference, StrictTiled, OnlineExperimental, SplitKvExperimental };

struct AttentionKernelConfig {
    AttentionKernelMode mode = AttentionKernelMode::Reference;
    size_t block_queries = 1;
    size_t block_keys = 64;
    size_t work_group = 64;
    size_t splits = 1;

    bool operator==(const AttentionKernelConfig &o) const {
        return mode == o.mode && block_queries == o.block_queries && block_keys == o.block_keys &&
               work_group == o.work_group && splits == o.splits;
    }
    bool operator!=(const AttentionKernelConfig &o) const { return !(*this == o); }

    // JSON with serde(default, deny_unknown_fields): missing fields keep their
    // default, unknown fields and wrongly typed values throw Error.
    static AttentionKernelConfig from_json(const std::string &text);
    static AttentionKernelConfig from_value(const json::Value &value);
    std::string to_json() const;

    bool experimental() const;                               // :37-42
    void validate() const;                                   // :43-80
    void check_snapshot(const json::Value *recorded) const;  // :82-94
    void validate_activation(bool allow_experimental) const; // :96-103
    std::string id() const;                                  // :104-113
    size_t local_bytes(size_t head_dim) const;               // :116-126
    size_t decode_scratch_bytes(size_t heads, size_t head_dim) const;  // :127-139

    // split_tokens argument of mslim_attn_decode_* for a single-query decode
    // over `history` tokens: split-KV asks for min(splits, history)
    // partitions (tiled_attention.rs:208-213), rounded to whole 64-token
    // units; every other mode leaves the split to the library (0).
    int decode_split_tokens(size_t history) const;
};

const char *mode_json_name(AttentionKernelMode mode);

// The prefill knobs a calibration profile may carry (calibration_profile.rs:
// 21-54): prompt tokens per causal chunk (none = one token at a time), GEMV
// weight reuse, and a bit-exact attention configuration.  On gfx950 the
// decoder runner's chunk is batch_tokens; weight reuse has no counterpart
// (a chunk's projections read each weight once whatever the reuse) and is
// kept for the profile identity.  The profile registry and its transactions
// stay with the caller.
struct PrefillSettings {
    std::optional<size_t> batch_tokens;
    size_t weight_reuse_tokens = 0;
    AttentionKernelConfig attention;

    bool operator==(const PrefillSettings &o) const {
        return batch_tokens == o.batch_tokens && weight_reuse_tokens == o.weight_reuse_tokens &&
               attention == o.attention;
    }
    // serde(deny_unknown_fields): `weight_reuse_tokens` required,
    // `batch_tokens` may be absent or null, `attention` defaults.
    static PrefillSettings from_json(const std::string &text);
    static PrefillSettings from_value(const json::Value &value);
    void validate() const;   // :29-40
    std::string id() const;  // :41-54
    std::string to_json() const;
    // Prompt tokens per runner chunk: batch_tokens, or 1 when sequential.
    int chunk_tokens() const { return batch_tokens ? (int)*batch_tokens : 1; }
};

}  // namespace mslim
