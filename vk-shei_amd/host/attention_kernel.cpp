#include "attention_kernel.hpp"

#include <cctype>

#include "native.hpp"

namespace mslim {

namespace {

struct ModeName {
    AttentionKernelMode mode;
    const char *json;   // serde snake_case
    const char *debug;  // Rust Debug name, used by id()
};
constexpr ModeName kModes[] = {
    {AttentionKernelMode::Reference, "reference", "Reference"},
    {AttentionKernelMode::StrictTiled, "strict_tiled", "StrictTiled"},
    {AttentionKernelMode::OnlineExperimental, "online_experimental", "OnlineExperimental"},
    {AttentionKernelMode::SplitKvExperimental, "split_kv_experimental", "SplitKvExperimental"},
};

const ModeName &mode_name(AttentionKernelMode m) {
    for (const auto &n : kModes)
        if (n.mode == m) return n;
    return kModes[0];
}

bool one_of(size_t v, std::initializer_list<size_t> allowed) {
    for (size_t a : allowed)
        if (v == a) return true;
    return false;
}

bool mul_ok(size_t a, size_t b, size_t *out) { return !__builtin_mul_overflow(a, b, out); }

}  // namespace

const char *mode_json_name(AttentionKernelMode mode) { return mode_name(mode).json; }

AttentionKernelConfig AttentionKernelConfig::from_json(const std::string &text) {
    return from_value(json::parse(text));
}

AttentionKernelConfig AttentionKernelConfig::from_value(const json::Value &value) {
    ensure(value.kind == json::Value::Kind::Object,
           "invalid type: expected struct AttentionKernelConfig");
    AttentionKernelConfig c;
    for (const auto &m : value.members) {
        const std::string &k = m.first;
        const json::Value &v = m.second;
        if (k == "mode") {
            ensure(v.kind == json::Value::Kind::String, "invalid type for `mode`: expected a string");
            bool found = false;
            for (const auto &n : kModes)
                if (v.text == n.json) { c.mode = n.mode; found = true; }
            ensure(found, "unknown variant `" + v.text +
                              "`, expected one of `reference`, `strict_tiled`, "
                              "`online_experimental`, `split_kv_experimental`");
        } else if (k == "block_queries") {
            c.block_queries = (size_t)v.as_usize(k);
        } else if (k == "block_keys") {
            c.block_keys = (size_t)v.as_usize(k);
        } else if (k == "work_group") {
            c.work_group = (size_t)v.as_usize(k);
        } else if (k == "splits") {
            c.splits = (size_t)v.as_usize(k);
        } else {
            throw Error("unknown field `" + k +
                        "`, expected one of `mode`, `block_queries`, `block_keys`, `work_group`, `splits`");
        }
    }
    return c;
}

std::string AttentionKernelConfig::to_json() const {
    return std::string("{\"mode\":") + json::quote(mode_json_name(mode)) +
           ",\"block_queries\":" + std::to_string(block_queries) +
           ",\"block_keys\":" + std::to_string(block_keys) +
           ",\"work_group\":" + std::to_string(work_group) + ",\"splits\":" + std::to_string(splits) +
           "}";
}

bool AttentionKernelConfig::experimental() const {
    return mode == AttentionKernelMode::OnlineExperimental ||
           mode == AttentionKernelMode::SplitKvExperimental;
}

void AttentionKernelConfig::validate() const {
    ensure(one_of(block_queries, {1, 2, 4}), "attention block_queries must be 1,2,4");
    ensure(one_of(block_keys, {32, 64, 128}), "attention block_keys must be 32,64,128");
    ensure(one_of(work_group, {32, 64, 128}), "attention work_group must be 32,64,128");
    ensure(splits >= 1 && splits <= 64, "attention splits must be 1..=64");
    if (mode == AttentionKernelMode::SplitKvExperimental)
        ensure(block_queries == 1 && splits >= 2,
               "split-KV requires one query per group and at least two splits");
    else
        ensure(splits == 1, "only explicit split-KV may request multiple splits");
    if (mode == AttentionKernelMode::Reference)
        ensure(*this == AttentionKernelConfig{}, "reference attention cannot carry ignored tuning values");
}

void AttentionKernelConfig::check_snapshot(const json::Value *recorded) const {
    // A snapshot without an attention record was taken before tiled kernels
    // existed: it compares as the default (reference) configuration.
    const AttentionKernelConfig r = recorded ? from_value(*recorded) : AttentionKernelConfig{};
    r.validate();
    ensure(*this == r, "snapshot attention numeric configuration mismatch");
}

void AttentionKernelConfig::validate_activation(bool allow_experimental) const {
    validate();
    ensure(!experimental() || allow_experimental,
           "experimental attention requires explicit numeric-contract opt-in");
}

std::string AttentionKernelConfig::id() const {
    if (mode == AttentionKernelMode::Reference) return "reference";
    std::string s = std::string(mode_name(mode).debug) + "-q" + std::to_string(block_queries) + "-k" +
                    std::to_string(block_keys) + "-wg" + std::to_string(work_group) + "-s" +
                    std::to_string(splits);
    for (char &ch : s) ch = (char)std::tolower((unsigned char)ch);
    return s;
}

size_t AttentionKernelConfig::local_bytes(size_t head_dim) const {
    validate();
    ensure(head_dim >= 1 && head_dim <= 256, "tiled attention head dimension must be 1..=256");
    return 2 * block_keys * head_dim + 2 * block_queries * head_dim + 4 * block_queries * block_keys +
           4 * block_queries * 4;
}

size_t AttentionKernelConfig::decode_scratch_bytes(size_t heads, size_t head_dim) const {
    validate();
    if (mode != AttentionKernelMode::SplitKvExperimental) return 0;
    size_t a = 0, b = 0, bytes = 0;
    const bool ok = mul_ok(heads, splits, &a) && head_dim <= SIZE_MAX - 2 && mul_ok(a, head_dim + 2, &b) &&
                    mul_ok(b, 4, &bytes);
    ensure(ok && bytes > 0 && bytes <= 16u * 1024 * 1024,
           "split-KV scratch exceeds its 16 MiB bound or overflows");
    return bytes;
}

int AttentionKernelConfig::decode_split_tokens(size_t history) const {
    if (mode != AttentionKernelMode::SplitKvExperimental || history == 0) return 0;
    const size_t parts = splits < history ? splits : history;
    const size_t per = (history + parts - 1) / parts;
    return (int)((per + 63) / 64 * 64);
}

// calibration_profile.rs:21-27 with serde's rules for this struct.
PrefillSettings PrefillSettings::from_json(const std::string &text) {
    return from_value(json::parse(text));
}

PrefillSettings PrefillSettings::from_value(const json::Value &value) {
    ensure(value.kind == json::Value::Kind::Object, "invalid type: expected struct PrefillSettings");
    PrefillSettings p;
    bool have_reuse = false;
    for (const auto &m : value.members) {
        const std::string &k = m.first;
        const json::Value &v = m.second;
        if (k == "batch_tokens") {
            if (v.kind == json::Value::Kind::Null) p.batch_tokens.reset();
            else p.batch_tokens = (size_t)v.as_usize(k);
        } else if (k == "weight_reuse_tokens") {
            p.weight_reuse_tokens = (size_t)v.as_usize(k);
            have_reuse = true;
        } else if (k == "attention") {
            p.attention = AttentionKernelConfig::from_value(v);
        } else {
            throw Error("unknown field `" + k +
                        "`, expected one of `batch_tokens`, `weight_reuse_tokens`, `attention`");
        }
    }
    ensure(have_reuse, "missing field `weight_reuse_tokens`");
    return p;
}

// calibration_profile.rs:29-40
void PrefillSettings::validate() const {
    attention.validate_activation(false);
    ensure(!batch_tokens || (*batch_tokens >= 1 && *batch_tokens <= 512), "prefill batch must be 1..=512");
    ensure(weight_reuse_tokens == 1 || weight_reuse_tokens == 8 || weight_reuse_tokens == 16 ||
               weight_reuse_tokens == 32,
           "prefill reuse must be 1,8,16,32");
}

std::string PrefillSettings::to_json() const {
    return std::string("{\"batch_tokens\":") + (batch_tokens ? std::to_string(*batch_tokens) : std::string("null")) +
           ",\"weight_reuse_tokens\":" + std::to_string(weight_reuse_tokens) + ",\"attention\":" +
           attention.to_json() + "}";
}

// calibration_profile.rs:41-54
std::string PrefillSettings::id() const {
    const std::string base = "batch-" + (batch_tokens ? std::to_string(*batch_tokens) : std::string("sequential")) +
                             "-reuse-" + std::to_string(weight_reuse_tokens);
    return attention == AttentionKernelConfig{} ? base : base + "-" + attention.id();
}

}  // namespace mslim
