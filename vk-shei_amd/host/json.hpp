// Minimal strict JSON reader/writer for the host configuration types (the
// role serde_json plays for AttentionKernelConfig).  Values: null, bool,
// number (kept as its text so integers round-trip exactly), string, array,
// object (insertion-ordered, duplicate keys rejected as serde does).
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <utility>
#include <vector>

namespace mslim {
namespace json {

struct Value {
    enum class Kind { Null, Bool, Number, String, Array, Object } kind = Kind::Null;
    bool boolean = false;
    std::string text;  // number literal or string contents
    std::vector<Value> items;
    std::vector<std::pair<std::string, Value>> members;

    const Value *find(const std::string &key) const;
    // Non-negative integer (serde usize): throws on sign, fraction, exponent
    // or overflow.
    uint64_t as_usize(const std::string &field) const;
};

// Parses one JSON document; throws mslim::Error with a serde-like message.
Value parse(const std::string &text);

std::string quote(const std::string &s);

}  // namespace json
}  // namespace mslim
