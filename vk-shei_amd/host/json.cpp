#include "json.hpp"

#include <cctype>

#include "native.hpp"

namespace mslim {
namespace json {

const Value *Value::find(const std::string &key) const {
    for (const auto &m : members)
        if (m.first == key) return &m.second;
    return nullptr;
}

uint64_t Value::as_usize(const std::string &field) const {
    ensure(kind == Kind::Number, "invalid type for `" + field + "`: expected usize");
    ensure(!text.empty() && text[0] != '-', "invalid value for `" + field + "`: expected usize");
    uint64_t v = 0;
    for (char c : text) {
        ensure(c >= '0' && c <= '9', "invalid type for `" + field + "`: floating point, expected usize");
        const uint64_t next = v * 10 + (uint64_t)(c - '0');
        ensure(next / 10 == v, "invalid value for `" + field + "`: out of range for usize");
        v = next;
    }
    return v;
}

namespace {

struct Parser {
    const std::string &s;
    size_t i = 0;

    [[noreturn]] void fail(const std::string &what) {
        throw Error(what + " at offset " + std::to_string(i));
    }
    void ws() {
        while (i < s.size() && (s[i] == ' ' || s[i] == '\n' || s[i] == '\r' || s[i] == '\t')) ++i;
    }
    bool eat(char c) {
        ws();
        if (i < s.size() && s[i] == c) { ++i; return true; }
        return false;
    }
    void expect(char c) {
        if (!eat(c)) fail(std::string("expected `") + c + "`");
    }
    bool literal(const char *word) {
        size_t n = 0;
        while (word[n]) ++n;
        if (s.compare(i, n, word) == 0) { i += n; return true; }
        return false;
    }

    std::string string_body() {
        std::string out;
        while (true) {
            if (i >= s.size()) fail("EOF while parsing a string");
            char c = s[i++];
            if (c == '"') return out;
            if ((unsigned char)c < 0x20) fail("control character in string");
            if (c != '\\') { out.push_back(c); continue; }
            if (i >= s.size()) fail("EOF in escape");
            c = s[i++];
            switch (c) {
                case '"': out.push_back('"'); break;
                case '\\': out.push_back('\\'); break;
                case '/': out.push_back('/'); break;
                case 'b': out.push_back('\b'); break;
                case 'f': out.push_back('\f'); break;
                case 'n': out.push_back('\n'); break;
                case 'r': out.push_back('\r'); break;
                case 't': out.push_back('\t'); break;
                case 'u': {
                    if (i + 4 > s.size()) fail("short unicode escape");
                    unsigned cp = 0;
                    for (int k = 0; k < 4; ++k) {
                        const char h = s[i++];
                        cp <<= 4;
                        if (h >= '0' && h <= '9') cp |= (unsigned)(h - '0');
                        else if (h >= 'a' && h <= 'f') cp |= (unsigned)(h - 'a' + 10);
                        else if (h >= 'A' && h <= 'F') cp |= (unsigned)(h - 'A' + 10);
                        else fail("bad unicode escape");
                    }
                    if (cp < 0x80) out.push_back((char)cp);
                    else if (cp < 0x800) {
                        out.push_back((char)(0xC0 | (cp >> 6)));
                        out.push_back((char)(0x80 | (cp & 0x3F)));
                    } else {
                        out.push_back((char)(0xE0 | (cp >> 12)));
                        out.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
                        out.push_back((char)(0x80 | (cp & 0x3F)));
                    }
                    break;
                }
                default: fail("invalid escape");
            }
        }
    }

    Value value() {
        ws();
        if (i >= s.size()) fail("EOF while parsing a value");
        Value v;
        const char c = s[i];
        if (c == '{') {
            ++i;
            v.kind = Value::Kind::Object;
            if (eat('}')) return v;
            do {
                ws();
                if (i >= s.size() || s[i] != '"') fail("key must be a string");
                ++i;
                std::string key = string_body();
                if (v.find(key)) fail("duplicate field `" + key + "`");
                expect(':');
                v.members.emplace_back(std::move(key), value());
            } while (eat(','));
            expect('}');
            return v;
        }
        if (c == '[') {
            ++i;
            v.kind = Value::Kind::Array;
            if (eat(']')) return v;
            do v.items.push_back(value());
            while (eat(','));
            expect(']');
            return v;
        }
        if (c == '"') {
            ++i;
            v.kind = Value::Kind::String;
            v.text = string_body();
            return v;
        }
        if (literal("true")) { v.kind = Value::Kind::Bool; v.boolean = true; return v; }
        if (literal("false")) { v.kind = Value::Kind::Bool; return v; }
        if (literal("null")) return v;
        // number: -?(0|[1-9][0-9]*)(\.[0-9]+)?([eE][+-]?[0-9]+)?
        const size_t start = i;
        if (s[i] == '-') ++i;
        if (i >= s.size() || !isdigit((unsigned char)s[i])) fail("expected value");
        if (s[i] == '0') ++i;
        else while (i < s.size() && isdigit((unsigned char)s[i])) ++i;
        if (i < s.size() && s[i] == '.') {
            ++i;
            if (i >= s.size() || !isdigit((unsigned char)s[i])) fail("invalid number");
            while (i < s.size() && isdigit((unsigned char)s[i])) ++i;
        }
        if (i < s.size() && (s[i] == 'e' || s[i] == 'E')) {
            ++i;
            if (i < s.size() && (s[i] == '+' || s[i] == '-')) ++i;
            if (i >= s.size() || !isdigit((unsigned char)s[i])) fail("invalid number");
            while (i < s.size() && isdigit((unsigned char)s[i])) ++i;
        }
        v.kind = Value::Kind::Number;
        v.text = s.substr(start, i - start);
        return v;
    }
};

}  // namespace

Value parse(const std::string &text) {
    Parser p{text};
    Value v = p.value();
    p.ws();
    if (p.i != text.size()) p.fail("trailing characters");
    return v;
}

std::string quote(const std::string &s) {
    std::string out = "\"";
    for (char c : s) {
        if (c == '"' || c == '\\') { out.push_back('\\'); out.push_back(c); }
        else if ((unsigned char)c < 0x20) {
            static const char *hex = "0123456789abcdef";
            out += "\\u00";
            out.push_back(hex[(c >> 4) & 0xF]);
            out.push_back(hex[c & 0xF]);
        } else out.push_back(c);
    }
    out.push_back('"');
    return out;
}

}  // namespace json
}  // namespace mslim
