#include "portable.hpp"

#include <chrono>
#include <cmath>
#include <cstring>

#include "../csrc/sha256.hpp"

namespace mslim {
namespace portable {

namespace {

std::string display(PortableError::Kind kind, const std::string &m) {
    switch (kind) {
        case PortableError::Kind::InvalidGeometry: return "invalid geometry: " + m;
        case PortableError::Kind::ShapeMismatch: return "shape mismatch: " + m;
        case PortableError::Kind::NonFinite: return "non-finite computation: " + m;
        case PortableError::Kind::UnsupportedDevice: return "no native kernel registered for " + m;
        case PortableError::Kind::BackendFailure: return "backend failure: " + m;
    }
    return m;
}

[[noreturn]] void raise(PortableError::Kind k, const std::string &m) { throw PortableError(k, m); }

float bits_to_f32(uint32_t b) {
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}

float half_bits_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 31u, frac = h & 1023u;
    if (e == 0) return (h & 0x8000u ? -1.0f : 1.0f) * std::ldexp((float)frac, -24);
    if (e == 31) return bits_to_f32(sign | 0x7f800000u | (frac << 13));
    return bits_to_f32(sign | ((e - 15u + 127u) << 23) | (frac << 13));
}

}  // namespace

size_t bytes_per_element(FloatFormat f) { return f == FloatFormat::F32 ? 4 : 2; }

const char *label(FloatFormat f) {
    switch (f) {
        case FloatFormat::Bf16: return "BF16";
        case FloatFormat::F16: return "FP16";
        case FloatFormat::F32: return "FP32";
    }
    return "?";
}

int format_code(FloatFormat f) {
    switch (f) {
        case FloatFormat::Bf16: return MSLIM_ATTN_FORMAT_BF16;
        case FloatFormat::F16: return MSLIM_ATTN_FORMAT_F16;
        case FloatFormat::F32: return MSLIM_ATTN_FORMAT_F32;
    }
    return 0;
}

PortableError::PortableError(Kind kind, const std::string &message)
    : std::runtime_error(display(kind, message)), kind_(kind), message_(message) {}

// ---- RawTensor ---------------------------------------------------------
RawTensor RawTensor::from_le_bytes(FloatFormat dtype, std::vector<size_t> shape, std::vector<uint8_t> bytes) {
    size_t elements = 1;
    bool ok = !shape.empty();
    for (size_t d : shape) ok = ok && d > 0 && !__builtin_mul_overflow(elements, d, &elements);
    if (!ok) raise(PortableError::Kind::InvalidGeometry, "shape empty, zero-sized or overflowing");
    size_t expected = 0;
    if (__builtin_mul_overflow(elements, bytes_per_element(dtype), &expected))
        raise(PortableError::Kind::InvalidGeometry, "tensor byte count overflows");
    if (bytes.size() != expected)
        raise(PortableError::Kind::ShapeMismatch, "payload length differs from dtype*shape");
    return RawTensor(dtype, std::move(shape), std::make_shared<const std::vector<uint8_t>>(std::move(bytes)));
}

RawTensor RawTensor::from_f32(std::vector<size_t> shape, const std::vector<float> &data) {
    std::vector<uint8_t> bytes(data.size() * 4);
    if (!data.empty()) std::memcpy(bytes.data(), data.data(), bytes.size());
    return from_le_bytes(FloatFormat::F32, std::move(shape), std::move(bytes));
}

std::vector<float> RawTensor::decode_f32() const {
    const std::vector<uint8_t> &b = *bytes_;
    const size_t n = b.size() / bytes_per_element(dtype_);
    std::vector<float> out(n);
    for (size_t i = 0; i < n; ++i) {
        if (dtype_ == FloatFormat::F32) {
            const uint32_t u = (uint32_t)b[4 * i] | ((uint32_t)b[4 * i + 1] << 8) |
                               ((uint32_t)b[4 * i + 2] << 16) | ((uint32_t)b[4 * i + 3] << 24);
            out[i] = bits_to_f32(u);
        } else {
            const uint16_t h = (uint16_t)(b[2 * i] | (b[2 * i + 1] << 8));
            out[i] = dtype_ == FloatFormat::Bf16 ? bits_to_f32((uint32_t)h << 16) : half_bits_to_f32(h);
        }
    }
    return out;
}

// ---- AttentionGeometry ---------------------------------------------------
AttentionGeometry AttentionGeometry::create(size_t query_heads, size_t kv_heads, size_t head_dim) {
    size_t tmp = 0;
    if (query_heads == 0 || kv_heads == 0 || head_dim == 0 || query_heads % kv_heads != 0 ||
        __builtin_mul_overflow(query_heads, head_dim, &tmp) || __builtin_mul_overflow(kv_heads, head_dim, &tmp))
        raise(PortableError::Kind::InvalidGeometry,
              "heads and dimension must be positive, q_heads divisible by kv_heads, products finite");
    AttentionGeometry g;
    g.query_heads = query_heads;
    g.kv_heads = kv_heads;
    g.head_dim = head_dim;
    return g;
}

size_t AttentionGeometry::kv_head_for_query(size_t query_head) const {
    if (query_head >= query_heads) raise(PortableError::Kind::ShapeMismatch, "query head out of range");
    return query_head / (query_heads / kv_heads);
}

// ---- ExactKvFrames -------------------------------------------------------
void ExactKvFrames::append(RawTensor key, RawTensor value) {
    auto matches = [&](const std::vector<size_t> &s) {
        return s.size() == 3 && s[1] == geometry_.kv_heads && s[2] == geometry_.head_dim;
    };
    if (!matches(key.shape()) || key.shape() != value.shape())
        raise(PortableError::Kind::ShapeMismatch, "KV frame needs [tokens, kv_heads, head_dim]");
    size_t tokens = 0;
    if (__builtin_add_overflow(tokens_, key.shape()[0], &tokens))
        raise(PortableError::Kind::InvalidGeometry, "token count overflow");
    frames_.emplace_back(std::move(key), std::move(value));
    tokens_ = tokens;
}

size_t ExactKvFrames::payload_bytes() const {
    size_t n = 0;
    for (const auto &f : frames_) n += f.first.len_bytes() + f.second.len_bytes();
    return n;
}

std::string ExactKvFrames::digest_sha256() const {
    Sha256 h;
    static const char tag[] = "mslim-portable-exact-kv-v1";
    h.update(tag, sizeof tag - 1);
    auto put_u64 = [&](uint64_t v) {
        uint8_t le[8];
        for (int i = 0; i < 8; ++i) le[i] = (uint8_t)(v >> (8 * i));
        h.update(le, 8);
    };
    for (size_t n : {geometry_.query_heads, geometry_.kv_heads, geometry_.head_dim, tokens_}) put_u64(n);
    for (const auto &f : frames_) {
        for (const RawTensor *t : {&f.first, &f.second}) {
            const uint8_t code = (uint8_t)format_code(t->dtype());
            h.update(&code, 1);
            for (size_t d : t->shape()) put_u64(d);
            h.update(t->as_le_bytes().data(), t->len_bytes());
        }
    }
    uint8_t digest[32];
    h.finish(digest);
    static const char *hex = "0123456789abcdef";
    std::string out;
    for (uint8_t b : digest) {
        out.push_back(hex[b >> 4]);
        out.push_back(hex[b & 15]);
    }
    return out;
}

std::vector<float> ExactKvFrames::decode(const AttentionBackend &backend, const std::vector<float> &query) const {
    return backend.decode(*this, query);
}

// ---- GpuBackend ------------------------------------------------------------
GpuBackend::GpuBackend() {
    try {
        ctx_ = NativeContext::create();
    } catch (const NativeError &e) {
        raise(PortableError::Kind::UnsupportedDevice, e.details());
    }
    mslim_attn_device_info d{};
    ctx_->check("device info", mslim_attn_get_device_info(ctx_->handle(), &d));
    info_.name = d.name;
    info_.vendor = d.vendor;
    info_.arch = d.arch;
    info_.driver_version = std::to_string(d.driver_version);
    info_.max_compute_units = d.compute_units;
    info_.reported_global_memory_bytes = d.global_memory_bytes;
    info_.max_allocation_bytes = d.max_allocation_bytes;
}

std::optional<GpuTimings> GpuBackend::last_timings() const {
    std::lock_guard<std::mutex> g(timings_mutex_);
    return last_;
}

std::vector<float> GpuBackend::decode(const ExactKvFrames &cache, const std::vector<float> &query) const {
    const AttentionGeometry g = cache.geometry();
    if (query.size() != g.query_elements()) raise(PortableError::Kind::ShapeMismatch, "GPU Q shape");
    for (float v : query)
        if (!std::isfinite(v)) raise(PortableError::Kind::NonFinite, "GPU Q");
    if (cache.is_empty()) return std::vector<float>(query.size(), 0.0f);

    const FloatFormat kf = cache.frames()[0].first.dtype();
    const FloatFormat vf = cache.frames()[0].second.dtype();
    std::vector<uint8_t> kraw, vraw;
    kraw.reserve(cache.payload_bytes() / 2);
    vraw.reserve(cache.payload_bytes() / 2);
    for (const auto &f : cache.frames()) {
        if (f.first.dtype() != kf || f.second.dtype() != vf)
            raise(PortableError::Kind::BackendFailure, "GPU backend requires uniform K and V formats across frames");
        kraw.insert(kraw.end(), f.first.as_le_bytes().begin(), f.first.as_le_bytes().end());
        vraw.insert(vraw.end(), f.second.as_le_bytes().begin(), f.second.as_le_bytes().end());
    }
    std::vector<float> out(query.size());
    mslim_attn_timings t{};
    int rc;
    {
        std::lock_guard<std::mutex> lock(ctx_->mutex());
        rc = mslim_attn_backend_decode(ctx_->handle(), query.data(), kraw.data(), format_code(kf), vraw.data(),
                                       format_code(vf), (int64_t)cache.tokens(), (int)g.query_heads,
                                       (int)g.kv_heads, (int)g.head_dim, out.data(), &t);
    }
    if (rc == MSLIM_ATTN_ERR_NONFINITE) {
        const std::string what = mslim_attn_last_error();
        raise(PortableError::Kind::NonFinite, what.find("GPU Q") != std::string::npos ? "GPU Q" : "GPU output");
    }
    if (rc != 0) raise(PortableError::Kind::BackendFailure, "GPU decode: " + std::string(mslim_attn_last_error()));
    {
        std::lock_guard<std::mutex> lock(timings_mutex_);
        GpuTimings gt;
        gt.dispatch_ms = t.dispatch_ms;
        gt.kernel_ms = t.kernel_ms;
        gt.input_kv_bytes = (size_t)t.input_kv_bytes;
        gt.scratch_bytes = (size_t)t.scratch_bytes;
        gt.output_bytes = (size_t)t.output_bytes;
        last_ = gt;
    }
    return out;
}

}  // namespace portable
}  // namespace mslim
