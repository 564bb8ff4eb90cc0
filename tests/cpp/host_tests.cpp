// Tests of the C++ host layer (vk-shei_amd/host) written after the
// reference's own Rust tests: attention_kernel.rs:143-206,
// tests/tiled_attention_policy.rs, portable.rs:661-825 and
// gpu_backend.rs:379-469.  Cases named gpu_* need an MI355X; the others run
// on the CPU.  The CPU oracle (oracle/) is the checker.
//
//   host_tests --list        print every case name
//   host_tests NAME...       run the named cases (all when none given)
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <limits>
#include <string>
#include <vector>

#include "../../oracle/oracle.h"
#include "harness.hpp"
#include "../../vk-shei_amd/host/attention_kernel.hpp"
#include "../../vk-shei_amd/host/portable.hpp"
#include "../../vk-shei_amd/host/tiled_attention.hpp"

using namespace mslim;
using namespace mslim::portable;

namespace {

using harness::expect_throw;
using harness::Failure;

template <class F>
PortableError::Kind expect_portable(F f) {
    try {
        f();
    } catch (const PortableError &e) {
        return e.kind();
    }
    throw Failure("expected a PortableError");
}

uint16_t f16_bits(float x);  // test encoder, defined with the GPU cases

// ---- AttentionKernelConfig (attention_kernel.rs:143-206) ---------------
TEST(config_default_is_reference_and_experimental_opt_in_is_mandatory) {
    CHECK(AttentionKernelConfig::from_json("{}") == AttentionKernelConfig{});
    AttentionKernelConfig c;
    c.mode = AttentionKernelMode::OnlineExperimental;
    expect_throw<Error>([&] { c.validate_activation(false); });
    c.validate_activation(true);
}

TEST(config_reject_ignored_or_unbounded_configuration) {
    std::vector<AttentionKernelConfig> bad(5);
    bad[0].work_group = 0;
    bad[1].block_keys = 33;
    bad[2].splits = 2;
    bad[3].mode = AttentionKernelMode::StrictTiled;
    bad[3].splits = 2;
    bad[4].mode = AttentionKernelMode::SplitKvExperimental;
    bad[4].splits = 65;
    for (const auto &c : bad) expect_throw<Error>([&] { c.validate(); });
    const std::string msg = expect_throw<Error>([] { AttentionKernelConfig::from_json(R"({"epsilon":0.1})"); });
    CHECK(msg.find("unknown field `epsilon`") != std::string::npos);
}

TEST(config_scratch_is_bounded_and_strict_has_no_global_scores) {
    AttentionKernelConfig c;
    c.mode = AttentionKernelMode::StrictTiled;
    CHECK(c.decode_scratch_bytes(32, 128) == 0);
    CHECK(c.local_bytes(128) < 64 * 1024);
    AttentionKernelConfig split;
    split.mode = AttentionKernelMode::SplitKvExperimental;
    split.splits = 8;
    CHECK(split.decode_scratch_bytes(32, 128) == 32 * 8 * 130 * 4);
    expect_throw<Error>([&] { split.decode_scratch_bytes(std::numeric_limits<size_t>::max(), 128); });
}

TEST(config_validation_messages_and_local_bytes) {
    AttentionKernelConfig c;
    c.mode = AttentionKernelMode::StrictTiled;
    c.block_queries = 3;
    CHECK(expect_throw<Error>([&] { c.validate(); }) == "attention block_queries must be 1,2,4");
    c.block_queries = 2;
    c.block_keys = 128;
    // 2*BN*D + 2*BM*D + 4*BM*BN + 16*BM (attention_kernel.rs:116-126)
    CHECK(c.local_bytes(64) == 2 * 128 * 64 + 2 * 2 * 64 + 4 * 2 * 128 + 16 * 2);
    CHECK(expect_throw<Error>([&] { c.local_bytes(257); }) == "tiled attention head dimension must be 1..=256");
    AttentionKernelConfig split;
    split.mode = AttentionKernelMode::SplitKvExperimental;
    split.splits = 2;
    split.block_queries = 2;
    CHECK(expect_throw<Error>([&] { split.validate(); }) ==
          "split-KV requires one query per group and at least two splits");
    AttentionKernelConfig ref;
    ref.block_keys = 128;
    CHECK(expect_throw<Error>([&] { ref.validate(); }) == "reference attention cannot carry ignored tuning values");
}

TEST(config_snapshots_cannot_cross_numeric_contracts) {
    // tests/tiled_attention_policy.rs:26-46
    const AttentionKernelConfig reference;
    reference.check_snapshot(nullptr);
    AttentionKernelConfig strict = reference, online = reference;
    strict.mode = AttentionKernelMode::StrictTiled;
    online.mode = AttentionKernelMode::OnlineExperimental;
    expect_throw<Error>([&] { strict.check_snapshot(nullptr); });
    const json::Value online_json = json::parse(online.to_json());
    expect_throw<Error>([&] { reference.check_snapshot(&online_json); });
    const json::Value strict_json = json::parse(strict.to_json());
    strict.check_snapshot(&strict_json);
}

TEST(config_ids_and_json_form) {
    AttentionKernelConfig c;
    CHECK(c.id() == "reference");
    c.mode = AttentionKernelMode::StrictTiled;
    CHECK(c.id() == "stricttiled-q1-k64-wg64-s1");
    c.mode = AttentionKernelMode::SplitKvExperimental;
    c.splits = 8;
    c.block_keys = 128;
    CHECK(c.id() == "splitkvexperimental-q1-k128-wg64-s8");
    CHECK(c.to_json() ==
          R"({"mode":"split_kv_experimental","block_queries":1,"block_keys":128,"work_group":64,"splits":8})");
    CHECK(AttentionKernelConfig::from_json(c.to_json()) == c);
    CHECK(AttentionKernelConfig::from_json(R"({"mode":"online_experimental","block_keys":32})").block_keys == 32);
    for (const char *bad : {R"({"splits":-1})", R"({"splits":1.5})", R"({"mode":"fast"})", R"({"mode":1})",
                            R"({"splits":2,"splits":3})", R"([])", R"({"splits":99999999999999999999999})"})
        expect_throw<Error>([&] { AttentionKernelConfig::from_json(bad); });
}

TEST(prefill_settings_legacy_profile_retains_reference_and_id) {
    // tests/tiled_attention_policy.rs:5-12
    const PrefillSettings s = PrefillSettings::from_json(R"({"batch_tokens":64,"weight_reuse_tokens":8})");
    CHECK(s.attention == AttentionKernelConfig{});
    CHECK(s.id() == "batch-64-reuse-8");
    s.validate();
    CHECK(s.chunk_tokens() == 64);
}

TEST(prefill_settings_exact_calibration_cannot_promote_online_contract) {
    // tests/tiled_attention_policy.rs:13-25
    PrefillSettings s;
    s.batch_tokens = 64;
    s.weight_reuse_tokens = 8;
    s.attention.mode = AttentionKernelMode::OnlineExperimental;
    expect_throw<Error>([&] { s.validate(); });
    s.attention.mode = AttentionKernelMode::StrictTiled;
    s.validate();
    CHECK(s.id() != "batch-64-reuse-8");
    CHECK(s.id() == "batch-64-reuse-8-stricttiled-q1-k64-wg64-s1");
}

TEST(prefill_settings_bounds_and_json_rules) {
    // calibration_profile.rs:21-54: batch 1..=512 or sequential, reuse in
    // {1, 8, 16, 32}; serde: reuse required, batch optional, no unknown fields
    PrefillSettings s = PrefillSettings::from_json(R"({"batch_tokens":null,"weight_reuse_tokens":1})");
    CHECK(!s.batch_tokens && s.id() == "batch-sequential-reuse-1" && s.chunk_tokens() == 1);
    s.validate();
    s = PrefillSettings::from_json(R"({"weight_reuse_tokens":32,"batch_tokens":512})");
    s.validate();
    for (size_t bad : {(size_t)0, (size_t)513}) {
        s.batch_tokens = bad;
        CHECK(expect_throw<Error>([&] { s.validate(); }) == "prefill batch must be 1..=512");
    }
    s.batch_tokens = 16;
    s.weight_reuse_tokens = 4;
    CHECK(expect_throw<Error>([&] { s.validate(); }) == "prefill reuse must be 1,8,16,32");
    const PrefillSettings nested = PrefillSettings::from_json(
        R"({"weight_reuse_tokens":16,"attention":{"mode":"strict_tiled","block_keys":128}})");
    CHECK(nested.attention.mode == AttentionKernelMode::StrictTiled && nested.attention.block_keys == 128);
    for (const char *bad : {R"({"batch_tokens":64})", R"({"weight_reuse_tokens":8,"fast":true})",
                            R"({"weight_reuse_tokens":-8})", R"({"weight_reuse_tokens":8,"attention":{"mode":"x"}})",
                            R"([])"})
        expect_throw<Error>([&] { PrefillSettings::from_json(bad); });
}

TEST(config_split_tokens_for_the_decode_kernel) {
    AttentionKernelConfig c;
    CHECK(c.decode_split_tokens(32768) == 0);  // library choice
    c.mode = AttentionKernelMode::SplitKvExperimental;
    c.splits = 8;
    CHECK(c.decode_split_tokens(32768) == 4096);
    CHECK(c.decode_split_tokens(1000) == 128);  // ceil(1000/8) = 125 -> 128
    CHECK(c.decode_split_tokens(5) == 64);      // min(splits, history) parts
}

// ---- portable.rs:661-825 (host logic) ----------------------------------
TEST(portable_exact_bits_for_all_float_formats) {
    struct C {
        FloatFormat f;
        std::vector<uint8_t> bytes;
    };
    const C cases[] = {{FloatFormat::Bf16, {0x80, 0x3f, 0xc1, 0x7f}},
                       {FloatFormat::F16, {0x00, 0x3c, 0x01, 0x7e}},
                       {FloatFormat::F32, {0, 0, 0x80, 0x3f, 1, 0, 0xc0, 0x7f}}};
    for (const auto &c : cases) {
        const RawTensor t = RawTensor::from_le_bytes(c.f, {2}, c.bytes);
        CHECK(t.as_le_bytes() == c.bytes);
        CHECK(t.decode_f32()[0] == 1.0f);
        CHECK(std::isnan(t.decode_f32()[1]));
    }
    const RawTensor sub = RawTensor::from_le_bytes(FloatFormat::F16, {1}, {1, 0});
    CHECK(sub.decode_f32()[0] == std::ldexp(1.0f, -24));
    const RawTensor z = RawTensor::from_f32({1}, {-0.0f});
    const uint8_t neg_zero[4] = {0, 0, 0, 0x80};
    CHECK(std::memcmp(z.as_le_bytes().data(), neg_zero, 4) == 0);
}

TEST(test_f16_encoder_matches_ieee) {
    // Pins the test's own encoder: exact values, ties to even, subnormals.
    CHECK(f16_bits(1.0f) == 0x3c00 && f16_bits(-2.0f) == 0xc000 && f16_bits(0.0625f) == 0x2c00);
    CHECK(f16_bits(std::ldexp(1.0f, -24)) == 0x0001 && f16_bits(std::ldexp(1.0f, -25)) == 0x0000);
    CHECK(f16_bits(std::ldexp(3.0f, -25)) == 0x0002);  // 1.5 units -> 2 (even)
    CHECK(f16_bits(1.0f + std::ldexp(1.0f, -11)) == 0x3c00);  // tie -> even
    CHECK(f16_bits(1.0f + std::ldexp(3.0f, -11)) == 0x3c02);  // tie -> even (up)
    CHECK(f16_bits(65520.0f) == 0x7c00 && f16_bits(65504.0f) == 0x7bff);
}

TEST(portable_reject_incorrect_shapes) {
    CHECK(expect_portable([] { AttentionGeometry::create(3, 2, 32); }) == PortableError::Kind::InvalidGeometry);
    CHECK(expect_portable([] { RawTensor::from_le_bytes(FloatFormat::Bf16, {2, 3}, std::vector<uint8_t>(6)); }) ==
          PortableError::Kind::ShapeMismatch);
    CHECK(expect_portable([] { RawTensor::from_le_bytes(FloatFormat::Bf16, {0}, {}); }) ==
          PortableError::Kind::InvalidGeometry);
    ExactKvFrames cache(AttentionGeometry::create(1, 1, 2));
    const RawTensor good = RawTensor::from_f32({1, 1, 2}, {1.0f, 2.0f});
    const RawTensor bad = RawTensor::from_f32({1, 1, 3}, {1.0f, 2.0f, 3.0f});
    CHECK(expect_portable([&] { cache.append(good, bad); }) == PortableError::Kind::ShapeMismatch);
    CHECK(cache.tokens() == 0);
    const std::string msg = PortableError(PortableError::Kind::NonFinite, "GPU Q").what();
    CHECK(msg == "non-finite computation: GPU Q");
}

// Independent serialisation of ExactKvFrames::digest_sha256 (portable.rs:511-545)
// hashed with the oracle's SHA-256.
std::string oracle_digest(const ExactKvFrames &kv) {
    std::vector<uint8_t> b;
    const char *tag = "mslim-portable-exact-kv-v1";
    b.insert(b.end(), tag, tag + std::strlen(tag));
    auto u64 = [&](uint64_t v) {
        for (int i = 0; i < 8; ++i) b.push_back((uint8_t)(v >> (8 * i)));
    };
    const auto g = kv.geometry();
    u64(g.query_heads);
    u64(g.kv_heads);
    u64(g.head_dim);
    u64(kv.tokens());
    for (const auto &f : kv.frames())
        for (const RawTensor *t : {&f.first, &f.second}) {
            b.push_back(t->dtype() == FloatFormat::Bf16 ? 1 : t->dtype() == FloatFormat::F16 ? 2 : 3);
            for (size_t d : t->shape()) u64(d);
            b.insert(b.end(), t->as_le_bytes().begin(), t->as_le_bytes().end());
        }
    uint8_t out[32];
    orc_sha256(b.data(), b.size(), out);
    static const char *hex = "0123456789abcdef";
    std::string s;
    for (uint8_t x : out) {
        s.push_back(hex[x >> 4]);
        s.push_back(hex[x & 15]);
    }
    return s;
}

TEST(portable_chunks_keep_exact_payload_and_digests) {
    ExactKvFrames cache(AttentionGeometry::create(2, 1, 2));
    const RawTensor key = RawTensor::from_le_bytes(FloatFormat::Bf16, {1, 1, 2}, {0, 0, 0x80, 0x3f});
    const RawTensor value = RawTensor::from_le_bytes(FloatFormat::F16, {1, 1, 2}, {0, 0x3c, 0, 0x40});
    cache.append(key, value);
    CHECK(cache.payload_bytes() == 8);
    CHECK(cache.frames()[0].first.as_le_bytes() == key.as_le_bytes());
    CHECK(cache.frames()[0].second.as_le_bytes() == value.as_le_bytes());
    const std::string previous = cache.digest_sha256();
    CHECK(previous == oracle_digest(cache));
    cache.append(key, value);
    CHECK(previous != cache.digest_sha256());
    CHECK(cache.digest_sha256() == oracle_digest(cache));
    CHECK(cache.tokens() == 2);
}

// ---- GPU backend (gpu_backend.rs:379-469) --------------------------------
// f32 -> IEEE binary16, round to nearest even (the half crate's
// f16::from_f32 that the reference test uses to build its frames).
uint16_t f16_bits(float x) {
    uint32_t b;
    std::memcpy(&b, &x, 4);
    const uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    const uint32_t exp = (b >> 23) & 0xffu, mant = b & 0x7fffffu;
    if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (mant ? 0x200u | (mant >> 13) : 0u));
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {  // subnormal result: units of 2^-24, rounded half to even
        const double units = std::nearbyint(std::fabs((double)x) * 16777216.0);
        return (uint16_t)(sign | (uint16_t)units);
    }
    uint32_t r = mant >> 13;
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
    if (r == 0x400u) {
        r = 0;
        if (++e >= 31) return (uint16_t)(sign | 0x7c00u);
    }
    return (uint16_t)(sign | (uint16_t)(e << 10) | (uint16_t)r);
}

std::vector<uint8_t> encode(const std::vector<float> &v, FloatFormat f) {
    std::vector<uint8_t> out;
    for (float x : v) {
        if (f == FloatFormat::F32) {
            uint8_t b[4];
            std::memcpy(b, &x, 4);
            out.insert(out.end(), b, b + 4);
            continue;
        }
        uint16_t h;
        if (f == FloatFormat::Bf16) {
            h = orc_write_bf16(x);
        } else {
            h = f16_bits(x);
        }
        out.push_back((uint8_t)(h & 0xff));
        out.push_back((uint8_t)(h >> 8));
    }
    return out;
}

std::vector<float> cpu_reference(const ExactKvFrames &kv, const std::vector<float> &q) {
    std::vector<uint8_t> k, v;
    for (const auto &f : kv.frames()) {
        k.insert(k.end(), f.first.as_le_bytes().begin(), f.first.as_le_bytes().end());
        v.insert(v.end(), f.second.as_le_bytes().begin(), f.second.as_le_bytes().end());
    }
    const auto g = kv.geometry();
    std::vector<float> out(q.size());
    const int rc = orc_cpu_reference_decode_formats((int)g.query_heads, (int)g.kv_heads, (int)g.head_dim, q.data(),
                                                    k.data(), format_code(kv.frames()[0].first.dtype()), v.data(),
                                                    format_code(kv.frames()[0].second.dtype()), (int)kv.tokens(),
                                                    out.data());
    CHECK(rc == 0);
    return out;
}

void gpu_roundtrip(FloatFormat dtype) {
    GpuBackend device;
    CHECK(device.device_info().arch.rfind("gfx950", 0) == 0);
    const auto shape = AttentionGeometry::create(4, 2, 4);
    std::vector<float> k(32), v(32);
    for (int i = 0; i < 32; ++i) {
        k[i] = (float)(i % 11 - 5) * 0.0625f;
        v[i] = (float)(i % 13 - 6) * 0.0625f;
    }
    ExactKvFrames cache(shape);
    cache.append(RawTensor::from_le_bytes(dtype, {4, 2, 4}, encode(k, dtype)),
                 RawTensor::from_le_bytes(dtype, {4, 2, 4}, encode(v, dtype)));
    const std::vector<float> query(16, 0.15f);
    const auto cpu = cpu_reference(cache, query);
    const auto gpu = cache.decode(device, query);
    for (size_t i = 0; i < cpu.size(); ++i) CHECK(std::fabs(cpu[i] - gpu[i]) < 0.0001f);
    CHECK(device.last_timings().has_value() && device.last_timings()->kernel_ms > 0.0);
}

void gpu_geometry_roundtrip(size_t query_heads, size_t kv_heads) {
    GpuBackend backend;
    const auto geometry = AttentionGeometry::create(query_heads, kv_heads, 8);
    const size_t tokens = 5, count = tokens * kv_heads * 8;
    std::vector<float> key(count), value(count), query(geometry.query_elements());
    for (size_t i = 0; i < count; ++i) {
        key[i] = ((float)(i % 19) - 9.0f) * 0.0625f;
        value[i] = ((float)(i % 17) - 8.0f) * 0.0625f;
    }
    for (size_t i = 0; i < query.size(); ++i) query[i] = ((float)(i % 7) - 3.0f) * 0.125f;
    ExactKvFrames cache(geometry);
    cache.append(RawTensor::from_f32({tokens, kv_heads, 8}, key), RawTensor::from_f32({tokens, kv_heads, 8}, value));
    const auto cpu = cpu_reference(cache, query);
    const auto gpu = cache.decode(backend, query);
    for (size_t i = 0; i < cpu.size(); ++i) CHECK(std::fabs(cpu[i] - gpu[i]) < 0.0001f);
}

TEST(gpu_actual_mha_4q_4kv) { gpu_geometry_roundtrip(4, 4); }
TEST(gpu_actual_mqa_4q_1kv) { gpu_geometry_roundtrip(4, 1); }
TEST(gpu_actual_bf16) { gpu_roundtrip(FloatFormat::Bf16); }
TEST(gpu_actual_f16) { gpu_roundtrip(FloatFormat::F16); }
TEST(gpu_actual_f32) { gpu_roundtrip(FloatFormat::F32); }

TEST(gpu_backend_contract) {
    GpuBackend backend;
    const auto info = backend.device_info();
    CHECK(info.max_compute_units >= 256);
    CHECK(info.reported_global_memory_bytes > 250ull * 1000 * 1000 * 1000);
    ExactKvFrames cache(AttentionGeometry::create(2, 1, 2));
    // empty cache: zeros (gpu_backend.rs:157-159)
    CHECK(cache.decode(backend, {1.0f, 2.0f, 3.0f, 4.0f}) == std::vector<float>(4, 0.0f));
    cache.append(RawTensor::from_f32({1, 1, 2}, {0.0f, 0.0f}), RawTensor::from_f32({1, 1, 2}, {1.0f, -1.0f}));
    CHECK(expect_portable([&] { cache.decode(backend, {0.0f}); }) == PortableError::Kind::ShapeMismatch);
    CHECK(expect_portable([&] { cache.decode(backend, {NAN, 0, 0, 0}); }) == PortableError::Kind::NonFinite);
    CHECK(cache.decode(backend, {0, 0, 0, 0}) == (std::vector<float>{1.0f, -1.0f, 1.0f, -1.0f}));
    cache.append(RawTensor::from_le_bytes(FloatFormat::Bf16, {1, 1, 2}, {0, 0, 0, 0}),
                 RawTensor::from_f32({1, 1, 2}, {1.0f, 1.0f}));
    CHECK(expect_portable([&] { cache.decode(backend, {0, 0, 0, 0}); }) == PortableError::Kind::BackendFailure);
    ExactKvFrames inf_cache(AttentionGeometry::create(1, 1, 2));
    inf_cache.append(RawTensor::from_f32({1, 1, 2}, {INFINITY, 0.0f}), RawTensor::from_f32({1, 1, 2}, {1.0f, 1.0f}));
    CHECK(expect_portable([&] { inf_cache.decode(backend, {1.0f, 1.0f}); }) == PortableError::Kind::NonFinite);
    CHECK(std::string(backend.name()) == "mi355x-hip-fused-decode");
}

// ---- TiledAttention on the gfx950 kernels --------------------------------
struct DeviceBuffer {
    std::shared_ptr<NativeContext> ctx;
    void *ptr = nullptr;
    size_t bytes = 0;
    DeviceBuffer(std::shared_ptr<NativeContext> c, const void *host, size_t n) : ctx(std::move(c)), bytes(n) {
        ptr = mslim_attn_buf_upload(ctx->handle(), static_cast<const uint8_t *>(host), n);
        if (!ptr) throw Failure(mslim_attn_last_error());
    }
    DeviceBuffer(std::shared_ptr<NativeContext> c, size_t n) : ctx(std::move(c)), bytes(n) {
        ptr = mslim_attn_buf_alloc(ctx->handle(), n);
        if (!ptr) throw Failure(mslim_attn_last_error());
    }
    ~DeviceBuffer() { mslim_attn_buf_free(ctx->handle(), ptr); }
    std::vector<uint16_t> read_u16() const {
        std::vector<uint16_t> out(bytes / 2);
        ctx->check("read", mslim_attn_buf_read(ctx->handle(), ptr, 0, reinterpret_cast<uint8_t *>(out.data()), bytes));
        return out;
    }
};

std::vector<uint16_t> lcg_bf16(size_t n, uint64_t seed) {
    std::vector<uint16_t> out(n);
    for (size_t i = 0; i < n; ++i) {
        seed = seed * 6364136223846793005ull + 1442695040888963407ull;
        const float u = (float)(seed >> 40) / 16777216.0f - 0.5f;
        out[i] = orc_write_bf16(u * 4.0f);
    }
    return out;
}

TEST(gpu_tiled_attention_modes) {
    auto ctx = NativeContext::create();
    const auto geom = AttentionGeometry::create(8, 2, 64);
    AttentionKernelConfig ref;
    CHECK(expect_throw<Error>([&] { TiledAttention::build(ctx, ref, geom); }) ==
          "reference does not compile tiled kernels");
    AttentionKernelConfig split;
    split.mode = AttentionKernelMode::SplitKvExperimental;
    split.splits = 8;
    auto tiled = TiledAttention::build(ctx, split, geom);
    const size_t prior = 700, queries = 1, history = prior + queries;
    const auto q = lcg_bf16(queries * 8 * 64, 1), k = lcg_bf16(history * 2 * 64, 2), v = lcg_bf16(history * 2 * 64, 3);
    DeviceBuffer dq(ctx, q.data(), q.size() * 2), dk(ctx, k.data(), k.size() * 2), dv(ctx, v.data(), v.size() * 2);
    DeviceBuffer dout(ctx, q.size() * 2);
    tiled->run(dq.ptr, dk.ptr, dv.ptr, dout.ptr, queries, prior, geom);
    const auto got = dout.read_u16();
    std::vector<float> qf(q.size()), want(q.size());
    orc_bf16_to_f32_array(q.data(), qf.data(), q.size());
    CHECK(orc_dense_attention_bf16(8, 2, 64, qf.data(), k.data(), v.data(), (int)history, want.data()) == 0);
    for (size_t i = 0; i < got.size(); ++i) CHECK(std::fabs(orc_read_bf16(got[i]) - want[i]) <= 2e-2f);
    CHECK(tiled->diagnostics().find("\"split_dispatches_since_configuration\":1") != std::string::npos);
    CHECK(expect_throw<Error>([&] { tiled->run(dq.ptr, dk.ptr, dv.ptr, dout.ptr, 513, 0, geom); }) ==
          "attention query count must be 1..=512");
    CHECK(expect_throw<Error>([&] { tiled->run(dq.ptr, dk.ptr, dv.ptr, dq.ptr, 1, 0, geom); }) ==
          "tiled attention output must not alias read-only Q/K/V");
    CHECK(expect_throw<Error>([&] {
              tiled->run(dq.ptr, dk.ptr, dv.ptr, dout.ptr, 1, 0, AttentionGeometry::create(8, 1, 64));
          }) == "kernel specialization does not match geometry");
}

TEST(gpu_tiled_attention_multi_query_prefill) {
    auto ctx = NativeContext::create();
    const auto geom = AttentionGeometry::create(8, 2, 128);
    AttentionKernelConfig online;
    online.mode = AttentionKernelMode::OnlineExperimental;
    online.validate_activation(true);
    auto tiled = TiledAttention::build(ctx, online, geom);
    const size_t prior = 37, queries = 300, history = prior + queries;
    const auto q = lcg_bf16(queries * 8 * 128, 4), k = lcg_bf16(history * 2 * 128, 5),
               v = lcg_bf16(history * 2 * 128, 6);
    DeviceBuffer dq(ctx, q.data(), q.size() * 2), dk(ctx, k.data(), k.size() * 2), dv(ctx, v.data(), v.size() * 2);
    DeviceBuffer dout(ctx, q.size() * 2);
    tiled->run(dq.ptr, dk.ptr, dv.ptr, dout.ptr, queries, prior, geom);
    const auto got = dout.read_u16();
    std::vector<float> qf(q.size()), want(q.size());
    orc_bf16_to_f32_array(q.data(), qf.data(), q.size());
    CHECK(orc_prefill_causal_cpu(8, 2, 128, qf.data(), k.data(), v.data(), (int)queries, (int)prior, want.data()) == 0);
    float worst = 0.0f;
    for (size_t i = 0; i < got.size(); ++i) worst = std::fmax(worst, std::fabs(orc_read_bf16(got[i]) - want[i]));
    CHECK(worst <= 2e-2f);
}

}  // namespace

int main(int argc, char **argv) { return harness::run_cases(argc, argv); }
