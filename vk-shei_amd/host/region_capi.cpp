// C ABI of the exact region store (include/mslim_region.h): handles over
// mslim::region::RegionStore, exceptions turned into -1 and a message.
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "../../include/mslim_region.h"
#include "region_store.hpp"

namespace {

thread_local std::string g_region_error;

int region_fail(const std::exception &e) {
    g_region_error = e.what();
    return -1;
}

mslim::region::RegionStore &store_of(void *s) {
    mslim::ensure(s != nullptr, "null region store handle");
    return *static_cast<mslim::region::RegionStore *>(s);
}

}  // namespace

extern "C" {

const char *mslim_region_last_error(void) { return g_region_error.c_str(); }

void *mslim_region_new(int q_heads, int kv_heads, int head_dim, int layers, const char *directory,
                       int stage_tokens) {
    g_region_error.clear();
    try {
        mslim::ensure(q_heads > 0 && kv_heads > 0 && head_dim > 0 && layers > 0, "invalid region store geometry");
        mslim::ensure(stage_tokens > 0, "LOD stage_tokens must be in 1..=1024");
        const auto g = mslim::portable::AttentionGeometry::create((size_t)q_heads, (size_t)kv_heads,
                                                                  (size_t)head_dim);
        mslim::region::RegionConfig config;
        config.stage_tokens = (size_t)stage_tokens;
        if (directory) config.cold_directory = std::string(directory);
        return new mslim::region::RegionStore(g, (size_t)layers, config);
    } catch (const std::exception &e) {
        region_fail(e);
        return nullptr;
    }
}

void mslim_region_destroy(void *store) { delete static_cast<mslim::region::RegionStore *>(store); }

int64_t mslim_region_layer_tokens(void *store, int layer) {
    g_region_error.clear();
    try {
        mslim::region::RegionStore &s = store_of(store);
        mslim::ensure(layer >= 0 && (size_t)layer < s.layer_count(), "GPU LOD layer out of range");
        return (int64_t)s.layer_tokens((size_t)layer);
    } catch (const std::exception &e) {
        return region_fail(e);
    }
}

int mslim_region_append(void *store, int layer, int64_t position, const void *keys, const void *values,
                        int tokens, int page_tokens) {
    g_region_error.clear();
    try {
        mslim::region::RegionStore &s = store_of(store);
        mslim::ensure(keys && values && tokens > 0 && layer >= 0 && position >= 0, "invalid region append arguments");
        const size_t bytes = (size_t)tokens * s.geometry().kv_elements_per_token() * 2;
        const auto *k = static_cast<const uint8_t *>(keys);
        const auto *v = static_cast<const uint8_t *>(values);
        s.append_batch((size_t)layer, (size_t)position, std::vector<uint8_t>(k, k + bytes),
                       std::vector<uint8_t>(v, v + bytes), (size_t)page_tokens);
        return 0;
    } catch (const std::exception &e) {
        return region_fail(e);
    }
}

int mslim_region_read(void *store, int layer, int part, const int64_t *positions, int count, void *out) {
    g_region_error.clear();
    try {
        mslim::region::RegionStore &s = store_of(store);
        mslim::ensure(layer >= 0 && (part == 0 || part == 1) && count >= 0 && (count == 0 || (positions && out)),
                      "invalid region read arguments");
        std::vector<size_t> pos((size_t)count);
        for (int i = 0; i < count; ++i) {
            mslim::ensure(positions[i] >= 0, "negative token position");
            pos[(size_t)i] = (size_t)positions[i];
        }
        const std::vector<uint8_t> rows =
            part == 0 ? s.read_keys((size_t)layer, pos) : s.read_values((size_t)layer, pos);
        if (!rows.empty()) std::memcpy(out, rows.data(), rows.size());
        return 0;
    } catch (const std::exception &e) {
        return region_fail(e);
    }
}

int mslim_region_logical_kv_sha256(void *store, char *hex_out) {
    g_region_error.clear();
    try {
        mslim::ensure(hex_out != nullptr, "null digest output");
        const std::string hex = store_of(store).logical_kv_sha256();
        std::memcpy(hex_out, hex.c_str(), hex.size() + 1);
        return 0;
    } catch (const std::exception &e) {
        return region_fail(e);
    }
}

}  // extern "C"
