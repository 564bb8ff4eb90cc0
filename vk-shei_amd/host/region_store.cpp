// Exact GPU region store (gpu_region_store.rs:118-928).
#include "region_store.hpp"

#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>

#include "../csrc/sha256.hpp"

namespace mslim {
namespace region {

namespace {

const char *kStoreFile = "pages-exact.kv";  // gpu_region_store.rs:161

float bf16_to_f32(uint16_t bits) {
    const uint32_t w = (uint32_t)bits << 16;
    float f;
    std::memcpy(&f, &w, 4);
    return f;
}

uint16_t load_u16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

bool is_dir(const std::string &path) {
    struct stat st;
    return stat(path.c_str(), &st) == 0 && S_ISDIR(st.st_mode);
}

bool exists(const std::string &path) {
    struct stat st;
    return stat(path.c_str(), &st) == 0;
}

std::string make_temp_dir(const RegionConfig &c) {
    if (c.cold_directory) return std::string();
    const char *tmp = std::getenv("TMPDIR");
    std::string pattern = std::string(tmp && *tmp ? tmp : "/tmp") + "/mslim-gpu-region-XXXXXX";
    std::vector<char> buf(pattern.begin(), pattern.end());
    buf.push_back('\0');
    if (!mkdtemp(buf.data())) throw Error("cannot create a temporary ColdStore directory");
    return std::string(buf.data());
}

cold::ColdStore open_store(const RegionConfig &c, const std::string &temp_dir) {
    if (c.cold_directory) {
        const std::string path = *c.cold_directory + "/" + kStoreFile;
        return exists(path) ? cold::ColdStore::open(path, 0) : cold::ColdStore::create(path, 0);
    }
    return cold::ColdStore::create(temp_dir + "/" + kStoreFile, 0);
}

const RegionConfig &validated(const RegionConfig &c) {
    c.validate();
    return c;
}

std::string hex(const uint8_t *d, size_t n) {
    static const char digits[] = "0123456789abcdef";
    std::string s;
    for (size_t i = 0; i < n; ++i) {
        s.push_back(digits[d[i] >> 4]);
        s.push_back(digits[d[i] & 15]);
    }
    return s;
}

bool bf16_nonfinite(uint16_t bits) { return (bits & 0x7f80u) == 0x7f80u; }

}  // namespace

void RegionConfig::validate() const {
    ensure(std::isfinite(epsilon) && epsilon >= 0.0 && epsilon <= 0.1, "LOD epsilon must be finite within 0..=0.1");
    ensure(stage_tokens >= 1 && stage_tokens <= 1024, "LOD stage_tokens must be in 1..=1024");
    if (cold_directory) ensure(is_dir(*cold_directory), "LOD cold directory does not exist: " + *cold_directory);
    ensure(epsilon == 0.0, "positive-epsilon LOD selection is not part of this build (exact mode only)");
}

RegionStore::RegionStore(portable::AttentionGeometry geometry, size_t layer_count, RegionConfig config)
    : config_(validated(config)),
      geometry_(geometry),
      temp_dir_(make_temp_dir(config_)),
      cold_(open_store(config_, temp_dir_)) {
    ensure(layer_count > 0, "LOD model must contain at least one layer");
    pages_.resize(layer_count);
    value_abs_max_.assign(layer_count, std::vector<double>(geometry_.kv_heads, 0.0));
    stats.gpu_stage_tokens = config_.stage_tokens;
    stats.shared_original_cpu_algorithms = true;
    restore_catalogue();
}

RegionStore::~RegionStore() {
    // A private temporary store is removed; its descriptor closes with cold_.
    if (!temp_dir_.empty()) {
        ::unlink(cold_.path().c_str());
        ::rmdir(temp_dir_.c_str());
    }
}

// gpu_region_store.rs:209-292
void RegionStore::restore_catalogue() {
    const std::vector<cold::PageMeta> metadata = cold_.metadata();
    if (metadata.empty()) return;
    const size_t row_bytes = geometry_.head_dim * 2;
    const size_t token_bytes = geometry_.kv_elements_per_token() * 2;
    for (const cold::PageMeta &meta : metadata) {
        const size_t layer = meta.geometry.layer;
        ensure(layer < pages_.size(), "persisted KV layer out of range");
        ensure(meta.geometry.heads == geometry_.kv_heads && meta.geometry.head_dim == geometry_.head_dim,
               "persisted KV geometry does not match model");
        const size_t start = meta.geometry.token_start;
        const size_t count = meta.geometry.tokens;
        ensure(pages_[layer].size() == start, "persisted KV pages are not a contiguous causal prefix");
        auto payload = cold_.read_page(meta.page_id);
        ensure(payload->key.size() == count * token_bytes && payload->value.size() == count * token_bytes,
               "persisted KV payload shape mismatch");
        // Head-major V; every value must be finite (:246-261).
        for (size_t head = 0; head < geometry_.kv_heads; ++head) {
            for (size_t token = 0; token < count; ++token) {
                const uint8_t *row = payload->value.data() + (head * count + token) * row_bytes;
                for (size_t d = 0; d < geometry_.head_dim; ++d) {
                    const float x = bf16_to_f32(load_u16(row + 2 * d));
                    ensure(std::isfinite(x), "persisted KV contains nonfinite V");
                    value_abs_max_[layer][head] = std::max(value_abs_max_[layer][head], (double)std::fabs(x));
                }
            }
        }
        if (layer == 0) axis_tokens_ += count;
        for (size_t offset = 0; offset < count; ++offset) pages_[layer].push_back({meta.page_id, offset});
    }
    stats.physical_cold_store_pages = cold_.metadata().size();
    stats.physical_cold_store_bytes = cold_.stats().committed_bytes;
}

size_t RegionStore::layer_tokens(size_t layer) const {
    return layer < pages_.size() ? pages_[layer].size() : 0;
}

// gpu_region_store.rs:341-371
std::string RegionStore::logical_kv_sha256() {
    const size_t tokens = axis_tokens_;
    for (const auto &layer : pages_)
        ensure(layer.size() == tokens, "canonical ColdStore layers do not share a complete causal prefix");
    std::vector<size_t> positions(tokens);
    for (size_t i = 0; i < tokens; ++i) positions[i] = i;
    const size_t head_bytes = geometry_.head_dim * 2;
    const size_t token_bytes = geometry_.kv_elements_per_token() * 2;
    Sha256 sha;
    static const char tag[] = "mslim-dense-kv-state-v1";
    sha.update(tag, sizeof tag - 1);
    uint8_t le[8];
    for (int i = 0; i < 8; ++i) le[i] = (uint8_t)((uint64_t)tokens >> (8 * i));
    sha.update(le, 8);
    for (size_t layer = 0; layer < pages_.size(); ++layer) {
        for (int part = 0; part < 2; ++part) {
            const std::vector<uint8_t> token_major =
                tokens ? (part == 0 ? read_keys(layer, positions) : read_values(layer, positions))
                       : std::vector<uint8_t>();
            ensure(token_major.size() == tokens * token_bytes, "canonical ColdStore logical K/V shape mismatch");
            for (size_t head = 0; head < geometry_.kv_heads; ++head)
                for (size_t token = 0; token < tokens; ++token)
                    sha.update(token_major.data() + (token * geometry_.kv_heads + head) * head_bytes, head_bytes);
        }
    }
    uint8_t digest[32];
    sha.finish(digest);
    return hex(digest, 32);
}

void RegionStore::append(size_t layer, size_t position, const uint8_t *key, const uint8_t *value,
                         size_t token_bytes) {
    append_batch(layer, position, std::vector<uint8_t>(key, key + token_bytes),
                 std::vector<uint8_t>(value, value + token_bytes), 1);
}

// gpu_region_store.rs:391-520
void RegionStore::append_batch(size_t layer, size_t position, const std::vector<uint8_t> &keys,
                               const std::vector<uint8_t> &values, size_t page_tokens) {
    ensure(page_tokens >= 1 && page_tokens <= 512, "GPU ColdStore page size must be 1..512 tokens");
    const size_t token_bytes = geometry_.kv_elements_per_token() * 2;
    ensure(!keys.empty() && keys.size() == values.size() && keys.size() % token_bytes == 0,
           "GPU LOD batched BF16 K/V shape mismatch");
    const size_t count = keys.size() / token_bytes;
    ensure(layer < pages_.size(), "GPU LOD batch layer out of range");
    ensure(pages_[layer].size() == position, "GPU LOD append needs sequential tokens");
    const size_t kvh = geometry_.kv_heads;
    const size_t row_bytes = geometry_.head_dim * 2;
    // Every value, and each layer-zero key, is validated before any page is
    // committed.
    std::vector<double> maxima = value_abs_max_[layer];
    for (size_t i = 0; i < count; ++i) {
        const uint8_t *k = keys.data() + i * token_bytes;
        const uint8_t *v = values.data() + i * token_bytes;
        if (layer == 0)
            for (size_t j = 0; j < token_bytes; j += 2)
                ensure(std::isfinite(bf16_to_f32(load_u16(k + j))), "GPU ColdStore K nonfinite");
        for (size_t h = 0; h < kvh; ++h)
            for (size_t d = 0; d < geometry_.head_dim; ++d) {
                const float x = bf16_to_f32(load_u16(v + h * row_bytes + d * 2));
                ensure(std::isfinite(x), "GPU ColdStore V nonfinite");
                maxima[h] = std::max(maxima[h], (double)std::fabs(x));
            }
    }
    const uint32_t tile = geometry_.head_dim % 16 == 0 ? 16 : 1;
    for (size_t start = 0; start < count; start += page_tokens) {
        const size_t n = std::min(page_tokens, count - start);
        std::vector<uint8_t> k(n * token_bytes), v(n * token_bytes);
        for (size_t head = 0; head < kvh; ++head)
            for (size_t token = 0; token < n; ++token) {
                const size_t source = ((start + token) * kvh + head) * row_bytes;
                const size_t dest = (head * n + token) * row_bytes;
                std::memcpy(k.data() + dest, keys.data() + source, row_bytes);
                std::memcpy(v.data() + dest, values.data() + source, row_bytes);
            }
        cold::PageGeometry g;
        g.layer = (uint32_t)layer;
        g.token_start = position + start;
        g.tokens = (uint32_t)n;
        g.heads = (uint32_t)kvh;
        g.head_dim = (uint32_t)geometry_.head_dim;
        g.tile = tile;
        const cold::PageMeta meta = cold_.append_page(g, k, v, false);
        for (size_t offset = 0; offset < n; ++offset) pages_[layer].push_back({meta.page_id, offset});
        stats.prefill_batched_page_tokens = std::max(stats.prefill_batched_page_tokens, n);
    }
    value_abs_max_[layer] = maxima;
    if (layer == 0) axis_tokens_ += count;
    const cold::ColdStoreStats info = cold_.stats();
    stats.physical_cold_store_bytes = info.committed_bytes;
    stats.physical_cold_store_pages = info.pages;
}

// gpu_region_store.rs:642-661
SelectionResult RegionStore::select_dense_exact(size_t layer) {
    const size_t tokens = layer_tokens(layer);
    ensure(tokens > 0, "no BF16 K/V tokens for exact LOD");
    ensure(axis_tokens_ == tokens, "canonical axis not synchronized");
    const size_t heads = geometry_.query_heads;
    stats.queries += 1;
    stats.exact_k_scores_computed_on_gpu += tokens * heads;
    stats.exact_fallbacks += 1;
    SelectionResult r;
    r.positions.resize(tokens);
    for (size_t i = 0; i < tokens; ++i) r.positions[i] = i;
    r.selected_mass_per_head.assign(heads, 1.0f);
    r.bounds.assign(heads, 0.0);
    return r;
}

// gpu_region_store.rs:828-927: runs of positions on one page are read with
// one verified partial read; output token-major.
std::vector<uint8_t> RegionStore::read_rows(size_t layer, const std::vector<size_t> &positions, bool key) {
    const char *what = key ? "LOD K" : "GPU LOD";
    ensure(layer < pages_.size(), key ? "LOD read layer missing" : "GPU LOD read layer missing");
    const std::vector<PageAddress> &pages = pages_[layer];
    const size_t bytes_per_token = geometry_.kv_elements_per_token() * 2;
    const size_t head_bytes = geometry_.head_dim * 2;
    std::vector<uint8_t> out;
    out.reserve(positions.size() * bytes_per_token);
    size_t cursor = 0;
    while (cursor < positions.size()) {
        ensure(positions[cursor] < pages.size(), std::string(what) + " token not recorded");
        const PageAddress first = pages[positions[cursor]];
        std::vector<size_t> offsets{first.offset};
        size_t end = cursor + 1;
        while (end < positions.size()) {
            ensure(positions[end] < pages.size(), std::string(what) + " token not recorded");
            const PageAddress next = pages[positions[end]];
            if (next.page_id != first.page_id) break;
            ensure(next.offset > offsets.back(), key ? "LOD selected K positions must be sorted and unique"
                                                      : "GPU LOD selected positions must be sorted and unique");
            offsets.push_back(next.offset);
            ++end;
        }
        const std::vector<uint8_t> data =
            key ? cold_.read_key_tokens(first.page_id, offsets) : cold_.read_value_tokens(first.page_id, offsets);
        ensure(data.size() == offsets.size() * bytes_per_token,
               key ? "canonical ColdStore partial K BF16 dimensions invalid"
                   : "canonical ColdStore partial page BF16 dimensions invalid");
        for (size_t local = 0; local < offsets.size(); ++local)
            for (size_t head = 0; head < geometry_.kv_heads; ++head) {
                const uint8_t *src = data.data() + (head * offsets.size() + local) * head_bytes;
                out.insert(out.end(), src, src + head_bytes);
            }
        cursor = end;
    }
    return out;
}

std::vector<uint8_t> RegionStore::read_values(size_t layer, const std::vector<size_t> &positions) {
    std::vector<uint8_t> out = read_rows(layer, positions, false);
    stats.exact_v_tokens_read_from_cold += positions.size();
    stats.cold_value_read_calls = cold_.stats().reads;
    return out;
}

std::vector<uint8_t> RegionStore::read_keys(size_t layer, const std::vector<size_t> &positions) {
    return read_rows(layer, positions, true);
}

// ---- device page pool ----------------------------------------------------------

namespace {

// Device buffer owned for the duration of one call.
struct DeviceBuffer {
    NativeContext &ctx;
    void *ptr = nullptr;
    DeviceBuffer(NativeContext &c, size_t bytes) : ctx(c) {
        ptr = mslim_attn_buf_alloc(ctx.handle(), bytes ? bytes : 16);
        if (!ptr) throw NativeError("buffer alloc", -1, mslim_attn_last_error());
    }
    DeviceBuffer(NativeContext &c, const void *host, size_t bytes) : ctx(c) {
        ptr = mslim_attn_buf_upload(ctx.handle(), static_cast<const uint8_t *>(host), bytes);
        if (!ptr) throw NativeError("buffer upload", -1, mslim_attn_last_error());
    }
    ~DeviceBuffer() {
        if (ptr) mslim_attn_buf_free(ctx.handle(), ptr);
    }
    DeviceBuffer(const DeviceBuffer &) = delete;
    DeviceBuffer &operator=(const DeviceBuffer &) = delete;
    void read(void *host, size_t bytes) {
        ctx.check("buffer read", mslim_attn_buf_read(ctx.handle(), ptr, 0, static_cast<uint8_t *>(host), bytes));
    }
    void write(const void *host, size_t bytes) {
        ctx.check("buffer write",
                  mslim_attn_buf_write(ctx.handle(), ptr, 0, static_cast<const uint8_t *>(host), bytes));
    }
};

void check_pool(const DevicePagePool &pool, const portable::AttentionGeometry &g) {
    ensure(pool.k_pool && pool.v_pool && pool.pool_pages > 0, "device page pool is not set");
    ensure(pool.page_tokens >= 1 && pool.page_tokens <= 512 && (pool.page_tokens & (pool.page_tokens - 1)) == 0,
           "device page pool page_tokens must be a power of two in 1..512");
    ensure(g.head_dim % 8 == 0, "device page pool needs head_dim a multiple of 8");
}

}  // namespace

void RegionStore::seal_device_pages(NativeContext &ctx, size_t layer, size_t position, const DevicePagePool &pool,
                                    const std::vector<int32_t> &blocks, size_t count) {
    check_pool(pool, geometry_);
    ensure(layer < pages_.size(), "GPU LOD batch layer out of range");
    ensure(pages_[layer].size() == position, "GPU LOD append needs sequential tokens");
    ensure(count > 0, "GPU LOD batched BF16 K/V shape mismatch");
    const size_t P = (size_t)pool.page_tokens;
    ensure(position % P == 0, "device seal must start at a pool page boundary");
    const size_t records = (count + P - 1) / P;
    ensure(blocks.size() >= records, "device seal needs a pool page for every logical page");
    const size_t kvh = geometry_.kv_heads, row_bytes = geometry_.head_dim * 2;
    const size_t page_bytes = kvh * P * row_bytes;
    const uint32_t tile = geometry_.head_dim % 16 == 0 ? 16 : 1;
    const uint64_t first_page_id = cold_.metadata().size();

    std::vector<mslim_attn_page_record> descs(records);
    for (size_t i = 0; i < records; ++i) {
        ensure(blocks[i] >= 0 && blocks[i] < pool.pool_pages, "device seal pool page out of range");
        descs[i].page_id = first_page_id + i;
        descs[i].token_start = position + i * P;
        descs[i].layer = (uint32_t)layer;
        descs[i].tokens = (uint32_t)std::min(P, count - i * P);
        descs[i].pool_page = blocks[i];
        descs[i].reserved = 0;
    }
    const int64_t slot = mslim_attn_record_frame_bytes((int)P);
    std::vector<uint8_t> frames(records * slot), k(records * page_bytes), v(records * page_bytes);
    {
        std::lock_guard<std::mutex> guard(ctx.mutex());
        DeviceBuffer d_desc(ctx, descs.data(), descs.size() * sizeof(mslim_attn_page_record));
        DeviceBuffer d_frames(ctx, frames.size()), d_k(ctx, k.size()), d_v(ctx, v.size());
        ctx.check("record frames",
                  mslim_attn_record_frames(ctx.handle(), pool.k_pool, pool.v_pool, pool.pool_pages, (int)P, (int)kvh,
                                           (int)geometry_.head_dim, tile,
                                           static_cast<const mslim_attn_page_record *>(d_desc.ptr), (int)records,
                                           d_frames.ptr));
        ctx.check("record payloads",
                  mslim_attn_record_payloads(ctx.handle(), pool.k_pool, pool.v_pool, pool.pool_pages, (int)P,
                                             (int)kvh, (int)geometry_.head_dim,
                                             static_cast<const mslim_attn_page_record *>(d_desc.ptr), (int)records,
                                             d_k.ptr, d_v.ptr, 0));
        d_frames.read(frames.data(), frames.size());
        d_k.read(k.data(), k.size());
        d_v.read(v.data(), v.size());
    }
    // Same validation as append_batch, before anything is committed.
    std::vector<double> maxima = value_abs_max_[layer];
    for (size_t i = 0; i < records; ++i) {
        const size_t n = descs[i].tokens;
        const uint8_t *kp = k.data() + i * page_bytes;
        const uint8_t *vp = v.data() + i * page_bytes;
        if (layer == 0)
            for (size_t j = 0; j < n * kvh * row_bytes; j += 2)
                ensure(!bf16_nonfinite(load_u16(kp + j)), "GPU ColdStore K nonfinite");
        for (size_t h = 0; h < kvh; ++h)
            for (size_t j = 0; j < n * row_bytes; j += 2) {
                const float x = bf16_to_f32(load_u16(vp + h * n * row_bytes + j));
                ensure(std::isfinite(x), "GPU ColdStore V nonfinite");
                maxima[h] = std::max(maxima[h], (double)std::fabs(x));
            }
    }
    for (size_t i = 0; i < records; ++i) {
        const size_t n = descs[i].tokens;
        const uint8_t *frame = frames.data() + i * slot;
        const cold::PageMeta meta = cold_.append_framed(frame, (size_t)slot, k.data() + i * page_bytes,
                                                        v.data() + i * page_bytes, n * kvh * row_bytes, false);
        for (size_t offset = 0; offset < n; ++offset) pages_[layer].push_back({meta.page_id, offset});
        stats.prefill_batched_page_tokens = std::max(stats.prefill_batched_page_tokens, n);
    }
    value_abs_max_[layer] = maxima;
    if (layer == 0) axis_tokens_ += count;
    stats.device_sealed_pages += records;
    const cold::ColdStoreStats info = cold_.stats();
    stats.physical_cold_store_bytes = info.committed_bytes;
    stats.physical_cold_store_pages = info.pages;
}

void RegionStore::restore_to_device(NativeContext &ctx, size_t layer, const DevicePagePool &pool,
                                    const std::vector<int32_t> &blocks) {
    check_pool(pool, geometry_);
    ensure(layer < pages_.size(), "GPU LOD read layer missing");
    const size_t P = (size_t)pool.page_tokens;
    const size_t kvh = geometry_.kv_heads, row_bytes = geometry_.head_dim * 2;
    const size_t page_bytes = kvh * P * row_bytes;
    const uint32_t tile = geometry_.head_dim % 16 == 0 ? 16 : 1;
    // The layer's records, in token order.
    std::vector<uint64_t> ids;
    for (const PageAddress &a : pages_[layer])
        if (ids.empty() || ids.back() != a.page_id) ids.push_back(a.page_id);
    if (ids.empty()) return;
    const size_t records = ids.size();
    const int64_t slot = mslim_attn_record_frame_bytes((int)P);
    std::vector<mslim_attn_page_record> descs(records);
    std::vector<uint8_t> stored(records * slot), k(records * page_bytes, 0), v(records * page_bytes, 0);
    std::vector<uint8_t> frame, key, value;
    for (size_t i = 0; i < records; ++i) {
        const cold::PageMeta &m = cold_.metadata().at(ids[i]);
        ensure(m.geometry.token_start % P == 0 && m.geometry.tokens <= P,
               "layer pages are not aligned to the device pool pages");
        const size_t block = m.geometry.token_start / P;
        ensure(block < blocks.size() && blocks[block] >= 0 && blocks[block] < pool.pool_pages,
               "device restore pool page out of range");
        cold_.read_record_raw(ids[i], (uint32_t)P, frame, key, value);
        std::memcpy(stored.data() + i * slot, frame.data(), slot);
        std::memcpy(k.data() + i * page_bytes, key.data(), key.size());
        std::memcpy(v.data() + i * page_bytes, value.data(), value.size());
        descs[i].page_id = m.page_id;
        descs[i].token_start = m.geometry.token_start;
        descs[i].layer = m.geometry.layer;
        descs[i].tokens = m.geometry.tokens;
        descs[i].pool_page = blocks[block];
        descs[i].reserved = 0;
    }
    std::vector<uint8_t> recomputed(records * slot);
    {
        std::lock_guard<std::mutex> guard(ctx.mutex());
        DeviceBuffer d_desc(ctx, descs.data(), descs.size() * sizeof(mslim_attn_page_record));
        DeviceBuffer d_k(ctx, k.data(), k.size()), d_v(ctx, v.data(), v.size()), d_frames(ctx, recomputed.size());
        ctx.check("record payloads",
                  mslim_attn_record_payloads(ctx.handle(), pool.k_pool, pool.v_pool, pool.pool_pages, (int)P,
                                             (int)kvh, (int)geometry_.head_dim,
                                             static_cast<const mslim_attn_page_record *>(d_desc.ptr), (int)records,
                                             d_k.ptr, d_v.ptr, 1));
        ctx.check("record frames",
                  mslim_attn_record_frames(ctx.handle(), pool.k_pool, pool.v_pool, pool.pool_pages, (int)P, (int)kvh,
                                           (int)geometry_.head_dim, tile,
                                           static_cast<const mslim_attn_page_record *>(d_desc.ptr), (int)records,
                                           d_frames.ptr));
        d_frames.read(recomputed.data(), recomputed.size());
    }
    // The stored frame must equal the one recomputed from the pool bytes:
    // header (payload checksums), token hashes, record checksum and SHA-256.
    for (size_t i = 0; i < records; ++i) {
        const uint8_t *want = stored.data() + i * slot;
        const uint8_t *got = recomputed.data() + i * slot;
        const size_t prefix = cold::kHeaderLen + 16ull * descs[i].tokens;
        if (std::memcmp(want, got, prefix) != 0 ||
            std::memcmp(want + slot - cold::kFooterLen, got + slot - cold::kFooterLen, cold::kFooterLen) != 0)
            throw cold::ColdStoreError(cold::ColdStoreError::Kind::InvalidData,
                                       "device verification failed for KV page " + std::to_string(descs[i].page_id));
    }
    stats.device_restored_pages += records;
}

}  // namespace region
}  // namespace mslim
