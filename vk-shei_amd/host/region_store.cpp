// Exact GPU region store (gpu_region_store.rs:118-928).
#include "region_store.hpp"

#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <mutex>
#include <thread>

#include "../csrc/sha256.hpp"
#include "parallel.hpp"

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

// Scan `count` little-endian BF16 values: returns the largest magnitude's
// bits (sign cleared; among finite BF16 the integer order of these bits is
// the order of |x|) and sets *nonfinite when any exponent field is all ones.
// Integer-only so the loop vectorises.
__attribute__((optimize("O3"))) uint16_t bf16_scan(const uint8_t *p, size_t count, bool *nonfinite) {
    uint16_t top = 0;
    for (size_t i = 0; i < count; ++i) {
        uint16_t bits;
        std::memcpy(&bits, p + 2 * i, 2);
        const uint16_t mag = (uint16_t)(bits & 0x7fffu);
        top = mag > top ? mag : top;
    }
    *nonfinite = top >= 0x7f80u;
    return top;
}

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
    const size_t token_bytes = geometry_.kv_elements_per_token() * 2;
    const size_t kvh = geometry_.kv_heads;
    // The shape of the catalogue first, in record order, up to the first
    // record that does not fit it.
    std::vector<size_t> held(pages_.size(), 0);
    std::vector<uint64_t> ids;
    ids.reserve(metadata.size());
    std::exception_ptr shape_error;
    try {
        for (const cold::PageMeta &meta : metadata) {
            const size_t layer = meta.geometry.layer;
            ensure(layer < pages_.size(), "persisted KV layer out of range");
            ensure(meta.geometry.heads == geometry_.kv_heads && meta.geometry.head_dim == geometry_.head_dim,
                   "persisted KV geometry does not match model");
            ensure(held[layer] == meta.geometry.token_start,
                   "persisted KV pages are not a contiguous causal prefix");
            held[layer] += meta.geometry.tokens;
            ids.push_back(meta.page_id);
        }
    } catch (const Error &) {
        shape_error = std::current_exception();
    }
    // Every record before it read back and verified, then its V checked
    // finite (gpu_region_store.rs:246-261) with per-head magnitude maxima;
    // records on several threads.  The failure reported is the one a
    // record-by-record walk meets first.
    std::vector<uint16_t> top(ids.size() * kvh, 0);
    cold_.for_each_verified(ids, [&](size_t i, const cold::ColdPagePayload &payload) {
        const size_t count = metadata[i].geometry.tokens;
        ensure(payload.key.size() == count * token_bytes && payload.value.size() == count * token_bytes,
               "persisted KV payload shape mismatch");
        const size_t head_bytes = count * geometry_.head_dim * 2;
        for (size_t head = 0; head < kvh; ++head) {
            bool bad = false;
            top[i * kvh + head] = bf16_scan(payload.value.data() + head * head_bytes, head_bytes / 2, &bad);
            ensure(!bad, "persisted KV contains nonfinite V");
        }
    });
    if (shape_error) std::rethrow_exception(shape_error);
    for (size_t i = 0; i < metadata.size(); ++i) {
        const cold::PageMeta &meta = metadata[i];
        const size_t layer = meta.geometry.layer, count = meta.geometry.tokens;
        for (size_t head = 0; head < kvh; ++head)
            value_abs_max_[layer][head] =
                std::max(value_abs_max_[layer][head], (double)bf16_to_f32(top[i * kvh + head]));
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
    // All checks run first (each value row, and the keys of layer 0), so a
    // rejected batch changes no page.
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

DeviceStaging::~DeviceStaging() {
    for (void *p : {d_desc, d_frames, d_k, d_v})
        if (p) mslim_attn_buf_free(ctx_.handle(), p);
    for (uint8_t *p : {h_desc, h_frames, h_k, h_v})
        if (p) mslim_attn_host_free(ctx_.handle(), p);
}

void DeviceStaging::grow(size_t &cap, size_t bytes, void **dev, uint8_t **host) {
    if (cap >= bytes) return;
    if (*dev) mslim_attn_buf_free(ctx_.handle(), *dev);
    if (*host) mslim_attn_host_free(ctx_.handle(), *host);
    *dev = nullptr;
    *host = nullptr;
    cap = 0;
    *dev = mslim_attn_buf_alloc(ctx_.handle(), bytes);
    if (!*dev) throw NativeError("allocate seal staging", -1, mslim_attn_last_error());
    *host = static_cast<uint8_t *>(mslim_attn_host_alloc(ctx_.handle(), bytes));
    if (!*host) throw NativeError("allocate pinned seal staging", -1, mslim_attn_last_error());
    cap = bytes;
}

void DeviceStaging::reserve(size_t records, size_t frame_slot, size_t payload_bytes) {
    records = std::max<size_t>(records, 1);
    grow(desc_cap_, records * sizeof(mslim_attn_page_record), &d_desc, &h_desc);
    grow(frames_cap_, records * frame_slot, &d_frames, &h_frames);
    // K and V share one capacity figure; both buffers grow together.
    if (payload_cap_ < records * payload_bytes) {
        size_t cap_v = payload_cap_;
        grow(payload_cap_, records * payload_bytes, &d_k, &h_k);
        grow(cap_v, records * payload_bytes, &d_v, &h_v);
    }
}

void RegionStore::seal_device_layers(DeviceStaging &st, size_t position, size_t count, const DevicePagePool &pool,
                                     const std::vector<LayerBlocks> &layers, size_t max_group_bytes) {
    NativeContext &ctx = st.ctx();
    check_pool(pool, geometry_);
    ensure(count > 0, "GPU LOD batched BF16 K/V shape mismatch");
    const size_t P = (size_t)pool.page_tokens;
    const size_t kvh = geometry_.kv_heads, row_bytes = geometry_.head_dim * 2;
    const size_t page_bytes = kvh * P * row_bytes;
    const uint32_t tile = geometry_.head_dim % 16 == 0 ? 16 : 1;
    const int64_t slot = mslim_attn_record_frame_bytes((int)P);
    // Records of one layer: the first starts at position % P inside its page.
    const size_t first_row = position % P;
    std::vector<size_t> starts;  // token offsets of the records within [0, count)
    for (size_t t = 0; t < count; t += (t == 0 ? P - first_row : P)) starts.push_back(t);
    const size_t per_layer = starts.size();
    const size_t logical0 = position / P;
    for (const LayerBlocks &lb : layers) {
        ensure(lb.layer < pages_.size(), "GPU LOD batch layer out of range");
        ensure(pages_[lb.layer].size() == position, "GPU LOD append needs sequential tokens");
        ensure(lb.blocks.size() >= logical0 + per_layer, "device seal needs a pool page for every logical page");
    }
    const size_t group_layers = std::max<size_t>(1, max_group_bytes / std::max<size_t>(1, per_layer * page_bytes));
    for (size_t g0 = 0; g0 < layers.size(); g0 += group_layers) {
        const size_t g1 = std::min(layers.size(), g0 + group_layers);
        const size_t records = (g1 - g0) * per_layer;
        st.reserve(records, (size_t)slot, page_bytes);
        auto *descs = reinterpret_cast<mslim_attn_page_record *>(st.h_desc);
        uint64_t page_id = cold_.metadata().size();
        for (size_t li = g0; li < g1; ++li)
            for (size_t r = 0; r < per_layer; ++r) {
                const int32_t block = layers[li].blocks[logical0 + r];
                ensure(block >= 0 && block < pool.pool_pages, "device seal pool page out of range");
                const size_t t0 = starts[r];
                const size_t t1 = r + 1 < per_layer ? starts[r + 1] : count;
                mslim_attn_page_record &d = descs[(li - g0) * per_layer + r];
                d.page_id = page_id++;
                d.token_start = position + t0;
                d.layer = (uint32_t)layers[li].layer;
                d.tokens = (uint32_t)(t1 - t0);
                d.pool_page = block;
                d.first_row = (uint32_t)(r == 0 ? first_row : 0);
            }
        const bool host_frames = records < host_framing_below_;
        {
            std::lock_guard<std::mutex> guard(ctx.mutex());
            void *h = ctx.handle();
            ctx.check("upload record descriptors",
                      mslim_attn_buf_write(h, st.d_desc, 0, st.h_desc, records * sizeof(mslim_attn_page_record)));
            if (!host_frames)
                ctx.check("record frames",
                          mslim_attn_record_frames(h, pool.k_pool, pool.v_pool, pool.pool_pages, (int)P, (int)kvh,
                                                   (int)geometry_.head_dim, tile,
                                                   static_cast<const mslim_attn_page_record *>(st.d_desc),
                                                   (int)records, st.d_frames));
            ctx.check("record payloads",
                      mslim_attn_record_payloads(h, pool.k_pool, pool.v_pool, pool.pool_pages, (int)P, (int)kvh,
                                                 (int)geometry_.head_dim,
                                                 static_cast<const mslim_attn_page_record *>(st.d_desc),
                                                 (int)records, st.d_k, st.d_v, 0));
            if (!host_frames)
                ctx.check("read record frames", mslim_attn_buf_read(h, st.d_frames, 0, st.h_frames, records * slot));
            ctx.check("read K payloads", mslim_attn_buf_read(h, st.d_k, 0, st.h_k, records * page_bytes));
            ctx.check("read V payloads", mslim_attn_buf_read(h, st.d_v, 0, st.h_v, records * page_bytes));
        }
        // Same validation as append_batch, before anything of the group is
        // committed.
        std::vector<std::vector<double>> maxima(g1 - g0);
        for (size_t li = g0; li < g1; ++li) {
            const size_t layer = layers[li].layer;
            maxima[li - g0] = value_abs_max_[layer];
            for (size_t r = 0; r < per_layer; ++r) {
                const size_t i = (li - g0) * per_layer + r;
                const size_t n = descs[i].tokens;
                const uint8_t *kp = st.h_k + i * page_bytes;
                const uint8_t *vp = st.h_v + i * page_bytes;
                bool bad = false;
                if (layer == 0) {
                    bf16_scan(kp, n * kvh * row_bytes / 2, &bad);
                    ensure(!bad, "GPU ColdStore K nonfinite");
                }
                for (size_t hd = 0; hd < kvh; ++hd) {
                    const uint16_t top = bf16_scan(vp + hd * n * row_bytes, n * row_bytes / 2, &bad);
                    ensure(!bad, "GPU ColdStore V nonfinite");
                    maxima[li - g0][hd] = std::max(maxima[li - g0][hd], (double)bf16_to_f32(top));
                }
            }
        }
        std::vector<cold::PreparedPage> prepared;
        if (host_frames) {
            prepared.resize(records);
            parallel_indices(records, host_worker_threads(), [&](size_t i) {
                cold::PageGeometry pg;
                pg.layer = descs[i].layer;
                pg.token_start = descs[i].token_start;
                pg.tokens = descs[i].tokens;
                pg.heads = (uint32_t)kvh;
                pg.head_dim = (uint32_t)geometry_.head_dim;
                pg.tile = tile;
                const size_t len = (size_t)descs[i].tokens * kvh * row_bytes;
                prepared[i] = cold::ColdStore::prepare_page(descs[i].page_id, pg, st.h_k + i * page_bytes, len,
                                                            st.h_v + i * page_bytes, len);
            });
        }
        for (size_t li = g0; li < g1; ++li) {
            const size_t layer = layers[li].layer;
            for (size_t r = 0; r < per_layer; ++r) {
                const size_t i = (li - g0) * per_layer + r;
                const size_t n = descs[i].tokens;
                const cold::PageMeta meta =
                    host_frames ? cold_.append_prepared(std::move(prepared[i]), false)
                                : cold_.append_framed(st.h_frames + i * slot, (size_t)slot, st.h_k + i * page_bytes,
                                                      st.h_v + i * page_bytes, n * kvh * row_bytes, false);
                for (size_t offset = 0; offset < n; ++offset) pages_[layer].push_back({meta.page_id, offset});
                stats.prefill_batched_page_tokens = std::max(stats.prefill_batched_page_tokens, n);
            }
            value_abs_max_[layer] = maxima[li - g0];
            if (layer == 0) axis_tokens_ += count;
        }
        stats.device_sealed_pages += records;
    }
    const cold::ColdStoreStats info = cold_.stats();
    stats.physical_cold_store_bytes = info.committed_bytes;
    stats.physical_cold_store_pages = info.pages;
}

size_t RegionStore::restore_device_layers(DeviceStaging &st, const DevicePagePool &pool,
                                          const std::vector<LayerBlocks> &layers) {
    NativeContext &ctx = st.ctx();
    check_pool(pool, geometry_);
    const size_t P = (size_t)pool.page_tokens;
    const size_t kvh = geometry_.kv_heads, row_bytes = geometry_.head_dim * 2;
    const size_t page_bytes = kvh * P * row_bytes;
    const uint32_t tile = geometry_.head_dim % 16 == 0 ? 16 : 1;
    const int64_t slot = mslim_attn_record_frame_bytes((int)P);
    // Every record of the listed layers, in token order per layer.
    struct Item {
        uint64_t page_id;
        int32_t pool_page;
    };
    std::vector<Item> items;
    for (const LayerBlocks &lb : layers) {
        ensure(lb.layer < pages_.size(), "GPU LOD read layer missing");
        uint64_t last = UINT64_MAX;
        for (const PageAddress &a : pages_[lb.layer]) {
            if (a.page_id == last) continue;
            last = a.page_id;
            const cold::PageMeta &m = cold_.metadata().at(a.page_id);
            const size_t row = m.geometry.token_start % P;
            ensure(row + m.geometry.tokens <= P, "a persisted record does not fit in one device pool page");
            const size_t block = m.geometry.token_start / P;
            ensure(block < lb.blocks.size() && lb.blocks[block] >= 0 && lb.blocks[block] < pool.pool_pages,
                   "device restore pool page out of range");
            items.push_back({a.page_id, lb.blocks[block]});
        }
    }
    const size_t records = items.size();
    if (records == 0) return 0;
    st.reserve(records, (size_t)slot, page_bytes);
    auto *descs = reinterpret_cast<mslim_attn_page_record *>(st.h_desc);
    std::vector<uint8_t> stored(records * slot);
    for (size_t i = 0; i < records; ++i) {
        const cold::PageMeta &m = cold_.metadata().at(items[i].page_id);
        ensure(m.key_len <= page_bytes && m.value_len <= page_bytes, "a persisted record exceeds a pool page");
        cold_.read_record_into(items[i].page_id, (uint32_t)P, stored.data() + i * slot, st.h_k + i * page_bytes,
                               st.h_v + i * page_bytes);
        descs[i].page_id = m.page_id;
        descs[i].token_start = m.geometry.token_start;
        descs[i].layer = m.geometry.layer;
        descs[i].tokens = m.geometry.tokens;
        descs[i].pool_page = items[i].pool_page;
        descs[i].first_row = (uint32_t)(m.geometry.token_start % P);
    }
    std::lock_guard<std::mutex> guard(ctx.mutex());
    void *h = ctx.handle();
    ctx.check("upload record descriptors",
              mslim_attn_buf_write(h, st.d_desc, 0, st.h_desc, records * sizeof(mslim_attn_page_record)));
    ctx.check("upload K payloads", mslim_attn_buf_write(h, st.d_k, 0, st.h_k, records * page_bytes));
    ctx.check("upload V payloads", mslim_attn_buf_write(h, st.d_v, 0, st.h_v, records * page_bytes));
    // Frames recomputed from the staged copies, compared with the stored
    // ones, before the payloads move into the pool.
    ctx.check("staged record frames",
              mslim_attn_record_frames_staged(h, st.d_k, st.d_v, (int)P, (int)kvh, (int)geometry_.head_dim, tile,
                                              static_cast<const mslim_attn_page_record *>(st.d_desc), (int)records,
                                              st.d_frames));
    ctx.check("read record frames", mslim_attn_buf_read(h, st.d_frames, 0, st.h_frames, records * slot));
    for (size_t i = 0; i < records; ++i) {
        const uint8_t *want = stored.data() + i * slot;
        const uint8_t *got = st.h_frames + i * slot;
        const size_t prefix = cold::kHeaderLen + 16ull * descs[i].tokens;
        if (std::memcmp(want, got, prefix) != 0 ||
            std::memcmp(want + slot - cold::kFooterLen, got + slot - cold::kFooterLen, cold::kFooterLen) != 0)
            throw cold::ColdStoreError(cold::ColdStoreError::Kind::InvalidData,
                                       "device verification failed for KV page " + std::to_string(descs[i].page_id));
    }
    ctx.check("record payloads",
              mslim_attn_record_payloads(h, pool.k_pool, pool.v_pool, pool.pool_pages, (int)P, (int)kvh,
                                         (int)geometry_.head_dim,
                                         static_cast<const mslim_attn_page_record *>(st.d_desc), (int)records,
                                         st.d_k, st.d_v, 1));
    ctx.check("restore barrier", mslim_attn_synchronize(h));
    stats.device_restored_pages += records;
    return records;
}

void RegionStore::seal_device_pages(NativeContext &ctx, size_t layer, size_t position, const DevicePagePool &pool,
                                    const std::vector<int32_t> &blocks, size_t count) {
    check_pool(pool, geometry_);
    const size_t P = (size_t)pool.page_tokens;
    std::vector<int32_t> logical(position / P, 0);
    logical.insert(logical.end(), blocks.begin(), blocks.end());
    DeviceStaging st(ctx);
    seal_device_layers(st, position, count, pool, {LayerBlocks{layer, logical}});
}

void RegionStore::restore_to_device(NativeContext &ctx, size_t layer, const DevicePagePool &pool,
                                    const std::vector<int32_t> &blocks) {
    DeviceStaging st(ctx);
    restore_device_layers(st, pool, {LayerBlocks{layer, blocks}});
}

}  // namespace region
}  // namespace mslim
