// Append-only ColdStore of exact BF16 K/V pages (cold_store.rs:92-956):
// the same self-describing record format, commit footer, torn-tail recovery,
// verified whole-page and per-token partial reads, bounded LRU residency and
// statistics as the reference, so files are interchangeable between the two.
//
// Record (cold_store.rs:269-349), all integers little-endian:
//   header (104 B): "TSKVPG04", version 3, header length, page_id, layer, 0,
//     token_start, tokens, heads, head_dim, tile, key_len, value_len,
//     FNV(key), FNV(value), FNV(key hash table), FNV(value hash table)
//   key token hashes  (u64 per token: FNV-1a-64 of that token over all heads)
//   value token hashes
//   key payload   [heads][tokens][bytes per head-token]
//   value payload [heads][tokens][bytes per head-token]
//   footer (56 B): "TSKVCMIT", FNV(record before the footer), record length,
//     SHA-256(record before the footer)
//
// Errors are ColdStoreError carrying the std::io::ErrorKind the reference
// returns for the same condition.
#pragma once

#include <cstddef>
#include <cstdint>
#include <deque>
#include <functional>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

namespace mslim {
namespace cold {

constexpr size_t kHeaderLen = 104;  // cold_store.rs:23
constexpr size_t kFooterLen = 56;   // cold_store.rs:24
constexpr uint32_t kVersion = 3;    // cold_store.rs:22

class ColdStoreError : public std::runtime_error {
public:
    // The io::ErrorKind values the reference produces (cold_store.rs).
    enum class Kind { NotFound, InvalidData, WouldBlock, AlreadyExists, UnexpectedEof, Other };
    ColdStoreError(Kind kind, const std::string &message) : std::runtime_error(message), kind_(kind) {}
    Kind kind() const { return kind_; }

private:
    Kind kind_;
};

// cold_store.rs:28-36
struct PageGeometry {
    uint32_t layer = 0;
    uint64_t token_start = 0;
    uint32_t tokens = 0;
    uint32_t heads = 0;
    uint32_t head_dim = 0;
    uint32_t tile = 0;
    bool operator==(const PageGeometry &o) const {
        return layer == o.layer && token_start == o.token_start && tokens == o.tokens && heads == o.heads &&
               head_dim == o.head_dim && tile == o.tile;
    }
};

// cold_store.rs:38-42
struct ColdPagePayload {
    std::vector<uint8_t> key;
    std::vector<uint8_t> value;
};

// cold_store.rs:44-61
struct PageMeta {
    uint64_t page_id = 0;
    PageGeometry geometry;
    uint64_t record_offset = 0;
    uint64_t payload_offset = 0;
    uint64_t key_hashes_offset = 0;
    uint64_t value_hashes_offset = 0;
    uint64_t key_len = 0;
    uint64_t value_len = 0;
    uint64_t key_checksum = 0;
    uint64_t value_checksum = 0;
    uint64_t key_hashes_checksum = 0;
    uint64_t value_hashes_checksum = 0;
    uint64_t record_checksum = 0;
    uint8_t record_digest[32] = {};
    uint64_t record_len = 0;
};

// cold_store.rs:63-68: one record's bytes built outside the store (on any
// thread); the offsets in its metadata count from the record's first byte
// until append places it in the file.
struct PreparedPage {
    PageMeta meta;
    std::vector<uint8_t> record;
};

// cold_store.rs:70-89
struct ColdStoreStats {
    size_t pages = 0;
    uint64_t committed_bytes = 0;
    uint64_t reads = 0;
    uint64_t cache_hits = 0;
    uint64_t cache_misses = 0;
    uint64_t evictions = 0;
    size_t hot_pages = 0;
    size_t hot_bytes = 0;
    size_t hot_capacity = 0;
    uint64_t bytes_read = 0;
    uint64_t partial_value_reads = 0;
    uint64_t partial_value_payload_bytes = 0;
    uint64_t partial_value_bytes_avoided = 0;
    uint64_t partial_key_reads = 0;
    uint64_t partial_key_payload_bytes = 0;
    uint64_t partial_key_bytes_avoided = 0;
    uint64_t cryptographic_digests_verified = 0;
};

// FNV-1a-64 (cold_store.rs:909-922) and the per-token table (:725-742).
uint64_t fnv1a64(const uint8_t *bytes, size_t n, uint64_t state = 0xcbf29ce484222325ull);
std::vector<uint64_t> token_hashes(const uint8_t *payload, size_t len, const PageGeometry &g);

class ColdStore {
public:
    // cold_store.rs:135-170
    static ColdStore create(const std::string &path, size_t hot_capacity);
    static ColdStore open(const std::string &path, size_t hot_capacity);
    static ColdStore open_read_only(const std::string &path, size_t hot_capacity);
    ColdStore(ColdStore &&other) noexcept;
    ColdStore &operator=(ColdStore &&other) noexcept;
    ColdStore(const ColdStore &) = delete;
    ColdStore &operator=(const ColdStore &) = delete;
    ~ColdStore();

    bool is_read_only() const { return read_only_; }
    const std::string &path() const { return path_; }
    const std::vector<PageMeta> &metadata() const { return pages_; }
    ColdStoreStats stats() const;

    // cold_store.rs:242-259: verify every committed record through a
    // read-only mapping, records in parallel.
    void audit_mapped();
    // cold_store.rs:261-273
    PageMeta append_page(const PageGeometry &geometry, const uint8_t *key, size_t key_len,
                         const uint8_t *value, size_t value_len, bool durable);
    PageMeta append_page(const PageGeometry &g, const std::vector<uint8_t> &k, const std::vector<uint8_t> &v,
                         bool durable) {
        return append_page(g, k.data(), k.size(), v.data(), v.size(), durable);
    }
    // cold_store.rs:275-349
    static PreparedPage prepare_page(uint64_t page_id, const PageGeometry &geometry, const uint8_t *key,
                                     size_t key_len, const uint8_t *value, size_t value_len);
    // cold_store.rs:353-390
    PageMeta append_prepared(PreparedPage prepared, bool durable);
    // Appends a record whose header, token-hash tables and footer were
    // computed elsewhere (the device codec, mslim_attn_record_frames) from the
    // same payload bytes.  `frame` is prefix (header + both tables) followed
    // at frame_len - 56 by the footer.  The header must describe the payloads
    // given, carry the next page id, and the footer must carry the record
    // length; the checksums are taken as computed.
    PageMeta append_framed(const uint8_t *frame, size_t frame_len, const uint8_t *key, const uint8_t *value,
                           size_t payload_len, bool durable);

    // cold_store.rs:412-447
    std::shared_ptr<const ColdPagePayload> read_page(uint64_t page_id);
    // read_page for many records at once, on several threads: each record is
    // read and verified afresh (the LRU cache is neither consulted nor
    // filled) and handed to fn(i, payload) for ids[i], possibly concurrently;
    // reads are counted as read_page misses.  The failure of the smallest
    // index is rethrown, the one a sequential loop would report first.
    void for_each_verified(const std::vector<uint64_t> &ids,
                           const std::function<void(size_t, const ColdPagePayload &)> &fn);
    // cold_store.rs:449-477
    std::vector<uint8_t> read_key(uint64_t page_id);
    std::vector<uint8_t> read_value(uint64_t page_id);
    // cold_store.rs:479-500: head-major [heads][selected][bytes per head-token].
    std::vector<uint8_t> read_value_tokens(uint64_t page_id, const std::vector<size_t> &token_indices);
    std::vector<uint8_t> read_key_tokens(uint64_t page_id, const std::vector<size_t> &token_indices);
    // Raw committed bytes of a record without host verification: the frame
    // (header | tables | footer, laid out like mslim_attn_record_frames with
    // page_tokens slots) and both payloads.  For a caller that verifies on the
    // device by recomputing the frame.
    void read_record_raw(uint64_t page_id, uint32_t slot_tokens, std::vector<uint8_t> &frame,
                         std::vector<uint8_t> &key, std::vector<uint8_t> &value);
    // The same into caller buffers: `frame` of kHeaderLen + 16 * slot_tokens
    // + kFooterLen bytes (the rows of absent tokens zeroed), `key` and
    // `value` of the record's payload lengths.
    void read_record_into(uint64_t page_id, uint32_t slot_tokens, uint8_t *frame, uint8_t *key, uint8_t *value);
    // cold_store.rs:627-633
    void audit() const;

    // Test hook (cold_store.rs:116-119, fail_append_after_bytes): the next
    // append writes that many bytes of its record, then reports an I/O error
    // (a short write that leaves a partial record in the file).
    void fail_next_append_after(size_t bytes) { fail_append_after_bytes_ = bytes; }
    bool hot_contains(uint64_t page_id) const { return hot_.count(page_id) != 0; }

private:
    ColdStore(std::string path, int fd, bool read_only, size_t hot_capacity);
    void rebuild_catalogue();
    uint64_t committed_end() const;
    void write_record(const uint8_t *const *parts, const size_t *lens, int nparts, bool durable);
    const PageMeta &page_meta(uint64_t page_id) const;
    std::vector<uint8_t> read_token_subset(uint64_t page_id, const std::vector<size_t> &tokens, bool key);
    std::shared_ptr<const std::vector<uint64_t>> read_hash_table(uint64_t offset, size_t tokens,
                                                                 uint64_t expected_checksum);
    void touch(uint64_t page_id);
    PageMeta commit(PageMeta meta, const uint8_t *const *parts, const size_t *lens, int nparts, bool durable);

    std::string path_;
    int fd_ = -1;
    bool read_only_ = false;
    std::vector<PageMeta> pages_;
    size_t hot_capacity_ = 0;
    std::unordered_map<uint64_t, std::shared_ptr<const ColdPagePayload>> hot_;
    std::unordered_map<uint64_t, std::shared_ptr<const std::vector<uint64_t>>> hash_tables_;
    std::deque<uint64_t> lru_;
    uint64_t reads_ = 0, hits_ = 0, misses_ = 0, evictions_ = 0, committed_bytes_ = 0, bytes_read_ = 0;
    uint64_t partial_value_reads_ = 0, partial_value_payload_bytes_ = 0, partial_value_bytes_avoided_ = 0;
    uint64_t partial_key_reads_ = 0, partial_key_payload_bytes_ = 0, partial_key_bytes_avoided_ = 0;
    uint64_t cryptographic_digests_verified_ = 0;
    std::optional<size_t> fail_append_after_bytes_;
};

}  // namespace cold
}  // namespace mslim
