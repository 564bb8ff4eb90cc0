// ColdStore (cold_store.rs:92-956) over POSIX file descriptors.
#include "cold_store.hpp"

#include <fcntl.h>
#include <sys/file.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <limits.h>
#include <sys/uio.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <cstring>
#include <exception>
#include <mutex>
#include <thread>

#include "../csrc/sha256.hpp"
#include "parallel.hpp"

namespace mslim {
namespace cold {

namespace {

using Kind = ColdStoreError::Kind;

const uint8_t kHeaderMagic[8] = {'T', 'S', 'K', 'V', 'P', 'G', '0', '4'};  // cold_store.rs:20
const uint8_t kFooterMagic[8] = {'T', 'S', 'K', 'V', 'C', 'M', 'I', 'T'};  // cold_store.rs:21
constexpr uint64_t kFnvOffset = 0xcbf29ce484222325ull;
constexpr uint64_t kFnvPrime = 0x100000001b3ull;

[[noreturn]] void invalid(const std::string &message) { throw ColdStoreError(Kind::InvalidData, message); }

[[noreturn]] void io_error(const std::string &what, int err) {
    Kind kind = Kind::Other;
    if (err == ENOENT) kind = Kind::NotFound;
    else if (err == EEXIST) kind = Kind::AlreadyExists;
    else if (err == EWOULDBLOCK || err == EAGAIN) kind = Kind::WouldBlock;
    throw ColdStoreError(kind, what + ": " + std::strerror(err));
}

void put_u32(std::vector<uint8_t> &out, uint32_t v) {
    for (int i = 0; i < 4; ++i) out.push_back((uint8_t)(v >> (8 * i)));
}
void put_u64(std::vector<uint8_t> &out, uint64_t v) {
    for (int i = 0; i < 8; ++i) out.push_back((uint8_t)(v >> (8 * i)));
}
uint32_t get_u32(const uint8_t *p, size_t off) {
    uint32_t v = 0;
    for (int i = 0; i < 4; ++i) v |= (uint32_t)p[off + i] << (8 * i);
    return v;
}
uint64_t get_u64(const uint8_t *p, size_t off) {
    uint64_t v = 0;
    for (int i = 0; i < 8; ++i) v |= (uint64_t)p[off + i] << (8 * i);
    return v;
}

struct Span {
    const uint8_t *p;
    size_t n;
};

// FNV-1a 64 of the same bytes continued in two states: a record checksum and
// a payload checksum read every payload byte in the same order, and the two
// multiply chains overlap in the pipeline instead of running back to back.
void fnv1a64_two(const uint8_t *b, size_t n, uint64_t &first, uint64_t &second) {
    uint64_t x = first, y = second;
    for (size_t i = 0; i < n; ++i) {
        x = (x ^ b[i]) * kFnvPrime;
        y = (y ^ b[i]) * kFnvPrime;
    }
    first = x;
    second = y;
}


uint64_t checksum_many(std::initializer_list<Span> parts) {
    uint64_t s = kFnvOffset;
    for (const Span &part : parts) s = fnv1a64(part.p, part.n, s);
    return s;
}

void digest_many(std::initializer_list<Span> parts, uint8_t out[32]) {
    Sha256 sha;
    for (const Span &part : parts) sha.update(part.p, part.n);
    sha.finish(out);
}

std::vector<uint8_t> u64_bytes(const std::vector<uint64_t> &values) {
    std::vector<uint8_t> out;
    out.reserve(values.size() * 8);
    for (uint64_t v : values) put_u64(out, v);
    return out;
}

// cold_store.rs:706-713
size_t bytes_per_head_token(uint64_t length, const PageGeometry &g) {
    const uint64_t elements = (uint64_t)g.heads * g.tokens;
    if (elements == 0 || length % elements) invalid("KV payload not divisible by heads and tokens");
    return (size_t)(length / elements);
}

// cold_store.rs:690-704
void validate_geometry(const PageGeometry &g, size_t key_len, size_t value_len) {
    if (g.tokens == 0 || g.heads == 0 || g.head_dim == 0 || g.tile == 0) invalid("KV geometry contains zero");
    if (g.head_dim % g.tile) invalid("head_dim is not a multiple of tile");
    if (key_len == 0 || value_len == 0) invalid("converted KV page cannot be empty");
    bytes_per_head_token(key_len, g);
    bytes_per_head_token(value_len, g);
}

// cold_store.rs:752-789: header fields; offsets relative to record_offset.
PageMeta parse_header(const uint8_t *h, uint64_t record_offset) {
    if (std::memcmp(h, kHeaderMagic, 8) != 0) invalid("invalid KV page header");
    if (get_u32(h, 8) != kVersion || get_u32(h, 12) != kHeaderLen) invalid("unsupported KV page version");
    PageMeta m;
    m.geometry.layer = get_u32(h, 24);
    m.geometry.token_start = get_u64(h, 32);
    m.geometry.tokens = get_u32(h, 40);
    m.geometry.heads = get_u32(h, 44);
    m.geometry.head_dim = get_u32(h, 48);
    m.geometry.tile = get_u32(h, 52);
    m.key_len = get_u64(h, 56);
    m.value_len = get_u64(h, 64);
    if (m.key_len == 0 || m.value_len == 0) invalid("invalid cold KV length");
    m.page_id = get_u64(h, 16);
    m.record_offset = record_offset;
    m.key_hashes_offset = record_offset + kHeaderLen;
    m.value_hashes_offset = m.key_hashes_offset + (uint64_t)m.geometry.tokens * 8;
    m.payload_offset = m.value_hashes_offset + (uint64_t)m.geometry.tokens * 8;
    m.key_checksum = get_u64(h, 72);
    m.value_checksum = get_u64(h, 80);
    m.key_hashes_checksum = get_u64(h, 88);
    m.value_hashes_checksum = get_u64(h, 96);
    return m;
}

uint64_t file_len(int fd) {
    struct stat st;
    if (fstat(fd, &st) != 0) io_error("fstat", errno);
    return (uint64_t)st.st_size;
}

// Positional read of exactly n bytes (std::os::unix::fs::FileExt::read_exact_at).
void read_exact_at(int fd, uint64_t offset, uint8_t *out, size_t n) {
    while (n) {
        const ssize_t r = pread(fd, out, n, (off_t)offset);
        if (r < 0) {
            if (errno == EINTR) continue;
            io_error("pread", errno);
        }
        if (r == 0) throw ColdStoreError(Kind::UnexpectedEof, "failed to fill whole buffer");
        out += r;
        n -= (size_t)r;
        offset += (uint64_t)r;
    }
}

// cold_store.rs:791-838
ColdPagePayload read_and_verify(int fd, const PageMeta &m) {
    std::vector<uint8_t> header(kHeaderLen), key_hashes(m.geometry.tokens * 8ull),
        value_hashes(m.geometry.tokens * 8ull);
    ColdPagePayload out;
    out.key.resize(m.key_len);
    out.value.resize(m.value_len);
    read_exact_at(fd, m.record_offset, header.data(), header.size());
    read_exact_at(fd, m.key_hashes_offset, key_hashes.data(), key_hashes.size());
    read_exact_at(fd, m.value_hashes_offset, value_hashes.data(), value_hashes.size());
    read_exact_at(fd, m.payload_offset, out.key.data(), out.key.size());
    read_exact_at(fd, m.payload_offset + m.key_len, out.value.data(), out.value.size());
    const std::string page = std::to_string(m.page_id);
    // The record checksum runs over header, hash tables, K and V; the K and V
    // checksums ride along on the same pass.
    uint64_t record = checksum_many({{header.data(), header.size()},
                                     {key_hashes.data(), key_hashes.size()},
                                     {value_hashes.data(), value_hashes.size()}});
    uint64_t key_sum = kFnvOffset, value_sum = kFnvOffset;
    fnv1a64_two(out.key.data(), out.key.size(), record, key_sum);
    fnv1a64_two(out.value.data(), out.value.size(), record, value_sum);
    if (key_sum != m.key_checksum || value_sum != m.value_checksum ||
        fnv1a64(key_hashes.data(), key_hashes.size()) != m.key_hashes_checksum ||
        fnv1a64(value_hashes.data(), value_hashes.size()) != m.value_hashes_checksum)
        invalid("invalid K/V checksum in page " + page);
    if (u64_bytes(token_hashes(out.key.data(), out.key.size(), m.geometry)) != key_hashes ||
        u64_bytes(token_hashes(out.value.data(), out.value.size(), m.geometry)) != value_hashes)
        invalid("inconsistent per-token hash table in page " + page);
    const std::initializer_list<Span> parts = {{header.data(), header.size()},
                                               {key_hashes.data(), key_hashes.size()},
                                               {value_hashes.data(), value_hashes.size()},
                                               {out.key.data(), out.key.size()},
                                               {out.value.data(), out.value.size()}};
    if (record != m.record_checksum) invalid("invalid record checksum in page " + page);
    uint8_t digest[32];
    digest_many(parts, digest);
    if (std::memcmp(digest, m.record_digest, 32) != 0) invalid("invalid cryptographic digest in page " + page);
    return out;
}

// cold_store.rs:840-893
void verify_mapped_record(const uint8_t *map, uint64_t map_len, const PageMeta &m) {
    auto range = [&](uint64_t offset, uint64_t length) -> Span {
        if (offset > map_len || length > map_len - offset) invalid("truncated mapped KV record");
        return {map + offset, (size_t)length};
    };
    const uint64_t hash_len = m.geometry.tokens * 8ull;
    const Span header = range(m.record_offset, kHeaderLen);
    const Span kh = range(m.key_hashes_offset, hash_len);
    const Span vh = range(m.value_hashes_offset, hash_len);
    const Span key = range(m.payload_offset, m.key_len);
    const Span value = range(m.payload_offset + m.key_len, m.value_len);
    const Span footer = range(m.record_offset + m.record_len - kFooterLen, kFooterLen);
    const std::string page = std::to_string(m.page_id);
    if (std::memcmp(footer.p, kFooterMagic, 8) != 0 || get_u64(footer.p, 8) != m.record_checksum ||
        get_u64(footer.p, 16) != m.record_len || std::memcmp(footer.p + 24, m.record_digest, 32) != 0)
        invalid("invalid mapped commit in page " + page);
    uint64_t record = checksum_many({header, kh, vh});
    uint64_t key_sum = kFnvOffset, value_sum = kFnvOffset;
    fnv1a64_two(key.p, key.n, record, key_sum);
    fnv1a64_two(value.p, value.n, record, value_sum);
    if (key_sum != m.key_checksum || value_sum != m.value_checksum ||
        fnv1a64(kh.p, kh.n) != m.key_hashes_checksum || fnv1a64(vh.p, vh.n) != m.value_hashes_checksum ||
        record != m.record_checksum)
        invalid("invalid mapped checksum in page " + page);
    uint8_t digest[32];
    digest_many({header, kh, vh, key, value}, digest);
    if (std::memcmp(digest, m.record_digest, 32) != 0) invalid("invalid mapped cryptographic digest in page " + page);
    if (u64_bytes(token_hashes(key.p, key.n, m.geometry)) != std::vector<uint8_t>(kh.p, kh.p + kh.n) ||
        u64_bytes(token_hashes(value.p, value.n, m.geometry)) != std::vector<uint8_t>(vh.p, vh.p + vh.n))
        invalid("invalid mapped per-token hash in page " + page);
}

}  // namespace

uint64_t fnv1a64(const uint8_t *bytes, size_t n, uint64_t state) {
    for (size_t i = 0; i < n; ++i) state = (state ^ bytes[i]) * kFnvPrime;
    return state;
}

// cold_store.rs:725-742
std::vector<uint64_t> token_hashes(const uint8_t *payload, size_t len, const PageGeometry &g) {
    const size_t per = bytes_per_head_token(len, g);
    std::vector<uint64_t> out(g.tokens);
    uint32_t t0 = 0;
    // Four tokens at a time: their rows sit side by side in each head's
    // block, and the four chains are independent.
    for (; t0 + 4 <= g.tokens; t0 += 4) {
        uint64_t s0 = kFnvOffset, s1 = kFnvOffset, s2 = kFnvOffset, s3 = kFnvOffset;
        for (uint32_t h = 0; h < g.heads; ++h) {
            const uint8_t *p = payload + ((size_t)h * g.tokens + t0) * per;
            for (size_t i = 0; i < per; ++i) {
                s0 = (s0 ^ p[i]) * kFnvPrime;
                s1 = (s1 ^ p[per + i]) * kFnvPrime;
                s2 = (s2 ^ p[2 * per + i]) * kFnvPrime;
                s3 = (s3 ^ p[3 * per + i]) * kFnvPrime;
            }
        }
        out[t0] = s0;
        out[t0 + 1] = s1;
        out[t0 + 2] = s2;
        out[t0 + 3] = s3;
    }
    for (uint32_t t = t0; t < g.tokens; ++t) {
        uint64_t s = kFnvOffset;
        for (uint32_t h = 0; h < g.heads; ++h) s = fnv1a64(payload + ((size_t)h * g.tokens + t) * per, per, s);
        out[t] = s;
    }
    return out;
}

// ---- construction -----------------------------------------------------------

ColdStore::ColdStore(std::string path, int fd, bool read_only, size_t hot_capacity)
    : path_(std::move(path)), fd_(fd), read_only_(read_only), hot_capacity_(hot_capacity) {}

ColdStore::ColdStore(ColdStore &&o) noexcept { *this = std::move(o); }

ColdStore &ColdStore::operator=(ColdStore &&o) noexcept {
    if (this != &o) {
        if (fd_ >= 0) ::close(fd_);
        path_ = std::move(o.path_);
        fd_ = o.fd_;
        o.fd_ = -1;
        read_only_ = o.read_only_;
        pages_ = std::move(o.pages_);
        hot_capacity_ = o.hot_capacity_;
        hot_ = std::move(o.hot_);
        hash_tables_ = std::move(o.hash_tables_);
        lru_ = std::move(o.lru_);
        reads_ = o.reads_; hits_ = o.hits_; misses_ = o.misses_; evictions_ = o.evictions_;
        committed_bytes_ = o.committed_bytes_; bytes_read_ = o.bytes_read_;
        partial_value_reads_ = o.partial_value_reads_;
        partial_value_payload_bytes_ = o.partial_value_payload_bytes_;
        partial_value_bytes_avoided_ = o.partial_value_bytes_avoided_;
        partial_key_reads_ = o.partial_key_reads_;
        partial_key_payload_bytes_ = o.partial_key_payload_bytes_;
        partial_key_bytes_avoided_ = o.partial_key_bytes_avoided_;
        cryptographic_digests_verified_ = o.cryptographic_digests_verified_;
        fail_append_after_bytes_ = o.fail_append_after_bytes_;
    }
    return *this;
}

ColdStore::~ColdStore() {
    if (fd_ >= 0) ::close(fd_);  // closing releases the writer lock
}

namespace {
// cold_store.rs:121-133: one exclusive writer per file.
void lock_exclusive_writer(int fd, const std::string &path) {
    if (flock(fd, LOCK_EX | LOCK_NB) == 0) return;
    const int err = errno;
    ::close(fd);
    if (err == EWOULDBLOCK)
        throw ColdStoreError(Kind::WouldBlock, "ColdStore " + path + " already has an exclusive writer");
    io_error("lock " + path, err);
}
}  // namespace

ColdStore ColdStore::create(const std::string &path, size_t hot_capacity) {
    const int fd = ::open(path.c_str(), O_CREAT | O_EXCL | O_RDWR | O_APPEND | O_CLOEXEC, 0644);
    if (fd < 0) io_error("create " + path, errno);
    lock_exclusive_writer(fd, path);
    return ColdStore(path, fd, false, hot_capacity);
}

ColdStore ColdStore::open(const std::string &path, size_t hot_capacity) {
    const int fd = ::open(path.c_str(), O_RDWR | O_APPEND | O_CLOEXEC);
    if (fd < 0) io_error("open " + path, errno);
    lock_exclusive_writer(fd, path);
    ColdStore store(path, fd, false, hot_capacity);
    store.rebuild_catalogue();
    return store;
}

ColdStore ColdStore::open_read_only(const std::string &path, size_t hot_capacity) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) io_error("open " + path, errno);
    ColdStore store(path, fd, true, hot_capacity);
    store.rebuild_catalogue();
    return store;
}

ColdStoreStats ColdStore::stats() const {
    ColdStoreStats s;
    s.pages = pages_.size();
    s.committed_bytes = committed_bytes_;
    s.reads = reads_;
    s.cache_hits = hits_;
    s.cache_misses = misses_;
    s.evictions = evictions_;
    s.hot_pages = hot_.size();
    for (const auto &kv : hot_) s.hot_bytes += kv.second->key.size() + kv.second->value.size();
    s.hot_capacity = hot_capacity_;
    s.bytes_read = bytes_read_;
    s.partial_value_reads = partial_value_reads_;
    s.partial_value_payload_bytes = partial_value_payload_bytes_;
    s.partial_value_bytes_avoided = partial_value_bytes_avoided_;
    s.partial_key_reads = partial_key_reads_;
    s.partial_key_payload_bytes = partial_key_payload_bytes_;
    s.partial_key_bytes_avoided = partial_key_bytes_avoided_;
    s.cryptographic_digests_verified = cryptographic_digests_verified_;
    return s;
}

// ---- integrity ---------------------------------------------------------------

void ColdStore::audit_mapped() {
    if (!read_only_ && fdatasync(fd_) != 0) io_error("sync " + path_, errno);
    const uint64_t len = file_len(fd_);
    if (len == 0) invalid("empty KV store cannot be mapped");
    void *map = mmap(nullptr, (size_t)len, PROT_READ, MAP_SHARED, fd_, 0);
    if (map == MAP_FAILED) io_error("mmap " + path_, errno);
    const uint8_t *bytes = static_cast<const uint8_t *>(map);
    try {
        parallel_indices(pages_.size(), host_worker_threads(),
                         [&](size_t i) { verify_mapped_record(bytes, len, pages_[i]); });
    } catch (...) {
        munmap(map, (size_t)len);
        throw;
    }
    munmap(map, (size_t)len);
    cryptographic_digests_verified_ += pages_.size();
}

void ColdStore::audit() const {
    parallel_indices(pages_.size(), host_worker_threads(), [&](size_t i) { read_and_verify(fd_, pages_[i]); });
}

// ---- append ------------------------------------------------------------------

PageMeta ColdStore::append_page(const PageGeometry &geometry, const uint8_t *key, size_t key_len,
                                const uint8_t *value, size_t value_len, bool durable) {
    return append_prepared(prepare_page(pages_.size(), geometry, key, key_len, value, value_len), durable);
}

PreparedPage ColdStore::prepare_page(uint64_t page_id, const PageGeometry &g, const uint8_t *key,
                                     size_t key_len, const uint8_t *value, size_t value_len) {
    validate_geometry(g, key_len, value_len);
    PageMeta m;
    m.page_id = page_id;
    m.geometry = g;
    m.key_len = key_len;
    m.value_len = value_len;
    m.key_checksum = fnv1a64(key, key_len);
    m.value_checksum = fnv1a64(value, value_len);
    const std::vector<uint8_t> kh = u64_bytes(token_hashes(key, key_len, g));
    const std::vector<uint8_t> vh = u64_bytes(token_hashes(value, value_len, g));
    m.key_hashes_checksum = fnv1a64(kh.data(), kh.size());
    m.value_hashes_checksum = fnv1a64(vh.data(), vh.size());

    std::vector<uint8_t> header;
    header.reserve(kHeaderLen);
    header.insert(header.end(), kHeaderMagic, kHeaderMagic + 8);
    put_u32(header, kVersion);
    put_u32(header, (uint32_t)kHeaderLen);
    put_u64(header, page_id);
    put_u32(header, g.layer);
    put_u32(header, 0);
    put_u64(header, g.token_start);
    put_u32(header, g.tokens);
    put_u32(header, g.heads);
    put_u32(header, g.head_dim);
    put_u32(header, g.tile);
    put_u64(header, key_len);
    put_u64(header, value_len);
    put_u64(header, m.key_checksum);
    put_u64(header, m.value_checksum);
    put_u64(header, m.key_hashes_checksum);
    put_u64(header, m.value_hashes_checksum);

    const std::initializer_list<Span> parts = {
        {header.data(), header.size()}, {kh.data(), kh.size()}, {vh.data(), vh.size()}, {key, key_len}, {value, value_len}};
    m.record_checksum = checksum_many(parts);
    digest_many(parts, m.record_digest);
    m.record_len = kHeaderLen + kh.size() + vh.size() + key_len + value_len + kFooterLen;

    PreparedPage p;
    p.record.reserve(m.record_len);
    for (const Span &s : parts) p.record.insert(p.record.end(), s.p, s.p + s.n);
    p.record.insert(p.record.end(), kFooterMagic, kFooterMagic + 8);
    put_u64(p.record, m.record_checksum);
    put_u64(p.record, m.record_len);
    p.record.insert(p.record.end(), m.record_digest, m.record_digest + 32);
    m.key_hashes_offset = kHeaderLen;
    m.value_hashes_offset = kHeaderLen + kh.size();
    m.payload_offset = m.value_hashes_offset + vh.size();
    p.meta = m;
    return p;
}

uint64_t ColdStore::committed_end() const {
    return pages_.empty() ? 0 : pages_.back().record_offset + pages_.back().record_len;
}

void ColdStore::write_record(const uint8_t *const *parts, const size_t *lens, int nparts, bool durable) {
    std::vector<struct iovec> iov;
    size_t total = 0;
    for (int i = 0; i < nparts; ++i) {
        iov.push_back({const_cast<uint8_t *>(parts[i]), lens[i]});
        total += lens[i];
    }
    bool simulated_failure = false;
    if (fail_append_after_bytes_) {
        size_t limit = std::min(*fail_append_after_bytes_, total);
        fail_append_after_bytes_.reset();
        simulated_failure = true;
        // Keep only the first `limit` bytes of the parts.
        std::vector<struct iovec> cut;
        for (const auto &v : iov) {
            if (!limit) break;
            const size_t n = std::min(limit, v.iov_len);
            cut.push_back({v.iov_base, n});
            limit -= n;
        }
        iov.swap(cut);
    }
    size_t idx = 0;
    while (idx < iov.size()) {
        const ssize_t w = writev(fd_, iov.data() + idx, (int)std::min<size_t>(iov.size() - idx, IOV_MAX));
        if (w < 0) {
            if (errno == EINTR) continue;
            io_error("write " + path_, errno);
        }
        size_t left = (size_t)w;
        while (idx < iov.size() && left >= iov[idx].iov_len) left -= iov[idx++].iov_len;
        if (idx < iov.size()) {
            iov[idx].iov_base = static_cast<uint8_t *>(iov[idx].iov_base) + left;
            iov[idx].iov_len -= left;
        }
    }
    if (simulated_failure) throw ColdStoreError(Kind::Other, "simulated write failure");
    if (durable && fdatasync(fd_) != 0) io_error("sync " + path_, errno);
}

PageMeta ColdStore::commit(PageMeta meta, const uint8_t *const *parts, const size_t *lens, int nparts,
                           bool durable) {
    // cold_store.rs:367-389: a record is written at the end of the committed
    // records (bytes an earlier failed append left there are cut off first);
    // if this write fails, the file is cut back to that same offset.
    const uint64_t record_offset = committed_end();
    if (file_len(fd_) != record_offset && ftruncate(fd_, (off_t)record_offset) != 0)
        io_error("truncate " + path_, errno);
    try {
        write_record(parts, lens, nparts, durable);
    } catch (...) {
        if (ftruncate(fd_, (off_t)record_offset) != 0) {
            // The next append retries the rollback through the check above.
        }
        throw;
    }
    meta.record_offset = record_offset;
    meta.key_hashes_offset += record_offset;
    meta.value_hashes_offset += record_offset;
    meta.payload_offset += record_offset;
    committed_bytes_ += meta.record_len;
    pages_.push_back(meta);
    return meta;
}

PageMeta ColdStore::append_prepared(PreparedPage prepared, bool durable) {
    if (read_only_) invalid("immutable KV store does not accept appends");
    if (prepared.meta.page_id != pages_.size()) invalid("prepared KV sequence is not monotonic");
    if (prepared.record.size() != prepared.meta.record_len) invalid("prepared KV record has an invalid length");
    const uint8_t *parts[1] = {prepared.record.data()};
    const size_t lens[1] = {prepared.record.size()};
    return commit(prepared.meta, parts, lens, 1, durable);
}

PageMeta ColdStore::append_framed(const uint8_t *frame, size_t frame_len, const uint8_t *key,
                                  const uint8_t *value, size_t payload_len, bool durable) {
    if (read_only_) invalid("immutable KV store does not accept appends");
    if (frame_len < kHeaderLen + kFooterLen) invalid("KV frame too short");
    PageMeta m = parse_header(frame, 0);
    if (m.page_id != pages_.size()) invalid("framed KV sequence is not monotonic");
    if (m.key_len != payload_len || m.value_len != payload_len) invalid("KV frame does not describe the payloads");
    validate_geometry(m.geometry, payload_len, payload_len);
    const size_t prefix = kHeaderLen + 16ull * m.geometry.tokens;
    if (prefix + kFooterLen > frame_len) invalid("KV frame too short for its token tables");
    const uint8_t *footer = frame + frame_len - kFooterLen;
    m.record_len = prefix + 2ull * payload_len + kFooterLen;
    if (std::memcmp(footer, kFooterMagic, 8) != 0) invalid("invalid KV frame commit footer");
    if (get_u64(footer, 16) != m.record_len) invalid("inconsistent KV frame record length");
    m.record_checksum = get_u64(footer, 8);
    std::memcpy(m.record_digest, footer + 24, 32);
    const uint8_t *parts[4] = {frame, key, value, footer};
    const size_t lens[4] = {prefix, payload_len, payload_len, kFooterLen};
    return commit(m, parts, lens, 4, durable);
}

// ---- catalogue ---------------------------------------------------------------

void ColdStore::rebuild_catalogue() {
    // cold_store.rs:641-687: walk the headers and footers in file order, then
    // verify every record (on several threads; the first failure in file
    // order is the one reported, before any structural error found later in
    // the file, as the sequential walk reports).
    const uint64_t len = file_len(fd_);
    uint64_t offset = 0;
    std::vector<PageMeta> found;
    std::exception_ptr structural;
    try {
        while (offset < len) {
            const uint64_t remaining = len - offset;
            // Too short for a header: a write stopped before any record
            // could commit, so the file's store ends here.
            if (remaining < kHeaderLen) break;
            uint8_t header[kHeaderLen];
            read_exact_at(fd_, offset, header, kHeaderLen);
            PageMeta m = parse_header(header, offset);
            const uint64_t record_len =
                kHeaderLen + (uint64_t)m.geometry.tokens * 16 + m.key_len + m.value_len + kFooterLen;
            // The header promises more bytes than the file holds, so the
            // footer of this record was never written: not committed either.
            if (record_len > remaining) break;
            uint8_t footer[kFooterLen];
            read_exact_at(fd_, offset + record_len - kFooterLen, footer, kFooterLen);
            if (std::memcmp(footer, kFooterMagic, 8) != 0) invalid("invalid KV commit footer");
            if (get_u64(footer, 16) != record_len) invalid("inconsistent KV record length");
            if (m.page_id != found.size()) invalid("KV page_id sequence is not monotonic");
            m.record_checksum = get_u64(footer, 8);
            std::memcpy(m.record_digest, footer + 24, 32);
            m.record_len = record_len;
            found.push_back(m);
            offset += record_len;
        }
    } catch (const ColdStoreError &) {
        structural = std::current_exception();
    }
    parallel_indices(found.size(), host_worker_threads(), [&](size_t i) { read_and_verify(fd_, found[i]); });
    if (structural) std::rethrow_exception(structural);
    for (const PageMeta &m : found) committed_bytes_ += m.record_len;
    pages_ = std::move(found);
    // Recovery cuts the file to the end of its last complete record, so the
    // next append lands where a later open finds it; a store opened read-only
    // leaves the file untouched and simply stops reading at that point.
    if (offset < len && !read_only_) {
        if (ftruncate(fd_, (off_t)offset) != 0) io_error("truncate " + path_, errno);
        if (fdatasync(fd_) != 0) io_error("sync " + path_, errno);
    }
}

const PageMeta &ColdStore::page_meta(uint64_t page_id) const {
    if (page_id >= pages_.size() || pages_[page_id].page_id != page_id)
        throw ColdStoreError(Kind::NotFound, "KV page " + std::to_string(page_id) + " absent");
    return pages_[page_id];
}

void ColdStore::touch(uint64_t page_id) {
    auto it = std::find(lru_.begin(), lru_.end(), page_id);
    if (it != lru_.end()) lru_.erase(it);
    lru_.push_back(page_id);
}

// ---- reads -------------------------------------------------------------------

std::shared_ptr<const ColdPagePayload> ColdStore::read_page(uint64_t page_id) {
    auto hot = hot_.find(page_id);
    if (hot != hot_.end()) {
        ++hits_;
        auto page = hot->second;
        touch(page_id);
        return page;
    }
    const PageMeta m = page_meta(page_id);
    ++misses_;
    ++reads_;
    auto payload = std::make_shared<const ColdPagePayload>(read_and_verify(fd_, m));
    ++cryptographic_digests_verified_;
    bytes_read_ += m.record_len - kFooterLen;
    if (hot_capacity_ > 0) {
        while (hot_.size() >= hot_capacity_ && !lru_.empty()) {
            const uint64_t oldest = lru_.front();
            lru_.pop_front();
            if (hot_.erase(oldest)) ++evictions_;
        }
        hot_[page_id] = payload;
        touch(page_id);
    }
    return payload;
}

void ColdStore::for_each_verified(const std::vector<uint64_t> &ids,
                                  const std::function<void(size_t, const ColdPagePayload &)> &fn) {
    std::vector<const PageMeta *> metas;
    metas.reserve(ids.size());
    for (uint64_t id : ids) metas.push_back(&page_meta(id));
    parallel_indices(ids.size(), host_worker_threads(), [&](size_t i) { fn(i, read_and_verify(fd_, *metas[i])); });
    for (const PageMeta *m : metas) {
        ++misses_;
        ++reads_;
        ++cryptographic_digests_verified_;
        bytes_read_ += m->record_len - kFooterLen;
    }
}

std::vector<uint8_t> ColdStore::read_key(uint64_t page_id) {
    const PageMeta m = page_meta(page_id);
    std::vector<uint8_t> key(m.key_len);
    read_exact_at(fd_, m.payload_offset, key.data(), key.size());
    if (fnv1a64(key.data(), key.size()) != m.key_checksum) invalid("invalid cold K checksum");
    ++reads_;
    ++misses_;
    bytes_read_ += m.key_len;
    return key;
}

std::vector<uint8_t> ColdStore::read_value(uint64_t page_id) {
    const PageMeta m = page_meta(page_id);
    std::vector<uint8_t> value(m.value_len);
    read_exact_at(fd_, m.payload_offset + m.key_len, value.data(), value.size());
    if (fnv1a64(value.data(), value.size()) != m.value_checksum) invalid("invalid cold V checksum");
    ++reads_;
    ++misses_;
    bytes_read_ += m.value_len;
    return value;
}

std::vector<uint8_t> ColdStore::read_value_tokens(uint64_t page_id, const std::vector<size_t> &t) {
    return read_token_subset(page_id, t, false);
}

std::vector<uint8_t> ColdStore::read_key_tokens(uint64_t page_id, const std::vector<size_t> &t) {
    return read_token_subset(page_id, t, true);
}

std::shared_ptr<const std::vector<uint64_t>> ColdStore::read_hash_table(uint64_t offset, size_t tokens,
                                                                        uint64_t expected) {
    auto it = hash_tables_.find(offset);
    if (it != hash_tables_.end()) return it->second;
    std::vector<uint8_t> bytes(tokens * 8);
    read_exact_at(fd_, offset, bytes.data(), bytes.size());
    if (fnv1a64(bytes.data(), bytes.size()) != expected) invalid("invalid per-token hash table");
    auto table = std::make_shared<std::vector<uint64_t>>(tokens);
    for (size_t i = 0; i < tokens; ++i) (*table)[i] = get_u64(bytes.data(), i * 8);
    hash_tables_[offset] = table;
    return table;
}

// cold_store.rs:502-593
std::vector<uint8_t> ColdStore::read_token_subset(uint64_t page_id, const std::vector<size_t> &idx, bool key) {
    const PageMeta m = page_meta(page_id);
    const size_t tokens = m.geometry.tokens;
    if (idx.empty() || std::any_of(idx.begin(), idx.end(), [&](size_t t) { return t >= tokens; }))
        invalid("invalid partial KV coordinates");
    for (size_t i = 1; i < idx.size(); ++i)
        if (idx[i - 1] >= idx[i]) invalid("partial KV coordinates must be strictly increasing");
    if (idx.size() == tokens) {
        bool all = true;
        for (size_t i = 0; i < tokens; ++i) all = all && idx[i] == i;
        if (all) return key ? read_key(page_id) : read_value(page_id);
    }
    const uint64_t hashes_offset = key ? m.key_hashes_offset : m.value_hashes_offset;
    const uint64_t hashes_checksum = key ? m.key_hashes_checksum : m.value_hashes_checksum;
    const uint64_t payload_offset = key ? m.payload_offset : m.payload_offset + m.key_len;
    const uint64_t payload_len = key ? m.key_len : m.value_len;
    auto hashes = read_hash_table(hashes_offset, tokens, hashes_checksum);
    const size_t heads = m.geometry.heads;
    const size_t per = bytes_per_head_token(payload_len, m.geometry);
    std::vector<uint8_t> out(heads * idx.size() * per);
    size_t pos = 0;
    for (size_t h = 0; h < heads; ++h) {
        size_t run_start = 0;
        while (run_start < idx.size()) {
            size_t run_end = run_start + 1;
            while (run_end < idx.size() && idx[run_end] == idx[run_end - 1] + 1) ++run_end;
            const uint64_t source = payload_offset + (h * tokens + idx[run_start]) * per;
            const size_t n = (run_end - run_start) * per;
            read_exact_at(fd_, source, out.data() + pos, n);
            pos += n;
            run_start = run_end;
        }
    }
    // Hashes cover all heads of a token while the output is head-major.
    for (size_t sel = 0; sel < idx.size(); ++sel) {
        uint64_t s = 0xcbf29ce484222325ull;
        for (size_t h = 0; h < heads; ++h) s = fnv1a64(out.data() + (h * idx.size() + sel) * per, per, s);
        if (s != (*hashes)[idx[sel]])
            invalid(std::string("invalid ") + (key ? "K" : "V") + " checksum of token " + std::to_string(idx[sel]) +
                    " in page " + std::to_string(page_id));
    }
    ++reads_;
    ++misses_;
    bytes_read_ += tokens * 8 + out.size();
    if (key) {
        ++partial_key_reads_;
        partial_key_payload_bytes_ += out.size();
        partial_key_bytes_avoided_ += m.key_len - out.size();
    } else {
        ++partial_value_reads_;
        partial_value_payload_bytes_ += out.size();
        partial_value_bytes_avoided_ += m.value_len - out.size();
    }
    return out;
}

void ColdStore::read_record_raw(uint64_t page_id, uint32_t slot_tokens, std::vector<uint8_t> &frame,
                                std::vector<uint8_t> &key, std::vector<uint8_t> &value) {
    const PageMeta &m = page_meta(page_id);
    frame.resize(kHeaderLen + 16ull * slot_tokens + kFooterLen);
    key.resize(m.key_len);
    value.resize(m.value_len);
    read_record_into(page_id, slot_tokens, frame.data(), key.data(), value.data());
}

void ColdStore::read_record_into(uint64_t page_id, uint32_t slot_tokens, uint8_t *frame, uint8_t *key,
                                 uint8_t *value) {
    const PageMeta m = page_meta(page_id);
    if (m.geometry.tokens > slot_tokens) invalid("KV record has more tokens than the frame slot");
    const size_t prefix = kHeaderLen + 16ull * m.geometry.tokens;
    const size_t frame_len = kHeaderLen + 16ull * slot_tokens + kFooterLen;
    // Header and hash tables, then (after the payloads) the footer: the
    // record's first `prefix` bytes and its last kFooterLen bytes.
    read_exact_at(fd_, m.record_offset, frame, prefix);
    std::memset(frame + prefix, 0, frame_len - kFooterLen - prefix);
    read_exact_at(fd_, m.record_offset + m.record_len - kFooterLen, frame + frame_len - kFooterLen, kFooterLen);
    read_exact_at(fd_, m.payload_offset, key, m.key_len);
    read_exact_at(fd_, m.payload_offset + m.key_len, value, m.value_len);
    ++reads_;
    ++misses_;
    bytes_read_ += m.record_len;
}

}  // namespace cold
}  // namespace mslim
