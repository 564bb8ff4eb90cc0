// ColdStore record codec for pages already resident in the device pool.
//
// A ColdStore record (cold_store.rs:269-349) is
//   header[104] | K token hashes[8*tokens] | V token hashes[8*tokens] |
//   K payload | V payload | footer[56]
// where the payloads are head-major [heads][tokens][row] byte images.  A
// pool page is exactly such a payload (page_tokens rows per head), so the
// bytes that make a record out of a pool page are the "frame": the header,
// both token-hash tables and the footer.  This file computes frames on the
// device; the host writes frame prefix | payloads | footer to the file (seal)
// or compares a stored record's frame with a recomputed one (verified
// restore).  Every value is byte-identical to the host codec.
//
// A record's tokens are rows first_row .. first_row + tokens - 1 of its pool
// page (a record can start inside a page when a turn ended there).  In staged
// mode the payloads are read instead from compacted staging slots (slot i of
// k_pool / v_pool holds record i as [heads][tokens][row], the layout
// record_payloads writes), so a stored record can be verified before any of
// its bytes reach the pool.
//
// Two launches:
//   * token_hashes_kernel: one lane per (record, K/V, token) computes the
//     FNV-1a-64 of that token's bytes over all heads (cold_store.rs:725-742).
//     These lanes are independent, so this launch streams the payloads at
//     close to HBM rate;
//   * frame_kernel: one lane of each of two wavefronts per record computes
//     the payload and hash-table checksums (FNV-1a-64, cold_store.rs:909-922),
//     assembles the header, then runs the record checksum and SHA-256
//     (FIPS 180-4) over header | hashes | K | V and writes the footer.  FNV-1a
//     and SHA-256 are sequential chains over the record's bytes, so this
//     launch is bounded by the longest chain (SHA-256 of one record), not by
//     bandwidth; it is meant for sealing or verifying many records at once.
#include "common.hpp"
#include "kernels.hpp"

namespace mslim {

namespace {

constexpr uint64_t kFnvOffset = 0xcbf29ce484222325ull;
constexpr uint64_t kFnvPrime = 0x100000001b3ull;
constexpr int kHeaderWords = kRecordHeaderBytes / 4;   // 26
constexpr int kFooterWords = kRecordFooterBytes / 4;   // 14

__device__ __forceinline__ uint64_t fnv_byte(uint64_t s, uint32_t b) { return (s ^ b) * kFnvPrime; }

// FNV-1a over the four little-endian bytes of a word.
__device__ __forceinline__ uint64_t fnv_word(uint64_t s, uint32_t w) {
    s = fnv_byte(s, w & 0xffu);
    s = fnv_byte(s, (w >> 8) & 0xffu);
    s = fnv_byte(s, (w >> 16) & 0xffu);
    return fnv_byte(s, w >> 24);
}

__device__ __forceinline__ uint64_t fnv_chunk(uint64_t s, const u32x4_t &c) {
    s = fnv_word(s, c[0]);
    s = fnv_word(s, c[1]);
    s = fnv_word(s, c[2]);
    return fnv_word(s, c[3]);
}

__device__ __forceinline__ bool record_valid(const RecordDesc &r, int page_tokens, int64_t pool_pages) {
    return r.tokens >= 1 && (uint64_t)r.first_row + r.tokens <= (uint64_t)page_tokens && r.pool_page >= 0 &&
           (int64_t)r.pool_page < pool_pages;
}

// A record the frame kernels can read: in staged mode its pool page and
// first row are not used.
__device__ __forceinline__ bool record_ok(const FramesCodecLaunch &a, const RecordDesc &r) {
    if (a.staged) return r.tokens >= 1 && r.tokens <= (uint32_t)a.page_tokens;
    return record_valid(r, a.page_tokens, a.pool_pages);
}

// Row 0 of head 0 of record `rec`'s payload and the byte distance between
// heads: inside its pool page, or in its compacted staging slot.
struct PayloadAt {
    const unsigned char *base;
    int64_t head_stride;
};
__device__ __forceinline__ PayloadAt payload_at(const FramesCodecLaunch &a, const void *src, const RecordDesc &r,
                                                int rec, int row_bytes) {
    const int64_t page_bytes = (int64_t)a.kv_heads * a.page_tokens * row_bytes;
    const unsigned char *s = static_cast<const unsigned char *>(src);
    if (a.staged) return {s + (int64_t)rec * page_bytes, (int64_t)r.tokens * row_bytes};
    return {s + (int64_t)r.pool_page * page_bytes + (int64_t)r.first_row * row_bytes,
            (int64_t)a.page_tokens * row_bytes};
}

// Iterates the 16-byte chunks of one token's bytes over all heads (or of a
// whole head-major payload when `rows_per_head` rows are taken per head):
// heads outer, rows, then 16-byte columns.
struct ChunkWalk {
    const unsigned char *head_base;  // row 0 of the current head
    const unsigned char *row;        // current row
    int64_t head_stride;             // bytes between heads in the pool page
    int row_bytes;
    int col;
    int rows_left;                   // rows left in this head after `row`
    int rows_per_head;

    __device__ __forceinline__ const u32x4_t *ptr() const {
        return reinterpret_cast<const u32x4_t *>(row + col);
    }
    __device__ __forceinline__ void advance() {
        col += 16;
        if (col == row_bytes) {
            col = 0;
            if (rows_left > 0) {
                row += row_bytes;
                --rows_left;
            } else {
                head_base += head_stride;
                row = head_base;
                rows_left = rows_per_head - 1;
            }
        }
    }
};

// One lane per (record, part, token).  Chunks are loaded kPrefetch ahead of
// the FNV chain so every lane keeps several 16-byte loads in flight.
constexpr int kPrefetch = 8;

__global__ __launch_bounds__(256) void token_hashes_kernel(FramesCodecLaunch a) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t per_record = 2 * (int64_t)a.page_tokens;
    if (gid >= (int64_t)a.count * per_record) return;
    const int rec = (int)(gid / per_record);
    const int rem = (int)(gid - (int64_t)rec * per_record);
    const int part = rem / a.page_tokens;  // 0 = K, 1 = V
    const int token = rem - part * a.page_tokens;
    const RecordDesc r = a.records[rec];
    if (!record_ok(a, r) || token >= (int)r.tokens) return;

    const int row_bytes = a.head_dim * 2;
    const PayloadAt at = payload_at(a, part ? a.v_pool : a.k_pool, r, rec, row_bytes);
    ChunkWalk w;
    w.head_base = at.base + (int64_t)token * row_bytes;
    w.row = w.head_base;
    w.head_stride = at.head_stride;
    w.row_bytes = row_bytes;
    w.col = 0;
    w.rows_left = 0;
    w.rows_per_head = 1;
    const int chunks = a.kv_heads * (row_bytes / 16);

    u32x4_t buf[kPrefetch];
    ChunkWalk ld = w;
#pragma unroll
    for (int i = 0; i < kPrefetch; ++i) {
        if (i < chunks) {
            buf[i] = *ld.ptr();
            ld.advance();
        }
    }
    uint64_t s = kFnvOffset;
    int c = 0;
    for (; c + kPrefetch <= chunks; c += kPrefetch) {
#pragma unroll
        for (int i = 0; i < kPrefetch; ++i) {
            const u32x4_t cur = buf[i];
            if (c + kPrefetch + i < chunks) {
                buf[i] = *ld.ptr();
                ld.advance();
            }
            s = fnv_chunk(s, cur);
        }
    }
#pragma unroll
    for (int i = 0; i < kPrefetch; ++i)
        if (c + i < chunks) s = fnv_chunk(s, buf[i]);

    unsigned char *frame = static_cast<unsigned char *>(a.frames) + (int64_t)rec * a.frame_bytes;
    uint64_t *table = reinterpret_cast<uint64_t *>(frame + kRecordHeaderBytes);
    table[part * (int)r.tokens + token] = s;
}

// ---- SHA-256 (FIPS 180-4) -------------------------------------------------

__device__ __constant__ uint32_t kSha256K[64] = {
    0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u, 0x923f82a4u, 0xab1c5ed5u,
    0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u, 0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u,
    0xe49b69c1u, 0xefbe4786u, 0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
    0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u, 0x06ca6351u, 0x14292967u,
    0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u, 0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u,
    0xa2bfe8a1u, 0xa81a664bu, 0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
    0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au, 0x5b9cca4fu, 0x682e6ff3u,
    0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u, 0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};

__device__ __forceinline__ uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

// One compression of the 16 big-endian message words w into h.
__device__ __forceinline__ void sha256_compress(uint32_t h[8], uint32_t w[16]) {
    uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], k = h[7];
#pragma unroll
    for (int i = 0; i < 64; ++i) {
        uint32_t wi;
        if (i < 16) {
            wi = w[i];
        } else {
            const uint32_t w15 = w[(i + 1) & 15], w2 = w[(i + 14) & 15];
            const uint32_t s0 = rotr(w15, 7) ^ rotr(w15, 18) ^ (w15 >> 3);
            const uint32_t s1 = rotr(w2, 17) ^ rotr(w2, 19) ^ (w2 >> 10);
            wi = w[i & 15] + s0 + w[(i + 9) & 15] + s1;
            w[i & 15] = wi;
        }
        const uint32_t t1 = k + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + kSha256K[i] + wi;
        const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
        k = g;
        g = f;
        f = e;
        e = d + t1;
        d = c;
        c = b;
        b = a;
        a = t1 + t2;
    }
    h[0] += a; h[1] += b; h[2] += c; h[3] += d;
    h[4] += e; h[5] += f; h[6] += g; h[7] += k;
}

// Streams `n` 16-byte chunks of a walk through `f`, keeping N loads in
// flight ahead of the chain.  `group` runs after every N chunks (and once
// after the tail), outside the unrolled body, so what it inlines appears
// once.
template <int N, class F, class G>
__device__ __forceinline__ void stream_chunks(ChunkWalk ld, int64_t n, F &&f, G &&group) {
    u32x4_t buf[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        if (i < n) {
            buf[i] = *ld.ptr();
            ld.advance();
        }
    }
    int64_t c = 0;
    for (; c + N <= n; c += N) {
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const u32x4_t cur = buf[i];
            if (c + N + i < n) {
                buf[i] = *ld.ptr();
                ld.advance();
            }
            f(cur);
        }
        group();
    }
#pragma unroll
    for (int i = 0; i < N; ++i)
        if (c + i < n) f(buf[i]);
    group();
}

// The same over two walks of equal length, in lockstep.
template <int N, class F>
__device__ __forceinline__ void stream_chunks2(ChunkWalk la, ChunkWalk lb, int64_t n, F &&f) {
    u32x4_t ba[N], bb[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        if (i < n) {
            ba[i] = *la.ptr();
            bb[i] = *lb.ptr();
            la.advance();
            lb.advance();
        }
    }
    int64_t c = 0;
    for (; c + N <= n; c += N) {
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const u32x4_t ca = ba[i], cb = bb[i];
            if (c + N + i < n) {
                ba[i] = *la.ptr();
                bb[i] = *lb.ptr();
                la.advance();
                lb.advance();
            }
            f(ca, cb);
        }
    }
#pragma unroll
    for (int i = 0; i < N; ++i)
        if (c + i < n) f(ba[i], bb[i]);
}

// SHA-256 message state of one lane.  Words enter a 64-word ring in LDS
// (which takes a dynamic index); `drain` compresses every complete block.
constexpr int kFrameThreads = 64;
constexpr int kRingWords = 64;

struct ShaStream {
    uint32_t *ring;  // LDS, kRingWords words at stride kFrameThreads
    uint32_t h[8];
    uint32_t wpos, rpos;

    __device__ __forceinline__ void init(uint32_t *lds) {
        ring = lds;
        h[0] = 0x6a09e667u; h[1] = 0xbb67ae85u; h[2] = 0x3c6ef372u; h[3] = 0xa54ff53au;
        h[4] = 0x510e527fu; h[5] = 0x9b05688cu; h[6] = 0x1f83d9abu; h[7] = 0x5be0cd19u;
        wpos = rpos = 0;
    }
    __device__ __forceinline__ void push_be(uint32_t be) {
        ring[(wpos & (kRingWords - 1)) * kFrameThreads] = be;
        ++wpos;
    }
    __device__ __forceinline__ void drain() {
        while (wpos - rpos >= 16) {
            uint32_t w[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) w[i] = ring[((rpos + i) & (kRingWords - 1)) * kFrameThreads];
            sha256_compress(h, w);
            rpos += 16;
        }
    }
};

__device__ __forceinline__ uint32_t lo32(uint64_t x) { return (uint32_t)x; }
__device__ __forceinline__ uint32_t hi32(uint64_t x) { return (uint32_t)(x >> 32); }

constexpr int kFramePrefetch = 8;

// Two wavefronts per 64 records, each running one chain per lane: in the
// first pass wavefront 0 checksums the K payloads and wavefront 1 the V
// payloads; in the second, over header | tables | K | V, wavefront 0 runs
// SHA-256 and wavefront 1 the record FNV.  A lane's chains are sequential,
// so splitting them over the two wavefronts (on different SIMDs) shortens
// the critical path; they meet through LDS at two barriers.
__global__ __launch_bounds__(2 * kFrameThreads) void frame_kernel(FramesCodecLaunch a) {
    __shared__ uint32_t rings[kRingWords * kFrameThreads];
    __shared__ uint64_t payload_sums[2][kFrameThreads];
    __shared__ uint64_t record_sums[kFrameThreads];
    const int lane = threadIdx.x & (kFrameThreads - 1);
    const int role = threadIdx.x / kFrameThreads;  // wavefront 0 or 1
    const int rec = blockIdx.x * kFrameThreads + lane;
    const bool live = rec < a.count;
    RecordDesc r = {};
    if (live) r = a.records[rec];
    const bool valid = live && record_ok(a, r);
    uint32_t *frame_words = reinterpret_cast<uint32_t *>(static_cast<unsigned char *>(a.frames) +
                                                         (int64_t)(live ? rec : 0) * a.frame_bytes);
    const int frame_words_n = (int)(a.frame_bytes / 4);
    const int tokens = valid ? (int)r.tokens : 0;
    const int row_bytes = a.head_dim * 2;
    const int64_t payload_len = (int64_t)a.kv_heads * tokens * row_bytes;
    const int64_t payload_chunks = payload_len / 16;
    RecordDesc rv = r;
    if (!valid) rv = RecordDesc{0, 0, 0, 1, 0, 0};
    const PayloadAt kat = payload_at(a, a.k_pool, rv, valid ? rec : 0, row_bytes);
    const PayloadAt vat = payload_at(a, a.v_pool, rv, valid ? rec : 0, row_bytes);
    const unsigned char *kpage = kat.base;
    const unsigned char *vpage = vat.base;

    // Head-major payload of `tokens` rows per head.
    auto payload_walk = [&](const unsigned char *page) __attribute__((always_inline)) {
        ChunkWalk w;
        w.head_base = page;
        w.row = page;
        w.head_stride = kat.head_stride;
        w.row_bytes = row_bytes;
        w.col = 0;
        w.rows_left = tokens - 1;
        w.rows_per_head = tokens;
        return w;
    };
    auto no_group = []() __attribute__((always_inline)) {};

    // Pass 1: payload checksums, K on wavefront 0 and V on wavefront 1.
    {
        uint64_t sum = kFnvOffset;
        if (valid)
            stream_chunks<kFramePrefetch>(payload_walk(role == 0 ? kpage : vpage), payload_chunks,
                                          [&](const u32x4_t &c) __attribute__((always_inline)) {
                                              sum = fnv_chunk(sum, c);
                                          },
                                          no_group);
        payload_sums[role][lane] = sum;
    }
    __syncthreads();
    const uint64_t key_sum = payload_sums[0][lane], value_sum = payload_sums[1][lane];

    // Hash-table checksums over the little-endian u64 tables (written by
    // token_hashes_kernel into this frame) and the header
    // (cold_store.rs:291-309), on both wavefronts.
    const uint32_t *tables = frame_words + kHeaderWords;
    uint64_t key_hashes_sum = kFnvOffset, value_hashes_sum = kFnvOffset;
    for (int i = 0; i < 2 * tokens; ++i) key_hashes_sum = fnv_word(key_hashes_sum, tables[i]);
    for (int i = 2 * tokens; i < 4 * tokens; ++i) value_hashes_sum = fnv_word(value_hashes_sum, tables[i]);
    uint32_t hdr[kHeaderWords];
    hdr[0] = 0x564b5354u;  // "TSKV"
    hdr[1] = 0x34304750u;  // "PG04"
    hdr[2] = kRecordVersion;
    hdr[3] = kRecordHeaderBytes;
    hdr[4] = lo32(r.page_id);
    hdr[5] = hi32(r.page_id);
    hdr[6] = r.layer;
    hdr[7] = 0u;
    hdr[8] = lo32(r.token_start);
    hdr[9] = hi32(r.token_start);
    hdr[10] = r.tokens;
    hdr[11] = (uint32_t)a.kv_heads;
    hdr[12] = (uint32_t)a.head_dim;
    hdr[13] = a.tile;
    hdr[14] = lo32((uint64_t)payload_len);
    hdr[15] = hi32((uint64_t)payload_len);
    hdr[16] = lo32((uint64_t)payload_len);
    hdr[17] = hi32((uint64_t)payload_len);
    hdr[18] = lo32(key_sum);
    hdr[19] = hi32(key_sum);
    hdr[20] = lo32(value_sum);
    hdr[21] = hi32(value_sum);
    hdr[22] = lo32(key_hashes_sum);
    hdr[23] = hi32(key_hashes_sum);
    hdr[24] = lo32(value_hashes_sum);
    hdr[25] = hi32(value_hashes_sum);

    // Pass 2 over header | tables | K | V: SHA-256 on wavefront 0, the record
    // FNV on wavefront 1.
    const uint64_t record_len =
        (uint64_t)kRecordHeaderBytes + 16ull * tokens + 2ull * (uint64_t)payload_len + kRecordFooterBytes;
    ShaStream sha;
    sha.init(rings + lane);
    if (role == 0) {
        if (valid) {
#pragma unroll
            for (int i = 0; i < kHeaderWords; ++i) sha.push_be(__builtin_bswap32(hdr[i]));
            sha.drain();
            for (int i = 0; i < 4 * tokens; ++i) {
                sha.push_be(__builtin_bswap32(tables[i]));
                if (sha.wpos - sha.rpos >= 16) sha.drain();
            }
            auto push_chunk = [&](const u32x4_t &c) __attribute__((always_inline)) {
                sha.push_be(__builtin_bswap32(c[0]));
                sha.push_be(__builtin_bswap32(c[1]));
                sha.push_be(__builtin_bswap32(c[2]));
                sha.push_be(__builtin_bswap32(c[3]));
            };
            auto drain = [&]() __attribute__((always_inline)) { sha.drain(); };
            stream_chunks<kFramePrefetch>(payload_walk(kpage), payload_chunks, push_chunk, drain);
            stream_chunks<kFramePrefetch>(payload_walk(vpage), payload_chunks, push_chunk, drain);
            // FIPS 180-4 padding: 0x80, zeros to 56 mod 64, 64-bit big-endian length.
            const uint64_t message_bits = (record_len - kRecordFooterBytes) * 8;
            sha.push_be(0x80000000u);
            while (((sha.wpos - sha.rpos) & 15) != 14) sha.push_be(0u);
            sha.push_be(hi32(message_bits));
            sha.push_be(lo32(message_bits));
            sha.drain();
        }
    } else {
        uint64_t record_sum = kFnvOffset;
        if (valid) {
#pragma unroll
            for (int i = 0; i < kHeaderWords; ++i) record_sum = fnv_word(record_sum, hdr[i]);
            for (int i = 0; i < 4 * tokens; ++i) record_sum = fnv_word(record_sum, tables[i]);
            auto fnv_of = [&](const u32x4_t &c) __attribute__((always_inline)) { record_sum = fnv_chunk(record_sum, c); };
            stream_chunks<kFramePrefetch>(payload_walk(kpage), payload_chunks, fnv_of, no_group);
            stream_chunks<kFramePrefetch>(payload_walk(vpage), payload_chunks, fnv_of, no_group);
        }
        record_sums[lane] = record_sum;
    }
    __syncthreads();
    if (role != 0 || !live) return;
    if (!valid) {
        for (int i = 0; i < frame_words_n; ++i) frame_words[i] = 0u;
        return;
    }
    const uint64_t record_sum = record_sums[lane];
#pragma unroll
    for (int i = 0; i < kHeaderWords; ++i) frame_words[i] = hdr[i];
    for (int i = kHeaderWords + 4 * tokens; i < frame_words_n - kFooterWords; ++i) frame_words[i] = 0u;
    uint32_t *footer = frame_words + frame_words_n - kFooterWords;
    footer[0] = 0x564b5354u;  // "TSKV"
    footer[1] = 0x54494d43u;  // "CMIT"
    footer[2] = lo32(record_sum);
    footer[3] = hi32(record_sum);
    footer[4] = lo32(record_len);
    footer[5] = hi32(record_len);
#pragma unroll
    for (int i = 0; i < 8; ++i) footer[6 + i] = __builtin_bswap32(sha.h[i]);
}

// Payload moves between pool pages and contiguous staging: staging slot i
// (one pool page's bytes) holds record i's head-major payload compacted to
// its `tokens` rows per head.  One lane moves one 16-byte piece of K and of V;
// consecutive lanes take consecutive pieces of a pool page, so the pool side
// is coalesced and the staging side is coalesced within each row run.
template <bool TO_STAGING>
__global__ __launch_bounds__(256) void record_payloads_kernel(PayloadMoveLaunch a) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int cpr = a.head_dim * 2 / 16;  // 16-byte pieces per row
    const int64_t per_page = (int64_t)a.kv_heads * a.page_tokens * cpr;
    if (gid >= (int64_t)a.count * per_page) return;
    const int rec = (int)(gid / per_page);
    const int64_t c = gid - (int64_t)rec * per_page;
    const RecordDesc r = a.records[rec];
    if (!record_valid(r, a.page_tokens, a.pool_pages)) return;
    const int col = (int)(c % cpr);
    const int64_t hr = c / cpr;  // head * page_tokens + row of the pool page
    const int page_row = (int)(hr % a.page_tokens);
    const int head = (int)(hr / a.page_tokens);
    const int row = page_row - (int)r.first_row;  // row of the record
    if (row < 0 || row >= (int)r.tokens) return;
    const int64_t page_bytes = per_page * 16;
    const int64_t pool_off = (int64_t)r.pool_page * page_bytes + c * 16;
    const int64_t stage_off = (int64_t)rec * page_bytes + (((int64_t)head * r.tokens + row) * cpr + col) * 16;
    unsigned char *kp = static_cast<unsigned char *>(a.k_pool), *vp = static_cast<unsigned char *>(a.v_pool);
    unsigned char *ks = static_cast<unsigned char *>(a.k_stage), *vs = static_cast<unsigned char *>(a.v_stage);
    if constexpr (TO_STAGING) {
        *reinterpret_cast<u32x4_t *>(ks + stage_off) = *reinterpret_cast<const u32x4_t *>(kp + pool_off);
        *reinterpret_cast<u32x4_t *>(vs + stage_off) = *reinterpret_cast<const u32x4_t *>(vp + pool_off);
    } else {
        *reinterpret_cast<u32x4_t *>(kp + pool_off) = *reinterpret_cast<const u32x4_t *>(ks + stage_off);
        *reinterpret_cast<u32x4_t *>(vp + pool_off) = *reinterpret_cast<const u32x4_t *>(vs + stage_off);
    }
}

}  // namespace

int64_t record_frame_bytes(int page_tokens) {
    return (int64_t)kRecordHeaderBytes + 16ll * page_tokens + kRecordFooterBytes;
}

hipError_t launch_record_frames(const FramesCodecLaunch &a, hipStream_t stream) {
    if (a.count == 0) return hipSuccess;
    const int64_t lanes = (int64_t)a.count * 2 * a.page_tokens;
    hipLaunchKernelGGL(token_hashes_kernel, dim3((unsigned)((lanes + 255) / 256)), dim3(256), 0, stream, a);
    if (hipError_t e = hipGetLastError()) return e;
    hipLaunchKernelGGL(frame_kernel, dim3((unsigned)((a.count + kFrameThreads - 1) / kFrameThreads)),
                       dim3(2 * kFrameThreads), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_record_payloads(const PayloadMoveLaunch &a, bool to_staging, hipStream_t stream) {
    if (a.count == 0) return hipSuccess;
    const int64_t lanes = (int64_t)a.count * a.kv_heads * a.page_tokens * (a.head_dim * 2 / 16);
    const dim3 grid((unsigned)((lanes + 255) / 256));
    if (to_staging)
        hipLaunchKernelGGL(record_payloads_kernel<true>, grid, dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(record_payloads_kernel<false>, grid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace mslim
