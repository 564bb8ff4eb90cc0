// SHA-256 block compression for the host (FIPS 180-4 section 6.2.2).
//
// Two paths with the same result: the x86 SHA extensions (SHA256RNDS2 does
// two rounds on the state held as the ABEF / CDGH register pair,
// SHA256MSG1/MSG2 extend the message schedule four words at a time), chosen
// at run time when CPUID reports them, and a portable loop that keeps the
// eight working variables in locals.  ColdStore verification hashes every
// record of a store on open, so the digest rate bounds how fast a session
// restores.
#include "sha256.hpp"

#include <cpuid.h>
#include <immintrin.h>

namespace mslim {
namespace {

alignas(16) const uint32_t kRound[64] = {
    0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u, 0x923f82a4u, 0xab1c5ed5u,
    0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u, 0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u,
    0xe49b69c1u, 0xefbe4786u, 0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
    0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u, 0x06ca6351u, 0x14292967u,
    0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u, 0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u,
    0xa2bfe8a1u, 0xa81a664bu, 0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
    0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au, 0x5b9cca4fu, 0x682e6ff3u,
    0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u, 0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};

inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

void compress_portable(uint32_t state[8], const uint8_t *p, size_t blocks) {
    for (; blocks; --blocks, p += 64) {
        uint32_t w[64];
        for (int i = 0; i < 16; ++i)
            w[i] = (uint32_t)p[4 * i] << 24 | (uint32_t)p[4 * i + 1] << 16 | (uint32_t)p[4 * i + 2] << 8 |
                   (uint32_t)p[4 * i + 3];
        for (int i = 16; i < 64; ++i) {
            const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
            const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
            w[i] = w[i - 16] + s0 + w[i - 7] + s1;
        }
        uint32_t a = state[0], b = state[1], c = state[2], d = state[3];
        uint32_t e = state[4], f = state[5], g = state[6], h = state[7];
        for (int i = 0; i < 64; ++i) {
            const uint32_t t1 = h + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + kRound[i] + w[i];
            const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
            h = g; g = f; f = e; e = d + t1;
            d = c; c = b; b = a; a = t1 + t2;
        }
        state[0] += a; state[1] += b; state[2] += c; state[3] += d;
        state[4] += e; state[5] += f; state[6] += g; state[7] += h;
    }
}

// The state lives in two registers: ABEF = (F, E, B, A) and CDGH = (H, G, D,
// C) from the low lane up, the operand layout of SHA256RNDS2.  Each group of
// four rounds adds the round constants to four schedule words; RNDS2 takes
// the low two, the high two after a lane swap.
__attribute__((target("sha,sse4.1,ssse3"))) void compress_shani(uint32_t state[8], const uint8_t *p,
                                                                 size_t blocks) {
    const __m128i byteswap = _mm_set_epi64x(0x0c0d0e0f08090a0bll, 0x0405060700010203ll);
    __m128i dcba = _mm_loadu_si128(reinterpret_cast<const __m128i *>(state));      // A B C D
    __m128i hgfe = _mm_loadu_si128(reinterpret_cast<const __m128i *>(state + 4));  // E F G H
    const __m128i cdab = _mm_shuffle_epi32(dcba, 0xB1);                               // B A D C
    const __m128i efgh = _mm_shuffle_epi32(hgfe, 0x1B);                               // H G F E
    __m128i abef = _mm_alignr_epi8(cdab, efgh, 8);                                    // F E B A
    __m128i cdgh = _mm_blend_epi16(efgh, cdab, 0xF0);                                 // H G D C
    for (; blocks; --blocks, p += 64) {
        const __m128i abef0 = abef, cdgh0 = cdgh;
        __m128i w[4];
#pragma GCC unroll 16
        for (int q = 0; q < 16; ++q) {
            if (q < 4) {
                w[q] = _mm_shuffle_epi8(_mm_loadu_si128(reinterpret_cast<const __m128i *>(p + 16 * q)), byteswap);
            } else {
                // words 4q..4q+3: W[t-16] + s0(W[t-15]) + W[t-7] + s1(W[t-2])
                __m128i t = _mm_sha256msg1_epu32(w[(q - 4) & 3], w[(q - 3) & 3]);
                t = _mm_add_epi32(t, _mm_alignr_epi8(w[(q - 1) & 3], w[(q - 2) & 3], 4));
                w[q & 3] = _mm_sha256msg2_epu32(t, w[(q - 1) & 3]);
            }
            __m128i wk = _mm_add_epi32(w[q & 3], _mm_load_si128(reinterpret_cast<const __m128i *>(kRound + 4 * q)));
            cdgh = _mm_sha256rnds2_epu32(cdgh, abef, wk);  // rounds 4q, 4q+1: new ABEF
            wk = _mm_shuffle_epi32(wk, 0x0E);
            abef = _mm_sha256rnds2_epu32(abef, cdgh, wk);  // rounds 4q+2, 4q+3: roles back in place
        }
        abef = _mm_add_epi32(abef, abef0);
        cdgh = _mm_add_epi32(cdgh, cdgh0);
    }
    const __m128i feba = _mm_shuffle_epi32(abef, 0x1B);   // A B E F
    const __m128i dchg = _mm_shuffle_epi32(cdgh, 0xB1);   // G H C D
    dcba = _mm_blend_epi16(feba, dchg, 0xF0);              // A B C D
    hgfe = _mm_alignr_epi8(dchg, feba, 8);                 // E F G H
    _mm_storeu_si128(reinterpret_cast<__m128i *>(state), dcba);
    _mm_storeu_si128(reinterpret_cast<__m128i *>(state + 4), hgfe);
}

bool cpu_has_sha() {
    unsigned a = 0, b = 0, c = 0, d = 0;
    if (!__get_cpuid_count(7, 0, &a, &b, &c, &d)) return false;
    const bool sha = (b >> 29) & 1u;
    if (!__get_cpuid(1, &a, &b, &c, &d)) return false;
    const bool sse41 = (c >> 19) & 1u, ssse3 = (c >> 9) & 1u;
    return sha && sse41 && ssse3;
}

const bool g_sha = cpu_has_sha();

}  // namespace

void sha256_compress(uint32_t state[8], const uint8_t *data, size_t blocks) {
    if (g_sha)
        compress_shani(state, data, blocks);
    else
        compress_portable(state, data, blocks);
}

void sha256_compress_portable(uint32_t state[8], const uint8_t *data, size_t blocks) {
    compress_portable(state, data, blocks);
}

bool sha256_uses_cpu_extensions() { return g_sha; }

}  // namespace mslim
