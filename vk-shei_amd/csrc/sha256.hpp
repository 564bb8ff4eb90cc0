// FIPS 180-4 SHA-256 for the ColdStore record digests and the logical K/V
// digest (the role the sha2 crate plays at cold_store.rs:275-349 and
// gpu_region_store.rs:350-370).  The block compression lives in
// sha256_host.cpp (host code only): the x86 SHA extensions when the CPU has
// them, a portable FIPS 180-4 loop otherwise.
#pragma once

#include <stddef.h>
#include <stdint.h>
#include <string.h>

namespace mslim {

// Compress `blocks` 64-byte blocks into `state` (FIPS 180-4 section 6.2.2).
void sha256_compress(uint32_t state[8], const uint8_t *data, size_t blocks);
// The portable loop alone, for tests that compare the two paths.
void sha256_compress_portable(uint32_t state[8], const uint8_t *data, size_t blocks);
// True when sha256_compress uses the x86 SHA extensions.
bool sha256_uses_cpu_extensions();

class Sha256 {
public:
    Sha256() {
        static const uint32_t iv[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                                       0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
        memcpy(state_, iv, sizeof iv);
    }

    void update(const void *data, size_t n) {
        const uint8_t *p = static_cast<const uint8_t *>(data);
        total_ += n;
        if (fill_) {
            const size_t take = n < 64 - fill_ ? n : 64 - fill_;
            memcpy(block_ + fill_, p, take);
            fill_ += take; p += take; n -= take;
            if (fill_ < 64) return;
            sha256_compress(state_, block_, 1);
            fill_ = 0;
        }
        if (n >= 64) {
            sha256_compress(state_, p, n / 64);
            p += n & ~(size_t)63;
            n &= 63;
        }
        memcpy(block_, p, n);
        fill_ = n;
    }

    void finish(uint8_t out[32]) {
        const uint64_t bits = total_ * 8;
        uint8_t pad[72] = {0x80};
        const size_t zeros = (fill_ < 56 ? 56 - fill_ : 120 - fill_);
        for (int i = 0; i < 8; ++i) pad[zeros + i] = (uint8_t)(bits >> (56 - 8 * i));
        update(pad, zeros + 8);
        for (int i = 0; i < 8; ++i)
            for (int j = 0; j < 4; ++j) out[4 * i + j] = (uint8_t)(state_[i] >> (24 - 8 * j));
    }

private:
    uint32_t state_[8];
    uint8_t block_[64];
    size_t fill_ = 0;
    uint64_t total_ = 0;
};

}  // namespace mslim
