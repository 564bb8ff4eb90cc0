// TiledAttention (gpu_llm/tiled_attention.rs:23-293) on libmslim_attn: the
// configured attention for `queries` new rows after `prior` cached tokens.
// build() applies the reference's configuration and resource checks against
// MI355X limits; run() applies its launch checks and dispatches the gfx950
// decode (queries == 1) or causal prefill kernel.  Buffers are device
// pointers: Q [queries][q_heads][D], K/V token-major [prior+queries][kv_heads]
// [D], output like Q, all BF16.
#pragma once

#include <atomic>
#include <cstddef>
#include <memory>
#include <string>

#include "attention_kernel.hpp"
#include "native.hpp"
#include "portable.hpp"

namespace mslim {

class TiledAttention {
public:
    static constexpr size_t kMaxQueries = 512;                   // tiled_attention.rs:172-175
    static constexpr size_t kLdsBytesPerWorkgroup = 160 * 1024;  // gfx950 LDS per CU

    static std::unique_ptr<TiledAttention> build(std::shared_ptr<NativeContext> ctx,
                                                 AttentionKernelConfig config,
                                                 portable::AttentionGeometry geometry);
    void run(const void *q, const void *k, const void *v, void *output, size_t queries, size_t prior,
             portable::AttentionGeometry geometry);
    // JSON diagnostics (tiled_attention.rs:142-158).
    std::string diagnostics() const;
    const AttentionKernelConfig &config() const { return config_; }

private:
    TiledAttention(std::shared_ptr<NativeContext> ctx, AttentionKernelConfig c, portable::AttentionGeometry g,
                   size_t local_bytes, size_t scratch)
        : ctx_(std::move(ctx)), config_(c), geometry_(g), local_bytes_(local_bytes), scratch_bytes_(scratch) {}
    std::shared_ptr<NativeContext> ctx_;
    AttentionKernelConfig config_;
    portable::AttentionGeometry geometry_;
    size_t local_bytes_;
    size_t scratch_bytes_;
    std::atomic<uint64_t> calls_{0}, split_calls_{0};
};

}  // namespace mslim
