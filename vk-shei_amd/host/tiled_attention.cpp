#include "tiled_attention.hpp"

#include <cmath>
#include <cstdint>
#include <mutex>

namespace mslim {

std::unique_ptr<TiledAttention> TiledAttention::build(std::shared_ptr<NativeContext> ctx,
                                                      AttentionKernelConfig config,
                                                      portable::AttentionGeometry geometry) {
    config.validate();
    geometry = portable::AttentionGeometry::create(geometry.query_heads, geometry.kv_heads, geometry.head_dim);
    ensure(config.mode != AttentionKernelMode::Reference, "reference does not compile tiled kernels");
    const size_t estimate = config.local_bytes(geometry.head_dim);
    ensure(config.work_group <= 1024, "attention workgroup exceeds device limit");
    ensure(estimate <= kLdsBytesPerWorkgroup, "attention tile exceeds device local-memory limit");
    const size_t scratch = config.decode_scratch_bytes(geometry.query_heads, geometry.head_dim);
    return std::unique_ptr<TiledAttention>(
        new TiledAttention(std::move(ctx), config, geometry, estimate, scratch));
}

void TiledAttention::run(const void *q, const void *k, const void *v, void *output, size_t queries,
                         size_t prior, portable::AttentionGeometry geometry) {
    ensure(queries > 0 && queries <= kMaxQueries, "attention query count must be 1..=512");
    ensure(geometry == geometry_, "kernel specialization does not match geometry");
    size_t history = 0;
    ensure(!__builtin_add_overflow(prior, queries, &history), "attention history overflow");
    ensure(history <= (size_t)UINT32_MAX - 64, "attention history exceeds indexing bound");
    // The gfx950 kernels index tokens with 32-bit signed integers.
    ensure(history <= (size_t)INT32_MAX - 64, "attention history exceeds indexing bound");
    ensure(output != q && output != k && output != v, "tiled attention output must not alias read-only Q/K/V");
    const float scale = (float)(1.0 / std::sqrt((double)geometry.head_dim));
    const int qh = (int)geometry.query_heads, kvh = (int)geometry.kv_heads, d = (int)geometry.head_dim;
    std::lock_guard<std::mutex> lock(ctx_->mutex());
    if (queries == 1) {
        const int32_t len = (int32_t)history;
        const int split = config_.decode_split_tokens(history);
        ctx_->check("dispatch tiled attention",
                    mslim_attn_decode_dense(ctx_->handle(), q, k, v, output, 1, &len, (int64_t)history, qh, kvh,
                                            d, scale, split));
        if (split > 0 && (size_t)split < history) split_calls_.fetch_add(1, std::memory_order_relaxed);
    } else {
        ctx_->check("dispatch tiled attention",
                    mslim_attn_prefill_causal(ctx_->handle(), q, k, v, output, (int)queries, (int)prior, qh, kvh,
                                              d, scale));
    }
    calls_.fetch_add(1, std::memory_order_relaxed);
}

std::string TiledAttention::diagnostics() const {
    return std::string("{\"settings\":") + config_.to_json() +
           ",\"numeric_contract\":\"online_f32_accumulation_within_2e-2\"" +
           ",\"local_bytes_estimate\":" + std::to_string(local_bytes_) +
           ",\"global_score_matrix_bytes\":0" + ",\"split_scratch_bytes\":" + std::to_string(scratch_bytes_) +
           ",\"dispatches_since_configuration\":" + std::to_string(calls_.load()) +
           ",\"split_dispatches_since_configuration\":" + std::to_string(split_calls_.load()) +
           ",\"split_policy\":\"split only single-query decode; multi-query prefill uses online blocks\"}";
}

}  // namespace mslim
