// Decoder runner over the C ABI: see model.hpp for the layer order.
#include "model.hpp"

#include <chrono>
#include <climits>
#include <cmath>
#include <cerrno>
#include <cstring>

#include "../../include/mslim_model.h"

#include <sys/stat.h>
#include <unistd.h>

namespace mslim {
namespace model {

void ModelSpec::validate() const {
    ensure(layers > 0 && hidden > 0 && intermediate > 0 && vocab > 0, "model dimensions must be positive");
    ensure(q_heads > 0 && kv_heads > 0 && q_heads % kv_heads == 0, "query heads must be a multiple of kv heads");
    ensure(head_dim >= 8 && head_dim <= 256 && head_dim % 8 == 0, "head_dim must be a multiple of 8 up to 256");
    ensure(hidden % 8 == 0, "hidden size must be a multiple of 8");
    ensure(hidden <= 32768 && intermediate <= 32768 && (int64_t)q_heads * head_dim <= 32768,
           "projection inner dimension above 32768");
    ensure(rms_eps > 0.0f && std::isfinite(rms_eps), "rms_norm_eps must be positive");
    ensure(rope_theta > 0.0f && std::isfinite(rope_theta), "rope_theta must be positive");
    if (llama3)
        ensure(rope_factor > 0.0f && rope_low > 0.0f && rope_high > rope_low && rope_original_max > 0.0f,
               "invalid llama3 RoPE scaling");
}

DecoderRunner::DecoderRunner(std::shared_ptr<NativeContext> ctx, ModelSpec spec, ModelWeights weights,
                             int max_batch, int chunk_tokens, int max_context, KvLayout layout)
    : ctx_(std::move(ctx)), spec_(spec), w_(std::move(weights)), layout_(layout), max_batch_(max_batch),
      chunk_tokens_(chunk_tokens), max_context_(max_context) {
    ensure(ctx_ != nullptr, "no device context");
    spec_.validate();
    ensure((int)w_.layers.size() == spec_.layers, "layer weight count does not match the model");
    ensure(w_.embed && w_.final_norm && w_.lm_head, "embedding, final norm and LM head weights are required");
    for (const auto &l : w_.layers)
        ensure(l.input_norm && l.q && l.k && l.v && l.o && l.post_norm && l.gate && l.up && l.down,
               "every layer needs all nine weight tensors");
    ensure(max_batch_ >= 1 && max_batch_ <= kMaxSlots, "max_batch must be 1..=64");
    ensure(chunk_tokens_ >= 1 && chunk_tokens_ <= 512, "prefill chunk must be 1..=512 tokens");
    ensure(max_context_ >= 1 && max_context_ <= (1 << 24), "max_context must be 1..=16777216 tokens");
    ensure(layout_ == KvLayout::Paged || layout_ == KvLayout::Dense, "unknown K/V layout");
    // The dense layout is a pool of one-token pages (token-major rows) under
    // the identity table: slot s, token t -> row s * max_context + t.
    page_tokens_ = layout_ == KvLayout::Dense ? 1 : kPageTokens;
    pages_per_seq_ = (max_context_ + page_tokens_ - 1) / page_tokens_;
    rows_cap_ = std::max(max_batch_, chunk_tokens_);
    // set_batch_prefill_tokens (mod.rs:742-760): a batch of 8 or more reads
    // each weight once for 8 tokens or more.
    settings_.batch_tokens = (size_t)chunk_tokens_;
    settings_.weight_reuse_tokens = chunk_tokens_ >= 8 ? 8 : 1;
    scale_ = (float)(1.0 / std::sqrt((double)spec_.head_dim));
    positions_.assign(max_batch_, 0);
    poisoned_.assign(max_batch_, 0);

    const size_t kvd = (size_t)spec_.kv_heads * spec_.head_dim, qd = (size_t)spec_.q_heads * spec_.head_dim;
    const size_t pool_pages = (size_t)max_batch_ * pages_per_seq_;
    try {
        // One allocation for every layer's K pages and one for V: layer l's
        // pool is pages [l * pool_pages, (l + 1) * pool_pages), so the
        // ColdStore seal and restore of a slot cover all layers per launch.
        const size_t layer_bytes = pool_pages * page_tokens_ * kvd * 2;
        k_base_ = alloc(layer_bytes * spec_.layers);
        v_base_ = alloc(layer_bytes * spec_.layers);
        for (int l = 0; l < spec_.layers; ++l) {
            k_pools_.push_back(static_cast<char *>(k_base_) + layer_bytes * l);
            v_pools_.push_back(static_cast<char *>(v_base_) + layer_bytes * l);
        }
        // Paged: slot s, logical page p -> physical page p * max_batch + s, so
        // the slots interleave in the pool and every read goes through the
        // table.  Dense: the identity.
        std::vector<int32_t> table(pool_pages);
        for (int s = 0; s < max_batch_; ++s)
            for (int p = 0; p < pages_per_seq_; ++p)
                table[(size_t)s * pages_per_seq_ + p] =
                    (int32_t)(layout_ == KvLayout::Dense ? (size_t)s * pages_per_seq_ + p : (size_t)p * max_batch_ + s);
        host_table_ = table;
        table_ = static_cast<int32_t *>(alloc(table.size() * 4));
        ctx_->check("upload page table", mslim_attn_buf_write(ctx_->handle(), table_, 0,
                                                              reinterpret_cast<const uint8_t *>(table.data()),
                                                              table.size() * 4));
        const size_t r = rows_cap_;
        ids_ = static_cast<int32_t *>(alloc(r * 4));
        pos_ = static_cast<int32_t *>(alloc(r * 4));
        next_ = static_cast<int32_t *>(alloc(r * 4));
        x_ = static_cast<uint16_t *>(alloc(r * spec_.hidden * 2));
        q_ = static_cast<uint16_t *>(alloc(r * qd * 2));
        qr_ = static_cast<uint16_t *>(alloc(r * qd * 2));
        attn_ = static_cast<uint16_t *>(alloc(r * qd * 2));
        k_ = static_cast<uint16_t *>(alloc(r * kvd * 2));
        kr_ = static_cast<uint16_t *>(alloc(r * kvd * 2));
        v_ = static_cast<uint16_t *>(alloc(r * kvd * 2));
        act_ = static_cast<uint16_t *>(alloc(r * spec_.intermediate * 2));
        if (layout_ == KvLayout::Paged) {
            kd_ = static_cast<uint16_t *>(alloc((size_t)max_context_ * kvd * 2));
            vd_ = static_cast<uint16_t *>(alloc((size_t)max_context_ * kvd * 2));
        }
        logits_ = static_cast<uint16_t *>(alloc((size_t)max_batch_ * spec_.vocab * 2));
        cold_.resize(max_batch_);
        cold_report_.assign(max_batch_, ColdReport{});
    } catch (...) {
        for (void *p : owned_) mslim_attn_buf_free(ctx_->handle(), p);
        throw;
    }
}

DecoderRunner::~DecoderRunner() {
    cold_.clear();
    staging_.reset();
    for (void *p : owned_) mslim_attn_buf_free(ctx_->handle(), p);
}

void *DecoderRunner::alloc(size_t bytes) {
    void *p = mslim_attn_buf_alloc(ctx_->handle(), bytes ? bytes : 1);
    if (!p) throw NativeError("allocate runner buffer", 0, mslim_attn_last_error());
    owned_.push_back(p);
    return p;
}

// Final norm, LM head and greedy token of `rows` hidden rows.
void DecoderRunner::head(const uint16_t *rows_in, int rows) {
    void *h = ctx_->handle();
    ctx_->check("final norm + LM head", mslim_attn_rmsnorm_gemm_bf16(h, w_.final_norm, spec_.rms_eps, w_.lm_head,
                                                                     rows_in, logits_, spec_.hidden, spec_.vocab,
                                                                     rows));
    ctx_->check("argmax", mslim_attn_argmax(h, logits_, rows, spec_.vocab, next_));
    logits_rows_ = rows;
}

// One causal chunk of slot `seq`: tokens ids[0..n) at positions prior..prior+n
// (run_batch_layer, prefill.rs:897-1061, for every layer).
void DecoderRunner::chunk(int seq, const int32_t *ids, int n, int64_t prior) {
    void *h = ctx_->handle();
    const ModelSpec &s = spec_;
    const int qd = s.q_heads * s.head_dim, kvd = s.kv_heads * s.head_dim;
    ctx_->check("upload token ids", mslim_attn_buf_write(h, ids_, 0, reinterpret_cast<const uint8_t *>(ids),
                                                         (size_t)n * 4));
    ctx_->check("embed", mslim_attn_embed(h, w_.embed, s.vocab, s.hidden, ids_, n, x_, nullptr));
    for (int l = 0; l < s.layers; ++l) {
        const LayerWeights &w = w_.layers[l];
        check_cancel("GPU batch prefill cancelled at layer boundary", l);
        injected_error(l);
        ctx_->check("input norm + QKV projection",
                    mslim_attn_rmsnorm_gemm_qkv(h, w.input_norm, s.rms_eps, w.q, w.k, w.v, x_, q_, k_, v_, s.hidden,
                                                qd, kvd, n));
        ctx_->check("RoPE", mslim_attn_rope_qk(h, q_, qr_, k_, kr_, n, s.q_heads, s.kv_heads, s.head_dim, (int)prior,
                                               s.rope_theta, s.llama3, s.rope_factor, s.rope_low, s.rope_high,
                                               s.rope_original_max));
        ctx_->check("page write", mslim_attn_pages_write(h, k_pools_[l], v_pools_[l], table_row(seq), page_tokens_,
                                                         s.kv_heads, s.head_dim, prior, n, kr_, v_));
        const void *keys = kr_, *values = v_;
        if (layout_ == KvLayout::Dense) {
            keys = dense_rows(k_pools_[l], seq);
            values = dense_rows(v_pools_[l], seq);
        } else if (prior > 0) {
            // Earlier chunks live only in the pages: gather the slot's whole
            // history token-major for the causal kernel.
            ctx_->check("gather keys", mslim_attn_pages_gather(h, k_pools_[l], table_row(seq), kPageTokens,
                                                               s.kv_heads, s.head_dim, 0, prior + n, kd_));
            ctx_->check("gather values", mslim_attn_pages_gather(h, v_pools_[l], table_row(seq), kPageTokens,
                                                                 s.kv_heads, s.head_dim, 0, prior + n, vd_));
            keys = kd_;
            values = vd_;
        }
        ctx_->check("causal attention", mslim_attn_prefill_causal(h, qr_, keys, values, attn_, n, (int)prior,
                                                                  s.q_heads, s.kv_heads, s.head_dim, scale_));
        mlp(w, n);
    }
}

// O projection + residual, post norm, gate/up + SwiGLU, down + residual over
// `n` rows of x_ (attention output in attn_).
void DecoderRunner::mlp(const LayerWeights &w, int n) {
    void *h = ctx_->handle();
    const ModelSpec &s = spec_;
    const int qd = s.q_heads * s.head_dim;
    ctx_->check("O projection + residual", mslim_attn_gemm_bf16_add(h, w.o, attn_, x_, x_, qd, s.hidden, n));
    ctx_->check("post norm + gate/up + SwiGLU",
                mslim_attn_rmsnorm_gemm_swiglu(h, w.post_norm, s.rms_eps, w.gate, w.up, x_, act_, s.hidden,
                                               s.intermediate, n));
    ctx_->check("down projection + residual",
                mslim_attn_gemm_bf16_add(h, w.down, act_, x_, x_, s.intermediate, s.hidden, n));
}

Step DecoderRunner::prefill_only(int seq, const std::vector<int32_t> &prompt) {
    ensure(seq >= 0 && seq < max_batch_, "sequence slot out of range");
    ensure(!prompt.empty(), "GPU prompt IDs empty");
    ensure(prompt.size() < (size_t)max_context_, "GPU context capacity not large enough for prompt");
    for (int32_t id : prompt) ensure(id >= 0 && id < spec_.vocab, "token id outside the vocabulary");
    check_healthy(seq);
    if (cold_[seq])
        ensure(cold_report_[seq].committed_tokens == 0,
               "GPU prefill into a slot whose ColdStore already holds a session; restore it or attach an empty "
               "directory");
    int32_t next = 0;
    const int n_total = (int)prompt.size();
    // From here on a failure (or a cancellation) leaves the slot's K/V
    // written for some chunks or layers only: the slot is poisoned
    // (prefill_batched's error path, gpu_llm/mod.rs:2545-2550).
    try {
        {
            std::lock_guard<std::mutex> lock(ctx_->mutex());
            positions_[seq] = 0;
            for (int start = 0; start < n_total; start += chunk_tokens_) {
                check_cancel("GPU batch prefill cancelled", -1);
                const int n = std::min(chunk_tokens_, n_total - start);
                chunk(seq, prompt.data() + start, n, start);
                if (start + n == n_total) head(x_ + (size_t)(n - 1) * spec_.hidden, 1);
            }
            positions_[seq] = n_total;
            ctx_->check("read greedy token", mslim_attn_buf_read(ctx_->handle(), next_, 0,
                                                                 reinterpret_cast<uint8_t *>(&next), 4));
        }
        if (cold_[seq]) {
            // The prompt's K/V are committed to the canonical ColdStore at the
            // end of prefill (gpu_llm/prefill.rs:760-790).
            const auto t0 = std::chrono::steady_clock::now();
            seal_slot(seq, 0, n_total);
            cold_report_[seq].prefill_seal_seconds =
                std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        }
    } catch (...) {
        poisoned_[seq] = 1;
        throw;
    }
    return Step{next, n_total};
}

std::vector<Step> DecoderRunner::forward_batch(const std::vector<int32_t> &tokens) {
    const int b = (int)tokens.size();
    ensure(b >= 1 && b <= max_batch_, "decode batch must be 1..=max_batch slots");
    for (int32_t id : tokens) ensure(id >= 0 && id < spec_.vocab, "token id outside the vocabulary");
    std::vector<int32_t> pos(b), lens(b);
    for (int i = 0; i < b; ++i) {
        check_healthy(i);
        ensure(positions_[i] < max_context_, "GPU KV capacity exceeded: configure larger --max-context-tokens");
        pos[i] = (int32_t)positions_[i];
        lens[i] = pos[i] + 1;
    }
    // A token boundary: nothing of this step has run, so a cancellation here
    // leaves every slot consistent.
    check_cancel("GPU generation cancelled by client", -1);
    // The context lock covers the step's device work only: an immediate
    // commit below takes it again.  A failure inside poisons every slot of
    // the batch (forward_token_internal, gpu_llm/mod.rs:2476-2482).
    std::vector<int32_t> next(b);
    try {
        std::lock_guard<std::mutex> lock(ctx_->mutex());
        void *h = ctx_->handle();
        const ModelSpec &s = spec_;
        ctx_->check("upload token ids",
                    mslim_attn_buf_write(h, ids_, 0, reinterpret_cast<const uint8_t *>(tokens.data()), (size_t)b * 4));
        ctx_->check("upload positions", mslim_attn_buf_write(h, pos_, 0, reinterpret_cast<const uint8_t *>(pos.data()),
                                                             (size_t)b * 4));
        ctx_->check("embed", mslim_attn_embed(h, w_.embed, s.vocab, s.hidden, ids_, b, x_, nullptr));
        for (int l = 0; l < s.layers; ++l) {
            const LayerWeights &w = w_.layers[l];
            injected_error(l);
            ctx_->check("input norm + QKV + RoPE + K/V append",
                        mslim_attn_rmsnorm_qkv_rope_append(h, w.input_norm, s.rms_eps, w.q, w.k, w.v, x_, qr_,
                                                           k_pools_[l], v_pools_[l], table_, pages_per_seq_,
                                                           page_tokens_, b, pos_, s.hidden, s.q_heads, s.kv_heads,
                                                           s.head_dim, s.rope_theta, s.llama3, s.rope_factor,
                                                           s.rope_low, s.rope_high, s.rope_original_max));
            if (layout_ == KvLayout::Dense)
                ctx_->check("dense attention",
                            mslim_attn_decode_dense(h, qr_, k_pools_[l], v_pools_[l], attn_, b, lens.data(), max_context_,
                                                    s.q_heads, s.kv_heads, s.head_dim, scale_, 0));
            else
                ctx_->check("paged attention",
                            mslim_attn_decode_paged(h, qr_, k_pools_[l], v_pools_[l], attn_, b, lens.data(), table_,
                                                    pages_per_seq_, kPageTokens, s.q_heads, s.kv_heads, s.head_dim,
                                                    scale_, 0));
            mlp(w, b);
        }
        head(x_, b);
        ctx_->check("read greedy tokens", mslim_attn_buf_read(h, next_, 0, reinterpret_cast<uint8_t *>(next.data()),
                                                              (size_t)b * 4));
    } catch (...) {
        for (int i = 0; i < b; ++i) poisoned_[i] = 1;
        throw;
    }
    std::vector<Step> steps(b);
    for (int i = 0; i < b; ++i) {
        positions_[i] += 1;
        steps[i] = Step{next[i], positions_[i]};
    }
    // Immediate mode (gpu_llm/mod.rs:2162-2164): each step's K/V is committed
    // before the step returns; a failed commit poisons its slot.
    if (!deferred_cold_)
        for (int i = 0; i < b; ++i)
            if (cold_[i]) {
                try {
                    flush_cold(i);
                } catch (...) {
                    poisoned_[i] = 1;
                    throw;
                }
            }
    return steps;
}

void DecoderRunner::set_deferred_cold_commit(bool deferred) {
    if (!deferred)
        for (int i = 0; i < max_batch_; ++i)
            if (cold_[i] && !poisoned_[i] && cold_report_[i].committed_tokens < positions_[i]) flush_cold(i);
    deferred_cold_ = deferred;
}

std::vector<int32_t> DecoderRunner::generate(int seq, const std::vector<int32_t> &prompt, int max_new,
                                             const std::vector<int32_t> &eos_ids) {
    ensure(max_new > 0, "max_new_tokens must be positive");
    ensure(prompt.size() + (size_t)max_new <= (size_t)max_context_,
           "GPU context capacity not large enough for prompt + generation");
    ensure(seq == 0, "generate drives slot 0; use forward_batch for several slots");
    Step current = prefill_only(seq, prompt);
    std::vector<int32_t> generated;
    for (int step = 0; step < max_new; ++step) {
        if (cancel_ && __atomic_load_n(cancel_, __ATOMIC_RELAXED)) {
            // A cancelled turn's decoded prefix is sealed before the error
            // (generate_cancellable, gpu_llm/mod.rs:2704-2712); a failed seal
            // poisons the slot.
            if (cold_[seq] && deferred_cold_ && cold_report_[seq].committed_tokens < positions_[seq]) {
                try {
                    flush_cold(seq);
                } catch (...) {
                    poisoned_[seq] = 1;
                    throw;
                }
            }
            throw Error("GPU generation cancelled by client");
        }
        const int32_t token = current.argmax_token;
        bool eos = false;
        for (int32_t e : eos_ids) eos = eos || e == token;
        if (eos) break;
        generated.push_back(token);
        if (step + 1 < max_new) current = forward_batch({token})[0];
    }
    return generated;
}

void DecoderRunner::set_calibration_prefill_settings(const PrefillSettings &settings) {
    settings.validate();
    for (int i = 0; i < max_batch_; ++i)
        ensure(positions_[i] == 0 && !poisoned_[i], "prefill tuning requires a healthy, empty session");
    ensure(settings.chunk_tokens() <= rows_cap_, "prefill batch exceeds the chunk this runner was built for");
    chunk_tokens_ = settings.chunk_tokens();
    settings_ = settings;
}

void DecoderRunner::reset(int seq) {
    ensure(seq >= 0 && seq < max_batch_, "sequence slot out of range");
    // A poisoned slot's deferred K/V are not committed: its device state is
    // not trusted.  The reset discards it and clears the poison.
    const bool was_poisoned = poisoned_[seq] != 0;
    poisoned_[seq] = 0;
    if (cold_[seq]) {
        // reset_session (gpu_llm/mod.rs:1530-1577): commit what is deferred,
        // then continue in a fresh ColdStore namespace
        // <parent>/session-<pid>-<nonce> beside the current directory, so
        // the finished session stays on disk for a later restore.
        if (!was_poisoned && cold_report_[seq].committed_tokens < positions_[seq]) flush_cold(seq);
        std::string current = *cold_[seq]->config().cold_directory;
        while (current.size() > 1 && current.back() == '/') current.pop_back();
        const size_t cut = current.find_last_of('/');
        const std::string root = cut == std::string::npos ? std::string(".") : cut == 0 ? std::string("/")
                                                                                         : current.substr(0, cut);
        const long long nonce = (long long)std::chrono::duration_cast<std::chrono::nanoseconds>(
                                    std::chrono::system_clock::now().time_since_epoch()).count();
        const std::string next = root + (root == "/" ? "" : "/") + "session-" + std::to_string((long long)getpid()) +
                                 "-" + std::to_string(nonce);
        ensure(mkdir(next.c_str(), 0777) == 0 || errno == EEXIST,
               "create canonical ColdStore namespace " + next + ": " + std::strerror(errno));
        cold_[seq].reset();
        positions_[seq] = 0;
        attach_cold_store(seq, next);
        return;
    }
    positions_[seq] = 0;
}

std::string DecoderRunner::cold_directory(int seq) const {
    ensure(seq >= 0 && seq < max_batch_, "sequence slot out of range");
    return cold_[seq] ? *cold_[seq]->config().cold_directory : std::string();
}

region::DevicePagePool DecoderRunner::all_layer_pool() const {
    region::DevicePagePool pool;
    pool.k_pool = k_base_;
    pool.v_pool = v_base_;
    pool.pool_pages = (int64_t)max_batch_ * pages_per_seq_ * spec_.layers;
    pool.page_tokens = kPageTokens;
    return pool;
}

std::vector<region::LayerBlocks> DecoderRunner::slot_blocks(int seq) const {
    const int64_t per_layer = (int64_t)max_batch_ * pages_per_seq_;
    std::vector<region::LayerBlocks> out(spec_.layers);
    for (int l = 0; l < spec_.layers; ++l) {
        out[l].layer = (size_t)l;
        out[l].blocks.resize(pages_per_seq_);
        for (int p = 0; p < pages_per_seq_; ++p)
            out[l].blocks[p] = (int32_t)(l * per_layer + host_table_[(size_t)seq * pages_per_seq_ + p]);
    }
    return out;
}

// Commit tokens [from, to) of every layer of slot `seq` from the pool.
void DecoderRunner::seal_slot(int seq, int64_t from, int64_t to) {
    if (to <= from) return;
    if (!staging_) staging_ = std::make_unique<region::DeviceStaging>(*ctx_);
    cold_[seq]->seal_device_layers(*staging_, (size_t)from, (size_t)(to - from), all_layer_pool(), slot_blocks(seq));
    cold_report_[seq].committed_tokens = to;
}

void DecoderRunner::attach_cold_store(int seq, const std::string &directory) {
    ensure(seq >= 0 && seq < max_batch_, "sequence slot out of range");
    ensure(layout_ == KvLayout::Paged, "the ColdStore-exact route needs the paged K/V layout");
    check_healthy(seq);
    ensure(positions_[seq] == 0, "attach a ColdStore to an empty slot");
    region::RegionConfig config;
    config.cold_directory = directory;
    const auto g = portable::AttentionGeometry::create((size_t)spec_.q_heads, (size_t)spec_.kv_heads,
                                                       (size_t)spec_.head_dim);
    auto store = std::make_unique<region::RegionStore>(g, (size_t)spec_.layers, config);
    const size_t held = store->layer_tokens(0);
    for (int l = 1; l < spec_.layers; ++l)
        ensure(store->layer_tokens(l) == held, "persisted ColdStore layers do not share a complete causal prefix");
    cold_[seq] = std::move(store);
    cold_report_[seq] = ColdReport{};
    cold_report_[seq].attached = true;
    cold_report_[seq].committed_tokens = (int64_t)held;
}

void DecoderRunner::detach_cold_store(int seq) {
    ensure(seq >= 0 && seq < max_batch_, "sequence slot out of range");
    cold_[seq].reset();
    cold_report_[seq] = ColdReport{};
}

void DecoderRunner::flush_cold(int seq) {
    ensure(seq >= 0 && seq < max_batch_, "sequence slot out of range");
    ensure(cold_[seq] != nullptr, "deferred commit requires canonical ColdStore");
    check_healthy(seq);
    const auto t0 = std::chrono::steady_clock::now();
    const int64_t from = cold_report_[seq].committed_tokens, to = positions_[seq];
    ensure(from <= to, "GPU ColdStore prefill prefix missing/longer than in-flight KV");
    seal_slot(seq, from, to);
    cold_report_[seq].last_commit_seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    cold_report_[seq].last_committed_token_layers = (to - from) * spec_.layers;
}

void DecoderRunner::restore_session(int seq, int64_t tokens) {
    ensure(seq >= 0 && seq < max_batch_, "sequence slot out of range");
    ensure(cold_[seq] != nullptr, "canonical GPU restore requires persistent LOD/ColdStore");
    check_healthy(seq);
    ensure(positions_[seq] == 0, "canonical GPU restore requires a fresh session");
    ensure(tokens > 0, "canonical GPU restore prefix is empty");
    ensure(tokens < max_context_, "canonical GPU restore must leave capacity for continuation");
    for (int l = 0; l < spec_.layers; ++l)
        ensure((int64_t)cold_[seq]->layer_tokens(l) == tokens,
               "canonical GPU restore layer " + std::to_string(l) + " is not a complete causal prefix");
    const auto t0 = std::chrono::steady_clock::now();
    if (!staging_) staging_ = std::make_unique<region::DeviceStaging>(*ctx_);
    // Every record is verified on the device before any byte reaches the
    // pool; on failure the slot stays empty.
    cold_[seq]->restore_device_layers(*staging_, all_layer_pool(), slot_blocks(seq));
    positions_[seq] = tokens;
    cold_report_[seq].committed_tokens = tokens;
    cold_report_[seq].last_restore_seconds =
        std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
}

std::string DecoderRunner::cold_logical_kv_sha256(int seq) {
    ensure(seq >= 0 && seq < max_batch_, "sequence slot out of range");
    ensure(cold_[seq] != nullptr, "no ColdStore attached to this slot");
    return cold_[seq]->logical_kv_sha256();
}

ColdReport DecoderRunner::cold_report(int seq) const {
    ensure(seq >= 0 && seq < max_batch_, "sequence slot out of range");
    return cold_report_[seq];
}

std::vector<uint16_t> DecoderRunner::last_logits() const {
    std::vector<uint16_t> out((size_t)logits_rows_ * spec_.vocab);
    if (!out.empty())
        ctx_->check("read logits", mslim_attn_buf_read(ctx_->handle(), logits_, 0,
                                                       reinterpret_cast<uint8_t *>(out.data()), out.size() * 2));
    return out;
}

bool DecoderRunner::poisoned(int seq) const {
    ensure(seq >= 0 && seq < max_batch_, "sequence slot out of range");
    return poisoned_[seq] != 0;
}

void DecoderRunner::check_healthy(int seq) const {
    ensure(!poisoned_[seq], "GPU slot " + std::to_string(seq) +
                                " was poisoned by an earlier failed forward pass; reset the slot");
}

void DecoderRunner::inject_failure(int kind, int layer) {
    ensure(kind == 0 || kind == kInjectArgumentError || kind == kInjectCancel, "unknown failure injection");
    ensure(layer >= 0 && layer < spec_.layers, "injected failure layer out of range");
    inject_kind_ = kind;
    inject_layer_ = layer;
}

void DecoderRunner::check_cancel(const char *where, int layer) {
    bool raised = cancel_ && __atomic_load_n(cancel_, __ATOMIC_RELAXED) != 0;
    if (inject_kind_ == kInjectCancel && layer == inject_layer_) {
        inject_kind_ = 0;
        raised = true;
    }
    ensure(!raised, where);
}

void DecoderRunner::injected_error(int layer) {
    if (inject_kind_ != kInjectArgumentError || layer != inject_layer_) return;
    inject_kind_ = 0;
    // A launch with an invalid shape: the library rejects it before any work.
    const LayerWeights &w = w_.layers[layer];
    ctx_->check("input norm + QKV projection",
                mslim_attn_rmsnorm_gemm_qkv(ctx_->handle(), w.input_norm, spec_.rms_eps, w.q, w.k, w.v, x_, q_, k_,
                                            v_, spec_.hidden, spec_.q_heads * spec_.head_dim,
                                            spec_.kv_heads * spec_.head_dim, -1));
}

std::string DecoderRunner::logical_kv_sha256(int seq) const {
    ensure(seq >= 0 && seq < max_batch_, "sequence slot out of range");
    check_healthy(seq);
    std::vector<const int32_t *> tables(spec_.layers, table_row(seq));
    std::vector<const void *> keys(k_pools_.begin(), k_pools_.end()), values(v_pools_.begin(), v_pools_.end());
    const bool dense = layout_ == KvLayout::Dense;
    if (dense)
        for (int l = 0; l < spec_.layers; ++l) {
            keys[l] = dense_rows(k_pools_[l], seq);
            values[l] = dense_rows(v_pools_[l], seq);
        }
    char hex[65] = {0};
    ctx_->check("logical K/V digest",
                mslim_attn_logical_kv_sha256(ctx_->handle(), spec_.layers, positions_[seq], spec_.kv_heads,
                                             spec_.head_dim, keys.data(), values.data(),
                                             dense ? nullptr : tables.data(), dense ? 0 : kPageTokens, hex));
    return std::string(hex);
}

}  // namespace model
}  // namespace mslim

// ---- C API ------------------------------------------------------------------

namespace {

thread_local std::string g_model_error;

int model_fail(const std::exception &e) {
    g_model_error = e.what();
    return -1;
}

struct ModelHandle {
    std::unique_ptr<mslim::model::DecoderRunner> runner;
};

mslim::model::DecoderRunner &runner_of(void *m) {
    mslim::ensure(m != nullptr, "null model handle");
    return *static_cast<ModelHandle *>(m)->runner;
}

}  // namespace

extern "C" {

const char *mslim_model_last_error(void) { return g_model_error.c_str(); }

void *mslim_model_new(void *attn_ctx, const mslim_model_spec *spec, const void *const *weights, int max_batch,
                      int chunk_tokens, int max_context, int kv_layout) {
    g_model_error.clear();
    try {
        mslim::ensure(attn_ctx && spec && weights, "null model arguments");
        mslim::ensure(kv_layout == MSLIM_MODEL_KV_PAGED || kv_layout == MSLIM_MODEL_KV_DENSE, "unknown K/V layout");
        mslim::model::ModelSpec s;
        s.layers = spec->layers;
        s.hidden = spec->hidden;
        s.q_heads = spec->q_heads;
        s.kv_heads = spec->kv_heads;
        s.head_dim = spec->head_dim;
        s.intermediate = spec->intermediate;
        s.vocab = spec->vocab;
        s.rms_eps = spec->rms_eps;
        s.rope_theta = spec->rope_theta;
        s.llama3 = spec->llama3_scaling;
        s.rope_factor = spec->rope_factor;
        s.rope_low = spec->rope_low_freq_factor;
        s.rope_high = spec->rope_high_freq_factor;
        s.rope_original_max = spec->rope_original_max_position;
        mslim::ensure(s.layers > 0 && s.layers <= 4096, "layer count must be 1..=4096");
        mslim::model::ModelWeights w;
        w.embed = weights[0];
        w.final_norm = weights[1];
        w.lm_head = weights[2];
        for (int l = 0; l < s.layers; ++l) {
            const void *const *p = weights + 3 + (size_t)l * MSLIM_MODEL_LAYER_TENSORS;
            mslim::model::LayerWeights lw;
            lw.input_norm = p[0];
            lw.q = p[1];
            lw.k = p[2];
            lw.v = p[3];
            lw.o = p[4];
            lw.post_norm = p[5];
            lw.gate = p[6];
            lw.up = p[7];
            lw.down = p[8];
            w.layers.push_back(lw);
        }
        auto handle = std::make_unique<ModelHandle>();
        handle->runner = std::make_unique<mslim::model::DecoderRunner>(
            mslim::NativeContext::borrow(attn_ctx), s, std::move(w), max_batch, chunk_tokens, max_context,
            static_cast<mslim::model::KvLayout>(kv_layout));
        return handle.release();
    } catch (const std::exception &e) {
        model_fail(e);
        return nullptr;
    }
}

void mslim_model_destroy(void *model) { delete static_cast<ModelHandle *>(model); }

int mslim_model_prefill(void *model, int seq, const int32_t *prompt, int tokens, int32_t *next_token) {
    g_model_error.clear();
    try {
        mslim::ensure(next_token && tokens >= 0 && (prompt || !tokens), "invalid prefill arguments");
        const std::vector<int32_t> ids = tokens ? std::vector<int32_t>(prompt, prompt + tokens) : std::vector<int32_t>();
        *next_token = runner_of(model).prefill_only(seq, ids).argmax_token;
        return 0;
    } catch (const std::exception &e) {
        return model_fail(e);
    }
}

int mslim_model_forward_batch(void *model, const int32_t *tokens, int batch, int32_t *next_tokens) {
    g_model_error.clear();
    try {
        mslim::ensure(tokens && batch > 0 && next_tokens, "invalid forward arguments");
        const auto steps = runner_of(model).forward_batch(std::vector<int32_t>(tokens, tokens + batch));
        for (int i = 0; i < batch; ++i) next_tokens[i] = steps[i].argmax_token;
        return 0;
    } catch (const std::exception &e) {
        return model_fail(e);
    }
}

int mslim_model_generate(void *model, const int32_t *prompt, int tokens, int max_new, const int32_t *eos_ids,
                         int eos_count, int32_t *out, int *generated) {
    g_model_error.clear();
    try {
        mslim::ensure(prompt && tokens > 0 && out && generated && eos_count >= 0 && (eos_ids || !eos_count),
                      "invalid generate arguments");
        const auto got = runner_of(model).generate(0, std::vector<int32_t>(prompt, prompt + tokens), max_new,
                                                   std::vector<int32_t>(eos_ids, eos_ids + eos_count));
        std::memcpy(out, got.data(), got.size() * 4);
        *generated = (int)got.size();
        return 0;
    } catch (const std::exception &e) {
        return model_fail(e);
    }
}

int64_t mslim_model_position(void *model, int seq) {
    g_model_error.clear();
    try {
        return runner_of(model).position(seq);
    } catch (const std::exception &e) {
        model_fail(e);
        return -1;
    }
}

int mslim_model_reset(void *model, int seq) {
    g_model_error.clear();
    try {
        runner_of(model).reset(seq);
        return 0;
    } catch (const std::exception &e) {
        return model_fail(e);
    }
}

int mslim_model_logits(void *model, uint16_t *out, size_t capacity, int *rows) {
    g_model_error.clear();
    try {
        mslim::ensure(out && rows, "invalid logits arguments");
        auto &r = runner_of(model);
        const auto l = r.last_logits();
        mslim::ensure(l.size() <= capacity, "logits buffer too small");
        std::memcpy(out, l.data(), l.size() * 2);
        *rows = (int)(l.size() / r.spec().vocab);
        return 0;
    } catch (const std::exception &e) {
        return model_fail(e);
    }
}

int mslim_model_prefill_settings(void *model, char *json_out, size_t capacity) {
    g_model_error.clear();
    try {
        mslim::ensure(json_out != nullptr, "null settings buffer");
        const std::string text = runner_of(model).prefill_settings().to_json();
        mslim::ensure(text.size() < capacity, "settings buffer too small");
        std::memcpy(json_out, text.c_str(), text.size() + 1);
        return 0;
    } catch (const std::exception &e) {
        return model_fail(e);
    }
}

int mslim_model_set_prefill_settings(void *model, const char *json) {
    g_model_error.clear();
    try {
        mslim::ensure(json != nullptr, "null settings");
        runner_of(model).set_calibration_prefill_settings(mslim::PrefillSettings::from_json(json));
        return 0;
    } catch (const std::exception &e) {
        return model_fail(e);
    }
}

int mslim_model_attach_cold_store(void *model, int seq, const char *directory) {
    g_model_error.clear();
    try {
        mslim::ensure(directory != nullptr, "null ColdStore directory");
        runner_of(model).attach_cold_store(seq, directory);
        return 0;
    } catch (const std::exception &e) {
        return model_fail(e);
    }
}

int mslim_model_detach_cold_store(void *model, int seq) {
    g_model_error.clear();
    try {
        runner_of(model).detach_cold_store(seq);
        return 0;
    } catch (const std::exception &e) {
        return model_fail(e);
    }
}

int mslim_model_flush_cold(void *model, int seq) {
    g_model_error.clear();
    try {
        runner_of(model).flush_cold(seq);
        return 0;
    } catch (const std::exception &e) {
        return model_fail(e);
    }
}

int mslim_model_restore_session(void *model, int seq, int64_t tokens) {
    g_model_error.clear();
    try {
        runner_of(model).restore_session(seq, tokens);
        return 0;
    } catch (const std::exception &e) {
        return model_fail(e);
    }
}

int mslim_model_cold_logical_kv_sha256(void *model, int seq, char *hex_out) {
    g_model_error.clear();
    try {
        mslim::ensure(hex_out != nullptr, "null digest buffer");
        const std::string hex = runner_of(model).cold_logical_kv_sha256(seq);
        std::memcpy(hex_out, hex.c_str(), hex.size() + 1);
        return 0;
    } catch (const std::exception &e) {
        return model_fail(e);
    }
}

int mslim_model_set_deferred_cold_commit(void *model, int deferred) {
    g_model_error.clear();
    try {
        runner_of(model).set_deferred_cold_commit(deferred != 0);
        return 0;
    } catch (const std::exception &e) {
        return model_fail(e);
    }
}

int mslim_model_cold_directory(void *model, int seq, char *out, size_t capacity) {
    g_model_error.clear();
    try {
        mslim::ensure(out != nullptr, "null output");
        const std::string dir = runner_of(model).cold_directory(seq);
        mslim::ensure(dir.size() < capacity, "ColdStore directory does not fit in the output buffer");
        std::memcpy(out, dir.c_str(), dir.size() + 1);
        return 0;
    } catch (const std::exception &e) {
        return model_fail(e);
    }
}

int mslim_model_cold_report(void *model, int seq, mslim_model_cold_info *out) {
    g_model_error.clear();
    try {
        mslim::ensure(out != nullptr, "null report");
        const mslim::model::ColdReport r = runner_of(model).cold_report(seq);
        out->attached = r.attached ? 1 : 0;
        out->committed_tokens = r.committed_tokens;
        out->prefill_seal_seconds = r.prefill_seal_seconds;
        out->last_commit_seconds = r.last_commit_seconds;
        out->last_committed_token_layers = r.last_committed_token_layers;
        out->last_restore_seconds = r.last_restore_seconds;
        return 0;
    } catch (const std::exception &e) {
        return model_fail(e);
    }
}

int mslim_model_logical_kv_sha256(void *model, int seq, char *hex_out) {
    g_model_error.clear();
    try {
        mslim::ensure(hex_out != nullptr, "null digest buffer");
        const std::string hex = runner_of(model).logical_kv_sha256(seq);
        std::memcpy(hex_out, hex.c_str(), hex.size() + 1);
        return 0;
    } catch (const std::exception &e) {
        return model_fail(e);
    }
}

/* ---- failure handling ---------------------------------------------------- */

int mslim_model_set_cancel_flag(void *model, const int32_t *flag) {
    g_model_error.clear();
    try {
        runner_of(model).set_cancel_flag(flag);
        return 0;
    } catch (const std::exception &e) {
        return model_fail(e);
    }
}

int mslim_model_poisoned(void *model, int seq) {
    g_model_error.clear();
    try {
        return runner_of(model).poisoned(seq) ? 1 : 0;
    } catch (const std::exception &e) {
        return model_fail(e);
    }
}

int mslim_model_inject_failure(void *model, int kind, int layer) {
    g_model_error.clear();
    try {
        runner_of(model).inject_failure(kind, layer);
        return 0;
    } catch (const std::exception &e) {
        return model_fail(e);
    }
}

}  // extern "C"
