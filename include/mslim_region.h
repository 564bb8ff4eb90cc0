/* Exact region store over a canonical ColdStore (exported by libmslim_host).
 *
 * The public API of the reference's GpuRegionStore (src/gpu_region_store.rs:
 * 118-928) in exact mode (epsilon = 0): per-layer token -> (ColdStore page,
 * offset) catalogue, token-major <-> head-major page conversion, non-finite
 * rejection on append, partial K/V reads and the logical K/V SHA-256.  The
 * reference's native CPU runtime keeps its K/V here (native_cpu_adapter.rs:
 * 337, :458-484) and the GPU-region runtime commits its pages here.  Files
 * are the reference's pages-exact.kv byte for byte.
 *
 * Every entry point returns 0 on success and -1 with mslim_region_last_error()
 * set on failure; a handle is used from one thread at a time. */
#ifndef MSLIM_REGION_H
#define MSLIM_REGION_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

const char *mslim_region_last_error(void);

/* GpuRegionStore::new (gpu_region_store.rs:137-207): opens <directory>/
 * pages-exact.kv with its committed records (each verified) or creates it;
 * a NULL directory gives a private temporary store removed on destroy.
 * stage_tokens 1..1024 (GpuRegionConfig::stage_tokens).  NULL on failure. */
void *mslim_region_new(int q_heads, int kv_heads, int head_dim, int layers, const char *directory,
                       int stage_tokens);
void mslim_region_destroy(void *store);

/* Tokens held by `layer` (GpuRegionStore::layer_tokens), or -1. */
int64_t mslim_region_layer_tokens(void *store, int layer);

/* GpuRegionStore::append_batch (gpu_region_store.rs:391-520): `tokens`
 * token-major BF16 rows [tokens][kv_heads][head_dim] of K and of V at
 * `position` (= layer_tokens(layer)), committed as ColdStore records of up to
 * page_tokens (1..512) tokens each.  page_tokens 1 is GpuRegionStore::append
 * (:376-384), the single-token decode writer.  V must be finite on every
 * layer, K on layer 0, checked before any record is committed. */
int mslim_region_append(void *store, int layer, int64_t position, const void *keys, const void *values,
                        int tokens, int page_tokens);

/* GpuRegionStore::read_keys / read_values (gpu_region_store.rs:828-927):
 * token-major BF16 rows of the given positions into `out` (count * kv_heads *
 * head_dim * 2 bytes); part 0 reads K, 1 reads V.  Every page read is
 * verified against its stored per-token hashes. */
int mslim_region_read(void *store, int layer, int part, const int64_t *positions, int count, void *out);

/* GpuRegionStore::logical_kv_sha256 (gpu_region_store.rs:341-371) as 64 hex
 * digits and a NUL: the digest GpuLlm::logical_kv_sha256 gives for the same
 * K/V, so a store and a device cache can be compared. */
int mslim_region_logical_kv_sha256(void *store, char *hex_out);

#ifdef __cplusplus
}
#endif

#endif /* MSLIM_REGION_H */
