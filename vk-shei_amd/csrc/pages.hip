// ColdStore-exact page pool: token-major rows <-> head-major pages, and the
// canonical head-major serialisation behind the logical K/V SHA-256.
//
// A page of the device pool is the ColdStore page payload itself,
// [kv_heads][page_tokens][head_dim] BF16 (cold_store.rs:480-483,
// gpu_region_store.rs:459-472), so a verified payload can be copied into a
// pool slot unchanged.  These are byte moves in 16-byte units: every lane
// moves one contiguous 8-element piece of a row, and consecutive lanes move
// consecutive pieces, so both sides are coalesced.
#include "common.hpp"
#include "kernels.hpp"

namespace mslim {

namespace {


__global__ __launch_bounds__(256) void pages_write_kernel(uint16_t *k_pool, uint16_t *v_pool,
                                                          const int32_t *table, int shift,
                                                          int kv_heads, int head_dim,
                                                          int64_t first, int64_t tokens,
                                                          const uint16_t *k_rows,
                                                          const uint16_t *v_rows) {
    const int chunks = head_dim / 8;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= tokens * kv_heads * chunks) return;
    const int dc = (int)(i % chunks);
    const int64_t th = i / chunks;  // token * kv_heads + head
    const int head = (int)(th % kv_heads);
    const int64_t t = th / kv_heads;
    const int64_t dst = page_row(table, shift, kv_heads, head, first + t) * head_dim + dc * 8;
    const int64_t src = th * head_dim + dc * 8;
    *reinterpret_cast<uint4 *>(k_pool + dst) = *reinterpret_cast<const uint4 *>(k_rows + src);
    *reinterpret_cast<uint4 *>(v_pool + dst) = *reinterpret_cast<const uint4 *>(v_rows + src);
}

// Decode-step append: work item (b, head, 8-element chunk) of row b.
__global__ __launch_bounds__(256) void pages_append_kernel(uint16_t *k_pool, uint16_t *v_pool,
                                                           const int32_t *table, int pages_per_seq,
                                                           int shift, int kv_heads, int head_dim,
                                                           int batch, const int32_t *positions,
                                                           const uint16_t *k_rows,
                                                           const uint16_t *v_rows) {
    const int chunks = head_dim / 8;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)batch * kv_heads * chunks) return;
    const int dc = (int)(i % chunks);
    const int64_t bh = i / chunks;  // b * kv_heads + head
    const int head = (int)(bh % kv_heads);
    const int b = (int)(bh / kv_heads);
    const int64_t position = positions[b];
    if (position < 0 || position >= ((int64_t)pages_per_seq << shift)) return;
    const int64_t dst =
        page_row(table + (int64_t)b * pages_per_seq, shift, kv_heads, head, position) * head_dim + dc * 8;
    const int64_t src = bh * head_dim + dc * 8;
    *reinterpret_cast<uint4 *>(k_pool + dst) = *reinterpret_cast<const uint4 *>(k_rows + src);
    *reinterpret_cast<uint4 *>(v_pool + dst) = *reinterpret_cast<const uint4 *>(v_rows + src);
}

__global__ __launch_bounds__(256) void pages_gather_kernel(const uint16_t *pool, const int32_t *table,
                                                           int shift, int kv_heads, int head_dim,
                                                           int64_t first, int64_t tokens,
                                                           uint16_t *out) {
    const int chunks = head_dim / 8;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= tokens * kv_heads * chunks) return;
    const int dc = (int)(i % chunks);
    const int64_t th = i / chunks;
    const int head = (int)(th % kv_heads);
    const int64_t t = th / kv_heads;
    const int64_t src = page_row(table, shift, kv_heads, head, first + t) * head_dim + dc * 8;
    *reinterpret_cast<uint4 *>(out + th * head_dim + dc * 8) =
        *reinterpret_cast<const uint4 *>(pool + src);
}

__global__ __launch_bounds__(256) void canonical_rows_kernel(const uint16_t *src, const int32_t *table,
                                                             int shift, int kv_heads, int head_dim,
                                                             int head, int64_t first, int64_t count,
                                                             uint16_t *out) {
    const int chunks = head_dim / 8;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count * chunks) return;
    const int dc = (int)(i % chunks);
    const int64_t t = first + i / chunks;
    const int64_t row = table ? page_row(table, shift, kv_heads, head, t) : t * kv_heads + head;
    *reinterpret_cast<uint4 *>(out + i * 8) =
        *reinterpret_cast<const uint4 *>(src + row * head_dim + dc * 8);
}

int log2_exact(int v) {
    int s = 0;
    while ((1 << s) < v) ++s;
    return s;
}

}  // namespace

hipError_t launch_pages_write(uint16_t *k_pool, uint16_t *v_pool, const int32_t *page_table,
                              int page_tokens, int kv_heads, int head_dim, int64_t first_token,
                              int64_t tokens, const uint16_t *k_rows, const uint16_t *v_rows,
                              hipStream_t stream) {
    const int64_t work = tokens * kv_heads * (head_dim / 8);
    hipLaunchKernelGGL(pages_write_kernel, dim3((unsigned)((work + 255) / 256)), dim3(256), 0, stream,
                       k_pool, v_pool, page_table, log2_exact(page_tokens), kv_heads, head_dim,
                       first_token, tokens, k_rows, v_rows);
    return hipGetLastError();
}

hipError_t launch_pages_append(uint16_t *k_pool, uint16_t *v_pool, const int32_t *page_table,
                               int pages_per_seq, int page_tokens, int kv_heads, int head_dim,
                               int batch, const int32_t *positions, const uint16_t *k_rows,
                               const uint16_t *v_rows, hipStream_t stream) {
    const int64_t work = (int64_t)batch * kv_heads * (head_dim / 8);
    hipLaunchKernelGGL(pages_append_kernel, dim3((unsigned)((work + 255) / 256)), dim3(256), 0, stream,
                       k_pool, v_pool, page_table, pages_per_seq, log2_exact(page_tokens), kv_heads,
                       head_dim, batch, positions, k_rows, v_rows);
    return hipGetLastError();
}

hipError_t launch_pages_gather(const uint16_t *pool, const int32_t *page_table, int page_tokens,
                               int kv_heads, int head_dim, int64_t first_token, int64_t tokens,
                               uint16_t *rows_out, hipStream_t stream) {
    const int64_t work = tokens * kv_heads * (head_dim / 8);
    hipLaunchKernelGGL(pages_gather_kernel, dim3((unsigned)((work + 255) / 256)), dim3(256), 0, stream,
                       pool, page_table, log2_exact(page_tokens), kv_heads, head_dim, first_token,
                       tokens, rows_out);
    return hipGetLastError();
}

hipError_t launch_canonical_rows(const uint16_t *src, const int32_t *page_table, int page_tokens,
                                 int kv_heads, int head_dim, int head, int64_t first,
                                 int64_t count, uint16_t *out, hipStream_t stream) {
    const int64_t work = count * (head_dim / 8);
    hipLaunchKernelGGL(canonical_rows_kernel, dim3((unsigned)((work + 255) / 256)), dim3(256), 0,
                       stream, src, page_table, page_table ? log2_exact(page_tokens) : 0, kv_heads,
                       head_dim, head, first, count, out);
    return hipGetLastError();
}

}  // namespace mslim
