/*
 * CPU oracle for the M-SLIM attention hot path -- TEST INFRASTRUCTURE ONLY.
 * See oracle.h for the contract and the pinning status of each function.
 * Build with -ffp-contract=off: the reference's CPU path never fuses a
 * multiply and an add, and the reference GPU path's fused steps are written
 * here explicitly with fmaf().
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- BF16 codec --------------------------------------------------------- */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float orc_read_bf16(uint16_t bits) { return u2f(((uint32_t)bits) << 16); }

uint16_t orc_write_bf16(float value) {
    uint32_t bits = f2u(value);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((bits >> 16) | 0x0040u);
    bits += 0x7fffu + ((bits >> 16) & 1u);
    return (uint16_t)(bits >> 16);
}

uint16_t orc_half_bf16_from_f32(float value) {
    const uint32_t x = f2u(value);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x0040u);
    const uint32_t round_bit = 0x8000u;
    if ((x & round_bit) != 0 && (x & (3u * round_bit - 1u)) != 0)
        return (uint16_t)((x >> 16) + 1u);
    return (uint16_t)(x >> 16);
}

uint16_t orc_bf16_round_independent(float value) {
    const uint32_t x = f2u(value);
    if (isnan(value)) return (uint16_t)((x >> 16) | 0x0040u);
    if (isinf(value) || value == 0.0f) return (uint16_t)(x >> 16);
    /* ulp of an 8-bit significand at this binade; bf16 subnormals share
     * f32's minimum exponent, so the ulp floor is 2^-133. */
    int e;
    frexp((double)value, &e); /* value = m * 2^e, 0.5 <= |m| < 1 */
    int ulp_exp = e - 8;
    if (ulp_exp < -133) ulp_exp = -133;
    const double scaled = ldexp((double)value, -ulp_exp); /* exact */
    const double rounded = ldexp(nearbyint(scaled), ulp_exp);
    if (fabs(rounded) >= ldexp(1.0, 128))
        return (uint16_t)(value < 0 ? 0xff80u : 0x7f80u);
    return (uint16_t)(f2u((float)rounded) >> 16);
}

uint64_t orc_bf16_encoder_mismatches(uint64_t start, uint64_t count) {
    uint64_t bad = 0;
    for (uint64_t i = 0; i < count; ++i) {
        const float f = u2f((uint32_t)(start + i));
        const uint16_t a = orc_write_bf16(f);
        if (a != orc_half_bf16_from_f32(f) || a != orc_bf16_round_independent(f)) ++bad;
    }
    return bad;
}

void orc_bf16_to_f32_array(const uint16_t *in, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_read_bf16(in[i]);
}
void orc_f32_to_bf16_array(const float *in, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_write_bf16(in[i]);
}

/* native_cpu_adapter.rs:179-181 round_bf16 = half from_f32 then to_f32. */
static inline float round_bf16(float v) { return orc_read_bf16(orc_half_bf16_from_f32(v)); }

/* Once-rounded transcendentals (see file header). */
static inline float exp_f(float x) { return (float)exp((double)x); }
static inline float log_f(float x) { return (float)log((double)x); }
static inline float cos_f(float x) { return (float)cos((double)x); }
static inline float sin_f(float x) { return (float)sin((double)x); }
static inline float pow_f(float x, float y) { return (float)pow((double)x, (double)y); }

/* ---- Attention oracles -------------------------------------------------- */
void orc_softmax(float *values, int n) {
    /* native_cpu_adapter.rs:223-233; f32::max ignores a NaN operand. */
    float max = -INFINITY;
    for (int i = 0; i < n; ++i) max = fmaxf(max, values[i]);
    float sum = 0.0f;
    for (int i = 0; i < n; ++i) {
        values[i] = exp_f(values[i] - max);
        sum += values[i];
    }
    for (int i = 0; i < n; ++i) values[i] /= sum;
}

int orc_dense_attention_bf16(int query_heads, int kv_heads, int head_dim,
                             const float *query, const uint16_t *keys,
                             const uint16_t *values, int tokens, float *out) {
    if (query_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || tokens < 0 ||
        query_heads % kv_heads) return -1;
    const int group = query_heads / kv_heads;
    const float scale = 1.0f / sqrtf((float)head_dim); /* :235-237 */
    float *scores = (float *)malloc(sizeof(float) * (size_t)(tokens > 0 ? tokens : 1));
    if (!scores) return -1;
    for (int qh = 0; qh < query_heads; ++qh) {
        const int kh = qh / group;
        const float *q = query + (size_t)qh * head_dim;
        for (int t = 0; t < tokens; ++t) {
            const uint16_t *k = keys + ((size_t)t * kv_heads + kh) * head_dim;
            float dot = -0.0f; /* f32 `Sum` starts from -0.0 */
            for (int d = 0; d < head_dim; ++d) dot += q[d] * orc_read_bf16(k[d]);
            scores[t] = dot * scale;
        }
        orc_softmax(scores, tokens);
        float *o = out + (size_t)qh * head_dim;
        for (int d = 0; d < head_dim; ++d) o[d] = 0.0f;
        for (int t = 0; t < tokens; ++t) {
            const uint16_t *v = values + ((size_t)t * kv_heads + kh) * head_dim;
            for (int d = 0; d < head_dim; ++d) o[d] += scores[t] * orc_read_bf16(v[d]);
        }
        for (int d = 0; d < head_dim; ++d) o[d] = round_bf16(o[d]);
    }
    free(scores);
    return 0;
}

static float f16_to_f32(uint16_t raw) {
    const uint32_t sign = (uint32_t)(raw & 0x8000u) << 16;
    const uint32_t e = (raw >> 10) & 31u, frac = raw & 1023u;
    if (e == 0) {
        if (frac == 0) return u2f(sign);
        return (raw & 0x8000u ? -1.0f : 1.0f) * ldexpf((float)frac, -24);
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (frac << 13));
    return u2f(sign | ((e - 15u + 127u) << 23) | (frac << 13));
}

static float element(const void *data, size_t i, int dtype) {
    if (dtype == 1) return orc_read_bf16(((const uint16_t *)data)[i]);
    if (dtype == 2) return f16_to_f32(((const uint16_t *)data)[i]);
    return ((const float *)data)[i];
}

int orc_cpu_reference_decode(int query_heads, int kv_heads, int head_dim,
                             const float *query, const void *keys,
                             const void *values, int dtype, int tokens,
                             float *out) {
    return orc_cpu_reference_decode_formats(query_heads, kv_heads, head_dim, query, keys, dtype,
                                            values, dtype, tokens, out);
}

int orc_cpu_reference_decode_formats(int query_heads, int kv_heads, int head_dim,
                                     const float *query, const void *keys, int key_dtype,
                                     const void *values, int value_dtype, int tokens,
                                     float *out) {
    if (query_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || query_heads % kv_heads ||
        key_dtype < 1 || key_dtype > 3 || value_dtype < 1 || value_dtype > 3 || tokens < 0)
        return 1;
    const size_t qn = (size_t)query_heads * head_dim;
    for (size_t i = 0; i < qn; ++i) if (!isfinite(query[i])) return 2;
    if (tokens == 0) { for (size_t i = 0; i < qn; ++i) out[i] = 0.0f; return 0; }
    const double scale = 1.0 / sqrt((double)head_dim);
    double *weighted = (double *)malloc(sizeof(double) * (size_t)head_dim);
    if (!weighted) return 1;
    const int group = query_heads / kv_heads;
    for (int qh = 0; qh < query_heads; ++qh) {
        const int kh = qh / group;
        const float *q = query + (size_t)qh * head_dim;
        double max_score = -INFINITY, denominator = 0.0;
        for (int d = 0; d < head_dim; ++d) weighted[d] = 0.0;
        for (int t = 0; t < tokens; ++t) {
            const size_t off = ((size_t)t * kv_heads + kh) * head_dim;
            double dot = 0.0;
            for (int d = 0; d < head_dim; ++d) {
                const float kv = element(keys, off + d, key_dtype);
                if (!isfinite(kv)) { free(weighted); return 2; }
                dot += (double)q[d] * (double)kv;
            }
            const double score = dot * scale;
            if (!isfinite(score)) { free(weighted); return 2; }
            const double next_max = fmax(max_score, score);
            const double prior = exp(max_score - next_max);
            const double current = exp(score - next_max);
            denominator = denominator * prior + current;
            for (int d = 0; d < head_dim; ++d) {
                const float item = element(values, off + d, value_dtype);
                if (!isfinite(item)) { free(weighted); return 2; }
                weighted[d] = weighted[d] * prior + current * (double)item;
            }
            max_score = next_max;
        }
        if (!isfinite(denominator) || denominator <= 0.0) { free(weighted); return 2; }
        for (int d = 0; d < head_dim; ++d) {
            const double v = weighted[d] / denominator;
            if (!isfinite(v) || fabs(v) > 3.4028234663852886e38) { free(weighted); return 2; }
            out[(size_t)qh * head_dim + d] = (float)v;
        }
    }
    free(weighted);
    return 0;
}

int orc_prefill_causal_cpu(int query_heads, int kv_heads, int head_dim,
                           const float *query, const uint16_t *keys,
                           const uint16_t *values, int queries, int prior,
                           float *out) {
    const size_t row = (size_t)query_heads * head_dim;
    for (int i = 0; i < queries; ++i) {
        const int rc = orc_dense_attention_bf16(query_heads, kv_heads, head_dim,
                                                query + row * i, keys, values,
                                                prior + i + 1, out + row * i);
        if (rc) return rc;
    }
    return 0;
}

int orc_gpu_reference_attention(int query_heads, int kv_heads, int head_dim,
                                const uint16_t *query, const uint16_t *keys,
                                const uint16_t *values, int queries, int prior,
                                uint16_t *out) {
    if (query_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || query_heads % kv_heads ||
        queries <= 0 || prior < 0) return -1;
    const int group = query_heads / kv_heads;
    const int history = prior + queries;
    const float rs = 1.0f / sqrtf((float)head_dim);
    float *s = (float *)malloc(sizeof(float) * (size_t)history);
    if (!s) return -1;
    for (int token = 0; token < queries; ++token) {
        const int valid = prior + token + 1;
        for (int qh = 0; qh < query_heads; ++qh) {
            const int kh = qh / group;
            const uint16_t *q = query + ((size_t)token * query_heads + qh) * head_dim;
            for (int k = 0; k < valid; ++k) {
                const uint16_t *kr = keys + ((size_t)k * kv_heads + kh) * head_dim;
                float dot = 0.0f;
                for (int d = 0; d < head_dim; ++d)
                    dot = fmaf(orc_read_bf16(q[d]), orc_read_bf16(kr[d]), dot);
                s[k] = dot * rs;
            }
            float maxval = -INFINITY;
            for (int k = 0; k < valid; ++k) maxval = fmaxf(maxval, s[k]);
            float denom = 0.0f;
            for (int k = 0; k < valid; ++k) { s[k] = exp_f(s[k] - maxval); denom += s[k]; }
            for (int k = 0; k < valid; ++k) s[k] /= denom;
            uint16_t *o = out + ((size_t)token * query_heads + qh) * head_dim;
            for (int d = 0; d < head_dim; ++d) {
                float sum = 0.0f;
                for (int k = 0; k < valid; ++k)
                    sum = fmaf(s[k], orc_read_bf16(values[((size_t)k * kv_heads + kh) * head_dim + d]), sum);
                o[d] = orc_write_bf16(sum);
            }
        }
    }
    free(s);
    return 0;
}

/* ---- Feeder kernels ----------------------------------------------------- */
void orc_rms_norm_cpu(const float *x, const float *w, int n, float eps, float *out) {
    float sum = -0.0f;
    for (int i = 0; i < n; ++i) sum += x[i] * x[i];
    const float mean = sum / (float)n;
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int i = 0; i < n; ++i) {
        const float normalized = round_bf16(x[i] * scale);
        out[i] = round_bf16(normalized * w[i]);
    }
}

void orc_rmsnorm_gpu(const uint16_t *x, const uint16_t *w, int tokens, int hidden,
                     float eps, uint16_t *out) {
    float partials[128];
    for (int t = 0; t < tokens; ++t) {
        const uint16_t *row = x + (size_t)t * hidden;
        for (int tid = 0; tid < 128; ++tid) {
            float s = 0.0f;
            for (int i = tid; i < hidden; i += 128) {
                const float v = orc_read_bf16(row[i]);
                s = fmaf(v, v, s);
            }
            partials[tid] = s;
        }
        for (int stride = 64; stride > 0; stride >>= 1)
            for (int tid = 0; tid < stride; ++tid) partials[tid] += partials[tid + stride];
        const float factor = 1.0f / sqrtf(partials[0] / (float)hidden + eps);
        for (int i = 0; i < hidden; ++i) {
            const uint16_t normalized = orc_write_bf16(orc_read_bf16(row[i]) * factor);
            out[(size_t)t * hidden + i] =
                orc_write_bf16(orc_read_bf16(normalized) * orc_read_bf16(w[i]));
        }
    }
}

float orc_rope_inverse_frequency(int frequency_dim, int head_dim, float theta,
                                 int llama3, float factor, float low_freq,
                                 float high_freq, float original_max_position) {
    const float exponent = (-(float)frequency_dim * log_f(theta)) / (float)head_dim;
    float inv = exp_f(exponent);
    if (llama3) {
        const float wavelength = 6.28318530717958647692f / inv;
        const float low_wavelength = original_max_position / low_freq;
        const float high_wavelength = original_max_position / high_freq;
        if (wavelength > low_wavelength) {
            inv /= factor;
        } else if (wavelength >= high_wavelength) {
            const float smooth = (original_max_position / wavelength - low_freq) /
                                 (high_freq - low_freq);
            const float a = (1.0f - smooth) * (inv / factor);
            const float b = smooth * inv;
            inv = a + b;
        }
    }
    return inv;
}

void orc_rope_gpu(const uint16_t *x, uint16_t *out, int tokens, int heads,
                  int head_dim, int start_position, float theta, int llama3,
                  float factor, float low_freq, float high_freq,
                  float original_max_position) {
    const int half = head_dim / 2;
    const size_t elements = (size_t)heads * head_dim;
    for (int t = 0; t < tokens; ++t) {
        for (size_t in_token = 0; in_token < elements; ++in_token) {
            const size_t i = (size_t)t * elements + in_token;
            const int head = (int)(in_token / head_dim), d = (int)(in_token % head_dim);
            const size_t src = (size_t)t * elements + (size_t)head * head_dim +
                               (d < half ? d + half : d - half);
            const float rotated = d < half ? -orc_read_bf16(x[src]) : orc_read_bf16(x[src]);
            const int fd = (d % half) * 2;
            const float inv = orc_rope_inverse_frequency(fd, head_dim, theta, llama3, factor,
                                                         low_freq, high_freq,
                                                         original_max_position);
            const float phase = (float)(start_position + t) * inv;
            const float c = orc_read_bf16(orc_write_bf16(cos_f(phase)));
            const float s = orc_read_bf16(orc_write_bf16(sin_f(phase)));
            const float left = orc_read_bf16(orc_write_bf16(orc_read_bf16(x[i]) * c));
            const float right = orc_read_bf16(orc_write_bf16(rotated * s));
            out[i] = orc_write_bf16(left + right);
        }
    }
}

void orc_rope_cpu(float *values, int heads, int dim, int position, float theta) {
    const int half = dim / 2;
    for (int head = 0; head < heads; ++head) {
        float *base = values + (size_t)head * dim;
        for (int i = 0; i < half; ++i) {
            const float angle = (float)position / pow_f(theta, (float)(2 * i) / (float)dim);
            const float sn = round_bf16(sin_f(angle));
            const float cs = round_bf16(cos_f(angle));
            const float a = base[i], b = base[i + half];
            base[i] = round_bf16(round_bf16(a * cs) - round_bf16(b * sn));
            base[i + half] = round_bf16(round_bf16(b * cs) + round_bf16(a * sn));
        }
    }
}

void orc_swiglu(const uint16_t *gate, const uint16_t *up, size_t n, uint16_t *out) {
    for (size_t i = 0; i < n; ++i) {
        const float g = orc_read_bf16(gate[i]);
        const float activated = g / (1.0f + exp_f(-g));
        const uint16_t gb = orc_write_bf16(activated);
        out[i] = orc_write_bf16(orc_read_bf16(gb) * orc_read_bf16(up[i]));
    }
}

/* gpu_llm.cl:214-222 llm_add: one f32 add, one BF16 rounding. */
void orc_add_bf16(const uint16_t *a, const uint16_t *b, size_t n, uint16_t *out) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_write_bf16(orc_read_bf16(a[i]) + orc_read_bf16(b[i]));
}

/* gpu_llm.cl:239-270 llm_argmax with one lane: the scan's update rule alone
 * fixes the result, whatever the lane count of the reduction. */
void orc_argmax_bf16(const uint16_t *logits, int rows, int vocab, int32_t *out) {
    for (int r = 0; r < rows; ++r) {
        const uint16_t *l = logits + (size_t)r * vocab;
        float best = -INFINITY;
        int32_t index = 0;
        for (int i = 0; i < vocab; ++i) {
            const float x = orc_read_bf16(l[i]);
            if (x > best || (x == best && i < index)) {
                best = x;
                index = i;
            }
        }
        out[r] = index;
    }
}

/* Eight rows per step of the inner loops below: eight independent sums, each
 * still added in ascending order, so every output is unchanged. */
#define ORC_ROWS 8

/* hipblaslt_bridge.cpp:203-233 tv_hip_matrix_multiply: out[t][r] =
 * BF16(sum_i in[t][i] * w[r][i]), products and sum in fp32 (ascending i),
 * one rounding at the end.  pin: identity weight reproduces the input bit for
 * bit, linearity in the weight, f64 brute force on small shapes. */
void orc_matmul_bf16(const uint16_t *w, const uint16_t *in, int inner, int rows, int tokens, uint16_t *out) {
    /* Outputs are independent: rows split over OpenMP threads, each sum in
     * ascending i as before. */
    const int blocks = (rows + ORC_ROWS - 1) / ORC_ROWS;
    for (int t = 0; t < tokens; ++t) {
        const uint16_t *xt = in + (size_t)t * inner;
#pragma omp parallel for schedule(static)
        for (int blk = 0; blk < blocks; ++blk) {
            const int r0 = blk * ORC_ROWS;
            const int n = rows - r0 < ORC_ROWS ? rows - r0 : ORC_ROWS;
            const uint16_t *wr[ORC_ROWS];
            float acc[ORC_ROWS];
            for (int j = 0; j < ORC_ROWS; ++j) {
                wr[j] = w + (size_t)(r0 + (j < n ? j : 0)) * inner;
                acc[j] = 0.0f;
            }
            for (int i = 0; i < inner; ++i) {
                const float xi = orc_read_bf16(xt[i]);
                for (int j = 0; j < ORC_ROWS; ++j) acc[j] = fmaf(orc_read_bf16(wr[j][i]), xi, acc[j]);
            }
            for (int j = 0; j < n; ++j) out[(size_t)t * rows + r0 + j] = orc_write_bf16(acc[j]);
        }
    }
}

void orc_matvec_cpu(const uint16_t *w, const float *x, int rows, int cols, float *out) {
    const int blocks = (rows + ORC_ROWS - 1) / ORC_ROWS;
#pragma omp parallel for schedule(static)
    for (int blk = 0; blk < blocks; ++blk) {
        const int r0 = blk * ORC_ROWS;
        const int n = rows - r0 < ORC_ROWS ? rows - r0 : ORC_ROWS;
        const uint16_t *wr[ORC_ROWS];
        float sum[ORC_ROWS];
        for (int j = 0; j < ORC_ROWS; ++j) {
            wr[j] = w + (size_t)(r0 + (j < n ? j : 0)) * cols;
            sum[j] = -0.0f;
        }
        for (int i = 0; i < cols; ++i) {
            const float xi = x[i];
            for (int j = 0; j < ORC_ROWS; ++j) {
                const float product = orc_read_bf16(wr[j][i]) * xi;
                sum[j] += product;
            }
        }
        for (int j = 0; j < n; ++j) out[r0 + j] = round_bf16(sum[j]);
    }
}

/* IEEE total order key of an f32 (Rust's f32::total_cmp). */
static int32_t total_key(float x) {
    int32_t bits;
    memcpy(&bits, &x, 4);
    return bits ^ (int32_t)(((uint32_t)(bits >> 31)) >> 1);
}

int32_t orc_argmax_total_last(const float *logits, int n) {
    int32_t index = 0;
    for (int i = 1; i < n; ++i)
        if (total_key(logits[i]) >= total_key(logits[index])) index = i;
    return n > 0 ? index : -1;
}

/* ---- Integrity primitives ----------------------------------------------- */
uint64_t orc_fnv1a64(const uint8_t *bytes, size_t n, uint64_t state) {
    for (size_t i = 0; i < n; ++i) {
        state ^= (uint64_t)bytes[i];
        state *= 0x100000001b3ull;
    }
    return state;
}

static const uint32_t K256[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
    0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
    0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
    0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
    0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
    0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};

static inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

static void sha_block(uint32_t h[8], const uint8_t *p) {
    uint32_t w[64];
    for (int i = 0; i < 16; ++i)
        w[i] = (uint32_t)p[4 * i] << 24 | (uint32_t)p[4 * i + 1] << 16 |
               (uint32_t)p[4 * i + 2] << 8 | p[4 * i + 3];
    for (int i = 16; i < 64; ++i) {
        const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
        const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
        w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
    for (int i = 0; i < 64; ++i) {
        const uint32_t t1 = hh + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) +
                            K256[i] + w[i];
        const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
        hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
    }
    h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
}

void orc_sha256_init(orc_sha256_ctx *c) {
    static const uint32_t iv[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                                   0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    memcpy(c->h, iv, sizeof iv);
    c->len = 0;
    c->fill = 0;
}

void orc_sha256_update(orc_sha256_ctx *c, const uint8_t *data, size_t n) {
    c->len += n;
    while (n) {
        const size_t take = (64 - c->fill) < n ? (64 - c->fill) : n;
        memcpy(c->buf + c->fill, data, take);
        c->fill += take; data += take; n -= take;
        if (c->fill == 64) { sha_block(c->h, c->buf); c->fill = 0; }
    }
}

void orc_sha256_final(orc_sha256_ctx *c, uint8_t out[32]) {
    const uint64_t bits = c->len * 8;
    uint8_t pad = 0x80;
    orc_sha256_update(c, &pad, 1);
    const uint8_t zero = 0;
    while (c->fill != 56) orc_sha256_update(c, &zero, 1);
    uint8_t len[8];
    for (int i = 0; i < 8; ++i) len[i] = (uint8_t)(bits >> (56 - 8 * i));
    orc_sha256_update(c, len, 8);
    for (int i = 0; i < 8; ++i) {
        out[4 * i] = (uint8_t)(c->h[i] >> 24); out[4 * i + 1] = (uint8_t)(c->h[i] >> 16);
        out[4 * i + 2] = (uint8_t)(c->h[i] >> 8); out[4 * i + 3] = (uint8_t)c->h[i];
    }
}

void orc_sha256(const uint8_t *data, size_t n, uint8_t out[32]) {
    orc_sha256_ctx c;
    orc_sha256_init(&c);
    orc_sha256_update(&c, data, n);
    orc_sha256_final(&c, out);
}

/* ---- ColdStore record and region store --------------------------------- */
int orc_token_hashes(const uint8_t *payload, size_t len, uint32_t tokens,
                     uint32_t heads, uint64_t *out) {
    const uint64_t elements = (uint64_t)heads * tokens;
    if (!elements || len % elements) return -1;
    const size_t per = (size_t)(len / elements);
    for (uint32_t t = 0; t < tokens; ++t) {
        uint64_t state = 0xcbf29ce484222325ull;
        for (uint32_t h = 0; h < heads; ++h)
            state = orc_fnv1a64(payload + ((size_t)h * tokens + t) * per, per, state);
        out[t] = state;
    }
    return 0;
}

static void put_u32(uint8_t *p, uint32_t v) { for (int i = 0; i < 4; ++i) p[i] = (uint8_t)(v >> (8 * i)); }
static void put_u64(uint8_t *p, uint64_t v) { for (int i = 0; i < 8; ++i) p[i] = (uint8_t)(v >> (8 * i)); }

size_t orc_coldstore_record(uint64_t page_id, uint32_t layer, uint64_t token_start,
                            uint32_t tokens, uint32_t heads, uint32_t head_dim,
                            uint32_t tile, const uint8_t *key, size_t key_len,
                            const uint8_t *value, size_t value_len,
                            uint8_t *record, size_t cap) {
    /* cold_store.rs:702-723 validate_geometry */
    if (!tokens || !heads || !head_dim || !tile || head_dim % tile || !key_len || !value_len)
        return 0;
    const uint64_t elements = (uint64_t)heads * tokens;
    if (key_len % elements || value_len % elements) return 0;
    const size_t hash_bytes = (size_t)tokens * 8;
    const size_t total = 104 + 2 * hash_bytes + key_len + value_len + 56;
    if (!record || cap < total) return total;
    uint64_t *kh = (uint64_t *)malloc(hash_bytes), *vh = (uint64_t *)malloc(hash_bytes);
    if (!kh || !vh) { free(kh); free(vh); return 0; }
    orc_token_hashes(key, key_len, tokens, heads, kh);
    orc_token_hashes(value, value_len, tokens, heads, vh);
    uint8_t *p = record;
    memcpy(p, "TSKVPG04", 8);
    put_u32(p + 8, 3); put_u32(p + 12, 104); put_u64(p + 16, page_id);
    put_u32(p + 24, layer); put_u32(p + 28, 0); put_u64(p + 32, token_start);
    put_u32(p + 40, tokens); put_u32(p + 44, heads); put_u32(p + 48, head_dim);
    put_u32(p + 52, tile); put_u64(p + 56, key_len); put_u64(p + 64, value_len);
    uint8_t *khb = p + 104, *vhb = khb + hash_bytes;
    for (uint32_t t = 0; t < tokens; ++t) { put_u64(khb + 8 * t, kh[t]); put_u64(vhb + 8 * t, vh[t]); }
    const uint64_t basis = 0xcbf29ce484222325ull;
    put_u64(p + 72, orc_fnv1a64(key, key_len, basis));
    put_u64(p + 80, orc_fnv1a64(value, value_len, basis));
    put_u64(p + 88, orc_fnv1a64(khb, hash_bytes, basis));
    put_u64(p + 96, orc_fnv1a64(vhb, hash_bytes, basis));
    memcpy(vhb + hash_bytes, key, key_len);
    memcpy(vhb + hash_bytes + key_len, value, value_len);
    const size_t body = total - 56;
    uint8_t *footer = p + body;
    memcpy(footer, "TSKVCMIT", 8);
    put_u64(footer + 8, orc_fnv1a64(p, body, basis));
    put_u64(footer + 16, (uint64_t)total);
    orc_sha256(p, body, footer + 24);
    free(kh); free(vh);
    return total;
}

void orc_token_to_head_major(const uint8_t *token_major, uint32_t n, uint32_t kvh,
                             uint32_t row_bytes, uint8_t *head_major) {
    for (uint32_t h = 0; h < kvh; ++h)
        for (uint32_t t = 0; t < n; ++t)
            memcpy(head_major + ((size_t)h * n + t) * row_bytes,
                   token_major + ((size_t)t * kvh + h) * row_bytes, row_bytes);
}

void orc_gather_token_major(const uint8_t *pool, size_t page_bytes,
                            uint32_t page_tokens, uint32_t kvh, uint32_t row_bytes,
                            const uint32_t *page_of, const uint32_t *offset_of,
                            const uint32_t *positions, size_t count, uint8_t *out) {
    for (size_t i = 0; i < count; ++i) {
        const uint32_t t = positions[i];
        const uint8_t *page = pool + (size_t)page_of[t] * page_bytes;
        for (uint32_t h = 0; h < kvh; ++h)
            memcpy(out + (i * kvh + h) * row_bytes,
                   page + ((size_t)h * page_tokens + offset_of[t]) * row_bytes, row_bytes);
    }
}

void orc_logical_kv_sha256(uint32_t layers, uint64_t tokens, uint32_t kvh,
                           uint32_t row_bytes, const uint8_t *const *keys,
                           const uint8_t *const *values, uint8_t out[32]) {
    orc_sha256_ctx c;
    orc_sha256_init(&c);
    static const char tag[] = "mslim-dense-kv-state-v1";
    orc_sha256_update(&c, (const uint8_t *)tag, sizeof tag - 1);
    uint8_t le[8];
    put_u64(le, tokens);
    orc_sha256_update(&c, le, 8);
    for (uint32_t layer = 0; layer < layers; ++layer) {
        const uint8_t *parts[2] = {keys[layer], values[layer]};
        for (int p = 0; p < 2; ++p)
            for (uint32_t h = 0; h < kvh; ++h)
                for (uint64_t t = 0; t < tokens; ++t)
                    orc_sha256_update(&c, parts[p] + ((size_t)t * kvh + h) * row_bytes, row_bytes);
    }
    orc_sha256_final(&c, out);
}
