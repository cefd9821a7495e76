/* attention_oracle.c — TEST INFRASTRUCTURE ONLY. A serial CPU restatement of the reference's attention
 * bodies, used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the CHECKER. The
 * product (silvann_amd/) never links, loads or calls it.
 *
 * It follows engine/src/packages/nn/gpu/kernels/kernels.cuh as the reference's host family runs those
 * bodies: one lane of one block (silicon_families/host/nn.cuh:115-162 — lanes()=1, lanes_sum/max the
 * identity), libm expf/sqrtf, every sum serial and in the body's order, no contraction into FMA
 * (built with -ffp-contract=off; oracle_rope_rows writes the reference build's two FMAs out). Each function names
 * the body it restates.
 *
 * How each function is pinned (tests/test_oracle_*.py):
 *   - against the reference's own x86_avx2 family built from /root/reference (oracle/_ref), bit for bit
 *     on the rows that family runs through the generic body (scores, merge, finish, causal_scores,
 *     scores_grouped, softmax_rows, causal_softmax, scores_grouped_rows, softmax_lens, mix_rows), and
 *     within fp32 rounding on the rows it overrides with its own loop order (mix, weights,
 *     residual_mix, causal_scores_grouped, causal_mix);
 *   - against committed golden vectors made by that family (tests/golden/);
 *   - against closed forms in float64 (one position gives v; constant keys give the mean of v; causal
 *     row r equals decode at first + r; merge(A, B) equals one call over A ∪ B) and against exhaustive
 *     half<->float round trips.
 * The paged functions are the reference's decode/causal over the gathered-contiguous cache (the reference
 * has no pages); they are pinned by the page-table permutation invariance and by the contiguous form. */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define FAULT_OVERFLOW 0x4E504F56u /* "NPOV", contracts/objects/primitives.cuh:57 */

/* kernels.cuh:2733-2757 — exact widening of a half. */
float oracle_half_to_float(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t exp = ((uint32_t)h >> 10) & 0x1Fu;
    const uint32_t mant = (uint32_t)h & 0x3FFu;
    uint32_t bits;
    if (exp == 0u) {
        if (mant == 0u) {
            bits = sign;
        } else {
            uint32_t top = 0u, walk = mant;
            while ((walk >> 1) != 0u) { walk >>= 1; top += 1u; }
            bits = sign | ((uint32_t)((int)top - 24 + 127) << 23) | ((mant - (1u << top)) << (23u - top));
        }
    } else if (exp == 31u) {
        bits = sign | 0x7F800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* kernels.cuh:2763-2808 — round to nearest even, subnormals kept; a finite input that lands past the
 * largest half (including by the rounding carry) sets *over; inf/NaN inputs pass through unflagged. */
uint16_t oracle_float_to_half(float f, int* over) {
    uint32_t bits;
    memcpy(&bits, &f, 4);
    const uint32_t sign = (bits >> 16) & 0x8000u;
    const uint32_t e = (bits >> 23) & 0xFFu;
    uint32_t m = bits & 0x7FFFFFu;
    if (e == 0xFFu) return (uint16_t)(sign | 0x7C00u | (m != 0u ? ((m >> 13) | 0x200u) : 0u));
    int32_t he = (int32_t)e - 127 + 15;
    if (he >= 0x1F) { if (over) *over = 1; return (uint16_t)(sign | 0x7C00u); }
    if (he > 0) {
        uint32_t mh = m >> 13;
        const uint32_t rem = m & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (mh & 1u) != 0u)) {
            mh += 1u;
            if (mh == 0x400u) {
                mh = 0u;
                he += 1;
                if (he >= 0x1F) { if (over) *over = 1; return (uint16_t)(sign | 0x7C00u); }
            }
        }
        return (uint16_t)(sign | ((uint32_t)he << 10) | mh);
    }
    if (he < -10) return (uint16_t)sign;
    m |= 0x800000u;
    const uint32_t shift = (uint32_t)(14 - he);
    uint32_t mh = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1u);
    if (rem > halfway || (rem == halfway && (mh & 1u) != 0u)) mh += 1u;
    return (uint16_t)(sign | mh);
}

static inline float h2f(uint16_t h) { return oracle_half_to_float(h); }

/* host/nn.cuh:155-158 and x86_avx2/primitives/nn.cuh:49-52 — (c + lo·lo) + hi·hi. */
static inline float dot2(uint32_t a, uint32_t b, float c) {
    return (c + h2f((uint16_t)(a & 0xffffu)) * h2f((uint16_t)(b & 0xffffu))) + h2f((uint16_t)(a >> 16)) * h2f((uint16_t)(b >> 16));
}

/* kernels.cuh:894-915 — one query head's scores, their largest, the softmax, serially. */
static void scores_head(float* ph, const uint16_t* qh, const uint16_t* kh, uint64_t row, uint64_t head_dim,
                        uint64_t length, float scale) {
    float top = -INFINITY;
    for (uint64_t t = 0; t < length; ++t) {
        float dot = 0.0f;
        for (uint64_t e = 0; e < head_dim; ++e) dot += h2f(qh[e]) * h2f(kh[t * row + e]);
        ph[t] = dot * scale;
        if (ph[t] > top) top = ph[t];
    }
    float part = 0.0f;
    for (uint64_t t = 0; t < length; ++t) {
        ph[t] = expf(ph[t] - top);
        part += ph[t];
    }
    const float inv = 1.0f / part;
    for (uint64_t t = 0; t < length; ++t) ph[t] *= inv;
}

/* kernels.cuh:1133-1141 */
void oracle_attention_scores(float* p, const uint16_t* q, const uint16_t* k, uint64_t q_heads, uint64_t kv_heads,
                             uint64_t head_dim, uint64_t length) {
    const uint64_t group = q_heads / kv_heads, row = kv_heads * head_dim;
    const float scale = 1.0f / sqrtf((float)head_dim);
    for (uint64_t h = 0; h < q_heads; ++h)
        scores_head(p + h * length, q + h * head_dim, k + (h / group) * head_dim, row, head_dim, length, scale);
}

/* kernels.cuh:1144-1154 */
static void mix_head(uint16_t* oh, const float* ph, const uint16_t* vh, uint64_t row, uint64_t head_dim,
                     uint64_t length, uint32_t* over) {
    for (uint64_t e = 0; e < head_dim; ++e) {
        float sum = 0.0f;
        for (uint64_t t = 0; t < length; ++t) sum += ph[t] * h2f(vh[t * row + e]);
        int hit = 0;
        oh[e] = oracle_float_to_half(sum, &hit);
        if (hit) *over = FAULT_OVERFLOW;
    }
}

/* kernels.cuh:1156-1164 */
void oracle_attention_mix(uint16_t* o, const float* p, const uint16_t* v, uint64_t q_heads, uint64_t kv_heads,
                          uint64_t head_dim, uint64_t length, uint32_t* over) {
    const uint64_t group = q_heads / kv_heads, row = kv_heads * head_dim;
    for (uint64_t h = 0; h < q_heads; ++h)
        mix_head(o + h * head_dim, p + h * length, v + (h / group) * head_dim, row, head_dim, length, over);
}

/* kernels.cuh:1190-1221 — unnormalised weights e^(s - m) into p, {m, l} into res. */
void oracle_attention_weights(float* p, float* res, const uint16_t* q, const uint16_t* k, uint64_t q_heads,
                              uint64_t kv_heads, uint64_t head_dim, uint64_t length) {
    const uint64_t group = q_heads / kv_heads, row = kv_heads * head_dim, w = head_dim + 2;
    const float scale = 1.0f / sqrtf((float)(uint32_t)head_dim);
    for (uint64_t h = 0; h < q_heads; ++h) {
        const uint16_t* qh = q + h * head_dim;
        const uint16_t* kh = k + (h / group) * head_dim;
        float* ph = p + h * length;
        float top = -INFINITY;
        for (uint64_t t = 0; t < length; ++t) {
            float dot = 0.0f;
            for (uint64_t e = 0; e < head_dim; ++e) dot += h2f(qh[e]) * h2f(kh[t * row + e]);
            ph[t] = dot * scale;
            if (ph[t] > top) top = ph[t];
        }
        float part = 0.0f;
        for (uint64_t t = 0; t < length; ++t) {
            ph[t] = expf(ph[t] - top);
            part += ph[t];
        }
        res[h * w] = top;
        res[h * w + 1] = part;
    }
}

/* kernels.cuh:1224-1238 */
void oracle_attention_residual_mix(float* res, const float* p, const uint16_t* v, uint64_t q_heads,
                                   uint64_t kv_heads, uint64_t head_dim, uint64_t length) {
    const uint64_t group = q_heads / kv_heads, row = kv_heads * head_dim, w = head_dim + 2;
    for (uint64_t h = 0; h < q_heads; ++h) {
        const float* ph = p + h * length;
        const uint16_t* vh = v + (h / group) * head_dim;
        float* acc = res + h * w + 2;
        for (uint64_t e = 0; e < head_dim; ++e) {
            float sum = 0.0f;
            for (uint64_t t = 0; t < length; ++t) sum += ph[t] * h2f(vh[t * row + e]);
            acc[e] = sum;
        }
    }
}

/* kernels.cuh:1243-1255 — a head's two m and l read before anything is written, so `into` may alias. */
void oracle_attention_merge(float* into, const float* a, const float* b, uint64_t q_heads, uint64_t head_dim) {
    const uint64_t w = head_dim + 2;
    for (uint64_t h = 0; h < q_heads; ++h) {
        const float ma = a[h * w], la = a[h * w + 1], mb = b[h * w], lb = b[h * w + 1];
        const float m = ma > mb ? ma : mb;
        const float fa = expf(ma - m), fb = expf(mb - m);
        for (uint64_t e = 0; e < head_dim; ++e) into[h * w + 2 + e] = a[h * w + 2 + e] * fa + b[h * w + 2 + e] * fb;
        into[h * w] = m;
        into[h * w + 1] = la * fa + lb * fb;
    }
}

/* kernels.cuh:1258-1267 */
void oracle_attention_finish(uint16_t* o, const float* res, uint64_t q_heads, uint64_t head_dim, uint32_t* over) {
    const uint64_t w = head_dim + 2, n = q_heads * head_dim;
    for (uint64_t i = 0; i < n; ++i) {
        const uint64_t h = i / head_dim;
        int hit = 0;
        o[i] = oracle_float_to_half(res[h * w + 2 + i % head_dim] / res[h * w + 1], &hit);
        if (hit) *over = FAULT_OVERFLOW;
    }
}

/* kernels.cuh:2039-2049 */
void oracle_attention_causal_scores(float* p, const uint16_t* q, const uint16_t* k, uint64_t q_heads,
                                    uint64_t kv_heads, uint64_t head_dim, uint64_t first, uint64_t rows) {
    const uint64_t group = q_heads / kv_heads, row = kv_heads * head_dim, span = first + rows;
    const float scale = 1.0f / sqrtf((float)head_dim);
    for (uint64_t i = 0; i < rows * q_heads; ++i) {
        const uint64_t r = i / q_heads, h = i - r * q_heads;
        scores_head(p + i * span, q + i * head_dim, k + (h / group) * head_dim, row, head_dim, first + r + 1, scale);
    }
}

/* kernels.cuh:2051-2060 */
void oracle_attention_causal_mix(uint16_t* o, const float* p, const uint16_t* v, uint64_t q_heads,
                                 uint64_t kv_heads, uint64_t head_dim, uint64_t first, uint64_t rows,
                                 uint32_t* over) {
    const uint64_t group = q_heads / kv_heads, row = kv_heads * head_dim, span = first + rows;
    for (uint64_t i = 0; i < rows * q_heads; ++i) {
        const uint64_t r = i / q_heads, h = i - r * q_heads;
        mix_head(o + i * head_dim, p + i * span, v + (h / group) * head_dim, row, head_dim, first + r + 1, over);
    }
}

/* kernels.cuh:976-992 — the dot of one query head with `span` key rows from t0, two halves a step through
 * dot2 where the operands are 4-byte aligned, else the plain per-element sum. */
static void dots(float* dot, const uint16_t* qh, const uint16_t* kh, uint64_t row, uint64_t head_dim, uint64_t t0,
                 uint64_t span) {
    for (uint64_t j = 0; j < span; ++j) dot[j] = 0.0f;
    if (head_dim % 2 == 0 && row % 2 == 0 && ((uintptr_t)qh) % 4u == 0 && ((uintptr_t)kh) % 4u == 0) {
        const uint32_t* q2 = (const uint32_t*)qh;
        const uint32_t* k2 = (const uint32_t*)kh;
        for (uint64_t e = 0; e < head_dim / 2; ++e) {
            const uint32_t qe = q2[e];
            for (uint64_t j = 0; j < span; ++j) dot[j] = dot2(qe, k2[((t0 + j) * row) / 2 + e], dot[j]);
        }
    } else {
        for (uint64_t e = 0; e < head_dim; ++e) {
            const float qe = h2f(qh[e]);
            for (uint64_t j = 0; j < span; ++j) dot[j] += qe * h2f(kh[(t0 + j) * row + e]);
        }
    }
}

#define GROUP_SPAN 8u /* kernels.cuh:925 NN__ATTENTION__GROUP_SPAN */

/* kernels.cuh:928-948 — raw scaled scores, a tile of 8 positions a step (order-neutral per dot). */
void oracle_attention_scores_grouped(float* p, const uint16_t* q, const uint16_t* k, uint64_t q_heads,
                                     uint64_t kv_heads, uint64_t head_dim, uint64_t length) {
    const uint64_t group = q_heads / kv_heads, row = kv_heads * head_dim;
    const float scale = 1.0f / sqrtf((float)head_dim);
    float dot[GROUP_SPAN];
    for (uint64_t h = 0; h < q_heads; ++h)
        for (uint64_t t0 = 0; t0 < length; t0 += GROUP_SPAN) {
            const uint64_t span = length - t0 < GROUP_SPAN ? length - t0 : GROUP_SPAN;
            dots(dot, q + h * head_dim, k + (h / group) * head_dim, row, head_dim, t0, span);
            for (uint64_t j = 0; j < span; ++j) p[h * length + t0 + j] = dot[j] * scale;
        }
}

/* kernels.cuh:953-972 */
void oracle_attention_scores_grouped_rows(float* p, uint64_t p_row, const uint16_t* q, uint64_t q_row,
                                          const uint16_t* k, uint64_t k_row, const uint32_t* lens, uint64_t q_heads,
                                          uint64_t kv_heads, uint64_t head_dim, uint64_t most, uint64_t rows) {
    (void)most;
    const uint64_t group = q_heads / kv_heads, row = kv_heads * head_dim;
    const float scale = 1.0f / sqrtf((float)head_dim);
    float dot[GROUP_SPAN];
    for (uint64_t u = 0; u < rows; ++u) {
        const uint64_t length = lens[u];
        for (uint64_t h = 0; h < q_heads; ++h)
            for (uint64_t t0 = 0; t0 < length; t0 += GROUP_SPAN) {
                const uint64_t span = length - t0 < GROUP_SPAN ? length - t0 : GROUP_SPAN;
                dots(dot, q + u * q_row + h * head_dim, k + u * k_row + (h / group) * head_dim, row, head_dim, t0, span);
                for (uint64_t j = 0; j < span; ++j) p[u * p_row + h * length + t0 + j] = dot[j] * scale;
            }
    }
}

/* kernels.cuh:1028-1061 — each stored score is one `dots` sum (the 4-row form keeps each dot's order). */
void oracle_attention_causal_scores_grouped(float* p, const uint16_t* q, const uint16_t* k, uint64_t q_heads,
                                            uint64_t kv_heads, uint64_t head_dim, uint64_t first, uint64_t rows) {
    const uint64_t group = q_heads / kv_heads, row = kv_heads * head_dim, span_all = first + rows;
    const float scale = 1.0f / sqrtf((float)head_dim);
    float dot[GROUP_SPAN];
    for (uint64_t r = 0; r < rows; ++r)
        for (uint64_t h = 0; h < q_heads; ++h) {
            const uint64_t len = first + r + 1;
            for (uint64_t t0 = 0; t0 < len; t0 += GROUP_SPAN) {
                const uint64_t span = span_all - t0 < GROUP_SPAN ? span_all - t0 : GROUP_SPAN;
                dots(dot, q + (r * q_heads + h) * head_dim, k + (h / group) * head_dim, row, head_dim, t0, span);
                for (uint64_t j = 0; j < span && t0 + j < len; ++j) p[(r * q_heads + h) * span_all + t0 + j] = dot[j] * scale;
            }
        }
}

/* kernels.cuh:1085-1094 */
static void softmax_row(float* ph, uint64_t length) {
    float top = -INFINITY;
    for (uint64_t t = 0; t < length; ++t) if (ph[t] > top) top = ph[t];
    float part = 0.0f;
    for (uint64_t t = 0; t < length; ++t) {
        ph[t] = expf(ph[t] - top);
        part += ph[t];
    }
    const float inv = 1.0f / part;
    for (uint64_t t = 0; t < length; ++t) ph[t] *= inv;
}

/* kernels.cuh:1065-1081 */
void oracle_attention_causal_softmax(float* p, uint64_t q_heads, uint64_t first, uint64_t rows) {
    const uint64_t span_all = first + rows;
    for (uint64_t i = 0; i < rows * q_heads; ++i) softmax_row(p + i * span_all, first + i / q_heads + 1);
}

/* kernels.cuh:1095-1097 */
void oracle_attention_softmax_rows(float* p, uint64_t rows, uint64_t length) {
    for (uint64_t r = 0; r < rows; ++r) softmax_row(p + r * length, length);
}

/* kernels.cuh:1104-1110 */
void oracle_attention_softmax_lens(float* p, uint64_t p_row, const uint32_t* lens, uint64_t heads, uint64_t rows) {
    for (uint64_t b = 0; b < rows * heads; ++b) {
        const uint64_t u = b / heads, h = b - u * heads;
        softmax_row(p + u * p_row + h * lens[u], lens[u]);
    }
}

/* kernels.cuh:1169-1178 */
void oracle_attention_mix_rows(uint16_t* o, uint64_t o_row, const float* p, uint64_t p_row, const uint16_t* v,
                               uint64_t v_row, const uint32_t* lens, uint64_t q_heads, uint64_t kv_heads,
                               uint64_t head_dim, uint64_t rows, uint32_t* over) {
    const uint64_t group = q_heads / kv_heads, row = kv_heads * head_dim;
    for (uint64_t b = 0; b < rows * q_heads; ++b) {
        const uint64_t u = b / q_heads, h = b - u * q_heads, length = lens[u];
        mix_head(o + u * o_row + h * head_dim, p + u * p_row + h * length, v + u * v_row + (h / group) * head_dim, row,
                 head_dim, length, over);
    }
}

/* doors.cuh:417-424 — attention_weights a row at a time, row r over first + r + 1 positions. */
void oracle_attention_weights_rows(float* p, float* res, const uint16_t* q, const uint16_t* k, uint64_t q_heads,
                                   uint64_t kv_heads, uint64_t head_dim, uint64_t first, uint64_t rows) {
    const uint64_t span = first + rows, rf = head_dim + 2;
    for (uint64_t r = 0; r < rows; ++r)
        oracle_attention_weights(p + r * q_heads * span, res + r * q_heads * rf, q + r * q_heads * head_dim, k, q_heads,
                                 kv_heads, head_dim, first + r + 1);
}

/* doors.cuh:425-432 */
void oracle_attention_residual_mix_rows(float* res, const float* p, const uint16_t* v, uint64_t q_heads,
                                        uint64_t kv_heads, uint64_t head_dim, uint64_t first, uint64_t rows) {
    const uint64_t span = first + rows, rf = head_dim + 2;
    for (uint64_t r = 0; r < rows; ++r)
        oracle_attention_residual_mix(res + r * q_heads * rf, p + r * q_heads * span, v, q_heads, kv_heads, head_dim,
                                      first + r + 1);
}

/* ── TurboQuant rows: keys and values as d-bit codes with one fp16 scale a row ─────────────────────── */

/* kernels.cuh:2810-2817 — a container is 16 bits holding 16 / d codes; a row is whole containers. */
static uint64_t tq_per(uint64_t d) { return 16u / d; }
uint64_t oracle_tq_row_bytes(uint64_t d, uint64_t cols) {
    const uint64_t per = tq_per(d);
    return ((cols + per - 1u) / per) * 2u;
}

/* kernels.cuh:2957-2961 (+ level, 2650-2653) — element c of a row: its code's level times the row's scale.
 * `levels` is width d's table as fp16 bits (the test passes the reference's, read through its own door). */
static float tq_element(const uint8_t* row, float scale, uint64_t d, uint64_t c, const uint16_t* levels) {
    const uint64_t per = tq_per(d);
    const uint32_t unit = (uint32_t)row[(c / per) * 2u] | ((uint32_t)row[(c / per) * 2u + 1u] << 8);
    return scale * h2f(levels[(unit >> (uint32_t)(d * (c % per))) & ((1u << (uint32_t)d) - 1u)]);
}

/* kernels.cuh:2963-3000 — the first pass over TurboQuant keys (row t·kv_heads + g): scaled dots, then
 * e^(s - m) unnormalised into p and {m, l} into res. The body's word-at-a-time path takes the same products
 * in the same order, so the serial form is both. */
void oracle_attention_weights_tq(float* p, float* res, const uint16_t* q, const uint8_t* codes,
                                 const uint16_t* scales, uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim,
                                 uint64_t length, uint64_t d, const uint16_t* levels) {
    const uint64_t group = q_heads / kv_heads, row_bytes = oracle_tq_row_bytes(d, head_dim), w = head_dim + 2;
    const float inv = 1.0f / sqrtf((float)(uint32_t)head_dim);
    for (uint64_t h = 0; h < q_heads; ++h) {
        const uint16_t* qh = q + h * head_dim;
        const uint64_t g = h / group;
        float* ph = p + h * length;
        float top = -INFINITY;
        for (uint64_t t = 0; t < length; ++t) {
            const uint64_t r = t * kv_heads + g;
            const uint8_t* kr = codes + r * row_bytes;
            const float scale = h2f(scales[r]);
            float dot = 0.0f;
            for (uint64_t e = 0; e < head_dim; ++e) dot += h2f(qh[e]) * tq_element(kr, scale, d, e, levels);
            ph[t] = dot * inv;
            if (ph[t] > top) top = ph[t];
        }
        float part = 0.0f;
        for (uint64_t t = 0; t < length; ++t) {
            ph[t] = expf(ph[t] - top);
            part += ph[t];
        }
        res[h * w] = top;
        res[h * w + 1] = part;
    }
}

/* kernels.cuh:3005-3026 — its second pass: acc[e] = sum_t p[t] · value_t[e], the values TurboQuant rows. */
void oracle_attention_residual_mix_tq(float* res, const float* p, const uint8_t* codes, const uint16_t* scales,
                                      uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim, uint64_t length,
                                      uint64_t d, const uint16_t* levels) {
    const uint64_t group = q_heads / kv_heads, row_bytes = oracle_tq_row_bytes(d, head_dim), w = head_dim + 2;
    for (uint64_t h = 0; h < q_heads; ++h) {
        const float* ph = p + h * length;
        const uint64_t g = h / group;
        float* acc = res + h * w + 2;
        for (uint64_t e = 0; e < head_dim; ++e) {
            float sum = 0.0f;
            for (uint64_t t = 0; t < length; ++t) {
                const uint64_t r = t * kv_heads + g;
                sum += ph[t] * tq_element(codes + r * row_bytes, h2f(scales[r]), d, e, levels);
            }
            acc[e] = sum;
        }
    }
}

/* doors.cuh:433-441 — weights_tq a row at a time: row r's queries at q + r·q_heads·head_dim, all over the same
 * `length` keys, its weights at p + r·q_heads·length, its residuals at res + r·q_heads·(head_dim + 2). */
void oracle_attention_weights_tq_rows(float* p, float* res, const uint16_t* q, const uint8_t* codes,
                                      const uint16_t* scales, uint64_t q_heads, uint64_t kv_heads,
                                      uint64_t head_dim, uint64_t length, uint64_t d, uint64_t rows,
                                      const uint16_t* levels) {
    for (uint64_t r = 0; r < rows; ++r)
        oracle_attention_weights_tq(p + r * q_heads * length, res + r * q_heads * (head_dim + 2),
                                    q + r * q_heads * head_dim, codes, scales, q_heads, kv_heads, head_dim, length, d,
                                    levels);
}

/* doors.cuh:442-450 */
void oracle_attention_residual_mix_tq_rows(float* res, const float* p, const uint8_t* codes, const uint16_t* scales,
                                           uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim, uint64_t length,
                                           uint64_t d, uint64_t rows, const uint16_t* levels) {
    for (uint64_t r = 0; r < rows; ++r)
        oracle_attention_residual_mix_tq(res + r * q_heads * (head_dim + 2), p + r * q_heads * length, codes, scales,
                                         q_heads, kv_heads, head_dim, length, d, levels);
}

/* ── paged forms (the reference has none: its answer over the gathered-contiguous cache) ───────────── */

/* Positions [0, length) of a paged plane gathered into `out` as [position][kv_heads][head_dim]. */
void oracle_gather_pages(uint16_t* out, const uint16_t* pool, const uint32_t* pages, uint64_t page_size,
                         uint64_t row, uint64_t length) {
    for (uint64_t t = 0; t < length; ++t) {
        const uint64_t phys = (uint64_t)pages[t / page_size] * page_size + t % page_size;
        memcpy(out + t * row, pool + phys * row, row * sizeof(uint16_t));
    }
}

/* The reference's decode verb (attention__abi.cuh:129-160: attention_scores then attention_mix) for each row
 * over its gathered cache. `pages` NULL: row u's cache at k + u·k_row. lens[u] == 0 answers zeros. */
void oracle_attention_decode_paged(uint16_t* o, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                   const uint32_t* pages, uint64_t pages_row, uint64_t page_size, uint64_t k_row,
                                   const uint32_t* lens, uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim,
                                   uint64_t rows, uint32_t* over) {
    const uint64_t row = kv_heads * head_dim;
    for (uint64_t u = 0; u < rows; ++u) {
        const uint64_t len = lens[u];
        uint16_t* ou = o + u * q_heads * head_dim;
        if (len == 0) { memset(ou, 0, q_heads * head_dim * sizeof(uint16_t)); continue; }
        const uint16_t* ku = k + u * k_row;
        const uint16_t* vu = v + u * k_row;
        uint16_t *kg = 0, *vg = 0;
        if (pages) {
            kg = (uint16_t*)malloc(len * row * sizeof(uint16_t));
            vg = (uint16_t*)malloc(len * row * sizeof(uint16_t));
            oracle_gather_pages(kg, k, pages + u * pages_row, page_size, row, len);
            oracle_gather_pages(vg, v, pages + u * pages_row, page_size, row, len);
            ku = kg; vu = vg;
        }
        float* p = (float*)malloc(q_heads * len * sizeof(float));
        oracle_attention_scores(p, q + u * q_heads * head_dim, ku, q_heads, kv_heads, head_dim, len);
        oracle_attention_mix(ou, p, vu, q_heads, kv_heads, head_dim, len, over);
        free(p); free(kg); free(vg);
    }
}

/* Causal prefill restricted to the rows listed in `which` (count of them): row r of the chunk is the
 * reference's decode at position first + r over positions 0 .. first + r (attention__abi.cuh:336-342, the
 * causal rows are the one-position program's), so a subset of rows costs only those rows. Output row i is
 * chunk row which[i]. `pages` NULL for a contiguous cache. */
void oracle_attention_causal_rows(uint16_t* o, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                  const uint32_t* pages, uint64_t page_size, uint64_t q_heads, uint64_t kv_heads,
                                  uint64_t head_dim, uint64_t first, const uint32_t* which, uint64_t count,
                                  uint32_t* over) {
    const uint64_t row = kv_heads * head_dim;
    uint64_t most = 0;
    for (uint64_t i = 0; i < count; ++i) if (which[i] + 1 > most) most = which[i] + 1;
    const uint64_t len_all = first + most;
    const uint16_t* kk = k;
    const uint16_t* vv = v;
    uint16_t *kg = 0, *vg = 0;
    if (pages) {
        kg = (uint16_t*)malloc(len_all * row * sizeof(uint16_t));
        vg = (uint16_t*)malloc(len_all * row * sizeof(uint16_t));
        oracle_gather_pages(kg, k, pages, page_size, row, len_all);
        oracle_gather_pages(vg, v, pages, page_size, row, len_all);
        kk = kg; vv = vg;
    }
    float* p = (float*)malloc(q_heads * len_all * sizeof(float));
    for (uint64_t i = 0; i < count; ++i) {
        const uint64_t r = which[i], len = first + r + 1;
        oracle_attention_scores(p, q + r * q_heads * head_dim, kk, q_heads, kv_heads, head_dim, len);
        oracle_attention_mix(o + i * q_heads * head_dim, p, vv, q_heads, kv_heads, head_dim, len, over);
    }
    free(p); free(kg); free(vg);
}

/* kernels.cuh:1115-1131 — each of `rows` rows of `length` weights (row r at p + r·length) its softmax with a sink:
 * the top over sink[r] and the row, e^(x - top), normalised by their sum plus e^(sink[r] - top). */
void oracle_attention_softmax_sink(float* p, const uint16_t* sink, uint64_t rows, uint64_t length) {
    for (uint64_t r = 0; r < rows; ++r) {
        float* ph = p + r * length;
        const float sk = h2f(sink[r]);
        float top = sk;
        for (uint64_t t = 0; t < length; ++t) if (ph[t] > top) top = ph[t];
        float part = 0.0f;
        for (uint64_t t = 0; t < length; ++t) {
            ph[t] = expf(ph[t] - top);
            part += ph[t];
        }
        const float inv = 1.0f / (part + expf(sk - top));
        for (uint64_t t = 0; t < length; ++t) ph[t] *= inv;
    }
}

/* kernels.cuh:1710-1726 (`rope_rows`) — each row's heads turned by that row's angles: row r's at cs + r·rot, the rot/2
 * cosines then the rot/2 sines; of every head (head_stride apart; rows row_stride apart) elements k and k + rot/2,
 * for k < rot/2, become a·c − b·s and b·c + a·s, rounded to fp16 (overflow to *over). o may be x.
 * The one place the oracle fuses: the reference family is C++ built without -ffp-contract=off, which GCC then
 * contracts into fma(a, c, −(b·s)) and fma(b, c, a·s) — found by testing every form against its rope_rows door,
 * and held to it bit for bit by tests/test_cache.py (the unfused sums differ in the last bit now and then). */
void oracle_rope_rows(uint16_t* o, const uint16_t* x, const float* cs, uint64_t rows, uint64_t heads,
                      uint64_t head_stride, uint64_t row_stride, uint64_t rot, uint32_t* over) {
    const uint64_t pairs = rot / 2u;
    for (uint64_t r = 0; r < rows; ++r)
        for (uint64_t e = 0; e < heads; ++e)
            for (uint64_t k = 0; k < pairs; ++k) {
                const uint64_t at = r * row_stride + e * head_stride + k;
                const float a = h2f(x[at]), b = h2f(x[at + pairs]);
                const float c = cs[r * rot + k], s = cs[r * rot + pairs + k];
                int hit = 0;
                o[at] = oracle_float_to_half(fmaf(a, c, -(b * s)), &hit);
                if (hit) *over = FAULT_OVERFLOW;
                hit = 0;
                o[at + pairs] = oracle_float_to_half(fmaf(b, c, a * s), &hit);
                if (hit) *over = FAULT_OVERFLOW;
            }
}

/* The page-aware cache writer (no reference counterpart: the reference's rows verb turns the chunk's keys with
 * rope_rows straight into the contiguous cache and places the values there, attention__abi.cuh:398-406). Row r of
 * k / v belongs to sequence u = r / rows_per_seq at position positions[u] + r % rows_per_seq; its slot is page
 * pages[u·pages_row + position / page_size] at offset position % page_size (pages NULL: u·capacity + position). The
 * key is copied there and its first rot elements turned in place by oracle_rope_rows with row r's angles (cs NULL:
 * not turned); the value is copied. A position at or past capacity writes nothing and stores "NPBN", which
 * outranks an overflow: NPOV goes into *over only when no row was out of bounds and *over was clear. */
void oracle_attention_cache_write_paged(uint16_t* kc, uint16_t* vc, const uint32_t* pages, uint64_t pages_row,
                                        uint64_t page_size, uint64_t capacity, const uint32_t* positions,
                                        uint64_t rows_per_seq, const uint16_t* k, const uint16_t* v, const float* cs,
                                        uint64_t rot, uint64_t rows, uint64_t kv_heads, uint64_t head_dim,
                                        uint32_t* over) {
    const uint64_t row = kv_heads * head_dim;
    uint32_t turned = 0;
    int out = 0;
    for (uint64_t r = 0; r < rows; ++r) {
        const uint64_t u = r / rows_per_seq, p = (uint64_t)positions[u] + r % rows_per_seq;
        if (p >= capacity) { out = 1; continue; }
        const uint64_t slot = pages ? (uint64_t)pages[u * pages_row + p / page_size] * page_size + p % page_size
                                    : u * capacity + p;
        memcpy(kc + slot * row, k + r * row, row * sizeof(uint16_t));
        memcpy(vc + slot * row, v + r * row, row * sizeof(uint16_t));
        if (cs && rot)
            oracle_rope_rows(kc + slot * row, kc + slot * row, cs + r * rot, 1u, kv_heads, head_dim, row, rot, &turned);
    }
    if (out) *over = 0x4E50424Eu;   /* "NPBN", contracts/objects/primitives.cuh:5 */
    else if (turned && *over == 0) *over = turned;
}
