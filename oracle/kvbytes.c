/*
 * kvbytes.c -- TEST INFRASTRUCTURE ONLY: the CPU oracle for kvpath's byte-level rules.
 *
 * Plain C restatements, bit-exact by construction, of:
 *   oracle_kv_append_bytes   write_kv (kelpie/kelpie-models/kelpie_models/kernels/ops/
 *                            paged_attention.py:44-54) for a same-dtype cache: each row's K and V
 *                            copied to slot_mapping[t] (flat slot = page * block + row).
 *   oracle_kv_gather         the gather in _attend (ops/paged_attention.py:172-177):
 *                            out[r, j] = K[table[r, j / block] * block + j % block].
 *   oracle_copy_blocks       page dst[i] <- page src[i] (no reference counterpart; the closed
 *                            form this library defines), with the fp8 scales.
 *   oracle_e4m3_encode/decode  OCP e4m3fn conversion, round to nearest even, written from the
 *                            format's definition (bias 7, 3 mantissa bits, max 448, subnormals
 *                            m * 2^-9, 0x7f NaN); pinned against torch's float8_e4m3fn cast.
 *   oracle_kv_append_fp8     the library's quantize-on-append rule (no reference counterpart):
 *                            per page a step touches and per (member, kv head), grouped by page
 *                            as a set of rows, with t = absmax(rows) / 448,
 *                              fresh = the step writes the page's row 0
 *                              s_old = fresh ? 0 : scale
 *                              s_new = t                    when s_old == 0
 *                                      s_old * 2^k          when t > s_old > 0, k >= 1 the
 *                                                           smallest with s_old * 2^k >= t
 *                                      s_old                otherwise
 *                              r_new = 1 / s_new (0 when s_new == 0, and when s_new == inf)
 *                              if k > 0: every row the step does not write becomes
 *                                e4m3(clamp(f32(q) * 2^-k, +-448)), exact unless it falls below
 *                                e4m3's normals (the clamp only turns a stale NaN byte into -448)
 *                              each written row becomes e4m3(clamp(x * r_new, +-448)), or 0
 *                                when r_new == 0 (a run of zeros, or one holding an inf);
 *                              scale = s_new.
 *                            A fresh page's largest element is stored exactly (it maps to 448);
 *                            a scale only ever grows by a power of two, so requantizing the rows
 *                            already in a page is an exponent shift and the e4m3 rounding does not
 *                            compound over a decode stream. One reciprocal per (page, member,
 *                            head), then a product per value (the form vLLM's scaled fp8
 *                            quantization uses).
 * Floating point here is IEEE binary32, one rounding per operation (built with
 * -ffp-contract=off, no fast-math). Strides are in elements; offsets are 64-bit.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

typedef struct ocache {
    uint8_t* base;
    int64_t num_pages, block, hkv, d;
    int64_t s_page, s_kv, s_row, s_head; /* elements */
    int32_t elem_size;
    float* scale; /* fp8 only: [pages, 2, hkv] */
} ocache;

static int64_t elem_offset(const ocache* c, int64_t page, int m, int64_t row, int64_t h) {
    return page * c->s_page + m * c->s_kv + row * c->s_row + h * c->s_head;
}

/* ---- e4m3fn ------------------------------------------------------------------------------- */

uint8_t oracle_e4m3_encode(float x) {
    const uint8_t sign = signbit(x) ? 0x80 : 0x00;
    float a = fabsf(x);
    if (isnan(a)) return sign | 0x7f;
    if (a > 448.0f) a = 448.0f; /* callers clamp first; saturate anyway */
    if (a < 0x1p-6f) {
        /* subnormal range: a = m * 2^-9, m in [0, 8]; m == 8 is the smallest normal 0x08 */
        return sign | (uint8_t)(int)rintf(a * 0x1p9f);
    }
    int e;
    const float f = frexpf(a, &e); /* a = f * 2^e, f in [0.5, 1) */
    int exp2 = e - 1;              /* a = (1 + frac) * 2^exp2 */
    int m = (int)rintf(ldexpf(f, 4)) - 8; /* 8 * (1 + frac), rounded to even, minus the 1 */
    if (m == 8) {
        exp2 += 1;
        m = 0;
    }
    return sign | (uint8_t)(((exp2 + 7) << 3) | m);
}

float oracle_e4m3_decode(uint8_t q) {
    const int e = (q >> 3) & 15, m = q & 7;
    float a;
    if (e == 15 && m == 7) return NAN;
    if (e == 0)
        a = ldexpf((float)m, -9);
    else
        a = ldexpf(1.0f + (float)m / 8.0f, e - 7);
    return (q & 0x80) ? -a : a;
}

void oracle_e4m3_encode_array(const float* x, uint8_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_e4m3_encode(x[i]);
}

void oracle_e4m3_decode_array(const uint8_t* q, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_e4m3_decode(q[i]);
}

static float clamp448(float x) { return fminf(fmaxf(x, -448.0f), 448.0f); }

/* x quantized against a page scale s through its reciprocal r = 1 / s (r == 0: s == 0). */
uint8_t oracle_fp8_quantize(float x, float r) {
    if (!(r > 0.0f)) return 0;
    return oracle_e4m3_encode(clamp448(x * r));
}

float oracle_fp8_reciprocal(float s) { return s > 0.0f ? 1.0f / s : 0.0f; }

/* The smallest k >= 1 with s_old * 2^k >= t (t > s_old > 0), by exact power-of-two products. */
int oracle_fp8_growth(float s_old, float t) {
    int k = 1;
    while (ldexpf(s_old, k) < t) ++k;
    return k;
}

/* ---- same-dtype append, gather, copy ------------------------------------------------------ */

void oracle_kv_append_bytes(ocache* c, const uint8_t* k, const uint8_t* v, int64_t k_srow,
                            int64_t k_shead, int64_t v_srow, int64_t v_shead,
                            const int32_t* slots, int64_t T) {
    const int64_t es = c->elem_size, pool = c->num_pages * c->block;
    for (int64_t t = 0; t < T; ++t) {
        const int64_t slot = slots[t];
        if (slot < 0 || slot >= pool) continue;
        const int64_t page = slot / c->block, row = slot % c->block;
        for (int m = 0; m < 2; ++m) {
            const uint8_t* src = m ? v : k;
            const int64_t srow = m ? v_srow : k_srow, shead = m ? v_shead : k_shead;
            for (int64_t h = 0; h < c->hkv; ++h)
                memcpy(c->base + elem_offset(c, page, m, row, h) * es,
                       src + (t * srow + h * shead) * es, (size_t)(c->d * es));
        }
    }
}

void oracle_kv_gather(const ocache* c, const int32_t* table, int64_t table_stride, int64_t R,
                      int64_t width, uint8_t* out_k, uint8_t* out_v) {
    const int64_t es = c->elem_size, cols = width * c->block, row_bytes = c->hkv * c->d * es;
    for (int64_t r = 0; r < R; ++r)
        for (int64_t j = 0; j < cols; ++j) {
            const int64_t page = table[r * table_stride + j / c->block];
            for (int m = 0; m < 2; ++m) {
                uint8_t* out = (m ? out_v : out_k) + (r * cols + j) * row_bytes;
                for (int64_t h = 0; h < c->hkv; ++h) {
                    uint8_t* dst = out + h * c->d * es;
                    if (page < 0 || page >= c->num_pages)
                        memset(dst, 0, (size_t)(c->d * es));
                    else
                        memcpy(dst, c->base + elem_offset(c, page, m, j % c->block, h) * es,
                               (size_t)(c->d * es));
                }
            }
        }
}

void oracle_copy_blocks(ocache* c, const int32_t* src, const int32_t* dst, int64_t n) {
    const int64_t es = c->elem_size;
    for (int64_t i = 0; i < n; ++i) {
        if (src[i] < 0 || src[i] >= c->num_pages || dst[i] < 0 || dst[i] >= c->num_pages) continue;
        for (int m = 0; m < 2; ++m)
            for (int64_t row = 0; row < c->block; ++row)
                for (int64_t h = 0; h < c->hkv; ++h)
                    memmove(c->base + elem_offset(c, dst[i], m, row, h) * es,
                            c->base + elem_offset(c, src[i], m, row, h) * es, (size_t)(c->d * es));
        if (c->scale)
            for (int64_t k = 0; k < 2 * c->hkv; ++k)
                c->scale[dst[i] * 2 * c->hkv + k] = c->scale[src[i] * 2 * c->hkv + k];
    }
}

/* ---- fp8 quantize-on-append ---------------------------------------------------------------- */

/* k, v: f32 [T, hkv, d] with the given strides (bf16 inputs widen exactly). Cache elem_size 1. */
void oracle_kv_append_fp8(ocache* c, const float* k, const float* v, int64_t k_srow,
                          int64_t k_shead, int64_t v_srow, int64_t v_shead, const int32_t* slots,
                          int64_t T, uint8_t* done /* scratch, T bytes */) {
    const int64_t pool = c->num_pages * c->block;
    memset(done, 0, (size_t)T);
    for (int64_t t0 = 0; t0 < T; ++t0) {
        if (done[t0] || slots[t0] < 0 || slots[t0] >= pool) continue;
        const int64_t page = slots[t0] / c->block;
        /* the set of this step's rows that land in `page` */
        uint8_t written[64];
        memset(written, 0, sizeof written);
        for (int64_t t = t0; t < T; ++t)
            if (slots[t] >= 0 && slots[t] < pool && slots[t] / c->block == page) {
                done[t] = 1;
                written[slots[t] % c->block] = 1;
            }
        const int fresh = written[0];
        for (int m = 0; m < 2; ++m) {
            const float* src = m ? v : k;
            const int64_t srow = m ? v_srow : k_srow, shead = m ? v_shead : k_shead;
            for (int64_t h = 0; h < c->hkv; ++h) {
                float amax = 0.0f;
                for (int64_t t = t0; t < T; ++t) {
                    if (slots[t] < 0 || slots[t] >= pool || slots[t] / c->block != page) continue;
                    for (int64_t d = 0; d < c->d; ++d)
                        amax = fmaxf(amax, fabsf(src[t * srow + h * shead + d]));
                }
                float* scale = c->scale + (page * 2 + m) * c->hkv + h;
                const float s_old = fresh ? 0.0f : *scale;
                const float t_new = amax / 448.0f;
                const int k = (s_old > 0.0f && t_new > s_old) ? oracle_fp8_growth(s_old, t_new) : 0;
                const float s_new = s_old > 0.0f ? ldexpf(s_old, k) : t_new;
                const float r_new = oracle_fp8_reciprocal(s_new);
                if (k > 0) {
                    for (int64_t row = 0; row < c->block; ++row) {
                        if (written[row]) continue;
                        uint8_t* q = c->base + elem_offset(c, page, m, row, h);
                        for (int64_t d = 0; d < c->d; ++d)
                            q[d] = oracle_e4m3_encode(clamp448(ldexpf(oracle_e4m3_decode(q[d]), -k)));
                    }
                }
                for (int64_t t = t0; t < T; ++t) {
                    if (slots[t] < 0 || slots[t] >= pool || slots[t] / c->block != page) continue;
                    uint8_t* q = c->base + elem_offset(c, page, m, slots[t] % c->block, h);
                    for (int64_t d = 0; d < c->d; ++d)
                        q[d] = oracle_fp8_quantize(src[t * srow + h * shead + d], r_new);
                }
                *scale = s_new;
            }
        }
    }
}
