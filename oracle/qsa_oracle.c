/*
 * qsa_oracle.c -- CPU restatement of the q8_0 KV cache + QSA decode path.
 * TEST INFRASTRUCTURE ONLY (see qsa_oracle.h): the checker for the HIP path
 * and the CPU baseline of bench.py.  Built with -ffp-contract=off.
 */
#include "qsa_oracle.h"

#include <math.h>
#ifdef __F16C__
#include <immintrin.h>
#endif
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* fp16                                                                      */
/* ------------------------------------------------------------------------ */

/* IEEE binary32 -> binary16, round to nearest even.  ggml stores the q8_0
 * scale with GGML_FP32_TO_FP16 (F16C _cvtss_sh with RNE on x86). */
uint16_t qwfn_oracle_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) {                       /* inf / nan */
        if (ax == 0x7F800000u) return sign | 0x7C00u;
        return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
    }
    const int32_t exp = (int32_t)(ax >> 23);       /* biased, 0 = subnormal */
    const uint32_t mant = ax & 0x7FFFFFu;
    const int32_t e16 = exp - 127 + 15;
    if (e16 >= 31) return sign | 0x7C00u;          /* >= 2^16: overflow */
    if (e16 >= 1) {                                /* normal half */
        uint32_t h = ((uint32_t)e16 << 10) | (mant >> 13);
        const uint32_t rem = mant & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u; /* may carry to inf */
        return (uint16_t)(sign | h);
    }
    if (exp == 0) return sign;                     /* f32 subnormal < 2^-126 */
    /* subnormal half: value / 2^-24 = mf * 2^(exp-126) */
    const uint32_t mf = mant | 0x800000u;
    const int32_t sh = 126 - exp;                  /* >= 14 */
    if (sh >= 25) return sign;                     /* < half of 2^-24 */
    uint32_t h = mf >> sh;
    const uint32_t rem = mf & ((1u << sh) - 1u);
    const uint32_t half = 1u << (sh - 1);
    if (rem > half || (rem == half && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

float qwfn_oracle_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = ((uint32_t)h >> 10) & 0x1Fu;
    const uint32_t m = (uint32_t)h & 0x3FFu;
    uint32_t x;
    if (e == 0x1Fu) {
        x = sign | 0x7F800000u | (m << 13);
    } else if (e != 0) {
        x = sign | ((e - 15u + 127u) << 23) | (m << 13);
    } else if (m == 0) {
        x = sign;
    } else {                                       /* subnormal half: m * 2^-24 */
        const float v = (float)m * 5.9604644775390625e-08f;   /* exact */
        memcpy(&x, &v, 4);
        x |= sign;
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void qwfn_oracle_f32_to_f16_n(const float *x, int64_t n, uint16_t *out) {
    for (int64_t i = 0; i < n; i++) out[i] = qwfn_oracle_f32_to_f16(x[i]);
}

/* ------------------------------------------------------------------------ */
/* q8_0                                                                      */
/* ------------------------------------------------------------------------ */

static int8_t to_i8(float r) {
    if (r != r) return 0;                          /* documented: NaN -> 0 */
    if (r > 127.0f) return 127;
    if (r < -128.0f) return -128;
    return (int8_t)r;
}

/* ggml's q8_0 quantizer, restated from its published algorithm: amax over the
 * 32 values, d = amax/127 stored as fp16, then either the x86 SIMD form
 * (id = 127/amax, round half even) or the reference/CUDA form (id = 1/d,
 * roundf).  Reached by ggml_set_rows / ggml_cpy into the q8_0 cache
 * (/root/reference src/qwfn_graph.cpp:525-526, 353-360). */
void qwfn_oracle_quantize_block(const float *x, int32_t variant, uint16_t *dout,
                                int8_t *qs) {
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) {
        const float a = fabsf(x[j]);
        if (a > amax) amax = a;                    /* NaN never wins */
    }
    const float d = amax / 127.0f;
    *dout = qwfn_oracle_f32_to_f16(d);
    float id;
    if (variant == QWFN_Q8_X86_RNE)
        id = amax != 0.0f ? 127.0f / amax : 0.0f;
    else
        id = d != 0.0f ? 1.0f / d : 0.0f;
    for (int j = 0; j < 32; j++) {
        const float v = x[j] * id;
        const float r = (variant == QWFN_Q8_X86_RNE) ? rintf(v) : roundf(v);
        qs[j] = to_i8(r);
    }
}

void qwfn_oracle_quantize_row_ggml(const float *x, int64_t n, int32_t variant,
                                   uint8_t *out) {
    for (int64_t b = 0; b < n / 32; b++) {
        uint16_t d;
        qwfn_oracle_quantize_block(x + 32 * b, variant, &d, (int8_t *)(out + 34 * b + 2));
        memcpy(out + 34 * b, &d, 2);
    }
}

/* ggml's q4_0 quantizer (quantize_row_q4_0_ref), restated from its published
 * algorithm: m = the element of largest magnitude (the first one; it starts at
 * +0 and only a strictly larger |x| replaces it, so NaN never wins), d = m / -8
 * stored as fp16, id = 1/d (0 when d == 0), q = min(15, (int8)(x*id + 8.5)),
 * qs[j] = q[j] | q[j+16] << 4.  A NaN x*id + 8.5 stores 0 (x86's truncating
 * conversion gives INT_MIN, whose low byte is 0).  Reached through the
 * reference's --kv q4_0 (tools/qwfn_gen.cpp:55-57). */
void qwfn_oracle_quantize_block_q4_0(const float *x, uint16_t *dout, uint8_t *qs) {
    float amax = 0.0f, m = 0.0f;
    for (int j = 0; j < 32; j++) {
        const float a = fabsf(x[j]);
        if (amax < a) { amax = a; m = x[j]; }
    }
    const float d = m / -8.0f;
    *dout = qwfn_oracle_f32_to_f16(d);
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint8_t q[32];
    for (int j = 0; j < 32; j++) {
        const float r = x[j] * id + 8.5f;
        const int t = r != r ? 0 : (int)r;
        q[j] = (uint8_t)(t < 15 ? t : 15);
    }
    for (int j = 0; j < 16; j++) qs[j] = (uint8_t)(q[j] | (q[j + 16] << 4));
}

/* One row of n values in ggml's layout of the cache type: q8_0 34-byte blocks,
 * q4_0 18-byte blocks {fp16 d; qs[16]}, or fp16 values. */
void qwfn_oracle_quantize_row_type(const float *x, int64_t n, int32_t kv_type, int32_t variant,
                                   uint8_t *out) {
    if (kv_type == QWFN_KV_F16) {
        for (int64_t i = 0; i < n; i++) {
            const uint16_t h = qwfn_oracle_f32_to_f16(x[i]);
            memcpy(out + 2 * i, &h, 2);
        }
    } else if (kv_type == QWFN_KV_Q4_0) {
        for (int64_t b = 0; b < n / 32; b++) {
            uint16_t d;
            qwfn_oracle_quantize_block_q4_0(x + 32 * b, &d, out + 18 * b + 2);
            memcpy(out + 18 * b, &d, 2);
        }
    } else {
        qwfn_oracle_quantize_row_ggml(x, n, variant, out);
    }
}

/* ------------------------------------------------------------------------ */
/* layout                                                                    */
/* ------------------------------------------------------------------------ */

/* Bytes of a head row of K (or V) in a page: q8_0 one per value, q4_0 a
 * nibble, fp16 two. */
static int64_t row_bytes(const qwfn_qsa_shape *s) {
    return s->kv_type == QWFN_KV_Q4_0 ? s->head_dim / 2 : s->kv_type == QWFN_KV_F16 ? 2 * s->head_dim
                                                                                    : s->head_dim;
}

static size_t quant_bytes_per_page(const qwfn_qsa_shape *s) {
    return (size_t)s->n_head_kv * (size_t)s->page_tokens * (size_t)row_bytes(s);
}

size_t qwfn_oracle_page_bytes(const qwfn_qsa_shape *s) {
    if (s->kv_type == QWFN_KV_F16) return quant_bytes_per_page(s);
    return quant_bytes_per_page(s) +
           (size_t)s->n_head_kv * (size_t)s->page_tokens * (size_t)(s->head_dim / 32) * 2u;
}

/* Byte offset of value d of head g's row in a page (for q4_0: the byte whose
 * low (d%32 < 16) or high nibble holds it; for fp16: its first byte). */
int64_t qwfn_oracle_quant_offset(const qwfn_qsa_shape *s, int32_t which, int32_t g,
                                 int32_t row, int32_t d) {
    const int64_t tiles = s->page_tokens / 64, chunks = row_bytes(s) / 16;
    const int64_t tile_row = ((int64_t)g * tiles + row / 64);
    if (s->kv_type == QWFN_KV_Q4_0)                /* chunk = ggml block d/32's qs bytes */
        return (tile_row * chunks + d / 32) * 1024 + (int64_t)(row % 64) * 16 + d % 16;
    if (s->kv_type == QWFN_KV_F16)                 /* chunk = dims 8c .. 8c+7 */
        return (tile_row * chunks + d / 8) * 1024 + (int64_t)(row % 64) * 16 + (d % 8) * 2;
    if (which && s->block_tokens % 64 == 0)       /* q8_0 V, dim-major 64-token tiles */
        return (tile_row * s->head_dim + d) * 64 + row % 64;
    return (tile_row * chunks + d / 16) * 1024 + (int64_t)(row % 64) * 16 + d % 16;
}

int64_t qwfn_oracle_scale_offset(const qwfn_qsa_shape *s, int32_t g, int32_t row,
                                 int32_t j) {
    return (int64_t)quant_bytes_per_page(s) +
           (((int64_t)g * s->page_tokens + row) * (s->head_dim / 32) + j) * 2;
}

/* Physical page base for (seq, t), or NULL with *status bits set. */
static uint8_t *page_of(const qwfn_qsa_shape *s, const qwfn_kv_view *v, const void *pool,
                        int32_t seq, int32_t t, int32_t *status) {
    if (seq < 0 || seq >= v->n_seq) { *status |= QWFN_STATUS_SEQ_RANGE; return NULL; }
    if (t < 0 || (int64_t)t >= (int64_t)v->pages_per_seq * s->page_tokens) {
        *status |= QWFN_STATUS_POS_RANGE; return NULL;
    }
    const int32_t phys = v->page_table[(int64_t)seq * v->pages_per_seq + t / s->page_tokens];
    if (phys < 0 || phys >= v->n_phys_pages) { *status |= QWFN_STATUS_PAGE_RANGE; return NULL; }
    return (uint8_t *)pool + (size_t)phys * qwfn_oracle_page_bytes(s);
}

static float src_at(const void *src, int32_t dtype, int64_t i) {
    if (dtype == QWFN_SRC_F16) return qwfn_oracle_f16_to_f32(((const uint16_t *)src)[i]);
    return ((const float *)src)[i];
}

/* Decode append (src/qwfn_graph.cpp:520-528) and prefill chunk append
 * (src/qwfn_graph.cpp:349-360): quantize each [n_head_kv][head_dim] row and
 * overwrite it at its position.  Returns status bits (0 = every row written). */
int qwfn_oracle_append(const qwfn_qsa_shape *s, const qwfn_kv_view *v,
                       const void *k_src, const void *v_src, int32_t src_dtype,
                       const int32_t *seq_ids, const int32_t *pos, int32_t n_rows) {
    const int32_t H = s->n_head_kv, hd = s->head_dim;
    int32_t status = 0;
    float x[32];
    for (int32_t i = 0; i < n_rows; i++) {
        const int32_t seq = seq_ids ? seq_ids[i] : 0, t = pos[i];
        for (int which = 0; which < 2; which++) {
            const void *src = which ? v_src : k_src;
            uint8_t *page = page_of(s, v, which ? v->v_pages : v->k_pages, seq, t, &status);
            if (!page) continue;
            const int32_t row = t % s->page_tokens;
            for (int32_t g = 0; g < H; g++)
                for (int32_t j = 0; j < hd / 32; j++) {
                    for (int e = 0; e < 32; e++)
                        x[e] = src_at(src, src_dtype, ((int64_t)i * H + g) * hd + 32 * j + e);
                    uint16_t d;
                    if (s->kv_type == QWFN_KV_F16) {
                        for (int e = 0; e < 32; e++) {
                            d = qwfn_oracle_f32_to_f16(x[e]);
                            memcpy(page + qwfn_oracle_quant_offset(s, which, g, row, 32 * j + e), &d, 2);
                        }
                    } else if (s->kv_type == QWFN_KV_Q4_0) {
                        uint8_t qs[16];
                        qwfn_oracle_quantize_block_q4_0(x, &d, qs);
                        memcpy(page + qwfn_oracle_scale_offset(s, g, row, j), &d, 2);
                        for (int e = 0; e < 16; e++) page[qwfn_oracle_quant_offset(s, which, g, row, 32 * j + e)] = qs[e];
                    } else {
                        int8_t qs[32];
                        qwfn_oracle_quantize_block(x, s->quant_variant, &d, qs);
                        memcpy(page + qwfn_oracle_scale_offset(s, g, row, j), &d, 2);
                        for (int e = 0; e < 32; e++)
                            page[qwfn_oracle_quant_offset(s, which, g, row, 32 * j + e)] = (uint8_t)qs[e];
                    }
                }
        }
    }
    return status;
}

/* ggml_get_rows of q8_0 -> f32 (src/qwfn_graph.cpp:531): x = fp32(d) * q, exact. */
int qwfn_oracle_dequant_row(const qwfn_qsa_shape *s, const qwfn_kv_view *v,
                            const void *pool, int32_t seq, int32_t t, int32_t g,
                            float *out) {
    int32_t status = 0;
    const uint8_t *page = page_of(s, v, pool, seq, t, &status);
    if (!page) return status;
    const int32_t row = t % s->page_tokens;
    const int32_t which = pool == v->v_pages;
    for (int32_t d = 0; d < s->head_dim; d++) {
        uint16_t h;
        const int64_t off = qwfn_oracle_quant_offset(s, which, g, row, d);
        if (s->kv_type == QWFN_KV_F16) {           /* ggml_get_rows of F16: the value itself */
            memcpy(&h, page + off, 2);
            out[d] = qwfn_oracle_f16_to_f32(h);
            continue;
        }
        memcpy(&h, page + qwfn_oracle_scale_offset(s, g, row, d / 32), 2);
        if (s->kv_type == QWFN_KV_Q4_0) {           /* dequantize_row_q4_0: (nibble - 8) * d */
            const uint8_t b = page[off];
            const int q = (d % 32 < 16 ? (b & 15) : (b >> 4)) - 8;
            out[d] = (float)q * qwfn_oracle_f16_to_f32(h);
            continue;
        }
        const int8_t q = (int8_t)page[off];
        out[d] = qwfn_oracle_f16_to_f32(h) * (float)q;
    }
    return 0;
}

static int64_t blocks_per_seq(const qwfn_qsa_shape *s, const qwfn_kv_view *v) {
    return (int64_t)v->pages_per_seq * s->page_tokens / s->block_tokens;
}

/* Mean of a block's member keys: qsa_pool_blocks' sequential ggml_add chain over
 * the r member slices, then ggml_scale(1/r) (src/qwfn_graph.cpp:415-422), with
 * the members read from the dequantized K cache (the configuration pools K
 * itself; no norm or rope follows). */
int qwfn_oracle_pool_block(const qwfn_qsa_shape *s, const qwfn_kv_view *v,
                           int32_t seq, int32_t b) {
    const int32_t hd = s->head_dim, bt = s->block_tokens;
    if (seq < 0 || seq >= v->n_seq) return QWFN_STATUS_SEQ_RANGE;
    if (b < 0 || b >= blocks_per_seq(s, v)) return QWFN_STATUS_BLOCK_RANGE;
    float *acc = (float *)malloc(sizeof(float) * 2 * hd), *row = acc + hd;
    int32_t status = 0;
    for (int32_t g = 0; g < s->n_head_kv; g++) {
        status |= qwfn_oracle_dequant_row(s, v, v->k_pages, seq, b * bt, g, acc);
        for (int32_t t = 1; t < bt; t++) {
            status |= qwfn_oracle_dequant_row(s, v, v->k_pages, seq, b * bt + t, g, row);
            for (int32_t d = 0; d < hd; d++) acc[d] = acc[d] + row[d];
        }
        if (status) break;
        const float inv = 1.0f / (float)bt;
        float *dst = v->pooled + (((int64_t)seq * s->n_head_kv + g) * blocks_per_seq(s, v) + b) * hd;
        for (int32_t d = 0; d < hd; d++) dst[d] = acc[d] * inv;
    }
    free(acc);
    return status;
}

/* ------------------------------------------------------------------------ */
/* indexer + selection                                                       */
/* ------------------------------------------------------------------------ */

/* Score of one block for one KV head: for each head h of the group, the dot
 * q_h . p as four fmaf chains (chain j takes the dims d with (d/4)%4 == j, in
 * increasing d) combined as (c0+c1)+(c2+c3); optionally relu'd; then the heads
 * summed in order.  This is the score of src/qwfn_graph.cpp:485-492 (mul_mat,
 * relu, sum_rows over heads) at the configuration's shapes, in the fixed order
 * the HIP indexer evaluates (four lanes share one dot). */
float qwfn_oracle_block_score(const qwfn_qsa_shape *s, const float *q_group,
                              const float *p) {
    const int32_t hd = s->head_dim, G = s->n_head / s->n_head_kv;
    float score = 0.0f;
    for (int32_t h = 0; h < G; h++) {
        const float *q = q_group + (int64_t)h * hd;
        float c[4];
        for (int j = 0; j < 4; j++) {
            float acc = 0.0f;
            for (int32_t i = 0; i < hd / 16; i++)
                for (int e = 0; e < 4; e++) {
                    const int32_t d = 16 * i + 4 * j + e;
                    acc = fmaf(q[d], p[d], acc);
                }
            c[j] = acc;
        }
        float dot = (c[0] + c[1]) + (c[2] + c[3]);
        if (s->relu_per_head) dot = dot > 0.0f ? dot : 0.0f;
        score = (h == 0) ? dot : score + dot;
    }
    return score;
}

/* Forced and eligible ranges of one (sequence, KV head) at length seq_len.
 * The reference forces the incomplete tail block with a +1e9 bias and leaves
 * whole blocks at 0 (src/qwfn_engine.cpp:748-753, decode; :936-950, prefill);
 * the configuration generalises the forced set to the sink blocks plus every
 * block meeting the last local_tokens tokens.  Eligible = whole blocks in
 * [sink_blocks, first_window_block). */
static void qsa_ranges(const qwfn_qsa_shape *s, int32_t seq_len, int32_t *b_last,
                       int32_t *fw, int32_t *e_lo, int32_t *e_hi) {
    const int32_t bt = s->block_tokens, last = seq_len - 1;
    const int32_t w0 = last - s->local_tokens + 1;
    *b_last = last / bt;
    *fw = w0 > 0 ? w0 / bt : 0;
    const int32_t nbw = seq_len / bt;
    *e_lo = s->sink_blocks;
    *e_hi = nbw < *fw ? nbw : *fw;
    if (*e_hi < *e_lo) *e_hi = *e_lo;
}

/* Eligible blocks kept at this length: top_k_blocks, less the forced ones
 * (sink + window) when topk_counts_forced says the count includes them. */
static int32_t eff_topk(const qwfn_qsa_shape *s, int32_t seq_len) {
    int32_t b_last, fw, e_lo, e_hi;
    qsa_ranges(s, seq_len, &b_last, &fw, &e_lo, &e_hi);
    if (!s->topk_counts_forced) return s->top_k_blocks;
    const int32_t k = s->top_k_blocks - s->sink_blocks - (b_last - fw + 1);
    return k > 0 ? k : 0;
}

static uint32_t score_key(float x) {
    uint32_t u;
    if (x != x) return 0u;                         /* NaN ranks lowest */
    if (x == 0.0f) x = 0.0f;                       /* -0 ties +0 */
    memcpy(&u, &x, 4);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

typedef struct { uint32_t key; int32_t b; } cand_t;

static int cand_cmp(const void *a, const void *b) {
    const cand_t *x = (const cand_t *)a, *y = (const cand_t *)b;
    if (x->key != y->key) return x->key > y->key ? -1 : 1;   /* score desc */
    return x->b < y->b ? -1 : (x->b > y->b);                 /* index asc  */
}

static int int_cmp(const void *a, const void *b) {
    const int32_t x = *(const int32_t *)a, y = *(const int32_t *)b;
    return x < y ? -1 : (x > y);
}

int32_t qwfn_oracle_max_selected(const qwfn_qsa_shape *s, int32_t max_seq_len) {
    const int32_t bt = s->block_tokens;
    const int32_t all = (max_seq_len + bt - 1) / bt;
    if (s->top_k_blocks <= 0) return all;
    const int32_t win = (s->local_tokens + bt - 2) / bt + 1;
    const int64_t cap = (int64_t)s->top_k_blocks + s->sink_blocks + win;
    return cap < all ? (int32_t)cap : all;
}

/* ggml_top_k over the biased scores (src/qwfn_graph.cpp:493) with the tie rule
 * the build fixes (score desc, then lower block index), the forced blocks
 * added, emitted ascending. */
int32_t qwfn_oracle_select(const qwfn_qsa_shape *s, const float *scores,
                           int32_t seq_len, int32_t *sel, int32_t max_sel) {
    if (seq_len < 1) return QWFN_EINVAL;
    int32_t b_last, fw, e_lo, e_hi, n = 0;
    qsa_ranges(s, seq_len, &b_last, &fw, &e_lo, &e_hi);
    if (s->top_k_blocks <= 0) {
        if (b_last + 1 > max_sel) return QWFN_ERANGE;
        for (int32_t b = 0; b <= b_last; b++) sel[n++] = b;
        return n;
    }
    /* forced */
    int32_t *out = (int32_t *)malloc(sizeof(int32_t) * (size_t)(b_last + 1));
    for (int32_t b = 0; b <= b_last; b++)
        if (b < s->sink_blocks || b >= fw) out[n++] = b;
    const int32_t ne = e_hi - e_lo, k = eff_topk(s, seq_len);
    if (ne <= k) {
        for (int32_t b = e_lo; b < e_hi; b++) out[n++] = b;
    } else {
        cand_t *c = (cand_t *)malloc(sizeof(cand_t) * (size_t)ne);
        for (int32_t i = 0; i < ne; i++) { c[i].key = score_key(scores[e_lo + i]); c[i].b = e_lo + i; }
        qsort(c, (size_t)ne, sizeof(cand_t), cand_cmp);
        for (int32_t i = 0; i < k; i++) out[n++] = c[i].b;
        free(c);
    }
    qsort(out, (size_t)n, sizeof(int32_t), int_cmp);
    int32_t rc = n;
    if (n > max_sel) rc = QWFN_ERANGE;
    else memcpy(sel, out, sizeof(int32_t) * (size_t)n);
    free(out);
    return rc;
}

int qwfn_oracle_indexer_topk(const qwfn_qsa_shape *s, const qwfn_kv_view *v,
                             const float *q, const int32_t *seq_len, int32_t n_seq,
                             int32_t *sel, int32_t *n_sel, int32_t max_sel) {
    const int32_t H = s->n_head_kv, hd = s->head_dim, G = s->n_head / H;
    const int64_t bps = blocks_per_seq(s, v);
    int32_t status = 0;
    float *scores = (float *)malloc(sizeof(float) * (size_t)(bps > 0 ? bps : 1));
    float *sum = (float *)malloc(sizeof(float) * (size_t)(bps > 0 ? bps : 1));
    for (int32_t seq = 0; seq < n_seq; seq++) {
        const int32_t L = seq_len[seq];
        for (int32_t g = 0; g < H; g++) {
            int32_t *ns = n_sel + (int64_t)seq * H + g;
            *ns = 0;
            if (L < 1 || (int64_t)L > (int64_t)v->pages_per_seq * s->page_tokens) {
                status |= QWFN_STATUS_LEN_RANGE;
                continue;
            }
            int32_t b_last, fw, e_lo, e_hi;
            qsa_ranges(s, L, &b_last, &fw, &e_lo, &e_hi);
            if (s->top_k_blocks > 0 && e_hi - e_lo > eff_topk(s, L)) {
                const float *qg = q + ((int64_t)seq * s->n_head + (int64_t)g * G) * hd;
                const float *pb = v->pooled + ((int64_t)seq * H + g) * bps * hd;
                for (int32_t b = e_lo; b < e_hi; b++)
                    scores[b] = qwfn_oracle_block_score(s, qg, pb + (int64_t)b * hd);
                /* shared selection: the heads' scores summed in head order */
                if (s->shared_selection)
                    for (int32_t b = e_lo; b < e_hi; b++) sum[b] = g == 0 ? scores[b] : sum[b] + scores[b];
            }
            if (s->shared_selection && g < H - 1) continue;   /* select once, after the last head */
            const int32_t r = qwfn_oracle_select(s, s->shared_selection ? sum : scores, L,
                                                 sel + ((int64_t)seq * H + g) * max_sel, max_sel);
            if (r < 0) { free(scores); free(sum); return r; }
            *ns = r;
            if (s->shared_selection)                          /* the same selection for every head */
                for (int32_t h = 0; h < H - 1; h++) {
                    memcpy(sel + ((int64_t)seq * H + h) * max_sel, sel + ((int64_t)seq * H + g) * max_sel,
                           sizeof(int32_t) * (size_t)r);
                    n_sel[(int64_t)seq * H + h] = r;
                }
        }
    }
    free(scores);
    free(sum);
    return status;
}

/* ------------------------------------------------------------------------ */
/* attention                                                                 */
/* ------------------------------------------------------------------------ */

/* ggml_flash_attn_ext (prec F32, scale 1/sqrt(hd), no bias or softcap) over the
 * selected cells with the cell mask cell <= n_past (src/qwfn_graph.cpp:
 * 497-502, 539-541), restated as the textbook softmax in fp64 on the exactly
 * dequantized K/V.  GQA: query head h reads KV head h / (n_head/n_head_kv). */
static float f16_round(float x) { return qwfn_oracle_f16_to_f32(qwfn_oracle_f32_to_f16(x)); }

/* x[0..n) rounded to fp16 and back (round to nearest even, as
 * qwfn_oracle_f32_to_f16), eight at a time with F16C where the build has it. */
static void round_f16_row(float *x, int32_t n) {
    int32_t d = 0;
#ifdef __F16C__
    for (; d + 8 <= n; d += 8) {
        const __m256 a = _mm256_loadu_ps(x + d);
        _mm256_storeu_ps(x + d, _mm256_cvtph_ps(_mm256_cvtps_ph(a, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC)));
    }
#endif
    for (; d < n; d++) x[d] = f16_round(x[d]);
}

/* With kv_round_f16 every dequantized K and V value is rounded to fp16 first:
 * the reference's gather casts its rows to F16 before flash_attn_ext
 * (src/qwfn_graph.cpp:530-537). */
int qwfn_oracle_attention_f64(const qwfn_qsa_shape *s, const qwfn_kv_view *v,
                              const float *q, const int32_t *seq_len, int32_t n_seq,
                              const int32_t *sel, const int32_t *n_sel,
                              int32_t max_sel, double *out) {
    const int32_t H = s->n_head_kv, hd = s->head_dim, G = s->n_head / H, bt = s->block_tokens;
    int32_t status = 0;
    float *krow = (float *)malloc(sizeof(float) * 2 * hd), *vrow = krow + hd;
    for (int32_t seq = 0; seq < n_seq; seq++) {
        const int32_t L = seq_len[seq];
        for (int32_t g = 0; g < H; g++) {
            double *o = out + ((int64_t)seq * s->n_head + (int64_t)g * G) * hd;
            memset(o, 0, sizeof(double) * (size_t)G * hd);
            if (L < 1 || (int64_t)L > (int64_t)v->pages_per_seq * s->page_tokens) {
                status |= QWFN_STATUS_LEN_RANGE;
                continue;
            }
            const int32_t nb = sel ? n_sel[(int64_t)seq * H + g] : (L - 1) / bt + 1;
            int64_t nc = 0;
            int32_t *cells = (int32_t *)malloc(sizeof(int32_t) * (size_t)nb * bt + 1);
            for (int32_t i = 0; i < nb; i++) {
                const int32_t b = sel ? sel[((int64_t)seq * H + g) * max_sel + i] : i;
                for (int32_t t = b * bt; t < b * bt + bt && t < L; t++) cells[nc++] = t;
            }
            double *lg = (double *)malloc(sizeof(double) * (size_t)(nc * G + 1));
            const double scale = 1.0 / sqrt((double)hd);
            for (int64_t c = 0; c < nc; c++) {
                status |= qwfn_oracle_dequant_row(s, v, v->k_pages, seq, cells[c], g, krow);
                if (s->kv_round_f16) round_f16_row(krow, hd);
                for (int32_t h = 0; h < G; h++) {
                    const float *qh = q + ((int64_t)seq * s->n_head + (int64_t)g * G + h) * hd;
                    double acc = 0.0;
                    for (int32_t d = 0; d < hd; d++) acc += (double)qh[d] * (double)krow[d];
                    lg[c * G + h] = acc * scale;
                }
            }
            for (int32_t h = 0; h < G; h++) {
                double m = -INFINITY, l = 0.0;
                for (int64_t c = 0; c < nc; c++) if (lg[c * G + h] > m) m = lg[c * G + h];
                for (int64_t c = 0; c < nc; c++) {
                    const double p = exp(lg[c * G + h] - m);
                    lg[c * G + h] = p;
                    l += p;
                }
                for (int64_t c = 0; c < nc; c++) lg[c * G + h] /= l;
            }
            for (int64_t c = 0; c < nc; c++) {
                status |= qwfn_oracle_dequant_row(s, v, v->v_pages, seq, cells[c], g, vrow);
                if (s->kv_round_f16) round_f16_row(vrow, hd);
                for (int32_t h = 0; h < G; h++)
                    for (int32_t d = 0; d < hd; d++) o[(int64_t)h * hd + d] += lg[c * G + h] * (double)vrow[d];
            }
            free(lg);
            free(cells);
        }
    }
    free(krow);
    return status;
}

/* ------------------------------------------------------------------------ */
/* CPU baseline: the whole decode token in fp32                              */
/* Prefill of queries pos0 .. pos0+n_q-1 of sequence seq over a cache whose
 * rows and whole-block pooled keys are in place: query i is a decode step at
 * seq_len = pos0+i+1 without the append (its selection by
 * qwfn_oracle_indexer_topk, its attention by qwfn_oracle_attention_f64), the
 * per-query causal rule the reference's prefill builds with the bias of
 * src/qwfn_engine.cpp:936-950 and the mask of src/qwfn_graph.cpp:367-398.
 * sel [n_q][n_head_kv][max_sel], n_sel [n_q][n_head_kv], out [n_q][n_head][hd]
 * (doubles).  OpenMP over queries. */
int qwfn_oracle_prefill_f64(const qwfn_qsa_shape *s, const qwfn_kv_view *v, const float *q,
                            int32_t seq, int32_t pos0, int32_t n_q, int32_t *sel, int32_t *n_sel,
                            int32_t max_sel, double *out) {
    return qwfn_oracle_prefill_f64_strided(s, v, q, seq, pos0, n_q, 1, sel, n_sel, max_sel, out);
}

int qwfn_oracle_prefill_f64_strided(const qwfn_qsa_shape *s, const qwfn_kv_view *v, const float *q,
                                    int32_t seq, int32_t pos0, int32_t n_q, int32_t attn_stride,
                                    int32_t *sel, int32_t *n_sel, int32_t max_sel, double *out) {
    if (attn_stride < 1) return QWFN_EINVAL;
    if (seq < 0 || seq >= v->n_seq || pos0 < 0 || n_q < 1) return QWFN_EINVAL;
    if ((int64_t)pos0 + n_q > (int64_t)v->pages_per_seq * s->page_tokens) return QWFN_ERANGE;
    qwfn_qsa_shape s0 = *s;                        /* prefill reads the exact rows (kv_round_f16 is decode's) */
    s0.kv_round_f16 = 0;
    s = &s0;
    qwfn_kv_view sv = *v;                          /* the one sequence as a view */
    const int64_t bps = (int64_t)v->pages_per_seq * s->page_tokens / s->block_tokens;
    sv.pooled = v->pooled + (int64_t)seq * s->n_head_kv * bps * s->head_dim;
    sv.page_table = v->page_table + (int64_t)seq * v->pages_per_seq;
    sv.n_seq = 1;
    const int64_t qstride = (int64_t)s->n_head * s->head_dim;
    int rc_all = 0;
#pragma omp parallel for schedule(dynamic) reduction(min : rc_all)
    for (int32_t i = 0; i < n_q; ++i) {
        int32_t L = pos0 + i + 1;
        int32_t *si = sel + (int64_t)i * s->n_head_kv * max_sel;
        int32_t *ni = n_sel + (int64_t)i * s->n_head_kv;
        int rc = qwfn_oracle_indexer_topk(s, &sv, q + i * qstride, &L, 1, si, ni, max_sel);
        if (rc >= 0 && (i % attn_stride == 0 || i == n_q - 1))
            rc = qwfn_oracle_attention_f64(s, &sv, q + i * qstride, &L, 1, si, ni, max_sel, out + i * qstride);
        else if (rc >= 0)
            memset(out + i * qstride, 0, sizeof(double) * (size_t)qstride);
        if (rc < rc_all) rc_all = rc;
    }
    return rc_all < 0 ? rc_all : 0;
}

/* ------------------------------------------------------------------------ */

/* Token t of KV head g of one pool as the reference's attention sees it:
 * dequantized (ggml_get_rows of q8_0: each 32-value block's fp16 scale times
 * its quants) and cast to F16 (src/qwfn_graph.cpp:530-532).  q8_0 rows are
 * read straight from their page (K quants in 16-byte chunks 1024 bytes apart,
 * V quants dim-major 64 bytes apart); other types through
 * qwfn_oracle_dequant_row. */
static int32_t baseline_row(const qwfn_qsa_shape *s, const qwfn_kv_view *v, const void *pool, int32_t seq,
                            int32_t t, int32_t g, float *out) {
    const int32_t hd = s->head_dim;
    if (s->kv_type != QWFN_KV_Q8_0) {
        const int32_t rc = qwfn_oracle_dequant_row(s, v, pool, seq, t, g, out);
        if (!rc) round_f16_row(out, hd);
        return rc;
    }
    int32_t status = 0;
    const uint8_t *page = page_of(s, v, pool, seq, t, &status);
    if (!page) return status;
    const int32_t row = t % s->page_tokens, is_v = pool == v->v_pages;
    float scale[16];
    for (int32_t j = 0; j < hd / 32; j++) {
        uint16_t h;
        memcpy(&h, page + qwfn_oracle_scale_offset(s, g, row, j), 2);
        scale[j] = qwfn_oracle_f16_to_f32(h);
    }
    const int8_t *q0 = (const int8_t *)(page + qwfn_oracle_quant_offset(s, is_v, g, row, 0));
    if (is_v && s->block_tokens % 64 == 0)
        for (int32_t d = 0; d < hd; d++) out[d] = scale[d / 32] * (float)q0[(int64_t)d * 64];
    else
        for (int32_t d = 0; d < hd; d++) out[d] = scale[d / 32] * (float)q0[(d / 16) * 1024 + d % 16];
    round_f16_row(out, hd);
    return 0;
}

/* a . b over n (a multiple of 8) as eight interleaved partial sums. */
static float dot8(const float *a, const float *b, int32_t n) {
    float p[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    for (int32_t d = 0; d < n; d += 8)
        for (int j = 0; j < 8; j++) p[j] += a[d + j] * b[d + j];
    return ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
}

int qwfn_oracle_decode_step_f32(const qwfn_qsa_shape *s, const qwfn_kv_view *v,
                                const float *q, const float *k_new,
                                const float *v_new, const int32_t *seq_len,
                                int32_t n_seq, float *out, int32_t *sel,
                                int32_t *n_sel, int32_t max_sel) {
    const int32_t H = s->n_head_kv, hd = s->head_dim, G = s->n_head / H, bt = s->block_tokens;
    if (G > 16 || hd > 512 || hd % 32) return QWFN_EINVAL;      /* the per-task buffers below */
    const int64_t bps = blocks_per_seq(s, v);
    int threads = 1;
#ifdef _OPENMP
    threads = omp_get_max_threads();
#endif
    /* append + pool on completion (src/qwfn_graph.cpp:465-476, 520-528) */
    for (int32_t seq = 0; seq < n_seq; seq++) {
        const int32_t p = seq_len[seq] - 1;
        if (qwfn_oracle_append(s, v, k_new + (int64_t)seq * H * hd, v_new + (int64_t)seq * H * hd,
                               QWFN_SRC_F32, &seq, &p, 1))
            return QWFN_ERANGE;
        if ((p + 1) % bt == 0) qwfn_oracle_pool_block(s, v, seq, p / bt);
    }
    float *scores = (float *)malloc(sizeof(float) * (size_t)(bps > 0 ? bps : 1));
    if (s->shared_selection) {                    /* the general (serial) indexer handles the sum */
        const int rc = qwfn_oracle_indexer_topk(s, v, q, seq_len, n_seq, sel, n_sel, max_sel);
        if (rc < 0) { free(scores); return rc; }
    }
    for (int32_t seq = 0; seq < n_seq && !s->shared_selection; seq++)
        for (int32_t g = 0; g < H; g++) {
            const int32_t L = seq_len[seq];
            int32_t b_last, fw, e_lo, e_hi;
            qsa_ranges(s, L, &b_last, &fw, &e_lo, &e_hi);
            if (s->top_k_blocks > 0 && e_hi - e_lo > eff_topk(s, L)) {
                const float *qg = q + ((int64_t)seq * s->n_head + (int64_t)g * G) * hd;
                const float *pb = v->pooled + ((int64_t)seq * H + g) * bps * hd;
#pragma omp parallel for schedule(static)
                for (int32_t b = e_lo; b < e_hi; b++)
                    scores[b] = qwfn_oracle_block_score(s, qg, pb + (int64_t)b * hd);
            }
            n_sel[seq * H + g] = qwfn_oracle_select(s, scores, L, sel + ((int64_t)seq * H + g) * max_sel, max_sel);
        }
    free(scores);
    /* attention: one task per (sequence, KV head, split of its selected
     * blocks).  Each selected row is dequantized and cast to F16 once (the
     * reference gathers and casts K/V once per KV head, src/qwfn_graph.cpp:
     * 530-541) and serves the group's G query heads, each with its own online
     * softmax; the splits are merged per query head. */
    const int32_t splits = 16;
    const int64_t n_task = (int64_t)n_seq * H * splits;
    const int64_t rec = (int64_t)hd + 2;
    float *part = (float *)malloc(sizeof(float) * (size_t)(n_task * G * rec));
    int32_t row_err = 0;
#pragma omp parallel for schedule(dynamic)
    for (int64_t task = 0; task < n_task; task++) {
        const int32_t sp = (int32_t)(task % splits);
        const int32_t g = (int32_t)((task / splits) % H);
        const int32_t seq = (int32_t)(task / splits / H);
        const int32_t L = seq_len[seq];
        const int32_t nb = n_sel[seq * H + g];
        const int32_t *sl = sel + ((int64_t)seq * H + g) * max_sel;
        const float *qg = q + ((int64_t)seq * s->n_head + (int64_t)g * G) * hd;
        float m[16], l[16], sc[16];
        float acc[16 * 512], kr[512], vr[512];
        for (int32_t h = 0; h < G; h++) { m[h] = -INFINITY; l[h] = 0.0f; }
        for (int64_t i = 0; i < (int64_t)G * hd; i++) acc[i] = 0.0f;
        const float scale = 1.0f / sqrtf((float)hd);
        for (int32_t i = sp; i < nb; i += splits) {
            const int32_t b = sl[i];
            for (int32_t t = b * bt; t < b * bt + bt && t < L; t++) {
                if (baseline_row(s, v, v->k_pages, seq, t, g, kr) || baseline_row(s, v, v->v_pages, seq, t, g, vr)) {
#pragma omp atomic write
                    row_err = 1;
                    continue;
                }
                for (int32_t h = 0; h < G; h++) sc[h] = dot8(qg + (int64_t)h * hd, kr, hd) * scale;
                for (int32_t h = 0; h < G; h++) {
                    const float mn = sc[h] > m[h] ? sc[h] : m[h];
                    const float corr = expf(m[h] - mn), pw = expf(sc[h] - mn);
                    float *a = acc + (int64_t)h * hd;
                    for (int32_t d = 0; d < hd; d++) a[d] = a[d] * corr + pw * vr[d];
                    l[h] = l[h] * corr + pw;
                    m[h] = mn;
                }
            }
        }
        for (int32_t h = 0; h < G; h++) {
            float *pp = part + (task * G + h) * rec;
            pp[0] = m[h];
            pp[1] = l[h];
            memcpy(pp + 2, acc + (int64_t)h * hd, sizeof(float) * (size_t)hd);
        }
    }
    if (row_err) { free(part); return QWFN_ERANGE; }
    for (int32_t seq = 0; seq < n_seq; seq++)
        for (int32_t hq = 0; hq < s->n_head; hq++) {
            const int32_t g = hq / G, h = hq % G;
            float M = -INFINITY, Lsum = 0.0f;
            for (int32_t sp = 0; sp < splits; sp++) {
                const float *x = part + ((((int64_t)seq * H + g) * splits + sp) * G + h) * rec;
                if (x[1] > 0.0f && x[0] > M) M = x[0];
            }
            float *o = out + ((int64_t)seq * s->n_head + hq) * hd;
            for (int32_t d = 0; d < hd; d++) o[d] = 0.0f;
            for (int32_t sp = 0; sp < splits; sp++) {
                const float *x = part + ((((int64_t)seq * H + g) * splits + sp) * G + h) * rec;
                if (x[1] == 0.0f) continue;
                const float w = expf(x[0] - M);
                Lsum += w * x[1];
                for (int32_t d = 0; d < hd; d++) o[d] += w * x[2 + d];
            }
            for (int32_t d = 0; d < hd; d++) o[d] = Lsum > 0.0f ? o[d] / Lsum : 0.0f;
        }
    free(part);
    return threads;
}

/* ---- the checkpoint's own indexer keys ------------------------------------ */

/* Pooled key of block b from its block_tokens raw fp16 members [bt][D]
 * (qsa_pool_blocks, src/qwfn_graph.cpp:410-429): the mean by a sequential
 * fp32 add chain then * fp32(1/bt) (:415-422); RMSNorm with the fp32 squares
 * summed in fp64 (ggml_rms_norm sums in fp64 too) -- 64 lane partials over
 * dims l + 64k, then a butterfly over lane distances 32..1 --, mean =
 * fp32(sum / D), scale = 1 / sqrtf(mean + eps), x * scale * k_norm (:423);
 * then the rotation of the block's first position b*bt (IMROPE with every
 * section at that position, :425-427; src/qwfn_engine.cpp:741-743, 926,
 * 934): pairs (i, i + nd/2), the angle of ggml's rope (ggml, not in the tree:
 * theta_scale = powf(base, -2/nd), theta_0 = pos, theta_{i+1} = theta_i *
 * theta_scale in fp32), cos / sin of that fp32 angle in fp64 rounded to
 * fp32; finally fp16 round to nearest even (the F16 pool cache,
 * src/qwfn_engine.cpp:389-394), returned as fp32. */
int qwfn_oracle_idx_pool_block(const qwfn_qsa_shape *s, const qwfn_idx_shape *is,
                               const uint16_t *members, const float *k_norm, int32_t b,
                               float *out) {
    const int32_t D = is->idx_dim, nd = is->rope_dim, bt = s->block_tokens;
    if (D % 64 || D > 256 || nd < 0 || nd % 2 || nd > D) return QWFN_EINVAL;
    float x[256], y[256];
    for (int32_t d = 0; d < D; d++) {
        float a = qwfn_oracle_f16_to_f32(members[d]);
        for (int32_t r = 1; r < bt; r++) a = a + qwfn_oracle_f16_to_f32(members[(int64_t)r * D + d]);
        x[d] = a * (1.0f / (float)bt);
    }
    double lanes[64];
    for (int32_t l = 0; l < 64; l++) {
        double acc = 0.0;
        for (int32_t k = 0; k < D / 64; k++) {
            const float sq = x[l + 64 * k] * x[l + 64 * k];
            acc = acc + (double)sq;
        }
        lanes[l] = acc;
    }
    for (int32_t off = 32; off >= 1; off >>= 1) {
        double nxt[64];
        for (int32_t l = 0; l < 64; l++) nxt[l] = lanes[l] + lanes[l ^ off];
        memcpy(lanes, nxt, sizeof lanes);
    }
    const float mean = (float)(lanes[0] / (double)D);
    const float scale = 1.0f / sqrtf(mean + is->rms_eps);
    for (int32_t d = 0; d < D; d++) y[d] = (x[d] * scale) * k_norm[d];
    const int32_t half = nd / 2, t0 = b * bt;
    const float theta_scale = powf(is->rope_freq_base, -2.0f / (float)nd);
    float theta[128];
    theta[0] = (float)t0;
    for (int32_t i = 1; i < half; i++) theta[i] = theta[i - 1] * theta_scale;
    for (int32_t d = 0; d < D; d++) {
        float o = y[d];
        if (d < nd) {
            const int32_t i = d < half ? d : d - half;
            const double th = (double)theta[i];
            const float c = (float)cos(th), sn = (float)sin(th);
            const float x0 = y[i], x1 = y[i + half];
            o = d < half ? x0 * c - x1 * sn : x0 * sn + x1 * c;
        }
        out[d] = f16_round(o);
    }
    return 0;
}
