/*
 * qsa_oracle.h -- CPU restatement of the q8_0 KV cache + QSA decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the HIP path is
 * compared against, and (qwfn_oracle_decode_step_f32) the CPU baseline timed
 * beside it.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it; the product library never does.
 *
 * The arithmetic of the reference path lives in ggml (not vendored; pinned at
 * unslothai/llama.cpp ca1426903fabe9af26cd10c42034cb4bbd2e0e11,
 * /root/reference README.md:133-136) and cannot be built here, so each function
 * restates the published algorithm and cites the reference call site it
 * serves.  All buffers are host memory in the device layout documented in
 * include/qwfn_qsa.h, so a device buffer copied to the host compares
 * byte-for-byte.  fp32 throughout, no contraction (-ffp-contract=off), every
 * fused multiply-add written as fmaf.
 *
 * Pinning (what checks each function independently of this restatement):
 *   fp16 conversion   numpy float16 over special values and random sweeps
 *   q8_0 quantize     closed-form known answers + numpy rint/round restatement
 *   q4_0 quantize     closed-form known answers (d = m/-8, grids of exact
 *                     multiples, ties of magnitude, signs), reconstruction bound
 *   layout / gather   exact round trip, brute force over tiny caches
 *   pooling           numpy sequential float32 chain + constant-block invariant
 *   block score       exact rational arithmetic (fractions) on small cases
 *   selection         brute-force sort in Python + special cases
 *   attention (f64)   numpy float64 textbook softmax + closed-form cases
 *   indexer pooling   numpy float64 mean / RMSNorm on unrotated blocks, the
 *                     rotation's closed form on basis vectors, norm and
 *                     pass-through invariants
 * No function is unpinned.
 */
#ifndef QWFN_QSA_ORACLE_H
#define QWFN_QSA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/qwfn_qsa.h"

#ifdef __cplusplus
extern "C" {
#endif

/* fp32 <-> fp16, IEEE binary16, round to nearest even, subnormals kept. */
uint16_t qwfn_oracle_f32_to_f16(float x);
float    qwfn_oracle_f16_to_f32(uint16_t h);
void     qwfn_oracle_f32_to_f16_n(const float *x, int64_t n, uint16_t *out);

/* One q8_0 block (32 values): *d = fp16 scale, qs = quants. */
void qwfn_oracle_quantize_block(const float *x, int32_t variant, uint16_t *d,
                                int8_t *qs);
/* n values (a multiple of 32) -> ggml block_q8_0 bytes (34 per block). */
void qwfn_oracle_quantize_row_ggml(const float *x, int64_t n, int32_t variant,
                                   uint8_t *out);
/* One q4_0 block (32 values): *d = fp16 scale, qs = 16 packed nibble bytes. */
void qwfn_oracle_quantize_block_q4_0(const float *x, uint16_t *d, uint8_t *qs);
/* n values -> ggml's row bytes of the cache type (kv_type QWFN_KV_*). */
void qwfn_oracle_quantize_row_type(const float *x, int64_t n, int32_t kv_type, int32_t variant,
                                   uint8_t *out);

/* Byte offsets inside one page (see include/qwfn_qsa.h); which = 0 for a K
 * page, 1 for a V page (V quants are dim-major when block_tokens % 64 == 0). */
size_t  qwfn_oracle_page_bytes(const qwfn_qsa_shape *s);
int64_t qwfn_oracle_quant_offset(const qwfn_qsa_shape *s, int32_t which, int32_t g,
                                 int32_t row, int32_t d);
int64_t qwfn_oracle_scale_offset(const qwfn_qsa_shape *s, int32_t g, int32_t row,
                                 int32_t j);

/* Host-memory cache operations on a qwfn_kv_view whose pointers are host
 * pointers.  Return 0, or a negative QWFN_E* code on a bad index. */
int qwfn_oracle_append(const qwfn_qsa_shape *s, const qwfn_kv_view *v,
                       const void *k_src, const void *v_src, int32_t src_dtype,
                       const int32_t *seq_ids, const int32_t *pos, int32_t n_rows);
/* Dequantized row of head g at position t of sequence seq from pool
 * (k_pages or v_pages) -> out[head_dim]. */
int qwfn_oracle_dequant_row(const qwfn_qsa_shape *s, const qwfn_kv_view *v,
                            const void *pool, int32_t seq, int32_t t, int32_t g,
                            float *out);
int qwfn_oracle_pool_block(const qwfn_qsa_shape *s, const qwfn_kv_view *v,
                           int32_t seq, int32_t b);

/* Score of one block for one KV head: q_group = the G query heads of the group
 * [G][head_dim], p = pooled key [head_dim]. */
float qwfn_oracle_block_score(const qwfn_qsa_shape *s, const float *q_group,
                              const float *p);
/* Kept blocks of one (sequence, KV head) at length seq_len, ascending, given
 * the scores of all blocks (scores[b] for b < seq_len/block_tokens; entries of
 * non-eligible blocks are ignored).  Returns the count (<= max_sel) or < 0. */
int32_t qwfn_oracle_select(const qwfn_qsa_shape *s, const float *scores,
                           int32_t seq_len, int32_t *sel, int32_t max_sel);
int32_t qwfn_oracle_max_selected(const qwfn_qsa_shape *s, int32_t max_seq_len);
/* Scores + selection for every (sequence, KV head): q [n_seq][n_head][hd],
 * sel [n_seq][n_head_kv][max_sel], n_sel [n_seq][n_head_kv]. */
int qwfn_oracle_indexer_topk(const qwfn_qsa_shape *s, const qwfn_kv_view *v,
                             const float *q, const int32_t *seq_len, int32_t n_seq,
                             int32_t *sel, int32_t *n_sel, int32_t max_sel);
/* Reference attention in fp64 over a selection (sel == NULL: dense).
 * out [n_seq][n_head][hd] as doubles. */
int qwfn_oracle_attention_f64(const qwfn_qsa_shape *s, const qwfn_kv_view *v,
                              const float *q, const int32_t *seq_len, int32_t n_seq,
                              const int32_t *sel, const int32_t *n_sel,
                              int32_t max_sel, double *out);

/* Prefill of queries pos0 .. pos0+n_q-1 of sequence seq (rows and pooled keys
 * in place): query i is the decode rule at seq_len = pos0+i+1 without the
 * append.  sel [n_q][n_head_kv][max_sel], n_sel [n_q][n_head_kv],
 * out [n_q][n_head][hd] as doubles. */
int qwfn_oracle_prefill_f64(const qwfn_qsa_shape *s, const qwfn_kv_view *v, const float *q,
                            int32_t seq, int32_t pos0, int32_t n_q, int32_t *sel, int32_t *n_sel,
                            int32_t max_sel, double *out);
/* The same with the attention of every attn_stride-th query only (query i with
 * i % attn_stride == 0, and the last query); the other queries get their
 * selection and zero outputs.  A chunk of thousands of long-context queries
 * checks every selection and a strided sample of the outputs. */
int qwfn_oracle_prefill_f64_strided(const qwfn_qsa_shape *s, const qwfn_kv_view *v, const float *q,
                                    int32_t seq, int32_t pos0, int32_t n_q, int32_t attn_stride,
                                    int32_t *sel, int32_t *n_sel, int32_t max_sel, double *out);
/* CPU baseline: one decode token of the whole path in fp32 (append at
 * seq_len-1, pool on block completion, scores, selection, attention with the
 * gathered K/V cast to fp16 as the reference's decode does, online softmax).
 * Like the reference's CPU path it dequantizes and casts each selected row once
 * per KV head and serves the group's query heads from it; OpenMP over scoring
 * blocks and over (sequence, KV head, split) attention tasks.  Its selection
 * equals qwfn_oracle_indexer_topk's and its output is within the attention
 * tolerance of qwfn_oracle_attention_f64's (tests/test_oracle_baseline.py).
 * head_dim <= 512 (a multiple of 32), at most 16 query heads a KV head.
 * Returns the thread count used, or < 0. */
int qwfn_oracle_decode_step_f32(const qwfn_qsa_shape *s, const qwfn_kv_view *v,
                                const float *q, const float *k_new,
                                const float *v_new, const int32_t *seq_len,
                                int32_t n_seq, float *out, int32_t *sel,
                                int32_t *n_sel, int32_t max_sel);

/* The checkpoint indexer's pooled key of block b: members = the block's
 * block_tokens raw fp16 keys [bt][idx_dim]; out [idx_dim] (fp16-rounded values
 * as fp32).  Arithmetic order as documented for qwfn_idx_append_pool. */
int qwfn_oracle_idx_pool_block(const qwfn_qsa_shape *s, const qwfn_idx_shape *is,
                               const uint16_t *members, const float *k_norm, int32_t b,
                               float *out);

#ifdef __cplusplus
}
#endif
#endif
