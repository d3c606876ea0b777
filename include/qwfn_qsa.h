/*
 * qwfn_qsa.h -- C ABI of the MI355X (gfx950) q8_0 KV cache and Qwen Sparse
 * Attention (QSA) decode path.
 *
 * The reference engine builds this path out of ggml graph nodes inside
 * qwfn::graph_builder; every entry point below replaces one group of those
 * nodes and names the reference lines it stands in for.  The caller owns all
 * device memory (the reference's `state` owns the cache buffers,
 * src/qwfn_state.cpp:74-87); nothing here allocates on the hot path.
 *
 * Conventions
 *  - Every function returns QWFN_OK (0) or a negative QWFN_E* code; the message
 *    of the last failure on the calling thread is qwfn_qsa_last_error().
 *    Shapes, counts and sizes are validated on the host before anything is
 *    enqueued; a failed validation enqueues nothing and touches no device
 *    memory.  Nothing aborts.
 *  - Work is only enqueued on `stream` (a hipStream_t passed as void*, NULL =
 *    the null stream).  No call synchronises, so calls can be captured into a
 *    hipGraph and replayed, as the reference replays its per-layer CUDA graphs
 *    (src/qwfn_engine.cpp:2066-2081).
 *  - Per-token indices (sequence ids, positions, sequence lengths) live in
 *    device memory so a captured graph can be replayed with new values.  The
 *    kernels bound-check them; a row, block or sequence that is out of range is
 *    skipped and the matching QWFN_STATUS_* bit is OR-ed into view->status
 *    (when non-NULL).  qwfn_qsa_read_status() fetches and clears it.
 *  - Bit-exactness: q8_0 bytes, pooled keys of whole blocks, selected block ids
 *    and gathered cells are deterministic and bit-exact against the CPU
 *    restatement; attention outputs are fp32 within max-abs 2e-3 + 1e-3*|ref|.
 *
 * Device data layout (one K pool and one V pool per attention layer)
 *  page  = n_head_kv * page_tokens * (head_dim + head_dim/16) bytes:
 *    K quants : int8  [n_head_kv][page_tokens/64][head_dim/16][64][16]
 *             (64-token tiles; each 16-byte chunk of a token's head row is
 *              interleaved with the same chunk of the tile's other 63 tokens,
 *              so lane t of a wave reading chunk c of token t is one contiguous
 *              1 KiB load)
 *    V quants : int8  [n_head_kv][page_tokens/64][head_dim][64] when
 *             block_tokens % 64 == 0 (dim-major tiles: dim d of the tile's 64
 *             tokens is 64 contiguous bytes, the operand of a per-dim dot
 *             product over tokens); otherwise the K layout
 *    scales : fp16  [n_head_kv][page_tokens][head_dim/32]  (one per q8_0 block)
 *  Other kv_type values keep the K layout's 16-byte chunks for K and V alike
 *  (R = a head row's bytes, R/16 chunks per row):
 *    Q4_0 : R = head_dim/2, chunk j = the 16 qs bytes of ggml block j (ggml's
 *           nibble order), then the fp16 scales as above
 *    F16  : R = 2*head_dim, chunk c = dims 8c .. 8c+7, no scales
 *  A logical position t of sequence s lives in physical page
 *  page_table[s*pages_per_seq + t/page_tokens] at row t%page_tokens.
 *  pooled = fp32 [n_seq][n_head_kv][blocks_per_seq][head_dim], where
 *  blocks_per_seq = pages_per_seq*page_tokens/block_tokens.
 *  The reference's cache (src/qwfn_state.cpp:50-54) is a different byte
 *  layout: one 1-D tensor per layer of token-major ggml block_q8_0 rows (each
 *  head row a run of 34-byte blocks, fp16 scale then 32 quants).  The kernels
 *  read only the layout above; state::init allocates these pages in its place
 *  (qwfn_qsa_page_bytes), and rows in the reference's format enter or leave
 *  through qwfn_kv_import_q8_0 / qwfn_kv_export_q8_0, a copy.
 */
#ifndef QWFN_QSA_H
#define QWFN_QSA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QWFN_QSA_ABI_VERSION 5

/* return codes */
#define QWFN_OK        0
#define QWFN_EHIP     (-5)   /* a HIP runtime call failed */
#define QWFN_EINVAL   (-22)  /* bad shape, pointer or count */
#define QWFN_ERANGE   (-34)  /* a length or size exceeds what the view holds */
#define QWFN_ENOTSUP  (-95)  /* a valid shape this build has no kernel for */

/* q8_0 rounding variants of ggml's quantizer (block_q8_0: fp16 d; int8 qs[32])
 *  X86_RNE   : id = 127/amax, q = round-half-even(x*id)  (ggml-cpu AVX path)
 *  REF_ROUNDF: id = 1/d,      q = roundf(x*id)           (quantize_row_q8_0_ref,
 *                                                          ggml-cuda set_rows)
 * Both store d = fp16_rne(amax/127).  A non-finite x*id stores q = 0.        */
#define QWFN_Q8_X86_RNE     0
#define QWFN_Q8_REF_ROUNDF  1

/* K/V cache element types (the reference's --kv q8_0|q4_0|f16,
 * tools/qwfn_gen.cpp:55-57; README.md:176):
 *  Q8_0: ggml block_q8_0 {fp16 d; int8 qs[32]}, quant_variant's rounding
 *  Q4_0: ggml block_q4_0 {fp16 d; uint8 qs[16]}: d = m / -8 with m the element
 *        of largest magnitude (the first such), q = min(15, trunc(x/d + 8.5)),
 *        qs[j] = q[j] | q[j+16] << 4 (quantize_row_q4_0_ref)
 *  F16 : fp16, round to nearest even                                          */
#define QWFN_KV_Q8_0  0
#define QWFN_KV_Q4_0  1
#define QWFN_KV_F16   2

/* element type of K/V rows handed to the append */
#define QWFN_SRC_F32  0
#define QWFN_SRC_F16  1

/* bits of view->status */
#define QWFN_STATUS_POS_RANGE    0x1  /* a position >= the view's capacity     */
#define QWFN_STATUS_SEQ_RANGE    0x2  /* a sequence id outside [0, n_seq)      */
#define QWFN_STATUS_PAGE_RANGE   0x4  /* a page-table entry outside the pool   */
#define QWFN_STATUS_LEN_RANGE    0x8  /* a seq_len < 1 or > max_seq_len        */
#define QWFN_STATUS_BLOCK_RANGE  0x10 /* a block id beyond the view           */

typedef struct qwfn_qsa_shape {
    int32_t n_head;          /* query heads (16)                               */
    int32_t n_head_kv;       /* KV heads (2); GQA group = n_head/n_head_kv     */
    int32_t head_dim;        /* 128                                            */
    int32_t block_tokens;    /* tokens pooled into one indexer block (64)      */
    int32_t page_tokens;     /* tokens per cache page, a multiple of 64 (256)  */
    int32_t top_k_blocks;    /* scored blocks kept (64); <= 0 = dense          */
    int32_t sink_blocks;     /* leading blocks always kept (1)                 */
    int32_t local_tokens;    /* trailing tokens whose blocks are kept (512);
                              * 0: only a partial tail block is kept (the
                              * checkpoint's bias, src/qwfn_engine.cpp:748-753:
                              * 1e9 for the incomplete tail block, 0 for every
                              * whole block, the tail's included)           */
    int32_t relu_per_head;   /* 1: score = sum_h relu(q_h.p) (lightning idx)   */
    int32_t shared_selection;/* 1: one selection for all KV heads, on their
                              * scores summed in head order (the checkpoint's
                              * rule, src/qwfn_graph.cpp:477-495)            */
    int32_t quant_variant;   /* QWFN_Q8_X86_RNE or QWFN_Q8_REF_ROUNDF          */
    int32_t topk_counts_forced; /* 1: the kept set is top_k_blocks blocks in
                              * all, the forced ones included (top_k of the
                              * biased scores with k_blocks = top_k_blocks,
                              * src/qwfn_graph.cpp:493, src/qwfn_engine.cpp:
                              * 430); 0: top_k_blocks scored blocks on top of
                              * the forced ones                              */
    int32_t kv_type;         /* QWFN_KV_Q8_0 / QWFN_KV_Q4_0 / QWFN_KV_F16       */
    int32_t kv_round_f16;    /* 1: the decode attention rounds every dequantized
                              * K and V value to fp16 (round to nearest even)
                              * before its arithmetic: the F16 cast of the
                              * gathered K/V ahead of flash_attn_ext
                              * (src/qwfn_graph.cpp:530-537).  What ggml's
                              * flash_attn_ext then does with Q and its
                              * accumulators is not in the reference tree, so
                              * parity beyond the K/V cast is unpinned; the
                              * attention here stays fp32 over the rounded
                              * values.  0: the exact dequantized values.  Prefill
                              * ignores it (the reference's prefill reads the
                              * cache rows directly, src/qwfn_graph.cpp:
                              * 365-403)                                     */
} qwfn_qsa_shape;

typedef struct qwfn_kv_view {
    void          *k_pages;      /* [n_phys_pages][page bytes], device          */
    void          *v_pages;      /* same for V                                  */
    float         *pooled;       /* fp32 pooled keys, layout above, device      */
    const int32_t *page_table;   /* [n_seq][pages_per_seq], device              */
    int32_t       *status;       /* one device int32, or NULL                   */
    int32_t        n_seq;
    int32_t        pages_per_seq;
    int32_t        n_phys_pages;
} qwfn_kv_view;

/* ---- introspection / sizing ------------------------------------------------ */
int         qwfn_qsa_abi_version(void);
const char *qwfn_qsa_last_error(void);
/* Measurement hook; it has no counterpart in the reference and serves
 * benchmarks and profilers of the path.  Arms per-kernel timing of the next
 * qwfn_sparse_attn_decode / qwfn_decode_append_select /
 * qwfn_sparse_decode_attn call on the calling thread.  events[0..5] are
 * hipEvent_t created with timing (or NULL pairs): (0, 1) the indexer launch,
 * (2, 3) the attention launch, (4, 5) the merge launch.  Each armed kernel is
 * launched with hipExtLaunchKernel, which stamps its pair with that kernel's
 * own begin and end; read them with hipEventElapsedTime once the stream has
 * completed.  A call on a capturing stream times nothing.  The call disarms
 * what it did not use; events == NULL disarms.                               */
int         qwfn_qsa_time_next_call(void *const events[6]);
/* Test hook; it has no counterpart in the reference and serves the tests that
 * check the prefill scoring's error bound on the hardware.  Runs the
 * prefill's approximate matrix-core scoring alone: queries q
 * [n_q][n_head][head_dim] (fp32) of sequence `seq` against the pooled blocks
 * [sink_blocks, n_blk) of every KV head, writing the approximate scores to
 * scores [n_q][n_head_kv][nb_cap] and each block's key norm, rounded up, to
 * pnorm [n_head_kv][nb_cap] (device fp32; other entries untouched).  The
 * prefill's selection is exact because |approximate - exact| <= 1.05e-3 *
 * (sum over the query's group of |q_h|) * |p| + 1e-37.  QWFN_ENOTSUP for shapes
 * without the matrix-core scoring (group * head_dim > 1024).                */
int qwfn_qsa_test_prefill_scores(const qwfn_qsa_shape *shape, const qwfn_kv_view *view,
                                 const float *q, int32_t n_q, int32_t seq, int32_t n_blk,
                                 float *scores, float *pnorm, int32_t nb_cap, void *stream);
/* Test hook; it has no counterpart in the reference and serves the tests of
 * the attention's own selection over long score rows (the checkpoint layer's
 * decode past 8192 eligible blocks).  Runs that selection alone, one
 * workgroup per sequence: the forced/eligible rule and the exact top-k by
 * (score desc, block asc) of row s of scores [n_seq][nb_cap] (device fp32,
 * 16-byte aligned, nb_cap a multiple of 4 and at least max_seq_len /
 * block_tokens + 4) at length seq_len[s], into sel [n_seq][max_sel] and
 * n_sel [n_seq] (device int32).  QWFN_ERANGE when a row of max_seq_len holds
 * more eligible blocks than that selection covers (49,152) or max_sel is
 * outside [qwfn_qsa_max_selected, 1024].                                       */
int qwfn_qsa_test_select_rows(const qwfn_qsa_shape *shape, const float *scores, int32_t nb_cap,
                              const int32_t *seq_len, int32_t n_seq, int32_t max_seq_len, int32_t *sel,
                              int32_t *n_sel, int32_t max_sel, void *stream);
/* Test hook; it has no counterpart in the reference and serves the tests of
 * the checkpoint decode's failure path past 8192 eligible blocks.  There the
 * indexer launch's scoring workgroups wait for the launch's sampled cut by at
 * most `polls` reads of its slots (default 65536, for calls that start after
 * this one); a wait that runs out leaves no candidates, and the attention then
 * selects over the whole score row, with the same result.  polls = 0 makes
 * every wait run out at once.  *previous (optional) gets the bound it
 * replaces.  QWFN_EINVAL for a negative bound.                                */
int qwfn_qsa_test_set_cut_polls(int32_t polls, int32_t *previous);
/* Validates a shape (QWFN_EINVAL) and whether this build has kernels for it
 * (QWFN_ENOTSUP).  Replaces the reference's shape constants
 * (src/qwfn_hparams.h:22-36, src/qwfn_engine.cpp:382-435).                   */
int qwfn_qsa_check_shape(const qwfn_qsa_shape *shape);
/* Bytes of one K (or V) page.  Replaces the per-layer cache sizing of
 * state::init (src/qwfn_state.cpp:39-54).                                      */
int qwfn_qsa_page_bytes(const qwfn_qsa_shape *shape, size_t *bytes);
/* Bytes of the pooled-key array for n_seq sequences of pages_per_seq pages
 * (the reference's pool_cache_, src/qwfn_engine.cpp:389-394).                 */
int qwfn_qsa_pooled_bytes(const qwfn_qsa_shape *shape, int32_t n_seq,
                          int32_t pages_per_seq, size_t *bytes);
/* Upper bound on blocks one (sequence, KV head) selects at a length up to
 * max_seq_len: the reference's k_blocks plus the forced blocks
 * (src/qwfn_engine.cpp:430, 748-753).                                          */
int qwfn_qsa_max_selected(const qwfn_qsa_shape *shape, int32_t max_seq_len,
                          int32_t *max_sel);
/* Workspace for qwfn_indexer_topk / qwfn_sparse_decode_attn /
 * qwfn_sparse_attn_decode at n_seq sequences up to max_seq_len tokens.  The
 * workspace carries completion counters that every call leaves at zero:
 * initialise a new workspace once with qwfn_qsa_workspace_init (a fill kernel,
 * not a memset, so it may also be captured).  Calls that overlap on one
 * workspace race.                                                              */
int qwfn_qsa_workspace_bytes(const qwfn_qsa_shape *shape, int32_t n_seq,
                             int32_t max_seq_len, size_t *bytes);
int qwfn_qsa_workspace_init(void *ws, size_t ws_bytes, void *stream);
/* Synchronously copies view->status to *status and clears it.                 */
int qwfn_qsa_read_status(const qwfn_kv_view *view, int32_t *status, void *stream);

/* ---- format interop ------------------------------------------------------ */
/* Format interop with the reference's cache tensors: per attention layer a
 * 1-D q8_0 tensor whose row t holds the token's n_head_kv * head_dim elements,
 * head-major (src/qwfn_state.cpp:40, 52-53), i.e. n_head_kv * head_dim / 32
 * ggml block_q8_0 {fp16 d; int8 qs[32]} of 34 bytes, rows back to back.
 * qwfn_kv_row_bytes gives one row's size.  Export copies positions
 * [pos0, pos0 + n_tokens) of sequence `seq` out of the paged cache into such
 * rows (device memory, 2-byte aligned); import writes such rows into the pages
 * byte for byte (an idempotent overwrite).  Import leaves the pooled keys
 * alone: pool the blocks it completes with qwfn_pool_rebuild /
 * qwfn_pool_update.  Either row pointer may be NULL (K or V only).  These
 * replace no reference call: they convert its state layout (the tensors of
 * state::init, src/qwfn_state.cpp:50-54) to and from the paged layout.      */
int qwfn_kv_row_bytes(const qwfn_qsa_shape *shape, size_t *bytes);
int qwfn_kv_export_q8_0(const qwfn_qsa_shape *shape, const qwfn_kv_view *view,
                        int32_t seq, int32_t pos0, int32_t n_tokens,
                        void *k_rows, void *v_rows, void *stream);
int qwfn_kv_import_q8_0(const qwfn_qsa_shape *shape, const qwfn_kv_view *view,
                        int32_t seq, int32_t pos0, int32_t n_tokens,
                        const void *k_rows, const void *v_rows, void *stream);

/* ---- cache writes -------------------------------------------------------- */
/* Quantize n_rows K and V rows ([n_head_kv][head_dim] each, F32 or F16) to
 * q8_0 and write them at (seq_ids[i], pos[i]).  An idempotent overwrite: a
 * rewritten position gets exactly the bytes a first write would.
 * Replaces ggml_set_rows into the q8_0 cache at write_idx (decode,
 * src/qwfn_graph.cpp:520-528) and ggml_cpy of a chunk into a view of the cache
 * (prefill, src/qwfn_graph.cpp:349-360).  seq_ids may be NULL (all 0).        */
int qwfn_kv_append_q8_0(const qwfn_qsa_shape *shape, const qwfn_kv_view *view,
                        const void *k_src, const void *v_src, int32_t src_dtype,
                        const int32_t *seq_ids, const int32_t *pos,
                        int32_t n_rows, void *stream);
/* Recompute the pooled key of each listed block from its block_tokens
 * dequantized K members: a sequential fp32 add chain, then *(1/block_tokens).
 * Replaces qsa_pool_blocks' add chain and ggml_scale (src/qwfn_graph.cpp:
 * 410-422) as used by the decode update (:471-476).  A block whose members are
 * not all written gets an unspecified (but finite-input-deterministic) value;
 * it is never scored while partial.  seq_ids may be NULL (all 0).             */
int qwfn_pool_update(const qwfn_qsa_shape *shape, const qwfn_kv_view *view,
                     const int32_t *seq_ids, const int32_t *block_ids,
                     int32_t n_blocks, void *stream);
/* Pool blocks [0, n_whole) of sequence `seq` (host value): the reference's
 * qsa_pool_rebuild after a prefill (src/qwfn_graph.cpp:431-448,
 * src/qwfn_engine.cpp:761-798).                                               */
int qwfn_pool_rebuild(const qwfn_qsa_shape *shape, const qwfn_kv_view *view,
                      int32_t seq, int32_t n_whole, void *stream);

/* ---- selection ------------------------------------------------------------ */
/* Indexer + top-k for one decode token per sequence.  q is fp32
 * [n_seq][n_head][head_dim]; seq_len (device) is each sequence's length
 * including the token just appended (the reference's n_past+1).  Per
 * (sequence, KV head g) the score of whole block b is
 *    sum over the group's heads h of dot(q_h, pooled[b][g])   (relu'd per head
 *    when relu_per_head), in a fixed fp32 order shared with the CPU oracle;
 * the forced set F = sink blocks U blocks meeting the last local_tokens tokens;
 * the eligible set E = whole blocks not in F; the kept set is F U top_k(E) by
 * (score desc, block asc).  sel receives the kept block ids ascending,
 * [n_seq][n_head_kv][max_sel]; n_sel [n_seq][n_head_kv] their count.
 * Replaces the scores / relu / sum_rows / bias add / ggml_top_k nodes
 * (src/qwfn_graph.cpp:477-495) and the host bias window (src/qwfn_engine.cpp:
 * 748-759).                                                                    */
int qwfn_indexer_topk(const qwfn_qsa_shape *shape, const qwfn_kv_view *view,
                      const float *q, const int32_t *seq_len, int32_t n_seq,
                      int32_t max_seq_len, int32_t *sel, int32_t *n_sel,
                      int32_t max_sel, void *ws, size_t ws_bytes, void *stream);
/* The cells of a selection, dequantized: fp32 k_out/v_out
 * [n_seq][n_head_kv][max_sel*block_tokens][head_dim], cells
 * [n_seq][n_head_kv][max_sel*block_tokens] (-1 past seq_len or the count).
 * A parity/debug entry point; the attention kernels gather in place.
 * Replaces ggml_get_rows q8_0->f32 of the selected cells (src/qwfn_graph.cpp:
 * 494-495, 530-537).                                                           */
int qwfn_gather_dequant(const qwfn_qsa_shape *shape, const qwfn_kv_view *view,
                        const int32_t *seq_len, int32_t n_seq,
                        const int32_t *sel, const int32_t *n_sel, int32_t max_sel,
                        float *k_out, float *v_out, int32_t *cells, void *stream);

/* ---- attention ------------------------------------------------------------ */
/* GQA softmax attention of one query token per sequence over the cells of a
 * given selection (cells at positions >= seq_len are masked), scale
 * 1/sqrt(head_dim), fp32 out [n_seq][n_head][head_dim].  sel == NULL means
 * dense: every block below seq_len.  Replaces the cell mask
 * (src/qwfn_graph.cpp:497-502) and ggml_flash_attn_ext with GGML_PREC_F32
 * (:539-542).                                                                  */
int qwfn_sparse_decode_attn(const qwfn_qsa_shape *shape, const qwfn_kv_view *view,
                            const float *q, const int32_t *seq_len, int32_t n_seq,
                            int32_t max_seq_len, const int32_t *sel,
                            const int32_t *n_sel, int32_t max_sel, float *out,
                            void *ws, size_t ws_bytes, void *stream);
/* The first launch of qwfn_sparse_attn_decode on its own: append k_new/v_new
 * at seq_len-1, re-pool the block that position completes, score and select
 * (sel/n_sel as in qwfn_indexer_topk, max_sel >= qwfn_qsa_max_selected).
 * Replaces src/qwfn_graph.cpp:465-495 and 520-528 (the writes, scores and
 * top-k of one decode token).                                                  */
int qwfn_decode_append_select(const qwfn_qsa_shape *shape, const qwfn_kv_view *view,
                              const float *q, const void *k_new, const void *v_new,
                              int32_t src_dtype, const int32_t *seq_len,
                              int32_t n_seq, int32_t max_seq_len, int32_t *sel,
                              int32_t *n_sel, int32_t max_sel,
                              void *ws, size_t ws_bytes, void *stream);
/* One decode token of graph_builder::sparse_attn_decode (src/qwfn_graph.cpp:
 * 450-546) from the K/V projections on: append k_new/v_new
 * ([n_seq][n_head_kv][head_dim], src_dtype) at position seq_len-1, re-pool the
 * block that position completes, score + select, and attend.  sel_out/n_sel_out
 * (optional) receive the selection as qwfn_indexer_topk would.  Three
 * launches: the indexer, the attention and the merge of its partials (five
 * with local_tokens = 0, where the block a token completes is eligible at
 * once: its append and pooling then run first, as launches of their own, so
 * the scoring reads the completed key).  Up to
 * eight sequences with per-head selections (shared_selection 0) of at most
 * 8192 eligible blocks and max selected blocks <= 1024, the indexer only
 * scores and the attention's workgroups select for themselves; otherwise the
 * launches are qwfn_decode_append_select's and qwfn_sparse_decode_attn's.     */
int qwfn_sparse_attn_decode(const qwfn_qsa_shape *shape, const qwfn_kv_view *view,
                            const float *q, const void *k_new, const void *v_new,
                            int32_t src_dtype, const int32_t *seq_len,
                            int32_t n_seq, int32_t max_seq_len, float *out,
                            int32_t *sel_out, int32_t *n_sel_out,
                            void *ws, size_t ws_bytes, void *stream);
/* n_pos (1 .. 8) chained decode positions of every sequence in one call: the
 * multi-position decode of the MTP verify step, where the engine builds T
 * sparse_attn_decode calls into one graph and each reads through the writes
 * of the ones before (src/qwfn_engine.cpp:1892-1906, the qsa_chain of
 * src/qwfn_graph.h:104-109).  Position k of sequence s appends k_new[k][s] at
 * seq_len[s] - 1 + k and attends with length seq_len[s] + k, exactly as the
 * k-th of n_pos qwfn_sparse_attn_decode calls would: q [n_pos][n_seq][n_head]
 * [head_dim], k_new / v_new [n_pos][n_seq][n_head_kv][head_dim], out
 * [n_pos][n_seq][n_head][head_dim], sel_out [n_pos][n_seq][n_head_kv]
 * [qwfn_qsa_max_selected] and n_sel_out [n_pos][n_seq][n_head_kv] (optional).
 * max_seq_len bounds seq_len + n_pos - 1.  One small launch derives the
 * positions' lengths into the workspace, then each position makes
 * qwfn_sparse_attn_decode's launches; all on `stream`, so the chain captures
 * into one hipGraph.  n_pos = 1 is qwfn_sparse_attn_decode.                   */
int qwfn_sparse_attn_decode_chain(const qwfn_qsa_shape *shape, const qwfn_kv_view *view,
                                  const float *q, const void *k_new, const void *v_new,
                                  int32_t src_dtype, const int32_t *seq_len, int32_t n_seq,
                                  int32_t n_pos, int32_t max_seq_len, float *out,
                                  int32_t *sel_out, int32_t *n_sel_out,
                                  void *ws, size_t ws_bytes, void *stream);

/* qwfn_sparse_attn_decode without a workspace argument, for callers that
 * cannot allocate device memory (code under hipGraph capture that may not
 * call hipMalloc, tight serving loops, harnesses that forbid allocation).  No
 * counterpart in the reference.  The workspace is a file-scope device array
 * of the library, 8 MiB per device, held until the process ends: calls whose
 * qwfn_qsa_workspace_bytes(shape, n_seq, max_seq_len) exceeds it return
 * QWFN_ERANGE (8 MiB holds eight sequences of the BASELINE shape up to 1M
 * tokens).  The first call on a device enqueues one fill kernel on `stream`
 * that clears the array, unless `stream` is capturing (the array is zero when
 * the library loads, and a captured fill would rerun on every replay).  Every
 * call leaves the array's counters at zero.  Every call on a device shares its array, so calls
 * that overlap on one device (other streams, other threads) race; calls in
 * stream order do not.  Nothing here allocates or frees.                    */
int qwfn_sparse_attn_decode_noalloc(const qwfn_qsa_shape *shape, const qwfn_kv_view *view,
                                    const float *q, const void *k_new, const void *v_new,
                                    int32_t src_dtype, const int32_t *seq_len, int32_t n_seq,
                                    int32_t max_seq_len, float *out, int32_t *sel_out,
                                    int32_t *n_sel_out, void *stream);

/* ---- prefill ------------------------------------------------------------- */

/* Workspace for qwfn_sparse_attn_prefill processing q_batch queries per
 * launch pair, contexts up to max_seq_len.  A larger workspace lets the call
 * take more queries per launch; any size from q_batch = 1 up works. */
int qwfn_qsa_prefill_workspace_bytes(const qwfn_qsa_shape *shape, int32_t max_seq_len,
                                     int32_t q_batch, size_t *bytes);

/* Prefill chunk of sequence `seq`: queries at positions pos0 .. pos0+n_q-1.
 * Replaces the QSA part of graph_builder::sparse_attn / qsa_top_k
 * (src/qwfn_graph.cpp:235-408: the chunk's block pooling :257-269, per-query
 * scores, bias and ggml_top_k :282-305, the K/V copy into the cache :349-360,
 * the selected-cell causal mask :367-398 and the masked flash-attention
 * :400-403) and the host-built per-chunk tables and bias of
 * src/qwfn_engine.cpp:884-957.
 *  - k_new/v_new ([n_q][n_head_kv][head_dim], src_dtype), when non-NULL, are
 *    appended at pos0.. and every whole block in [pos0/bt, (pos0+n_q)/bt) is
 *    re-pooled.  With NULL the rows and pooled keys must already be in place.
 *  - Query i (q [n_q][n_head][head_dim] fp32) attends causally over its own
 *    selection, exactly as a decode step at seq_len = pos0 + i + 1: the sink
 *    blocks, its top_k eligible blocks by pooled-key score, the blocks of its
 *    local window, cells <= pos0 + i.  out [n_q][n_head][head_dim] fp32.
 *  - sel_out [n_q][n_head_kv][max_sel] / n_sel_out [n_q][n_head_kv] (optional)
 *    receive each query's selection.
 * The queries are processed in batches sized to ws_bytes (see
 * qwfn_qsa_prefill_workspace_bytes), each batch a scoring, a selection and
 * an attention launch (and the merge of its partials for the general
 * attention kernel) on `stream`. */
int qwfn_sparse_attn_prefill(const qwfn_qsa_shape *shape, const qwfn_kv_view *view,
                             const float *q, const void *k_new, const void *v_new,
                             int32_t src_dtype, int32_t seq, int32_t pos0, int32_t n_q,
                             float *out, int32_t *sel_out, int32_t *n_sel_out,
                             int32_t max_sel, void *ws, size_t ws_bytes, void *stream);

/* ---- the checkpoint's own indexer ---------------------------------------- */
/* The released checkpoint scores blocks with a separate indexer
 * (src/qwfn_graph.cpp:233-305 prefill, 410-495 decode): per token a RAW key of
 * idx_dim values is cached as F16 (the idx cache, :244-254, 465-470); a block
 * of block_tokens (its ratio r, 4) is keyed by the mean of its members' raw
 * keys, RMSNorm'd * indexer.k_norm and rotated to the block's first position
 * (qsa_pool_blocks, :410-429), held in an F16 pool cache
 * (src/qwfn_engine.cpp:389-394); the score of a block is
 * sum over the n_idx_head indexer query heads of relu(q_h . pooled[b]) (:477-
 * 492), and ONE top-k selection serves every KV head.
 *
 * Here the raw keys are paged like K and V (the KV view's page table and
 * page_tokens); the pooled keys are fp16, as in the reference's pool cache.
 * The selection rule comes from qwfn_qsa_shape as usual: the
 * checkpoint's is sink_blocks 0, local_tokens 0, topk_counts_forced 1,
 * top_k_blocks = k_blocks (513 = ceil((idx_top_k + r - 1) / r), src/
 * qwfn_engine.cpp:430), relu_per_head 1.  The selection is written to each of
 * the n_head_kv rows of sel, so qwfn_sparse_decode_attn takes it unchanged.
 *
 * Pooling arithmetic (fixed, and repeated by the CPU oracle):
 *   mean    fp32 add chain over the members in position order, * fp32(1/r)
 *   RMSNorm sum of fp32 squares in fp64, lane partials (dims d = l + 64k)
 *           then a butterfly over lanes 32..1; scale = 1/sqrtf(fp32(sum/D) +
 *           eps); x * scale * k_norm[d]
 *   rotary  pairs (i, i + rope_dim/2), ggml's angle: theta_0 = (float)pos,
 *           theta_{i+1} = theta_i * theta_scale, each product rounded to
 *           fp32, theta_scale = powf(rope_base, -2/rope_dim) on the host;
 *           cos / sin of that fp32 angle evaluated in fp64 and rounded to
 *           fp32; dims >= rope_dim pass through.
 *           The reference's IMROPE gives all four position sections the same
 *           position for text (src/qwfn_engine.cpp:741, 781, 926, 934), which
 *           makes it this rotation; per-section (vision) positions are not
 *           supported.
 *   store   fp16 round to nearest even.                                     */
typedef struct qwfn_idx_shape {
    int32_t idx_dim;         /* 128: indexer key length (src/qwfn_hparams.h:53) */
    int32_t n_idx_head;      /* 4: indexer query heads (:52)                     */
    int32_t rope_dim;        /* 64: rotated dims (:35)                           */
    float   rope_freq_base;  /* the checkpoint's rope_freq_base                  */
    float   rms_eps;         /* the checkpoint's rms_eps                         */
} qwfn_idx_shape;

typedef struct qwfn_idx_view {
    void        *raw;        /* fp16 [n_phys_pages][page_tokens][idx_dim], device,
                              * paged by the KV view's page_table (16-B aligned) */
    void        *pooled;     /* fp16 [n_seq][blocks_per_seq][idx_dim], device   */
    const float *k_norm;     /* fp32 [idx_dim] indexer.k_norm.weight, device    */
} qwfn_idx_view;

/* Bytes of one raw-key page and of the pooled keys of n_seq sequences
 * (replaces the idx cache and pool cache sizing, src/qwfn_state.cpp via
 * st_->idx_cache and src/qwfn_engine.cpp:389-394). */
int qwfn_idx_cache_bytes(const qwfn_qsa_shape *shape, const qwfn_idx_shape *ishape,
                         int32_t n_seq, int32_t pages_per_seq,
                         size_t *raw_page_bytes, size_t *pooled_bytes);
/* Workspace of qwfn_idx_select and qwfn_idx_sparse_attn_decode (counters
 * shared with qwfn_qsa_workspace_*: one workspace initialised once serves both
 * when it is the larger size).  It holds the indexer's layout and, after it,
 * the attention's, so that the decode call can leave rows of more than 8,192
 * candidate blocks to the attention's own selection. */
int qwfn_idx_workspace_bytes(const qwfn_qsa_shape *shape, const qwfn_idx_shape *ishape,
                             int32_t n_seq, int32_t max_seq_len, size_t *bytes);
/* Write n_rows raw keys k_raw [n_rows][idx_dim] (F32 rounded to fp16, or F16)
 * at (seq_ids[i] or 0, pos[i]), then re-pool the block holding each row from
 * its members (written or not, as the decode update does: the block is forced
 * while partial, so its key is only read once it is whole).  A run of rows in
 * one block pools it once.  Replaces the raw-key set_rows and the one-block
 * pool update of a decode step (src/qwfn_graph.cpp:463-476; inputs
 * src/qwfn_engine.cpp:737-744). */
int qwfn_idx_append_pool(const qwfn_qsa_shape *shape, const qwfn_kv_view *view,
                         const qwfn_idx_shape *ishape, const qwfn_idx_view *iview,
                         const void *k_raw, int32_t src_dtype, const int32_t *seq_ids,
                         const int32_t *pos, int32_t n_rows, void *stream);
/* Pool blocks [0, n_whole) of sequence seq from the raw keys: the rebuild after
 * a prefill (qsa_pool_rebuild, src/qwfn_graph.cpp:431-448; src/qwfn_engine.cpp:
 * 761-798). */
int qwfn_idx_pool_rebuild(const qwfn_qsa_shape *shape, const qwfn_kv_view *view,
                          const qwfn_idx_shape *ishape, const qwfn_idx_view *iview,
                          int32_t seq, int32_t n_whole, void *stream);
/* Scores and selection of one decode token per sequence: q_idx fp32
 * [n_seq][n_idx_head][idx_dim] (RMSNorm'd and rotated by the caller, src/
 * qwfn_graph.cpp:480-484), seq_len as in qwfn_indexer_topk.  Block score =
 * dots of the heads (each over idx_dim in four strided fp32 fma chains
 * combined (c0+c1)+(c2+c3)), relu'd when relu_per_head, summed in head order;
 * the kept set follows the shape's rule; sel [n_seq][n_head_kv][max_sel] gets
 * the same ascending block ids in every row, n_sel [n_seq][n_head_kv] the
 * count.  Replaces src/qwfn_graph.cpp:477-495 and the bias window
 * (src/qwfn_engine.cpp:748-759). */
int qwfn_idx_select(const qwfn_qsa_shape *shape, const qwfn_kv_view *view,
                    const qwfn_idx_shape *ishape, const qwfn_idx_view *iview,
                    const float *q_idx, const int32_t *seq_len, int32_t n_seq,
                    int32_t max_seq_len, int32_t *sel, int32_t *n_sel, int32_t max_sel,
                    void *ws, size_t ws_bytes, void *stream);
/* One decode token of graph_builder::sparse_attn_decode with the checkpoint's
 * indexer (src/qwfn_graph.cpp:450-546): for sequence i < n_seq (at most 64)
 * at position seq_len[i]-1, the raw indexer key k_raw [n_seq][idx_dim] is
 * written and its block re-pooled (:463-476) and k_new / v_new
 * [n_seq][n_head_kv][head_dim] appended (:520-528), all in one launch; then
 * the indexer's scores and selection from q_idx as qwfn_idx_select
 * (:477-495) and the attention of q over it as qwfn_sparse_decode_attn
 * (:497-542).  src_dtype covers k_new, v_new and k_raw.  sel [n_seq]
 * [n_head_kv][max_sel] and n_sel [n_seq][n_head_kv] (required: the selection
 * passes through them) receive the selection as qwfn_idx_select writes it.
 * Workspace: qwfn_idx_workspace_bytes.  Up to 8,192 candidate blocks the
 * indexer scores (its launch also appends the rows and pools and scores the
 * block the token completes) and every attention workgroup selects from the
 * row: three launches.
 * Past 8,192 candidate blocks (the 4-token blocks past 32,768 tokens), also
 * three: 16 more workgroups of the indexer launch score 1,024 sampled blocks
 * of each row and place a cut, the scoring workgroups wait for it and keep
 * each chunk's scores above it, and the attention workgroups rank those
 * candidates exactly (a fallback over the whole row where the cut leaves too
 * few or too many), so no selection launch runs.  That covers the
 * checkpoint's heads (24 x 256, 4 indexer heads of at most 128) up to 49,152
 * blocks (an indexer of more than one KV head puts the append and the cut in a
 * launch of their own first); longer rows, other shapes and a workspace
 * smaller than qwfn_idx_workspace_bytes (at least what
 * qwfn_qsa_workspace_bytes and qwfn_idx_select each need) select in the
 * indexer's last workgroup or a selection launch, as qwfn_idx_select does.
 * Replaces the four calls qwfn_kv_append_q8_0, qwfn_idx_append_pool,
 * qwfn_idx_select and qwfn_sparse_decode_attn of a decode step (five
 * launches, six past 8,192 blocks) with three. */
int qwfn_idx_sparse_attn_decode(const qwfn_qsa_shape *shape, const qwfn_kv_view *view,
                                const qwfn_idx_shape *ishape, const qwfn_idx_view *iview,
                                const float *q, const float *q_idx, const void *k_new,
                                const void *v_new, const void *k_raw, int32_t src_dtype,
                                const int32_t *seq_len, int32_t n_seq, int32_t max_seq_len,
                                float *out, int32_t *sel, int32_t *n_sel, int32_t max_sel,
                                void *ws, size_t ws_bytes, void *stream);
/* qwfn_sparse_attn_prefill with the checkpoint's indexer: k_raw (optional,
 * with k_new / v_new) [n_q][idx_dim] is written at pos0.. and every block it
 * touches re-pooled; query i is selected by q_idx [n_q][n_idx_head][idx_dim]
 * against the indexer's pooled keys (one selection for every KV head), then
 * attends as in qwfn_sparse_attn_prefill.  Workspace: qwfn_qsa_prefill_
 * workspace_bytes of the attention shape.  Replaces qsa_top_k and the masked
 * attention of graph_builder::sparse_attn (src/qwfn_graph.cpp:233-408) and the
 * per-chunk tables of src/qwfn_engine.cpp:884-957. */
int qwfn_idx_sparse_attn_prefill(const qwfn_qsa_shape *shape, const qwfn_kv_view *view,
                                 const qwfn_idx_shape *ishape, const qwfn_idx_view *iview,
                                 const float *q, const float *q_idx, const void *k_new,
                                 const void *v_new, const void *k_raw, int32_t src_dtype,
                                 int32_t seq, int32_t pos0, int32_t n_q, float *out,
                                 int32_t *sel_out, int32_t *n_sel_out, int32_t max_sel,
                                 void *ws, size_t ws_bytes, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* QWFN_QSA_H */
