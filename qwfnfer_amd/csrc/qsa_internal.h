// qsa_internal.h -- geometry, workspace map and launcher declarations shared by
// the gfx950 kernels (qsa_kernels.hip) and the C ABI (qsa_abi.hip).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/qwfn_qsa.h"

namespace qwfn_qsa {

// Everything a kernel needs to know about the shape and the view, flattened
// into one by-value kernel argument.
struct Geo {
    int32_t H, Hkv, hd, G;           // query heads, KV heads, head dim, group
    int32_t bt, pt;                  // block tokens, page tokens
    int32_t topk, sink, local;       // selection
    int32_t relu, variant;           // indexer relu, q8_0 rounding
    int32_t shared;                  // one selection for all KV heads (scores summed in head order)
    int32_t keep_total;              // top_k counts the forced blocks (topk_counts_forced)
    int32_t kt;                      // K/V element type (QWFN_KV_*)
    int32_t round_f16;               // decode attention rounds dequantized K/V to fp16 (kv_round_f16)
    int32_t chunks;                  // 16-byte chunks in a head row of K/V (head_dim/16 for q8_0)
    int32_t sel_rows;                // rows a shared selection is written to per sequence (Hkv;
                                     // the attention's n_head_kv for the checkpoint indexer)
    int32_t pps, n_phys, n_seq_view; // pages per sequence, pool pages, view seqs
    int32_t bps;                     // pooled blocks per sequence
    int32_t vdim;                    // V quants dim-major per 64-token tile (bt % 64 == 0)
    int32_t pooled_f16;              // view.pooled holds fp16 keys (the checkpoint indexer's)
    int64_t page_bytes, qbytes;      // page size, quant bytes per page
    float inv_bt;                    // 1.0f / block_tokens (host-rounded)
    float scale_log2;                // log2(e) / sqrt(head_dim)
    // Prefill mode (pf = 1): "sequence" s of a launch is query s of cache
    // sequence pf_seq at position pf_pos0 + s, i.e. seq_len pf_pos0 + s + 1.
    int32_t pf, pf_seq, pf_pos0;
};

// Device pointers into a caller workspace (see qwfn_qsa_workspace_bytes).
// The counter region sits at a fixed offset with a fixed capacity so every
// call layout agrees on it; all other regions are per-call scratch.
constexpr int32_t kMaxCounters = 4096;   // (sequence, KV head) pairs per call
constexpr int32_t kPrefillBatchMax = 32768;   // queries per prefill batch (one grid dimension)
constexpr int32_t kVmaxWg = 64;               // partial V-scale maxima per KV head (prefill)
// Eligible blocks the indexer workgroup selects from registers; longer decode
// contexts select in a launch of their own, over kCutKeys scores per
// workgroup when at most kCutWgMax workgroups cover them.
constexpr int32_t kIdxRegKeys = 8192;
constexpr int32_t kCutKeys = 4096;
constexpr int32_t kCutWgMax = 64;
constexpr int32_t kMaxChain = 8;          // positions of one chained decode call (qwfn_sparse_attn_decode_chain)
constexpr int32_t kScoreRecBlocks = 16;   // blocks per (min, max) score record of the fused call's scoring
constexpr int32_t kIdxChunkBlocks = 64;   // blocks an indexer workgroup scores (its candidate slots)
constexpr int32_t kIdxCutSamples = 1024;  // sampled scores of a long decode row's cut
struct Ws {
    int32_t *cnt_idx;    // [kMaxCounters] indexer completion counters
    int32_t *sel;        // [n_seq][Hkv][max_sel]  selection of the fused step
    int32_t *nsel;       // [n_seq][Hkv]
    float   *scores;     // [n_seq][Hkv][nb_cap]
    float   *part_o;     // [n_seq][Hkv][n_tiles][G][hd]
    float   *part_ml;    // [n_seq][Hkv][n_tiles][G][2]
    uint2   *cand;       // [n_seq][Hkv][cut_wg][kCutKeys] (key, block) candidates of the multi-workgroup selection
    int32_t *ccnt;       // [n_seq][Hkv][kCutWgMax] their counts; past kIdxRegKeys decode blocks also
                         // [n_seq][n_chunks] the indexer workgroups' candidate counts (cand: 64 slots a chunk)
    uint32_t *cutk;      // [n_seq][Hkv][kIdxCutParts] a long decode row's cut keys (the append launch's)
    float2  *cmm;        // [n_seq][Hkv][nb_cap / kScoreRecBlocks] (min, max) eligible score of each record's blocks
                         // (the attention's own selection reads them; (+inf, -inf) when empty)
    int32_t *lens;       // [kMaxChain][n_seq] lengths of a chained call's positions
    float   *vmax;       // [Hkv][kVmaxWg] partial maxima of the V scales a prefill call reads
    float   *pnorm;      // [Hkv][nb_cap] prefill: each pooled block's key norm (the scoring bound)
    int32_t  nb_cap, max_sel, n_tiles;
    int32_t  cut_wg;     // workgroups of the multi-workgroup selection (0: one workgroup)
};

struct WsLayout {
    size_t sel, nsel, scores, part_o, part_ml, cand, ccnt, cutk, cmm, lens, vmax, pnorm, total;
    int32_t nb_cap, max_sel, n_tiles, cut_wg;
};
// partials = false: no attention partials (the prefill kernel keeps its state on chip);
// cut = false: no multi-workgroup selection regions (prefill selects per query)
WsLayout ws_layout(const Geo &g, int32_t n_seq, int32_t max_seq_len, int32_t max_sel, bool partials = true,
                   bool cut = true);
Ws ws_bind(void *base, const WsLayout &l);

// Fused-append arguments of the decode step (enabled == 0: plain indexer).
struct FusedAppend {
    const void *k_new, *v_new;       // [n_seq][Hkv][hd]
    int32_t src_f16, enabled;
};

bool kernels_for(int32_t hd, int32_t G);   // an instantiation exists

// Per-kernel timing of a decode call (qwfn_qsa_time_next_call).  While a
// kind's pair of events is armed, its next launch on this thread goes
// through hipExtLaunchKernel, which stamps the pair with that kernel's own
// begin and end, and the pair is disarmed.  A stream under capture launches
// as usual (the pair is dropped).  The decode entry points disarm whatever
// their call did not use before they return.
enum TimedKind { kTimedIndexer = 0, kTimedAttention = 1, kTimedMerge = 2, kTimedKinds = 3 };
struct KernelTimer {
    hipEvent_t ev[kTimedKinds][2];
};
extern thread_local KernelTimer g_kernel_timer;

// The armed pair of `kind` (disarming it), or false when it is unarmed or
// the stream is capturing.
inline bool take_timer(int kind, hipStream_t st, hipEvent_t *a, hipEvent_t *b) {
    hipEvent_t *e = g_kernel_timer.ev[kind];
    if (e[0] == nullptr) return false;
    *a = e[0];
    *b = e[1];
    e[0] = e[1] = nullptr;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(st, &cs) == hipSuccess && cs == hipStreamCaptureStatusNone;
}

#define QWFN_LAUNCH_SHM(kind, kern, grid, block, shm, st, ...)                        \
    do {                                                                              \
        hipEvent_t qwfn_a_, qwfn_b_;                                                  \
        if (take_timer((kind), (st), &qwfn_a_, &qwfn_b_))                             \
            hipExtLaunchKernelGGL(kern, grid, block, shm, st, qwfn_a_, qwfn_b_, 0, __VA_ARGS__); \
        else                                                                          \
            hipLaunchKernelGGL(kern, grid, block, shm, st, __VA_ARGS__);              \
    } while (0)
#define QWFN_LAUNCH(kind, kern, grid, block, st, ...) QWFN_LAUNCH_SHM(kind, kern, grid, block, 0, st, __VA_ARGS__)

// Bytes of one token's head row of K (or V) quants / values in a page.
inline int32_t kv_row_bytes(int32_t kt, int32_t hd) {
    return kt == QWFN_KV_Q4_0 ? hd / 2 : kt == QWFN_KV_F16 ? 2 * hd : hd;
}

hipError_t launch_fill_zero(void *p, size_t bytes, hipStream_t st);
// lens[k][s] = seq_len[s] + k for k < n_pos (one small launch)
hipError_t launch_chain_lens(const int32_t *seq_len, int32_t n_seq, int32_t n_pos, int32_t *lens, hipStream_t st);

// The checkpoint's own indexer keys (qwfn_idx_shape): raw fp16 keys of `dim`
// values per token, pooled per block with RMSNorm * k_norm, then the first nd
// dims rotated in pairs (i, i + nd/2) at the block's first position pos, by
// ggml's rope angle: theta_0 = (float)pos, theta_{i+1} = theta_i * theta_scale
// in fp32, theta_scale = powf(base, -2/nd) computed on the host; cos / sin of
// the fp32 angle in fp64, rounded to fp32.
constexpr int kIdxMaxPairs = 64;
struct IdxGeo {
    int32_t dim, nd;
    float eps;
    float theta_scale;
};
bool idx_kernels_for(int32_t dim);
// Rows [n_rows][dim] (fp32, rounded to nearest even, or fp16) into the raw
// cache at (seq_ids[r] or seq_const, pos[r] or pos0 + r).
hipError_t launch_idx_write(const Geo &g, const qwfn_kv_view &v, const IdxGeo &ig, uint16_t *raw,
                            const void *src, int32_t src_f16, const int32_t *seq_ids, const int32_t *pos,
                            int32_t n_rows, int32_t seq_const, int32_t pos0, hipStream_t st);
// Pool the blocks of rows (seq_ids[i] or 0, pos[i] / bt) when pos != NULL (a
// run of rows in one block pools it once), else blocks blk0 + [0, n_items) of
// sequence seq_const.
hipError_t launch_idx_pool(const Geo &g, const qwfn_kv_view &v, const IdxGeo &ig, const uint16_t *raw,
                           uint16_t *pooled, const float *k_norm, const int32_t *seq_ids, const int32_t *pos,
                           int32_t n_items, int32_t seq_const, int32_t blk0, hipStream_t st);
// Write and pool in one launch, for calls of at most 64 rows (a decode step):
// among rows with the same (sequence, position) the last one is kept.
// Rows of one k_idx_append_pool launch (a decode step of up to this many
// rows).  len (the fused decode step, k_idx_decode_append): row r is sequence
// r's at position len[r] - 1, and kv (when enabled) brings the rows' K and V,
// appended by the same launch.
constexpr int kIdxFuseRows = 64;
// The cut of a long decode row, placed by the fused decode step's append
// launch for the attention's own selection (launch_dec_selbig): q_idx
// [n_seq][n_head][dim] (fp32) scores kIdxCutSamples evenly spaced eligible
// blocks of each sequence from the pool cache, kIdxCutParts workgroups a
// sequence, and cutk[s][p] receives part p's threshold: the ceil(rs /
// kIdxCutParts)-th largest key of its samples (0, every key a candidate, when
// no cut applies).  Every key at or above their mean is a candidate (keys
// are monotone in the score, so the mean lies between the parts' estimates;
// about 3.5 topk keys at the checkpoint's shape, and the attention checks
// that there are at least topk and at most its list's capacity).  q_idx
// NULL: no cut.
constexpr int kIdxCutParts = 16;
constexpr int kIdxMaxCutHeads = 16;   // query heads * dim <= 16 * 128
// The same cut placed inside the indexer launch (launch_indexer's in_cut): per
// sequence kCutSlots slots, key + 1 (0 while unwritten), of the kIdxCutParts
// part keys and then the key of the block the token completes (the append
// workgroup's score), at the top of the counter region from kCutReadyBase.
// Every call leaves that region at zero and calls on one workspace do not
// overlap, so the slots are zero when the indexer launch starts; the attention
// launch that reads the candidates clears them again.
constexpr int kCutSlots = 32;
constexpr int kCutReadyBase = kMaxCounters - kIdxFuseRows * kCutSlots;
static_assert(kCutReadyBase >= 0, "the cut slots fit the counter region");
struct IdxCut {
    const float *q_idx;
    uint32_t *cutk;
    int32_t n_head, max_seq_len;
};
hipError_t launch_idx_append_pool(const Geo &g, const qwfn_kv_view &v, const IdxGeo &ig, uint16_t *raw,
                                  uint16_t *pooled, const float *k_norm, const void *src, int32_t src_f16,
                                  const int32_t *seq_ids, const int32_t *pos, int32_t n_rows, hipStream_t st,
                                  const FusedAppend &kv = FusedAppend{nullptr, nullptr, 0, 0},
                                  const int32_t *len = nullptr, const IdxCut &cut = IdxCut{nullptr, nullptr, 0, 0});
// seq_ids NULL: every row in seq_const; pos NULL: row r at position pos0 + r;
// len (decode): row r is sequence r's token at position len[r] - 1.
hipError_t launch_append(const Geo &g, const qwfn_kv_view &v, const void *k, const void *vv,
                         int32_t src_f16, const int32_t *seq_ids, const int32_t *pos,
                         int32_t n_rows, int32_t seq_const, int32_t pos0, hipStream_t st,
                         const int32_t *len = nullptr);
// seq_ids NULL: every block in seq_const; block_ids NULL: blocks blk0 + [0, n_blocks);
// len (decode): sequence i's block holding len[i] - 1 when that token completes it.
hipError_t launch_pool(const Geo &g, const qwfn_kv_view &v, const int32_t *seq_ids,
                       const int32_t *block_ids, int32_t n_blocks, int32_t seq_const,
                       int32_t blk0, hipStream_t st, const int32_t *len = nullptr);
// The checkpoint indexer's append workgroup inside the indexer launch (the
// fused decode step when the attention selects from the indexer's row): the
// token's K / V rows into the attention's pages (ga, va), its raw key src
// [n_seq][ig.dim] (fp16 or fp32) into the raw cache, its block re-pooled and,
// when the token completes the block, scored (idx_append_wg).
struct IdxAppend {
    Geo ga;
    qwfn_kv_view va;
    IdxGeo ig;
    FusedAppend kv;
    const void *src;
    const float *k_norm;
    uint16_t *raw;
    int32_t f16, enabled;
    uint32_t *slots;     // the in-launch cut's slots (in_cut), else NULL
    int32_t polls;       // the bound on a scoring workgroup's reads of them
};
constexpr int32_t kCutPollsDefault = 1 << 16;
// select = false: scores only (the attention selects, launch_attention_select);
// sel_launch = false: the indexer does not select and no selection launch
// follows: rows past its workgroup's registers leave each chunk's candidates
// (the attention ranks them, launch_dec_selbig), shorter rows are scored only
// (every attention workgroup selects from the row, launch_dec_selrow).
// in_cut (with sel_launch false, rows past the registers, one KV head, a local
// window): kIdxCutParts leading workgroups per sequence place the sampled cut
// into ws.cutk (the slots at kCutReadyBase) and the chunks wait for it, instead
// of reading the append launch's
hipError_t launch_indexer(const Geo &g, const qwfn_kv_view &v, const float *q,
                          const int32_t *seq_len, int32_t n_seq, int32_t max_seq_len,
                          int32_t *sel, int32_t *nsel, int32_t max_sel, const Ws &ws,
                          const FusedAppend &fa, hipStream_t st, bool select = true, bool sel_launch = true,
                          const IdxAppend *ia = nullptr, bool in_cut = false);
// Prefill: scores of n_q queries (Geo::pf) into ws.scores, then each query's
// selection into sel / nsel.
hipError_t launch_prefill_index(const Geo &g, const qwfn_kv_view &v, const float *q, int32_t n_q,
                                int32_t max_seq_len, int32_t *sel, int32_t *nsel, int32_t max_sel,
                                const Ws &ws, hipStream_t st);
// The prefill's approximate matrix-core scores alone (k_pf_approx): n_q
// queries of sequence g.pf_seq against blocks [g.sink, n_blk) of every KV
// head into scores [n_q][Hkv][nb_cap], each block's key norm (rounded up)
// into pnorm [Hkv][nb_cap].  For the test entry point that checks the
// scoring bound on the hardware.
bool pf_approx_fits_shape(int32_t hd, int32_t G);
hipError_t launch_pf_approx_scores(const Geo &g, const qwfn_kv_view &v, const float *q, int32_t n_q,
                                   int32_t n_blk, float *scores, int32_t nb_cap, float *pnorm, hipStream_t st);
// The largest q8_0 V scale of each KV head over positions [0, n_pos) of
// sequence g.pf_seq, as kVmaxWg partial maxima per head (vmax).
hipError_t launch_prefill_vmax(const Geo &g, const qwfn_kv_view &v, int32_t n_pos, float *vmax, hipStream_t st);
// Prefill attention on the matrix cores (block_tokens % 64 == 0): one wave
// per (query, KV head) over its selection, no partials; vmax from
// launch_prefill_vmax over every position the queries read.
hipError_t launch_prefill_attention(const Geo &g, const qwfn_kv_view &v, const float *q, int32_t n_q,
                                    const int32_t *sel, const int32_t *nsel, int32_t max_sel, const float *vmax,
                                    float *out, hipStream_t st);
// Decode attention that makes its own selection from the scores of a
// scores-only indexer launch, writing it to sel / nsel (the q8_0 matrix-core
// kernel for its shapes, the general kernel for the other element types and
// block sizes; per-head selections of at most 8192 eligible blocks, at most
// eight sequences, max_sel <= 1024: attn_select_fits).
bool attn_select_fits(const Geo &g, int32_t n_seq, int32_t max_seq_len, int32_t max_sel);
hipError_t launch_attention_select(const Geo &g, const qwfn_kv_view &v, const float *q, const int32_t *seq_len,
                                   int32_t n_seq, int32_t max_seq_len, int32_t *sel, int32_t *nsel,
                                   int32_t max_sel, float *out, const Ws &ws, hipStream_t st);
// Combine of the attention partials: og = sum_i w_i O_i / sum_i w_i l_i over
// the parts of tg tiles each (dense: every block below the length).
hipError_t launch_merge(const Geo &g, const qwfn_kv_view &v, const int32_t *seq_len, int32_t n_seq,
                        int32_t max_seq_len, const int32_t *nsel, int32_t max_sel, bool dense, float *out,
                        const Ws &ws, int32_t tg, hipStream_t st);
// The decode attention of q8_0 caches whose blocks are whole 64-token tiles
// (qsa_decode.hip): over a given selection (sel), dense (sel NULL), or
// selecting from the indexer's scores (select; writes sel / nsel), then the
// merge.  dec_select_fits: per-head selections of at most 8192 eligible
// blocks and 1024 selected.
bool dec_kernels_for(const Geo &g);
// q4_0 / F16 caches (qsa_decode_kv.hip): a shape with instantiations, and the
// attention with its merge, as launch_dec_attention
bool dec_kv_shape(const Geo &g);
// Prefill attention of the K layouts (q8_0 in blocks shorter than a tile,
// q4_0, F16) over a given per-query selection, one workgroup per (query, KV
// head) walking all its tiles (k_dec_loop): the normalised output, no
// partials; vmax from launch_prefill_vmax (unused for F16).  Fits: prefill
// geometry (Geo::pf) of such a shape, max_sel <= 1024.
bool dec_loop_fits(const Geo &g, int32_t max_sel);
hipError_t launch_dec_loop(const Geo &g, const qwfn_kv_view &v, const float *q, int32_t n_q, int32_t max_seq_len,
                           const int32_t *sel, const int32_t *nsel, int32_t max_sel, const float *vmax, float *out,
                           hipStream_t st);
hipError_t launch_dec_kv_loop(const Geo &g, const qwfn_kv_view &v, const float *q, int32_t n_q, int32_t max_seq_len,
                              const int32_t *sel, const int32_t *nsel, int32_t max_sel, const float *vmax, float *out,
                              hipStream_t st);
hipError_t launch_dec_kv(const Geo &g, const qwfn_kv_view &v, const float *q, const int32_t *seq_len, int32_t n_seq,
                         int32_t max_seq_len, const int32_t *sel, const int32_t *nsel, int32_t max_sel, float *out,
                         const Ws &ws, bool select, hipStream_t st);
bool dec_select_fits(const Geo &g, int32_t max_seq_len, int32_t max_sel);
hipError_t launch_dec_attention(const Geo &g, const qwfn_kv_view &v, const float *q, const int32_t *seq_len,
                                int32_t n_seq, int32_t max_seq_len, const int32_t *sel, const int32_t *nsel,
                                int32_t max_sel, float *out, const Ws &ws, bool select, hipStream_t st);
// The checkpoint's decode attention selecting for itself from the indexer's
// per-chunk candidates of each sequence's shared row (ws.cand / ws.ccnt: the
// eligible keys at or above the append launch's sampled cut; ws.scores, rows
// of ws.nb_cap, for the fallback), then the merge: every workgroup ranks the
// candidates exactly (the radix passes over the row when they number fewer
// than topk or more than its list holds) and writes the selection to sel /
// nsel.  Fits: q8_0 blocks shorter than a tile at head_dim 256 and group 12,
// a shared selection, rows up to 49,152 blocks, max_sel <= 1024.
bool dec_selbig_fits(const Geo &g, int32_t max_seq_len, int32_t max_sel);
bool dec_selrow_fits(const Geo &g, int32_t max_seq_len, int32_t max_sel);
hipError_t launch_dec_selrow(const Geo &g, const qwfn_kv_view &v, const float *q, const int32_t *seq_len,
                             int32_t n_seq, int32_t max_seq_len, int32_t *sel, int32_t *nsel, int32_t max_sel,
                             float *out, const Ws &ws, hipStream_t st);
hipError_t launch_dec_selbig(const Geo &g, const qwfn_kv_view &v, const float *q, const int32_t *seq_len,
                             int32_t n_seq, int32_t max_seq_len, int32_t *sel, int32_t *nsel, int32_t max_sel,
                             float *out, const Ws &ws, hipStream_t st);
// That selection alone over given score rows (rows of nb_cap), one workgroup
// a sequence: the test entry point's.
hipError_t launch_test_select_big(const Geo &g, const float *scores, int32_t nb_cap, const int32_t *seq_len,
                                  int32_t n_seq, int32_t max_seq_len, int32_t *sel, int32_t *nsel, int32_t max_sel,
                                  hipStream_t st);
hipError_t launch_attention(const Geo &g, const qwfn_kv_view &v, const float *q,
                            const int32_t *seq_len, int32_t n_seq, int32_t max_seq_len,
                            const int32_t *sel, const int32_t *nsel, int32_t max_sel,
                            float *out, const Ws &ws, hipStream_t st);
// Positions pos0 .. pos0+n-1 of sequence seq between the paged layout and the
// reference's token-major block_q8_0 rows (to_rows: export; else import).
hipError_t launch_kv_rows(const Geo &g, const qwfn_kv_view &v, bool to_rows, int32_t seq, int32_t pos0,
                          int32_t n, void *k_rows, void *v_rows, hipStream_t st);
hipError_t launch_gather(const Geo &g, const qwfn_kv_view &v, const int32_t *seq_len,
                         int32_t n_seq, const int32_t *sel, const int32_t *nsel,
                         int32_t max_sel, float *k_out, float *v_out, int32_t *cells,
                         hipStream_t st);

}  // namespace qwfn_qsa
