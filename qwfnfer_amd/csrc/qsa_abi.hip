// qsa_abi.hip -- the extern "C" boundary of libqwfn_qsa.so: host-side
// validation, workspace layout and kernel dispatch.  No allocation, no
// synchronisation (except qwfn_qsa_read_status), no exceptions across the ABI.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include "qsa_internal.h"

using namespace qwfn_qsa;

thread_local KernelTimer qwfn_qsa::g_kernel_timer{};

namespace {

thread_local std::string g_err;

// The bound on the in-launch cut's polls of the checkpoint decode calls that
// start after it is set (qwfn_qsa_test_set_cut_polls).
std::atomic<int32_t> g_cut_polls{kCutPollsDefault};

// Disarms, on return from a decode entry point, the kernel timing its call
// did not use (qwfn_qsa_time_next_call arms it for one call only).
struct TimerDisarm {
    ~TimerDisarm() { g_kernel_timer = KernelTimer{}; }
};

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int ok() {
    g_err.clear();
    return QWFN_OK;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(QWFN_EHIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned(const void *p, size_t a) { return ((uintptr_t)p % a) == 0; }

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

int check_shape(const qwfn_qsa_shape *s) {
    if (!s) return fail(QWFN_EINVAL, "shape is NULL");
    if (s->n_head_kv < 1 || s->n_head < s->n_head_kv || s->n_head % s->n_head_kv)
        return fail(QWFN_EINVAL, "n_head (%d) must be a positive multiple of n_head_kv (%d)",
                    s->n_head, s->n_head_kv);
    if (s->head_dim < 32 || s->head_dim % 32)
        return fail(QWFN_EINVAL, "head_dim (%d) must be a positive multiple of 32 (q8_0 block)", s->head_dim);
    if (s->page_tokens < 64 || s->page_tokens % 64)
        return fail(QWFN_EINVAL, "page_tokens (%d) must be a positive multiple of 64", s->page_tokens);
    if (s->block_tokens < 1 || s->page_tokens % s->block_tokens)
        return fail(QWFN_EINVAL, "block_tokens (%d) must divide page_tokens (%d)", s->block_tokens,
                    s->page_tokens);
    if (s->sink_blocks < 0) return fail(QWFN_EINVAL, "sink_blocks (%d) < 0", s->sink_blocks);
    if (s->local_tokens < 0) return fail(QWFN_EINVAL, "local_tokens (%d) < 0", s->local_tokens);
    if (s->quant_variant != QWFN_Q8_X86_RNE && s->quant_variant != QWFN_Q8_REF_ROUNDF)
        return fail(QWFN_EINVAL, "quant_variant %d unknown", s->quant_variant);
    if (s->kv_type != QWFN_KV_Q8_0 && s->kv_type != QWFN_KV_Q4_0 && s->kv_type != QWFN_KV_F16)
        return fail(QWFN_EINVAL, "kv_type %d unknown", s->kv_type);
    if ((s->relu_per_head | s->shared_selection | s->topk_counts_forced | s->kv_round_f16) & ~1)
        return fail(QWFN_EINVAL, "relu_per_head / shared_selection / topk_counts_forced / kv_round_f16 are 0 or 1");
    if (s->topk_counts_forced && s->top_k_blocks > 0 &&
        s->top_k_blocks < s->sink_blocks + (s->local_tokens + s->block_tokens - 2) / s->block_tokens + 1)
        return fail(QWFN_EINVAL, "topk_counts_forced: top_k_blocks (%d) must hold the sink and window blocks",
                    s->top_k_blocks);
    const int G = s->n_head / s->n_head_kv;
    if (!kernels_for(s->head_dim, G))
        return fail(QWFN_ENOTSUP, "no kernel instantiation for head_dim %d, group %d", s->head_dim, G);
    return QWFN_OK;
}

int check_view(const qwfn_qsa_shape *s, const qwfn_kv_view *v) {
    if (!v) return fail(QWFN_EINVAL, "view is NULL");
    if (!v->k_pages || !v->v_pages || !v->pooled || !v->page_table)
        return fail(QWFN_EINVAL, "view has a NULL k_pages / v_pages / pooled / page_table");
    if (!aligned(v->k_pages, 16) || !aligned(v->v_pages, 16) || !aligned(v->pooled, 16))
        return fail(QWFN_EINVAL, "k_pages, v_pages and pooled must be 16-byte aligned");
    if (v->n_seq < 1 || v->pages_per_seq < 1 || v->n_phys_pages < 1)
        return fail(QWFN_EINVAL, "view n_seq / pages_per_seq / n_phys_pages must be >= 1");
    if ((int64_t)v->pages_per_seq * s->page_tokens > INT32_MAX / 2)
        return fail(QWFN_ERANGE, "pages_per_seq * page_tokens overflows the position range");
    return QWFN_OK;
}

// view_required: the call operates on a cache, so a NULL view is an error.
int make_geo(const qwfn_qsa_shape *s, const qwfn_kv_view *v, Geo *g, bool view_required = true) {
    int rc = check_shape(s);
    if (rc) return rc;
    if (view_required && !v) return fail(QWFN_EINVAL, "view is NULL");
    if (v && (rc = check_view(s, v))) return rc;
    g->H = s->n_head; g->Hkv = s->n_head_kv; g->hd = s->head_dim; g->G = s->n_head / s->n_head_kv;
    g->bt = s->block_tokens; g->pt = s->page_tokens;
    g->topk = s->top_k_blocks > 0 ? s->top_k_blocks : 0;
    g->sink = s->sink_blocks; g->local = s->local_tokens;
    g->relu = s->relu_per_head; g->variant = s->quant_variant; g->shared = s->shared_selection;
    g->keep_total = s->topk_counts_forced;
    g->sel_rows = s->n_head_kv;
    g->kt = s->kv_type;
    g->round_f16 = s->kv_round_f16;
    g->chunks = kv_row_bytes(s->kv_type, s->head_dim) / 16;
    g->qbytes = (int64_t)s->n_head_kv * s->page_tokens * kv_row_bytes(s->kv_type, s->head_dim);
    g->page_bytes = g->qbytes +
                    (s->kv_type == QWFN_KV_F16 ? 0 : (int64_t)s->n_head_kv * s->page_tokens * (s->head_dim / 32) * 2);
    g->inv_bt = 1.0f / (float)s->block_tokens;
    // the matrix-core kernels read q8_0 (V dim-major per 64-token tile); other
    // element types run the general kernels over the K layout
    g->vdim = s->block_tokens % 64 == 0 && s->kv_type == QWFN_KV_Q8_0;
    g->scale_log2 = (float)(1.4426950408889634 / std::sqrt((double)s->head_dim));
    g->pf = 0; g->pf_seq = 0; g->pf_pos0 = 0;
    g->pooled_f16 = 0;
    if (v) {
        g->pps = v->pages_per_seq; g->n_phys = v->n_phys_pages; g->n_seq_view = v->n_seq;
        g->bps = (int32_t)((int64_t)v->pages_per_seq * s->page_tokens / s->block_tokens);
    } else {
        g->pps = g->n_phys = g->n_seq_view = g->bps = 0;
    }
    return QWFN_OK;
}

int32_t max_selected(const qwfn_qsa_shape *s, int32_t max_seq_len) {
    const int32_t bt = s->block_tokens, all = (max_seq_len + bt - 1) / bt;
    if (s->top_k_blocks <= 0) return all;
    const int32_t win = (s->local_tokens + bt - 2) / bt + 1;
    const int64_t cap = (int64_t)s->top_k_blocks + s->sink_blocks + win;
    return cap < all ? (int32_t)cap : all;
}

// Common checks of the per-call sequence arguments.
int check_batch(const qwfn_qsa_shape *s, const qwfn_kv_view *v, int32_t n_seq, int32_t max_seq_len) {
    if (n_seq < 1 || n_seq > v->n_seq)
        return fail(QWFN_EINVAL, "n_seq %d outside [1, view n_seq %d]", n_seq, v->n_seq);
    if ((int64_t)n_seq * s->n_head_kv > kMaxCounters)
        return fail(QWFN_ERANGE, "n_seq * n_head_kv = %lld exceeds %d per call",
                    (long long)n_seq * s->n_head_kv, kMaxCounters);
    if (max_seq_len < 1) return fail(QWFN_EINVAL, "max_seq_len %d < 1", max_seq_len);
    if ((int64_t)max_seq_len > (int64_t)v->pages_per_seq * s->page_tokens)
        return fail(QWFN_ERANGE, "context exhausted: max_seq_len %d > capacity %lld", max_seq_len,
                    (long long)v->pages_per_seq * s->page_tokens);
    return QWFN_OK;
}

int bind_ws(const Geo &g, int32_t n_seq, int32_t max_seq_len, int32_t max_sel, void *ws,
            size_t ws_bytes, Ws *out) {
    const WsLayout l = ws_layout(g, n_seq, max_seq_len, max_sel);
    if (!ws) return fail(QWFN_EINVAL, "workspace is NULL");
    if (!aligned(ws, 256)) return fail(QWFN_EINVAL, "workspace must be 256-byte aligned");
    if (ws_bytes < l.total)
        return fail(QWFN_ERANGE, "workspace of %zu bytes < %zu needed for n_seq %d, max_seq_len %d",
                    ws_bytes, l.total, n_seq, max_seq_len);
    *out = ws_bind(ws, l);
    return QWFN_OK;
}

}  // namespace

namespace qwfn_qsa {

WsLayout ws_layout(const Geo &g, int32_t n_seq, int32_t max_seq_len, int32_t max_sel, bool partials, bool cut) {
    WsLayout l;
    // per-pair score rows padded to 64 floats: 16-byte vector loads of a row
    // stay aligned and inside it
    l.nb_cap = (int32_t)((((int64_t)(max_seq_len / g.bt > 0 ? max_seq_len / g.bt : 1)) + 63) / 64 * 64);
    l.max_sel = max_sel;
    l.n_tiles = (int32_t)(((int64_t)max_sel * g.bt + 63) / 64);
    const size_t pairs = (size_t)n_seq * g.Hkv;
    size_t off = align256((size_t)kMaxCounters * sizeof(int32_t));
    auto take = [&](size_t bytes) { const size_t o = off; off = align256(off + bytes); return o; };
    l.sel = take(pairs * max_sel * sizeof(int32_t));
    l.nsel = take(pairs * sizeof(int32_t));
    l.scores = take(pairs * l.nb_cap * sizeof(float));
    l.part_o = take(partials ? pairs * l.n_tiles * g.G * g.hd * sizeof(float) : 0);
    l.part_ml = take(partials ? pairs * l.n_tiles * g.G * 2 * sizeof(float) : 0);
    // the multi-workgroup selection: decode contexts past the register
    // selection, per-head or over one score row
    const int32_t nb_max = max_seq_len / g.bt;
    const int32_t cut_wg = (nb_max + kCutKeys - 1) / kCutKeys;
    l.cut_wg = cut && nb_max > kIdxRegKeys && !(g.shared && g.Hkv > 1) && cut_wg <= kCutWgMax ? cut_wg : 0;
    // ... and the per-chunk candidates of a long row's indexer workgroups
    // (the attention then selects from them, launch_dec_selbig)
    const int64_t n_chunks = (nb_max + kIdxChunkBlocks - 1) / kIdxChunkBlocks;
    const bool chunks = cut && nb_max > kIdxRegKeys;
    l.cand = take(pairs * std::max<int64_t>((int64_t)l.cut_wg * kCutKeys, chunks ? n_chunks * kIdxChunkBlocks : 0) *
                  sizeof(uint2));
    l.ccnt = take(l.cut_wg || chunks ? pairs * std::max<int64_t>(kCutWgMax, chunks ? n_chunks : 0) * sizeof(int32_t)
                                     : 0);
    l.cutk = take(chunks ? pairs * kIdxCutParts * sizeof(uint32_t) : 0);
    l.cmm = take(partials ? pairs * (l.nb_cap / kScoreRecBlocks) * sizeof(float2) : 0);
    l.lens = take((size_t)kMaxChain * n_seq * sizeof(int32_t));
    // prefill layouts (cut = false): the V-scale maxima of the matrix-core
    // attention (partials = false) and the pooled keys' norms of the scoring
    l.vmax = take(!cut && !partials ? (size_t)g.Hkv * kVmaxWg * sizeof(float) : 0);
    l.pnorm = take(!cut ? (size_t)g.Hkv * l.nb_cap * sizeof(float) : 0);
    l.total = off;
    return l;
}

Ws ws_bind(void *base, const WsLayout &l) {
    uint8_t *b = (uint8_t *)base;
    Ws w;
    w.cnt_idx = (int32_t *)b;
    w.sel = (int32_t *)(b + l.sel);
    w.nsel = (int32_t *)(b + l.nsel);
    w.scores = (float *)(b + l.scores);
    w.part_o = (float *)(b + l.part_o);
    w.part_ml = (float *)(b + l.part_ml);
    w.cand = (uint2 *)(b + l.cand);
    w.ccnt = (int32_t *)(b + l.ccnt);
    w.cutk = (uint32_t *)(b + l.cutk);
    w.cmm = (float2 *)(b + l.cmm);
    w.lens = (int32_t *)(b + l.lens);
    w.vmax = (float *)(b + l.vmax);
    w.pnorm = (float *)(b + l.pnorm);
    w.cut_wg = l.cut_wg;
    w.nb_cap = l.nb_cap;
    w.max_sel = l.max_sel;
    w.n_tiles = l.n_tiles;
    return w;
}

}  // namespace qwfn_qsa

extern "C" {

int qwfn_qsa_abi_version(void) { return QWFN_QSA_ABI_VERSION; }

const char *qwfn_qsa_last_error(void) { return g_err.c_str(); }

int qwfn_qsa_time_next_call(void *const events[6]) {
    g_kernel_timer = KernelTimer{};
    if (!events) return ok();
    for (int k = 0; k < kTimedKinds; ++k)
        if ((events[2 * k] == nullptr) != (events[2 * k + 1] == nullptr))
            return fail(QWFN_EINVAL, "time_next_call: kernel %d has a start event without a stop event, or "
                                     "the reverse", k);
    for (int k = 0; k < kTimedKinds; ++k) {
        g_kernel_timer.ev[k][0] = (hipEvent_t)events[2 * k];
        g_kernel_timer.ev[k][1] = (hipEvent_t)events[2 * k + 1];
    }
    return ok();
}

int qwfn_qsa_test_prefill_scores(const qwfn_qsa_shape *shape, const qwfn_kv_view *view, const float *q,
                                 int32_t n_q, int32_t seq, int32_t n_blk, float *scores, float *pnorm,
                                 int32_t nb_cap, void *stream) {
    Geo g;
    int rc = make_geo(shape, view, &g);
    if (rc) return rc;
    if (!pf_approx_fits_shape(g.hd, g.G))
        return fail(QWFN_ENOTSUP, "test_prefill_scores: no matrix-core scoring for head_dim %d, group %d", g.hd,
                    g.G);
    if (seq < 0 || seq >= view->n_seq) return fail(QWFN_EINVAL, "test_prefill_scores: seq %d outside the view", seq);
    if (n_q < 1 || !q || !aligned(q, 16) || !scores || !pnorm)
        return fail(QWFN_EINVAL, "test_prefill_scores: n_q < 1, NULL or misaligned q, NULL scores / pnorm");
    if (n_blk <= g.sink || n_blk > g.bps || nb_cap < n_blk)
        return fail(QWFN_ERANGE, "test_prefill_scores: n_blk %d outside (sink %d, %d] or above nb_cap %d", n_blk,
                    g.sink, g.bps, nb_cap);
    g.pf = 1;
    g.pf_seq = seq;
    const hipError_t e = launch_pf_approx_scores(g, *view, q, n_q, n_blk, scores, nb_cap, pnorm, (hipStream_t)stream);
    return e == hipSuccess ? ok() : hip_fail(e, "test_prefill_scores");
}

int qwfn_qsa_test_set_cut_polls(int32_t polls, int32_t *previous) {
    if (polls < 0) return fail(QWFN_EINVAL, "test_set_cut_polls: negative bound %d", polls);
    const int32_t old = g_cut_polls.exchange(polls);
    if (previous) *previous = old;
    return ok();
}

int qwfn_qsa_test_select_rows(const qwfn_qsa_shape *shape, const float *scores, int32_t nb_cap,
                              const int32_t *seq_len, int32_t n_seq, int32_t max_seq_len, int32_t *sel,
                              int32_t *n_sel, int32_t max_sel, void *stream) {
    Geo g;
    int rc = make_geo(shape, nullptr, &g, false);
    if (rc) return rc;
    if (!scores || !aligned(scores, 16) || !seq_len || !sel || !n_sel || n_seq < 1)
        return fail(QWFN_EINVAL, "test_select_rows: NULL or misaligned scores (16), NULL seq_len / sel / n_sel, "
                    "or n_seq < 1");
    if (max_seq_len < 1 || nb_cap % 4 || nb_cap < max_seq_len / g.bt + 4)
        return fail(QWFN_ERANGE, "test_select_rows: nb_cap %d not a multiple of 4 or below max_seq_len / "
                    "block_tokens + 4", nb_cap);
    const int32_t need = max_selected(shape, max_seq_len);
    if (max_sel < need || max_sel > 1024)
        return fail(QWFN_ERANGE, "test_select_rows: max_sel %d outside [%d, 1024]", max_sel, need);
    const hipError_t e = launch_test_select_big(g, scores, nb_cap, seq_len, n_seq, max_seq_len, sel, n_sel, max_sel,
                                                (hipStream_t)stream);
    if (e == hipErrorInvalidValue)
        return fail(QWFN_ERANGE, "test_select_rows: a row of max_seq_len %d is longer than the selection holds",
                    max_seq_len);
    return e == hipSuccess ? ok() : hip_fail(e, "test_select_rows");
}

int qwfn_qsa_check_shape(const qwfn_qsa_shape *shape) {
    const int rc = check_shape(shape);
    return rc ? rc : ok();
}

int qwfn_qsa_page_bytes(const qwfn_qsa_shape *shape, size_t *bytes) {
    Geo g;
    int rc = make_geo(shape, nullptr, &g, false);
    if (rc) return rc;
    if (!bytes) return fail(QWFN_EINVAL, "bytes is NULL");
    *bytes = (size_t)g.page_bytes;
    return ok();
}

int qwfn_qsa_pooled_bytes(const qwfn_qsa_shape *shape, int32_t n_seq, int32_t pages_per_seq,
                          size_t *bytes) {
    int rc = check_shape(shape);
    if (rc) return rc;
    if (!bytes || n_seq < 1 || pages_per_seq < 1)
        return fail(QWFN_EINVAL, "pooled_bytes: bytes NULL or n_seq / pages_per_seq < 1");
    const size_t bps = (size_t)pages_per_seq * shape->page_tokens / shape->block_tokens;
    *bytes = (size_t)n_seq * shape->n_head_kv * bps * shape->head_dim * sizeof(float);
    return ok();
}

int qwfn_qsa_max_selected(const qwfn_qsa_shape *shape, int32_t max_seq_len, int32_t *max_sel) {
    int rc = check_shape(shape);
    if (rc) return rc;
    if (!max_sel || max_seq_len < 1) return fail(QWFN_EINVAL, "max_selected: max_sel NULL or max_seq_len < 1");
    *max_sel = max_selected(shape, max_seq_len);
    return ok();
}

int qwfn_qsa_workspace_bytes(const qwfn_qsa_shape *shape, int32_t n_seq, int32_t max_seq_len,
                             size_t *bytes) {
    Geo g;
    int rc = make_geo(shape, nullptr, &g, false);
    if (rc) return rc;
    if (!bytes || n_seq < 1 || max_seq_len < 1)
        return fail(QWFN_EINVAL, "workspace_bytes: bytes NULL or n_seq / max_seq_len < 1");
    if ((int64_t)n_seq * shape->n_head_kv > kMaxCounters)
        return fail(QWFN_ERANGE, "n_seq * n_head_kv exceeds %d", kMaxCounters);
    *bytes = ws_layout(g, n_seq, max_seq_len, max_selected(shape, max_seq_len)).total;
    return ok();
}

int qwfn_qsa_workspace_init(void *ws, size_t ws_bytes, void *stream) {
    if (!ws || !aligned(ws, 256)) return fail(QWFN_EINVAL, "workspace NULL or not 256-byte aligned");
    const hipError_t e = launch_fill_zero(ws, ws_bytes, (hipStream_t)stream);
    return e == hipSuccess ? ok() : hip_fail(e, "workspace_init");
}

int qwfn_qsa_read_status(const qwfn_kv_view *view, int32_t *status, void *stream) {
    if (!view || !status) return fail(QWFN_EINVAL, "read_status: NULL view or status");
    if (!view->status) { *status = 0; return ok(); }
    hipStream_t st = (hipStream_t)stream;
    hipError_t e = hipMemcpyAsync(status, view->status, sizeof(int32_t), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e == hipSuccess) e = launch_fill_zero(view->status, sizeof(int32_t), st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return e == hipSuccess ? ok() : hip_fail(e, "read_status");
}

int qwfn_kv_append_q8_0(const qwfn_qsa_shape *shape, const qwfn_kv_view *view, const void *k_src,
                        const void *v_src, int32_t src_dtype, const int32_t *seq_ids,
                        const int32_t *pos, int32_t n_rows, void *stream) {
    Geo g;
    int rc = make_geo(shape, view, &g);
    if (rc) return rc;
    if (src_dtype != QWFN_SRC_F32 && src_dtype != QWFN_SRC_F16)
        return fail(QWFN_EINVAL, "src_dtype %d unknown", src_dtype);
    if (!k_src || !v_src || !pos) return fail(QWFN_EINVAL, "append: NULL k_src / v_src / pos");
    const size_t al = src_dtype == QWFN_SRC_F32 ? 16 : 8;
    if (!aligned(k_src, al) || !aligned(v_src, al))
        return fail(QWFN_EINVAL, "append: source rows must be %zu-byte aligned", al);
    if (n_rows < 1) return fail(QWFN_EINVAL, "append: n_rows %d < 1", n_rows);
    const hipError_t e = launch_append(g, *view, k_src, v_src, src_dtype == QWFN_SRC_F16, seq_ids, pos,
                                       n_rows, 0, 0, (hipStream_t)stream);
    return e == hipSuccess ? ok() : hip_fail(e, "append");
}

int qwfn_kv_row_bytes(const qwfn_qsa_shape *shape, size_t *bytes) {
    Geo g;
    int rc = make_geo(shape, nullptr, &g, false);
    if (rc) return rc;
    if (!bytes) return fail(QWFN_EINVAL, "bytes is NULL");
    // ggml's row of the cache type: block_q8_0 34 B, block_q4_0 18 B per 32
    // values; fp16 2 B per value
    *bytes = g.kt == QWFN_KV_F16 ? (size_t)g.Hkv * g.hd * 2u
                                 : (size_t)g.Hkv * (size_t)(g.hd / 32) * (g.kt == QWFN_KV_Q4_0 ? 18u : 34u);
    return ok();
}

static int kv_rows(const char *what, bool to_rows, const qwfn_qsa_shape *shape, const qwfn_kv_view *view,
                   int32_t seq, int32_t pos0, int32_t n_tokens, const void *k_rows, const void *v_rows,
                   void *stream) {
    Geo g;
    int rc = make_geo(shape, view, &g);
    if (rc) return rc;
    if (!k_rows && !v_rows) return fail(QWFN_EINVAL, "%s: k_rows and v_rows are both NULL", what);
    if (!aligned(k_rows, 2) || !aligned(v_rows, 2)) return fail(QWFN_EINVAL, "%s: rows must be 2-byte aligned", what);
    if (seq < 0 || seq >= view->n_seq) return fail(QWFN_EINVAL, "%s: seq %d outside the view", what, seq);
    if (pos0 < 0 || n_tokens < 1) return fail(QWFN_EINVAL, "%s: pos0 %d < 0 or n_tokens %d < 1", what, pos0, n_tokens);
    const int64_t end = (int64_t)pos0 + n_tokens;
    if (end > (int64_t)view->pages_per_seq * shape->page_tokens)
        return fail(QWFN_ERANGE, "%s: pos0 + n_tokens = %lld > capacity %lld", what, (long long)end,
                    (long long)view->pages_per_seq * shape->page_tokens);
    const hipError_t e = launch_kv_rows(g, *view, to_rows, seq, pos0, n_tokens, const_cast<void *>(k_rows),
                                        const_cast<void *>(v_rows), (hipStream_t)stream);
    return e == hipSuccess ? ok() : hip_fail(e, what);
}

int qwfn_kv_export_q8_0(const qwfn_qsa_shape *shape, const qwfn_kv_view *view, int32_t seq, int32_t pos0,
                        int32_t n_tokens, void *k_rows, void *v_rows, void *stream) {
    return kv_rows("kv_export", true, shape, view, seq, pos0, n_tokens, k_rows, v_rows, stream);
}

int qwfn_kv_import_q8_0(const qwfn_qsa_shape *shape, const qwfn_kv_view *view, int32_t seq, int32_t pos0,
                        int32_t n_tokens, const void *k_rows, const void *v_rows, void *stream) {
    return kv_rows("kv_import", false, shape, view, seq, pos0, n_tokens, k_rows, v_rows, stream);
}

int qwfn_pool_update(const qwfn_qsa_shape *shape, const qwfn_kv_view *view, const int32_t *seq_ids,
                     const int32_t *block_ids, int32_t n_blocks, void *stream) {
    Geo g;
    int rc = make_geo(shape, view, &g);
    if (rc) return rc;
    if (!block_ids) return fail(QWFN_EINVAL, "pool_update: block_ids is NULL");
    if (n_blocks < 1) return fail(QWFN_EINVAL, "pool_update: n_blocks %d < 1", n_blocks);
    if (g.hd > 256) return fail(QWFN_ENOTSUP, "pool_update: head_dim > 256");
    const hipError_t e = launch_pool(g, *view, seq_ids, block_ids, n_blocks, 0, 0, (hipStream_t)stream);
    return e == hipSuccess ? ok() : hip_fail(e, "pool_update");
}

int qwfn_pool_rebuild(const qwfn_qsa_shape *shape, const qwfn_kv_view *view, int32_t seq,
                      int32_t n_whole, void *stream) {
    Geo g;
    int rc = make_geo(shape, view, &g);
    if (rc) return rc;
    if (seq < 0 || seq >= view->n_seq) return fail(QWFN_EINVAL, "pool_rebuild: seq %d outside the view", seq);
    if (n_whole < 0) return fail(QWFN_EINVAL, "pool_rebuild: n_whole %d < 0", n_whole);
    if (n_whole > g.bps) return fail(QWFN_ERANGE, "pool_rebuild: n_whole %d > %d blocks", n_whole, g.bps);
    if (n_whole == 0) return ok();
    const hipError_t e = launch_pool(g, *view, nullptr, nullptr, n_whole, seq, 0, (hipStream_t)stream);
    return e == hipSuccess ? ok() : hip_fail(e, "pool_rebuild");
}

int qwfn_indexer_topk(const qwfn_qsa_shape *shape, const qwfn_kv_view *view, const float *q,
                      const int32_t *seq_len, int32_t n_seq, int32_t max_seq_len, int32_t *sel,
                      int32_t *n_sel, int32_t max_sel, void *ws, size_t ws_bytes, void *stream) {
    Geo g;
    int rc = make_geo(shape, view, &g);
    if (rc) return rc;
    if ((rc = check_batch(shape, view, n_seq, max_seq_len))) return rc;
    if (!q || !aligned(q, 16) || !seq_len || !sel || !n_sel)
        return fail(QWFN_EINVAL, "indexer_topk: NULL q / seq_len / sel / n_sel or q not 16-byte aligned");
    const int32_t need = max_selected(shape, max_seq_len);
    if (max_sel < need) return fail(QWFN_ERANGE, "indexer_topk: max_sel %d < %d", max_sel, need);
    Ws w;
    if ((rc = bind_ws(g, n_seq, max_seq_len, need, ws, ws_bytes, &w))) return rc;
    const FusedAppend fa{nullptr, nullptr, 0, 0};
    const hipError_t e = launch_indexer(g, *view, q, seq_len, n_seq, max_seq_len, sel, n_sel, max_sel, w,
                                        fa, (hipStream_t)stream);
    return e == hipSuccess ? ok() : hip_fail(e, "indexer_topk");
}

int qwfn_gather_dequant(const qwfn_qsa_shape *shape, const qwfn_kv_view *view,
                        const int32_t *seq_len, int32_t n_seq, const int32_t *sel,
                        const int32_t *n_sel, int32_t max_sel, float *k_out, float *v_out,
                        int32_t *cells, void *stream) {
    Geo g;
    int rc = make_geo(shape, view, &g);
    if (rc) return rc;
    if (n_seq < 1 || n_seq > view->n_seq) return fail(QWFN_EINVAL, "gather: n_seq %d outside the view", n_seq);
    if (!seq_len || !k_out || !v_out || !cells || (sel && !n_sel) || max_sel < 1)
        return fail(QWFN_EINVAL, "gather: NULL argument or max_sel < 1");
    if (g.hd > 256) return fail(QWFN_ENOTSUP, "gather: head_dim > 256");
    const hipError_t e = launch_gather(g, *view, seq_len, n_seq, sel, n_sel, max_sel, k_out, v_out, cells,
                                       (hipStream_t)stream);
    return e == hipSuccess ? ok() : hip_fail(e, "gather");
}

int qwfn_sparse_decode_attn(const qwfn_qsa_shape *shape, const qwfn_kv_view *view, const float *q,
                            const int32_t *seq_len, int32_t n_seq, int32_t max_seq_len,
                            const int32_t *sel, const int32_t *n_sel, int32_t max_sel, float *out,
                            void *ws, size_t ws_bytes, void *stream) {
    TimerDisarm disarm;
    Geo g;
    int rc = make_geo(shape, view, &g);
    if (rc) return rc;
    if ((rc = check_batch(shape, view, n_seq, max_seq_len))) return rc;
    if (!q || !aligned(q, 16) || !seq_len || !out || (sel && !n_sel))
        return fail(QWFN_EINVAL, "decode_attn: NULL q / seq_len / out (or sel without n_sel), or q misaligned");
    int32_t msel;
    if (sel) {
        if (max_sel < 1) return fail(QWFN_EINVAL, "decode_attn: max_sel %d < 1", max_sel);
        msel = max_sel;
    } else {
        msel = (max_seq_len + g.bt - 1) / g.bt;       // dense: every block below seq_len
    }
    Ws w;
    if ((rc = bind_ws(g, n_seq, max_seq_len, msel, ws, ws_bytes, &w))) return rc;
    const hipError_t e = launch_attention(g, *view, q, seq_len, n_seq, max_seq_len, sel, n_sel, msel, out,
                                          w, (hipStream_t)stream);
    return e == hipSuccess ? ok() : hip_fail(e, "decode_attn");
}

int qwfn_decode_append_select(const qwfn_qsa_shape *shape, const qwfn_kv_view *view, const float *q,
                              const void *k_new, const void *v_new, int32_t src_dtype,
                              const int32_t *seq_len, int32_t n_seq, int32_t max_seq_len, int32_t *sel,
                              int32_t *n_sel, int32_t max_sel, void *ws, size_t ws_bytes, void *stream) {
    TimerDisarm disarm;
    Geo g;
    int rc = make_geo(shape, view, &g);
    if (rc) return rc;
    if ((rc = check_batch(shape, view, n_seq, max_seq_len))) return rc;
    if (src_dtype != QWFN_SRC_F32 && src_dtype != QWFN_SRC_F16)
        return fail(QWFN_EINVAL, "src_dtype %d unknown", src_dtype);
    const size_t al = src_dtype == QWFN_SRC_F32 ? 16 : 8;
    if (!q || !aligned(q, 16) || !k_new || !v_new || !aligned(k_new, al) || !aligned(v_new, al) ||
        !seq_len || !sel || !n_sel)
        return fail(QWFN_EINVAL, "append_select: NULL or misaligned q / k_new / v_new / seq_len / sel / n_sel");
    const int32_t need = max_selected(shape, max_seq_len);
    if (max_sel < need) return fail(QWFN_ERANGE, "append_select: max_sel %d < %d", max_sel, need);
    Ws w;
    if ((rc = bind_ws(g, n_seq, max_seq_len, need, ws, ws_bytes, &w))) return rc;
    const FusedAppend fa{k_new, v_new, src_dtype == QWFN_SRC_F16, 1};
    const hipError_t e = launch_indexer(g, *view, q, seq_len, n_seq, max_seq_len, sel, n_sel, max_sel, w, fa,
                                        (hipStream_t)stream);
    return e == hipSuccess ? ok() : hip_fail(e, "append_select");
}


int qwfn_sparse_attn_decode(const qwfn_qsa_shape *shape, const qwfn_kv_view *view, const float *q,
                            const void *k_new, const void *v_new, int32_t src_dtype,
                            const int32_t *seq_len, int32_t n_seq, int32_t max_seq_len, float *out,
                            int32_t *sel_out, int32_t *n_sel_out, void *ws, size_t ws_bytes,
                            void *stream) {
    return qwfn_sparse_attn_decode_chain(shape, view, q, k_new, v_new, src_dtype, seq_len, n_seq, 1, max_seq_len,
                                         out, sel_out, n_sel_out, ws, ws_bytes, stream);
}

int qwfn_sparse_attn_decode_chain(const qwfn_qsa_shape *shape, const qwfn_kv_view *view, const float *q,
                                  const void *k_new, const void *v_new, int32_t src_dtype,
                                  const int32_t *seq_len, int32_t n_seq, int32_t n_pos, int32_t max_seq_len,
                                  float *out, int32_t *sel_out, int32_t *n_sel_out, void *ws, size_t ws_bytes,
                                  void *stream) {
    TimerDisarm disarm;
    Geo g;
    int rc = make_geo(shape, view, &g);
    if (rc) return rc;
    if ((rc = check_batch(shape, view, n_seq, max_seq_len))) return rc;
    if (n_pos < 1 || n_pos > kMaxChain) return fail(QWFN_EINVAL, "decode: n_pos %d outside [1, %d]", n_pos, kMaxChain);
    if (src_dtype != QWFN_SRC_F32 && src_dtype != QWFN_SRC_F16)
        return fail(QWFN_EINVAL, "src_dtype %d unknown", src_dtype);
    const size_t al = src_dtype == QWFN_SRC_F32 ? 16 : 8;
    if (!q || !aligned(q, 16) || !k_new || !v_new || !aligned(k_new, al) || !aligned(v_new, al) ||
        !seq_len || !out)
        return fail(QWFN_EINVAL, "decode: NULL or misaligned q / k_new / v_new / seq_len / out");
    if ((sel_out == nullptr) != (n_sel_out == nullptr))
        return fail(QWFN_EINVAL, "decode: pass both sel_out and n_sel_out or neither");
    const int32_t msel = max_selected(shape, max_seq_len);
    Ws w;
    if ((rc = bind_ws(g, n_seq, max_seq_len, msel, ws, ws_bytes, &w))) return rc;
    hipStream_t st = (hipStream_t)stream;
    // position k's lengths: seq_len + k (the first position reads seq_len itself)
    hipError_t e = n_pos > 1 ? launch_chain_lens(seq_len, n_seq, n_pos, w.lens, st) : hipSuccess;
    if (e != hipSuccess) return hip_fail(e, "decode: chain lengths");
    // one or a few sequences: the attention workgroups select for themselves
    // (no launch between the scores and the attention; at eight sequences a
    // selection launch of one workgroup per (sequence, KV head) before a
    // given-selection attention measured 29.4 against 26.9 us a step)
    const bool own = attn_select_fits(g, n_seq, max_seq_len, msel);
    const size_t row_b = (size_t)g.hd * (src_dtype == QWFN_SRC_F32 ? 4 : 2);
    for (int32_t k = 0; k < n_pos; ++k) {
        const int32_t *len_k = k == 0 ? seq_len : w.lens + (size_t)k * n_seq;
        const float *q_k = q + (size_t)k * n_seq * g.H * g.hd;
        const size_t kv_off = (size_t)k * n_seq * g.Hkv * row_b;
        const FusedAppend fa{(const uint8_t *)k_new + kv_off, (const uint8_t *)v_new + kv_off,
                             src_dtype == QWFN_SRC_F16, 1};
        float *out_k = out + (size_t)k * n_seq * g.H * g.hd;
        int32_t *sel = sel_out ? sel_out + (size_t)k * n_seq * g.Hkv * msel : w.sel;
        int32_t *nsel = n_sel_out ? n_sel_out + (size_t)k * n_seq * g.Hkv : w.nsel;
        e = launch_indexer(g, *view, q_k, len_k, n_seq, max_seq_len, sel, nsel, msel, w, fa, st, !own);
        if (e != hipSuccess) return hip_fail(e, "decode: indexer");
        e = own ? launch_attention_select(g, *view, q_k, len_k, n_seq, max_seq_len, sel, nsel, msel, out_k, w, st)
                : launch_attention(g, *view, q_k, len_k, n_seq, max_seq_len, sel, nsel, msel, out_k, w, st);
        if (e != hipSuccess) return hip_fail(e, "decode: attention");
    }
    return ok();
}

}  // extern "C"

namespace {

// The workspace of qwfn_sparse_attn_decode_noalloc: one array per device,
// held until the process ends.  In host code `scratch` names a host-side
// stand-in; the device address of each GPU's copy comes from
// hipGetSymbolAddress, looked up once per device and kept in g_scratch_ptr.
constexpr size_t kScratchBytes = (size_t)8 << 20;
constexpr int kScratchDevices = 64;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];
std::mutex g_scratch_mu;
void *g_scratch_ptr[kScratchDevices];

// This device's copy of `scratch`.  The first call on a device looks up its
// address and, unless `st` is capturing, clears it with a fill kernel on `st`
// (the workspace's completion counters must start at zero; every call leaves
// them at zero).  Under capture the fill would be recorded into the graph and
// rerun on every replay, so it is skipped: the array is zero when the code
// object is loaded, which is all the counters need.
int scratch_of_device(hipStream_t st, void **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "decode_noalloc: hipGetDevice");
    if (dev < 0 || dev >= kScratchDevices)
        return fail(QWFN_ENOTSUP, "decode_noalloc: device %d beyond the %d this library serves", dev,
                    kScratchDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return hip_fail(e, "decode_noalloc: hipGetSymbolAddress(scratch)");
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(st, &cs);
        if (e != hipSuccess) return hip_fail(e, "decode_noalloc: hipStreamIsCapturing");
        if (cs == hipStreamCaptureStatusNone) {
            e = launch_fill_zero(p, kScratchBytes, st);
            if (e != hipSuccess) return hip_fail(e, "decode_noalloc: clearing the scratch array");
        }
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return QWFN_OK;
}

}  // namespace

extern "C" {

int qwfn_sparse_attn_decode_noalloc(const qwfn_qsa_shape *shape, const qwfn_kv_view *view, const float *q,
                                    const void *k_new, const void *v_new, int32_t src_dtype,
                                    const int32_t *seq_len, int32_t n_seq, int32_t max_seq_len, float *out,
                                    int32_t *sel_out, int32_t *n_sel_out, void *stream) {
    size_t need = 0;
    int rc = qwfn_qsa_workspace_bytes(shape, n_seq, max_seq_len, &need);
    if (rc) return rc;
    if (need > kScratchBytes)
        return fail(QWFN_ERANGE,
                    "decode_noalloc: n_seq %d at max_seq_len %d needs %zu bytes of workspace, more than the "
                    "%zu of the library's scratch array; call qwfn_sparse_attn_decode with a workspace",
                    n_seq, max_seq_len, need, kScratchBytes);
    void *ws = nullptr;
    if ((rc = scratch_of_device((hipStream_t)stream, &ws))) return rc;
    return qwfn_sparse_attn_decode(shape, view, q, k_new, v_new, src_dtype, seq_len, n_seq, max_seq_len, out,
                                   sel_out, n_sel_out, ws, kScratchBytes, stream);
}

int qwfn_qsa_prefill_workspace_bytes(const qwfn_qsa_shape *shape, int32_t max_seq_len, int32_t q_batch,
                                     size_t *bytes) {
    Geo g;
    int rc = make_geo(shape, nullptr, &g, false);
    if (rc) return rc;
    if (!bytes || max_seq_len < 1 || q_batch < 1)
        return fail(QWFN_EINVAL, "prefill_workspace_bytes: bytes NULL or max_seq_len / q_batch < 1");
    // no completion counters: a batch is one grid dimension of every launch
    if (q_batch > kPrefillBatchMax) return fail(QWFN_ERANGE, "q_batch %d exceeds %d", q_batch, kPrefillBatchMax);
    Geo gpf = g;
    gpf.pf = 1;
    gpf.round_f16 = 0;
    const int32_t need = max_selected(shape, max_seq_len);
    const bool parts = !g.vdim && !dec_loop_fits(gpf, need);   // as prefill_impl lays it out
    *bytes = ws_layout(g, q_batch, max_seq_len, need, parts, false).total;
    return ok();
}

}  // extern "C"

namespace {

// The checkpoint indexer's part of a prefill call (qwfn_idx_sparse_attn_prefill).
struct IdxPrefill {
    Geo gi;                       // scoring geometry (idx_geo)
    IdxGeo ig;
    qwfn_kv_view vi;              // the KV view with the indexer's pooled keys
    const qwfn_idx_view *iv;
    const float *q_idx;           // [n_q][n_idx_head][idx_dim]
    const void *k_raw;            // [n_q][idx_dim] or NULL
};

int prefill_impl(const qwfn_qsa_shape *shape, const qwfn_kv_view *view, const IdxPrefill *ix, const float *q,
                 const void *k_new, const void *v_new, int32_t src_dtype, int32_t seq, int32_t pos0, int32_t n_q,
                 float *out, int32_t *sel_out, int32_t *n_sel_out, int32_t max_sel, void *ws, size_t ws_bytes,
                 void *stream) {
    Geo g;
    int rc = make_geo(shape, view, &g);
    if (rc) return rc;
    if (seq < 0 || seq >= view->n_seq) return fail(QWFN_EINVAL, "prefill: seq %d outside the view", seq);
    if (pos0 < 0 || n_q < 1) return fail(QWFN_EINVAL, "prefill: pos0 %d < 0 or n_q %d < 1", pos0, n_q);
    const int64_t end = (int64_t)pos0 + n_q;
    if (end > (int64_t)view->pages_per_seq * shape->page_tokens)
        return fail(QWFN_ERANGE, "prefill: context exhausted: pos0 + n_q = %lld > capacity %lld", (long long)end,
                    (long long)view->pages_per_seq * shape->page_tokens);
    if ((k_new == nullptr) != (v_new == nullptr))
        return fail(QWFN_EINVAL, "prefill: pass both k_new and v_new or neither");
    if (k_new && src_dtype != QWFN_SRC_F32 && src_dtype != QWFN_SRC_F16)
        return fail(QWFN_EINVAL, "src_dtype %d unknown", src_dtype);
    const size_t al = src_dtype == QWFN_SRC_F32 ? 16 : 8;
    if (!q || !aligned(q, 16) || !out || (k_new && (!aligned(k_new, al) || !aligned(v_new, al))))
        return fail(QWFN_EINVAL, "prefill: NULL or misaligned q / out / k_new / v_new");
    if ((sel_out == nullptr) != (n_sel_out == nullptr))
        return fail(QWFN_EINVAL, "prefill: pass both sel_out and n_sel_out or neither");
    const int32_t max_len = (int32_t)end;
    const int32_t need = max_selected(shape, max_len);
    if (sel_out && max_sel < need) return fail(QWFN_ERANGE, "prefill: max_sel %d < %d", max_sel, need);
    const int32_t sel_stride = sel_out ? max_sel : need;
    // the largest query batch whose workspace fits
    if (!ws || !aligned(ws, 256)) return fail(QWFN_EINVAL, "prefill: workspace NULL or not 256-byte aligned");
    Geo gpf = g;
    gpf.pf = 1;
    gpf.round_f16 = 0;
    // the K layouts' attention walks each query's tiles in one workgroup
    // (k_dec_loop); the general kernel merges partials in memory
    const bool loop = !g.vdim && dec_loop_fits(gpf, sel_stride);
    const bool parts = !g.vdim && !loop;
    int32_t batch = std::min<int32_t>(n_q, kPrefillBatchMax);
    while (batch > 1 && ws_layout(g, batch, max_len, need, parts, false).total > ws_bytes) batch = (batch + 1) / 2;
    if (ws_layout(g, batch, max_len, need, parts, false).total > ws_bytes)
        return fail(QWFN_ERANGE, "prefill: workspace of %zu bytes holds no query batch (need %zu)", ws_bytes,
                    ws_layout(g, 1, max_len, need, parts, false).total);
    const Ws w = ws_bind(ws, ws_layout(g, batch, max_len, need, parts, false));
    hipStream_t st = (hipStream_t)stream;
    hipError_t e = hipSuccess;
    // the chunk's rows, then every block they complete (and a block they finish)
    if (k_new) {
        e = launch_append(g, *view, k_new, v_new, src_dtype == QWFN_SRC_F16, nullptr, nullptr, n_q, seq, pos0, st);
        if (e != hipSuccess) return hip_fail(e, "prefill: append");
        const int32_t b0 = pos0 / g.bt, b1 = max_len / g.bt;   // whole blocks [b0, b1)
        if (b1 > b0) {
            e = launch_pool(g, *view, nullptr, nullptr, b1 - b0, seq, b0, st);
            if (e != hipSuccess) return hip_fail(e, "prefill: pool");
        }
    }
    if (ix && ix->k_raw) {
        // the chunk's raw indexer keys, then every block they touch (a
        // partial last block too: it is forced while partial, as in decode)
        e = launch_idx_write(g, *view, ix->ig, (uint16_t *)ix->iv->raw, ix->k_raw, src_dtype == QWFN_SRC_F16,
                             nullptr, nullptr, n_q, seq, pos0, st);
        if (e != hipSuccess) return hip_fail(e, "prefill: indexer keys");
        const int32_t b0 = pos0 / g.bt, b1 = (max_len + g.bt - 1) / g.bt;
        e = launch_idx_pool(g, *view, ix->ig, (const uint16_t *)ix->iv->raw, (uint16_t *)ix->iv->pooled, ix->iv->k_norm,
                            nullptr, nullptr, b1 - b0, seq, b0, st);
        if (e != hipSuccess) return hip_fail(e, "prefill: indexer pool");
    }
    Geo gp = g;
    gp.pf = 1;
    gp.pf_seq = seq;
    gp.round_f16 = 0;                              // prefill reads the exact rows (kv_round_f16 is decode's)
    if (g.vdim || (loop && g.kt != QWFN_KV_F16)) {
        e = launch_prefill_vmax(gp, *view, max_len, w.vmax, st);
        if (e != hipSuccess) return hip_fail(e, "prefill: V scales");
    }
    for (int32_t i0 = 0; i0 < n_q; i0 += batch) {
        const int32_t nb = std::min(batch, n_q - i0);
        gp.pf_pos0 = pos0 + i0;
        const float *qb = q + (int64_t)i0 * g.H * g.hd;
        float *ob = out + (int64_t)i0 * g.H * g.hd;
        int32_t *sb = sel_out ? sel_out + (int64_t)i0 * g.Hkv * sel_stride : w.sel;
        int32_t *nsb = n_sel_out ? n_sel_out + (int64_t)i0 * g.Hkv : w.nsel;
        // prefill mode ignores the seq_len value; the pointer only has to be
        // a readable device int that aliases no output of the attention kernel
        const int32_t *dummy_len = reinterpret_cast<const int32_t *>(w.scores);
        if (ix) {
            Geo gi = ix->gi;
            gi.pf = 1; gi.pf_seq = seq; gi.pf_pos0 = gp.pf_pos0;
            const float *qib = ix->q_idx + (int64_t)i0 * gi.H * gi.hd;
            e = launch_prefill_index(gi, ix->vi, qib, nb, max_len, sb, nsb, sel_stride, w, st);
        } else {
            e = launch_prefill_index(gp, *view, qb, nb, max_len, sb, nsb, sel_stride, w, st);
        }
        if (e != hipSuccess) return hip_fail(e, "prefill: indexer");
        e = g.vdim ? launch_prefill_attention(gp, *view, qb, nb, sb, nsb, sel_stride, w.vmax, ob, st)
            : loop ? launch_dec_loop(gp, *view, qb, nb, max_len, sb, nsb, sel_stride, w.vmax, ob, st)
                   : launch_attention(gp, *view, qb, dummy_len, nb, max_len, sb, nsb, sel_stride, ob, w, st);
        if (e != hipSuccess) return hip_fail(e, "prefill: attention");
    }
    return ok();
}

// ---- the checkpoint's own indexer (qwfn_idx_*) ----------------------------

int make_idx_geo(const qwfn_qsa_shape *s, const qwfn_idx_shape *is, IdxGeo *ig) {
    if (!is) return fail(QWFN_EINVAL, "idx shape is NULL");
    if (!idx_kernels_for(is->idx_dim))
        return fail(QWFN_ENOTSUP, "idx_dim %d: this build pools 64, 128 or 256", is->idx_dim);
    if (is->n_idx_head < 1) return fail(QWFN_EINVAL, "n_idx_head %d < 1", is->n_idx_head);
    if (!kernels_for(is->idx_dim, is->n_idx_head))
        return fail(QWFN_ENOTSUP, "no indexer instantiation for idx_dim %d, %d heads", is->idx_dim, is->n_idx_head);
    if (is->rope_dim < 0 || is->rope_dim % 2 || is->rope_dim > is->idx_dim || is->rope_dim / 2 > kIdxMaxPairs)
        return fail(QWFN_EINVAL, "rope_dim %d: even, at most idx_dim and %d", is->rope_dim, 2 * kIdxMaxPairs);
    if (!(is->rope_freq_base > 0.0f) || !std::isfinite(is->rope_freq_base))
        return fail(QWFN_EINVAL, "rope_freq_base must be positive and finite");
    if (!(is->rms_eps >= 0.0f) || !std::isfinite(is->rms_eps))
        return fail(QWFN_EINVAL, "rms_eps must be >= 0 and finite");
    (void)s;
    ig->dim = is->idx_dim;
    ig->nd = is->rope_dim;
    ig->eps = is->rms_eps;
    // ggml's theta_scale (fp32 powf, as ggml-cpu's rope computes it)
    ig->theta_scale = powf(is->rope_freq_base, -2.0f / (float)is->rope_dim);
    return QWFN_OK;
}

// The indexer's scoring geometry: one "KV head" of n_idx_head query heads over
// the indexer's pooled keys, one selection per sequence written to every one
// of the attention's n_head_kv rows.
Geo idx_scoring_geo(const Geo &g, const qwfn_idx_shape *is) {
    Geo gi = g;
    gi.H = is->n_idx_head; gi.Hkv = 1; gi.hd = is->idx_dim; gi.G = is->n_idx_head;
    gi.shared = 1;
    gi.sel_rows = g.Hkv;
    gi.pooled_f16 = 1;
    return gi;
}

int check_idx_view(const qwfn_idx_view *iv, bool raw, bool pooled, bool norm) {
    if (!iv) return fail(QWFN_EINVAL, "idx view is NULL");
    if ((raw && (!iv->raw || !aligned(iv->raw, 16))) || (pooled && (!iv->pooled || !aligned(iv->pooled, 16))) ||
        (norm && (!iv->k_norm || !aligned(iv->k_norm, 4))))
        return fail(QWFN_EINVAL, "idx view: NULL or misaligned raw (16) / pooled (16) / k_norm (4)");
    return QWFN_OK;
}

}  // namespace

extern "C" {

int qwfn_sparse_attn_prefill(const qwfn_qsa_shape *shape, const qwfn_kv_view *view, const float *q,
                             const void *k_new, const void *v_new, int32_t src_dtype, int32_t seq,
                             int32_t pos0, int32_t n_q, float *out, int32_t *sel_out, int32_t *n_sel_out,
                             int32_t max_sel, void *ws, size_t ws_bytes, void *stream) {
    return prefill_impl(shape, view, nullptr, q, k_new, v_new, src_dtype, seq, pos0, n_q, out, sel_out, n_sel_out,
                        max_sel, ws, ws_bytes, stream);
}

int qwfn_idx_cache_bytes(const qwfn_qsa_shape *shape, const qwfn_idx_shape *ishape, int32_t n_seq,
                         int32_t pages_per_seq, size_t *raw_page_bytes, size_t *pooled_bytes) {
    int rc = check_shape(shape);
    if (rc) return rc;
    IdxGeo ig;
    if ((rc = make_idx_geo(shape, ishape, &ig))) return rc;
    if (!raw_page_bytes || !pooled_bytes || n_seq < 1 || pages_per_seq < 1)
        return fail(QWFN_EINVAL, "idx_cache_bytes: NULL output or n_seq / pages_per_seq < 1");
    *raw_page_bytes = (size_t)shape->page_tokens * ishape->idx_dim * 2;
    *pooled_bytes = (size_t)n_seq * ((size_t)pages_per_seq * shape->page_tokens / shape->block_tokens) *
                    ishape->idx_dim * 2;
    return ok();
}

int qwfn_idx_workspace_bytes(const qwfn_qsa_shape *shape, const qwfn_idx_shape *ishape, int32_t n_seq,
                             int32_t max_seq_len, size_t *bytes) {
    Geo g;
    int rc = make_geo(shape, nullptr, &g, false);
    if (rc) return rc;
    IdxGeo ig;
    if ((rc = make_idx_geo(shape, ishape, &ig))) return rc;
    if (!bytes || n_seq < 1 || max_seq_len < 1)
        return fail(QWFN_EINVAL, "idx_workspace_bytes: bytes NULL or n_seq / max_seq_len < 1");
    if (n_seq > kMaxCounters) return fail(QWFN_ERANGE, "n_seq exceeds %d", kMaxCounters);
    // the indexer's layout, then the attention's (the fused decode call keeps
    // the indexer's candidates while the attention writes its partials)
    const int32_t need = max_selected(shape, max_seq_len);
    *bytes = align256(ws_layout(idx_scoring_geo(g, ishape), n_seq, max_seq_len, need, false).total) +
             ws_layout(g, n_seq, max_seq_len, need).total;
    return ok();
}

int qwfn_idx_append_pool(const qwfn_qsa_shape *shape, const qwfn_kv_view *view, const qwfn_idx_shape *ishape,
                         const qwfn_idx_view *iview, const void *k_raw, int32_t src_dtype, const int32_t *seq_ids,
                         const int32_t *pos, int32_t n_rows, void *stream) {
    Geo g;
    int rc = make_geo(shape, view, &g);
    if (rc) return rc;
    IdxGeo ig;
    if ((rc = make_idx_geo(shape, ishape, &ig)) || (rc = check_idx_view(iview, true, true, true))) return rc;
    if (src_dtype != QWFN_SRC_F32 && src_dtype != QWFN_SRC_F16) return fail(QWFN_EINVAL, "src_dtype %d unknown", src_dtype);
    if (!k_raw || !aligned(k_raw, 16) || !pos || n_rows < 0)
        return fail(QWFN_EINVAL, "idx_append_pool: NULL or misaligned k_raw (16) / NULL pos / n_rows < 0");
    if (n_rows == 0) return ok();
    hipStream_t st = (hipStream_t)stream;
    if (n_rows <= kIdxFuseRows) {                 // a decode step: one launch
        const hipError_t e1 = launch_idx_append_pool(g, *view, ig, (uint16_t *)iview->raw, (uint16_t *)iview->pooled,
                                                     iview->k_norm, k_raw, src_dtype == QWFN_SRC_F16, seq_ids, pos,
                                                     n_rows, st);
        return e1 == hipSuccess ? ok() : hip_fail(e1, "idx_append_pool");
    }
    hipError_t e = launch_idx_write(g, *view, ig, (uint16_t *)iview->raw, k_raw, src_dtype == QWFN_SRC_F16, seq_ids,
                                    pos, n_rows, 0, 0, st);
    if (e != hipSuccess) return hip_fail(e, "idx_append_pool: write");
    e = launch_idx_pool(g, *view, ig, (const uint16_t *)iview->raw, (uint16_t *)iview->pooled, iview->k_norm, seq_ids, pos,
                        n_rows, 0, 0, st);
    return e == hipSuccess ? ok() : hip_fail(e, "idx_append_pool: pool");
}

int qwfn_idx_pool_rebuild(const qwfn_qsa_shape *shape, const qwfn_kv_view *view, const qwfn_idx_shape *ishape,
                          const qwfn_idx_view *iview, int32_t seq, int32_t n_whole, void *stream) {
    Geo g;
    int rc = make_geo(shape, view, &g);
    if (rc) return rc;
    IdxGeo ig;
    if ((rc = make_idx_geo(shape, ishape, &ig)) || (rc = check_idx_view(iview, true, true, true))) return rc;
    if (seq < 0 || seq >= view->n_seq) return fail(QWFN_EINVAL, "idx_pool_rebuild: seq %d outside the view", seq);
    if (n_whole < 0) return fail(QWFN_EINVAL, "idx_pool_rebuild: n_whole %d < 0", n_whole);
    if (n_whole > g.bps) return fail(QWFN_ERANGE, "idx_pool_rebuild: n_whole %d > %d blocks", n_whole, g.bps);
    const hipError_t e = launch_idx_pool(g, *view, ig, (const uint16_t *)iview->raw, (uint16_t *)iview->pooled, iview->k_norm,
                                         nullptr, nullptr, n_whole, seq, 0, (hipStream_t)stream);
    return e == hipSuccess ? ok() : hip_fail(e, "idx_pool_rebuild");
}

int qwfn_idx_select(const qwfn_qsa_shape *shape, const qwfn_kv_view *view, const qwfn_idx_shape *ishape,
                    const qwfn_idx_view *iview, const float *q_idx, const int32_t *seq_len, int32_t n_seq,
                    int32_t max_seq_len, int32_t *sel, int32_t *n_sel, int32_t max_sel, void *ws, size_t ws_bytes,
                    void *stream) {
    Geo g;
    int rc = make_geo(shape, view, &g);
    if (rc) return rc;
    IdxGeo ig;
    if ((rc = make_idx_geo(shape, ishape, &ig)) || (rc = check_idx_view(iview, false, true, false))) return rc;
    if ((rc = check_batch(shape, view, n_seq, max_seq_len))) return rc;
    if (!q_idx || !aligned(q_idx, 16) || !seq_len || !sel || !n_sel)
        return fail(QWFN_EINVAL, "idx_select: NULL q_idx / seq_len / sel / n_sel or q_idx not 16-byte aligned");
    const int32_t need = max_selected(shape, max_seq_len);
    if (max_sel < need) return fail(QWFN_ERANGE, "idx_select: max_sel %d < %d", max_sel, need);
    const Geo gi = idx_scoring_geo(g, ishape);
    const WsLayout l = ws_layout(gi, n_seq, max_seq_len, need, false);
    if (!ws || !aligned(ws, 256)) return fail(QWFN_EINVAL, "idx_select: workspace NULL or not 256-byte aligned");
    if (ws_bytes < l.total) return fail(QWFN_ERANGE, "idx_select: workspace of %zu bytes < %zu", ws_bytes, l.total);
    const Ws w = ws_bind(ws, l);
    qwfn_kv_view vi = *view;
    vi.pooled = (float *)iview->pooled;                   // fp16 keys (Geo::pooled_f16)
    const FusedAppend fa{nullptr, nullptr, 0, 0};
    const hipError_t e = launch_indexer(gi, vi, q_idx, seq_len, n_seq, max_seq_len, sel, n_sel, max_sel, w, fa,
                                        (hipStream_t)stream);
    return e == hipSuccess ? ok() : hip_fail(e, "idx_select");
}

int qwfn_idx_sparse_attn_decode(const qwfn_qsa_shape *shape, const qwfn_kv_view *view, const qwfn_idx_shape *ishape,
                                const qwfn_idx_view *iview, const float *q, const float *q_idx, const void *k_new,
                                const void *v_new, const void *k_raw, int32_t src_dtype, const int32_t *seq_len,
                                int32_t n_seq, int32_t max_seq_len, float *out, int32_t *sel, int32_t *n_sel,
                                int32_t max_sel, void *ws, size_t ws_bytes, void *stream) {
    TimerDisarm disarm;
    Geo g;
    int rc = make_geo(shape, view, &g);
    if (rc) return rc;
    IdxGeo ig;
    if ((rc = make_idx_geo(shape, ishape, &ig)) || (rc = check_idx_view(iview, true, true, true))) return rc;
    if ((rc = check_batch(shape, view, n_seq, max_seq_len))) return rc;
    if (n_seq > kIdxFuseRows)
        return fail(QWFN_ERANGE, "idx decode: n_seq %d > %d (call qwfn_kv_append_q8_0, qwfn_idx_append_pool, "
                    "qwfn_idx_select and qwfn_sparse_decode_attn)", n_seq, kIdxFuseRows);
    if (src_dtype != QWFN_SRC_F32 && src_dtype != QWFN_SRC_F16) return fail(QWFN_EINVAL, "src_dtype %d unknown", src_dtype);
    const size_t al = src_dtype == QWFN_SRC_F32 ? 16 : 8;
    if (!q || !aligned(q, 16) || !q_idx || !aligned(q_idx, 16) || !k_new || !v_new || !aligned(k_new, al) ||
        !aligned(v_new, al) || !k_raw || !aligned(k_raw, 16) || !seq_len || !out || !sel || !n_sel)
        return fail(QWFN_EINVAL, "idx decode: NULL or misaligned q / q_idx / k_new / v_new / k_raw (16) / seq_len / "
                    "out / sel / n_sel");
    const int32_t need = max_selected(shape, max_seq_len);
    if (max_sel < need) return fail(QWFN_ERANGE, "idx decode: max_sel %d < %d", max_sel, need);
    // the indexer and the attention run one after the other over the same
    // workspace: it must hold the larger of their layouts
    const Geo gi = idx_scoring_geo(g, ishape);
    const WsLayout li = ws_layout(gi, n_seq, max_seq_len, need, false);
    const WsLayout la = ws_layout(g, n_seq, max_seq_len, max_sel);
    const size_t total = li.total > la.total ? li.total : la.total;
    if (!ws || !aligned(ws, 256)) return fail(QWFN_EINVAL, "idx decode: workspace NULL or not 256-byte aligned");
    if (ws_bytes < total) return fail(QWFN_ERANGE, "idx decode: workspace of %zu bytes < %zu", ws_bytes, total);
    hipStream_t st = (hipStream_t)stream;
    const int32_t f16 = src_dtype == QWFN_SRC_F16;
    // Rows longer than the indexer workgroup's registers hold: the attention
    // workgroups select for themselves (no selection launch).  The append
    // launch also places a sampled cut of each row, the indexer's workgroups
    // keep the keys above it as candidates, and the attention ranks those
    // exactly.  The attention's layout then follows the indexer's in the
    // workspace (qwfn_idx_workspace_bytes sizes both), so its partials never
    // touch the candidates; a workspace sized for one layout keeps the
    // selection launch.
    const bool split_ws = ws_bytes >= align256(li.total) + la.total;
    const bool fused_sel = max_seq_len / g.bt > kIdxRegKeys && dec_selbig_fits(g, max_seq_len, max_sel) &&
                           ishape->idx_dim <= 128 && ishape->n_idx_head * ishape->idx_dim <= kIdxMaxCutHeads * 128 &&
                           split_ws;
    // Rows the indexer workgroup's registers hold: the indexer only scores and
    // every attention workgroup selects from the row (no last-workgroup
    // selection in the indexer); the same split workspace.
    const bool row_sel = max_seq_len / g.bt <= kIdxRegKeys && dec_selrow_fits(g, max_seq_len, max_sel) && split_ws;
    // Past 8,192 blocks with one score row a sequence, the append workgroup
    // and the cut's sample workgroups run in the indexer launch too, ahead of
    // the chunks that wait for them (no sample is the row's last block, the
    // one the append may re-pool; the chunk holding it takes its key from the
    // append workgroup).
    const bool in_cut = fused_sel && gi.Hkv == 1;
    Ws wi = ws_bind(ws, li);
    const IdxCut cut{fused_sel && !in_cut ? q_idx : nullptr, wi.cutk, ishape->n_idx_head, max_seq_len};
    if (in_cut) wi.cutk = reinterpret_cast<uint32_t *>(wi.cnt_idx + kCutReadyBase);
    // the K/V rows, the raw indexer key and its block's pooled key: a launch of
    // their own, or (row_sel or in_cut, one score row a sequence) the indexer
    // launch's append workgroup, which also scores the block the token
    // completes when that block is eligible
    const IdxAppend ia{g, *view, ig, FusedAppend{k_new, v_new, f16, 1}, k_raw, iview->k_norm,
                       (uint16_t *)iview->raw, f16, (row_sel || in_cut) && gi.Hkv == 1 ? 1 : 0,
                       in_cut ? wi.cutk : nullptr, g_cut_polls.load()};
    hipError_t e = hipSuccess;
    if (!ia.enabled) {
        e = launch_idx_append_pool(g, *view, ig, (uint16_t *)iview->raw, (uint16_t *)iview->pooled, iview->k_norm,
                                   k_raw, f16, nullptr, nullptr, n_seq, st, FusedAppend{k_new, v_new, f16, 1},
                                   seq_len, cut);
        if (e != hipSuccess) return hip_fail(e, "idx decode: append");
    }
    qwfn_kv_view vi = *view;
    vi.pooled = (float *)iview->pooled;                   // fp16 keys (Geo::pooled_f16)
    e = launch_indexer(gi, vi, q_idx, seq_len, n_seq, max_seq_len, sel, n_sel, max_sel, wi,
                       FusedAppend{nullptr, nullptr, 0, 0}, st, true, !(fused_sel || row_sel),
                       ia.enabled ? &ia : nullptr, in_cut);
    if (e != hipSuccess) return hip_fail(e, "idx decode: indexer");
    if (fused_sel || row_sel) {
        Ws wa = ws_bind((uint8_t *)ws + align256(li.total), la);
        wa.scores = wi.scores;
        wa.nb_cap = wi.nb_cap;
        wa.cand = wi.cand;
        wa.ccnt = wi.ccnt;
        wa.cutk = in_cut ? wi.cutk : nullptr;     // kSelBig clears the in-launch cut's slots
        e = fused_sel ? launch_dec_selbig(g, *view, q, seq_len, n_seq, max_seq_len, sel, n_sel, max_sel, out, wa, st)
                      : launch_dec_selrow(g, *view, q, seq_len, n_seq, max_seq_len, sel, n_sel, max_sel, out, wa, st);
    } else {
        e = launch_attention(g, *view, q, seq_len, n_seq, max_seq_len, sel, n_sel, max_sel, out, ws_bind(ws, la), st);
    }
    return e == hipSuccess ? ok() : hip_fail(e, "idx decode: attention");
}

int qwfn_idx_sparse_attn_prefill(const qwfn_qsa_shape *shape, const qwfn_kv_view *view,
                                 const qwfn_idx_shape *ishape, const qwfn_idx_view *iview, const float *q,
                                 const float *q_idx, const void *k_new, const void *v_new, const void *k_raw,
                                 int32_t src_dtype, int32_t seq, int32_t pos0, int32_t n_q, float *out,
                                 int32_t *sel_out, int32_t *n_sel_out, int32_t max_sel, void *ws, size_t ws_bytes,
                                 void *stream) {
    Geo g;
    int rc = make_geo(shape, view, &g);
    if (rc) return rc;
    IdxPrefill ix;
    if ((rc = make_idx_geo(shape, ishape, &ix.ig)) || (rc = check_idx_view(iview, k_raw != nullptr, true, k_raw != nullptr)))
        return rc;
    if (!q_idx || !aligned(q_idx, 16)) return fail(QWFN_EINVAL, "idx prefill: NULL or misaligned q_idx");
    if (k_raw && (!aligned(k_raw, 16) || !k_new))
        return fail(QWFN_EINVAL, "idx prefill: k_raw must be 16-byte aligned and come with k_new / v_new");
    ix.gi = idx_scoring_geo(g, ishape);
    ix.vi = *view;
    ix.vi.pooled = (float *)iview->pooled;                // fp16 keys (Geo::pooled_f16)
    ix.iv = iview;
    ix.q_idx = q_idx;
    ix.k_raw = k_raw;
    return prefill_impl(shape, view, &ix, q, k_new, v_new, src_dtype, seq, pos0, n_q, out, sel_out, n_sel_out,
                        max_sel, ws, ws_bytes, stream);
}

}  // extern "C"
