// qsa_decode.hip -- dispatch of the matrix-core decode attention (k_dec,
// qsa_dec_kernel.h) and its q8_0 instantiations: V dim-major per 64-token
// tile (blocks of whole tiles, with or without kv_round_f16) and V in the K
// layout (blocks shorter than a tile, gathered).  q4_0 and F16 caches are
// instantiated in qsa_decode_kv.hip.
#include "qsa_dec_kernel.h"

namespace qwfn_qsa {

#define QWFN_FOR_EACH_DEC(X) X(128, 8) X(128, 4) X(128, 2) X(64, 8) X(256, 12) X(256, 8)
// Shapes whose fp16-rounded K/V (kv_round_f16) run here; the others take the
// general kernel, which dequantizes each value into LDS.
#define QWFN_FOR_EACH_DEC_RF(X) X(128, 8)
// Shapes whose q8_0 blocks are shorter than a tile (block_tokens dividing 64)
// run here with gathered tiles: the checkpoint's (256, 12), the tiny test
// shape's (128, 2) and the BASELINE heads.
#define QWFN_FOR_EACH_DEC_GATH(X) X(128, 8) X(128, 2) X(256, 12)

// The page layout k_dec reads for this shape and call, or -1 (the general
// kernel).  q8_0: V dim-major for blocks of whole tiles (decode only; the
// prefill of those runs k_pf_attn), else V in the K layout for blocks that
// divide a tile.  q4_0 and F16 (qsa_decode_kv.hip): V in the K layout for
// blocks that divide a tile or are whole tiles.  In the K layouts a scale
// row's 16-byte chunk (16 / (2 head_dim / 32) cells) must stay in one block.
int dec_layout(const Geo &g) {
    const bool whole = g.bt % 64 == 0, divides = g.bt >= 2 && 64 % g.bt == 0;
    const int cpl = 16 / (2 * (g.hd / 32));
    const bool chunk_ok = g.kt == QWFN_KV_F16 || cpl <= 1 || g.bt % cpl == 0;
    if (g.kt == QWFN_KV_Q8_0 && g.vdim) {
        if (g.pf) return -1;
        if (g.round_f16) {
#define X(HD_, G_) if (g.hd == HD_ && g.G == G_) return kLyQ8;
            QWFN_FOR_EACH_DEC_RF(X)
#undef X
            return -1;
        }
#define X(HD_, G_) if (g.hd == HD_ && g.G == G_) return kLyQ8;
        QWFN_FOR_EACH_DEC(X)
#undef X
        return -1;
    }
    if (g.kt == QWFN_KV_Q8_0) {
        if (g.round_f16 || !divides || !chunk_ok) return -1;
#define X(HD_, G_) if (g.hd == HD_ && g.G == G_) return kLyQ8K;
        QWFN_FOR_EACH_DEC_GATH(X)
#undef X
        return -1;
    }
    // q4_0 with kv_round_f16: the general kernel; F16 values are fp16 already
    if ((g.kt == QWFN_KV_Q4_0 && g.round_f16) || !(whole || divides) || !chunk_ok || !dec_kv_shape(g)) return -1;
    return g.kt == QWFN_KV_Q4_0 ? kLyQ4 : kLyF16;
}

bool dec_kernels_for(const Geo &g) { return dec_layout(g) >= 0; }

bool dec_select_fits(const Geo &g, int32_t max_seq_len, int32_t max_sel) {
    const int ly = dec_layout(g);
    return (ly == kLyQ8 || ly == kLyQ4 || ly == kLyF16) && !g.pf && !g.shared && g.topk > 0 &&
           max_sel <= kDecSelMax && max_seq_len / g.bt - (g.sink & ~3) <= 32 * kDecThreads;
}

bool dec_loop_fits(const Geo &g, int32_t max_sel) {
    const int ly = dec_layout(g);
    return g.pf && (ly == kLyQ8K || ly == kLyQ4 || ly == kLyF16) && max_sel >= 1 && max_sel <= kDecSelMax;
}

hipError_t launch_dec_loop(const Geo &g, const qwfn_kv_view &v, const float *q, int32_t n_q, int32_t max_seq_len,
                           const int32_t *sel, const int32_t *nsel, int32_t max_sel, const float *vmax, float *out,
                           hipStream_t st) {
    if (!dec_loop_fits(g, max_sel)) return hipErrorInvalidValue;
    const int ly = dec_layout(g);
    if (ly == kLyQ4 || ly == kLyF16)
        return launch_dec_kv_loop(g, v, q, n_q, max_seq_len, sel, nsel, max_sel, vmax, out, st);
#define X(HD_, G_)                                                                                               \
    if (g.hd == HD_ && g.G == G_)                                                                                \
        return launch_dec_loop_t<HD_, G_, kLyQ8K>(g, v, q, n_q, max_seq_len, sel, nsel, max_sel, vmax, out, st);
    QWFN_FOR_EACH_DEC_GATH(X)
#undef X
    return hipErrorInvalidValue;
}

// A long row the attention's own selection covers: at most kDecBigChunks
// indexer chunks of kIdxChunkBlocks blocks.
static bool dec_selbig_row(const Geo &g, int32_t max_seq_len) {
    return (int64_t)max_seq_len / g.bt <= (int64_t)kDecBigChunks * kIdxChunkBlocks;
}

bool dec_selbig_fits(const Geo &g, int32_t max_seq_len, int32_t max_sel) {
    return dec_layout(g) == kLyQ8K && g.shared && !g.pf && g.topk > 0 && max_sel <= kDecSelMax &&
           g.hd == 256 && g.G == 12 && dec_selbig_row(g, max_seq_len);
}

hipError_t launch_dec_selbig(const Geo &g, const qwfn_kv_view &v, const float *q, const int32_t *seq_len,
                             int32_t n_seq, int32_t max_seq_len, int32_t *sel, int32_t *nsel, int32_t max_sel,
                             float *out, const Ws &ws, hipStream_t st) {
    if (!dec_selbig_fits(g, max_seq_len, max_sel)) return hipErrorInvalidValue;
    return launch_dec_selbig_t<256, 12, kLyQ8K>(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel, out, ws, st);
}

// The checkpoint layer's shared row up to 32 keys a thread: every attention
// workgroup selects from it (kSelRow), the indexer only scores.
bool dec_selrow_fits(const Geo &g, int32_t max_seq_len, int32_t max_sel) {
    return dec_layout(g) == kLyQ8K && g.shared && !g.pf && g.topk > 0 && max_sel <= kDecSelMax && g.hd == 256 &&
           g.G == 12 && max_seq_len / g.bt - (g.sink & ~3) <= 32 * kDecThreads;
}

hipError_t launch_dec_selrow(const Geo &g, const qwfn_kv_view &v, const float *q, const int32_t *seq_len,
                             int32_t n_seq, int32_t max_seq_len, int32_t *sel, int32_t *nsel, int32_t max_sel,
                             float *out, const Ws &ws, hipStream_t st) {
    if (!dec_selrow_fits(g, max_seq_len, max_sel)) return hipErrorInvalidValue;
    return launch_dec_selrow_t<256, 12, kLyQ8K>(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel, out, ws, st);
}

hipError_t launch_test_select_big(const Geo &g, const float *scores, int32_t nb_cap, const int32_t *seq_len,
                                  int32_t n_seq, int32_t max_seq_len, int32_t *sel, int32_t *nsel, int32_t max_sel,
                                  hipStream_t st) {
    if (max_sel > kDecSelMax || !dec_selbig_row(g, max_seq_len)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_test_select_big, dim3((unsigned)n_seq), dim3(kDecThreads), (unsigned)sizeof(DecSelBig), st, g,
                       scores, nb_cap, seq_len, max_seq_len, sel, nsel, max_sel);
    return hipGetLastError();
}

hipError_t launch_dec_attention(const Geo &g, const qwfn_kv_view &v, const float *q, const int32_t *seq_len,
                                int32_t n_seq, int32_t max_seq_len, const int32_t *sel, const int32_t *nsel,
                                int32_t max_sel, float *out, const Ws &ws, bool select, hipStream_t st) {
    const int ly = dec_layout(g);
    if (ly < 0 || (select && !dec_select_fits(g, max_seq_len, max_sel))) return hipErrorInvalidValue;
    if (ly == kLyQ4 || ly == kLyF16)
        return launch_dec_kv(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel, out, ws, select, st);
    if (ly == kLyQ8K) {
#define X(HD_, G_)                                                                                              \
        if (g.hd == HD_ && g.G == G_)                                                                           \
            return launch_dec_shape<HD_, G_, false, kLyQ8K>(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel, \
                                                            out, ws, false, st);
        QWFN_FOR_EACH_DEC_GATH(X)
#undef X
        return hipErrorInvalidValue;
    }
    if (g.round_f16) {
#define X(HD_, G_)                                                                                              \
        if (g.hd == HD_ && g.G == G_)                                                                           \
            return launch_dec_shape<HD_, G_, true, kLyQ8>(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel, \
                                                          out, ws, select, st);
        QWFN_FOR_EACH_DEC_RF(X)
#undef X
        return hipErrorInvalidValue;
    }
#define X(HD_, G_)                                                                                        \
    if (g.hd == HD_ && g.G == G_)                                                                         \
        return launch_dec_shape<HD_, G_, false, kLyQ8>(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel, \
                                                       out, ws, select, st);
    QWFN_FOR_EACH_DEC(X)
#undef X
    return hipErrorInvalidValue;
}

}  // namespace qwfn_qsa
