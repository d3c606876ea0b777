// qsa_decode_kv.hip -- the matrix-core decode attention (k_dec,
// qsa_dec_kernel.h) for q4_0 and F16 caches: their K and V rows are 16-byte
// chunks of a head row in the K layout (q4_0: one ggml block of 32 nibbles,
// dims 0-15 low and 16-31 high, with fp16 scales as q8_0; F16: 8 dims, no
// scales), read a cell at a time; the nibbles and halves enter the fp16
// matrix cores exactly.
#include "qsa_dec_kernel.h"

namespace qwfn_qsa {

#define QWFN_FOR_EACH_DEC_KV(X) X(128, 8)

bool dec_kv_shape(const Geo &g) {
#define X(HD_, G_) if (g.hd == HD_ && g.G == G_) return true;
    QWFN_FOR_EACH_DEC_KV(X)
#undef X
    return false;
}

hipError_t launch_dec_kv(const Geo &g, const qwfn_kv_view &v, const float *q, const int32_t *seq_len, int32_t n_seq,
                         int32_t max_seq_len, const int32_t *sel, const int32_t *nsel, int32_t max_sel, float *out,
                         const Ws &ws, bool select, hipStream_t st) {
#define X(HD_, G_)                                                                                                    \
    if (g.hd == HD_ && g.G == G_) {                                                                                   \
        if (g.kt == QWFN_KV_Q4_0)                                                                                     \
            return launch_dec_shape<HD_, G_, false, kLyQ4>(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel,   \
                                                           out, ws, select, st);                                      \
        if (g.kt == QWFN_KV_F16)                                                                                      \
            return launch_dec_shape<HD_, G_, false, kLyF16>(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel,  \
                                                            out, ws, select, st);                                     \
    }
    QWFN_FOR_EACH_DEC_KV(X)
#undef X
    return hipErrorInvalidValue;
}

hipError_t launch_dec_kv_loop(const Geo &g, const qwfn_kv_view &v, const float *q, int32_t n_q, int32_t max_seq_len,
                              const int32_t *sel, const int32_t *nsel, int32_t max_sel, const float *vmax, float *out,
                              hipStream_t st) {
#define X(HD_, G_)                                                                                                 \
    if (g.hd == HD_ && g.G == G_) {                                                                                \
        if (g.kt == QWFN_KV_Q4_0)                                                                                  \
            return launch_dec_loop_t<HD_, G_, kLyQ4>(g, v, q, n_q, max_seq_len, sel, nsel, max_sel, vmax, out, st); \
        if (g.kt == QWFN_KV_F16)                                                                                   \
            return launch_dec_loop_t<HD_, G_, kLyF16>(g, v, q, n_q, max_seq_len, sel, nsel, max_sel, vmax, out, st); \
    }
    QWFN_FOR_EACH_DEC_KV(X)
#undef X
    return hipErrorInvalidValue;
}

}  // namespace qwfn_qsa
