// qsa_dec_kernel.h -- the matrix-core decode attention k_dec and its launch
// helpers, shared by qsa_decode.hip (q8_0) and qsa_decode_kv.hip (q4_0, F16),
// which instantiate disjoint sets of it: the attention of
// qwfn_sparse_decode_attn (a given selection or dense), of the fused
// qwfn_sparse_attn_decode (the workgroup selects from the indexer's scores),
// of the checkpoint layer's fused qwfn_idx_sparse_attn_decode past 8192
// blocks (the workgroup ranks the indexer's candidates) and of prefill chunks
// whose cache rows are in the K layout.
//
// One workgroup of four waves (one per SIMD) per part of TM tiles of a
// (sequence, KV head); wave w owns cells 16w .. 16w+15 of every tile, so a
// wave's logits need no other wave.  All of a part's tiles go out at once as
// 16-byte global -> LDS transfers into the wave's own staging slots (no
// registers held while they fly, no barrier before reading them), and the
// wave runs a two-pass softmax over them:
//   QK  v_mfma_f32_16x16x32_f16 per tile as it lands: the int8 key quants
//       (exact in fp16) against the query scaled by a power of two and split
//       into fp16 high + low parts, one accumulator per 32-dim q8_0 block,
//       combined with the keys' scales; the logits of all TM tiles stay in
//       registers, and their column maximum is the softmax reference.
//   PV  v_mfma_f32_16x16x16_f16 accumulating straight into O: the V quants
//       (exact in fp16) against the weights p * d_v * 2^k split into fp16
//       high + low parts, k fixed per column over the part (its largest V
//       scale near 2^15), so O needs no rescaling between tiles.  The QK
//       accumulator layout (cells 4lg..4lg+3 of column hn in lane 16lg+hn) is
//       the B-operand layout of this shape, so the weights never leave their
//       lanes.
// The four waves' states merge through LDS into one partial (max, sum,
// unnormalised O) per workgroup, which k_merge combines.
//
// The latency of one sequence is a chain of dependent steps, so everything
// that does not depend on the selection (the length, the score row, the query
// rows, the sequence's page-table row) is loaded in the first round trip and
// the selection is a short exact top-k over a 2048-bin histogram held by the
// four waves (kSelect), or over the candidates the indexer left (kSelBig).
#pragma once

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include <algorithm>
#include <atomic>

#include "qsa_device.h"
#include "qsa_select.h"

namespace qwfn_qsa {

namespace {

constexpr int kDecThreads = 256;
constexpr int kDecWaves = kDecThreads / 64;
constexpr int kDecBins = 2048;                  // selection histogram bins
constexpr int kDecCand = 256;                   // threshold-bin keys ranked pairwise
constexpr int kDecPtLds = 4096;                 // page-table entries parked in LDS at most
constexpr int kDecSelMax = 1024;                // selected blocks kept in LDS

enum DecMode { kGiven = 0, kDense = 1, kSelect = 2, kSelBig = 3, kSelRow = 4 };

// kSelBig: a long row of at most kDecBigRnd * kDecThreads * 4 = 49,152 blocks
// (longer rows take the selection launch), kDecBigChunks indexer chunks.
constexpr int kDecBigRnd = 48;
constexpr int kDecBigChunks = kDecBigRnd * kDecThreads * 4 / kIdxChunkBlocks;   // the indexer's chunks a row
constexpr int kDecBigCpt = kDecBigChunks / kDecThreads;                          // chunks a thread gathers
constexpr int kDecBigPre = 12;                  // candidate slots of a chunk read in the first round trip

typedef _Float16 h4v __attribute__((ext_vector_type(4)));
typedef uint32_t u2v __attribute__((ext_vector_type(2)));

// The selection's scratch (kSelect); it shares the dynamic LDS region with
// the tile staging and the waves' O, which are used only after it.
struct DecSel {
    uint32_t hist[kDecBins + 64];                // + one trash bin per lane
    uint32_t cand_key[kDecWaves * kDecCand + 64];   // threshold-bin keys, a region per wave
    int32_t cand_b[kDecWaves * kDecCand + 64];      // (+ one trash slot per lane)
};

// The selection scratch of kSelBig (the candidates, their histogram, the
// threshold bin and the winners' bit map); the fields the shared selection
// routines (sample_cut_of, hist_cut, select_radix) use.
struct DecSelBig {
    uint32_t hist[4096 + 64];                    // + one trash bin per lane
    u2v cand[kSelCandMax + 64];                  // candidates (key, block), in block order (+ one trash slot per lane)
    uint8_t cok[kSelCandMax];                    // the threshold bin's verdicts, by candidate
    int32_t rwin[kSelCandMax / kDecThreads * kDecWaves];   // winners of each (round, wave)
    u4v xch[kDecWaves];                          // each wave's (count, key min, key max, overflow)
    uint32_t cand_key[kCandMax + 64];            // the threshold bin's keys, blocks
    int32_t cand_b[kCandMax + 64];
    float red[2 * kDecWaves];
    uint32_t kred[2 * kDecWaves];
    int tmp[kDecWaves];
    int bin, need, cnt_b, ncand, nbin;
};

template <int G>
struct DecShared {
    float wml[kDecWaves][G][2];                  // the waves' (max, sum)
    int32_t wcnt[kDecWaves];
    int32_t ccnt[kDecWaves];
    float2 wlh[kDecWaves];                       // kSelRow: each wave's (smallest, largest) eligible score
    int32_t nsel;
    int32_t sel[kDecSelMax + 64];                // + one trash slot per lane
};

// One wave's share of a staged tile: the K quants of its 16 cells (chunk c at
// c * 256, cell i at i * 16), the V quants (dim d at d * 16: its 16 cells),
// then the K and the V scales of its 16 cells (cell-major, NB fp16 a cell).
// The page layouts k_dec reads (LY): q8_0 with V dim-major per 64-token tile
// (blocks of whole tiles), q8_0 with V in the K layout (blocks shorter than a
// tile, gathered 64 / block_tokens to a tile), q4_0 and F16 (V in the K
// layout, any block size).  In the K layout a page holds 16-byte chunks of a
// head row, chunk c of a 64-token tile's rows contiguous (1 KB).
constexpr int kLyQ8 = 0, kLyQ8K = 1, kLyQ4 = 2, kLyF16 = 3;

// For the K layouts the V region is K's: chunk c of the wave's cells at c * 256
// (cell i at i * 16).  F16 has no scales.
template <int HD, int LY = kLyQ8>
struct DecStage {
    static constexpr int NB = HD / 32, ND = HD / 16, NS = NB / 2;
    static constexpr int RB = LY == kLyQ4 ? HD / 2 : LY == kLyF16 ? 2 * HD : HD;   // bytes of a head row
    static constexpr int CH = RB / 16;                   // 16-byte chunks of a head row
    static constexpr int NKV = CH / 4;                   // 1 KB transfers of K (and of V) a tile
    static constexpr int KOFF = 0, VOFF = CH * 256, SOFF = 2 * CH * 256;
    static constexpr int SROW = LY == kLyF16 ? 0 : 16 * NB * 2;   // one scale set of the wave's 16 cells
    static constexpr int BYTES = SOFF + 2 * SROW;
    static constexpr int NL = 2 * NKV + (SROW > 0 ? 1 : 0);   // transfers a wave issues per tile
    static_assert(HD % 64 == 0 && CH % 4 == 0 && SROW % 16 == 0 && 2 * SROW / 16 <= 64, "whole 16-byte transfers");
};

// Bytes of the dynamic LDS region shared by the selection scratch, the
// staged tiles and the waves' O (the page-table row follows it).
template <int HD, int G, int MODE, int TM, int LY = kLyQ8>
constexpr int dec_union_bytes() {
    constexpr int st = TM * kDecWaves * DecStage<HD, LY>::BYTES;
    constexpr int wo = kDecWaves * G * HD * 4;
    constexpr int se = MODE == kSelect || MODE == kSelRow ? (int)sizeof(DecSel)
                       : MODE == kSelBig                   ? (int)sizeof(DecSelBig)
                                                           : 0;
    constexpr int m = st > wo ? st : wo;
    return ((m > se ? m : se) + 15) / 16 * 16;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Four int8 quants -> four exact fp16 values, in order (bias to unsigned, splice
// under the fp16 exponent of 1024, subtract 1152).
__device__ __forceinline__ h4v q8x4_to_h4(uint32_t w) {
    half2v lo, hi;
    q8x4_to_h2(w, lo, hi);
    h4v r;
    r[0] = lo[0]; r[1] = lo[1]; r[2] = hi[0]; r[3] = hi[1];
    return r;
}

// Four q4_0 nibbles, one a byte (0 .. 15), -> four exact fp16 values q - 8, in
// order (splice under the fp16 exponent of 1024, subtract 1032).
__device__ __forceinline__ h4v q4x4_to_h4(uint32_t w) {
    const half2v bias = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    const half2v lo = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u)) + bias;
    const half2v hi = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u)) + bias;
    h4v r;
    r[0] = lo[0]; r[1] = lo[1]; r[2] = hi[0]; r[3] = hi[1];
    return r;
}

// The low bytes of four words as one word, in order.
__device__ __forceinline__ uint32_t pack4_lo8(const uint32_t (&w)[4]) {
    const uint32_t p01 = __builtin_amdgcn_perm(w[1], w[0], 0x0c0c0400u);
    const uint32_t p23 = __builtin_amdgcn_perm(w[3], w[2], 0x0c0c0400u);
    return __builtin_amdgcn_perm(p23, p01, 0x05040100u);
}

// The selection histogram is stored transposed: bin b at word
// (b % 32) * 64 + b / 32, so lane l's 32 bins [32l, 32l+32) are the words
// j*64 + l, j = 0..31, and each of the wave's 32 reads touches 64 consecutive
// words (no bank conflicts; an untransposed 128-byte run per lane put every
// lane on the same banks).
__device__ __forceinline__ int hist_word(int b) { return (b & 31) * 64 + (b >> 5); }

// Threshold bin of the selection histogram (kDecBins bins in ascending key
// order) for the topk-th largest key, found by each wave on its own (no barrier
// after): lane l sums bins [32l, 32l+32), a scan finds the lane holding that
// key, then that lane's 32 bins are spread over lanes 0..31 for the same
// search.  Returns the bin; *need = keys of it still needed, *cnt = its keys.
__device__ __forceinline__ int dec_cut(const uint32_t *hist, int topk, int *need, int *cnt) {
    const int lane = threadIdx.x & 63;
    uint32_t own = 0;
#pragma unroll
    for (int j = 0; j < 32; ++j) own += hist[j * 64 + lane];
    const int incl = wave_incl_scan((int)own);
    const int total = __builtin_amdgcn_readlane(incl, 63);
    const int above = total - incl;                      // keys in the bins of higher lanes
    const int ls = __builtin_ctzll(__ballot(above < topk && above + (int)own >= topk));
    const int above_l = __builtin_amdgcn_readlane(above, ls);
    const int c = (int)hist[(lane & 31) * 64 + ls] & -(lane < 32);
    const int ic = wave_incl_scan(c);
    const int run = above_l + __builtin_amdgcn_readlane(ic, 31) - ic;   // keys in higher bins
    const int j = __builtin_ctzll(__ballot(lane < 32 && run < topk && run + c >= topk));
    *need = topk - __builtin_amdgcn_readlane(run, j);
    *cnt = __builtin_amdgcn_readlane(c, j);
    return ls * 32 + j;
}

// Block-wide exclusive prefix sum over the four waves; *total = the sum.  All
// threads call (one barrier).
__device__ __forceinline__ int dec_excl_sum(int v, int32_t *wcnt, int *total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int x = wave_incl_scan(v);
    if (lane == 63) wcnt[w] = x;
    __syncthreads();
    int base = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < kDecWaves; ++i) {
        const int t = wcnt[i];
        base += i < w ? t : 0;
        tot += t;
    }
    *total = tot;
    return base + x - v;
}

// The decode selection of one (sequence, KV head) into sh.sel / sh.nsel: the
// forced blocks (sink, window) and the topk eligible blocks by (score desc,
// block asc), ascending.  Thread t holds the scores of blocks base +
// [t*KPT, t*KPT + KPT) in sv (base = e_lo rounded down to 4, 0 past e_hi).
// A histogram linear in the score between the smallest and the largest
// eligible score lo, hi (from the scoring launch's per-chunk bounds; NaN in bin
// 0; with no finite spread every key lands in bin 0 and the exact fallback
// below decides), zeroed by the caller before its barrier, locates the
// threshold bin; every
// key above it is taken and, when the bin holds just the keys still needed
// (the usual case: near the threshold a bin holds about one key), all of its
// keys.  Otherwise the bin's keys are ranked exactly (at most kDecCand of
// them), or for heavier ties refined by radix passes over their 32-bit keys,
// ties then taken in block order.  Straight-line per key: no branch on a
// key's value or eligibility.  Ends with a barrier; sh.sel is then valid.
template <int KPT, int G>
__device__ __forceinline__ void dec_select(const Geo &g, const float (&sv)[KPT], const Ranges &r, int topk,
                                           float lo, float hi, DecSel &ss, DecShared<G> &sh) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int base = r.e_lo & ~3;
    const int b0 = base + tid * KPT;
    const uint32_t lo_i = (uint32_t)(r.e_lo - b0);     // keys i with i - lo_i < n_i are eligible
    const uint32_t n_i = (uint32_t)(r.e_hi - r.e_lo);
    auto valid = [&](int i) { return (uint32_t)i - lo_i < n_i; };
    const float span = hi - lo;
    float scale = (float)kDecBins / span;
    scale = hi > lo && span < INFINITY && scale < INFINITY ? scale : 0.0f;   // no finite spread: all in bin 0
    const float c0 = -lo * scale;
    // each key's bin: fma (monotone in the score), then a saturating conversion
    // (NaN and negatives to 0) and a clamp; -1 outside the eligible range
    int ib[KPT];
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
        const float f = __builtin_fmaf(sv[i], scale, c0);
        uint32_t u;
        asm("v_cvt_u32_f32 %0, %1" : "=v"(u) : "v"(f));
        ib[i] = valid(i) ? (int)min(u, (uint32_t)(kDecBins - 1)) : -1;
    }
#pragma unroll
    for (int i = 0; i < KPT; ++i) atomicAdd(&ss.hist[ib[i] >= 0 ? hist_word(ib[i]) : kDecBins + lane], 1u);
    __syncthreads();
    int need, cB;
    const int B = dec_cut(ss.hist, topk, &need, &cB);
    uint32_t mask = 0, cm = 0;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
        mask |= (uint32_t)(ib[i] > B) << i;
        cm |= (uint32_t)(ib[i] == B) << i;
    }
    if (cB == need) {                              // the whole threshold bin is taken
        mask |= cm;
    } else if (cB <= kDecCand) {
        // the bin's keys into a region per wave (wave-local offsets; keys of
        // other bins go to the lane's trash slot), then each owner ranks its
        // own, read back from LDS, against all of them: (key desc, block asc)
        const int c = __builtin_popcount(cm);
        const int wi = wave_incl_scan(c);
        const int slot0 = w * kDecCand + wi - c;
        int slot = slot0;
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const bool in = ib[i] == B;
            const int at = in ? slot : kDecWaves * kDecCand + lane;
            ss.cand_key[at] = score_key(sv[i]);
            ss.cand_b[at] = b0 + i;
            slot += in;
        }
        if (lane == 63) sh.ccnt[w] = wi;
        __syncthreads();
        for (int jo = slot0; jo < slot0 + c; ++jo) {
            const uint32_t k = ss.cand_key[jo];
            const int b = ss.cand_b[jo];
            int rank = 0;
#pragma unroll
            for (int ww = 0; ww < kDecWaves; ++ww) {
                const int n = sh.ccnt[ww];
                for (int jj = 0; jj < n; ++jj) {
                    const uint32_t kj = ss.cand_key[ww * kDecCand + jj];
                    rank += (kj > k) || (kj == k && ss.cand_b[ww * kDecCand + jj] < b);
                }
            }
            mask |= (uint32_t)(rank < need) << (b - b0);
        }
    } else {
        // Heavy ties: the need-th largest key of the bin by four 8-bit radix
        // passes over the bin's keys (256-bin histograms, each wave finding
        // the digit on its own), then
        // keys above it and the first ties in block order.
        uint32_t *h = ss.hist;
        uint32_t prefix = 0;
        int nd = need;
#pragma unroll 1
        for (int pass = 0; pass < 4; ++pass) {
            const int shift = 24 - 8 * pass;
            __syncthreads();                       // readers of the previous histogram are done
            h[tid] = 0u;
            __syncthreads();
#pragma unroll
            for (int i = 0; i < KPT; ++i) {
                const uint32_t k = score_key(sv[i]);
                const bool m = ib[i] == B && (uint32_t)((uint64_t)k >> (shift + 8)) == prefix;
                atomicAdd(&h[m ? (k >> shift) & 255u : 256u + (uint32_t)lane], 1u);
            }
            __syncthreads();
            // digit of the nd-th largest: lane l holds bins 4l .. 4l+3
            const u4v hv = reinterpret_cast<const u4v *>(h)[lane];
            const int own = (int)(hv[0] + hv[1] + hv[2] + hv[3]);
            const int incl = wave_incl_scan(own);
            const int above = __builtin_amdgcn_readlane(incl, 63) - incl;
            const int ls = __builtin_ctzll(__ballot(above < nd && above + own >= nd));
            const u4v hl = reinterpret_cast<const u4v *>(h)[ls];
            int run = __builtin_amdgcn_readlane(above, ls);
            int dig = 0;
#pragma unroll
            for (int q = 3; q >= 0; --q) {
                const bool here = dig == 0 && run < nd && run + (int)hl[q] >= nd;
                dig = here ? 4 * ls + q + 1 : dig;
                run += dig == 0 ? (int)hl[q] : 0;
            }
            nd -= run;
            prefix = (prefix << 8) | (uint32_t)(dig - 1);
        }
        const uint32_t T = prefix;                 // the threshold key; nd ties at T are taken
        int eq = 0;
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const uint32_t k = score_key(sv[i]);
            mask |= (uint32_t)(ib[i] == B && k > T) << i;
            eq += ib[i] == B && k == T;
        }
        int tot;
        int before = dec_excl_sum(eq, sh.wcnt, &tot);
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const bool tie = ib[i] == B && score_key(sv[i]) == T;
            mask |= (uint32_t)(tie && before < nd) << i;
            before += tie;
        }
        __syncthreads();                           // wcnt is reused below
    }
    // emission in block order after the sink blocks, then the forced ones
    int tot;
    int pos = g.sink + dec_excl_sum(__builtin_popcount(mask), sh.wcnt, &tot);
    for (uint32_t x = mask; x; x &= x - 1u) {
        sh.sel[pos < g.sink + topk && pos < kDecSelMax ? pos : kDecSelMax + lane] = b0 + __builtin_ctz(x);
        ++pos;
    }
    const int nwin = r.b_last - r.fw + 1;
    // forced blocks: thread t writes sink block t and window block t (a trash
    // slot when out of range); longer windows loop
    sh.sel[tid < g.sink && tid < kDecSelMax ? tid : kDecSelMax + lane] = tid;
    for (int i = tid + kDecThreads; i < g.sink && i < kDecSelMax; i += kDecThreads) sh.sel[i] = i;
    {
        const int at = g.sink + topk + tid;
        sh.sel[tid < nwin && at < kDecSelMax ? at : kDecSelMax + lane] = r.fw + tid;
    }
    for (int i = tid + kDecThreads; i < nwin; i += kDecThreads) {
        const int at = g.sink + topk + i;
        sh.sel[at < kDecSelMax ? at : kDecSelMax + lane] = r.fw + i;
    }
    if (tid == 0) sh.nsel = g.sink + topk + nwin;
    __syncthreads();
}

// Records (the scoring launch's (min, max) eligible score of each 16 blocks)
// a lane holds for a KPT-keys-a-thread selection: record lane + 64 k in
// rec[k].
template <int KPT> constexpr int dec_rpl() { return KPT / 4 + 2; }

// The selection's inputs of (sequence, KV head) `pair`, issued together: thread
// t's KPT scores of blocks base + [t*KPT, t*KPT + KPT) (base = sink rounded
// down to 4) and the lane's records.
template <int KPT>
__device__ __forceinline__ void dec_load_sel_inputs(const Geo &g, const Ws &ws, int pair, float (&sv)[KPT],
                                                    float2 (&rec)[dec_rpl<KPT>()]) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int base = g.sink & ~3;
    const BufRsrc rs = buf_rsrc(ws.scores + (int64_t)pair * ws.nb_cap, (uint32_t)ws.nb_cap * 4u);
#pragma unroll
    for (int k = 0; k < KPT / 4; ++k) {
        const auto x = BufLoad<4>::at(rs, (base + tid * KPT) * 4 + 16 * k, 0);
        sv[4 * k] = x[0]; sv[4 * k + 1] = x[1]; sv[4 * k + 2] = x[2]; sv[4 * k + 3] = x[3];
    }
    const int n_ch = ws.nb_cap / kScoreRecBlocks;
    const BufRsrc rr = buf_rsrc(ws.cmm + (int64_t)pair * n_ch, (uint32_t)n_ch * 8u);
#pragma unroll
    for (int k = 0; k < dec_rpl<KPT>(); ++k) {
        const auto x = BufLoad<2>::at(rr, (lane + 64 * k) * 8, 0);
        rec[k] = make_float2(x[0], x[1]);
    }
}

// Zero the selection histogram (before the caller's barrier).
__device__ __forceinline__ void dec_zero_hist(DecSel &ss) {
    const int tid = threadIdx.x;
    u4v *h4 = reinterpret_cast<u4v *>(ss.hist);
    const u4v z = {0u, 0u, 0u, 0u};
    h4[tid] = z;
    h4[tid + kDecThreads] = z;
    if (tid < 16) h4[2 * kDecThreads + tid] = z;
}

// The selection of one (sequence, KV head) of length L into sh.sel / sh.nsel
// (all threads; the histogram zeroed and a barrier passed since).  Returns
// min(count, max_sel), 0 for a length out of range.
template <int KPT, int G>
__device__ __forceinline__ int dec_choose(const Geo &g, const Ws &ws, int L, int max_seq_len, int max_sel,
                                          const float (&sv)[KPT], const float2 (&rec)[dec_rpl<KPT>()], DecSel &ss,
                                          DecShared<G> &sh) {
    const int tid = threadIdx.x, lane = tid & 63;
    if (!(L >= 1 && L <= max_seq_len)) return 0;
    const Ranges r = qsa_ranges(g, L);
    const int ne = r.e_hi - r.e_lo, topk = eff_topk(g, r);
    if (g.topk <= 0 || ne <= topk) {               // every block below the length
        const int nb = r.b_last + 1;
        for (int i = tid; i < nb && i < kDecSelMax; i += kDecThreads) sh.sel[i] = i;
        if (tid == 0) sh.nsel = nb;
        __syncthreads();
    } else if (topk == 0) {                        // the forced blocks fill the count
        const int nwin = r.b_last - r.fw + 1;
        for (int i = tid; i < g.sink && i < kDecSelMax; i += kDecThreads) sh.sel[i] = i;
        for (int i = tid; i < nwin; i += kDecThreads)
            if (g.sink + i < kDecSelMax) sh.sel[g.sink + i] = r.fw + i;
        if (tid == 0) sh.nsel = g.sink + nwin;
        __syncthreads();
    } else {
        // the score bounds over the records of eligible blocks (16 each, from
        // e_lo); bounds that miss some scores only make the threshold bin
        // larger, the selection stays exact
        const int n_rec = min(ws.nb_cap / kScoreRecBlocks, (ne + kScoreRecBlocks - 1) / kScoreRecBlocks);
        float lo = INFINITY, hi = -INFINITY;
#pragma unroll
        for (int k = 0; k < dec_rpl<KPT>(); ++k) {
            const bool in = lane + 64 * k < n_rec;
            lo = in && rec[k].x < lo ? rec[k].x : lo;
            hi = in && rec[k].y > hi ? rec[k].y : hi;
        }
        hi = wave_max(hi);
        lo = -wave_max(-lo);
        dec_select<KPT>(g, sv, r, topk, lo, hi, ss, sh);
    }
    return min(sh.nsel, max_sel);
}

// kSelRow: thread t's KPT scores of sequence s's shared row (the checkpoint
// indexer's, one row for every KV head), blocks base + [t*KPT, t*KPT + KPT),
// base = sink rounded down to 4.
template <int KPT>
__device__ __forceinline__ void dec_load_row(const Geo &g, const Ws &ws, int s, float (&sv)[KPT]) {
    const int tid = threadIdx.x;
    const int base = g.sink & ~3;
    const BufRsrc rs = buf_rsrc(ws.scores + (int64_t)s * ws.nb_cap, (uint32_t)ws.nb_cap * 4u);
#pragma unroll
    for (int k = 0; k < KPT / 4; ++k) {
        const auto x = BufLoad<4>::at(rs, (base + tid * KPT) * 4 + 16 * k, 0);
        sv[4 * k] = x[0]; sv[4 * k + 1] = x[1]; sv[4 * k + 2] = x[2]; sv[4 * k + 3] = x[3];
    }
}

// kSelRow: each wave's smallest and largest eligible score (NaN ignored) into
// sh.wlh, before the caller's barrier; the row has no scoring-launch records.
template <int KPT, int G>
__device__ __forceinline__ void dec_row_bounds(const Geo &g, int L, int max_seq_len, const float (&sv)[KPT],
                                               DecShared<G> &sh) {
    const int tid = threadIdx.x, lane = tid & 63;
    float lo = INFINITY, hi = -INFINITY;
    if (L >= 1 && L <= max_seq_len) {
        const Ranges r = qsa_ranges(g, L);
        const int b0 = (r.e_lo & ~3) + tid * KPT;
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const bool in = (uint32_t)(b0 + i - r.e_lo) < (uint32_t)(r.e_hi - r.e_lo);
            lo = in ? fminf(lo, sv[i]) : lo;
            hi = in ? fmaxf(hi, sv[i]) : hi;
        }
    }
    hi = wave_max(hi);
    lo = -wave_max(-lo);
    if (lane == 0) sh.wlh[tid >> 6] = make_float2(lo, hi);
}

// kSelRow: the selection of sequence s's shared row into sh.sel / sh.nsel (all
// threads; the histogram zeroed, the waves' bounds written and a barrier
// passed since).  Returns min(count, max_sel), 0 for a length out of range.
template <int KPT, int G>
__device__ __forceinline__ int dec_choose_row(const Geo &g, int L, int max_seq_len, int max_sel,
                                              const float (&sv)[KPT], DecSel &ss, DecShared<G> &sh) {
    const int tid = threadIdx.x;
    if (!(L >= 1 && L <= max_seq_len)) return 0;
    const Ranges r = qsa_ranges(g, L);
    const int ne = r.e_hi - r.e_lo, topk = eff_topk(g, r);
    if (g.topk <= 0 || ne <= topk) {               // every block below the length
        const int nb = r.b_last + 1;
        for (int i = tid; i < nb && i < kDecSelMax; i += kDecThreads) sh.sel[i] = i;
        if (tid == 0) sh.nsel = nb;
        __syncthreads();
    } else if (topk == 0) {                        // the forced blocks fill the count
        const int nwin = r.b_last - r.fw + 1;
        for (int i = tid; i < g.sink && i < kDecSelMax; i += kDecThreads) sh.sel[i] = i;
        for (int i = tid; i < nwin; i += kDecThreads)
            if (g.sink + i < kDecSelMax) sh.sel[g.sink + i] = r.fw + i;
        if (tid == 0) sh.nsel = g.sink + nwin;
        __syncthreads();
    } else {
        float lo = INFINITY, hi = -INFINITY;
#pragma unroll
        for (int w = 0; w < kDecWaves; ++w) {
            const float2 x = sh.wlh[w];
            lo = fminf(lo, x.x);
            hi = fmaxf(hi, x.y);
        }
        dec_select<KPT>(g, sv, r, topk, lo, hi, ss, sh);
    }
    return min(sh.nsel, max_sel);
}

// kSelBig: the histogram and the threshold bin's count start at zero (before
// the caller's first barrier).
__device__ __forceinline__ void dec_big_zero(DecSelBig &bs) {
    const int tid = threadIdx.x;
    u4v *h4 = reinterpret_cast<u4v *>(bs.hist);
    const u4v z = {0u, 0u, 0u, 0u};
    for (int i = tid; i < (4096 + 64) / 4; i += kDecThreads) h4[i] = z;
    if (tid == 0) { bs.ncand = 0; bs.nbin = 0; }
}

// The exact selection among the C candidates (key, block) of bs.cand, in
// block order, their keys within [kmin, kmax] (topk <= C <= kSelCandMax; the
// histogram zeroed): a 4096-bin histogram linear in the key locates the
// threshold bin; the keys above it are taken, and the bin's own keys too
// when it holds just the keys still needed, else they are ranked by (key
// desc, candidate asc -- block asc).  Thread t reads candidates u NT + t
// (consecutive lanes, consecutive LDS words) and keeps their bins, blocks and
// verdicts in registers; each round's winners are one ballot a wave.
// Candidate order is (round, wave, lane), so a winner's place is
// the winners of the (round, wave) pairs before its own (one exchange of the
// pairs' counts and a wave scan) plus those below its lane: the winners go
// out in block order after the sink blocks with no further LDS reads.
// Returns false, with nothing emitted, when the threshold bin holds more than
// kCandMax keys.  CPT rounds of kDecThreads candidates cover C (the caller
// takes the 8-round instance when C allows; dec_big_exact picks).
template <int CPT>
__device__ __forceinline__ bool dec_big_exact_r(const Geo &g, int C, int topk, uint32_t kmin, uint32_t kmax,
                                                const SelOut &out, DecSelBig &bs) {
    constexpr int NT = kDecThreads;
    static_assert(CPT * NT <= kSelCandMax && kSelCandMax / NT * kDecWaves == 64, "whole candidate rounds; a (round, wave) a lane");
    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const float sc2 = 4096.0f / ((float)(kmax - kmin) + 1.0f);
    // every round's reads are independent and go out together (a round past
    // the candidates reads slot 0 and changes nothing)
    uint32_t kb[CPT];
    int32_t bid[CPT];
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
        const int c = u * NT + tid;
        const u2v x = bs.cand[c < C ? c : 0];
        kb[u] = (uint32_t)fminf((float)(x[0] - kmin) * sc2, 4095.0f);
        bid[u] = (int32_t)x[1];
        atomicAdd(&bs.hist[c < C ? kb[u] : 4096u + (uint32_t)lane], 1u);
    }
    __syncthreads();
    if (wid == 0) hist_cut(bs, topk);
    __syncthreads();
    const uint32_t B = (uint32_t)bs.bin;
    const int need = bs.need, cB = bs.cnt_b;
    uint32_t wm = 0u;                              // bit u: candidate u NT + t is in
    if (cB > need) {                               // (uniform) rank the threshold bin
        if (cB > kCandMax) return false;
#pragma unroll
        for (int u = 0; u < CPT; ++u) {
            const int c = u * NT + tid;
            if (c < C && kb[u] == B) {
                const int at = atomicAdd(&bs.nbin, 1);
                bs.cand_key[at] = bs.cand[c][0];
                bs.cand_b[at] = c;
            }
        }
        __syncthreads();
        if (tid < cB) {
            const uint32_t k = bs.cand_key[tid];
            const int c = bs.cand_b[tid];
            int rk = 0;
            for (int jj = 0; jj < cB; ++jj) {
                const uint32_t kj = bs.cand_key[jj];
                rk += (kj > k) || (kj == k && bs.cand_b[jj] < c);
            }
            bs.cok[c] = rk < need;
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < CPT; ++u) {
            const int c = u * NT + tid;
            wm |= (uint32_t)(c < C && (kb[u] > B || (kb[u] == B && bs.cok[c]))) << u;
        }
    } else {                                       // every key of the threshold bin is in
#pragma unroll
        for (int u = 0; u < CPT; ++u) wm |= (uint32_t)(u * NT + tid < C && kb[u] >= B) << u;
    }
    // the ballots are recomputed where they are used (one compare each) rather
    // than kept: sixteen 64-bit masks would spill scalar registers
    int cnt = 0;                                   // lane u: round u's winners in this wave
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
        const int n = (int)__builtin_popcountll(__ballot((wm >> u) & 1u));
        cnt = lane == u ? n : cnt;
    }
    if (lane < kSelCandMax / NT) bs.rwin[lane * kDecWaves + wid] = cnt;   // (0 past CPT rounds)
    __syncthreads();
    const int x = bs.rwin[lane];                   // pair (lane / kDecWaves, lane % kDecWaves)
    const int ex = wave_incl_scan(x) - x;
    asm volatile("" : "+v"(wm));                   // no reuse of the counting loop's masks across the barrier
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
        const uint64_t mu = __ballot((wm >> u) & 1u);
        const int pos = __builtin_amdgcn_readlane(ex, u * kDecWaves + wid) +
                        (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mu >> 32),
                                                       __builtin_amdgcn_mbcnt_lo((uint32_t)mu, 0u));
        if (((wm >> u) & 1u) && pos < topk) out.put(g.sink + pos, bid[u]);
    }
    return true;
}

__device__ __forceinline__ bool dec_big_exact(const Geo &g, int C, int topk, uint32_t kmin, uint32_t kmax,
                                              const SelOut &out, DecSelBig &bs) {
    constexpr int R = kSelCandMax / kDecThreads;
    if (C <= R / 2 * kDecThreads) return dec_big_exact_r<R / 2>(g, C, topk, kmin, kmax, out, bs);   // (uniform)
    return dec_big_exact_r<R>(g, C, topk, kmin, kmax, out, bs);
}

// The end of a long row's selection from C candidates in bs.cand (an upper
// set of the row's eligible keys, in block order, their keys within [kmin,
// kmax]): the exact selection among them, or, when
// they number fewer than topk or more than kSelCandMax or their threshold bin
// overflows, the radix passes over the row sc; then the forced blocks.
__device__ __forceinline__ void dec_big_tail(const Geo &g, const Ranges &r, int C, int topk, uint32_t kmin,
                                             uint32_t kmax, const float *sc, const SelOut &out, DecSelBig &bs) {
    bool done = false;
    if (C >= topk && C <= kSelCandMax) done = dec_big_exact(g, C, topk, kmin, kmax, out, bs);   // (uniform)
    if (!done) {
        __syncthreads();                           // the candidate path's LDS reads are done
        select_radix<kDecThreads>(g, sc, r, topk, out, bs);
    }
    emit_forced<kDecThreads>(g, r, topk, out);
}

// kSelBig: the selection of sequence s's long row into sh.sel / sh.nsel by
// all threads (dec_big_zero and a barrier passed since).  The indexer's
// workgroups left, per chunk of kIdxChunkBlocks blocks, the eligible keys at
// or above the append launch's cut key (ws.cand, in block order, counts in
// ws.ccnt).  Thread t owns chunks kDecBigCpt t ..: their counts cc and first
// kDecBigPre slots ce came in the first round trip; they are placed into
// bs.cand in block order (a chunk's further candidates, rarely any, are read
// here) and dec_big_tail selects.  Returns min(count, max_sel), 0 for a length out of
// range.
template <int G>
__device__ __forceinline__ int dec_choose_big(const Geo &g, const Ws &ws, int s, int n_chunks,
                                              const int (&cc)[kDecBigCpt], const u2v (&ce)[kDecBigCpt][kDecBigPre], int L,
                                              int max_seq_len, int max_sel, DecSelBig &bs, DecShared<G> &sh) {
    constexpr int NT = kDecThreads;
    const int tid = threadIdx.x, lane = tid & 63;
    if (!(L >= 1 && L <= max_seq_len)) return 0;
    const Ranges r = qsa_ranges(g, L);
    const int ne = r.e_hi - r.e_lo, topk = eff_topk(g, r);
    const SelOut out{sh.sel, &sh.nsel, 0, 1};
    if (g.topk <= 0 || ne <= topk) {               // every block below the length
        const int nb = r.b_last + 1;
        for (int i = tid; i < nb && i < kDecSelMax; i += NT) sh.sel[i] = i;
        if (tid == 0) sh.nsel = nb;
    } else if (topk == 0) {                        // the forced blocks fill the count
        emit_forced<NT>(g, r, 0, out);
    } else {
        // one exchange gives every thread its offset, the count C, the range
        // of the preloaded keys and whether any chunk holds more than the
        // preloaded slots (then those keys widen the range: a second one)
        int my = 0, more = 0;
        uint32_t kmn = 0xffffffffu, kmx = 0u;
#pragma unroll
        for (int i = 0; i < kDecBigCpt; ++i) {
            const int n = cc[i];
            my += n;
            more |= n > kDecBigPre;
#pragma unroll
            for (int j = 0; j < kDecBigPre; ++j) {
                kmn = j < n ? min(kmn, ce[i][j][0]) : kmn;
                kmx = j < n ? max(kmx, ce[i][j][0]) : kmx;
            }
        }
        const int incl = wave_incl_scan(my);
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            kmn = min(kmn, (uint32_t)__shfl_xor((int)kmn, o));
            kmx = max(kmx, (uint32_t)__shfl_xor((int)kmx, o));
        }
        more = __ballot(more != 0) != 0ull;
        const int w = tid >> 6;
        if (lane == 63) bs.xch[w] = u4v{(uint32_t)incl, kmn, kmx, (uint32_t)more};
        __syncthreads();
        int off = incl - my, C = 0;
#pragma unroll
        for (int v = 0; v < kDecWaves; ++v) {
            const u4v e = bs.xch[v];
            off += v < w ? (int)e[0] : 0;
            C += (int)e[0];
            kmn = min(kmn, e[1]);
            kmx = max(kmx, e[2]);
            more |= (int)e[3];
        }
        if (C >= topk && C <= kSelCandMax) {       // (uniform)
            const uint2 *cand = ws.cand + (int64_t)s * n_chunks * kIdxChunkBlocks;
            uint32_t xmn = 0xffffffffu, xmx = 0u;  // keys past the preloaded slots
#pragma unroll
            for (int i = 0; i < kDecBigCpt; ++i) {
                const int n = cc[i];
#pragma unroll
                for (int j = 0; j < kDecBigPre; ++j) bs.cand[j < n ? off + j : kSelCandMax + lane] = ce[i][j];
                const uint2 *src = cand + (int64_t)(kDecBigCpt * tid + i) * kIdxChunkBlocks;
                for (int j = kDecBigPre; j < n; ++j) {
                    const uint2 x = src[j];
                    bs.cand[off + j] = u2v{x.x, x.y};
                    xmn = min(xmn, x.x);
                    xmx = max(xmx, x.x);
                }
                off += n;
            }
            if (more) {                            // (uniform) rare: widen the range by those keys
#pragma unroll
                for (int o = 32; o >= 1; o >>= 1) {
                    xmn = min(xmn, (uint32_t)__shfl_xor((int)xmn, o));
                    xmx = max(xmx, (uint32_t)__shfl_xor((int)xmx, o));
                }
                if (lane == 0) { bs.kred[w] = xmn; bs.kred[kDecWaves + w] = xmx; }
                __syncthreads();
#pragma unroll
                for (int v = 0; v < kDecWaves; ++v) { kmn = min(kmn, bs.kred[v]); kmx = max(kmx, bs.kred[kDecWaves + v]); }
            }
            __syncthreads();                       // the placed candidates, before dec_big_exact reads them
        }
        dec_big_tail(g, r, C, topk, kmn, kmx, ws.scores + (int64_t)s * ws.nb_cap, out, bs);
    }
    __syncthreads();
    return min(sh.nsel, max_sel);
}

// fp16 scale j (0 .. 4*NB-1, cell-major: cell i = j / NB, block kb = j % NB)
// of a lane's scale vector.
template <int NS>
__device__ __forceinline__ float scale_at(const u4v (&d)[NS], int j) {
    const uint32_t wd = d[j / 8][(j % 8) / 2];
    return h2f((uint16_t)(j % 2 ? wd >> 16 : wd & 0xffffu));
}

// grid (parts, Hkv, n_seq); part p attends tiles [p*tpw, p*tpw + tpw) of its
// (sequence, KV head), tpw <= TM.  MODE: kGiven (sel / nsel read), kDense
// (every block below the length), kSelect (the workgroup selects from
// ws.scores with KPT keys a thread; part 0 writes sel / nsel out).  Dynamic
// LDS: dec_union_bytes<HD, G, MODE, TM>() for the union, then npt_lds page
// entries (the sequence's page-table row, when parked).
template <int HD, int G, int MODE, int KPT, int TM, bool RF, int LY>
__global__ void __launch_bounds__(kDecThreads)
k_dec(Geo g, qwfn_kv_view v, const float *__restrict__ q, const int32_t *__restrict__ seq_len, int32_t max_seq_len,
      int32_t *sel, int32_t *nsel, int32_t max_sel, Ws ws, int32_t tpw, int32_t npt_lds) {
#pragma clang fp contract(off)
    // GATH: tiles of 64 cells addressed a cell at a time (V in the K layout)
    constexpr bool GATH = LY != kLyQ8;
    constexpr bool Q4 = LY == kLyQ4, F16 = LY == kLyF16;
    static_assert(G <= 16, "one matrix-core column per query head");
    static_assert(TM >= 1 && TM <= 4, "tiles a part");
    static_assert(!RF || LY == kLyQ8, "fp16-rounded K/V: q8_0 with V dim-major");
    static_assert(LY != kLyQ8K || MODE != kSelect, "gathered q8_0 tiles: a given selection, dense, kSelBig or kSelRow");
    static_assert(MODE != kSelRow || LY == kLyQ8K, "kSelRow: the checkpoint layer's shared row");
    using S = DecStage<HD, LY>;
    constexpr int NB = S::NB, ND = S::ND, NS = S::NS;
    constexpr int UB = dec_union_bytes<HD, G, MODE, TM, LY>();
    __shared__ DecShared<G> sh;
    extern __shared__ __attribute__((aligned(16))) uint8_t dec_dyn[];
    DecSel &ss = *reinterpret_cast<DecSel *>(dec_dyn);
    int32_t *ptab = reinterpret_cast<int32_t *>(dec_dyn + UB);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, hn = lane & 15, lg = lane >> 4;
    const int part = blockIdx.x, gh = blockIdx.y, s = blockIdx.z;
    const int pair = s * g.Hkv + gh;
    const int tpb = g.bt / 64;
    const int t_first = part * tpw;
    // ---- first round trip: everything that does not depend on the selection
    // (the query rows first: their split below runs while the rest is in flight)
    const int hq = min(hn, G - 1);
    float qv[NB][8];
    {
        // the B operand's eight k-values of block kb in the order of the keys' A
        // operand: dims 8 lg .. +7; q4_0 (low nibbles dims 0-15, high 16-31 of
        // a block's bytes): dims 4 lg .. +3 and 16 + 4 lg .. +3
        const float *qh = q + ((int64_t)s * g.H + (int64_t)gh * G + hq) * HD + (Q4 ? 4 : 8) * lg;
#pragma unroll
        for (int kb = 0; kb < NB; ++kb) {
            const float4 a = *reinterpret_cast<const float4 *>(qh + 32 * kb);
            const float4 b = *reinterpret_cast<const float4 *>(qh + 32 * kb + (Q4 ? 16 : 4));
            qv[kb][0] = a.x; qv[kb][1] = a.y; qv[kb][2] = a.z; qv[kb][3] = a.w;
            qv[kb][4] = b.x; qv[kb][5] = b.y; qv[kb][6] = b.z; qv[kb][7] = b.w;
        }
    }
    // prefill mode (gathered tiles): launch "sequence" s is query s of cache
    // sequence pf_seq, of length pf_pos0 + s + 1
    const int L = GATH ? seq_length(g, seq_len[g.pf ? 0 : s], s) : seq_len[s];
    const int32_t *prow = v.page_table + (int64_t)(GATH ? cache_seq(g, s) : s) * g.pps;
    const int npt = min(g.pps, (max_seq_len + g.pt - 1) / g.pt);
    const bool park = (MODE != kDense || GATH) && npt <= kDecPtLds;
    constexpr int PTV = kDecPtLds / (4 * kDecThreads);   // 16-byte page-table loads a thread at most
    u4v pt4[PTV];
    if (park) {                                    // entries past npt read 0 (never looked up)
        const BufRsrc prs = buf_rsrc(prow, (uint32_t)npt * 4u);
#pragma unroll
        for (int k = 0; k < PTV; ++k)
            if (4 * kDecThreads * k < npt_lds)
                pt4[k] = __builtin_bit_cast(u4v, BufLoad<4>::at(prs, (4 * tid + 4 * kDecThreads * k) * 4, 0));
    }
    // kSelect: the scores and the scoring launch's (min, max) records
    constexpr int KS = MODE == kSelect || MODE == kSelRow ? KPT : 4;
    float sv[KS];
    float2 rec[dec_rpl<KS>()];
    if constexpr (MODE == kSelect) dec_load_sel_inputs<KS>(g, ws, pair, sv, rec);
    if constexpr (MODE == kSelRow) dec_load_row<KS>(g, ws, s, sv);   // the sequence's shared row
    // kSelBig: the candidate counts of this thread's chunks of the sequence's row
    const int n_chunks = (max_seq_len / g.bt + kIdxChunkBlocks - 1) / kIdxChunkBlocks;
    int cc[kDecBigCpt];
    u2v ce[kDecBigCpt][kDecBigPre];                // (the first candidate slots of each chunk)
#pragma unroll
    for (int i = 0; i < kDecBigCpt; ++i) {
        const int ch = min(kDecBigCpt * tid + i, n_chunks - 1);
        cc[i] = 0;
        if constexpr (MODE == kSelBig) {
            cc[i] = kDecBigCpt * tid + i < n_chunks ? ws.ccnt[(int64_t)s * n_chunks + ch] : 0;
            const u4v *src = reinterpret_cast<const u4v *>(ws.cand + ((int64_t)s * n_chunks + ch) * kIdxChunkBlocks);
#pragma unroll
            for (int j = 0; j < kDecBigPre / 2; ++j) {
                const u4v x = src[j];
                ce[i][2 * j] = u2v{x[0], x[1]};
                ce[i][2 * j + 1] = u2v{x[2], x[3]};
            }
        }
    }
    // kSelBig after a cut placed in the indexer launch (ws.cutk set): workgroup
    // (0, 0) of the sequence sets its cut slots back to zero (that launch has
    // finished with them), for the next call
    if constexpr (MODE == kSelBig)
        if (ws.cutk && blockIdx.x == 0 && blockIdx.y == 0 && tid < kCutSlots)
            ws.cutk[(int64_t)s * kCutSlots + tid] = 0u;
    int n_given = 0;
    // kGiven: the tiles' blocks; kDense: their pages.  GATH: the block of the
    // lane's cell (lane & 15 of the wave's 16) in each tile
    int32_t pre[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int tile = t_first + min(i, tpw - 1);
        if constexpr (GATH) {
            const int slot = (tile * 64 + 16 * w + (lane & 15)) / g.bt;
            if constexpr (MODE == kGiven) pre[i] = sel[(int64_t)pair * max_sel + min(slot, max_sel - 1)];
            else pre[i] = slot;
        } else if constexpr (MODE == kGiven) {
            pre[i] = sel[(int64_t)pair * max_sel + min(tile / tpb, max_sel - 1)];
        } else if constexpr (MODE == kDense) {
            const int64_t t0 = (int64_t)(tile / tpb) * g.bt + (tile % tpb) * 64;
            pre[i] = prow[min((int)(t0 / g.pt), g.pps - 1)];
        } else {
            pre[i] = 0;
        }
    }
    if constexpr (MODE == kGiven) n_given = nsel[pair];
    if constexpr (MODE == kSelect || MODE == kSelRow) dec_zero_hist(ss);   // the selection histogram starts at zero
    if constexpr (MODE == kSelBig) dec_big_zero(*reinterpret_cast<DecSelBig *>(dec_dyn));
    // the query split: scaled by a power of two so its largest magnitude is in
    // [2^13, 2^14), then fp16 high + low parts (residual below 2^-22 of the
    // largest).  The query loads went out first, so this waits for them alone
    // and runs while the page table and the scores are still in flight.
    h8v qhi[NB], qlo[NB];
    float qfac;
    {
        float a = 0.0f;
#pragma unroll
        for (int kb = 0; kb < NB; ++kb)
#pragma unroll
            for (int e = 0; e < 8; ++e) a = fmaxf(a, fabsf(qv[kb][e]));
        a = col_max4(a);
        int ex = 0;
        frexpf(a, &ex);                            // a in [2^(ex-1), 2^ex)
        const float up = a > 0.0f ? ldexpf(1.0f, 14 - ex) : 1.0f;
        qfac = (a > 0.0f ? ldexpf(1.0f, ex - 14) : 1.0f) * g.scale_log2;
#pragma unroll
        for (int kb = 0; kb < NB; ++kb)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float x = qv[kb][e] * up;
                const _Float16 h = (_Float16)x;
                qhi[kb][e] = h;
                qlo[kb][e] = (_Float16)(x - (float)h);
            }
    }
    if (park) {
#pragma unroll
        for (int k = 0; k < PTV; ++k)
            if (4 * tid + 4 * kDecThreads * k < npt_lds)
                *reinterpret_cast<u4v *>(&ptab[4 * tid + 4 * kDecThreads * k]) = pt4[k];
    }
    const bool ok = L >= 1 && L <= max_seq_len;
    // ---- the blocks of this part's tiles
    int n = 0;
    if constexpr (MODE == kSelect) {
        __syncthreads();                           // the parked page table, the zeroed histogram
        n = dec_choose<KS>(g, ws, L, max_seq_len, max_sel, sv, rec, ss, sh);
        if (part == 0) {                           // the selection for the caller and the merge
            for (int i = tid; i < n; i += kDecThreads) sel[(int64_t)pair * max_sel + i] = sh.sel[i];
            if (tid == 0) nsel[pair] = n;
        }
    } else if constexpr (MODE == kSelRow) {
        // one shared row a sequence (ws.scores: the indexer's); its bounds from
        // the keys themselves, each wave's exchanged at the barrier
        dec_row_bounds<KS>(g, L, max_seq_len, sv, sh);
        __syncthreads();                           // the parked page table, the zeroed histogram, the bounds
        n = dec_choose_row<KS>(g, L, max_seq_len, max_sel, sv, ss, sh);
        if (part == 0) {
            for (int i = tid; i < n; i += kDecThreads) sel[(int64_t)pair * max_sel + i] = sh.sel[i];
            if (tid == 0) nsel[pair] = n;
        }
    } else if constexpr (MODE == kSelBig) {
        // one shared row a sequence (ws.scores, ws.cand, ws.ccnt: the indexer's)
        __syncthreads();                           // the parked page table, the zeroed bit map
        n = dec_choose_big<G>(g, ws, s, n_chunks, cc, ce, L, max_seq_len, max_sel,
                              *reinterpret_cast<DecSelBig *>(dec_dyn), sh);
        if (part == 0) {
            for (int i = tid; i < n; i += kDecThreads) sel[(int64_t)pair * max_sel + i] = sh.sel[i];
            if (tid == 0) nsel[pair] = n;
        }
    } else {
        if (MODE == kGiven || GATH) __syncthreads();   // the parked page table
        if (ok) {
            n = MODE == kDense ? (L - 1) / g.bt + 1 : n_given;
            n = n < max_sel ? n : max_sel;
        }
    }
    const int tiles_act = GATH ? (n * g.bt + 63) / 64 : n * tpb;
    if (!ok || t_first >= tiles_act) return;       // (uniform) no partial: the merge reads fewer parts
    const int nt = min(tpw, tiles_act - t_first);  // tiles of this part, 1 .. TM
    // ---- the tiles' pages, rows and valid cells (tiles past nt repeat the
    // last one's addresses with no valid cell, so every wait count below is
    // a constant)
    int32_t tpage[TM];
    int trow[TM], tnv[TM];
    uint32_t vm[TM];                               // GATH: valid cells of the wave's 16, bit i = cell 16w + i
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        if constexpr (GATH) {
            // the lane's cell (lane & 15): its block's token, page and row
            const int tile = t_first + min(i, nt - 1);
            const int cidx = tile * 64 + 16 * w + (lane & 15);
            const int slot = cidx / g.bt;
            int blk;
            if constexpr (MODE == kSelect || MODE == kSelBig || MODE == kSelRow) blk = sh.sel[min(slot, kDecSelMax - 1)];
            else blk = pre[min(i, nt - 1)];
            const int64_t t = (int64_t)blk * g.bt + cidx % g.bt;
            const bool in = i < nt && slot < n && blk >= 0 && t < L;
            const int tc = (int)min(max(t, (int64_t)0), (int64_t)g.pps * g.pt - 1);
            const int32_t praw = park ? ptab[min(tc / g.pt, npt - 1)] : prow[tc / g.pt];
            const bool pg_ok = praw >= 0 && praw < g.n_phys;
            if (in && !pg_ok) set_status(v.status, QWFN_STATUS_PAGE_RANGE);
            const bool valid = in && pg_ok;
            tpage[i] = valid ? praw : 0;           // an empty cell reads page 0, row 0 (in bounds), masked
            trow[i] = valid ? tc % g.pt : 0;
            vm[i] = (uint32_t)__ballot(valid) & 0xffffu;
            tnv[i] = 0;
            continue;
        }
        vm[i] = 0;
        const int tile = t_first + min(i, nt - 1);
        int blk;
        if constexpr (MODE == kSelect || MODE == kSelBig || MODE == kSelRow) blk = sh.sel[min(tile / tpb, kDecSelMax - 1)];
        else if constexpr (MODE == kGiven) blk = pre[min(i, nt - 1)];
        else blk = tile / tpb;
        const int64_t t0 = (int64_t)blk * g.bt + (tile % tpb) * 64;
        const int t0c = (int)min(max(t0, (int64_t)0), (int64_t)g.pps * g.pt - 1);
        int32_t praw;
        if constexpr (MODE == kDense) praw = pre[min(i, nt - 1)];
        else if (park) praw = ptab[min(t0c / g.pt, npt - 1)];
        else praw = prow[t0c / g.pt];
        const bool in = blk >= 0 && t0 < L;
        const bool pg_ok = praw >= 0 && praw < g.n_phys;
        if (i < nt && in && !pg_ok && tid == 0) set_status(v.status, QWFN_STATUS_PAGE_RANGE);
        tpage[i] = in && pg_ok ? praw : 0;         // an empty tile reads page 0 (in bounds), all masked
        trow[i] = t0c % g.pt;
        tnv[i] = i < nt && in && pg_ok ? min(64, L - t0c) : 0;
    }
    // ---- every transfer of the part's tiles, wave w its own cells' bytes:
    // K chunk c of cells 16w..16w+15 (256 B), V dim d of them (16 B), their
    // K and V scale rows; NL transfers a tile, in tile order
    const uint32_t sbase = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)dec_dyn);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const uint32_t wb = __builtin_amdgcn_readfirstlane(sbase + (uint32_t)((w * TM + i) * S::BYTES));
        if constexpr (GATH) {
            // lane l: chunk 4j + l/16 of cell l % 16, from that cell's page and
            // row; V in the K layout (token-major 16-byte chunks) the same way;
            // the scale rows a 16-byte chunk of CPL cells a lane (the cells of
            // one block: contiguous), addressed by the lane holding the first
            const uint8_t *kp = (const uint8_t *)v.k_pages + (int64_t)tpage[i] * g.page_bytes;
            const uint8_t *vp = (const uint8_t *)v.v_pages + (int64_t)tpage[i] * g.page_bytes;
            const int64_t co = ((int64_t)(gh * (g.pt / 64) + trow[i] / 64) * S::CH * 64 + trow[i] % 64) * 16;
#pragma unroll
            for (int j = 0; j < S::NKV; ++j)
                lds_dma16(kp + co + (int64_t)(4 * j + (lane >> 4)) * 1024, wb + S::KOFF + j * 1024);
#pragma unroll
            for (int j = 0; j < S::NKV; ++j)
                lds_dma16(vp + co + (int64_t)(4 * j + (lane >> 4)) * 1024, wb + S::VOFF + j * 1024);
            if constexpr (S::SROW > 0) {
                constexpr int SL = S::SROW / 16, CPL = 16 / (2 * NB);
                const int sc = (lane < SL ? lane : lane - SL) * CPL;
                const int32_t spg = __shfl(tpage[i], sc & 15), srw = __shfl(trow[i], sc & 15);
                const uint8_t *sp = (const uint8_t *)(lane < SL ? v.k_pages : v.v_pages) + (int64_t)spg * g.page_bytes;
                if (lane < 2 * SL) lds_dma16(sp + g.qbytes + (int64_t)(gh * g.pt + srw) * NB * 2, wb + S::SOFF);
            }
            continue;
        }
        const int64_t pb = (int64_t)tpage[i] * g.page_bytes;
        const uint8_t *kp = (const uint8_t *)v.k_pages + pb;
        const uint8_t *vp = (const uint8_t *)v.v_pages + pb;
        const int tl = gh * (g.pt / 64) + trow[i] / 64;
#pragma unroll
        for (int j = 0; j < S::NKV; ++j)
            lds_dma16(kp + ((int64_t)tl * ND + 4 * j + (lane >> 4)) * 1024 + (16 * w + (lane & 15)) * 16,
                      wb + S::KOFF + j * 1024);
#pragma unroll
        for (int j = 0; j < S::NKV; ++j)
            lds_dma16(vp + ((int64_t)tl * HD + 64 * j + lane) * 64 + 16 * w, wb + S::VOFF + j * 1024);
        constexpr int SL = S::SROW / 16;           // lanes a scale set takes
        const int64_t so = g.qbytes + (int64_t)(gh * g.pt + trow[i] + 16 * w) * NB * 2;
        const uint8_t *ssrc = lane < SL ? kp + so + 16 * lane : vp + so + 16 * (lane - SL);
        if (lane < 2 * SL) lds_dma16(ssrc, wb + S::SOFF);
    }
    // ---- pass 1: the logits of every tile as it lands, the largest V scale
    const int c0 = 16 * w + 4 * lg;                // the lane's cells c0 .. c0+3 (column hn)
    float sl[TM][4];
    u4v dvw[TM][NS];                               // the cells' V scales, 0 past the tile's valid cells
    h8v dmx = {};                                  // their running maximum magnitude
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        switch (TM - 1 - i) {                      // tile i has landed (transfers retire in order)
            case 0: wait_vmcnt<0>(); break;
            case 1: wait_vmcnt<S::NL>(); break;
            case 2: wait_vmcnt<2 * S::NL>(); break;
            default: wait_vmcnt<3 * S::NL>(); break;
        }
        const uint8_t *st = dec_dyn + (w * TM + i) * S::BYTES;
        // RF: the scales of the lane's A-operand cell hn (its K row), one a block
        uint32_t ksw[RF ? NB / 2 : 1];
        if constexpr (RF) {
#pragma unroll
            for (int k = 0; k < NB / 2; ++k)
                ksw[k] = *reinterpret_cast<const uint32_t *>(st + S::SOFF + hn * NB * 2 + 4 * k);
        }
        f4v acc[NB];
#pragma unroll
        for (int kb = 0; kb < NB; ++kb) {
            // the A operand: cell hn, the block's eight k-values of k-group lg
            h8v ka;
            if constexpr (F16) {                   // chunk 4 kb + lg: dims 32 kb + 8 lg .. +7
                ka = __builtin_bit_cast(h8v, *reinterpret_cast<const u4v *>(st + S::KOFF + (4 * kb + lg) * 256 + hn * 16));
            } else if constexpr (Q4) {             // bytes 4 lg .. +3 of chunk kb: low and high nibbles
                const uint32_t kw = *reinterpret_cast<const uint32_t *>(st + S::KOFF + kb * 256 + hn * 16 + 4 * lg);
                const h4v a = q4x4_to_h4(kw & 0x0f0f0f0fu), b = q4x4_to_h4((kw >> 4) & 0x0f0f0f0fu);
                ka = h8v{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
            } else {
                const u2v kw = *reinterpret_cast<const u2v *>(st + S::KOFF + (2 * kb + (lg >> 1)) * 256 + hn * 16 +
                                                              8 * (lg & 1));
                ka = q8x8_to_h8(make_uint2(kw[0], kw[1]));
            }
            if constexpr (RF) {
                // fp16(d * q) per element: the product of two fp16 values rounded
                // once, as the F16 cast of the exact fp32 d * q
                const half2v d2 = __builtin_bit_cast(half2v, ksw[kb / 2]);
                ka = ka * (kb % 2 ? d2[1] : d2[0]);
            }
            acc[kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qhi[kb], f4v{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
            acc[kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qlo[kb], acc[kb], 0, 0, 0);
        }
        h8v dk[NS];
#pragma unroll
        for (int k = 0; k < NS; ++k) {
            if constexpr (F16) {                   // no scales
                dk[k] = h8v{};
                dvw[i][k] = u4v{0u, 0u, 0u, 0u};
            } else {
                dk[k] = __builtin_bit_cast(h8v, *reinterpret_cast<const u4v *>(st + S::SOFF + 4 * lg * NB * 2 + 16 * k));
                dvw[i][k] = *reinterpret_cast<const u4v *>(st + S::SOFF + S::SROW + 4 * lg * NB * 2 + 16 * k);
            }
        }
        // logits of cells c0 + c (column hn): the keys' scales applied in block
        // order, each a fused multiply-add with the scale taken as fp16
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            float x = 0.0f;
#pragma unroll
            for (int kb = 0; kb < NB; ++kb)
                x = RF || F16 ? x + acc[kb][c]
                              : __builtin_fmaf((float)dk[(c * NB + kb) / 8][(c * NB + kb) % 8], acc[kb][c], x);
            const bool cv = GATH ? ((vm[i] >> (4 * lg + c)) & 1u) != 0 : c0 + c < tnv[i];
            sl[i][c] = cv ? x * qfac : -INFINITY;
        }
        // a word holds two blocks' scales of one cell: NB / 2 words a cell
#pragma unroll
        for (int k = 0; k < NS; ++k)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int cc = (4 * k + e) / (NB / 2);    // the word's cell, 0 .. 3
                const bool cv = GATH ? ((vm[i] >> (4 * lg + cc)) & 1u) != 0 : c0 + cc < tnv[i];
                if (!cv) dvw[i][k][e] = 0u;
            }
        // (q4_0 scales are signed, ggml's d = max / -8: their magnitudes)
        if constexpr (!RF && !F16)
#pragma unroll
            for (int k = 0; k < NS; ++k)
                dmx = __builtin_elementwise_max(dmx, __builtin_bit_cast(h8v, Q4 ? dvw[i][k] & 0x7fff7fffu : dvw[i][k]));
    }
    // the part's column maximum, and the column's weight scale 2^k that puts
    // its largest V scale near 2^15 (p <= 1, so every weight stays below 2^15)
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < TM; ++i)
        mx = fmaxf(mx, fmaxf(fmaxf(sl[i][0], sl[i][1]), fmaxf(sl[i][2], sl[i][3])));
    const float m = col_max4(mx);
    // RF: the V values carry their scales (F16: have none), so the weights
    // p <= 1 go up by 2^15
    float up = 0x1p15f, down = 0x1p-15f;
    if constexpr (!RF && !F16) {
        float dvm = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) dvm = fmaxf(dvm, (float)dmx[e]);
        dvm = col_max4(dvm);
        int ev = 0;
        frexpf(dvm, &ev);
        up = dvm > 0.0f ? ldexpf(1.0f, 15 - ev) : 1.0f;
        down = dvm > 0.0f ? ldexpf(1.0f, ev - 15) : 1.0f;
    }
    // ---- pass 2: weights and PV, O accumulated on the matrix cores
    f4v o[ND];
#pragma unroll
    for (int db = 0; db < ND; ++db) o[db] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
    float ls = 0.0f;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const uint8_t *st = dec_dyn + (w * TM + i) * S::BYTES;
        float pu[4];                               // the weights times 2^k (0 past the valid cells)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float p = sl[i][c] == -INFINITY ? 0.0f : fast_exp2(sl[i][c] - m);
            ls += p;
            pu[c] = p * up;
        }
        // weight of (cell c, block kb) = pu[c] * d_v(c, kb), rounded once, as
        // fp16 high + low parts (RF: pu[c] alone, the same for every block)
        constexpr int NW = RF || F16 ? 1 : NB;
        h4v bhi[NW], blo[NW];
#pragma unroll
        for (int kb = 0; kb < NW; ++kb)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                float dv = 1.0f;
                if constexpr (!RF && !F16) {
                    const h8v dw = __builtin_bit_cast(h8v, dvw[i][(c * NB + kb) / 8]);
                    dv = (float)dw[(c * NB + kb) % 8];
                }
                const _Float16 h = (_Float16)__builtin_fmaf(pu[c], dv, 0.0f);
                bhi[kb][c] = h;
                blo[kb][c] = (_Float16)__builtin_fmaf(pu[c], dv, -(float)h);
            }
        // RF: the four cells' V scales of each block (0 past the valid cells)
        h4v dvc[RF ? NB : 1];
        if constexpr (RF) {
#pragma unroll
            for (int kb = 0; kb < NB; ++kb)
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    dvc[kb][c] = __builtin_bit_cast(h8v, dvw[i][(c * NB + kb) / 8])[(c * NB + kb) % 8];
        }
        if constexpr (F16) {
            // V in the K layout, fp16: the A operand of MFMA db holds dim 16 db + hn
            // of cells 4 lg .. +3 (four 16-bit reads packed in pairs); cells that
            // carry no data are zeroed, so their zero weights meet no inf or NaN
            const uint32_t vb = vm[i] >> (4 * lg);
            const uint32_t m01 = ((vb & 1u) ? 0x0000ffffu : 0u) | ((vb & 2u) ? 0xffff0000u : 0u);
            const uint32_t m23 = ((vb & 4u) ? 0x0000ffffu : 0u) | ((vb & 8u) ? 0xffff0000u : 0u);
#pragma unroll
            for (int db = 0; db < ND; ++db) {
                uint32_t wv[4];
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    wv[c] = *reinterpret_cast<const uint16_t *>(st + S::VOFF + ((2 * db + (hn >> 3)) * 16 + 4 * lg + c) * 16 +
                                                               2 * (hn & 7));
                const uint32_t p01 = __builtin_amdgcn_perm(wv[1], wv[0], 0x05040100u) & m01;
                const uint32_t p23 = __builtin_amdgcn_perm(wv[3], wv[2], 0x05040100u) & m23;
                const h4v va = __builtin_bit_cast(h4v, u2v{p01, p23});
                o[db] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, bhi[0], o[db], 0, 0, 0);
                o[db] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, blo[0], o[db], 0, 0, 0);
            }
        } else if constexpr (Q4) {
            // V in the K layout, q4_0: byte hn of block kb's chunk holds dims
            // 32 kb + hn (low nibble) and 32 kb + 16 + hn (high); the four cells'
            // bytes packed, then the nibbles split: MFMAs 2 kb and 2 kb + 1
#pragma unroll
            for (int kb = 0; kb < NB; ++kb) {
                uint32_t wv[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) wv[c] = st[S::VOFF + (kb * 16 + 4 * lg + c) * 16 + hn];
                const uint32_t t = pack4_lo8(wv);
                const h4v v0 = q4x4_to_h4(t & 0x0f0f0f0fu), v1 = q4x4_to_h4((t >> 4) & 0x0f0f0f0fu);
                o[2 * kb] = __builtin_amdgcn_mfma_f32_16x16x16f16(v0, bhi[kb], o[2 * kb], 0, 0, 0);
                o[2 * kb] = __builtin_amdgcn_mfma_f32_16x16x16f16(v0, blo[kb], o[2 * kb], 0, 0, 0);
                o[2 * kb + 1] = __builtin_amdgcn_mfma_f32_16x16x16f16(v1, bhi[kb], o[2 * kb + 1], 0, 0, 0);
                o[2 * kb + 1] = __builtin_amdgcn_mfma_f32_16x16x16f16(v1, blo[kb], o[2 * kb + 1], 0, 0, 0);
            }
        } else if constexpr (GATH) {
            // V in the K layout: the A operand of block kb's MFMA j holds dims
            // 32 kb + 2 hn + j of cells 4 lg .. +3 (rows of one q8_0 block, so
            // the block's weights serve it), the four cells' two dims read as
            // 16-bit words and transposed with byte permutes
#pragma unroll
            for (int kb = 0; kb < NB; ++kb) {
                uint32_t wv[4];
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    wv[c] = *reinterpret_cast<const uint16_t *>(st + S::VOFF + ((2 * kb + (hn >> 3)) * 16 + 4 * lg + c) * 16 +
                                                               2 * (hn & 7));
                const uint32_t p01 = __builtin_amdgcn_perm(wv[1], wv[0], 0x05010400u);
                const uint32_t p23 = __builtin_amdgcn_perm(wv[3], wv[2], 0x05010400u);
                const uint32_t t2[2] = {__builtin_amdgcn_perm(p23, p01, 0x05040100u),
                                        __builtin_amdgcn_perm(p23, p01, 0x07060302u)};
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const h4v va = q8x4_to_h4(t2[j]);
                    o[2 * kb + j] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, bhi[kb], o[2 * kb + j], 0, 0, 0);
                    o[2 * kb + j] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, blo[kb], o[2 * kb + j], 0, 0, 0);
                }
            }
        } else {
#pragma unroll
            for (int db = 0; db < ND; ++db) {
                h4v va = q8x4_to_h4(*reinterpret_cast<const uint32_t *>(st + S::VOFF + (16 * db + hn) * 16 + 4 * lg));
                if constexpr (RF) va = va * dvc[db / 2];       // fp16(d * q) per element
                o[db] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, bhi[RF ? 0 : db / 2], o[db], 0, 0, 0);
                o[db] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, blo[RF ? 0 : db / 2], o[db], 0, 0, 0);
            }
        }
    }
    const float l = col_sum4(ls);
    // ---- the four waves' states into one partial.  A wave's O goes over its
    // own staging slots (only it reads them, so no barrier first) when they
    // hold it, else over the region start once every wave is done.
    constexpr bool kOwnSlots = G * HD * 4 <= TM * S::BYTES;
    auto wave_o = [&](int i) {
        return reinterpret_cast<float *>(dec_dyn + (kOwnSlots ? i * TM * S::BYTES : i * G * HD * 4));
    };
    if constexpr (!kOwnSlots) __syncthreads();
    if (hn < G) {
        if (lg == 0) { sh.wml[w][hn][0] = m; sh.wml[w][hn][1] = l; }
        float *wo = wave_o(w);
        if constexpr (LY == kLyQ8K) {              // o[2kb + j][r]: dim 32 kb + 8 lg + 2 r + j
#pragma unroll
            for (int kb = 0; kb < NB; ++kb) {
                const f4v a = o[2 * kb], b = o[2 * kb + 1];
                *reinterpret_cast<float4 *>(&wo[hn * HD + 32 * kb + 8 * lg]) =
                    make_float4(a[0] * down, b[0] * down, a[1] * down, b[1] * down);
                *reinterpret_cast<float4 *>(&wo[hn * HD + 32 * kb + 8 * lg + 4]) =
                    make_float4(a[2] * down, b[2] * down, a[3] * down, b[3] * down);
            }
        } else {
#pragma unroll
            for (int db = 0; db < ND; ++db)
                *reinterpret_cast<float4 *>(&wo[hn * HD + 16 * db + 4 * lg]) =
                    make_float4(o[db][0] * down, o[db][1] * down, o[db][2] * down, o[db][3] * down);
        }
    }
    __syncthreads();
    // thread t: head t / (HD / 4), dims 4 (t % (HD / 4)) .. +3; every wave's
    // (max, sum) and O of them read in one round, summed in wave order
    constexpr int TPH = HD / 4;
    const int64_t pb = ((int64_t)pair * ws.n_tiles + part) * G;
#pragma unroll
    for (int k = tid; k < G * TPH; k += kDecThreads) {
        const int h = k / TPH, d = 4 * (k % TPH);
        float mi[kDecWaves], li[kDecWaves];
        float4 oi[kDecWaves];
#pragma unroll
        for (int i = 0; i < kDecWaves; ++i) {
            mi[i] = sh.wml[i][h][0];
            li[i] = sh.wml[i][h][1];
            oi[i] = *reinterpret_cast<const float4 *>(&wave_o(i)[h * HD + d]);
        }
        float M = mi[0];
#pragma unroll
        for (int i = 1; i < kDecWaves; ++i) M = fmaxf(M, mi[i]);
        float4 O = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        float Ls = 0.0f;
#pragma unroll
        for (int i = 0; i < kDecWaves; ++i) {
            const float wt = mi[i] == -INFINITY ? 0.0f : fast_exp2(mi[i] - M);
            O.x += wt * oi[i].x;
            O.y += wt * oi[i].y;
            O.z += wt * oi[i].z;
            O.w += wt * oi[i].w;
            Ls += wt * li[i];
        }
        *reinterpret_cast<float4 *>(&ws.part_o[(pb + h) * HD + d]) = O;
        if (d == 0) *reinterpret_cast<float2 *>(&ws.part_ml[(pb + h) * 2]) = make_float2(M, Ls);
    }
}

// Prefill attention over a given per-query selection for the K layouts (LY
// != kLyQ8): grid (1, Hkv, n_q), one workgroup per (query, KV head) walking
// all of its 64-cell tiles, two staging slots a wave (tile t + 1's transfers
// in flight while tile t is computed), an online softmax per column across
// the tiles, and the four waves' states combined into the normalised output
// (no partials, no merge launch).  The tile math is k_dec's: QK with the
// query as fp16 hi + lo against exact fp16 keys, PV with the weights p * d_v *
// 2^kup as fp16 hi + lo against exact fp16 values; kup is fixed per KV head
// and call from the largest V-scale magnitude (vmax, k_pf_vmax's partial
// maxima; F16 has no scales: 2^15), so O needs no rescaling beyond the
// softmax's.  The selection row and the sequence's page-table row are parked
// in LDS.  Dynamic LDS: dec_loop_bytes<HD, G, LY>(), then npt_lds entries.
template <int HD, int G, int LY>
constexpr int dec_loop_bytes() {
    constexpr int st = 2 * kDecWaves * DecStage<HD, LY>::BYTES;
    constexpr int wo = kDecWaves * G * HD * 4;
    return ((st > wo ? st : wo) + 15) / 16 * 16;
}

template <int HD, int G, int LY>
__global__ void __launch_bounds__(kDecThreads, 2)
k_dec_loop(Geo g, qwfn_kv_view v, const float *__restrict__ q, int32_t max_seq_len, const int32_t *__restrict__ sel,
           const int32_t *__restrict__ nsel, int32_t max_sel, const float *__restrict__ vmax, float *__restrict__ out,
           int32_t npt_lds) {
#pragma clang fp contract(off)
    constexpr bool Q4 = LY == kLyQ4, F16 = LY == kLyF16;
    static_assert(LY != kLyQ8, "V in the K layout");
    static_assert(G <= 16, "one matrix-core column per query head");
    using S = DecStage<HD, LY>;
    constexpr int NB = S::NB, ND = S::ND, NS = S::NS;
    constexpr int UB = dec_loop_bytes<HD, G, LY>();
    __shared__ DecShared<G> sh;
    extern __shared__ __attribute__((aligned(16))) uint8_t dec_dyn[];
    int32_t *ptab = reinterpret_cast<int32_t *>(dec_dyn + UB);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, hn = lane & 15, lg = lane >> 4;
    const int gh = blockIdx.y, s = blockIdx.z;
    const int pair = s * g.Hkv + gh;
    // ---- first round trip: query rows, page-table row, selection row, V-scale maxima
    const int hq = min(hn, G - 1);
    float qv[NB][8];
    {
        const float *qh = q + ((int64_t)s * g.H + (int64_t)gh * G + hq) * HD + (Q4 ? 4 : 8) * lg;
#pragma unroll
        for (int kb = 0; kb < NB; ++kb) {
            const float4 a = *reinterpret_cast<const float4 *>(qh + 32 * kb);
            const float4 b = *reinterpret_cast<const float4 *>(qh + 32 * kb + (Q4 ? 16 : 4));
            qv[kb][0] = a.x; qv[kb][1] = a.y; qv[kb][2] = a.z; qv[kb][3] = a.w;
            qv[kb][4] = b.x; qv[kb][5] = b.y; qv[kb][6] = b.z; qv[kb][7] = b.w;
        }
    }
    const int L = seq_length(g, 0, s);
    const int32_t *prow = v.page_table + (int64_t)cache_seq(g, s) * g.pps;
    const int npt = min(g.pps, (max_seq_len + g.pt - 1) / g.pt);
    const bool park = npt <= kDecPtLds;
    constexpr int PTV = kDecPtLds / (4 * kDecThreads);
    u4v pt4[PTV];
    if (park) {
        const BufRsrc prs = buf_rsrc(prow, (uint32_t)npt * 4u);
#pragma unroll
        for (int k = 0; k < PTV; ++k)
            if (4 * kDecThreads * k < npt_lds)
                pt4[k] = __builtin_bit_cast(u4v, BufLoad<4>::at(prs, (4 * tid + 4 * kDecThreads * k) * 4, 0));
    }
    constexpr int SLV = kDecSelMax / kDecThreads;   // selection entries a thread parks
    int32_t sl4[SLV];
    {
        const BufRsrc srs = buf_rsrc(sel + (int64_t)pair * max_sel, (uint32_t)max_sel * 4u);
#pragma unroll
        for (int k = 0; k < SLV; ++k)
            sl4[k] = __builtin_bit_cast(int32_t, BufLoad<1>::at(srs, (tid + kDecThreads * k) * 4, 0)[0]);
    }
    const int n_raw = nsel[pair];
    float kup = 15.0f;                             // F16: the weights p <= 1 alone
    if constexpr (!F16) {
        float dvm = vmax[gh * kVmaxWg + lane % kVmaxWg];
        dvm = wave_max(dvm);
        int e2 = 0;
        frexpf(dvm, &e2);
        kup = dvm > 0.0f ? (float)(15 - e2) : 0.0f;
    }
    const float up = ldexpf(1.0f, (int)kup), down = ldexpf(1.0f, -(int)kup);
    // ---- the query split (as k_dec)
    h8v qhi[NB], qlo[NB];
    float qfac;
    {
        float a = 0.0f;
#pragma unroll
        for (int kb = 0; kb < NB; ++kb)
#pragma unroll
            for (int e = 0; e < 8; ++e) a = fmaxf(a, fabsf(qv[kb][e]));
        a = col_max4(a);
        int ex = 0;
        frexpf(a, &ex);
        const float qup = a > 0.0f ? ldexpf(1.0f, 14 - ex) : 1.0f;
        qfac = (a > 0.0f ? ldexpf(1.0f, ex - 14) : 1.0f) * g.scale_log2;
#pragma unroll
        for (int kb = 0; kb < NB; ++kb)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float x = qv[kb][e] * qup;
                const _Float16 h = (_Float16)x;
                qhi[kb][e] = h;
                qlo[kb][e] = (_Float16)(x - (float)h);
            }
    }
    if (park) {
#pragma unroll
        for (int k = 0; k < PTV; ++k)
            if (4 * tid + 4 * kDecThreads * k < npt_lds)
                *reinterpret_cast<u4v *>(&ptab[4 * tid + 4 * kDecThreads * k]) = pt4[k];
    }
#pragma unroll
    for (int k = 0; k < SLV; ++k) sh.sel[tid + kDecThreads * k] = sl4[k];
    __syncthreads();
    const bool ok = L >= 1 && L <= max_seq_len;
    const int n = ok ? min(n_raw, max_sel) : 0;
    const int tiles = (n * g.bt + 63) / 64;
    // ---- the lane's cell (lane & 15 of the wave's 16) of tile t: page, row, validity
    auto cell_of = [&](int t, int32_t &page, int &row) -> bool {
        const int cidx = t * 64 + 16 * w + (lane & 15);
        const int slot = cidx / g.bt;
        const int blk = sh.sel[min(slot, kDecSelMax - 1)];
        const int64_t tt = (int64_t)blk * g.bt + cidx % g.bt;
        const bool in = slot < n && blk >= 0 && tt < L;
        const int tc = (int)min(max(tt, (int64_t)0), (int64_t)g.pps * g.pt - 1);
        const int32_t praw = park ? ptab[min(tc / g.pt, npt - 1)] : prow[tc / g.pt];
        const bool pg_ok = praw >= 0 && praw < g.n_phys;
        if (in && !pg_ok) set_status(v.status, QWFN_STATUS_PAGE_RANGE);
        const bool valid = in && pg_ok;
        page = valid ? praw : 0;
        row = valid ? tc % g.pt : 0;
        return valid;
    };
    const uint32_t sbase = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)dec_dyn);
    // tile t's transfers into slot b: NL of them, as k_dec's gathered tiles
    auto issue = [&](int b, int32_t page, int row) {
        const uint32_t wb = __builtin_amdgcn_readfirstlane(sbase + (uint32_t)((w * 2 + b) * S::BYTES));
        const uint8_t *kp = (const uint8_t *)v.k_pages + (int64_t)page * g.page_bytes;
        const uint8_t *vp = (const uint8_t *)v.v_pages + (int64_t)page * g.page_bytes;
        const int64_t co = ((int64_t)(gh * (g.pt / 64) + row / 64) * S::CH * 64 + row % 64) * 16;
#pragma unroll
        for (int j = 0; j < S::NKV; ++j)
            lds_dma16(kp + co + (int64_t)(4 * j + (lane >> 4)) * 1024, wb + S::KOFF + j * 1024);
#pragma unroll
        for (int j = 0; j < S::NKV; ++j)
            lds_dma16(vp + co + (int64_t)(4 * j + (lane >> 4)) * 1024, wb + S::VOFF + j * 1024);
        if constexpr (S::SROW > 0) {
            constexpr int SL = S::SROW / 16, CPL = 16 / (2 * NB);
            const int sc = (lane < SL ? lane : lane - SL) * CPL;
            const int32_t spg = __shfl(page, sc & 15), srw = __shfl(row, sc & 15);
            const uint8_t *sp = (const uint8_t *)(lane < SL ? v.k_pages : v.v_pages) + (int64_t)spg * g.page_bytes;
            if (lane < 2 * SL) lds_dma16(sp + g.qbytes + (int64_t)(gh * g.pt + srw) * NB * 2, wb + S::SOFF);
        }
    };
    float m = -1e30f, ls = 0.0f;                   // running column max (finite floor) and the lane's sum
    f4v o[ND];
#pragma unroll
    for (int db = 0; db < ND; ++db) o[db] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
    int32_t pg_n = 0;
    int rw_n = 0;
    bool va_n = false;
    if (tiles > 0) {
        va_n = cell_of(0, pg_n, rw_n);
        issue(0, pg_n, rw_n);
    }
#pragma unroll 1
    for (int t = 0; t < tiles; ++t) {
        const uint32_t vm = (uint32_t)__ballot(va_n) & 0xffffu;   // this tile's valid cells of the wave
        if (t + 1 < tiles) {
            va_n = cell_of(t + 1, pg_n, rw_n);
            issue((t + 1) & 1, pg_n, rw_n);
            wait_vmcnt<S::NL>();                   // tile t has landed (transfers retire in order)
        } else {
            wait_vmcnt<0>();
        }
        const uint8_t *st = dec_dyn + (w * 2 + (t & 1)) * S::BYTES;
        // ---- QK
        f4v acc[NB];
#pragma unroll
        for (int kb = 0; kb < NB; ++kb) {
            h8v ka;
            if constexpr (F16) {
                ka = __builtin_bit_cast(h8v, *reinterpret_cast<const u4v *>(st + S::KOFF + (4 * kb + lg) * 256 + hn * 16));
            } else if constexpr (Q4) {
                const uint32_t kw = *reinterpret_cast<const uint32_t *>(st + S::KOFF + kb * 256 + hn * 16 + 4 * lg);
                const h4v a = q4x4_to_h4(kw & 0x0f0f0f0fu), b = q4x4_to_h4((kw >> 4) & 0x0f0f0f0fu);
                ka = h8v{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
            } else {
                const u2v kw = *reinterpret_cast<const u2v *>(st + S::KOFF + (2 * kb + (lg >> 1)) * 256 + hn * 16 +
                                                              8 * (lg & 1));
                ka = q8x8_to_h8(make_uint2(kw[0], kw[1]));
            }
            acc[kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qhi[kb], f4v{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
            acc[kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qlo[kb], acc[kb], 0, 0, 0);
        }
        h8v dk[NS];
        u4v dvw[NS];
#pragma unroll
        for (int k = 0; k < NS; ++k) {
            if constexpr (F16) {
                dk[k] = h8v{};
                dvw[k] = u4v{0u, 0u, 0u, 0u};
            } else {
                dk[k] = __builtin_bit_cast(h8v, *reinterpret_cast<const u4v *>(st + S::SOFF + 4 * lg * NB * 2 + 16 * k));
                dvw[k] = *reinterpret_cast<const u4v *>(st + S::SOFF + S::SROW + 4 * lg * NB * 2 + 16 * k);
            }
        }
        float sl[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            float x = 0.0f;
#pragma unroll
            for (int kb = 0; kb < NB; ++kb)
                x = F16 ? x + acc[kb][c] : __builtin_fmaf((float)dk[(c * NB + kb) / 8][(c * NB + kb) % 8], acc[kb][c], x);
            sl[c] = ((vm >> (4 * lg + c)) & 1u) ? x * qfac : -INFINITY;
        }
        if constexpr (!F16) {
#pragma unroll
            for (int k = 0; k < NS; ++k)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (!((vm >> (4 * lg + (4 * k + e) / (NB / 2))) & 1u)) dvw[k][e] = 0u;
        }
        // ---- online softmax of column hn
        const float tm = col_max4(fmaxf(fmaxf(sl[0], sl[1]), fmaxf(sl[2], sl[3])));
        const float m_new = fmaxf(m, tm);
        const float alpha = fast_exp2(m - m_new);
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
            for (int db = 0; db < ND; ++db) o[db] *= alpha;
        }
        ls *= alpha;
        m = m_new;
        float pu[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float p = sl[c] == -INFINITY ? 0.0f : fast_exp2(sl[c] - m);
            ls += p;
            pu[c] = p * up;
        }
        // ---- PV
        constexpr int NW = F16 ? 1 : NB;
        h4v bhi[NW], blo[NW];
#pragma unroll
        for (int kb = 0; kb < NW; ++kb)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                float dv = 1.0f;
                if constexpr (!F16) {
                    const h8v dw = __builtin_bit_cast(h8v, dvw[(c * NB + kb) / 8]);
                    dv = (float)dw[(c * NB + kb) % 8];
                }
                const _Float16 h = (_Float16)__builtin_fmaf(pu[c], dv, 0.0f);
                bhi[kb][c] = h;
                blo[kb][c] = (_Float16)__builtin_fmaf(pu[c], dv, -(float)h);
            }
        if constexpr (F16) {
            const uint32_t vb = vm >> (4 * lg);
            const uint32_t m01 = ((vb & 1u) ? 0x0000ffffu : 0u) | ((vb & 2u) ? 0xffff0000u : 0u);
            const uint32_t m23 = ((vb & 4u) ? 0x0000ffffu : 0u) | ((vb & 8u) ? 0xffff0000u : 0u);
#pragma unroll
            for (int db = 0; db < ND; ++db) {
                uint32_t wv[4];
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    wv[c] = *reinterpret_cast<const uint16_t *>(st + S::VOFF + ((2 * db + (hn >> 3)) * 16 + 4 * lg + c) * 16 +
                                                               2 * (hn & 7));
                const uint32_t p01 = __builtin_amdgcn_perm(wv[1], wv[0], 0x05040100u) & m01;
                const uint32_t p23 = __builtin_amdgcn_perm(wv[3], wv[2], 0x05040100u) & m23;
                const h4v va = __builtin_bit_cast(h4v, u2v{p01, p23});
                o[db] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, bhi[0], o[db], 0, 0, 0);
                o[db] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, blo[0], o[db], 0, 0, 0);
            }
        } else if constexpr (Q4) {
#pragma unroll
            for (int kb = 0; kb < NB; ++kb) {
                uint32_t wv[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) wv[c] = st[S::VOFF + (kb * 16 + 4 * lg + c) * 16 + hn];
                const uint32_t tq = pack4_lo8(wv);
                const h4v v0 = q4x4_to_h4(tq & 0x0f0f0f0fu), v1 = q4x4_to_h4((tq >> 4) & 0x0f0f0f0fu);
                o[2 * kb] = __builtin_amdgcn_mfma_f32_16x16x16f16(v0, bhi[kb], o[2 * kb], 0, 0, 0);
                o[2 * kb] = __builtin_amdgcn_mfma_f32_16x16x16f16(v0, blo[kb], o[2 * kb], 0, 0, 0);
                o[2 * kb + 1] = __builtin_amdgcn_mfma_f32_16x16x16f16(v1, bhi[kb], o[2 * kb + 1], 0, 0, 0);
                o[2 * kb + 1] = __builtin_amdgcn_mfma_f32_16x16x16f16(v1, blo[kb], o[2 * kb + 1], 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int kb = 0; kb < NB; ++kb) {
                uint32_t wv[4];
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    wv[c] = *reinterpret_cast<const uint16_t *>(st + S::VOFF + ((2 * kb + (hn >> 3)) * 16 + 4 * lg + c) * 16 +
                                                               2 * (hn & 7));
                const uint32_t p01 = __builtin_amdgcn_perm(wv[1], wv[0], 0x05010400u);
                const uint32_t p23 = __builtin_amdgcn_perm(wv[3], wv[2], 0x05010400u);
                const uint32_t t2[2] = {__builtin_amdgcn_perm(p23, p01, 0x05040100u),
                                        __builtin_amdgcn_perm(p23, p01, 0x07060302u)};
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const h4v va = q8x4_to_h4(t2[j]);
                    o[2 * kb + j] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, bhi[kb], o[2 * kb + j], 0, 0, 0);
                    o[2 * kb + j] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, blo[kb], o[2 * kb + j], 0, 0, 0);
                }
            }
        }
        // this slot's LDS reads are done before tile t + 2's transfers reuse it
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    const float l = col_sum4(ls);
    // ---- the four waves' states into the output of the query's heads
    __syncthreads();                               // every wave is done with the staging slots
    float *wo = reinterpret_cast<float *>(dec_dyn + w * G * HD * 4);
    if (hn < G) {
        if (lg == 0) { sh.wml[w][hn][0] = m; sh.wml[w][hn][1] = l; }
        if constexpr (LY == kLyQ8K) {              // o[2kb + j][r]: dim 32 kb + 8 lg + 2 r + j
#pragma unroll
            for (int kb = 0; kb < NB; ++kb) {
                const f4v a = o[2 * kb], b = o[2 * kb + 1];
                *reinterpret_cast<float4 *>(&wo[hn * HD + 32 * kb + 8 * lg]) =
                    make_float4(a[0] * down, b[0] * down, a[1] * down, b[1] * down);
                *reinterpret_cast<float4 *>(&wo[hn * HD + 32 * kb + 8 * lg + 4]) =
                    make_float4(a[2] * down, b[2] * down, a[3] * down, b[3] * down);
            }
        } else {
#pragma unroll
            for (int db = 0; db < ND; ++db)
                *reinterpret_cast<float4 *>(&wo[hn * HD + 16 * db + 4 * lg]) =
                    make_float4(o[db][0] * down, o[db][1] * down, o[db][2] * down, o[db][3] * down);
        }
    }
    __syncthreads();
    constexpr int TPH = HD / 4;
#pragma unroll
    for (int k = tid; k < G * TPH; k += kDecThreads) {
        const int h = k / TPH, d = 4 * (k % TPH);
        float mi[kDecWaves], li[kDecWaves];
        float4 oi[kDecWaves];
#pragma unroll
        for (int i = 0; i < kDecWaves; ++i) {
            mi[i] = sh.wml[i][h][0];
            li[i] = sh.wml[i][h][1];
            oi[i] = *reinterpret_cast<const float4 *>(dec_dyn + (i * G * HD + h * HD + d) * 4);
        }
        float M = mi[0];
#pragma unroll
        for (int i = 1; i < kDecWaves; ++i) M = fmaxf(M, mi[i]);
        float4 O = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        float Ls = 0.0f;
#pragma unroll
        for (int i = 0; i < kDecWaves; ++i) {
            const float wt = fast_exp2(mi[i] - M);
            O.x += wt * oi[i].x;
            O.y += wt * oi[i].y;
            O.z += wt * oi[i].z;
            O.w += wt * oi[i].w;
            Ls += wt * li[i];
        }
        const float inv = Ls > 0.0f ? 1.0f / Ls : 0.0f;
        *reinterpret_cast<float4 *>(&out[((int64_t)s * g.H + (int64_t)gh * G + h) * HD + d]) =
            make_float4(O.x * inv, O.y * inv, O.z * inv, O.w * inv);
    }
    if (!ok && tid == 0 && gh == 0) set_status(v.status, QWFN_STATUS_LEN_RANGE);
}

// Workgroups of one k_dec instantiation a CU holds: its register-bound
// occupancy (looked up once per device) against the LDS its launch asks for.
constexpr int kResDevices = 64;
struct DecRes {
    int per_cu, cus, lds_cu, lds_static;
};
template <int HD, int G, int MODE, int KPT, int TM, bool RF, int LY>
bool dec_res(DecRes *out) {
    static std::atomic<int> cache[kResDevices][4];
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kResDevices) return false;
    std::atomic<int> *c = cache[dev];
    if (c[0].load(std::memory_order_acquire) <= 0) {
        int per_cu = 0, cus = 0, lds_cu = 0;
        hipFuncAttributes fa;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_dec<HD, G, MODE, KPT, TM, RF, LY>, kDecThreads, 0) !=
                hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipDeviceGetAttribute(&lds_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) != hipSuccess ||
            hipFuncGetAttributes(&fa, reinterpret_cast<const void *>(k_dec<HD, G, MODE, KPT, TM, RF, LY>)) != hipSuccess)
            return false;
        c[1].store(cus, std::memory_order_relaxed);
        c[2].store(lds_cu, std::memory_order_relaxed);
        c[3].store((int)fa.sharedSizeBytes, std::memory_order_relaxed);
        c[0].store(per_cu > 0 ? per_cu : 1, std::memory_order_release);
    }
    out->per_cu = c[0].load(std::memory_order_acquire);
    out->cus = c[1].load(std::memory_order_relaxed);
    out->lds_cu = c[2].load(std::memory_order_relaxed);
    out->lds_static = c[3].load(std::memory_order_relaxed);
    return true;
}

// Parked page-table entries of a launch (0: the row is looked up in memory).
inline int dec_npt_lds(const Geo &g, int32_t max_seq_len, int mode) {
    const int npt = std::min(g.pps, (int)(((int64_t)max_seq_len + g.pt - 1) / g.pt));
    return mode != kDense && npt <= kDecPtLds ? (npt + 3) / 4 * 4 : 0;
}

// Resident workgroups of the TM instantiation at this launch's LDS (0 when
// unknown).
template <int HD, int G, int MODE, int KPT, int TM, bool RF, int LY>
int64_t dec_resident(int dyn_bytes) {
    DecRes r;
    if (!dec_res<HD, G, MODE, KPT, TM, RF, LY>(&r)) return 0;
    int per = r.per_cu;
    const int lds = r.lds_static + dyn_bytes;
    if (r.lds_cu > 0 && lds > 0) per = std::min(per, r.lds_cu / lds);
    return (int64_t)std::max(per, 0) * r.cus;
}

template <int HD, int G, int MODE, int KPT, int TM, bool RF, int LY>
void launch_dec_tm(const Geo &g, const qwfn_kv_view &v, const float *q, const int32_t *seq_len, int32_t n_seq,
                   int32_t max_seq_len, int32_t *sel, int32_t *nsel, int32_t max_sel, const Ws &ws, int npt_lds,
                   int dyn, hipStream_t st) {
    const int parts = (ws.n_tiles + TM - 1) / TM;
    QWFN_LAUNCH_SHM(kTimedAttention, (k_dec<HD, G, MODE, KPT, TM, RF, LY>),
                    dim3((unsigned)parts, (unsigned)g.Hkv, (unsigned)n_seq), dim3(kDecThreads), (unsigned)dyn, st,
                    g, v, q, seq_len, max_seq_len, sel, nsel, max_sel, ws, (int32_t)TM, (int32_t)npt_lds);
}

// Launches k_dec; returns the tiles a workgroup took.  One tile a workgroup
// unless the grid would then not be resident at once (a second round of
// workgroups starts only when the first ends): then two, or four when two do
// not fit either and four keep more tiles resident.
template <int HD, int G, int MODE, int KPT, bool RF, int LY>
int launch_dec_t(const Geo &g, const qwfn_kv_view &v, const float *q, const int32_t *seq_len, int32_t n_seq,
                 int32_t max_seq_len, int32_t *sel, int32_t *nsel, int32_t max_sel, const Ws &ws, hipStream_t st) {
    const int64_t pairs = (int64_t)n_seq * g.Hkv;
    const int npt_lds = dec_npt_lds(g, max_seq_len, LY != kLyQ8 ? kGiven : MODE);
    const int d1 = dec_union_bytes<HD, G, MODE, 1, LY>() + 4 * npt_lds;
    const int d2 = dec_union_bytes<HD, G, MODE, 2, LY>() + 4 * npt_lds;
    const int d4 = dec_union_bytes<HD, G, MODE, 4, LY>() + 4 * npt_lds;
    const int64_t r1 = dec_resident<HD, G, MODE, KPT, 1, RF, LY>(d1);
    if (r1 <= 0 || pairs * ws.n_tiles <= r1) {
        launch_dec_tm<HD, G, MODE, KPT, 1, RF, LY>(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel, ws, npt_lds,
                                           d1, st);
        return 1;
    }
    // a grid larger than the device holds: two tiles a workgroup unless four
    // keep more tiles in flight (measured: the checkpoint's prefill attention
    // 10.6 ms at two, 11.8 at four, where four leave one wave a SIMD)
    const int64_t r2 = dec_resident<HD, G, MODE, KPT, 2, RF, LY>(d2);
    const int64_t r4 = dec_resident<HD, G, MODE, KPT, 4, RF, LY>(d4);
    if (pairs * ((ws.n_tiles + 1) / 2) <= r2 || 2 * r2 >= 4 * r4) {
        launch_dec_tm<HD, G, MODE, KPT, 2, RF, LY>(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel, ws, npt_lds,
                                           d2, st);
        return 2;
    }
    launch_dec_tm<HD, G, MODE, KPT, 4, RF, LY>(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel, ws, npt_lds, d4,
                                       st);
    return 4;
}

template <int HD, int G, bool RF, int LY>
hipError_t launch_dec_shape(const Geo &g, const qwfn_kv_view &v, const float *q, const int32_t *seq_len,
                            int32_t n_seq, int32_t max_seq_len, const int32_t *sel, const int32_t *nsel,
                            int32_t max_sel, float *out, const Ws &ws, bool select, hipStream_t st) {
    int32_t *sl = const_cast<int32_t *>(sel), *ns = const_cast<int32_t *>(nsel);
    int tpw;
    if constexpr (LY == kLyQ8K) {                  // gathered q8_0 tiles: a given selection or dense
        if (select) return hipErrorInvalidValue;
        tpw = sel ? launch_dec_t<HD, G, kGiven, 4, RF, LY>(g, v, q, seq_len, n_seq, max_seq_len, sl, ns, max_sel, ws, st)
                  : launch_dec_t<HD, G, kDense, 4, RF, LY>(g, v, q, seq_len, n_seq, max_seq_len, sl, ns, max_sel, ws, st);
    } else if (select) {
        const Ranges span_r{0, 0, g.sink, max_seq_len / g.bt};
        const int span = span_r.e_hi - (span_r.e_lo & ~3);
        if (span <= 4 * kDecThreads)
            tpw = launch_dec_t<HD, G, kSelect, 4, RF, LY>(g, v, q, seq_len, n_seq, max_seq_len, sl, ns, max_sel, ws, st);
        else if (span <= 8 * kDecThreads)
            tpw = launch_dec_t<HD, G, kSelect, 8, RF, LY>(g, v, q, seq_len, n_seq, max_seq_len, sl, ns, max_sel, ws, st);
        else if (span <= 16 * kDecThreads)
            tpw = launch_dec_t<HD, G, kSelect, 16, RF, LY>(g, v, q, seq_len, n_seq, max_seq_len, sl, ns, max_sel, ws, st);
        else if (span <= 32 * kDecThreads)
            tpw = launch_dec_t<HD, G, kSelect, 32, RF, LY>(g, v, q, seq_len, n_seq, max_seq_len, sl, ns, max_sel, ws, st);
        else
            return hipErrorInvalidValue;
    } else if (sel) {
        tpw = launch_dec_t<HD, G, kGiven, 4, RF, LY>(g, v, q, seq_len, n_seq, max_seq_len, sl, ns, max_sel, ws, st);
    } else {
        tpw = launch_dec_t<HD, G, kDense, 4, RF, LY>(g, v, q, seq_len, n_seq, max_seq_len, sl, ns, max_sel, ws, st);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_merge(g, v, seq_len, n_seq, max_seq_len, select ? ns : nsel, max_sel, !select && !sel, out, ws,
                        tpw, st);
}

// kSelRow: the attention selecting from one shared row a sequence (the
// checkpoint indexer's scores, at most 32 keys a thread), then the merge.
template <int HD, int G, int LY>
hipError_t launch_dec_selrow_t(const Geo &g, const qwfn_kv_view &v, const float *q, const int32_t *seq_len,
                               int32_t n_seq, int32_t max_seq_len, int32_t *sel, int32_t *nsel, int32_t max_sel,
                               float *out, const Ws &ws, hipStream_t st) {
    const int span = max_seq_len / g.bt - (g.sink & ~3);
    int tpw;
    if (span <= 4 * kDecThreads)
        tpw = launch_dec_t<HD, G, kSelRow, 4, false, LY>(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel, ws, st);
    else if (span <= 8 * kDecThreads)
        tpw = launch_dec_t<HD, G, kSelRow, 8, false, LY>(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel, ws, st);
    else if (span <= 16 * kDecThreads)
        tpw = launch_dec_t<HD, G, kSelRow, 16, false, LY>(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel, ws, st);
    else if (span <= 32 * kDecThreads)
        tpw = launch_dec_t<HD, G, kSelRow, 32, false, LY>(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel, ws, st);
    else
        return hipErrorInvalidValue;
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_merge(g, v, seq_len, n_seq, max_seq_len, nsel, max_sel, false, out, ws, tpw, st);
}

// kSelBig: the attention selecting from one long shared row a sequence (the
// indexer's candidates ws.cand / ws.ccnt, its scores ws.scores for the
// fallback), one tile a workgroup, then the merge.
template <int HD, int G, int LY>
hipError_t launch_dec_selbig_t(const Geo &g, const qwfn_kv_view &v, const float *q, const int32_t *seq_len,
                               int32_t n_seq, int32_t max_seq_len, int32_t *sel, int32_t *nsel, int32_t max_sel,
                               float *out, const Ws &ws, hipStream_t st) {
    const int npt_lds = dec_npt_lds(g, max_seq_len, kGiven);
    const int dyn = dec_union_bytes<HD, G, kSelBig, 1, LY>() + 4 * npt_lds;
    launch_dec_tm<HD, G, kSelBig, kDecBigRnd, 1, false, LY>(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel,
                                                            ws, npt_lds, dyn, st);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_merge(g, v, seq_len, n_seq, max_seq_len, nsel, max_sel, false, out, ws, 1, st);
}

// The selection of kSelBig alone, for the test entry point: one workgroup a
// sequence over its score row (rows of nb_cap), the selection written out.
// The inputs the product path takes from the append and indexer launches are
// restated on the row itself: the cut from kIdxCutSamples evenly spaced scores
// (sample_cut_of, cut_key over the indexer's four samples a thread), then, per
// chunk of kIdxChunkBlocks eligible blocks (one a wave at a time), the keys at
// or above it as candidates in block order; dec_big_tail selects.
__global__ void __launch_bounds__(kDecThreads)
k_test_select_big(Geo g, const float *scores, int32_t nb_cap, const int32_t *seq_len, int32_t max_seq_len,
                  int32_t *sel, int32_t *nsel, int32_t max_sel) {
    constexpr int NT = kDecThreads;
    __shared__ DecShared<1> sh;
    extern __shared__ __attribute__((aligned(16))) uint8_t dec_dyn[];
    DecSelBig &bs = *reinterpret_cast<DecSelBig *>(dec_dyn);
    const int s = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int L = seq_len[s];
    const float *sc = scores + (int64_t)s * nb_cap;
    dec_big_zero(bs);
    __syncthreads();
    int n = 0;
    if (L >= 1 && L <= max_seq_len) {
        const Ranges r = qsa_ranges(g, L);
        const int ne = r.e_hi - r.e_lo, topk = eff_topk(g, r);
        const SelOut out{sh.sel, &sh.nsel, 0, 1};
        if (g.topk <= 0 || ne <= topk) {
            const int nb = r.b_last + 1;
            for (int i = tid; i < nb && i < kDecSelMax; i += NT) sh.sel[i] = i;
            if (tid == 0) sh.nsel = nb;
        } else if (topk == 0) {
            emit_forced<NT>(g, r, 0, out);
        } else {
            const BufRsrc rsc = buf_rsrc(sc, (uint32_t)r.e_hi * 4u);
            const int rs = sample_rank<kIdxCutSamples>(r, topk);
            uint32_t tk = 0u;                      // no cut: every key a candidate
            if (rs > 0) {
                float sv[kIdxCutSamples / NT];
                sample_load<NT, 0, kIdxCutSamples>(rsc, r, sv);
                const CutMap cut = sample_cut_of<NT>(sv, rs, bs);
                tk = cut_key<NT>(cut, sv, bs.kred);
                u4v *h4 = reinterpret_cast<u4v *>(bs.hist);
                for (int i = tid; i < (4096 + 64) / 4; i += NT) h4[i] = u4v{0u, 0u, 0u, 0u};
            }
            uint32_t kmn = 0xffffffffu, kmx = 0u;
            int run = 0;                           // candidates of the chunks before (uniform)
#pragma unroll 1
            for (int c0 = 0; c0 * kIdxChunkBlocks < ne; c0 += kDecWaves) {
                const int b = r.e_lo + (c0 + w) * kIdxChunkBlocks + lane;
                const uint32_t k = score_key(BufLoad<1>::at(rsc, b * 4, 0)[0]);
                const bool in = b < r.e_hi && k >= tk;
                const uint64_t m = __ballot(in);
                if (lane == 0) bs.tmp[w] = __builtin_popcountll(m);
                __syncthreads();
                int at = run + __builtin_popcountll(m & ((1ull << lane) - 1ull)), tot = 0;
#pragma unroll
                for (int i = 0; i < kDecWaves; ++i) {
                    at += i < w ? bs.tmp[i] : 0;
                    tot += bs.tmp[i];
                }
                if (in && at < kSelCandMax) bs.cand[at] = u2v{k, (uint32_t)b};
                kmn = in ? min(kmn, k) : kmn;
                kmx = in ? max(kmx, k) : kmx;
                run += tot;
                __syncthreads();
            }
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                kmn = min(kmn, (uint32_t)__shfl_xor((int)kmn, o));
                kmx = max(kmx, (uint32_t)__shfl_xor((int)kmx, o));
            }
            if (lane == 0) { bs.kred[w] = kmn; bs.kred[kDecWaves + w] = kmx; }
            __syncthreads();
#pragma unroll
            for (int i = 0; i < kDecWaves; ++i) { kmn = min(kmn, bs.kred[i]); kmx = max(kmx, bs.kred[kDecWaves + i]); }
            dec_big_tail(g, r, run, topk, kmn, kmx, sc, out, bs);
        }
        __syncthreads();
        n = min(sh.nsel, max_sel);
    }
    for (int i = tid; i < n; i += NT) sel[(int64_t)s * max_sel + i] = sh.sel[i];
    if (tid == 0) nsel[s] = n;
}

template <int HD, int G, int LY>
hipError_t launch_dec_loop_t(const Geo &g, const qwfn_kv_view &v, const float *q, int32_t n_q, int32_t max_seq_len,
                             const int32_t *sel, const int32_t *nsel, int32_t max_sel, const float *vmax, float *out,
                             hipStream_t st) {
    if (max_sel > kDecSelMax) return hipErrorInvalidValue;
    const int npt_lds = dec_npt_lds(g, max_seq_len, kGiven);
    const int dyn = dec_loop_bytes<HD, G, LY>() + 4 * npt_lds;
    hipLaunchKernelGGL((k_dec_loop<HD, G, LY>), dim3(1u, (unsigned)g.Hkv, (unsigned)n_q), dim3(kDecThreads),
                       (unsigned)dyn, st, g, v, q, max_seq_len, sel, nsel, max_sel, vmax, out, (int32_t)npt_lds);
    return hipGetLastError();
}

}  // namespace

}  // namespace qwfn_qsa
