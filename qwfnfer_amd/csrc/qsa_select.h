// qsa_select.h -- the block selection of the QSA indexer: the forced/eligible
// rule's top-k over a score row by (score desc, block asc), as device routines
// templated on the workgroup size and its LDS struct.  Shared by the indexer
// and selection kernels (qsa_kernels.hip) and by the matrix-core decode
// attention, whose workgroups select for themselves (qsa_dec_kernel.h).
// Compiled with fp contraction off by every including kernel.
#pragma once

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include "qsa_append.h"
#include "qsa_device.h"

namespace qwfn_qsa {

// ---------------------------------------------------------------------------
// indexer: scores of the eligible blocks, then top-k in the last workgroup
// ---------------------------------------------------------------------------

constexpr int kIdxThreads = 256;
constexpr int kBlocksPerChunk = kIdxThreads / 4;   // 4 lanes share one block's dot
static_assert(kBlocksPerChunk == kIdxChunkBlocks, "an indexer workgroup's candidate slots");
constexpr int kKeysMax = 32 * kIdxThreads;        // eligible blocks the register selection holds
static_assert(kKeysMax == kIdxRegKeys, "the workspace sizes the long-context selection by this bound");

constexpr int kCandMax = 256;                      // threshold-bin candidates ranked exactly

struct IdxShared {
    union {
        float q[16 * 256];                         // scoring: the group's query heads
        struct { int8_t q8[kStageRows * 256]; uint16_t sc[kStageRows * 8]; } st;  // pooling
    } u;
    uint32_t hist[4096 + 64];                      // + one trash bin per lane for masked-off keys
    uint32_t cand_key[kCandMax + 1];               // + a trash slot
    int32_t cand_b[kCandMax + 1];
    uint32_t tmask[kIdxThreads];                   // selection: each thread's taken-block bits
    uint32_t selbits[kKeysMax / 32 + 1];
    float newk[256];
    float red[2 * (kIdxThreads / 64)];             // selection: per-wave max, min
    int tmp[16];
    int flag, bin, need, ncand, cnt_b;
    uint32_t cut_tk, cut_kb;                       // the in-launch cut (idx_wait_cut)
    int cut_in;
};



// ---------------------------------------------------------------------------
// block selection
// ---------------------------------------------------------------------------
// The routines below are templates over the workgroup size NT and its LDS
// struct SH: IdxShared for the 256-thread indexer workgroup, BigSelShared for
// the 1024-thread selection of long contexts (k_select_big).  SH provides
// hist[4096 + 64], cand_key / cand_b[kCandMax + 1], tmask[NT] (32 or 64 bits a
// thread), selbits, red[2 * NT/64], tmp[NT/64] and bin, need, ncand, cnt_b.

template <int NT, int NB, typename SH> __device__ void find_bin(SH &sh, int need);

// One radix pass over the eligible keys that match `prefix` above bit
// shift+BITS: histogram of the BITS-bit digit at `shift`, then the digit of
// the need-th largest key.  Updates prefix (appending the digit) and need.
template <int NT, int BITS, typename SH>
__device__ void radix_pass(SH &sh, const float *sc, int e_lo, int e_hi, int shift, uint32_t &prefix,
                           int &need, bool first) {
    constexpr int NB = 1 << BITS;
    const int tid = threadIdx.x;
    for (int i = tid; i < NB; i += NT) sh.hist[i] = 0u;
    __syncthreads();
    for (int b = e_lo + tid; b < e_hi; b += NT) {
        const uint32_t k = score_key(sc[b]);
        if (first || (k >> (shift + BITS)) == prefix) atomicAdd(&sh.hist[(k >> shift) & (NB - 1)], 1u);
    }
    __syncthreads();
    find_bin<NT, NB>(sh, need);
    prefix = first ? (uint32_t)sh.bin : ((prefix << BITS) | (uint32_t)sh.bin);
    need = sh.need;
    __syncthreads();
}

// The digit of the need-th largest key from an NB-bin histogram in LDS
// (bins in ascending key order): sh.bin = that digit, sh.need = how many keys
// of that bin are still needed.  All threads call.
template <int NT, int NB, typename SH>
__device__ void find_bin(SH &sh, int need) {
    constexpr int PER = NB / NT > 0 ? NB / NT : 1;
    const int tid = threadIdx.x;
    int own = 0;
    if (tid * PER < NB)
#pragma unroll
        for (int i = 0; i < PER; ++i) own += (int)sh.hist[tid * PER + i];
    int total;
    const int excl = block_excl_sum<NT>(own, sh.tmp, &total);
    const int above = total - excl - own;          // keys in the bins of higher threads
    if (tid * PER < NB && above < need && above + own >= need) {
        int run = above;
        for (int i = PER - 1; i >= 0; --i) {
            const int c = (int)sh.hist[tid * PER + i];
            if (run + c >= need) { sh.bin = tid * PER + i; sh.need = need - run; break; }
            run += c;
        }
    }
    __syncthreads();
}

// Where a selection goes: row 0 and its count, and `rows` rows in all, each
// `stride` entries after the previous, with consecutive counts (a shared
// selection writes every KV head's row; otherwise rows = 1).
struct SelOut {
    int32_t *p, *n;
    int64_t stride;
    int rows;
    __device__ __forceinline__ void put(int i, int32_t b) const {
        for (int h = 0; h < rows; ++h) p[h * stride + i] = b;
    }
    __device__ __forceinline__ void count(int c) const {
        for (int h = 0; h < rows; ++h) n[h] = c;
    }
};
__device__ __forceinline__ SelOut sel_out(const Geo &g, int32_t *sel, int32_t *nsel, int32_t max_sel, int s,
                                          int pair) {
    return g.shared ? SelOut{sel + (int64_t)s * g.sel_rows * max_sel, nsel + s * g.sel_rows, max_sel, g.sel_rows}
                    : SelOut{sel + (int64_t)pair * max_sel, nsel + pair, max_sel, 1};
}

// The threshold bin of a 4096-bin histogram in LDS (bins in ascending key
// order) for the topk-th largest key, by wave 0: lane l sums bins [64l,
// 64l+64); the lane whose bins straddle that key is found by a scan and a
// ballot, then its 64 bins are spread over the wave for the same search.
// Sets sh.bin, sh.need (keys of that bin still needed) and sh.cnt_b (its
// keys).  Wave 0 calls it; the caller synchronizes after.
template <typename SH>
__device__ __forceinline__ void hist_cut(SH &sh, int topk) {
    const int lane = threadIdx.x & 63;
    const uint4 *h4 = reinterpret_cast<const uint4 *>(sh.hist);
    uint32_t own = 0;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const uint4 x = h4[lane * 16 + k];
        own += x.x + x.y + x.z + x.w;
    }
    const int incl = wave_incl_scan((int)own);
    const int total = __builtin_amdgcn_readlane(incl, 63);
    const int above = total - incl;                   // keys in the bins of higher lanes
    const int ls = __builtin_ctzll(__ballot(above < topk && above + (int)own >= topk));
    const int above_l = __builtin_amdgcn_readlane(above, ls);
    const int c = (int)sh.hist[ls * 64 + lane];
    const int ic = wave_incl_scan(c);
    const int run = above_l + __builtin_amdgcn_readlane(ic, 63) - ic;   // keys in higher bins
    const int j = __builtin_ctzll(__ballot(run < topk && run + c >= topk));
    if (lane == j) { sh.bin = ls * 64 + j; sh.need = topk - run; sh.cnt_b = c; }
}

// Selection of one (sequence, KV head): the topk eligible blocks by (score
// desc, index asc) on orderable 32-bit keys, emitted ascending between the
// forced sink and window blocks.
//
// Register path (select_regs): thread t holds the KPT scores of blocks
// base + [t*KPT, t*KPT+KPT) (base = e_lo rounded down to 4) in registers,
// loaded as aligned 16-byte vectors in one round trip.  A 4096-bin histogram,
// linear in the score between the smallest and largest score (monotone in
// the key order, NaN in bin 0; scores with no finite spread bin on the top 12
// key bits instead), locates the threshold bin; wave 0 finds it with DPP
// scans and ballots.  When that bin holds exactly the keys still needed (the
// usual case: near the threshold a bin holds about one key) every key of it
// is taken; otherwise its keys are ranked exactly against each other.  Each
// thread then publishes a bit mask of its taken blocks and wave 0 writes them
// in order.  The code is straight-line and predicated where it can be: in
// the indexer it runs once per layer in one workgroup, from a cold
// instruction cache.  KEEP keeps each key's bin in a register (else it is
// recomputed from the key: the 1024-thread variant has half the registers).
//
// Fallback (select_radix): a threshold bin of more than kCandMax keys (heavy
// ties) or more eligible blocks than the register path holds takes three
// radix passes over the keys in memory and an index-ordered tie count.
template <int NT, int KPT, bool KEEP, typename SH>
__device__ __forceinline__ bool select_regs(const Geo &g, const float *sc, const Ranges &r, int topk,
                                            const SelOut &out, SH &sh) {
    static_assert(KPT % 4 == 0 && (KPT <= 32 || (KPT % 8 == 0 && KPT <= 48) || KPT == 64),
                  "KPT: whole 16-byte vectors, a thread's bits within two aligned words");
    using MT = typename std::conditional<(KPT > 32), uint64_t, uint32_t>::type;
    static_assert(sizeof(sh.tmask) >= NT * sizeof(MT), "tmask holds a thread's bits");
    static_assert(sizeof(sh.selbits) >= (NT * KPT / 32 + 1) * 4, "selbits holds every key's bit");
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int base = r.e_lo & ~3;
    const int b0 = base + tid * KPT;
    // sc is 16-byte aligned; device-coherent buffer loads (the scoring
    // workgroups' released stores, no L2 invalidate), reads past e_hi give 0
    const BufRsrc rs = buf_rsrc(sc, (uint32_t)((r.e_hi + 3) & ~3) * 4u);   // whole vectors (row padded to 64)
    float sv[KPT];
#pragma unroll
    for (int k = 0; k < KPT / 4; ++k) {
        const auto x = BufLoad<4, kCpolSc1>::at(rs, b0 * 4 + 16 * k, 0);
        sv[4 * k] = x[0]; sv[4 * k + 1] = x[1]; sv[4 * k + 2] = x[2]; sv[4 * k + 3] = x[3];
    }
    auto valid = [&](int i) { return b0 + i >= r.e_lo && b0 + i < r.e_hi; };
    float lo = INFINITY, hi = -INFINITY;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
        const bool use = valid(i) && sv[i] == sv[i];
        lo = fminf(lo, use ? sv[i] : INFINITY);
        hi = fmaxf(hi, use ? sv[i] : -INFINITY);
    }
    hi = wave_max(hi);
    lo = -wave_max(-lo);
    if (lane == 0) { sh.red[wid] = hi; sh.red[NT / 64 + wid] = lo; }
    uint4 *h4 = reinterpret_cast<uint4 *>(sh.hist);
#pragma unroll
    for (int i = 0; i < 4096 / 4 / NT; ++i) h4[tid + i * NT] = make_uint4(0u, 0u, 0u, 0u);
    for (int i = tid; i < KPT * NT / 32 + 1; i += NT) sh.selbits[i] = 0u;
    if (tid == 0) sh.ncand = 0;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NT / 64; ++i) { hi = fmaxf(hi, sh.red[i]); lo = fminf(lo, sh.red[NT / 64 + i]); }
    const float span = hi - lo, scale = 4096.0f / span;
    const bool lin = hi > lo && span < INFINITY && scale < INFINITY;
    // both bin maps, blended with a uniform mask (no per-element branch)
    const uint32_t lm = lin ? 0xffffffffu : 0u;
    auto bin_of = [&](float x) -> uint32_t {
        const uint32_t lb = (uint32_t)fminf((x - lo) * scale, 4095.0f);   // x - lo >= 0 unless NaN
        return ((x == x ? lb : 0u) & lm) | ((score_key(x) >> 20) & ~lm);
    };
    uint32_t bin[KEEP ? KPT : 1];
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
        const uint32_t bi = bin_of(sv[i]);
        if (KEEP) bin[i] = bi;
        // unconditional (no skip branch); masked-off keys go to this lane's
        // trash bin, so they never pile onto one address
        atomicAdd(&sh.hist[valid(i) ? bi : 4096u + (uint32_t)lane], 1u);
    }
    auto bin_at = [&](int i) -> uint32_t { return KEEP ? bin[KEEP ? i : 0] : bin_of(sv[i]); };
    __syncthreads();
    if (wid == 0) hist_cut(sh, topk);               // the threshold bin
    __syncthreads();
    const uint32_t B = (uint32_t)sh.bin;
    const int need = sh.need;
    const int cB = sh.cnt_b;
    if (cB > kCandMax) return false;
    if (cB > need) {
        // rank the threshold bin's keys exactly: (key desc, index asc)
        int nc = 0;
#pragma unroll
        for (int i = 0; i < KPT; ++i) nc += (valid(i) && bin_at(i) == B);
        if (nc > 0) {
            int slot = atomicAdd(&sh.ncand, nc);
#pragma unroll
            for (int i = 0; i < KPT; ++i) {
                const bool c = valid(i) && bin_at(i) == B;
                const int at = c ? slot : kCandMax;
                sh.cand_key[at] = score_key(sv[i]);
                sh.cand_b[at] = b0 + i;
                slot += c;
            }
        }
        __syncthreads();
        if (tid < cB) {
            const uint32_t k = sh.cand_key[tid];
            const int b = sh.cand_b[tid];
            int rank = 0;
            for (int jj = 0; jj < cB; ++jj) {
                const uint32_t kj = sh.cand_key[jj];
                rank += (kj > k) || (kj == k && sh.cand_b[jj] < b);
            }
            if (rank < need) atomicOr(&sh.selbits[(b - base) >> 5], 1u << ((b - base) & 31));
        }
        __syncthreads();
    }
    // the thread's KPT bits start at bit tid*KPT: two words cover them
    uint64_t wb = ~0ull;
    if (cB > need) {
        const int e = tid * KPT;
        const uint64_t w2 = (uint64_t)sh.selbits[e >> 5] | ((uint64_t)sh.selbits[(e >> 5) + 1] << 32);
        wb = w2 >> (e & 31);
    }
    MT m = 0;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
        const uint32_t bi = bin_at(i);
        const bool take = valid(i) && (bi > B || (bi == B && ((wb >> i) & 1u)));
        m |= (MT)take << i;
    }
    MT *tm = reinterpret_cast<MT *>(sh.tmask);
    tm[tid] = m;
    __syncthreads();
    // ordered emission by wave 0: lane l owns threads TPL*l .. TPL*l + TPL-1
    if (wid == 0) {
        constexpr int TPL = NT / 64;
        int cnt = 0;
#pragma unroll
        for (int q = 0; q < TPL; ++q) cnt += (int)__builtin_popcountll((uint64_t)tm[TPL * lane + q]);
        int pos = wave_incl_scan(cnt) - cnt;
#pragma unroll
        for (int q = 0; q < TPL; ++q) {
            uint64_t x = (uint64_t)tm[TPL * lane + q];
            const int tb = base + (TPL * lane + q) * KPT;
            while (x) {
                if (pos < topk) out.put(g.sink + pos, tb + __builtin_ctzll(x));
                ++pos;
                x &= x - 1u;
            }
        }
    }
    return true;
}

// Streaming path (the 1024-thread k_select_big): thread t owns blocks base +
// [t*per, t*per + per) (per <= 64, a multiple of 4) and reads them three
// times, each in one round trip, keeping none in registers between the
// passes: min / max, the 4096-bin histogram (as in the register path), then
// the take bits together with the threshold bin's candidates, which are
// ranked in LDS; each owner then reads back its candidates' verdicts and
// writes its taken blocks at its exclusive-scan offset.  Vectors past `per`
// are skipped by a branch that is uniform over the workgroup.
template <int NT, typename SH>
__device__ __forceinline__ bool select_stream(const Geo &g, const float *sc, const Ranges &r, int topk,
                                              const SelOut &out, SH &sh) {
    constexpr int MAXV = 16;                       // 16-byte vectors a thread: 64 keys
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int base = r.e_lo & ~3;
    const int per = (((r.e_hi - base) + NT - 1) / NT + 3) & ~3;
    const int nv = per / 4;                        // uniform
    const int b0 = base + tid * per;
    const int i_lo = r.e_lo - b0, i_hi = r.e_hi - b0;   // this thread's valid slots: [i_lo, i_hi)
    const BufRsrc rs = buf_rsrc(sc, (uint32_t)((r.e_hi + 3) & ~3) * 4u);
#define QWFN_STREAM_LOAD(x)                                                                   \
    float x[4 * MAXV];                                                                        \
    _Pragma("unroll") for (int k = 0; k < MAXV; ++k) {                                        \
        if (k < nv) {                                                                         \
            const auto v_ = BufLoad<4, kCpolSc1>::at(rs, (b0 + 4 * k) * 4, 0);                \
            x[4 * k] = v_[0]; x[4 * k + 1] = v_[1]; x[4 * k + 2] = v_[2]; x[4 * k + 3] = v_[3]; \
        } else {                                                                              \
            x[4 * k] = x[4 * k + 1] = x[4 * k + 2] = x[4 * k + 3] = 0.0f;                     \
        }                                                                                     \
    }
    auto valid = [&](int i) { return i >= i_lo && i < i_hi; };
    float lo = INFINITY, hi = -INFINITY;
    {
        QWFN_STREAM_LOAD(x)
#pragma unroll
        for (int k = 0; k < MAXV; ++k) {
            if (k < nv) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int i = 4 * k + j;
                    const bool use = valid(i) && x[i] == x[i];
                    lo = fminf(lo, use ? x[i] : INFINITY);
                    hi = fmaxf(hi, use ? x[i] : -INFINITY);
                }
            }
        }
    }
    hi = wave_max(hi);
    lo = -wave_max(-lo);
    if (lane == 0) { sh.red[wid] = hi; sh.red[NT / 64 + wid] = lo; }
    uint4 *h4 = reinterpret_cast<uint4 *>(sh.hist);
    for (int i = tid; i < 4096 / 4; i += NT) h4[i] = make_uint4(0u, 0u, 0u, 0u);
    if (tid == 0) sh.ncand = 0;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NT / 64; ++i) { hi = fmaxf(hi, sh.red[i]); lo = fminf(lo, sh.red[NT / 64 + i]); }
    const float span = hi - lo, scale = 4096.0f / span;
    const bool lin = hi > lo && span < INFINITY && scale < INFINITY;
    const uint32_t lm = lin ? 0xffffffffu : 0u;
    auto bin_of = [&](float v) -> uint32_t {
        const uint32_t lb = (uint32_t)fminf((v - lo) * scale, 4095.0f);
        return ((v == v ? lb : 0u) & lm) | ((score_key(v) >> 20) & ~lm);
    };
    {
        QWFN_STREAM_LOAD(y)
#pragma unroll
        for (int k = 0; k < MAXV; ++k) {
            if (k < nv) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int i = 4 * k + j;
                    atomicAdd(&sh.hist[valid(i) ? bin_of(y[i]) : 4096u + (uint32_t)lane], 1u);
                }
            }
        }
    }
    __syncthreads();
    if (wid == 0) hist_cut(sh, topk);               // the threshold bin
    __syncthreads();
    const uint32_t B = (uint32_t)sh.bin;
    const int need = sh.need;
    const int cB = sh.cnt_b;
    if (cB > kCandMax) return false;
    const bool rank = cB > need;                   // else every key of bin B is taken
    uint64_t m = 0, cm = 0;                        // taken keys; the threshold bin's keys (to rank)
    int slot0 = 0;
    {
        QWFN_STREAM_LOAD(z)
#pragma unroll
        for (int k = 0; k < MAXV; ++k) {
            if (k < nv) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int i = 4 * k + j;
                    const uint32_t bi = bin_of(z[i]);
                    const bool v = valid(i);
                    m |= (uint64_t)(v && (bi > B || (!rank && bi == B))) << i;
                    cm |= (uint64_t)(rank && v && bi == B) << i;
                }
            }
        }
        if (cm) {
            slot0 = atomicAdd(&sh.ncand, (int)__builtin_popcountll(cm));
            int slot = slot0;
            for (uint64_t c2 = cm; c2; c2 &= c2 - 1ull) {
                const int i = __builtin_ctzll(c2);
                float zi = z[0];
#pragma unroll
                for (int k = 1; k < 4 * MAXV; ++k) zi = k == i ? z[k] : zi;
                sh.cand_key[slot] = score_key(zi);
                sh.cand_b[slot] = b0 + i;
                ++slot;
            }
        }
    }
#undef QWFN_STREAM_LOAD
    if (rank) {
        __syncthreads();
        if (tid < cB) {                            // rank: (key desc, index asc)
            const uint32_t k = sh.cand_key[tid];
            const int b = sh.cand_b[tid];
            int rk = 0;
            for (int jj = 0; jj < cB; ++jj) {
                const uint32_t kj = sh.cand_key[jj];
                rk += (kj > k) || (kj == k && sh.cand_b[jj] < b);
            }
            sh.cand_ok[tid] = rk < need;
        }
        __syncthreads();
        int slot = slot0;
        for (uint64_t c2 = cm; c2; c2 &= c2 - 1ull, ++slot)
            if (sh.cand_ok[slot]) m |= 1ull << __builtin_ctzll(c2);
    }
    const int cnt = (int)__builtin_popcountll(m);
    int tot;
    int pos = block_excl_sum<NT>(cnt, sh.tmp, &tot);
    while (m) {
        if (pos < topk) out.put(g.sink + pos, b0 + __builtin_ctzll(m));
        ++pos;
        m &= m - 1ull;
    }
    return true;
}

// Sampled cut (long contexts, the 1024-thread selections): a cut placed from
// kSelSample evenly spaced scores (block e_lo + j * eligible / kSelSample),
// low enough that the topk largest lie above it with a wide margin -- the
// sample's rs-th largest, rs = mu + 4 sqrt(mu) + 8 for mu = topk * kSelSample
// / eligible, the sample keys expected above the topk-th key -- leaves about
// rs / mu times topk candidates, on which the exact selection runs alone.
// The cut is a bin of a map that never decreases in the key order, so the
// candidates are every key at or above some key: when they number at least
// topk they hold the exact top topk, ties included.
constexpr int kSelSample = 4096;
constexpr int kSelCandMax = 4096;

// rs, or 0 when the sampled cut does not apply (few eligible blocks, or a
// topk that is a large share of them), for NS evenly spaced samples.
template <int NS = kSelSample>
__device__ __forceinline__ int sample_rank(const Ranges &r, int topk) {
    const int ne = r.e_hi - r.e_lo;
    if (ne < 2 * NS || topk <= 0) return 0;
    const float mu = (float)topk * (float)NS / (float)ne;
    const int rs = (int)ceilf(mu + 4.0f * sqrtf(mu) + 8.0f);
    return rs <= NS / 8 ? rs : 0;
}



// The bin map of the sample -- linear in the score over the sample's range
// (below it bin 0, above it bin 4095), NaN in bin 0; without a finite spread
// the top 12 key bits -- and the cut bin.
struct CutMap {
    float lo, scale;
    uint32_t lm, cut;
    __device__ __forceinline__ uint32_t bin(float x) const {
        const uint32_t lb = (uint32_t)fminf(fmaxf((x - lo) * scale, 0.0f), 4095.0f);
        return ((x == x ? lb : 0u) & lm) | ((score_key(x) >> 20) & ~lm);
    }
    __device__ __forceinline__ bool keep(float x) const { return bin(x) >= cut; }
};

// The smallest key among the samples sv the cut keeps, over the workgroup
// (one barrier; red: NT / 64 words).  Every key at or above it is a candidate
// of the cut: an upper set in the key order, so the candidates hold the exact
// top-k whenever they number at least topk.
template <int NT, int SPT>
__device__ __forceinline__ uint32_t cut_key(const CutMap &cut, const float (&sv)[SPT], uint32_t *red) {
    const int tid = threadIdx.x, lane = tid & 63;
    uint32_t tk = 0xffffffffu;
#pragma unroll
    for (int k = 0; k < SPT; ++k) tk = cut.keep(sv[k]) ? min(tk, score_key(sv[k])) : tk;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) tk = min(tk, (uint32_t)__shfl_xor((int)tk, o));
    if (lane == 0) red[tid >> 6] = tk;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NT / 64; ++i) tk = min(tk, red[i]);
    return tk;
}

// The sample's scores a thread loads: samples tid + k * NT, k < NS / NT, of
// the NS evenly spaced blocks e_lo + j * eligible / NS.
template <int NT, int CP = kCpolSc1, int NS = kSelSample>
__device__ __forceinline__ void sample_load(const BufRsrc &rsc, const Ranges &r, float (&sv)[NS / NT]) {
    constexpr int SPT = NS / NT;
    static_assert(SPT * NT == NS, "whole samples a thread");
    const int tid = threadIdx.x;
    const int ne = r.e_hi - r.e_lo;
#pragma unroll
    for (int k = 0; k < SPT; ++k) {
        const int j = tid + k * NT;
        sv[k] = BufLoad<1, CP>::at(rsc, (r.e_lo + (int)((int64_t)j * ne / NS)) * 4, 0)[0];
    }
}

// The cut of the sampled scores sv (sample_load's), by all NT threads; leaves
// sh.hist for reuse after a barrier.
template <int NT, int SPT, typename SH>
__device__ __forceinline__ CutMap sample_cut_of(const float (&sv)[SPT], int rs, SH &sh) {
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    float lo = INFINITY, hi = -INFINITY;
#pragma unroll
    for (int k = 0; k < SPT; ++k) {
        const bool use = sv[k] == sv[k];
        lo = fminf(lo, use ? sv[k] : INFINITY);
        hi = fmaxf(hi, use ? sv[k] : -INFINITY);
    }
    hi = wave_max(hi);
    lo = -wave_max(-lo);
    if (lane == 0) { sh.red[wid] = hi; sh.red[NT / 64 + wid] = lo; }
    uint4 *h4 = reinterpret_cast<uint4 *>(sh.hist);
    for (int i = tid; i < 4096 / 4; i += NT) h4[i] = make_uint4(0u, 0u, 0u, 0u);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NT / 64; ++i) { hi = fmaxf(hi, sh.red[i]); lo = fminf(lo, sh.red[NT / 64 + i]); }
    CutMap m;
    const float span = hi - lo;
    m.lo = lo;
    m.scale = 4096.0f / span;
    m.lm = hi > lo && span < INFINITY && m.scale < INFINITY ? 0xffffffffu : 0u;
    m.cut = 0;
#pragma unroll
    for (int k = 0; k < SPT; ++k) atomicAdd(&sh.hist[m.bin(sv[k])], 1u);
    __syncthreads();
    if (wid == 0) hist_cut(sh, rs);
    __syncthreads();
    m.cut = (uint32_t)sh.bin;
    return m;
}

// The sample's cut, by all NT threads (kSelSample / NT device-coherent loads
// each); leaves sh.hist for reuse after a barrier.
template <int NT, typename SH>
__device__ __forceinline__ CutMap sample_cut(const BufRsrc &rsc, const Ranges &r, int rs, SH &sh) {
    float sv[kSelSample / NT];
    sample_load<NT>(rsc, r, sv);
    return sample_cut_of<NT>(sv, rs, sh);
}

// The exact selection among C candidates in LDS (sh.ckey / sh.cblk[0, C), in
// block order, topk <= C <= kSelCandMax): a 4096-bin histogram linear in the
// key between the candidates' smallest and largest key, the threshold bin
// ranked by (key desc, index asc) -- the candidate index stands in for the
// block index --, emission in candidate (block) order after the sink blocks.
// Returns false, with nothing written, when that bin holds more than
// kCandMax keys.
template <int NT, typename SH>
__device__ __forceinline__ bool select_cands(const Geo &g, int C, int topk, const SelOut &out, SH &sh) {
    constexpr int CPT = kSelCandMax / NT;
    static_assert(CPT * NT == kSelCandMax, "whole candidates a thread");
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    uint4 *h4 = reinterpret_cast<uint4 *>(sh.hist);
    for (int i = tid; i < 4096 / 4; i += NT) h4[i] = make_uint4(0u, 0u, 0u, 0u);
    if (tid == 0) sh.ncand = 0;
    __syncthreads();
    // thread t owns candidates [CPT t, CPT t + CPT)
    uint32_t kc[CPT];
    uint32_t kmin = 0xffffffffu, kmax = 0u;
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
        const int c = CPT * tid + u;
        kc[u] = c < C ? sh.ckey[c] : 0u;
        kmin = c < C ? min(kmin, kc[u]) : kmin;
        kmax = c < C ? max(kmax, kc[u]) : kmax;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        kmin = min(kmin, (uint32_t)__shfl_xor((int)kmin, o));
        kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, o));
    }
    if (lane == 0) { sh.kred[wid] = kmin; sh.kred[NT / 64 + wid] = kmax; }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NT / 64; ++i) { kmin = min(kmin, sh.kred[i]); kmax = max(kmax, sh.kred[NT / 64 + i]); }
    const float sc2 = 4096.0f / ((float)(kmax - kmin) + 1.0f);
    auto bin2 = [&](uint32_t k) -> uint32_t { return (uint32_t)fminf((float)(k - kmin) * sc2, 4095.0f); };
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
        const int c = CPT * tid + u;
        atomicAdd(&sh.hist[c < C ? bin2(kc[u]) : 4096u + (uint32_t)lane], 1u);
    }
    __syncthreads();
    if (wid == 0) hist_cut(sh, topk);
    __syncthreads();
    const uint32_t B = (uint32_t)sh.bin;
    const int need = sh.need, cB = sh.cnt_b;
    if (cB > need) {                               // rank the threshold bin: (key desc, index asc)
        if (cB > kCandMax) return false;           // (uniform)
#pragma unroll
        for (int u = 0; u < CPT; ++u) {
            const int c = CPT * tid + u;
            if (c < C && bin2(kc[u]) == B) {
                const int at = atomicAdd(&sh.ncand, 1);
                sh.cand_key[at] = kc[u];
                sh.cand_b[at] = c;
            }
        }
        __syncthreads();
        if (tid < cB) {
            const uint32_t k = sh.cand_key[tid];
            const int c = sh.cand_b[tid];
            int rk = 0;
            for (int jj = 0; jj < cB; ++jj) {
                const uint32_t kj = sh.cand_key[jj];
                rk += (kj > k) || (kj == k && sh.cand_b[jj] < c);
            }
            sh.cok[c] = rk < need;
        }
        __syncthreads();
    }
    bool tk[CPT];
    int cnt = 0;
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
        const int c = CPT * tid + u;
        const uint32_t bi = bin2(kc[u]);
        tk[u] = c < C && (bi > B || (bi == B && (cB <= need || sh.cok[c])));
        cnt += tk[u];
    }
    int tot;
    int pos = block_excl_sum<NT>(cnt, sh.tmp, &tot);
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
        if (tk[u]) {
            if (pos < topk) out.put(g.sink + pos, sh.cblk[CPT * tid + u]);
            ++pos;
        }
    }
    return true;
}

// One workgroup: the sampled cut, then one pass over the scores (thread t owns
// blocks base + [t*per, t*per + per), per <= 64) compacting the candidates
// into LDS in block order, then the exact selection.  Fewer than topk
// candidates, more than kSelCandMax, or an overfull threshold bin: returns
// false with nothing written, and the streaming path runs.
template <int NT, typename SH>
__device__ __forceinline__ bool select_sample(const Geo &g, const float *sc, const Ranges &r, int topk,
                                              const SelOut &out, SH &sh) {
    constexpr int MAXV = 16;
    const int tid = threadIdx.x;
    const int rs = sample_rank(r, topk);
    if (rs == 0) return false;                     // (uniform)
    const BufRsrc rsc = buf_rsrc(sc, (uint32_t)((r.e_hi + 3) & ~3) * 4u);
    const CutMap cut = sample_cut<NT>(rsc, r, rs, sh);
    const int base = r.e_lo & ~3;
    const int per = (((r.e_hi - base) + NT - 1) / NT + 3) & ~3;
    const int nv = per / 4;                        // uniform
    const int b0 = base + tid * per;
    const int i_lo = r.e_lo - b0, i_hi = r.e_hi - b0;
    float z[4 * MAXV];
#pragma unroll
    for (int k = 0; k < MAXV; ++k) {
        if (k < nv) {
            const auto v_ = BufLoad<4, kCpolSc1>::at(rsc, (b0 + 4 * k) * 4, 0);
            z[4 * k] = v_[0]; z[4 * k + 1] = v_[1]; z[4 * k + 2] = v_[2]; z[4 * k + 3] = v_[3];
        } else {
            z[4 * k] = z[4 * k + 1] = z[4 * k + 2] = z[4 * k + 3] = 0.0f;
        }
    }
    uint64_t cm = 0;
#pragma unroll
    for (int k = 0; k < MAXV; ++k) {
        if (k < nv) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int i = 4 * k + j;
                cm |= (uint64_t)(i >= i_lo && i < i_hi && cut.keep(z[i])) << i;
            }
        }
    }
    int C;
    int slot = block_excl_sum<NT>((int)__builtin_popcountll(cm), sh.tmp, &C);
    if (C < topk || C > kSelCandMax) return false;   // (uniform)
#pragma unroll
    for (int k = 0; k < MAXV; ++k) {
        if (k < nv) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int i = 4 * k + j;
                if ((cm >> i) & 1ull) {
                    sh.ckey[slot] = score_key(z[i]);
                    sh.cblk[slot] = b0 + i;
                    ++slot;
                }
            }
        }
    }
    __syncthreads();
    return select_cands<NT>(g, C, topk, out, sh);
}

template <int NT, typename SH>
__device__ __forceinline__ void select_radix(const Geo &g, const float *sc, const Ranges &r, int topk,
                                             const SelOut &out, SH &sh) {
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");   // plain loads of the scores below
    const int tid = threadIdx.x;
    const int ne = r.e_hi - r.e_lo;
    const int per = (ne + NT - 1) / NT;
    const int b0 = r.e_lo + tid * per;
    const int b1 = min(b0 + per, r.e_hi);
    __syncthreads();                               // the register path may still read sh.hist
    uint32_t prefix = 0;
    int need = topk;
    radix_pass<NT, 12>(sh, sc, r.e_lo, r.e_hi, 20, prefix, need, true);
    radix_pass<NT, 12>(sh, sc, r.e_lo, r.e_hi, 8, prefix, need, false);
    radix_pass<NT, 8>(sh, sc, r.e_lo, r.e_hi, 0, prefix, need, false);
    const uint32_t T = prefix;
    int tot, eq = 0;
    for (int b = b0; b < b1; ++b) eq += (score_key(sc[b]) == T);
    int eqi = block_excl_sum<NT>(eq, sh.tmp, &tot);
    int cnt = 0;
    {
        int e2 = eqi;
        for (int b = b0; b < b1; ++b) {
            const uint32_t k = score_key(sc[b]);
            bool tk = k > T;
            if (k == T) tk = (e2++ < need);
            cnt += tk;
        }
    }
    int pos = g.sink + block_excl_sum<NT>(cnt, sh.tmp, &tot);
    for (int b = b0; b < b1; ++b) {
        const uint32_t k = score_key(sc[b]);
        bool tk = k > T;
        if (k == T) tk = (eqi++ < need);
        if (tk && pos < g.sink + topk) out.put(pos++, b);
    }
}

// Eligible blocks the register path of an NT-thread selection holds (256
// threads: 32 keys a thread; 512, the attention's in-kernel selection: 16),
// or, at 1024 threads, the streaming path.
template <int NT> constexpr int keys_max() { return NT == kIdxThreads ? kKeysMax : NT == 512 ? 16 * NT : 64 * NT; }

// The forced blocks around a selection of topk eligible blocks: the sink
// blocks first, the window blocks after the topk, and the count.
template <int NT>
__device__ __forceinline__ void emit_forced(const Geo &g, const Ranges &r, int topk, const SelOut &out) {
    const int tid = threadIdx.x;
    for (int i = tid; i < g.sink; i += NT) out.put(i, i);
    const int nwin = r.b_last - r.fw + 1;
    for (int i = tid; i < nwin; i += NT) out.put(g.sink + topk + i, r.fw + i);
    if (tid == 0) out.count(g.sink + topk + nwin);
}

// MAXSPAN: the most eligible blocks a caller passes (smaller register paths
// only; a longer span takes the radix fallback).
template <int NT, typename SH, int MAXSPAN = keys_max<NT>()>
__device__ __forceinline__ void select_blocks(const Geo &g, const float *sc, int L, const SelOut &out, SH &sh) {
    const int tid = threadIdx.x;
    const Ranges r = qsa_ranges(g, L);
    const int ne = r.e_hi - r.e_lo;
    const int topk = eff_topk(g, r);
    if (g.topk <= 0 || ne <= topk) {
        const int n = r.b_last + 1;
        for (int i = tid; i < n; i += NT) out.put(i, i);
        if (tid == 0) out.count(n);
        return;
    }
    if (topk > 0) {                               // (none scored when the forced blocks fill the count)
        bool done = false;
        const int span = r.e_hi - (r.e_lo & ~3);  // blocks the register path covers
        if constexpr (NT == kIdxThreads) {
            if (span <= 4 * NT) done = select_regs<NT, 4, true>(g, sc, r, topk, out, sh);
            else if (span <= 8 * NT) done = select_regs<NT, 8, true>(g, sc, r, topk, out, sh);
            else if (span <= 12 * NT) done = select_regs<NT, 12, true>(g, sc, r, topk, out, sh);
            else if (span <= 16 * NT) done = select_regs<NT, 16, true>(g, sc, r, topk, out, sh);
            else if constexpr (MAXSPAN > 16 * NT) {
                if (span <= 24 * NT) done = select_regs<NT, 24, true>(g, sc, r, topk, out, sh);
                else if (span <= keys_max<NT>()) done = select_regs<NT, keys_max<NT>() / NT, true>(g, sc, r, topk, out, sh);
            }
        } else if constexpr (NT == 512) {
            if (span <= 4 * NT) done = select_regs<NT, 4, true>(g, sc, r, topk, out, sh);
            else if (span <= 8 * NT) done = select_regs<NT, 8, true>(g, sc, r, topk, out, sh);
            else if (span <= 12 * NT) done = select_regs<NT, 12, true>(g, sc, r, topk, out, sh);
            else if (span <= keys_max<NT>()) done = select_regs<NT, 16, true>(g, sc, r, topk, out, sh);
        } else {
            if (span <= keys_max<NT>()) {
                done = select_sample<NT>(g, sc, r, topk, out, sh);
                if (!done) {
                    __syncthreads();               // the sampled path's LDS reads are done
                    done = select_stream<NT>(g, sc, r, topk, out, sh);
                }
            }
        }
        if (!done) select_radix<NT>(g, sc, r, topk, out, sh);
    }
    emit_forced<NT>(g, r, topk, out);
}

// Shared selection (shared_selection = 1): one selection for every KV head of
// a sequence, on the sum of the heads' block scores taken in head order
// (score = sum over all query heads of their -- relu'd when set -- dots, each
// KV head's group summed first).  Called by the one workgroup that saw every
// head's scores: it sums the rows into row 0 (device-coherent loads of the
// other workgroups' stores) and selects on it into every one of the
// g.sel_rows selection rows.
template <int NT, typename SH>
__device__ __forceinline__ void select_shared(const Geo &g, float *sc0, int64_t sc_stride, int L, const SelOut &out,
                                              SH &sh) {
    const int tid = threadIdx.x;
    const Ranges r = qsa_ranges(g, L);
    if (g.Hkv > 1) {                               // one score row needs no sum
        const BufRsrc rs = buf_rsrc(sc0, (uint32_t)(((int64_t)(g.Hkv - 1) * sc_stride + r.e_hi) * 4));
        // eight blocks a thread per round, every load of a round issued before
        // any is summed (a rolled loop would wait out one round trip per block)
        constexpr int U = 8;
        for (int b0 = r.e_lo + tid; b0 < r.e_hi; b0 += U * NT) {
            float acc[U];
#pragma unroll
            for (int u = 0; u < U; ++u) acc[u] = BufLoad<1, kCpolSc1>::at(rs, (b0 + u * NT) * 4, 0)[0];
            for (int h = 1; h < g.Hkv; ++h) {
                float x[U];
#pragma unroll
                for (int u = 0; u < U; ++u)
                    x[u] = BufLoad<1, kCpolSc1>::at(rs, (int)((h * sc_stride + b0 + u * NT) * 4), 0)[0];
#pragma unroll
                for (int u = 0; u < U; ++u) acc[u] += x[u];
            }
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (b0 + u * NT < r.e_hi) sc0[b0 + u * NT] = acc[u];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");   // the summed row, for the selection's loads
        __syncthreads();
    }
    select_blocks<NT>(g, sc0, L, out, sh);
}

}  // namespace qwfn_qsa
