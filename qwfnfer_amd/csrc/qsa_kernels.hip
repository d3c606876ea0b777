// qsa_kernels.hip -- gfx950 (CDNA4) kernels of the q8_0 KV cache and the QSA
// decode path.  Wave64 throughout; every cross-lane reduction is a
// __shfl_xor / __shfl_up ladder inside one wave, every cross-wave step goes
// through LDS.  Kernels that must be bit-exact against the CPU oracle (append,
// pool, indexer scores and selection) are compiled with fp contraction off and
// spell every fused multiply-add as fmaf.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include <type_traits>

#include "qsa_append.h"
#include "qsa_device.h"
#include "qsa_select.h"
#include "qsa_idx_pool.h"

namespace qwfn_qsa {

// ---------------------------------------------------------------------------
// fill
// ---------------------------------------------------------------------------

__global__ void k_fill_zero(uint32_t *p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

hipError_t launch_fill_zero(void *p, size_t bytes, hipStream_t st) {
    const size_t n = bytes / 4;
    if (n == 0) return hipSuccess;
    const unsigned blocks = (unsigned)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
    hipLaunchKernelGGL(k_fill_zero, dim3(blocks), dim3(256), 0, st, (uint32_t *)p, n);
    return hipGetLastError();
}

__global__ void k_chain_lens(const int32_t *__restrict__ seq_len, int32_t n_seq, int32_t n_pos,
                             int32_t *__restrict__ lens) {
    for (int i = (int)threadIdx.x; i < n_seq * n_pos; i += (int)blockDim.x) lens[i] = seq_len[i % n_seq] + i / n_seq;
}

hipError_t launch_chain_lens(const int32_t *seq_len, int32_t n_seq, int32_t n_pos, int32_t *lens, hipStream_t st) {
    hipLaunchKernelGGL(k_chain_lens, dim3(1), dim3(256), 0, st, seq_len, n_seq, n_pos, lens);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// append: quantize rows to q8_0 and overwrite them in the paged cache
// (the quantizers are in qsa_append.h)
// ---------------------------------------------------------------------------

// Lane i: 4 values of one 32-value block; blocks enumerate (row, K|V, head,
// j).  len (when set): row r is sequence r's token at position len[r] - 1.
__global__ void __launch_bounds__(256)
k_append(Geo g, qwfn_kv_view v, const void *ksrc, const void *vsrc, int32_t f16,
         const int32_t *seq_ids, const int32_t *pos, int32_t n_rows, int32_t seq_const, int32_t pos0,
         const int32_t *len) {
    const int64_t total = (int64_t)n_rows * 2 * g.Hkv * (g.hd / 32) * 8;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    append_lane(g, v, ksrc, vsrc, f16, i, [&](int r, int &seq, int &t) {
        seq = len ? r : seq_ids ? seq_ids[r] : seq_const;
        t = len ? len[r] - 1 : pos ? pos[r] : pos0 + r;
    });
}

hipError_t launch_append(const Geo &g, const qwfn_kv_view &v, const void *k, const void *vv,
                         int32_t src_f16, const int32_t *seq_ids, const int32_t *pos,
                         int32_t n_rows, int32_t seq_const, int32_t pos0, hipStream_t st,
                         const int32_t *len) {
    const int64_t total = (int64_t)n_rows * 2 * g.Hkv * (g.hd / 32) * 8;
    const int64_t blocks = (total + 255) / 256;
    hipLaunchKernelGGL(k_append, dim3((unsigned)blocks), dim3(256), 0, st, g, v, k, vv, src_f16,
                       seq_ids, pos, n_rows, seq_const, pos0, len);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// pooled keys: sequential fp32 add chain over the block's members, * 1/bt
// (pool_block_dev in qsa_append.h)
// ---------------------------------------------------------------------------

// grid (n_blocks, Hkv), 256 threads.  len (decode): entry bi is sequence bi's
// block holding position len[bi] - 1, pooled only when that token completes it.
template <int HD, int KT>
__global__ void __launch_bounds__(256)
k_pool(Geo g, qwfn_kv_view v, const int32_t *seq_ids, const int32_t *block_ids, int32_t seq_const,
       int32_t blk0, const int32_t *len) {
    __shared__ int8_t q8[kStageRows * HD];
    __shared__ uint16_t sc[kStageRows * (HD / 32)];
    const int bi = blockIdx.x, gh = blockIdx.y, tid = threadIdx.x;
    if (len && (len[bi] < 1 || len[bi] % g.bt)) return;   // no block completed (a bad length is the append's report)
    const int seq = len ? bi : seq_ids ? seq_ids[bi] : seq_const;
    const int b = len ? (len[bi] - 1) / g.bt : block_ids ? block_ids[bi] : blk0 + bi;
    const bool report = (gh == 0 && tid == 0);
    if (seq < 0 || seq >= g.n_seq_view) { if (report) set_status(v.status, QWFN_STATUS_SEQ_RANGE); return; }
    if (b < 0 || b >= g.bps) { if (report) set_status(v.status, QWFN_STATUS_BLOCK_RANGE); return; }
    const int t0 = b * g.bt;
    const int32_t pp = phys_page(g, v.page_table, seq, t0);   // a block never straddles pages
    if (pp < 0) { if (report) set_status(v.status, QWFN_STATUS_PAGE_RANGE); return; }
    const uint8_t *page = (const uint8_t *)v.k_pages + (int64_t)pp * g.page_bytes;
    pool_block_dev<HD, KT>(g, page, gh, t0 % g.pt, v.pooled + (((int64_t)seq * g.Hkv + gh) * g.bps + b) * HD,
                           nullptr, q8, sc, tid, 256);
}


// The selection of long contexts (more eligible blocks than the indexer
// workgroup's registers hold) as its own launch after a scoring-only
// indexer: one 1024-thread workgroup per (sequence or prefill query, KV head)
// -- per sequence with a shared selection -- holding up to 64 keys a thread.
constexpr int kBigSelThreads = 1024;
struct BigSelShared {
    uint32_t hist[4096 + 64];
    uint32_t cand_key[kCandMax + 1];
    int32_t cand_b[kCandMax + 1];
    int32_t cand_ok[kCandMax + 1];                // the ranking's verdicts
    uint32_t ckey[kSelCandMax];                   // sampled-cut candidates, in block order
    int32_t cblk[kSelCandMax];
    uint8_t cok[kSelCandMax];                     // their threshold-bin verdicts
    uint32_t kred[2 * (kBigSelThreads / 64)];
    int wpre[kCutWgMax];                          // multi-workgroup selection: region offsets
    int ctot, flag;
    float red[2 * (kBigSelThreads / 64)];
    int tmp[kBigSelThreads / 64];
    int bin, need, ncand, cnt_b;
};

// LDS of the general attention's in-kernel selection (k_attn with SEL):
// the register path's state at NT threads, and the selection itself.
constexpr int kAttnSelMax = 1024;                 // selected blocks it holds
template <int NT>
struct AttnSelShared {
    uint32_t hist[4096 + 64];
    uint32_t cand_key[kCandMax + 1];
    int32_t cand_b[kCandMax + 1];
    uint32_t tmask[NT];
    uint32_t selbits[keys_max<NT>() / 32 + 1];
    float red[2 * (NT / 64)];
    int tmp[NT / 64];
    int bin, need, ncand, cnt_b;
    int32_t sel[kAttnSelMax];
    int32_t nsel;
};

// The attention's own selection (SEL): every workgroup runs the decode
// selection of its (sequence, KV head) on the indexer's score row into LDS,
// with all of its threads, and takes its tiles' blocks from there; part 0 also
// writes the selection and its count out (for the caller and the merge).  The
// indexer launch before it only scores, so the decode step waits for no
// completion counter and no single selecting workgroup.
struct NoShared {};
template <int NT, typename SH>
__device__ __forceinline__ void attn_select(const Geo &g, const Ws &ws, int L, int max_seq_len, int max_sel,
                                            int pair, int part, int32_t *gsel, int32_t *gnsel, SH &ssh) {
    const int tid = threadIdx.x;
    if (L >= 1 && L <= max_seq_len) {
        const SelOut lo{ssh.sel, &ssh.nsel, 0, 1};
        select_blocks<NT>(g, ws.scores + (int64_t)pair * ws.nb_cap, L, lo, ssh);
    } else if (tid == 0) {
        ssh.nsel = 0;
    }
    __syncthreads();
    if (part == 0) {
        const int n = min(ssh.nsel, max_sel);
        for (int i = tid; i < n; i += NT) gsel[(int64_t)pair * max_sel + i] = ssh.sel[i];
        if (tid == 0) gnsel[pair] = n;
    }
}

// grid (shared ? 1 : Hkv, n_seq or n_q)
__global__ void __launch_bounds__(kBigSelThreads)
k_select_big(Geo g, qwfn_kv_view v, const int32_t *seq_len, int32_t max_seq_len, float *scores, int32_t nb_cap,
             int32_t *sel, int32_t *nsel, int32_t max_sel) {
    __shared__ BigSelShared sh;
    const int gh = blockIdx.x, s = blockIdx.y;
    const int L = seq_length(g, g.pf ? 0 : seq_len[s], s);
    const SelOut out = sel_out(g, sel, nsel, max_sel, s, s * g.Hkv + gh);
    if (L < 1 || L > max_seq_len) {
        if (threadIdx.x == 0) {
            out.count(0);
            set_status(v.status, QWFN_STATUS_LEN_RANGE);
        }
        return;
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");   // the scoring launch's stores
    if (g.shared)
        select_shared<kBigSelThreads>(g, scores + (int64_t)s * g.Hkv * nb_cap, nb_cap, L, out, sh);
    else
        select_blocks<kBigSelThreads>(g, scores + ((int64_t)s * g.Hkv + gh) * nb_cap, L, out, sh);
}

// The multi-workgroup selection of long decode contexts: ws.cut_wg
// workgroups a selection, each over kCutKeys scores (thread t: 4 aligned
// blocks).  Every workgroup takes the same sampled cut and compacts the
// candidates among its scores into its own region of ws.cand, in block order,
// with their count; the last to arrive gathers the regions in order into LDS
// and makes the exact selection on them.  A selection the cut does not serve
// (it does not apply, or the candidates number fewer than topk or more than
// kSelCandMax, or their threshold bin overflows) that last workgroup makes
// alone, as k_select_big does.  One score row a selection: per KV head, or
// shared with one scoring head group.
// grid (ws.cut_wg, shared ? 1 : Hkv, n_seq)
static_assert(kCutKeys == 4 * kBigSelThreads, "four scores a thread");
__global__ void __launch_bounds__(kBigSelThreads)
k_select_cut(Geo g, qwfn_kv_view v, const int32_t *seq_len, int32_t max_seq_len, Ws ws, int32_t *sel,
             int32_t *nsel, int32_t max_sel) {
    constexpr int NT = kBigSelThreads, CPT = kSelCandMax / NT;
    __shared__ BigSelShared sh;
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int w = blockIdx.x, nw = gridDim.x, gh = blockIdx.y, s = blockIdx.z;
    const int pair = s * g.Hkv + gh;
    const int L = seq_len[s];
    const bool ok = L >= 1 && L <= max_seq_len;
    const float *sc = ws.scores + (int64_t)pair * ws.nb_cap;
    Ranges r{0, 0, 0, 0};
    int topk = 0, rs = 0;                          // rs > 0: the cut serves this selection
    if (ok) {
        r = qsa_ranges(g, L);
        topk = eff_topk(g, r);
        const int span = r.e_hi - (r.e_lo & ~3);
        if (g.topk > 0 && r.e_hi - r.e_lo > topk && span <= nw * kCutKeys && span <= 64 * NT)
            rs = sample_rank(r, topk);
    }
    const BufRsrc rsc = buf_rsrc(sc, (uint32_t)((r.e_hi + 3) & ~3) * 4u);
    uint2 *cand = ws.cand + (int64_t)pair * nw * kCutKeys;
    int32_t *ccnt = ws.ccnt + (int64_t)pair * kCutWgMax;
    if (rs > 0) {                                  // (uniform over the selection's workgroups)
        const CutMap cut = sample_cut<NT>(rsc, r, rs, sh);
        const int b0 = (r.e_lo & ~3) + w * kCutKeys + 4 * tid;
        const auto z = BufLoad<4, kCpolSc1>::at(rsc, b0 * 4, 0);   // past e_hi: 0, not kept
        uint32_t cm = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) cm |= (uint32_t)(b0 + j >= r.e_lo && b0 + j < r.e_hi && cut.keep(z[j])) << j;
        int cw;
        int slot = block_excl_sum<NT>(__builtin_popcount(cm), sh.tmp, &cw);
        uint2 *reg = cand + (int64_t)w * kCutKeys;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if ((cm >> j) & 1u) reg[slot++] = make_uint2(score_key(z[j]), (uint32_t)(b0 + j));
        if (tid == 0) ccnt[w] = cw;
    }
    // the regions and counts are read with device-coherent loads
    if (!arrive_last<false>(&ws.cnt_idx[pair], nw, &sh.flag)) return;
    if (tid == 0) ws.cnt_idx[pair] = 0;
    const SelOut out = sel_out(g, sel, nsel, max_sel, s, pair);
    if (!ok) {
        if (tid == 0) {
            out.count(0);
            set_status(v.status, QWFN_STATUS_LEN_RANGE);
        }
        return;
    }
    bool done = false;
    if (rs > 0) {
        if (wid == 0) {                            // region offsets: an exclusive scan of the counts
            const BufRsrc rc = buf_rsrc(ccnt, (uint32_t)nw * 4u);
            const int c = lane < nw ? __builtin_bit_cast(int, BufLoad<1, kCpolSc1>::at(rc, lane * 4, 0)[0]) : 0;
            const int incl = wave_incl_scan(c);
            sh.wpre[lane] = incl - c;
            if (lane == 63) sh.ctot = incl;
        }
        __syncthreads();
        const int C = sh.ctot;
        if (C >= topk && C <= kSelCandMax) {       // (uniform)
            const BufRsrc rg = buf_rsrc(cand, (uint32_t)nw * kCutKeys * 8u);
            float2 e[CPT];
#pragma unroll
            for (int u = 0; u < CPT; ++u) {        // candidate c: the last region starting at or before it
                const int c = tid + u * NT;
                int lo = 0, hi = nw - 1;
                while (lo < hi) {
                    const int mid = (lo + hi + 1) >> 1;
                    if (sh.wpre[mid] <= c) lo = mid; else hi = mid - 1;
                }
                const int off = c < C ? (lo * kCutKeys + c - sh.wpre[lo]) * 8 : 0;
                const auto x = BufLoad<2, kCpolSc1>::at(rg, off, 0);
                e[u] = make_float2(x[0], x[1]);
            }
#pragma unroll
            for (int u = 0; u < CPT; ++u) {
                const int c = tid + u * NT;
                if (c < C) {
                    sh.ckey[c] = __builtin_bit_cast(uint32_t, e[u].x);
                    sh.cblk[c] = __builtin_bit_cast(int32_t, e[u].y);
                }
            }
            __syncthreads();
            done = select_cands<NT>(g, C, topk, out, sh);
            if (done) emit_forced<NT>(g, r, topk, out);
        }
    }
    if (!done) {
        __syncthreads();                           // LDS reads of the cut path are done
        select_blocks<NT>(g, sc, L, out, sh);
    }
}

// Part `part` of sequence s's sampled cut inside the indexer launch (mode 3):
// kBlocksPerChunk of the row's kIdxCutSamples evenly spaced eligible blocks
// (the append launch's samples, idx_sample_cut), each scored by four lanes as
// the chunks score, and the ceil(rs / kIdxCutParts)-th largest of their keys
// (0, every key a candidate, when no cut applies) stored + 1 into the part's
// slot (ws.cutk, kCutSlots a sequence) with an agent-scope store.  These
// workgroups wait for nothing.
template <int HD, int G>
__device__ __forceinline__ void idx_cut_part(const Geo &g, const qwfn_kv_view &v, const float *q,
                                             const int32_t *seq_len, int32_t max_seq_len, const Ws &ws, int s,
                                             int gh, int part, IdxShared &sh) {
#pragma clang fp contract(off)
    static_assert(kIdxCutSamples == kIdxCutParts * kBlocksPerChunk, "a part's samples: one a lane group");
    const int tid = threadIdx.x, bl = tid >> 2, j = tid & 3;
    const int L = seq_length(g, seq_len[s], s);
    int rs = 0;
    Ranges r{0, 0, 0, 0};
    if (L >= 1 && L <= max_seq_len && g.topk > 0) {
        r = qsa_ranges(g, L);
        const int topk = eff_topk(g, r);
        if (r.e_hi - r.e_lo > topk) rs = sample_rank<kIdxCutSamples>(r, topk);
    }
    uint32_t tk = 0u;
    if (rs > 0) {                                  // (uniform)
        const int b =
            r.e_lo + (int)((int64_t)(part * kBlocksPerChunk + bl) * (r.e_hi - r.e_lo) / kIdxCutSamples);
        const int64_t prow = (((int64_t)cache_seq(g, s) * g.Hkv + gh) * g.bps + b) * HD;
        float4 p4[HD / 16];
        if (g.pooled_f16) {
            const uint16_t *P = reinterpret_cast<const uint16_t *>(v.pooled) + prow;
#pragma unroll
            for (int i = 0; i < HD / 16; ++i) {
                const uint2 x = *reinterpret_cast<const uint2 *>(P + 16 * i + 4 * j);
                p4[i] = make_float4(h2f((uint16_t)x.x), h2f((uint16_t)(x.x >> 16)), h2f((uint16_t)x.y),
                                    h2f((uint16_t)(x.y >> 16)));
            }
        } else {
            const float *P = v.pooled + prow;
#pragma unroll
            for (int i = 0; i < HD / 16; ++i) p4[i] = *reinterpret_cast<const float4 *>(P + 16 * i + 4 * j);
        }
        const float4 *qg4 = reinterpret_cast<const float4 *>(q + ((int64_t)s * g.H + (int64_t)gh * G) * HD);
        for (int i = tid; i < G * HD / 4; i += kIdxThreads) reinterpret_cast<float4 *>(sh.u.q)[i] = qg4[i];
        __syncthreads();
        float acc[G];
#pragma unroll
        for (int h = 0; h < G; ++h) acc[h] = 0.0f;
#pragma unroll
        for (int i = 0; i < HD / 16; ++i) {
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float4 q4 = *reinterpret_cast<const float4 *>(&sh.u.q[h * HD + 16 * i + 4 * j]);
                acc[h] = fmaf(q4.x, p4[i].x, acc[h]);
                acc[h] = fmaf(q4.y, p4[i].y, acc[h]);
                acc[h] = fmaf(q4.z, p4[i].z, acc[h]);
                acc[h] = fmaf(q4.w, p4[i].w, acc[h]);
            }
        }
        float score = 0.0f;
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float t01 = acc[h] + __shfl_xor(acc[h], 1);
            float dot = t01 + __shfl_xor(t01, 2);
            if (g.relu) dot = dot > 0.0f ? dot : 0.0f;
            score = (h == 0) ? dot : score + dot;
        }
        if (j == 0) sh.cand_key[bl] = score_key(score);
        __syncthreads();
        if (tid < 64) {                            // wave 0: a sample key a lane
            const uint32_t k1 = sh.cand_key[tid];
            const int need = (rs + kIdxCutParts - 1) / kIdxCutParts;
#pragma unroll 1
            for (int bit = 31; bit >= 0; --bit) {
                const uint32_t t = tk | (1u << bit);
                tk = __builtin_popcountll(__ballot(k1 >= t)) >= need ? t : tk;
            }
        }
    }
    if (tid == 0)
        __hip_atomic_store(ws.cutk + (int64_t)(s * g.Hkv + gh) * kCutSlots + part, tk + 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// The in-launch cut for a chunk workgroup: wave 0 polls the kIdxCutParts part
// slots of its sequence (lane p reads part p with agent-scope loads) and, with
// want_b, the completed block's slot (lane kIdxCutParts) until every one is
// in; the mean of the part keys goes to tk and the block's key to kb.  The
// append and part workgroups come first in the grid and wait for nothing, so
// they are dispatched before any workgroup that polls and always finish; the
// bound on the polls (IdxAppend::polls, kCutPollsDefault) only makes every
// wave's exit certain.  Returns false (and no cut) when the bound is reached.
__device__ __forceinline__ bool idx_wait_cut(const uint32_t *slots, bool want_b, int polls, uint32_t &tk,
                                             uint32_t &kb, IdxShared &sh) {
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        const bool rd = lane < kIdxCutParts || (want_b && lane == kIdxCutParts);
        uint32_t x = 0u;
        int in = 0;
#pragma unroll 1
        for (int it = 0; it < polls; ++it) {
            x = rd ? __hip_atomic_load(slots + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 1u;
            if (__ballot(x == 0u) == 0ull) {       // (uniform)
                in = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        uint64_t sum = 0;
#pragma unroll
        for (int p = 0; p < kIdxCutParts; ++p) sum += (uint32_t)__builtin_amdgcn_readlane((int)x, p) - 1u;
        const uint32_t xb = (uint32_t)__builtin_amdgcn_readlane((int)x, kIdxCutParts);
        if (lane == 0) {
            sh.cut_tk = (uint32_t)(sum / kIdxCutParts);
            sh.cut_kb = xb - 1u;
            sh.cut_in = in;
        }
    }
    __syncthreads();
    tk = sh.cut_tk;
    kb = sh.cut_kb;
    return sh.cut_in != 0;
}

// grid (n_chunks [+1 with the fused append], Hkv, n_seq); mode 3 (with the
// checkpoint append) puts the append workgroup and then kIdxCutParts cut
// workgroups (idx_cut_part) before the chunks
template <int HD, int G>
__global__ void __launch_bounds__(kIdxThreads)
k_indexer(Geo g, qwfn_kv_view v, const float *__restrict__ q, const int32_t *seq_len, int32_t max_seq_len,
          int32_t *sel, int32_t *nsel, int32_t max_sel, Ws ws, int32_t n_chunks, FusedAppend fa,
          int32_t select_here, IdxAppend ia) {
#pragma clang fp contract(off)
    __shared__ IdxShared sh;
    const int tid = threadIdx.x, gh = blockIdx.y, s = blockIdx.z;
    const bool incut = select_here == 3;
    const int c = (int)blockIdx.x - (incut ? kIdxCutParts + 1 : 0);
    // the checkpoint indexer's append workgroup (one KV row): the first of the
    // grid in mode 3, else the last
    if (ia.enabled && (incut ? blockIdx.x == 0 : c == n_chunks)) {
        idx_append_wg<HD, G, kIdxThreads>(g, ia, q, seq_len, s, reinterpret_cast<uint16_t *>(v.pooled),
                                          ws.scores + (int64_t)s * g.Hkv * ws.nb_cap, sh.u.q);
        return;
    }
    if (c < 0) {                                   // mode 3: part blockIdx.x - 1 of the sequence's cut
        idx_cut_part<HD, G>(g, v, q, seq_len, max_seq_len, ws, s, gh, (int)blockIdx.x - 1, sh);
        return;
    }
    if (fa.enabled && c == n_chunks) {             // the append workgroup
        if (g.kt == QWFN_KV_Q4_0) fused_append_pool<HD, QWFN_KV_Q4_0, kIdxThreads>(g, v, fa, s, gh, seq_len, max_seq_len, sh);
        else if (g.kt == QWFN_KV_F16) fused_append_pool<HD, QWFN_KV_F16, kIdxThreads>(g, v, fa, s, gh, seq_len, max_seq_len, sh);
        else fused_append_pool<HD, QWFN_KV_Q8_0, kIdxThreads>(g, v, fa, s, gh, seq_len, max_seq_len, sh);
        return;
    }
    // select_here == 2 (a long decode row whose attention selects): the
    // chunk's eligible keys at or above the append launch's cut go to its
    // candidate slots, in block order, with their count; 3: the same with the
    // cut of this launch's part workgroups, waited for after the scoring (a
    // wait that runs out marks the chunk's count past kSelCandMax, and the
    // attention selects over the whole row)
    const bool emit = select_here >= 2;
    const int pair = s * g.Hkv + gh;
    uint32_t tk = 0u;
    if (select_here == 2) {                        // the append launch's part thresholds: their mean key
        static_assert(kIdxCutParts == 16, "four 16-byte loads");
        uint64_t sum = 0;
#pragma unroll
        for (int k = 0; k < kIdxCutParts / 4; ++k) {
            const u4v x = reinterpret_cast<const u4v *>(ws.cutk)[kIdxCutParts / 4 * pair + k];
            sum += (uint64_t)x[0] + x[1] + x[2] + x[3];
        }
        tk = (uint32_t)(sum / kIdxCutParts);
    }
    // the group's query rows do not depend on the length either
    constexpr int QV = (G * HD / 4 + kIdxThreads - 1) / kIdxThreads;
    const float4 *qg4 = reinterpret_cast<const float4 *>(q + ((int64_t)s * g.H + (int64_t)gh * G) * HD);
    float4 qv[QV];
#pragma unroll
    for (int i = 0; i < QV; ++i) qv[i] = qg4[min(tid + i * kIdxThreads, G * HD / 4 - 1)];
    const int L = seq_length(g, seq_len[g.pf ? 0 : s], s);
    const bool ok = L >= 1 && L <= max_seq_len;
    float *sc = ws.scores + (int64_t)pair * ws.nb_cap;
    int n_cand = 0;
    // The pooled keys this lane scores do not depend on the sequence length
    // (eligible blocks start at sink_blocks), so their loads go out together
    // with the length's; the length only decides which scores are kept.
    const int bl = tid >> 2, j = tid & 3;
    const int bi = c * kBlocksPerChunk + bl;
    const int bp = min(g.sink + bi, g.bps - 1);
    const int64_t prow = (((int64_t)cache_seq(g, s) * g.Hkv + gh) * g.bps + bp) * HD;
    float4 p4[HD / 16];
    if (g.pooled_f16) {                            // fp16 keys (the checkpoint indexer's pool cache)
        const uint16_t *P = reinterpret_cast<const uint16_t *>(v.pooled) + prow;
#pragma unroll
        for (int i = 0; i < HD / 16; ++i) {
            const uint2 x = *reinterpret_cast<const uint2 *>(P + 16 * i + 4 * j);
            p4[i] = make_float4(h2f((uint16_t)x.x), h2f((uint16_t)(x.x >> 16)), h2f((uint16_t)x.y),
                                h2f((uint16_t)(x.y >> 16)));
        }
    } else {
        const float *P = v.pooled + prow;
#pragma unroll
        for (int i = 0; i < HD / 16; ++i) p4[i] = *reinterpret_cast<const float4 *>(P + 16 * i + 4 * j);
    }
    if (ok && g.topk > 0) {
        const Ranges r = qsa_ranges(g, L);
        const int ne = r.e_hi - r.e_lo;
        if (ne > eff_topk(g, r) && c * kBlocksPerChunk < ne) {
            const int b = r.e_lo + bi;
            // the block this token completes is the append workgroup's to score
            const int bc = ia.enabled && L % g.bt == 0 ? (L - 1) / g.bt : -1;
            const bool act = bi < ne && b != bc;
#pragma unroll
            for (int i = 0; i < QV; ++i)
                if (tid + i * kIdxThreads < G * HD / 4) reinterpret_cast<float4 *>(sh.u.q)[tid + i * kIdxThreads] = qv[i];
            __syncthreads();
            float acc[G];
#pragma unroll
            for (int h = 0; h < G; ++h) acc[h] = 0.0f;
#pragma unroll
            for (int i = 0; i < HD / 16; ++i) {
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    const float4 q4 = *reinterpret_cast<const float4 *>(&sh.u.q[h * HD + 16 * i + 4 * j]);
                    acc[h] = fmaf(q4.x, p4[i].x, acc[h]);
                    acc[h] = fmaf(q4.y, p4[i].y, acc[h]);
                    acc[h] = fmaf(q4.z, p4[i].z, acc[h]);
                    acc[h] = fmaf(q4.w, p4[i].w, acc[h]);
                }
            }
            float score = 0.0f;
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float t01 = acc[h] + __shfl_xor(acc[h], 1);   // (c0+c1) / (c2+c3)
                float dot = t01 + __shfl_xor(t01, 2);               // (c0+c1)+(c2+c3)
                if (g.relu) dot = dot > 0.0f ? dot : 0.0f;
                score = (h == 0) ? dot : score + dot;
            }
            if (act && j == 0) sc[b] = score;
            if (emit) {                            // (uniform)
                // mode 3: the chunk holding the completed block takes that
                // block's key from the append workgroup, at the block's lane
                const int c0 = r.e_lo + c * kBlocksPerChunk;
                const bool want_b = incut && bc >= c0 && bc < c0 + kBlocksPerChunk && bc < r.e_hi;
                uint32_t kb = 0u;
                const bool cut_in =
                    !incut || idx_wait_cut(ws.cutk + (int64_t)pair * kCutSlots, want_b, ia.polls, tk, kb, sh);
                const uint32_t key = act ? score_key(score) : kb;
                const bool in = cut_in && (act || (want_b && b == bc)) && j == 0 && key >= tk;
                const uint64_t m = __ballot(in);
                const int lane = tid & 63, w = tid >> 6;
                if (lane == 0) sh.tmp[w] = __builtin_popcountll(m);
                __syncthreads();
                int at = __builtin_popcountll(m & ((1ull << lane) - 1ull));
#pragma unroll
                for (int i = 0; i < kIdxThreads / 64; ++i) {
                    at += i < w ? sh.tmp[i] : 0;
                    n_cand += sh.tmp[i];
                }
                if (in) ws.cand[((int64_t)pair * n_chunks + c) * kBlocksPerChunk + at] = make_uint2(key, (uint32_t)b);
                if (!cut_in) n_cand = kSelCandMax + 1;
            }
            __syncthreads();                       // q reads done before the union is reused
        }
    }
    if (emit && tid == 0) ws.ccnt[(int64_t)pair * n_chunks + c] = n_cand;   // 0 past the scored blocks
    // selection in a launch of its own (long contexts: k_select_big), or by
    // the attention
    if (select_here != 1) return;
    // completion count: the last workgroup of this (sequence, KV head) -- of
    // this sequence with a shared selection -- selects; the selection reads
    // the scores with device-coherent loads (or fences)
    const int cpair = g.shared ? s * g.Hkv : pair;
    if (!arrive_last<false>(&ws.cnt_idx[cpair], g.shared ? n_chunks * g.Hkv : n_chunks, &sh.flag)) return;
    if (tid == 0) ws.cnt_idx[cpair] = 0;
    const SelOut out = sel_out(g, sel, nsel, max_sel, s, pair);
    if (!ok) {
        if (tid == 0) {
            out.count(0);
            set_status(v.status, QWFN_STATUS_LEN_RANGE);
        }
        return;
    }
    if (g.shared)
        select_shared<kIdxThreads>(g, ws.scores + (int64_t)s * g.Hkv * ws.nb_cap, ws.nb_cap, L, out, sh);
    else
        select_blocks<kIdxThreads>(g, sc, L, out, sh);
}

// ---------------------------------------------------------------------------
// scoring of the fused decode call (the attention selects): small workgroups
// so the query rows every lane reads from LDS spread over many CUs
// ---------------------------------------------------------------------------

// Workgroup size and blocks a workgroup scores: 128 threads (two waves) and 16
// blocks, 256 and 32 at head_dim 256 (the append workgroup pools with one
// thread per dimension).  Every 128 threads keep one (min, max) record.
template <int HD> constexpr int score_threads() { return HD > 128 ? 256 : 128; }

template <int HD, int G>
struct ScoreShared {
    union {
        float q[G * HD];                           // the group's query rows
        struct { int8_t q8[kStageRows * 256]; uint16_t sc[kStageRows * 8]; } st;   // the append's pooling
    } u;
    float newk[256];
    float red[2][score_threads<HD>() / 64];
};

// grid (n_wg [+1 with the fused append], Hkv, n_seq).  Lane (b, hh, j) of a
// workgroup (j = tid & 3, hh = (tid >> 2) & 1, b = tid >> 3) holds dims
// 16i + 4j .. +3 of block b's pooled key and runs the decode indexer's four
// fmaf chains of heads hh*G/2 .. hh*G/2 + G/2 - 1 over them; the chains
// combine (c0+c1)+(c2+c3) across the j lanes and the heads sum in order, the
// second half continuing the first's sum (so every score is bit-identical to
// k_indexer's).  Each 128 threads write their 16 blocks' (min, max) eligible
// score to ws.cmm (+inf, -inf when none), the selection's histogram bounds;
// workgroups past the eligible blocks write nothing (the selection reads the
// records of eligible blocks only).
template <int HD, int G>
__global__ void __launch_bounds__(score_threads<HD>())
k_score(Geo g, qwfn_kv_view v, const float *__restrict__ q, const int32_t *seq_len, int32_t max_seq_len, Ws ws,
        int32_t n_wg, FusedAppend fa) {
#pragma clang fp contract(off)
    constexpr int NT = score_threads<HD>(), BPW = NT / 8, GH = G / 2;
    static_assert(G % 2 == 0 && NT >= HD, "two head halves; one pooling thread a dimension");
    __shared__ ScoreShared<HD, G> sh;
    const int tid = threadIdx.x, c = blockIdx.x, gh = blockIdx.y, s = blockIdx.z;
    if (fa.enabled && c == n_wg) {                 // the append workgroup
        if (g.kt == QWFN_KV_Q4_0) fused_append_pool<HD, QWFN_KV_Q4_0, NT>(g, v, fa, s, gh, seq_len, max_seq_len, sh);
        else if (g.kt == QWFN_KV_F16) fused_append_pool<HD, QWFN_KV_F16, NT>(g, v, fa, s, gh, seq_len, max_seq_len, sh);
        else fused_append_pool<HD, QWFN_KV_Q8_0, NT>(g, v, fa, s, gh, seq_len, max_seq_len, sh);
        return;
    }
    // one sequence: the length, the query rows and the pooled keys go out
    // together.  Several: the grid spans the longest one's blocks, so the
    // length comes first and a workgroup past its sequence's eligible blocks
    // ends before reading keys nothing uses
    const int L = seq_len[s];
    const bool ok = L >= 1 && L <= max_seq_len;
    if (gridDim.z > 1) {                           // (uniform)
        const Ranges r0 = qsa_ranges(g, L);
        const int ne0 = r0.e_hi - r0.e_lo;
        if (!(ok && g.topk > 0 && ne0 > eff_topk(g, r0) && c * BPW < ne0)) return;
    }
    constexpr int QV = (G * HD / 4 + NT - 1) / NT;
    const float4 *qg4 = reinterpret_cast<const float4 *>(q + ((int64_t)s * g.H + (int64_t)gh * G) * HD);
    float4 qv[QV];
#pragma unroll
    for (int i = 0; i < QV; ++i) qv[i] = qg4[min(tid + i * NT, G * HD / 4 - 1)];
    const int pair = s * g.Hkv + gh;
    const int j = tid & 3, hh = (tid >> 2) & 1, bl = tid >> 3;
    const int bi = c * BPW + bl;
    const int bp = min(g.sink + bi, g.bps - 1);
    const int64_t prow = (((int64_t)s * g.Hkv + gh) * g.bps + bp) * HD;
    float4 p4[HD / 16];
    if (g.pooled_f16) {
        const uint16_t *P = reinterpret_cast<const uint16_t *>(v.pooled) + prow;
#pragma unroll
        for (int i = 0; i < HD / 16; ++i) {
            const uint2 x = *reinterpret_cast<const uint2 *>(P + 16 * i + 4 * j);
            p4[i] = make_float4(h2f((uint16_t)x.x), h2f((uint16_t)(x.x >> 16)), h2f((uint16_t)x.y),
                                h2f((uint16_t)(x.y >> 16)));
        }
    } else {
        const float *P = v.pooled + prow;
#pragma unroll
        for (int i = 0; i < HD / 16; ++i) p4[i] = *reinterpret_cast<const float4 *>(P + 16 * i + 4 * j);
    }
    // a workgroup whose blocks are not scored (no selection at this length, or
    // past the eligible blocks) ends here: the selection reads the records of
    // the eligible blocks only
    const Ranges r = qsa_ranges(g, L);
    const int ne = r.e_hi - r.e_lo;
    if (!(ok && g.topk > 0 && ne > eff_topk(g, r) && c * BPW < ne)) return;
#pragma unroll
    for (int i = 0; i < QV; ++i)
        if (tid + i * NT < G * HD / 4) reinterpret_cast<float4 *>(sh.u.q)[tid + i * NT] = qv[i];
    __syncthreads();
    float cmx = -INFINITY, cmn = INFINITY;         // this record's largest / smallest score (not NaN)
    {
        const bool act = bi < ne;
        float acc[GH];
#pragma unroll
        for (int h = 0; h < GH; ++h) acc[h] = 0.0f;
#pragma unroll
        for (int i = 0; i < HD / 16; ++i) {
#pragma unroll
            for (int h = 0; h < GH; ++h) {
                const float4 q4 = *reinterpret_cast<const float4 *>(&sh.u.q[(hh * GH + h) * HD + 16 * i + 4 * j]);
                acc[h] = fmaf(q4.x, p4[i].x, acc[h]);
                acc[h] = fmaf(q4.y, p4[i].y, acc[h]);
                acc[h] = fmaf(q4.z, p4[i].z, acc[h]);
                acc[h] = fmaf(q4.w, p4[i].w, acc[h]);
            }
        }
        float dots[GH];
#pragma unroll
        for (int h = 0; h < GH; ++h) {
            const float t01 = acc[h] + __shfl_xor(acc[h], 1);   // (c0+c1) / (c2+c3)
            float dot = t01 + __shfl_xor(t01, 2);               // (c0+c1)+(c2+c3)
            dots[h] = g.relu && !(dot > 0.0f) ? 0.0f : dot;
        }
        // the sum of this half's heads in order; the second half (hh = 1)
        // continues from the first half's: dot_0 + dot_1 + ... + dot_{G-1}
        float part = dots[0];
#pragma unroll
        for (int h = 1; h < GH; ++h) part = part + dots[h];
        float score = __shfl_xor(part, 4) + dots[0];
#pragma unroll
        for (int h = 1; h < GH; ++h) score = score + dots[h];
        score = hh ? score : part;
        const int b = r.e_lo + bi;
        if (act && hh == 1 && j == 0) ws.scores[(int64_t)pair * ws.nb_cap + b] = score;
        cmx = act && score > cmx ? score : cmx;
        cmn = act && score < cmn ? score : cmn;
    }
    // this 128-thread half's (min, max) record
    cmx = wave_max(cmx);
    cmn = -wave_max(-cmn);
    const int w = tid >> 6;
    if ((tid & 63) == 0) { sh.red[0][w] = cmx; sh.red[1][w] = cmn; }
    __syncthreads();
    if ((tid & 127) == 0)
        ws.cmm[(int64_t)pair * (ws.nb_cap / kScoreRecBlocks) + c * (NT / 128) + (tid >> 7)] =
            make_float2(fminf(sh.red[1][w], sh.red[1][w + 1]), fmaxf(sh.red[0][w], sh.red[0][w + 1]));
}

template <int HD, int G>
static hipError_t launch_indexer_t(const Geo &g, const qwfn_kv_view &v, const float *q,
                                   const int32_t *seq_len, int32_t n_seq, int32_t max_seq_len,
                                   int32_t *sel, int32_t *nsel, int32_t max_sel, const Ws &ws,
                                   FusedAppend fa, hipStream_t st, bool select, bool sel_launch,
                                   const IdxAppend *ia, bool in_cut) {
    // The append workgroup's pooled block must not be one the scoring
    // workgroups read: with local_tokens = 0 a just-completed block is
    // eligible, so the append and the pooling run as launches of their own,
    // ordered before the scoring on the stream.
    if (fa.enabled && g.local == 0) {
        hipError_t e = launch_append(g, v, fa.k_new, fa.v_new, fa.src_f16, nullptr, nullptr, n_seq, 0, 0, st,
                                     seq_len);
        if (e != hipSuccess) return e;
        e = launch_pool(g, v, nullptr, nullptr, n_seq, 0, 0, st, seq_len);
        if (e != hipSuccess) return e;
        fa.enabled = 0;
    }
    if (!select) {                                 // the attention selects (k_dec / k_attn<..., SEL>)
        const int n_wg = ws.nb_cap / (score_threads<HD>() / 8);   // every (min, max) record written
        const dim3 grid((unsigned)(n_wg + (fa.enabled ? 1 : 0)), (unsigned)g.Hkv, (unsigned)n_seq);
        QWFN_LAUNCH(kTimedIndexer, (k_score<HD, G>), grid, dim3(score_threads<HD>()), st, g, v, q, seq_len,
                    max_seq_len, ws, n_wg, fa);
        return hipGetLastError();
    }
    const int nb_max = max_seq_len / g.bt;
    int n_chunks = (nb_max + kBlocksPerChunk - 1) / kBlocksPerChunk;
    if (n_chunks < 1) n_chunks = 1;
    IdxAppend ian{};
    if (ia) ian = *ia;
    const bool big = nb_max > kKeysMax;           // more eligible blocks than the workgroup's registers hold
    // 1: the last workgroup selects; 0: scores only (a selection launch
    // follows, or for a row the workgroup's registers hold the attention
    // selects: sel_launch false); 2: scores and each chunk's candidates (the
    // attention selects); 3: as 2 with the cut placed in this launch
    const int32_t mode = !big ? (sel_launch ? 1 : 0) : sel_launch ? 0 : in_cut ? 3 : 2;
    if (mode == 3 && !(ian.enabled && ian.slots && !fa.enabled)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((mode == 3 ? kIdxCutParts : 0) + n_chunks + (fa.enabled || ian.enabled ? 1 : 0)),
                    (unsigned)g.Hkv, (unsigned)n_seq);
    QWFN_LAUNCH(kTimedIndexer, (k_indexer<HD, G>), grid, dim3(kIdxThreads), st, g, v, q, seq_len, max_seq_len,
                sel, nsel, max_sel, ws, n_chunks, fa, mode, ian);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (!sel_launch) return hipSuccess;           // the attention selects (launch_dec_selbig / _selrow)
    if (big && ws.cut_wg > 0 && !(g.shared && g.Hkv > 1))
        hipLaunchKernelGGL(k_select_cut, dim3((unsigned)ws.cut_wg, (unsigned)(g.shared ? 1 : g.Hkv), (unsigned)n_seq),
                           dim3(kBigSelThreads), 0, st, g, v, seq_len, max_seq_len, ws, sel, nsel, max_sel);
    else if (big)
        hipLaunchKernelGGL(k_select_big, dim3((unsigned)(g.shared ? 1 : g.Hkv), (unsigned)n_seq),
                           dim3(kBigSelThreads), 0, st, g, v, seq_len, max_seq_len, ws.scores, ws.nb_cap, sel,
                           nsel, max_sel);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// attention: TG groups of NW waves per workgroup, one 64-cell tile per group;
// the groups merge in LDS into one partial softmax state per workgroup, and
// a merge launch (k_merge) combines the workgroups' partials.
// ---------------------------------------------------------------------------

// The combine of a (sequence, KV head)'s attention partials, a launch of its
// own after the attention: one workgroup per query head, so the parts are read
// by G workgroups on as many CUs rather than by one.
//   og = sum_i w_i O_i / sum_i w_i l_i,  w_i = exp2(m_i - max_i m_i)
// over the parts the attention wrote (its workgroups of tg tile groups, the
// count recomputed from the length and the selection as the attention counts
// it).  Thread (r, d), r = tid / HD (uniform in a wave), sums dimension d over
// the parts congruent to r mod R.  The length, the count, the (max, sum)
// pairs of parts lane and lane + 64, and the thread's first U part rows all go
// out in the first round trip (rows clamped to the most parts the attention
// can write, inside the pair's n_tiles rows).  Every wave reduces the maxima
// and weighted sums itself and takes a part's weight from the lane holding it
// (no LDS); one barrier adds the R sums.  A length out of range or no cell
// gives zeros (and, for a length, the status bit).
// grid (G, Hkv, n_seq or n_q), R * head_dim threads
template <int HD> constexpr int merge_r() { return HD > 128 ? 2 : 4; }
constexpr int kMergeRound = 24;                   // part rows a thread loads in one round
template <int G, int HD>
__global__ void __launch_bounds__(merge_r<HD>() * HD)
k_merge(Geo g, qwfn_kv_view v, const int32_t *seq_len, int32_t max_seq_len, const int32_t *nsel,
        int32_t max_sel, int32_t dense, float *__restrict__ out, Ws ws, int32_t tg) {
#pragma clang fp contract(off)
    constexpr int R = merge_r<HD>(), U = kMergeRound, PR = R * U;   // parts a round
    static_assert(PR <= 128 && HD % 64 == 0, "round weights in two lanes' registers; whole waves");
    __shared__ float red[R][HD];
    const int h = blockIdx.x, gh = blockIdx.y, s = blockIdx.z;
    const int tid = threadIdx.x, d = tid % HD, r = tid / HD, lane = tid & 63;
    const int pair = s * g.Hkv + gh;
    const int32_t *pl = seq_len + (g.pf ? 0 : s);
    const int L = seq_length(g, *pl, s);
    const int n_raw = *(dense ? pl : nsel + pair);
    const int64_t row = (int64_t)pair * ws.n_tiles * G + h;     // part i: row + i * G
    const float *pml = ws.part_ml + row * 2;
    const float *po = ws.part_o + row * HD + d;
    const int last = (ws.n_tiles + tg - 1) / tg - 1;
    float2 ml[2];
#pragma unroll
    for (int k = 0; k < 2; ++k)
        ml[k] = *reinterpret_cast<const float2 *>(pml + (int64_t)min(lane + 64 * k, last) * 2 * G);
    float x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) x[u] = po[(int64_t)min(r + R * u, last) * G * HD];
    const bool ok = L >= 1 && L <= max_seq_len;
    int n = 0;
    if (ok) {
        n = dense ? (L - 1) / g.bt + 1 : n_raw;
        n = n < max_sel ? n : max_sel;
    }
    const int parts = ((n * g.bt + 63) / 64 + tg - 1) / tg;
    float *og = out + ((int64_t)s * g.H + (int64_t)gh * G + h) * HD;
    if (!ok || parts == 0) {
        if (r == 0) og[d] = 0.0f;
        if (!ok && tid == 0 && gh == 0 && h == 0) set_status(v.status, QWFN_STATUS_LEN_RANGE);
        return;
    }
    auto m_of = [&](int i) { return pml[(int64_t)i * 2 * G]; };
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < 2; ++k) mx = lane + 64 * k < parts ? fmaxf(mx, ml[k].x) : mx;
    for (int i = lane + 128; i < parts; i += 64) mx = fmaxf(mx, m_of(i));
    const float M = wave_max(mx);
    auto weight = [&](float m) { return m == -INFINITY ? 0.0f : exp2f(m - M); };
    float wk[2];                                   // weights of parts lane, lane + 64 (0 past the parts)
    float ls = 0.0f;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const bool in = lane + 64 * k < parts;
        wk[k] = in ? weight(ml[k].x) : 0.0f;
        ls += wk[k] * (in ? ml[k].y : 0.0f);
    }
    for (int i = lane + 128; i < parts; i += 64) ls += weight(m_of(i)) * pml[(int64_t)i * 2 * G + 1];
    const float Ls = wave_sum(ls);
    // straight-line over the round: a part past the count has weight 0 and
    // its row, not written by this call, is replaced by 0
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int p = r + R * u;                   // wave-uniform
        const int w0 = __builtin_amdgcn_readlane(__builtin_bit_cast(int, wk[0]), p & 63);
        const int w1 = __builtin_amdgcn_readlane(__builtin_bit_cast(int, wk[1]), p & 63);
        const float wp = __builtin_bit_cast(float, p < 64 ? w0 : w1);
        acc += wp * (p < parts ? x[u] : 0.0f);
    }
    for (int i0 = PR; i0 < parts; i0 += PR) {     // more parts than one round
        float mu[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int p = min(i0 + r + R * u, parts - 1);
            x[u] = po[(int64_t)p * G * HD];
            mu[u] = m_of(p);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc += (i0 + r + R * u < parts ? weight(mu[u]) : 0.0f) * x[u];
    }
    red[r][d] = acc;
    __syncthreads();
    if (r == 0) {
        float o = red[0][d];
#pragma unroll
        for (int k = 1; k < R; ++k) o += red[k][d];
        og[d] = Ls > 0.0f ? o * (1.0f / Ls) : 0.0f;
    }
}

template <int G, int HD>
static void launch_merge_t(const Geo &g, const qwfn_kv_view &v, const int32_t *seq_len, int32_t n_seq,
                           int32_t max_seq_len, const int32_t *sel, const int32_t *nsel, int32_t max_sel,
                           float *out, const Ws &ws, int32_t tg, hipStream_t st) {
    QWFN_LAUNCH(kTimedMerge, (k_merge<G, HD>), dim3((unsigned)G, (unsigned)g.Hkv, (unsigned)n_seq),
                dim3(merge_r<HD>() * HD), st, g, v, seq_len, max_seq_len, nsel, max_sel, (int32_t)(sel == nullptr), out,
                ws, tg);
}

#define QWFN_FOR_EACH_MERGE(X) X(128, 8) X(128, 4) X(128, 2) X(64, 8) X(256, 12) X(256, 8)
hipError_t launch_merge(const Geo &g, const qwfn_kv_view &v, const int32_t *seq_len, int32_t n_seq,
                        int32_t max_seq_len, const int32_t *nsel, int32_t max_sel, bool dense, float *out,
                        const Ws &ws, int32_t tg, hipStream_t st) {
#define X(HD_, G_)                                                                                            \
    if (g.hd == HD_ && g.G == G_) {                                                                           \
        QWFN_LAUNCH(kTimedMerge, (k_merge<G_, HD_>), dim3((unsigned)G_, (unsigned)g.Hkv, (unsigned)n_seq),    \
                    dim3(merge_r<HD_>() * HD_), st, g, v, seq_len, max_seq_len, nsel, max_sel, (int32_t)dense, out, ws, \
                    tg);                                                                                      \
        return hipGetLastError();                                                                             \
    }
    QWFN_FOR_EACH_MERGE(X)
#undef X
    return hipErrorInvalidValue;
}


template <int HD, int G, int TG>
struct AttnCfg {
    static constexpr int NW = 4;                       // waves per group (a 64-cell tile)
    static constexpr int NTG = NW * 64;                // threads per group
    static constexpr int NT = TG * NTG;                // threads per workgroup
    static constexpr int ROWF = HD + 4;                // K' row (floats): cell-major, padded
    static constexpr int VROWF = 64 + 4;               // V' row (floats): dim-major, padded
    static constexpr int KVF = 64 * ROWF > HD * VROWF ? 64 * ROWF : HD * VROWF;   // K', then V', then O
    static constexpr int OPT = (G * HD + NT - 1) / NT; // merged outputs per thread
    static_assert(G <= 16, "one MFMA output column per query head");
    static_assert(HD % 64 == 0, "head_dim");
};

template <int HD, int G>
struct AttnGroup {
    float kv[AttnCfg<HD, G, 1>::KVF];          // K' [cell][HD], then V' [dim][cell], then the group's O [G][HD]
    float p[16][64 + 4];                       // softmax weights, [column][cell]
    uint16_t ksc[64][HD / 32], vsc[64][HD / 32];
    int32_t page[64], row[64];
    float m[G], l[G];
    float rm[4][16], rl[4][16];                // per-wave column max / sum
};

template <int HD, int G, int TG>
struct AttnShared {
    AttnGroup<HD, G> grp[TG];
};

// KT: the K/V element type (chunks of a head row, and their dequantization).
// SEL: the workgroups select for themselves; sel / nsel
// are then outputs.
template <int HD, int G, int TG, int KT, bool SEL = false>
__global__ void __launch_bounds__((AttnCfg<HD, G, TG>::NT))
k_attn(Geo g, qwfn_kv_view v, const float *__restrict__ q, const int32_t *seq_len,
       int32_t max_seq_len, const int32_t *sel, const int32_t *nsel, int32_t max_sel,
       float *__restrict__ out, Ws ws, int32_t n_parts) {
    using C = AttnCfg<HD, G, TG>;
    constexpr int CHK = row_bytes_t<HD, KT>() / 16;               // 16-byte chunks per head row
    const bool VDIM = KT == QWFN_KV_Q8_0 && g.vdim;               // V quants dim-major per 64-token tile
    constexpr int PERK = (64 * CHK + C::NTG - 1) / C::NTG;      // K (and V) chunk loads per thread
    static_assert(sizeof(AttnShared<HD, G, TG>) <= 160 * 1024, "LDS of the tile groups");
    __shared__ AttnShared<HD, G, TG> sh;
    __shared__ typename std::conditional<SEL, AttnSelShared<C::NT>, NoShared>::type ssh;
    const int tid = threadIdx.x, gh = blockIdx.y, s = blockIdx.z;
    const int gi = __builtin_amdgcn_readfirstlane(tid / C::NTG);   // tile group (wave-uniform)
    const int lt = tid % C::NTG;
    AttnGroup<HD, G> &gr = sh.grp[gi];
    const int pair = s * g.Hkv + gh;
    const int part = blockIdx.x;
    const int tile = part * TG + gi;
    const int lane = lt & 63, qcol = lane & 15, qk = lane >> 4;
    const int cidx = tile * 64 + lane;
    // The length, the selection count, the selected block of this lane's cell
    // and the query rows go out together: unconditional loads through pointers
    // chosen without a branch (the selection index clamped into the pair's
    // row; a dense call reads the length in place of the count and the block),
    // checked after they arrive.
    // With SEL the count and the blocks come from the workgroup's own
    // selection in LDS.
    const int32_t *pl = seq_len + (g.pf ? 0 : s);
    const bool has_sel = SEL || sel;
    int L, n_raw, blk_raw;
    if constexpr (SEL) {
        L = seq_length(g, *pl, s);
        attn_select<C::NT>(g, ws, L, max_seq_len, max_sel, pair, part, const_cast<int32_t *>(sel),
                           const_cast<int32_t *>(nsel), ssh);
        n_raw = ssh.nsel;
        blk_raw = ssh.sel[min(cidx / g.bt, kAttnSelMax - 1)];
    } else {
        const int32_t *pn = sel ? nsel + pair : pl;
        const int32_t *pb = sel ? sel + (int64_t)pair * max_sel + min(cidx / g.bt, max_sel - 1) : pl;
        L = seq_length(g, *pl, s);
        n_raw = *pn;
        blk_raw = *pb;
    }
    // the query as the QK operand: lane l holds head l%16 (0 past the
    // group), dims 16i + 4(l/16) .. +3 of every 16-dim step i
    float4 qreg[HD / 16];
    {
        const float *qh = q + ((int64_t)s * g.H + (int64_t)gh * G + min(qcol, G - 1)) * HD + 4 * qk;
#pragma unroll
        for (int i = 0; i < HD / 16; ++i) qreg[i] = *reinterpret_cast<const float4 *>(qh + 16 * i);
    }
    const bool ok = L >= 1 && L <= max_seq_len;
    int n = 0;
    if (ok) {
        n = has_sel ? n_raw : (L - 1) / g.bt + 1;
        n = n < max_sel ? n : max_sel;
    }
    const int tiles_act = (n * g.bt + 63) / 64;
    const int parts_act = (tiles_act + TG - 1) / TG;
    if (ok && part < parts_act) {
        const int wq = __builtin_amdgcn_readfirstlane(lt >> 6);
        if (qcol >= G) {
#pragma unroll
            for (int i = 0; i < HD / 16; ++i) qreg[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        const bool active = tile < tiles_act;
        // cells of this group's tile -> (physical page, row) or row -1
        if (lt < 64) {
            int pg = -1, rw = -1;
            const int slot = cidx / g.bt;
            if (active && slot < n) {
                const int blk = has_sel ? blk_raw : slot;
                const int t = blk * g.bt + cidx % g.bt;
                if (blk >= 0 && t < L) {
                    pg = phys_page(g, v.page_table, cache_seq(g, s), t);
                    rw = t % g.pt;
                    if (pg < 0) { set_status(v.status, QWFN_STATUS_PAGE_RANGE); rw = -1; }
                }
            }
            gr.page[lt] = pg;
            gr.row[lt] = rw;
        }
        __syncthreads();
        // every global load of the tile is issued before any is consumed
        uint4 kq[PERK], vq[PERK];
#pragma unroll
        for (int i = 0; i < PERK; ++i) {
            const int k = lt + i * C::NTG;
            kq[i] = make_uint4(0, 0, 0, 0);
            vq[i] = make_uint4(0, 0, 0, 0);
            if (k < 64 * CHK) {
                const int cell = k % 64, ch = k / 64, rw = gr.row[cell];
                if (rw >= 0) {
                    const int64_t off = (int64_t)gr.page[cell] * g.page_bytes +
                                        ((int64_t)(gh * (g.pt / 64) + rw / 64) * CHK + ch) * 1024 + (rw % 64) * 16;
                    kq[i] = *reinterpret_cast<const uint4 *>((const uint8_t *)v.k_pages + off);
                    if (!VDIM) vq[i] = *reinterpret_cast<const uint4 *>((const uint8_t *)v.v_pages + off);
                }
                // q8_0 in whole 64-token tiles: V quants dim-major, 64 bytes a
                // dim; chunk k = dim k / 4, cells 16 (k % 4) .. +15 of the tile
                // (one block, so one page and 64 aligned rows from cell 0's)
                const int rw0 = gr.row[0];
                if (VDIM && rw0 >= 0) {
                    const int64_t off = (int64_t)gr.page[0] * g.page_bytes +
                                        ((int64_t)(gh * (g.pt / 64) + rw0 / 64) * HD + k / 4) * 64 + (k % 4) * 16;
                    vq[i] = *reinterpret_cast<const uint4 *>((const uint8_t *)v.v_pages + off);
                }
            }
        }
        for (int k = lt; k < (KT == QWFN_KV_F16 ? 0 : 128); k += C::NTG) {
            const int cell = k % 64, rw = gr.row[cell];
            const bool isv = k >= 64;
            uint16_t *dst = isv ? gr.vsc[cell] : gr.ksc[cell];
            if (rw >= 0) {
                const uint16_t *src = reinterpret_cast<const uint16_t *>(
                    (const uint8_t *)(isv ? v.v_pages : v.k_pages) + (int64_t)gr.page[cell] * g.page_bytes +
                    g.qbytes + ((int64_t)(gh * g.pt + rw) * (HD / 32)) * 2);
#pragma unroll
                for (int jj = 0; jj < HD / 32; ++jj) dst[jj] = src[jj];
            } else {
#pragma unroll
                for (int jj = 0; jj < HD / 32; ++jj) dst[jj] = 0;
            }
        }
        __syncthreads();
        // dequantize exactly (fp16 scale times the quant, or the fp16 value;
        // then rounded to fp16 with kv_round_f16) into the group's LDS tile: K' cell-major, V' dim-major (transposed)
        auto dequant = [&](const uint4 *qv, uint16_t (*scl)[HD / 32], bool vt) {
            float *base = gr.kv;
#pragma unroll
            for (int i = 0; i < PERK; ++i) {
                const int k = lt + i * C::NTG;
                if (k < 64 * CHK) {
                    const int cell = k % 64, ch = k / 64;
                    const uint32_t w[4] = {qv[i].x, qv[i].y, qv[i].z, qv[i].w};
                    float x[KT == QWFN_KV_Q4_0 ? 32 : KT == QWFN_KV_F16 ? 8 : 16];
                    int d0;
                    if (KT == QWFN_KV_F16) {              // chunk = dims 8ch .. 8ch+7
                        d0 = 8 * ch;
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            x[2 * u] = h2f((uint16_t)w[u]);
                            x[2 * u + 1] = h2f((uint16_t)(w[u] >> 16));
                        }
                    } else if (KT == QWFN_KV_Q4_0) {      // chunk = ggml block ch: dims 32ch .. 32ch+31
                        d0 = 32 * ch;
                        const float scf = h2f(scl[cell][ch]);
#pragma unroll
                        for (int u = 0; u < 4; ++u)
#pragma unroll
                            for (int b = 0; b < 4; ++b) {
                                x[4 * u + b] = scf * (float)((int)((w[u] >> (8 * b)) & 15) - 8);
                                x[16 + 4 * u + b] = scf * (float)((int)((w[u] >> (8 * b + 4)) & 15) - 8);
                            }
                    } else if (VDIM && vt) {              // chunk = cells 16 (k % 4) .. +15 of dim k / 4
                        const int dim = k / 4, c0 = 16 * (k % 4);
#pragma unroll
                        for (int u = 0; u < 4; ++u)
#pragma unroll
                            for (int b = 0; b < 4; ++b) {
                                const int c = c0 + 4 * u + b;
                                const float xv = h2f(scl[c][dim / 32]) * (float)(int8_t)((w[u] >> (8 * b)) & 0xFF);
                                x[4 * u + b] = gr.row[c] >= 0 ? xv : 0.0f;
                            }
                        if (g.round_f16) {
#pragma unroll
                            for (int e = 0; e < 16; ++e) x[e] = (float)(_Float16)x[e];
                        }
#pragma unroll
                        for (int e = 0; e < 16; ++e) base[dim * C::VROWF + c0 + e] = x[e];
                        continue;
                    } else {                              // chunk = 16 dims of int8
                        d0 = 16 * ch;
                        const float scf = h2f(scl[cell][ch / 2]);
#pragma unroll
                        for (int u = 0; u < 4; ++u)
#pragma unroll
                            for (int b = 0; b < 4; ++b) x[4 * u + b] = scf * (float)(int8_t)((w[u] >> (8 * b)) & 0xFF);
                    }
                    constexpr int NX = sizeof(x) / sizeof(float);
                    if (g.round_f16) {                    // kv_round_f16: the reference's F16 cast (RNE)
#pragma unroll
                        for (int e = 0; e < NX; ++e) x[e] = (float)(_Float16)x[e];
                    }
                    if (vt) {                             // lanes hold consecutive cells: coalesced rows
#pragma unroll
                        for (int e = 0; e < NX; ++e) base[(d0 + e) * C::VROWF + cell] = x[e];
                    } else {
#pragma unroll
                        for (int e = 0; e < NX; e += 4)
                            *reinterpret_cast<float4 *>(base + cell * C::ROWF + d0 + e) =
                                make_float4(x[e], x[e + 1], x[e + 2], x[e + 3]);
                    }
                }
            }
        };
        dequant(kq, gr.ksc, false);
        __syncthreads();
        // QK on the matrix cores in fp32 (exact products): wave wq takes cells
        // 16wq .. +15, all 16 columns; v_mfma_f32_16x16x4f32 with the 16-dim
        // step's four k slots read as one 16-byte row segment per lane
        f4v sacc = f4v{0.0f, 0.0f, 0.0f, 0.0f};
        {
            const float *krow = &gr.kv[(16 * wq + qcol) * C::ROWF + 4 * qk];
#pragma unroll
            for (int i = 0; i < HD / 16; ++i) {
                const float4 a = *reinterpret_cast<const float4 *>(krow + 16 * i);
                sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, qreg[i].x, sacc, 0, 0, 0);
                sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, qreg[i].y, sacc, 0, 0, 0);
                sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, qreg[i].z, sacc, 0, 0, 0);
                sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, qreg[i].w, sacc, 0, 0, 0);
            }
        }
        // lane holds cells 16wq + 4qk + r (r < 4) of column qcol
        float s2[4];
        float tm = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const bool valid = gr.row[16 * wq + 4 * qk + r] >= 0;
            s2[r] = valid ? sacc[r] * g.scale_log2 : -INFINITY;
            tm = fmaxf(tm, s2[r]);
        }
        tm = col_max4(tm);
        if (qk == 0) gr.rm[wq][qcol] = tm;
        __syncthreads();                          // K' reads done, the waves' maxima visible
        const float m = fmaxf(fmaxf(gr.rm[0][qcol], gr.rm[1][qcol]), fmaxf(gr.rm[2][qcol], gr.rm[3][qcol]));
        float4 pw;
        float ts = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float pr = s2[r] == -INFINITY ? 0.0f : exp2f(s2[r] - m);
            (&pw.x)[r] = pr;
            ts += pr;
        }
        *reinterpret_cast<float4 *>(&gr.p[qcol][16 * wq + 4 * qk]) = pw;
        ts = col_sum4(ts);
        if (qk == 0) gr.rl[wq][qcol] = ts;
        dequant(vq, gr.vsc, true);
        __syncthreads();                          // V' and the weights visible
        if (lt < G) {
            gr.m[lt] = fmaxf(fmaxf(gr.rm[0][lt], gr.rm[1][lt]), fmaxf(gr.rm[2][lt], gr.rm[3][lt]));
            gr.l[lt] = (gr.rl[0][lt] + gr.rl[1][lt]) + (gr.rl[2][lt] + gr.rl[3][lt]);
        }
        // PV on the matrix cores: wave wq takes dim blocks wq, wq+4, ..; O[dim][column]
        constexpr int NDB = HD / 64;              // dim blocks per wave
        f4v o[NDB];
#pragma unroll
        for (int j = 0; j < NDB; ++j) {
            o[j] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
            const float *vrow = &gr.kv[(16 * (wq + 4 * j) + qcol) * C::VROWF + 4 * qk];
#pragma unroll
            for (int c = 0; c < 4; ++c) {         // 16 cells a step
                const float4 a = *reinterpret_cast<const float4 *>(vrow + 16 * c);
                const float4 b = *reinterpret_cast<const float4 *>(&gr.p[qcol][16 * c + 4 * qk]);
                o[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b.x, o[j], 0, 0, 0);
                o[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b.y, o[j], 0, 0, 0);
                o[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b.z, o[j], 0, 0, 0);
                o[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b.w, o[j], 0, 0, 0);
            }
        }
        __syncthreads();                          // V' reads done: kv becomes the group's O [head][dim]
        if (qcol < G) {
#pragma unroll
            for (int j = 0; j < NDB; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) gr.kv[qcol * HD + 16 * (wq + 4 * j) + 4 * qk + r] = o[j][r];
        }
        __syncthreads();
        // merge the TG groups into this workgroup's partial (unnormalised O, max, sum)
        const int64_t pb = ((int64_t)pair * ws.n_tiles + part) * G;
#pragma unroll
        for (int r = 0; r < C::OPT; ++r) {
            const int k = tid + r * C::NT;
            if (k < G * HD) {
                const int h = k / HD;
                float M = -INFINITY;
#pragma unroll
                for (int t = 0; t < TG; ++t)
                    if (part * TG + t < tiles_act) M = fmaxf(M, sh.grp[t].m[h]);
                float O = 0.0f, Ls = 0.0f;
#pragma unroll
                for (int t = 0; t < TG; ++t) {
                    if (part * TG + t < tiles_act) {
                        const float mt = sh.grp[t].m[h];
                        const float wt = mt == -INFINITY ? 0.0f : exp2f(mt - M);
                        O += wt * sh.grp[t].kv[k];
                        Ls += wt * sh.grp[t].l[h];
                    }
                }
                ws.part_o[pb * HD + k] = O;
                if (k % HD == 0) {
                    ws.part_ml[(pb + h) * 2 + 0] = M;
                    ws.part_ml[(pb + h) * 2 + 1] = Ls;
                }
            }
        }
    }
}

template <int HD, int G, int TG>
static void launch_attn_t(const Geo &g, const qwfn_kv_view &v, const float *q,
                          const int32_t *seq_len, int32_t n_seq, int32_t max_seq_len,
                          const int32_t *sel, const int32_t *nsel, int32_t max_sel, float *out,
                          const Ws &ws, hipStream_t st) {
    const int n_parts = (ws.n_tiles + TG - 1) / TG;
    const dim3 grid((unsigned)n_parts, (unsigned)g.Hkv, (unsigned)n_seq);
    const dim3 blk(AttnCfg<HD, G, TG>::NT);
    if (g.kt == QWFN_KV_Q4_0)
        QWFN_LAUNCH(kTimedAttention, (k_attn<HD, G, TG, QWFN_KV_Q4_0>), grid, blk, st, g, v, q, seq_len, max_seq_len,
                    sel, nsel, max_sel, out, ws, n_parts);
    else if (g.kt == QWFN_KV_F16)
        QWFN_LAUNCH(kTimedAttention, (k_attn<HD, G, TG, QWFN_KV_F16>), grid, blk, st, g, v, q, seq_len, max_seq_len,
                    sel, nsel, max_sel, out, ws, n_parts);
    else
        QWFN_LAUNCH(kTimedAttention, (k_attn<HD, G, TG, QWFN_KV_Q8_0>), grid, blk, st, g, v, q, seq_len, max_seq_len,
                    sel, nsel, max_sel, out, ws, n_parts);
    launch_merge_t<G, HD>(g, v, seq_len, n_seq, max_seq_len, sel, nsel, max_sel, out, ws, TG, st);
}

// The general attention selecting for itself (SEL): sel / nsel are outputs.
template <int HD, int G, int TG>
static void launch_attn_sel_t(const Geo &g, const qwfn_kv_view &v, const float *q,
                              const int32_t *seq_len, int32_t n_seq, int32_t max_seq_len,
                              int32_t *sel, int32_t *nsel, int32_t max_sel, float *out,
                              const Ws &ws, hipStream_t st) {
    const int n_parts = (ws.n_tiles + TG - 1) / TG;
    const dim3 grid((unsigned)n_parts, (unsigned)g.Hkv, (unsigned)n_seq);
    const dim3 blk(AttnCfg<HD, G, TG>::NT);
    if (g.kt == QWFN_KV_Q4_0)
        QWFN_LAUNCH(kTimedAttention, (k_attn<HD, G, TG, QWFN_KV_Q4_0, true>), grid, blk, st, g, v, q, seq_len,
                    max_seq_len, sel, nsel, max_sel, out, ws, n_parts);
    else if (g.kt == QWFN_KV_F16)
        QWFN_LAUNCH(kTimedAttention, (k_attn<HD, G, TG, QWFN_KV_F16, true>), grid, blk, st, g, v, q, seq_len,
                    max_seq_len, sel, nsel, max_sel, out, ws, n_parts);
    else
        QWFN_LAUNCH(kTimedAttention, (k_attn<HD, G, TG, QWFN_KV_Q8_0, true>), grid, blk, st, g, v, q, seq_len,
                    max_seq_len, sel, nsel, max_sel, out, ws, n_parts);
    launch_merge_t<G, HD>(g, v, seq_len, n_seq, max_seq_len, sel, nsel, max_sel, out, ws, TG, st);
}

// ---------------------------------------------------------------------------
// the reference's cache rows <-> the paged layout (format interop)
// ---------------------------------------------------------------------------

// One thread per (token, KV head, q8_0 block j) of positions pos0 .. pos0+n-1
// of sequence seq.  A row of the reference's cache is n_head_kv * head_dim / 32
// ggml blocks {fp16 d, int8 qs[32]} of 34 bytes, head-major, so block (h, j) of
// token t sits at row byte (h * head_dim/32 + j) * 34; rows are back to back.
// EXPORT copies the paged bytes out into rows, otherwise rows are written into
// the pages (an overwrite: the same bytes an append of the same values makes).
template <bool EXPORT>
__global__ void __launch_bounds__(256)
k_kv_rows(Geo g, qwfn_kv_view v, int32_t seq, int32_t pos0, int32_t n, uint8_t *k_rows, uint8_t *v_rows) {
    const int nb = g.hd / 32;
    const int64_t per_tok = (int64_t)g.Hkv * nb;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)n * per_tok) return;
    const int tl = (int)(i / per_tok), rem = (int)(i % per_tok);
    const int gh = rem / nb, j = rem % nb;
    const int t = pos0 + tl;
    const int32_t pp = phys_page(g, v.page_table, seq, t);
    if (pp < 0) { set_status(v.status, QWFN_STATUS_PAGE_RANGE); return; }
    const int row = t % g.pt;
#pragma unroll
    for (int which = 0; which < 2; ++which) {
        uint8_t *rows = which ? v_rows : k_rows;
        if (!rows) continue;
        uint8_t *page = (uint8_t *)(which ? v.v_pages : v.k_pages) + (int64_t)pp * g.page_bytes;
        if (g.kt != QWFN_KV_Q8_0) {
            // q4_0: ggml block {fp16 d; uint8 qs[16]} = the scale + chunk j;
            // fp16: the block's 32 values = chunks 4j .. 4j+3.  Rows are 2-byte aligned.
            const bool q4 = g.kt == QWFN_KV_Q4_0;
            uint16_t *rb = reinterpret_cast<uint16_t *>(rows + i * (q4 ? 18 : 64));
            uint16_t *cb = q4 ? rb + 1 : rb;
            const int nc = q4 ? 1 : 4, c0 = q4 ? j : 4 * j;
            for (int c = 0; c < nc; ++c) {
                uint4 *cp = reinterpret_cast<uint4 *>(page + chunk_off(g, gh, row, c0 + c));
                if (EXPORT) {
                    const uint4 a = *cp;
                    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        cb[8 * c + 2 * k] = (uint16_t)w[k];
                        cb[8 * c + 2 * k + 1] = (uint16_t)(w[k] >> 16);
                    }
                } else {
                    uint32_t w[4];
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        w[k] = (uint32_t)cb[8 * c + 2 * k] | ((uint32_t)cb[8 * c + 2 * k + 1] << 16);
                    *cp = make_uint4(w[0], w[1], w[2], w[3]);
                }
            }
            if (q4) {
                uint16_t *sp = reinterpret_cast<uint16_t *>(page + scale_off(g, gh, row, j));
                if (EXPORT) rb[0] = *sp;
                else *sp = rb[0];
            }
            continue;
        }
        uint16_t *rb = reinterpret_cast<uint16_t *>(rows + i * 34);          // 2-byte aligned
        uint16_t *sp = reinterpret_cast<uint16_t *>(page + scale_off(g, gh, row, j));
        if (!(which && g.vdim)) {                  // 16 dims of one token per 16-byte chunk
            uint4 *c0 = reinterpret_cast<uint4 *>(page + quant_off(g, gh, row, 32 * j));
            uint4 *c1 = reinterpret_cast<uint4 *>(page + quant_off(g, gh, row, 32 * j + 16));
            if (EXPORT) {
                const uint4 a = *c0, b = *c1;
                const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
                rb[0] = *sp;
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    rb[1 + 2 * k] = (uint16_t)w[k];
                    rb[2 + 2 * k] = (uint16_t)(w[k] >> 16);
                }
            } else {
                uint32_t w[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) w[k] = (uint32_t)rb[1 + 2 * k] | ((uint32_t)rb[2 + 2 * k] << 16);
                *c0 = make_uint4(w[0], w[1], w[2], w[3]);
                *c1 = make_uint4(w[4], w[5], w[6], w[7]);
                *sp = rb[0];
            }
        } else {                                   // V, dim-major tiles: one byte per dim
            if (EXPORT) {
                rb[0] = *sp;
#pragma unroll
                for (int e = 0; e < 32; e += 2)
                    rb[1 + e / 2] = (uint16_t)(page[vquant_off(g, gh, row, 32 * j + e)] |
                                               (page[vquant_off(g, gh, row, 32 * j + e + 1)] << 8));
            } else {
#pragma unroll
                for (int e = 0; e < 32; e += 2) {
                    const uint16_t x = rb[1 + e / 2];
                    page[vquant_off(g, gh, row, 32 * j + e)] = (uint8_t)x;
                    page[vquant_off(g, gh, row, 32 * j + e + 1)] = (uint8_t)(x >> 8);
                }
                *sp = rb[0];
            }
        }
    }
}

hipError_t launch_kv_rows(const Geo &g, const qwfn_kv_view &v, bool to_rows, int32_t seq, int32_t pos0,
                          int32_t n, void *k_rows, void *v_rows, hipStream_t st) {
    const int64_t threads = (int64_t)n * g.Hkv * (g.hd / 32);
    const dim3 grid((unsigned)((threads + 255) / 256));
    if (to_rows)
        hipLaunchKernelGGL(k_kv_rows<true>, grid, dim3(256), 0, st, g, v, seq, pos0, n, (uint8_t *)k_rows,
                           (uint8_t *)v_rows);
    else
        hipLaunchKernelGGL(k_kv_rows<false>, grid, dim3(256), 0, st, g, v, seq, pos0, n, (uint8_t *)k_rows,
                           (uint8_t *)v_rows);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// gather + dequant of a selection (parity / debug entry point)
// ---------------------------------------------------------------------------

// grid (n_cells_max, Hkv, n_seq), block = hd threads
__global__ void __launch_bounds__(256)
k_gather(Geo g, qwfn_kv_view v, const int32_t *seq_len, const int32_t *sel, const int32_t *nsel,
         int32_t max_sel, float *k_out, float *v_out, int32_t *cells) {
    const int c = blockIdx.x, gh = blockIdx.y, s = blockIdx.z, d = threadIdx.x;
    const int pair = s * g.Hkv + gh;
    const int ncell = max_sel * g.bt;
    const int L = seq_len[s];
    int t = -1;
    if (L >= 1 && (int64_t)L <= (int64_t)g.pps * g.pt) {
        const int n = sel ? min(nsel[pair], max_sel) : (L - 1) / g.bt + 1;
        const int slot = c / g.bt;
        if (slot < n) {
            const int blk = sel ? sel[(int64_t)pair * max_sel + slot] : slot;
            const int tt = blk * g.bt + c % g.bt;
            if (blk >= 0 && tt < L) t = tt;
        }
    }
    const int64_t o = ((int64_t)pair * ncell + c) * g.hd + d;
    int32_t pp = t >= 0 ? phys_page(g, v.page_table, s, t) : -1;
    if (t >= 0 && pp < 0) { if (d == 0) set_status(v.status, QWFN_STATUS_PAGE_RANGE); t = -1; }
    if (d == 0) cells[(int64_t)pair * ncell + c] = t;
    if (t < 0) { k_out[o] = 0.0f; v_out[o] = 0.0f; return; }
    const int rw = t % g.pt;
    k_out[o] = member_k(g, (const uint8_t *)v.k_pages + (int64_t)pp * g.page_bytes, gh, rw, d);
    v_out[o] = member_k(g, (const uint8_t *)v.v_pages + (int64_t)pp * g.page_bytes, gh, rw, d, true);
}

hipError_t launch_gather(const Geo &g, const qwfn_kv_view &v, const int32_t *seq_len,
                         int32_t n_seq, const int32_t *sel, const int32_t *nsel,
                         int32_t max_sel, float *k_out, float *v_out, int32_t *cells,
                         hipStream_t st) {
    const dim3 grid((unsigned)(max_sel * g.bt), (unsigned)g.Hkv, (unsigned)n_seq);
    hipLaunchKernelGGL(k_gather, grid, dim3((unsigned)g.hd), 0, st, g, v, seq_len, sel, nsel, max_sel,
                       k_out, v_out, cells);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// prefill: scores of a chunk's queries, then one selection per (query, KV head)
// ---------------------------------------------------------------------------

constexpr int kPfQA = 8;                   // queries per thread
constexpr int kPfQ = 16 * kPfQA, kPfB = 64;  // queries x blocks per scoring workgroup
constexpr int kPfSD = 8;                   // 16-byte dim chunks of the query rows per LDS stage

constexpr int kPfQPad = kPfQ + kPfQ / kPfQA;   // one spare chunk after every 8 queries

// Query qq of a stage sits at chunk qq + qq / 8 of its dim row: the four
// 8-query groups one wave reads at a time land 144 bytes apart, on different
// LDS banks.
__device__ __forceinline__ int pf_qslot(int qq) { return qq + qq / kPfQA; }

template <int HD>
struct PfScoreShared {
    float4 p[HD / 4][kPfB];                // the tile's pooled keys, dim-chunk major
    float4 q[kPfSD][kPfQPad];              // a 64-dim stage of the current head's query rows
};

// grid (ceil((n_blk - sink) / 64), ceil(n_q / 128), Hkv), 256 threads.  The
// workgroup scores 128 queries against 64 pooled blocks of one KV head: the
// pooled keys are loaded once into LDS (reused 128 times), the query rows
// 64 dims at a time (reused 64 times); thread t owns queries 8*(t/16) .. +8 x
// blocks t%16 + {0, 16, 32, 48} (16 consecutive blocks per read across a row
// of lanes: no LDS bank conflicts), so each pooled-key read feeds 32 FMAs.
// The next stage's query rows are loaded into registers while the current
// stage is computed, so the global reads of a stage overlap the FMAs.
// Each dot is formed in the decode indexer's order (chain j over the dims d
// with (d/4)%4 == j in increasing order, then (c0+c1)+(c2+c3), relu when set,
// heads summed in order), so a query's scores are bit-identical to a decode
// step's at its length.  Scores go to scores[(query * Hkv + gh) * nb_cap +
// block] for blocks sink .. n_blk-1.
template <int HD, int G>
__global__ void __launch_bounds__(256)
k_pf_scores(Geo g, qwfn_kv_view v, const float *__restrict__ q, int32_t n_q, int32_t n_blk,
            float *__restrict__ scores, int32_t nb_cap) {
#pragma clang fp contract(off)
    __shared__ PfScoreShared<HD> sh;
    constexpr int NDC = HD / 4, QA = kPfQA;
    constexpr int SD = NDC < kPfSD ? NDC : kPfSD;          // dim chunks per stage
    static_assert(NDC % SD == 0 && SD % 4 == 0, "whole stages of whole 16-dim groups");
    const int tid = threadIdx.x, gh = blockIdx.z;
    const int b_base = g.sink + (int)blockIdx.x * kPfB;
    const int q_base = (int)blockIdx.y * kPfQ;
    const int64_t prow = ((int64_t)g.pf_seq * g.Hkv + gh) * g.bps * HD;
    for (int i = tid; i < kPfB * NDC; i += 256) {
        const int b = i / NDC, dc = i % NDC;
        const int bb = min(b_base + b, g.bps - 1);
        if (g.pooled_f16) {                        // fp16 keys (the checkpoint indexer's pool cache)
            const uint2 x = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(v.pooled) + prow +
                                                             (int64_t)bb * HD + 4 * dc);
            sh.p[dc][b] = make_float4(h2f((uint16_t)x.x), h2f((uint16_t)(x.x >> 16)), h2f((uint16_t)x.y),
                                      h2f((uint16_t)(x.y >> 16)));
        } else {
            sh.p[dc][b] = *reinterpret_cast<const float4 *>(v.pooled + prow + (int64_t)bb * HD + 4 * dc);
        }
    }
    const int qi0 = QA * (tid / 16), bi0 = tid % 16;
    float score[QA][4];
#pragma unroll
    for (int a = 0; a < QA; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) score[a][b] = 0.0f;
    constexpr int NST = NDC / SD;                          // stages per head
    constexpr int QPT = kPfQ * SD / 256;                   // query chunks a thread stages
    static_assert(kPfQ * SD % 256 == 0, "whole stages per thread");
    // the next stage's chunks, in flight: thread t stages chunk i = t + 256 r
    // of (query i / SD, dim chunk i % SD) for r < QPT
    const float *qsrc[QPT];
#pragma unroll
    for (int r = 0; r < QPT; ++r) {
        const int i = tid + 256 * r;
        const int qn = min(q_base + i / SD, n_q - 1);
        qsrc[r] = q + ((int64_t)qn * g.H + gh * G) * HD + 4 * (i % SD);
    }
    f4v nq[QPT];
#pragma unroll
    for (int r = 0; r < QPT; ++r) nq[r] = *reinterpret_cast<const f4v *>(qsrc[r]);
    for (int h = 0; h < G; ++h) {
        float c[QA][4][4];                           // [query][block][chain]
#pragma unroll
        for (int a = 0; a < QA; ++a)
#pragma unroll
            for (int b = 0; b < 4; ++b)
#pragma unroll
                for (int j = 0; j < 4; ++j) c[a][b][j] = 0.0f;
        for (int sti = 0; sti < NST; ++sti) {
            const int st = sti * SD;
            __syncthreads();                         // the previous stage's rows are consumed
#pragma unroll
            for (int r = 0; r < QPT; ++r) {
                const int i = tid + 256 * r;
                *reinterpret_cast<f4v *>(&sh.q[i % SD][pf_qslot(i / SD)]) = nq[r];
            }
            __syncthreads();
            if (h * NST + sti + 1 < G * NST) {
                const int nx = h * NST + sti + 1;
                const int off = nx / NST * HD + nx % NST * SD * 4;   // head nx / NST, dims of stage nx % NST
#pragma unroll
                for (int r = 0; r < QPT; ++r) nq[r] = *reinterpret_cast<const f4v *>(qsrc[r] + off);
            }
            for (int d16 = 0; d16 < SD / 4; ++d16) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {        // dims 16*d16 + 4j .. +3 belong to chain j
                    const int dcl = 4 * d16 + j;
                    float4 qv[QA], pv[4];
                    const int qs0 = pf_qslot(qi0);   // the thread's 8 queries share one group
#pragma unroll
                    for (int a = 0; a < QA; ++a) qv[a] = sh.q[dcl][qs0 + a];
#pragma unroll
                    for (int b = 0; b < 4; ++b) pv[b] = sh.p[st + dcl][bi0 + 16 * b];
#pragma unroll
                    for (int a = 0; a < QA; ++a)
#pragma unroll
                        for (int b = 0; b < 4; ++b) {
                            float x = c[a][b][j];
                            x = fmaf(qv[a].x, pv[b].x, x);
                            x = fmaf(qv[a].y, pv[b].y, x);
                            x = fmaf(qv[a].z, pv[b].z, x);
                            x = fmaf(qv[a].w, pv[b].w, x);
                            c[a][b][j] = x;
                        }
                }
            }
        }
#pragma unroll
        for (int a = 0; a < QA; ++a)
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                float dot = (c[a][b][0] + c[a][b][1]) + (c[a][b][2] + c[a][b][3]);
                if (g.relu) dot = dot > 0.0f ? dot : 0.0f;
                score[a][b] = h == 0 ? dot : score[a][b] + dot;
            }
    }
#pragma unroll
    for (int a = 0; a < QA; ++a) {
        const int qn = q_base + qi0 + a;
        if (qn >= n_q) continue;
        float *row = scores + ((int64_t)qn * g.Hkv + gh) * nb_cap;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int blk = b_base + bi0 + 16 * b;
            if (blk < n_blk) row[blk] = score[a][b];
        }
    }
}

// grid (Hkv, n_q), kIdxThreads: query s's selection at its length pf_pos0+s+1
// from the scores k_pf_scores wrote (the decode selection, same rule).
__global__ void __launch_bounds__(kIdxThreads)
k_pf_select(Geo g, float *scores, int32_t nb_cap, int32_t *sel, int32_t *nsel, int32_t max_sel) {
    __shared__ IdxShared sh;
    const int gh = blockIdx.x, s = blockIdx.y;             // (gh = 0 with a shared selection)
    const int pair = s * g.Hkv + gh;
    const SelOut out = sel_out(g, sel, nsel, max_sel, s, pair);
    if (g.shared)
        select_shared<kIdxThreads>(g, scores + (int64_t)pair * nb_cap, nb_cap, g.pf_pos0 + s + 1, out, sh);
    else
        select_blocks<kIdxThreads>(g, scores + (int64_t)pair * nb_cap, g.pf_pos0 + s + 1, out, sh);
}

// ---------------------------------------------------------------------------
// prefill scoring on the matrix cores: approximate scores with an error
// bound, then exact scores for the blocks the bound leaves open
// ---------------------------------------------------------------------------

constexpr int kPaQ = 64;              // queries per approximate-scoring workgroup (16 a wave)
constexpr int kPaB = 64;              // pooled blocks per staged tile
constexpr int kPaSplit = 2;           // workgroups sharing one query tile's blocks (measured best of 1, 2, 4, 8)
constexpr int kPaSplitBig = 16;       // the same for one 40960-block row: 40 tiles a workgroup (8, 32, 64: within 0.1 ms)
constexpr int kRefineMax = 512;       // candidates ranked exactly (more: the whole row exactly)
constexpr int kRefineBlocks = 4096;   // eligible blocks the approximate path takes
// |approximate - exact| <= kPaRel * (sum over the group's heads of |q_h|) * |p|
// + kPaAbs (Euclidean norms: sum_d |q_hd p_d| <= |q_h| |p|).  The terms, each
// relative to sum_h |q_h| |p|: fp16 rounding of both operands, 2 * 2^-11 +
// 2^-22 of each product; the matrix cores' fp32 sums, one accumulator a chain
// of pa_chain<HD, G>(relu) heads (one with relu, else as many as keep the
// chain at 256 products: CH * HD - 1 adds, rounded at each in the worst case),
// then the G / CH chain sums in order (relu'd when set) and the
// power-of-two rescale (exact), below (CH * HD - 1 + G / CH - 1) * 2^-24 <=
// 258 * 2^-24 for every instantiation (G * HD <= 1024, so G / CH <= 4 without
// relu; HD <= 256, G <= 8 with it); the exact scores' own rounding (four chains of HD / 4 fmas,
// their two sums, the head sum), below 80 * 2^-24; fp16 subnormals, below
// 2^-30.  They sum to at most 9.97e-4; the 5 % left covers the rounding of
// the norms (rounded up by 2^-14) and of the bound itself.  The budget is
// restated and checked per instantiated shape on the CPU, and the kernel's
// outputs against it on the GPU.
constexpr float kPaRel = 1.05e-3f;
// an absolute floor: a score that underflows fp32 keeps no relative precision
constexpr float kPaAbs = 1e-37f;

template <int HD, int G> constexpr bool pf_approx_fits() { return G * HD <= 1024 && HD % 32 == 0 && 256 % G == 0; }
// heads whose products k_pf_approx sums in one accumulator (see kPaRel)
template <int HD, int G> constexpr int pa_chain(bool relu) {
    return relu || HD >= 256 ? 1 : (256 / HD < G ? 256 / HD : G);
}

// The power of two that scales a row whose largest magnitude is m into
// [2^14, 2^15) (fp16 keeps 11 significant bits there): 15 - e for m = f 2^e.
__device__ __forceinline__ int fp16_shift(float m) {
    int e = 0;
    frexpf(m, &e);
    return m > 0.0f ? 15 - e : 0;
}

// Chunk dc of pooled block b as fp32 (fp16 keys widened exactly).
__device__ __forceinline__ float4 pooled_chunk(const Geo &g, const qwfn_kv_view &v, int64_t off) {
    if (g.pooled_f16) {
        const uint2 w = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(v.pooled) + off);
        return make_float4(h2f((uint16_t)w.x), h2f((uint16_t)(w.x >> 16)), h2f((uint16_t)w.y),
                           h2f((uint16_t)(w.y >> 16)));
    }
    return *reinterpret_cast<const float4 *>(v.pooled + off);
}

// N chunks of the pooled keys as fp32, chunk i at element offset off(i):
// the format test taken once, every load issued before any is used (a test
// per load leaves one memory round trip per chunk).
template <int N, typename F>
__device__ __forceinline__ void pooled_chunks(const Geo &g, const qwfn_kv_view &v, F off, float4 (&x)[N]) {
    if (g.pooled_f16) {
        const uint16_t *p = reinterpret_cast<const uint16_t *>(v.pooled);
        uint2 w[N];
#pragma unroll
        for (int i = 0; i < N; ++i) w[i] = *reinterpret_cast<const uint2 *>(p + off(i));
#pragma unroll
        for (int i = 0; i < N; ++i)
            x[i] = make_float4(h2f((uint16_t)w[i].x), h2f((uint16_t)(w[i].x >> 16)), h2f((uint16_t)w[i].y),
                               h2f((uint16_t)(w[i].y >> 16)));
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) x[i] = *reinterpret_cast<const float4 *>(v.pooled + off(i));
    }
}

// The G query rows at qg (head h at qg + h HD) spread over the wave: lane l
// holds dims l + 64 t of every head, to be broadcast one value at a time.
template <int HD, int G>
struct PfQLanes {
    float x[G][HD / 64];
};
template <int HD, int G>
__device__ __forceinline__ PfQLanes<HD, G> pf_q_lanes(const float *qg) {
    const int lane = threadIdx.x & 63;
    PfQLanes<HD, G> r;
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int t = 0; t < HD / 64; ++t) r.x[h][t] = qg[h * HD + 64 * t + lane];
    return r;
}

// The exact score of the pooled block at element offset koff for those query
// rows, one lane a block, in k_pf_scores' order: per head four fmaf chains,
// chain j over the dims of the chunks 4 d16 + j, combined (c0 + c1) + (c2 +
// c3), relu'd when set, the heads summed in order.  Each query value is read
// out of its lane (v_readlane with a constant lane; every lane must be
// active, its value defined): the same values as broadcast LDS reads, two
// addresses a wave, measured ten times slower.
template <int HD, int G>
__device__ __forceinline__ float pf_exact_score(const Geo &g, const qwfn_kv_view &v, int64_t koff,
                                                const PfQLanes<HD, G> &ql) {
#pragma clang fp contract(off)
    constexpr int NCH = HD / 16;
    float c[G][4];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j) c[h][j] = 0.0f;
    auto qv = [&](int h, int d) -> float {
        return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ql.x[h][d / 64]), d % 64));
    };
#pragma unroll
    for (int d16 = 0; d16 < NCH; ++d16) {
        float4 k4[4];
        pooled_chunks<4>(g, v, [&](int j) -> int64_t { return koff + 16 * d16 + 4 * j; }, k4);
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d = 16 * d16 + 4 * j;
                c[h][j] = fmaf(qv(h, d + 0), k4[j].x, c[h][j]);
                c[h][j] = fmaf(qv(h, d + 1), k4[j].y, c[h][j]);
                c[h][j] = fmaf(qv(h, d + 2), k4[j].z, c[h][j]);
                c[h][j] = fmaf(qv(h, d + 3), k4[j].w, c[h][j]);
            }
    }
    float score = 0.0f;
#pragma unroll
    for (int h = 0; h < G; ++h) {
        float dot = (c[h][0] + c[h][1]) + (c[h][2] + c[h][3]);
        if (g.relu) dot = dot > 0.0f ? dot : 0.0f;
        score = h == 0 ? dot : score + dot;
    }
    return score;
}

template <int HD>
struct PaShared {
    uint2 p[kPaB][HD / 4 + 2];            // the tile's pooled keys as fp16, each block scaled; rows + 16 bytes
    int pe[kPaB];                         // the blocks' scale exponents
};

// grid (ceil(n_q / 64), split, Hkv), 256 threads.  Approximate scores of
// 64 queries against the eligible blocks [sink, n_blk) of KV head gh (tiles
// blockIdx.y, blockIdx.y + split, ... of 64 blocks): S[query][block] = sum
// over the group's heads of (relu'd when set) q_h . p on
// v_mfma_f32_16x16x32_f16.  The A operand, the query scaled by a power of two
// (its largest element over the group's heads in [2^14, 2^15)), stays in
// registers for the launch; each tile of pooled keys, every block scaled the
// same way, is staged in LDS as the B operand.  Wave w owns queries 16w ..
// 16w+15; a lane's outputs are 4 queries x 1 block, scaled back exactly.  The
// query-tile-0 workgroups also write each block's |p| (rounded up) to pnorm.
// Pooled keys are fp32, or fp16 (the checkpoint indexer's pool) widened exactly.
template <int HD, int G, bool RELU>
__global__ void __launch_bounds__(256, 2)
k_pf_approx(Geo g, qwfn_kv_view v, const float *__restrict__ q, int32_t n_q, int32_t n_blk,
            float *__restrict__ scores, int32_t nb_cap, float *__restrict__ pnorm) {
    constexpr int NK = HD / 32;                        // k-steps of one head
    constexpr int CPT = HD / 16;                       // 16-byte fp32 chunks a thread stages (4 threads a block)
    constexpr int CH = pa_chain<HD, G>(RELU);          // heads a chain
    static_assert(pf_approx_fits<HD, G>() && G % CH == 0, "a wave's query fragments fit its registers");
    __shared__ PaShared<HD> sh;
    const int tid = threadIdx.x, l = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int gh = blockIdx.z, row = l & 15, kg = l >> 4;
    const int qbase = (int)blockIdx.x * kPaQ + 16 * wv;
    // A operand: query qbase + row, dims 32 ks + 8 kg .. +8 of each head
    const float *qrow = q + ((int64_t)min(qbase + row, n_q - 1) * g.H + gh * G) * HD + 8 * kg;
    float qm = 0.0f;
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int ks = 0; ks < NK; ++ks) {
            const float4 a = *reinterpret_cast<const float4 *>(qrow + h * HD + 32 * ks);
            const float4 b = *reinterpret_cast<const float4 *>(qrow + h * HD + 32 * ks + 4);
            qm = fmaxf(qm, fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))));
            qm = fmaxf(qm, fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
        }
    qm = fmaxf(qm, __shfl_xor(qm, 16));
    qm = fmaxf(qm, __shfl_xor(qm, 32));
    const int qe = fp16_shift(qm);
    h8v qa[G][NK];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int ks = 0; ks < NK; ++ks) {
            const float4 a = *reinterpret_cast<const float4 *>(qrow + h * HD + 32 * ks);
            const float4 b = *reinterpret_cast<const float4 *>(qrow + h * HD + 32 * ks + 4);
            qa[h][ks] = h8v{(_Float16)ldexpf(a.x, qe), (_Float16)ldexpf(a.y, qe), (_Float16)ldexpf(a.z, qe),
                            (_Float16)ldexpf(a.w, qe), (_Float16)ldexpf(b.x, qe), (_Float16)ldexpf(b.y, qe),
                            (_Float16)ldexpf(b.z, qe), (_Float16)ldexpf(b.w, qe)};
        }
    // the scale exponents of this lane's output rows (queries qbase + 4 kg + i)
    int qe_o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) qe_o[i] = __shfl(qe, 4 * kg + i);
    const int n_tiles = (n_blk - g.sink + kPaB - 1) / kPaB;
    const int64_t prow = ((int64_t)g.pf_seq * g.Hkv + gh) * g.bps;   // the row's first pooled block
    const int sb = tid >> 2, sc = tid & 3;             // staging: block sb of the tile, chunks sc + 4 i
    for (int t = (int)blockIdx.y; t < n_tiles; t += (int)gridDim.y) {
        const int b0 = g.sink + t * kPaB;
        const int bb = min(b0 + sb, n_blk - 1);
        // chunks sc + 4 i of block bb: 4 consecutive dims each
        const auto chunk_off = [&](int i) -> int64_t { return (prow + bb) * HD + 4 * (sc + 4 * i); };
        // the block's largest element, then (a second, cache-hot read) its
        // scaled fp16 values and squares
        float m = 0.0f;
        {
            float4 xs[CPT];
            pooled_chunks<CPT>(g, v, chunk_off, xs);
#pragma unroll
            for (int i = 0; i < CPT; ++i) {
                const float4 x = xs[i];
                m = fmaxf(m, fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w))));
            }
        }
        m = fmaxf(m, __shfl_xor(m, 1));
        m = fmaxf(m, __shfl_xor(m, 2));
        const int pe = fp16_shift(m);
        __syncthreads();                               // the previous tile's fragments are read
        float ss = 0.0f;
        float4 xs[CPT];
        pooled_chunks<CPT>(g, v, chunk_off, xs);
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const float4 x = xs[i];
            const float y0 = ldexpf(x.x, pe), y1 = ldexpf(x.y, pe), y2 = ldexpf(x.z, pe), y3 = ldexpf(x.w, pe);
            ss = __builtin_fmaf(y0, y0, ss);
            ss = __builtin_fmaf(y1, y1, ss);
            ss = __builtin_fmaf(y2, y2, ss);
            ss = __builtin_fmaf(y3, y3, ss);
            const half2v lo2 = {(_Float16)y0, (_Float16)y1}, hi2 = {(_Float16)y2, (_Float16)y3};
            sh.p[sb][sc + 4 * i] = make_uint2(__builtin_bit_cast(uint32_t, lo2), __builtin_bit_cast(uint32_t, hi2));
        }
        if (sc == 0) sh.pe[sb] = pe;
        ss += __shfl_xor(ss, 1);
        ss += __shfl_xor(ss, 2);
        if (blockIdx.x == 0 && sc == 0 && b0 + sb < n_blk)
            pnorm[(int64_t)gh * nb_cap + b0 + sb] = ldexpf(sqrtf(ss) * (1.0f + 0x1p-14f), -pe);
        __syncthreads();
#pragma unroll
        for (int ct = 0; ct < kPaB / 16; ++ct) {
            h8v bf[NK];                                // B operand: block 16 ct + row, dims 32 ks + 8 kg .. +8
#pragma unroll
            for (int ks = 0; ks < NK; ++ks)
                bf[ks] = *reinterpret_cast<const h8v *>(&sh.p[16 * ct + row][2 * (4 * ks + kg)]);
            // one accumulator a chain of CH heads (CH * HD products), the
            // chains' sums (relu'd when set) added in order: the fp32 sums of
            // one score stay within (CH * HD - 1) + (G / CH - 1) roundings,
            // the budget of kPaRel
            f4v tot;
#pragma unroll
            for (int h0 = 0; h0 < G; h0 += CH) {
                f4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int h = h0; h < h0 + CH; ++h)
#pragma unroll
                    for (int ks = 0; ks < NK; ++ks)
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[h][ks], bf[ks], acc, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float x = RELU ? fmaxf(acc[i], 0.0f) : acc[i];
                    tot[i] = h0 == 0 ? x : tot[i] + x;
                }
            }
            const int blk = b0 + 16 * ct + row;
            const int pb = sh.pe[16 * ct + row];
            if (blk < n_blk) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int qo = qbase + 4 * kg + i;
                    if (qo < n_q) scores[((int64_t)qo * g.Hkv + gh) * nb_cap + blk] = ldexpf(tot[i], -(qe_o[i] + pb));
                }
            }
        }
    }
}

// Exact dots of a pooled block with heads [h0, h0 + NH) in the decode
// indexer's order (k_pf_scores): chain j over the dims d with (d / 4) % 4 == j
// in increasing order, then (c0 + c1) + (c2 + c3), relu'd when set.  pchunk(dc)
// gives the key's dims 4 dc .. 4 dc + 3; qs holds the group's query rows,
// qstride floats apart.  Each key chunk is read once and feeds NH * 4 fmas.
template <int HD, int NH, class PC>
__device__ __forceinline__ void pf_exact_dots(const Geo &g, PC pchunk, const float *qs, int qstride, int h0,
                                              float (&dot)[NH]) {
#pragma clang fp contract(off)
    float c[NH][4];
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j) c[h][j] = 0.0f;
#pragma unroll 2
    for (int d16 = 0; d16 < HD / 16; ++d16)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int dc = 4 * d16 + j;
            const float4 p4 = pchunk(dc);
#pragma unroll
            for (int h = 0; h < NH; ++h) {
                const float4 q4 = *reinterpret_cast<const float4 *>(qs + (h0 + h) * qstride + 4 * dc);
                float x = c[h][j];
                x = fmaf(q4.x, p4.x, x);
                x = fmaf(q4.y, p4.y, x);
                x = fmaf(q4.z, p4.z, x);
                x = fmaf(q4.w, p4.w, x);
                c[h][j] = x;
            }
        }
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        float d = (c[h][0] + c[h][1]) + (c[h][2] + c[h][3]);
        if (g.relu) d = d > 0.0f ? d : 0.0f;
        dot[h] = d;
    }
}


// LDS of the 256-thread selection (select_blocks: register path, radix
// fallback) without the indexer's scoring and pooling stage.
struct RefineSel {
    uint32_t hist[4096 + 64];
    uint32_t cand_key[kCandMax + 1];
    int32_t cand_b[kCandMax + 1];
    uint32_t tmask[kIdxThreads];
    uint32_t selbits[kKeysMax / 32 + 1];
    float red[2 * (kIdxThreads / 64)];
    int tmp[16];
    int flag, bin, need, ncand, cnt_b;
};

template <int HD, int G>
struct RefineShared {
    float q[G * (HD + 4)];                        // the group's query rows, padded
    RefineSel s;                                  // the histogram; select_blocks' state on the fallback
    uint32_t ckey[kRefineMax];                    // candidates in block order: exact score keys, blocks
    int32_t cblk[kRefineMax];
    int32_t rk[kRefineMax];                       // their ranks
    int32_t cbase[kRefineBlocks / 64];            // candidates before each (thread row, wave) group
    float qn[G];
};

// grid (Hkv, n_q), kIdxThreads: query s's selection for KV head gh at its
// length pf_pos0 + s + 1, identical to the selection on the exact scores.
// The exact score of block b (k_pf_scores' order) lies within E_b = kPaRel *
// sum_h |q_h| * |p_b| + kPaAbs of its approximate score a_b (k_pf_approx).
// Let T be the topk-th largest lower bound a_b - E_b over the eligible
// blocks: at least topk blocks score at least T exactly, so every block of
// the exact top-k has a_b + E_b >= T.  The candidates -- upper bounds in or
// above T's bin of a 4096-bin histogram of the lower bounds, a monotone map --
// are gathered in block order and scored exactly; the top-k of them by (score
// desc, index asc) is the selection, emitted at its prefix-sum places.  A
// non-finite approximate score or bound, or more than kRefineMax candidates,
// scores the whole row exactly for select_blocks instead.  Four waves a
// SIMD (128 registers; the fallback's registers spill) ran the config-4
// chunk faster than three or two.
template <int HD, int G>
__global__ void __launch_bounds__(kIdxThreads, 4)
k_pf_refine(Geo g, qwfn_kv_view v, const float *__restrict__ q, float *scores, int32_t nb_cap,
            const float *__restrict__ pnorm, int32_t *sel, int32_t *nsel, int32_t max_sel) {
#pragma clang fp contract(off)
    constexpr int NT = kIdxThreads, QS = HD + 4, KPT = kRefineBlocks / NT, NW = NT / 64;
    constexpr int NCH = HD / 16;                       // key chunks of one chain
    static_assert(pf_approx_fits<HD, G>() && KPT * NW <= kRefineBlocks / 64, "group table");
    __shared__ RefineShared<HD, G> sh;
    const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int gh = blockIdx.x, s = blockIdx.y;
    const int pair = s * g.Hkv + gh;
    const int L = g.pf_pos0 + s + 1;
    const SelOut out = sel_out(g, sel, nsel, max_sel, s, pair);
    float *row = scores + (int64_t)pair * nb_cap;
    const Ranges r = qsa_ranges(g, L);
    const int topk = eff_topk(g, r);
    if (g.topk <= 0 || r.e_hi - r.e_lo <= topk || topk == 0) {   // nothing ranked: no score is read
        select_blocks<NT, RefineSel, kRefineBlocks>(g, row, L, out, sh.s);
        return;
    }
    const int64_t prow = ((int64_t)g.pf_seq * g.Hkv + gh) * g.bps;
    // the approximate scores and key norms of this thread's blocks e_lo + tid + NT i
    float av[KPT], pv[KPT];
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
        const int b = min(r.e_lo + tid + NT * i, r.e_hi - 1);
        av[i] = row[b];
        pv[i] = pnorm[(int64_t)gh * nb_cap + b];
    }
    float *qs = sh.q;
    const float *qrow = q + ((int64_t)s * g.H + gh * G) * HD;
    for (int i = tid; i < G * HD / 4; i += NT) {
        const int h = i / (HD / 4), c = i % (HD / 4);
        *reinterpret_cast<float4 *>(qs + h * QS + 4 * c) = *reinterpret_cast<const float4 *>(qrow + h * HD + 4 * c);
    }
    __syncthreads();
    // |q_h| (rounded up), one wave a head, scaled by a power of two against overflow and underflow
    for (int h = wid; h < G; h += NW) {
        float m = 0.0f;
        for (int d = lane; d < HD; d += 64) m = fmaxf(m, fabsf(qs[h * QS + d]));
        const int e = fp16_shift(wave_max(m));
        float ss = 0.0f;
        for (int d = lane; d < HD; d += 64) {
            const float y = ldexpf(qs[h * QS + d], e);
            ss = __builtin_fmaf(y, y, ss);
        }
        ss = wave_sum(ss);
        if (lane == 0) sh.qn[h] = ldexpf(sqrtf(ss) * (1.0f + 0x1p-14f), -e);
    }
    __syncthreads();
    float qn = 0.0f;
#pragma unroll
    for (int h = 0; h < G; ++h) qn += sh.qn[h];
    const float ec = kPaRel * qn * (1.0f + 0x1p-14f);
    float lb[KPT], ub[KPT];
    bool bad = !(ec < INFINITY) || r.e_hi - r.e_lo > KPT * NT;   // (the launch keeps rows within KPT * NT)
    float lo = INFINITY, hi = -INFINITY;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
        const bool in = r.e_lo + tid + NT * i < r.e_hi;
        const float e = __builtin_fmaf(ec, pv[i], kPaAbs);
        lb[i] = in ? av[i] - e : -INFINITY;
        ub[i] = in ? av[i] + e : -INFINITY;
        bad |= in && (!(fabsf(av[i]) < INFINITY) || !(e < INFINITY));
        lo = fminf(lo, in ? lb[i] : INFINITY);
        hi = fmaxf(hi, lb[i]);
    }
    hi = wave_max(hi);
    lo = -wave_max(-lo);
    if (lane == 0) { sh.s.red[wid] = hi; sh.s.red[NW + wid] = lo; }
    uint4 *h4 = reinterpret_cast<uint4 *>(sh.s.hist);
#pragma unroll
    for (int i = 0; i < 4096 / 4 / NT; ++i) h4[tid + i * NT] = make_uint4(0u, 0u, 0u, 0u);
    bad = __syncthreads_or(bad);
    int nc = 0;
    if (!bad) {
#pragma unroll
        for (int i = 0; i < NW; ++i) { hi = fmaxf(hi, sh.s.red[i]); lo = fminf(lo, sh.s.red[NW + i]); }
        const float span = hi - lo, scale = 4096.0f / span;
        const bool lin = hi > lo && span < INFINITY && scale < INFINITY;
        // monotone in x: a linear map of [lo, hi], else the top 12 key bits
        auto bin_of = [&](float x) -> uint32_t {
            return lin ? (uint32_t)fminf(fmaxf((x - lo) * scale, 0.0f), 4095.0f) : score_key(x) >> 20;
        };
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const bool in = r.e_lo + tid + NT * i < r.e_hi;
            atomicAdd(&sh.s.hist[in ? bin_of(lb[i]) : 4096u + (uint32_t)lane], 1u);
        }
        __syncthreads();
        if (wid == 0) hist_cut(sh.s, topk);
        __syncthreads();
        const uint32_t B = (uint32_t)sh.s.bin;
        // candidates in block order: group (i, wave) holds blocks e_lo + NT i + 64 wave + lane
        uint32_t cm = 0;                              // this thread's candidate bits, one per i
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const bool c = r.e_lo + tid + NT * i < r.e_hi && bin_of(ub[i]) >= B;
            cm |= (uint32_t)c << i;
            const uint64_t m = __ballot(c);
            if (lane == 0) sh.cbase[i * NW + wid] = (int)__builtin_popcountll(m);
        }
        __syncthreads();
        if (wid == 0) {                               // exclusive scan of the group counts
            const int x = lane < KPT * NW ? sh.cbase[lane] : 0;
            const int incl = wave_incl_scan(x);
            if (lane < KPT * NW) sh.cbase[lane] = incl - x;
            if (lane == 63) sh.s.ncand = incl;
        }
        __syncthreads();
        nc = __builtin_amdgcn_readfirstlane(sh.s.ncand);   // uniform: scalar loop bounds below
        if (nc <= kRefineMax) {
            const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
            for (int i = 0; i < KPT; ++i) {
                const bool c = (cm >> i) & 1u;
                const uint64_t m = __ballot(c);
                if (c) sh.cblk[sh.cbase[i * NW + wid] + (int)__builtin_popcountll(m & below)] = r.e_lo + tid + NT * i;
            }
        }
        for (int i = tid; i < kRefineMax; i += NT) sh.rk[i] = 0;
        __syncthreads();
    }
    if (bad || nc > kRefineMax) {
        // the whole row exactly (k_pf_scores' values), then the plain selection
        constexpr int HPT = G < 4 ? G : 4;
        for (int b = r.e_lo + tid; b < r.e_hi; b += NT) {
            float sc = 0.0f;
            for (int h0 = 0; h0 < G; h0 += HPT) {     // HPT heads at a time, summed in head order
                float d[HPT];
                pf_exact_dots<HD, HPT>(g, [&](int dc) { return pooled_chunk(g, v, (prow + b) * HD + 4 * dc); }, qs,
                                       QS, h0, d);
#pragma unroll
                for (int h = 0; h < HPT; ++h) sc = h0 + h == 0 ? d[h] : sc + d[h];
            }
            row[b] = sc;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");   // the exact row, for the selection's loads
        __syncthreads();
        select_blocks<NT, RefineSel, kRefineBlocks>(g, row, L, out, sh.s);
        return;
    }
    // exact scores of the candidates, 128 at a time, two threads each: thread
    // half takes chains 2 half and 2 half + 1 of every head, reading its key
    // chunks 4 d16 + chain straight from memory (all of them in flight); the
    // pair combines (c0 + c1) + (c2 + c3), then the first sums the heads in order
    for (int c0 = 0; c0 < nc; c0 += NT / 2) {
        const int ci = c0 + (tid >> 1), half = tid & 1;
        const int b = sh.cblk[min(ci, nc - 1)];
        float4 pk[2 * NCH];                            // chunk 4 d16 + 2 half + k at pk[k NCH + d16]
        pooled_chunks<2 * NCH>(g, v, [&](int i) -> int64_t {
            return (prow + b) * HD + 4 * (4 * (i % NCH) + 2 * half + i / NCH);
        }, pk);
        float score = 0.0f;
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float cc[2];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                float x = 0.0f;
#pragma unroll
                for (int d16 = 0; d16 < NCH; ++d16) {
                    const float4 q4 = *reinterpret_cast<const float4 *>(qs + h * QS + 4 * (4 * d16 + 2 * half + k));
                    x = fmaf(q4.x, pk[k * NCH + d16].x, x);
                    x = fmaf(q4.y, pk[k * NCH + d16].y, x);
                    x = fmaf(q4.z, pk[k * NCH + d16].z, x);
                    x = fmaf(q4.w, pk[k * NCH + d16].w, x);
                }
                cc[k] = x;
            }
            const float pair_sum = cc[0] + cc[1];        // c0 + c1 (half 0), c2 + c3 (half 1)
            float dot = pair_sum + __shfl_xor(pair_sum, 1);
            if (g.relu) dot = dot > 0.0f ? dot : 0.0f;
            score = h == 0 ? dot : score + dot;
        }
        if (half == 0 && ci < nc) sh.ckey[ci] = score_key(score);
    }
    __syncthreads();
    // rank by (key desc, index asc) -- the order of the composite (key, ~block),
    // above 2^31 for every candidate -- the first topk taken.  Candidates i0 ..
    // i0+63 sit one a lane in every wave; each wave counts the larger keys among
    // 16 of every 64 candidates, broadcast from registers.
    auto order_key = [&](int i) -> uint64_t {
        return i < nc ? ((uint64_t)sh.ckey[i] << 32) | (uint32_t)~sh.cblk[i] : 0ull;
    };
    for (int i0 = 0; i0 < nc; i0 += 64) {
        const uint64_t ci = order_key(i0 + lane);
        int part = 0;
        for (int j0 = 0; j0 < nc; j0 += 64) {
            const uint64_t cj = order_key(j0 + lane);
            const uint32_t jh = (uint32_t)(cj >> 32), jl = (uint32_t)cj;
            const int k_end = min(min(64, nc - j0), 16 * wid + 16);
            for (int k = 16 * wid; k < k_end; ++k) {
                const uint64_t ck = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(jh, k) << 32) |
                                    (uint32_t)__builtin_amdgcn_readlane(jl, k);
                part += ck > ci;
            }
        }
        if (i0 + lane < nc) atomicAdd(&sh.rk[i0 + lane], part);
    }
    __syncthreads();
    // emission in block order between the sink and the window blocks: a taken
    // candidate's place is the count of taken candidates before it
    {
        constexpr int PER = kRefineMax / NT;          // candidates a thread, consecutive
        int cnt = 0;
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int i = PER * tid + k;
            cnt += i < nc && sh.rk[i] < topk;
        }
        int tot;
        int pos = block_excl_sum<NT>(cnt, sh.s.tmp, &tot);
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int i = PER * tid + k;
            if (i < nc && sh.rk[i] < topk) out.put(g.sink + pos++, sh.cblk[i]);
        }
    }
    emit_forced<NT>(g, r, topk, out);
}

// The same refinement for one score row of up to kRbBlocks eligible blocks
// (a single KV head, or a selection shared by every KV head through one
// scoring head group: the checkpoint indexer's 4-token blocks): one
// 1024-thread workgroup per query, thread t holding the 4-block groups
// base + 4 (t + 1024 j), j < kRbKpt / 4 (base = e_lo rounded down to a
// multiple of 4: coalesced 16-byte loads; every 64-lane wave row then covers
// 256 consecutive blocks, in block order by (j, wave, lane)), up to kRbMax
// candidates; the LDS of k_select_big, whose
// candidate arrays hold the candidates and whose selection is the fallback.
constexpr int kRbThreads = kBigSelThreads, kRbKpt = 40, kRbBlocks = kRbThreads * kRbKpt, kRbMax = 2048;
static_assert(kRbMax <= kSelCandMax, "the candidates fit BigSelShared's arrays");

template <int HD, int G>
struct RefineBigShared {
    BigSelShared s;                               // histogram, reductions; ckey / cblk: the candidates
    float q[G * (HD + 4)];                        // the group's query rows, padded
    int32_t cbase[kRbKpt / 4 * (kRbThreads / 64)]; // candidates before each (j, wave) row
    int32_t rk[kRbMax];                           // the ranks of the threshold bin's candidates
    int32_t mem[kRbMax];                          // the threshold bin's candidates
    float qn[G];
};

// grid (1, n_q), kRbThreads: query s's selection (g.Hkv == 1; with a shared
// selection every KV head's row) from k_pf_approx's scores, by the bound and
// candidate argument of k_pf_refine.
template <int HD, int G>
__global__ void __launch_bounds__(kRbThreads)
k_pf_refine_big(Geo g, qwfn_kv_view v, const float *__restrict__ q, float *scores, int32_t nb_cap,
                const float *__restrict__ pnorm, int32_t *sel, int32_t *nsel, int32_t max_sel) {
#pragma clang fp contract(off)
    constexpr int NT = kRbThreads, QS = HD + 4, KPT = kRbKpt, NW = NT / 64, NCH = HD / 16;
    constexpr int NJ = KPT / 4, NG = NJ * NW;          // 4-block groups a thread; (j, wave) rows
    static_assert(pf_approx_fits<HD, G>() && G * HD / 4 <= NT && G <= NW && KPT % 4 == 0 && NG <= NT, "shapes");
    __shared__ RefineBigShared<HD, G> sh;
    const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int s = blockIdx.y;
    const int L = g.pf_pos0 + s + 1;
    const SelOut out = sel_out(g, sel, nsel, max_sel, s, s);
    float *row = scores + (int64_t)s * nb_cap;
    const Ranges r = qsa_ranges(g, L);
    const int topk = eff_topk(g, r);
    if (g.topk <= 0 || r.e_hi - r.e_lo <= topk || topk == 0) {   // nothing ranked: no score is read
        select_blocks<NT>(g, row, L, out, sh.s);
        return;
    }
    const int64_t prow = (int64_t)g.pf_seq * g.bps;
    const int b0 = (r.e_lo & ~3) + 4 * tid;            // group j starts at b0 + 4 NT j
    // rows start 256-byte aligned (nb_cap is a multiple of 64) and every
    // 16-byte group read starts below e_hi <= nb_cap
    const int last4 = (r.e_hi - 1) & ~3;
    auto blk = [&](int i) { return b0 + 4 * NT * (i / 4) + (i % 4); };   // block of register i
    float av[KPT], pv[KPT];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int b = min(b0 + 4 * NT * j, last4);
        const float4 a4 = *reinterpret_cast<const float4 *>(row + b);
        const float4 p4 = *reinterpret_cast<const float4 *>(pnorm + b);
        av[4 * j] = a4.x; av[4 * j + 1] = a4.y; av[4 * j + 2] = a4.z; av[4 * j + 3] = a4.w;
        pv[4 * j] = p4.x; pv[4 * j + 1] = p4.y; pv[4 * j + 2] = p4.z; pv[4 * j + 3] = p4.w;
    }
    auto in_row = [&](int i) { return blk(i) >= r.e_lo && blk(i) < r.e_hi; };
    float *qs = sh.q;
    const float *qrow = q + (int64_t)s * g.H * HD;
    if (tid < G * HD / 4) {
        const int h = tid / (HD / 4), c = tid % (HD / 4);
        *reinterpret_cast<float4 *>(qs + h * QS + 4 * c) = *reinterpret_cast<const float4 *>(qrow + h * HD + 4 * c);
    }
    __syncthreads();
    if (wid < G) {                                     // |q_h| (rounded up), one wave a head
        float m = 0.0f;
        for (int d = lane; d < HD; d += 64) m = fmaxf(m, fabsf(qs[wid * QS + d]));
        const int e = fp16_shift(wave_max(m));
        float ss = 0.0f;
        for (int d = lane; d < HD; d += 64) {
            const float y = ldexpf(qs[wid * QS + d], e);
            ss = __builtin_fmaf(y, y, ss);
        }
        ss = wave_sum(ss);
        if (lane == 0) sh.qn[wid] = ldexpf(sqrtf(ss) * (1.0f + 0x1p-14f), -e);
    }
    __syncthreads();
    float qn = 0.0f;
#pragma unroll
    for (int h = 0; h < G; ++h) qn += sh.qn[h];
    const float ec = kPaRel * qn * (1.0f + 0x1p-14f);
    // bounds, in place: av becomes the lower, pv the upper bound
    bool bad = !(ec < INFINITY) || r.e_hi - (r.e_lo & ~3) > KPT * NT;   // (the launch keeps rows within)
    float lo = INFINITY, hi = -INFINITY;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
        const bool in = in_row(i);
        const float e = __builtin_fmaf(ec, pv[i], kPaAbs);
        bad |= in && (!(fabsf(av[i]) < INFINITY) || !(e < INFINITY));
        const float a = av[i];
        av[i] = in ? a - e : -INFINITY;
        pv[i] = in ? a + e : -INFINITY;
        lo = fminf(lo, in ? av[i] : INFINITY);
        hi = fmaxf(hi, av[i]);
    }
    hi = wave_max(hi);
    lo = -wave_max(-lo);
    if (lane == 0) { sh.s.red[wid] = hi; sh.s.red[NW + wid] = lo; }
    reinterpret_cast<uint4 *>(sh.s.hist)[tid] = make_uint4(0u, 0u, 0u, 0u);   // 4096 bins, 4 a thread
    if (tid < 64) sh.s.hist[4096 + tid] = 0u;
    bad = __syncthreads_or(bad);
    int nc = 0;
    if (!bad) {
#pragma unroll
        for (int i = 0; i < NW; ++i) { hi = fmaxf(hi, sh.s.red[i]); lo = fminf(lo, sh.s.red[NW + i]); }
        const float span = hi - lo, scale = 4096.0f / span;
        const bool lin = hi > lo && span < INFINITY && scale < INFINITY;
        auto bin_of = [&](float x) -> uint32_t {
            return lin ? (uint32_t)fminf(fmaxf((x - lo) * scale, 0.0f), 4095.0f) : score_key(x) >> 20;
        };
#pragma unroll
        for (int i = 0; i < KPT; ++i) atomicAdd(&sh.s.hist[in_row(i) ? bin_of(av[i]) : 4096u + (uint32_t)lane], 1u);
        __syncthreads();
        if (wid == 0) hist_cut(sh.s, topk);
        __syncthreads();
        const uint32_t B = (uint32_t)sh.s.bin;
        uint64_t cm = 0;
#pragma unroll
        for (int i = 0; i < KPT; ++i) cm |= (uint64_t)(in_row(i) && bin_of(pv[i]) >= B) << i;
        // in block order: row (j, wave) after the rows before it, lane after lane
        int ex[NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int c = (int)__builtin_popcount((uint32_t)(cm >> (4 * j)) & 0xFu);
            const int incl = wave_incl_scan(c);
            ex[j] = incl - c;
            if (lane == 63) sh.cbase[j * NW + wid] = incl;
        }
        __syncthreads();
        {
            const int x = tid < NG ? sh.cbase[tid] : 0;
            const int e = block_excl_sum<NT>(x, sh.s.tmp, &nc);
            if (tid < NG) sh.cbase[tid] = e;
        }
        __syncthreads();
        nc = __builtin_amdgcn_readfirstlane(nc);
        if (nc <= kRbMax) {
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                int pos = sh.cbase[j * NW + wid] + ex[j];
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if ((cm >> (4 * j + k)) & 1u) sh.s.cblk[pos++] = blk(4 * j + k);
            }
        }
        for (int i = tid; i < kRbMax; i += NT) sh.rk[i] = 0;
        __syncthreads();
    }
    if (bad || nc > kRbMax) {
        // the whole row exactly (k_pf_scores' values), then the plain selection
        for (int b = r.e_lo + tid; b < r.e_hi; b += NT) {
            float sc = 0.0f;
            float d[G];
            pf_exact_dots<HD, G>(g, [&](int dc) { return pooled_chunk(g, v, (prow + b) * HD + 4 * dc); }, qs, QS, 0, d);
#pragma unroll
            for (int h = 0; h < G; ++h) sc = h == 0 ? d[h] : sc + d[h];
            row[b] = sc;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");   // the exact row, for the selection's loads
        __syncthreads();
        select_blocks<NT>(g, row, L, out, sh.s);
        return;
    }
    // exact scores of the candidates, one a lane
    // (whole waves, every lane active: the query values are read out of lanes)
    const PfQLanes<HD, G> ql = pf_q_lanes<HD, G>(qrow);
    for (int c0 = 0; c0 < nc; c0 += NT) {
        if (c0 + 64 * wid >= nc) continue;             // wave-uniform
        const int ci = min(c0 + tid, nc - 1);
        const float sc = pf_exact_score<HD, G>(g, v, (prow + sh.s.cblk[ci]) * HD, ql);
        if (c0 + tid < nc) sh.s.ckey[ci] = score_key(sc);
    }
    __syncthreads();
    // The topk-th largest exact score lies among the candidates (every other
    // block scores below it): the bin of its top 12 key bits over the
    // candidates, then that bin's candidates ranked by (key desc, index asc).
    for (int i = tid; i < 4096 + 64; i += NT) sh.s.hist[i] = 0u;
    if (tid == 0) sh.s.ctot = 0;
    __syncthreads();
    for (int i = tid; i < nc; i += NT) atomicAdd(&sh.s.hist[sh.s.ckey[i] >> 20], 1u);
    __syncthreads();
    if (wid == 0) hist_cut(sh.s, topk);
    __syncthreads();
    const uint32_t B1 = (uint32_t)sh.s.bin;
    const int need = sh.s.need;
    for (int i = tid; i < nc; i += NT)
        if (sh.s.ckey[i] >> 20 == B1) sh.mem[atomicAdd(&sh.s.ctot, 1)] = i;
    __syncthreads();
    const int nm = __builtin_amdgcn_readfirstlane(sh.s.ctot);
    // members j0 .. j0+63 one a lane in every wave; each wave counts the larger
    // composite keys (key, ~block) among 64 / NW of every 64 members
    auto order_key = [&](int j) -> uint64_t {
        if (j >= nm) return 0ull;
        const int i = sh.mem[j];
        return ((uint64_t)sh.s.ckey[i] << 32) | (uint32_t)~sh.s.cblk[i];
    };
    constexpr int KW = 64 / NW;
    for (int i0 = 0; i0 < nm; i0 += 64) {
        const uint64_t ci = order_key(i0 + lane);
        int part = 0;
        for (int j0 = 0; j0 < nm; j0 += 64) {
            const uint64_t cj = order_key(j0 + lane);
            const uint32_t jh = (uint32_t)(cj >> 32), jl = (uint32_t)cj;
            const int k_end = min(min(64, nm - j0), KW * wid + KW);
            for (int k = KW * wid; k < k_end; ++k) {
                const uint64_t ck = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(jh, k) << 32) |
                                    (uint32_t)__builtin_amdgcn_readlane(jl, k);
                part += ck > ci;
            }
        }
        if (i0 + lane < nm) atomicAdd(&sh.rk[sh.mem[i0 + lane]], part);
    }
    __syncthreads();
    {
        constexpr int PER = kRbMax / NT;               // candidates a thread, consecutive
        auto taken = [&](int i) {
            const uint32_t bn = sh.s.ckey[i] >> 20;
            return i < nc && (bn > B1 || (bn == B1 && sh.rk[i] < need));
        };
        int cnt = 0;
#pragma unroll
        for (int k = 0; k < PER; ++k) cnt += taken(PER * tid + k);
        int tot;
        int pos = block_excl_sum<NT>(cnt, sh.s.tmp, &tot);
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int i = PER * tid + k;
            if (taken(i)) out.put(g.sink + pos++, sh.s.cblk[i]);
        }
    }
    emit_forced<NT>(g, r, topk, out);
}

template <int HD, int G>
static void launch_pf_approx(const Geo &g, dim3 grid, const qwfn_kv_view &v, const float *q, int32_t n_q,
                             int32_t n_blk, float *scores, int32_t nb_cap, float *pnorm, hipStream_t st) {
    if (g.relu)
        hipLaunchKernelGGL((k_pf_approx<HD, G, true>), grid, dim3(256), 0, st, g, v, q, n_q, n_blk, scores, nb_cap,
                           pnorm);
    else
        hipLaunchKernelGGL((k_pf_approx<HD, G, false>), grid, dim3(256), 0, st, g, v, q, n_q, n_blk, scores, nb_cap,
                           pnorm);
}

template <int HD, int G>
static void launch_pf_index_t(const Geo &g, const qwfn_kv_view &v, const float *q, int32_t n_q,
                              int32_t max_seq_len, int32_t *sel, int32_t *nsel, int32_t max_sel,
                              const Ws &ws, hipStream_t st) {
    const int32_t n_blk = max_seq_len / g.bt;                   // whole blocks of the longest query
    if constexpr (pf_approx_fits<HD, G>()) {
        // one score row (a single KV head, or one shared by every KV head) of up
        // to kRbBlocks eligible blocks: the 1024-thread refinement
        if (g.Hkv == 1 && g.topk > 0 && n_blk > g.sink && n_blk - g.sink > kRefineBlocks &&
            n_blk - g.sink <= kRbBlocks) {
            launch_pf_approx<HD, G>(g, dim3((unsigned)((n_q + kPaQ - 1) / kPaQ), (unsigned)kPaSplitBig, 1u), v, q, n_q,
                                    n_blk, ws.scores, ws.nb_cap, ws.pnorm, st);
            hipLaunchKernelGGL((k_pf_refine_big<HD, G>), dim3(1u, (unsigned)n_q), dim3(kRbThreads), 0, st, g, v, q,
                               ws.scores, ws.nb_cap, ws.pnorm, sel, nsel, max_sel);
            return;
        }
        // per-KV-head selections (or one KV head's row shared), up to kRefineBlocks eligible blocks
        if ((!g.shared || g.Hkv == 1) && g.topk > 0 && n_blk > g.sink && n_blk - g.sink <= kRefineBlocks) {
            launch_pf_approx<HD, G>(g, dim3((unsigned)((n_q + kPaQ - 1) / kPaQ), (unsigned)kPaSplit, (unsigned)g.Hkv),
                                    v, q, n_q, n_blk, ws.scores, ws.nb_cap, ws.pnorm, st);
            hipLaunchKernelGGL((k_pf_refine<HD, G>), dim3((unsigned)g.Hkv, (unsigned)n_q), dim3(kIdxThreads), 0, st, g,
                               v, q, ws.scores, ws.nb_cap, ws.pnorm, sel, nsel, max_sel);
            return;
        }
    }
    if (g.topk > 0 && n_blk > g.sink) {
        const dim3 grid((unsigned)((n_blk - g.sink + kPfB - 1) / kPfB), (unsigned)((n_q + kPfQ - 1) / kPfQ),
                        (unsigned)g.Hkv);
        hipLaunchKernelGGL((k_pf_scores<HD, G>), grid, dim3(256), 0, st, g, v, q, n_q, n_blk, ws.scores,
                           ws.nb_cap);
    }
    if (n_blk > kKeysMax)
        hipLaunchKernelGGL(k_select_big, dim3((unsigned)(g.shared ? 1 : g.Hkv), (unsigned)n_q),
                           dim3(kBigSelThreads), 0, st, g, v, nullptr, max_seq_len, ws.scores, ws.nb_cap, sel,
                           nsel, max_sel);
    else
        hipLaunchKernelGGL(k_pf_select, dim3((unsigned)(g.shared ? 1 : g.Hkv), (unsigned)n_q), dim3(kIdxThreads),
                           0, st, g, ws.scores, ws.nb_cap, sel, nsel, max_sel);
}

// ---------------------------------------------------------------------------
// dispatch over the instantiated (head_dim, group) pairs
// ---------------------------------------------------------------------------

// (head_dim, group, tile groups per general attention workgroup).  One group:
// the partials go to k_merge, so more groups per workgroup only add an LDS
// merge, and a smaller workgroup lets two or more share a CU's LDS (measured:
// checkpoint layer 49.6 -> 45.8 us, q4_0 / F16 layers 32.5 -> 30 us, checkpoint
// prefill chunk of 2048 queries 6.13 -> 5.25 ms, against 2-3 groups).
#define QWFN_FOR_EACH_SHAPE(X) X(128, 8, 1) X(128, 4, 1) X(128, 2, 1) X(64, 8, 1) X(256, 12, 1) X(256, 8, 1)

bool kernels_for(int32_t hd, int32_t G) {
#define X(HD_, G_, TG_) if (hd == HD_ && G == G_) return true;
    QWFN_FOR_EACH_SHAPE(X)
#undef X
    return false;
}

template <int KT>
static hipError_t launch_pool_t(const Geo &g, const qwfn_kv_view &v, const int32_t *seq_ids,
                                const int32_t *block_ids, int32_t n_blocks, int32_t seq_const, int32_t blk0,
                                hipStream_t st, const int32_t *len) {
    const dim3 grid((unsigned)n_blocks, (unsigned)g.Hkv);
    switch (g.hd) {
    case 64:  hipLaunchKernelGGL((k_pool<64, KT>), grid, dim3(256), 0, st, g, v, seq_ids, block_ids, seq_const, blk0, len); break;
    case 128: hipLaunchKernelGGL((k_pool<128, KT>), grid, dim3(256), 0, st, g, v, seq_ids, block_ids, seq_const, blk0, len); break;
    case 256: hipLaunchKernelGGL((k_pool<256, KT>), grid, dim3(256), 0, st, g, v, seq_ids, block_ids, seq_const, blk0, len); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_pool(const Geo &g, const qwfn_kv_view &v, const int32_t *seq_ids,
                       const int32_t *block_ids, int32_t n_blocks, int32_t seq_const,
                       int32_t blk0, hipStream_t st, const int32_t *len) {
    switch (g.kt) {
    case QWFN_KV_Q4_0: return launch_pool_t<QWFN_KV_Q4_0>(g, v, seq_ids, block_ids, n_blocks, seq_const, blk0, st, len);
    case QWFN_KV_F16:  return launch_pool_t<QWFN_KV_F16>(g, v, seq_ids, block_ids, n_blocks, seq_const, blk0, st, len);
    default:           return launch_pool_t<QWFN_KV_Q8_0>(g, v, seq_ids, block_ids, n_blocks, seq_const, blk0, st, len);
    }
}

hipError_t launch_indexer(const Geo &g, const qwfn_kv_view &v, const float *q,
                          const int32_t *seq_len, int32_t n_seq, int32_t max_seq_len,
                          int32_t *sel, int32_t *nsel, int32_t max_sel, const Ws &ws,
                          const FusedAppend &fa, hipStream_t st, bool select, bool sel_launch,
                          const IdxAppend *ia, bool in_cut) {
#define X(HD_, G_, TG_)                                                                          \
    if (g.hd == HD_ && g.G == G_)                                                                \
        return launch_indexer_t<HD_, G_>(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel, ws, fa, st, select, \
                                         sel_launch, ia, in_cut);
    QWFN_FOR_EACH_SHAPE(X)
#undef X
    return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// prefill attention on the matrix cores: one wave per (query, KV head)
// ---------------------------------------------------------------------------

// Order LDS traffic between the lanes of one wave: a wave's LDS operations
// execute in order, so only the compiler has to be kept from reordering (no
// wait is emitted; in-flight global loads stay in flight).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}


// grid (kVmaxWg, Hkv), 256 threads: partial maxima of KV head gh's q8_0 V
// scales over positions [0, n_pos) of sequence pf_seq, each a 64-cell tile's
// scale row read as 16-byte chunks (cell c's NJ scales are halfs c*NJ ..
// c*NJ+NJ-1 of the row); cells at or past n_pos and unmapped pages are left
// out.  vmax[gh * kVmaxWg + blockIdx.x] gets the workgroup's maximum.
template <int HD>
__global__ void __launch_bounds__(256)
k_pf_vmax(Geo g, qwfn_kv_view v, int32_t n_pos, float *__restrict__ vmax) {
    constexpr int NJ = HD / 32, CPT = 64 * NJ * 2 / 16;    // 16-byte chunks per tile scale row
    __shared__ float red[4];
    const int gh = blockIdx.y;
    const int n_chunks = (n_pos + 63) / 64 * CPT;
    float mx = 0.0f;
    for (int i = (int)blockIdx.x * 256 + (int)threadIdx.x; i < n_chunks; i += kVmaxWg * 256) {
        const int t0 = i / CPT * 64, c = i % CPT;
        const int32_t pg = phys_page(g, v.page_table, g.pf_seq, t0);
        if (pg < 0) continue;
        const uint8_t *vp = (const uint8_t *)v.v_pages + (int64_t)pg * g.page_bytes;
        const u4v w = *reinterpret_cast<const u4v *>(vp + scale_off(g, gh, t0 % g.pt, 0) + 16 * c);
        const h8v x = __builtin_bit_cast(h8v, w);
#pragma unroll
        for (int e = 0; e < 8; ++e)
            if (t0 + (8 * c + e) / NJ < n_pos) mx = fmaxf(mx, fabsf((float)x[e]));
    }
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    if (threadIdx.x == 0)
        vmax[gh * kVmaxWg + blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

hipError_t launch_prefill_vmax(const Geo &g, const qwfn_kv_view &v, int32_t n_pos, float *vmax, hipStream_t st) {
    const dim3 grid((unsigned)kVmaxWg, (unsigned)g.Hkv);
    switch (g.hd) {
    case 64:  hipLaunchKernelGGL((k_pf_vmax<64>), grid, dim3(256), 0, st, g, v, n_pos, vmax); break;
    case 128: hipLaunchKernelGGL((k_pf_vmax<128>), grid, dim3(256), 0, st, g, v, n_pos, vmax); break;
    case 256: hipLaunchKernelGGL((k_pf_vmax<256>), grid, dim3(256), 0, st, g, v, n_pos, vmax); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int HD, int G>
struct PfAttnCfg {
    static constexpr int NK4 = HD / 16;                   // 1 KB transfers per K (or V) tile
    static constexpr int NS4 = HD / 4;                    // 16-byte chunks of one tile's scale rows
    static constexpr int SCI = (2 * NS4 + 63) / 64;       // 1 KB transfers for both scale rows
    static constexpr int KOFF = 0, VOFF = HD * 64, SOFF = 2 * HD * 64;   // byte offsets in a buffer
    static constexpr int BUF16 = (2 * HD * 64 + 64 * SCI * 16) / 16;      // 16-byte chunks per buffer
    static constexpr int PER_WAVE = BUF16 * 16 + G * (64 + 4) * 4;        // LDS bytes per wave
    static constexpr int WAVES = 160 * 1024 / PER_WAVE >= 8 ? 8 : 160 * 1024 / PER_WAVE;   // per CU
};

// A wave's LDS: the tile buffer (K tile as in memory; V tile with each 64-byte
// dim row's four 16-byte quarters rotated by (dim / 4) % 4, so the PV operand
// reads of 16 dims are bank-conflict free; the K then V scale rows) and the
// softmax weights of the group's heads.
template <int HD, int G>
struct PfAttnLds {
    u4v buf[PfAttnCfg<HD, G>::BUF16];
    float p[G][64 + 4];
};

// grid ceil(n_q * Hkv / WAVES), WAVES waves; wave w owns (query s, KV head gh)
// = pair blockIdx.x*WAVES + w and walks its selected 64-cell tiles with an
// online softmax.  A tile's K, V and scale bytes (17 KB at hd 128) reach the
// wave's LDS buffer by coalesced 16-byte global -> LDS transfers that hold no
// registers; the next tile's transfer goes out as soon as the current tile's
// operands are in registers, and the other wave of the SIMD (two per SIMD:
// 19.6 KB of LDS per wave at hd 128) computes meanwhile.  Every contraction
// runs on
// v_mfma_f32_16x16x32_f16 (one output column per query head, up to 16):
//  - QK: S[cell][head] = sum_j dk(cell, j) * (K_j[cell][:] . q_j[:, head]) per
//    32-dim q8_0 block j, the int8 keys exact in fp16 and the query row (scaled
//    by a power of two qs) as fp16 hi + lo, so the products are exact and
//    only the fp32 accumulation rounds;
//  - PV: O[dim][head] += V[dim][cell] * P'_j[cell][head] with the V quants
//    exact in fp16 and P'_j = p * dv(cell, j) * 2^k split into fp16 hi + lo
//    (2^k, one per KV head and call, brings the head's largest V scale near
//    2^15, so P' stays finite in fp16 and its low half normal; the softmax
//    weights are formed as exp2(s * scale - m + k), and O and the weight sum
//    carry the same 2^k).
// Cells past the query's position have weight 0 and their V scale masked.
// K and V tiles are addressed from a wave-uniform base plus a fixed per-lane
// offset (no per-lane 64-bit address arithmetic per tile).
template <int HD, int G>
__global__ void __launch_bounds__((PfAttnCfg<HD, G>::WAVES * 64))
k_pf_attn(Geo g, qwfn_kv_view v, const float *__restrict__ q, int32_t n_q, const int32_t *__restrict__ sel,
          const int32_t *__restrict__ nsel, int32_t max_sel, const float *__restrict__ vmax,
          float *__restrict__ out) {
    using C = PfAttnCfg<HD, G>;
    constexpr int NJ = HD / 32, ND = HD / 16, NK4 = C::NK4, NS4 = C::NS4;
    static_assert(G <= 16, "one MFMA output column per query head");
    __shared__ PfAttnLds<HD, G> shw[C::WAVES];
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63;
    const int pair = (int)blockIdx.x * C::WAVES + wv;
    if (pair >= n_q * g.Hkv) return;                 // a whole wave; no workgroup barrier follows
    PfAttnLds<HD, G> &W = shw[wv];
    const int s = pair / g.Hkv, gh = pair - s * g.Hkv;
    const int L = g.pf_pos0 + s + 1;
    const int hn = l & 15, lg = l >> 4;              // MFMA column (head) and k-group of this lane
    const bool hv = hn < G;
    const int n = min(nsel[pair], max_sel);
    const int tpb = g.bt / 64;
    const int32_t *selp = sel + (int64_t)pair * max_sel;
    // PAIR (8 heads, head_dim >= 128): QK's 16 columns hold every head twice,
    // columns h + 8 jp taking q8_0 blocks jj + jp NJ/2 -- so a lane's key
    // scales are one half of a scale word -- and each lane keeps two of the
    // four rows of an MFMA tile after the halves are added; the softmax then
    // runs on 8 values a lane, not 16.  Else column hn is head hn (or zero).
    constexpr bool PAIR = G == 8 && NJ % 4 == 0;
    // SPLITCOL (with PAIR): PV's 16 columns carry the weights' fp16 high
    // halves in columns h and their low halves in columns h + 8, so one MFMA
    // takes both (the column halves share the head's softmax state), and the
    // two columns are added at the end
    constexpr bool SPLITCOL = PAIR;
    constexpr int NQ = PAIR ? NJ / 2 : NJ;           // query blocks a lane holds
    constexpr int R = PAIR ? 2 : 4;                  // rows of each 16-cell tile a lane keeps
    const int jp = PAIR ? hn >> 3 : 0;
    // query head hn (PAIR: hn mod 8), dims 32 j + 8 lg .. +8 of its blocks, as fp16 hi + lo of q / qs
    const float *qrow = q + ((int64_t)s * g.H + gh * G + (PAIR ? (hn & 7) : (hv ? hn : 0))) * HD;
    h8v qh[NQ], ql[NQ];
    float qs;
    {
        float x[NQ][8];
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < NQ; ++j) {
            const int blk = PAIR ? j + jp * (NJ / 2) : j;
            const float4 x0 = *reinterpret_cast<const float4 *>(qrow + 32 * blk + 8 * lg);
            const float4 x1 = *reinterpret_cast<const float4 *>(qrow + 32 * blk + 8 * lg + 4);
            x[j][0] = x0.x; x[j][1] = x0.y; x[j][2] = x0.z; x[j][3] = x0.w;
            x[j][4] = x1.x; x[j][5] = x1.y; x[j][6] = x1.z; x[j][7] = x1.w;
#pragma unroll
            for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(x[j][i]));
        }
        amax = fmaxf(amax, __shfl_xor(amax, 16));
        amax = fmaxf(amax, __shfl_xor(amax, 32));
        if constexpr (PAIR) amax = fmaxf(amax, dppf<kDppRowRor8>(0.0f, amax));
        int ex = 0;
        frexpf(amax, &ex);
        qs = amax > 0.0f ? ldexpf(1.0f, ex - 14) : 1.0f;   // |q / qs| < 2^14
        const float qinv = 1.0f / qs;                        // a power of two: exact
#pragma unroll
        for (int j = 0; j < NQ; ++j)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float y = PAIR || hv ? x[j][i] * qinv : 0.0f;
                const _Float16 hi = (_Float16)y;
                qh[j][i] = hi;
                ql[j][i] = (_Float16)(y - (float)hi);
            }
    }
    // PAIR: the B operands of the two column halves (the other half zero)
    h8v qb[PAIR ? 2 : 1][NQ][2];
    if constexpr (PAIR) {
        const h8v z = {};
#pragma unroll
        for (int j = 0; j < NQ; ++j) {
            qb[0][j][0] = jp == 0 ? qh[j] : z;
            qb[0][j][1] = jp == 0 ? ql[j] : z;
            qb[1][j][0] = jp == 1 ? qh[j] : z;
            qb[1][j][1] = jp == 1 ? ql[j] : z;
        }
    }
    const float lscale = qs * g.scale_log2;          // > 0
    // the weights enter PV scaled by 2^kup, which brings the KV head's largest
    // V scale (k_pf_vmax, over every row the call's queries read) near 2^15:
    // p * dv * 2^kup stays below the fp16 maximum and its low half normal
    float kup;
    {
        float dvm = vmax[gh * kVmaxWg + l % kVmaxWg];
        dvm = wave_max(dvm);
        int e2 = 0;
        frexpf(dvm, &e2);
        kup = dvm > 0.0f ? (float)(15 - e2) : 0.0f;
    }
    f4v o[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d) o[d] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
    // running max starts at a finite floor far below any score, so exp2 of
    // (score - max) never sees inf - inf
    float m = -1e30f, lsum = 0.0f;                   // lsum in units of 2^kup
    const int n_tiles = n * tpb;
    // lane l's 16 bytes of a V tile's 1 KB transfer: dim row l / 4, quarter
    // (l % 4) ^ (row / 4 % 4)
    const uint32_t v_lane = (uint32_t)((l >> 2) * 64 + (((l & 3) ^ ((l >> 4) & 3)) << 4));
    for (int tc = 0; tc < n_tiles; tc += 64) {
        // lane l describes tile tc + l: page, first row, cells at or before the
        // query -- looked up for 64 tiles at once, read back per tile by readlane
        int pg_l = 0, r0_l = 0, nv_l = 0;
        {
            const int t = tc + l;
            if (t < n_tiles) {
                const int blk = selp[t / tpb];
                const int64_t t0 = (int64_t)blk * g.bt + (t % tpb) * 64;
                if (blk >= 0 && t0 < L) {
                    const int32_t pg = phys_page(g, v.page_table, g.pf_seq, (int)t0);
                    if (pg >= 0) {
                        pg_l = pg;
                        r0_l = (int)(t0 % g.pt);
                        nv_l = (int)min((int64_t)64, (int64_t)L - t0);
                    } else {
                        set_status(v.status, QWFN_STATUS_PAGE_RANGE);
                    }
                }
            }
        }
        const int t_end = min(n_tiles - tc, 64);
        // tile ti -> the buffer, in two parts: the K chunks (as in memory) with
        // both scale rows, read by QK; the V chunks (rotated), read by PV
        const uint32_t base = __builtin_amdgcn_readfirstlane(
            (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)&W.buf[0]);
        auto tile_src = [&](int ti, const uint8_t *&kp, const uint8_t *&vp, int &tl, int &row0) {
            const int pg = __builtin_amdgcn_readlane(pg_l, ti);
            row0 = __builtin_amdgcn_readlane(r0_l, ti);
            kp = (const uint8_t *)v.k_pages + (int64_t)pg * g.page_bytes;
            vp = (const uint8_t *)v.v_pages + (int64_t)pg * g.page_bytes;
            tl = gh * (g.pt / 64) + row0 / 64;
        };
        auto issue_k = [&](int ti) {
            const uint8_t *kp, *vp;
            int tl, row0;
            tile_src(ti, kp, vp, tl, row0);
            const uint8_t *ksrc = kp + (int64_t)tl * (HD / 16) * 1024;
#pragma unroll
            for (int i = 0; i < NK4; ++i) lds_dma16_sv(ksrc + i * 1024, 16 * l, base + C::KOFF + i * 1024);
            const uint8_t *kss = kp + scale_off(g, gh, row0, 0);
            const uint8_t *vss = vp + scale_off(g, gh, row0, 0);
#pragma unroll
            for (int c = 0; c < C::SCI; ++c) {
                const int r = 64 * c + l;
                if (r < 2 * NS4) lds_dma16(r < NS4 ? kss + 16 * r : vss + 16 * (r - NS4), base + C::SOFF + c * 1024);
            }
        };
        auto issue_v = [&](int ti) {
            const uint8_t *kp, *vp;
            int tl, row0;
            tile_src(ti, kp, vp, tl, row0);
            const uint8_t *vsrc = vp + (int64_t)tl * HD * 64;
#pragma unroll
            for (int i = 0; i < NK4; ++i) lds_dma16_sv(vsrc + i * 1024, v_lane, base + C::VOFF + i * 1024);
        };
        issue_k(0);
        issue_v(0);
        for (int ti = 0; ti < t_end; ++ti) {
            const int nv = __builtin_amdgcn_readlane(nv_l, ti);
            wait_vmem_all();                         // tile ti has landed in the buffer
            // PV operands, read out of LDS before the next tile's transfer
            uint2 vwr[2][NJ][2];
            float pcr[2][8];
            u4v dvw_pv[2][NJ];
            if (nv > 0) {                            // uniform over the wave
                const uint8_t *wk = reinterpret_cast<const uint8_t *>(&W.buf[0]) + C::KOFF;
                const uint8_t *wvb = reinterpret_cast<const uint8_t *>(&W.buf[0]) + C::VOFF;
                // cell c's NJ fp16 scales: halfs c*NJ .. c*NJ+NJ of the K (V) scale row
                const u4v *wks = reinterpret_cast<const u4v *>(reinterpret_cast<const uint8_t *>(&W.buf[0]) + C::SOFF);
                const u4v *wvs = wks + NS4;
                // ---- QK: sv[mb][r] is cell 16 mb + 4 lg + (PAIR ? 2 jp : 0) + r
                float sv[4][R];
                auto cell_of = [&](int mb, int r) { return 16 * mb + 4 * lg + (PAIR ? 2 * jp : 0) + r; };
#pragma unroll
                for (int mb = 0; mb < 4; ++mb) {
                    if constexpr (PAIR) {
                        // the lane's blocks jj + jp NJ/2 of its cells 16mb+4lg+i: halves
                        // jj % 2 of the scale words (cell) NJ/2 + jp NJ/4 + jj/2
                        const uint32_t *wkw = reinterpret_cast<const uint32_t *>(wks);
                        uint32_t dkw[4][NJ / 4];
#pragma unroll
                        for (int i = 0; i < 4; ++i)
#pragma unroll
                            for (int w = 0; w < NJ / 4; ++w)
                                dkw[i][w] = wkw[(16 * mb + 4 * lg + i) * (NJ / 2) + jp * (NJ / 4) + w];
                        f4v c[NQ];
#pragma unroll
                        for (int jj = 0; jj < NQ; ++jj) {
                            c[jj] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                            for (int side = 0; side < 2; ++side) {
                                const int j = jj + side * (NJ / 2);
                                const uint2 kw = *reinterpret_cast<const uint2 *>(
                                    wk + ((2 * j + (lg >> 1)) * 64 + 16 * mb + hn) * 16 + 8 * (lg & 1));
                                const h8v kh = q8x8_to_h8(kw);
                                c[jj] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qb[side][jj][0], c[jj], 0, 0, 0);
                                c[jj] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qb[side][jj][1], c[jj], 0, 0, 0);
                            }
                        }
                        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                        for (int jj = 0; jj < NQ; ++jj)
#pragma unroll
                            for (int i = 0; i < 4; ++i)
                                acc[i] = __builtin_fmaf(
                                    (float)__builtin_bit_cast(half2v, dkw[i][jj / 2])[jj % 2], c[jj][i], acc[i]);
                        // add the column halves: lane jp keeps rows 2 jp, 2 jp + 1
                        const float k0 = jp ? acc[2] : acc[0], k1 = jp ? acc[3] : acc[1];
                        const float s0 = jp ? acc[0] : acc[2], s1 = jp ? acc[1] : acc[3];
                        sv[mb][0] = k0 + dppf<kDppRowRor8>(0.0f, s0);
                        sv[mb][1] = k1 + dppf<kDppRowRor8>(0.0f, s1);
                        continue;
                    }
                    h8v dk[NJ / 2];                  // cells 16mb+4lg .. +4, every block
#pragma unroll
                    for (int w = 0; w < NJ / 2; ++w)
                        dk[w] = __builtin_bit_cast(h8v, wks[(16 * mb + 4 * lg) * NJ / 8 + w]);
                    f4v c[NJ];                       // block j's dot products, independent chains
#pragma unroll
                    for (int j = 0; j < NJ; ++j) {
                        const uint2 kw = *reinterpret_cast<const uint2 *>(
                            wk + ((2 * j + (lg >> 1)) * 64 + 16 * mb + hn) * 16 + 8 * (lg & 1));
                        const h8v kh = q8x8_to_h8(kw);
                        c[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[j % NQ], f4v{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                        c[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[j % NQ], c[j], 0, 0, 0);
                    }
                    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            acc[i] = __builtin_fmaf((float)dk[(i * NJ + j) / 8][(i * NJ + j) % 8], c[j][i], acc[i]);
#pragma unroll
                    for (int i = 0; i < R; ++i) sv[mb][i] = acc[i];   // log2 units after * lscale
                }
                // V scales of this lane's PV cells 32ks+8lg .. +8, every block (NJ words per ks)
                u4v dvw[2][NJ];
#pragma unroll
                for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                    for (int w = 0; w < NJ; ++w) dvw[ks][w] = wvs[(32 * ks + 8 * lg) * NJ / 8 + w];
                // the K chunks and scale rows are consumed: the next tile's may land
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                if (ti + 1 < t_end) issue_k(ti + 1);
                if (nv < 64) {                       // a partial tile: cells past the query carry no data
#pragma unroll
                    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
                        for (int i = 0; i < R; ++i)
                            if (cell_of(mb, i) >= nv) sv[mb][i] = -INFINITY;
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                        for (int w = 0; w < NJ; ++w)
#pragma unroll
                            for (int e = 0; e < 4; ++e)  // a dword holds two blocks of one cell (NJ even)
                                if (32 * ks + 8 * lg + (8 * w + 2 * e) / NJ >= nv) dvw[ks][w][e] = 0u;
                }
                // ---- online softmax (head hn; the four lanes of a column reduce by xor 16, 32,
                // PAIR also with the other column half by xor 8).  Columns past the
                // group's heads see q = 0: their weights are finite and unused.
                float tm = -INFINITY;
#pragma unroll
                for (int mb = 0; mb < 4; ++mb)
#pragma unroll
                    for (int i = 0; i < R; ++i) tm = fmaxf(tm, sv[mb][i]);
                tm = col_max4(tm);
                if constexpr (PAIR) tm = fmaxf(tm, dppf<kDppRowRor8>(0.0f, tm));
                tm *= lscale;                        // lscale > 0: the max commutes
                const float m_new = fmaxf(m, tm);
                const float alpha = __builtin_amdgcn_exp2f(m - m_new);
                const float bias = kup - m_new;
                float tsum = 0.0f;
#pragma unroll
                for (int mb = 0; mb < 4; ++mb) {
                    float pr[R];
#pragma unroll
                    for (int i = 0; i < R; ++i) {
                        pr[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[mb][i], lscale, bias));
                        tsum += pr[i];
                    }
                    if constexpr (PAIR) {
                        *reinterpret_cast<float2 *>(&W.p[hn & 7][cell_of(mb, 0)]) = make_float2(pr[0], pr[1]);
                    } else if (hv) {
#pragma unroll
                        for (int i = 0; i < R; ++i) W.p[hn][cell_of(mb, i)] = pr[i];
                    }
                }
                tsum = col_sum4(tsum);
                if constexpr (PAIR) tsum += dppf<kDppRowRor8>(0.0f, tsum);
                lsum = lsum * alpha + tsum;
                m = m_new;
                if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
                    for (int d = 0; d < ND; ++d) o[d] *= alpha;
                }
                wave_lds_sync();
                // ---- PV operands: the weights of head hn and the V quants this lane feeds
                {
                    const int hq = SPLITCOL ? (hn & 7) : min(hn, G - 1);
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) {
                        const float4 p0 = *reinterpret_cast<const float4 *>(&W.p[hq][32 * ks + 8 * lg]);
                        const float4 p1 = *reinterpret_cast<const float4 *>(&W.p[hq][32 * ks + 8 * lg + 4]);
                        const float pc[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
                        for (int i = 0; i < 8; ++i) pcr[ks][i] = SPLITCOL || hv ? pc[i] : 0.0f;
#pragma unroll
                        for (int j = 0; j < NJ; ++j)
#pragma unroll
                            for (int db = 0; db < 2; ++db)
                                vwr[ks][j][db] = *reinterpret_cast<const uint2 *>(
                                    wvb + (16 * (2 * j + db) + hn) * 64 + (((2 * ks + (lg >> 1)) ^ (hn >> 2)) << 4) +
                                    8 * (lg & 1));
                    }
                }
#pragma unroll
                for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                    for (int w = 0; w < NJ; ++w) dvw_pv[ks][w] = dvw[ks][w];
            }
            // every LDS read of the tile has returned: the next tile's V may land
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (ti + 1 < t_end) {
                if (nv <= 0) issue_k(ti + 1);        // (a skipped tile issued no K part above)
                issue_v(ti + 1);
            }
            if (nv > 0) {
                // ---- PV
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
                    for (int j = 0; j < NJ; ++j) {
                        // cell i's block-j scale: half i * NJ + j of the cells' scale row,
                        // the low or high half of its word as j is even or odd
                        u4v bhw, blw;
#pragma unroll
                        for (int m = 0; m < 4; ++m) {
                            const int e0 = 2 * m * NJ + j, e1 = e0 + NJ;
                            const uint32_t d0 = dvw_pv[ks][e0 / 8][e0 % 8 / 2], d1 = dvw_pv[ks][e1 / 8][e1 % 8 / 2];
                            uint32_t hw, lw;
                            if (j % 2 == 0) p_split2<0>(pcr[ks][2 * m], d0, pcr[ks][2 * m + 1], d1, hw, lw);
                            else p_split2<1>(pcr[ks][2 * m], d0, pcr[ks][2 * m + 1], d1, hw, lw);
                            bhw[m] = hw;
                            blw[m] = lw;
                        }
                        const h8v bh = __builtin_bit_cast(h8v, bhw), bl = __builtin_bit_cast(h8v, blw);
                        const h8v bs = hn >= 8 ? bl : bh;   // SPLITCOL: this lane's column half
#pragma unroll
                        for (int db = 0; db < 2; ++db) {
                            const int dblk = 2 * j + db;
                            const h8v vh = q8x8_to_h8(vwr[ks][j][db]);
                            if constexpr (SPLITCOL) {
                                o[dblk] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, bs, o[dblk], 0, 0, 0);
                            } else {
                                o[dblk] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, bh, o[dblk], 0, 0, 0);
                                o[dblk] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, bl, o[dblk], 0, 0, 0);
                            }
                        }
                    }
                }
            }
            wave_lds_sync();                         // the weight strip is rewritten next
        }
    }
    if constexpr (SPLITCOL) {                        // column h += column h + 8 (the low halves' sums)
#pragma unroll
        for (int d = 0; d < ND; ++d)
#pragma unroll
            for (int i = 0; i < 4; ++i) o[d][i] += dppf<kDppRowRor8>(0.0f, o[d][i]);
    }
    if (hv) {
        const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
        float *orow = out + ((int64_t)s * g.H + gh * G + hn) * HD;
#pragma unroll
        for (int d = 0; d < ND; ++d)
            *reinterpret_cast<float4 *>(orow + 16 * d + 4 * lg) =
                make_float4(o[d][0] * inv, o[d][1] * inv, o[d][2] * inv, o[d][3] * inv);
    }
}

template <int HD, int G>
static void launch_pf_attn_t(const Geo &g, const qwfn_kv_view &v, const float *q, int32_t n_q,
                             const int32_t *sel, const int32_t *nsel, int32_t max_sel, const float *vmax,
                             float *out, hipStream_t st) {
    constexpr int WAVES = PfAttnCfg<HD, G>::WAVES;
    const int pairs = n_q * g.Hkv;
    hipLaunchKernelGGL((k_pf_attn<HD, G>), dim3((unsigned)((pairs + WAVES - 1) / WAVES)), dim3(WAVES * 64), 0, st, g,
                       v, q, n_q, sel, nsel, max_sel, vmax, out);
}

hipError_t launch_prefill_attention(const Geo &g, const qwfn_kv_view &v, const float *q, int32_t n_q,
                                    const int32_t *sel, const int32_t *nsel, int32_t max_sel, const float *vmax,
                                    float *out, hipStream_t st) {
#define X(HD_, G_, TG_)                                                                          \
    if (g.hd == HD_ && g.G == G_) {                                                              \
        launch_pf_attn_t<HD_, G_>(g, v, q, n_q, sel, nsel, max_sel, vmax, out, st);             \
        return hipGetLastError();                                                                \
    }
    QWFN_FOR_EACH_SHAPE(X)
#undef X
    return hipErrorInvalidValue;
}

hipError_t launch_prefill_index(const Geo &g, const qwfn_kv_view &v, const float *q, int32_t n_q,
                                int32_t max_seq_len, int32_t *sel, int32_t *nsel, int32_t max_sel,
                                const Ws &ws, hipStream_t st) {
#define X(HD_, G_, TG_)                                                                              if (g.hd == HD_ && g.G == G_) {                                                                      launch_pf_index_t<HD_, G_>(g, v, q, n_q, max_seq_len, sel, nsel, max_sel, ws, st);              return hipGetLastError();                                                                    }
    QWFN_FOR_EACH_SHAPE(X)
#undef X
    return hipErrorInvalidValue;
}

bool pf_approx_fits_shape(int32_t hd, int32_t G) {
#define X(HD_, G_, TG_) if (hd == HD_ && G == G_) return pf_approx_fits<HD_, G_>();
    QWFN_FOR_EACH_SHAPE(X)
#undef X
    return false;
}

hipError_t launch_pf_approx_scores(const Geo &g, const qwfn_kv_view &v, const float *q, int32_t n_q,
                                   int32_t n_blk, float *scores, int32_t nb_cap, float *pnorm, hipStream_t st) {
#define X(HD_, G_, TG_)                                                                                   \
    if constexpr (pf_approx_fits<HD_, G_>())                                                              \
        if (g.hd == HD_ && g.G == G_) {                                                                   \
            launch_pf_approx<HD_, G_>(g, dim3((unsigned)((n_q + kPaQ - 1) / kPaQ), (unsigned)kPaSplit,      \
                                              (unsigned)g.Hkv),                                            \
                                      v, q, n_q, n_blk, scores, nb_cap, pnorm, st);                        \
            return hipGetLastError();                                                                     \
        }
    QWFN_FOR_EACH_SHAPE(X)
#undef X
    return hipErrorInvalidValue;
}

hipError_t launch_attention(const Geo &g, const qwfn_kv_view &v, const float *q,
                            const int32_t *seq_len, int32_t n_seq, int32_t max_seq_len,
                            const int32_t *sel, const int32_t *nsel, int32_t max_sel,
                            float *out, const Ws &ws, hipStream_t st) {
    if (dec_kernels_for(g))
        return launch_dec_attention(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel, out, ws, false, st);
#define X(HD_, G_, TG_)                                                                         \
    if (g.hd == HD_ && g.G == G_) {                                                             \
        launch_attn_t<HD_, G_, TG_>(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel, out, ws, st); \
        return hipGetLastError();                                                               \
    }
    QWFN_FOR_EACH_SHAPE(X)
#undef X
    return hipErrorInvalidValue;
}

// Up to this many sequences the attention's own selection pays (measured at 1
// and 8: 21.5 against 23.8 us per layer, and 36.3 against 42.4 us per step of
// eight); past it the chip fills and the redundant selections would compete.
constexpr int32_t kAttnSelSeqs = 8;

bool attn_select_fits(const Geo &g, int32_t n_seq, int32_t max_seq_len, int32_t max_sel) {
    if (g.shared || g.topk <= 0 || g.pf || n_seq > kAttnSelSeqs) return false;
    if (dec_kernels_for(g))
        return dec_select_fits(g, max_seq_len, max_sel);
    if (max_sel > kAttnSelMax || max_seq_len / g.bt > kKeysMax) return false;
#define X(HD_, G_, TG_) if (g.hd == HD_ && g.G == G_) return true;
    QWFN_FOR_EACH_SHAPE(X)
#undef X
    return false;
}

hipError_t launch_attention_select(const Geo &g, const qwfn_kv_view &v, const float *q, const int32_t *seq_len,
                                   int32_t n_seq, int32_t max_seq_len, int32_t *sel, int32_t *nsel,
                                   int32_t max_sel, float *out, const Ws &ws, hipStream_t st) {
    if (!attn_select_fits(g, n_seq, max_seq_len, max_sel)) return hipErrorInvalidValue;
    if (dec_kernels_for(g))
        return launch_dec_attention(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel, out, ws, true, st);
#define X(HD_, G_, TG_)                                                                                     \
    if (g.hd == HD_ && g.G == G_) {                                                                         \
        launch_attn_sel_t<HD_, G_, TG_>(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel, out, ws, st); \
        return hipGetLastError();                                                                           \
    }
    QWFN_FOR_EACH_SHAPE(X)
#undef X
    return hipErrorInvalidValue;
}

}  // namespace qwfn_qsa
