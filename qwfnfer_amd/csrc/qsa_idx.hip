// qsa_idx.hip -- gfx950 kernels of the checkpoint's own indexer keys
// (src/qwfn_graph.cpp:244-275, 410-448, 463-476): a raw fp16 key cache of
// idx_dim values per token, paged like K and V, and its pooled block keys --
// the mean of a block's block_tokens raw keys, RMSNorm * k_norm, then the
// rotary position of the block's first token -- rounded to fp16 as the
// reference's fp16 pool cache holds them (src/qwfn_engine.cpp:389-394).
//
// Everything here is bandwidth- or latency-trivial next to the attention (one
// block per decode step, a few MB for a rebuild), so the kernels favour an
// evaluation order the CPU oracle repeats exactly over speed.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include "qsa_append.h"
#include "qsa_device.h"
#include "qsa_select.h"
#include "qsa_idx_pool.h"

namespace qwfn_qsa {

bool idx_kernels_for(int32_t dim) { return dim == 64 || dim == 128 || dim == 256; }

// One thread per 8 values of one row.  seq_ids NULL: every row in seq_const;
// pos NULL: row r at position pos0 + r.
__global__ void __launch_bounds__(256)
k_idx_write(Geo g, qwfn_kv_view v, int32_t dim, uint16_t *raw, const void *src, int32_t f16,
            const int32_t *seq_ids, const int32_t *pos, int32_t n_rows, int32_t seq_const, int32_t pos0) {
    const int per = dim / 8;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)n_rows * per) return;
    const int r = (int)(i / per), c = (int)(i % per);
    const int seq = seq_ids ? seq_ids[r] : seq_const;
    const int t = pos ? pos[r] : pos0 + r;
    const bool report = c == 0;
    if (seq < 0 || seq >= g.n_seq_view) { if (report) set_status(v.status, QWFN_STATUS_SEQ_RANGE); return; }
    if (t < 0 || (int64_t)t >= (int64_t)g.pps * g.pt) { if (report) set_status(v.status, QWFN_STATUS_POS_RANGE); return; }
    const int32_t pp = phys_page(g, v.page_table, seq, t);
    if (pp < 0) { if (report) set_status(v.status, QWFN_STATUS_PAGE_RANGE); return; }
    uint4 out;
    if (f16) {
        out = reinterpret_cast<const uint4 *>((const uint16_t *)src + (int64_t)r * dim)[c];
    } else {
        const float4 *s4 = reinterpret_cast<const float4 *>((const float *)src + (int64_t)r * dim) + 2 * c;
        const float4 a = s4[0], b = s4[1];
        out.x = (uint32_t)f2h(a.x) | (uint32_t)f2h(a.y) << 16;
        out.y = (uint32_t)f2h(a.z) | (uint32_t)f2h(a.w) << 16;
        out.z = (uint32_t)f2h(b.x) | (uint32_t)f2h(b.y) << 16;
        out.w = (uint32_t)f2h(b.z) | (uint32_t)f2h(b.w) << 16;
    }
    reinterpret_cast<uint4 *>(raw + ((int64_t)pp * g.pt + t % g.pt) * dim)[c] = out;
}

hipError_t launch_idx_write(const Geo &g, const qwfn_kv_view &v, const IdxGeo &ig, uint16_t *raw,
                            const void *src, int32_t src_f16, const int32_t *seq_ids, const int32_t *pos,
                            int32_t n_rows, int32_t seq_const, int32_t pos0, hipStream_t st) {
    const int64_t total = (int64_t)n_rows * (ig.dim / 8);
    hipLaunchKernelGGL(k_idx_write, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, g, v, ig.dim, raw,
                       src, src_f16, seq_ids, pos, n_rows, seq_const, pos0);
    return hipGetLastError();
}


// The pooled key of one block from its bt members m[0 .. bt) (fp16 rows of D
// values, position order), by one wave; lane l owns dims l + 64k (k < D/64).
// ys is the wave's own D floats of LDS.
//   mean   : fp32 add chain over the members in position order, * (1/bt)
//            (ggml_add chain + ggml_scale, src/qwfn_graph.cpp:415-422); the
//            members' loads go out eight at a time before any is summed
//   RMSNorm: sum of the fp32 squares in fp64 -- per lane in k order, then a
//            butterfly over lane distance 32, 16, .., 1 --, mean = (float)
//            (sum / D), scale = 1 / sqrtf(mean + eps), x * scale * k_norm[d]
//            (ggml_rms_norm also sums in fp64; :423)
//   rotary : pair (i, i + nd/2) turned by (x0 c - x1 s, x0 s + x1 c), dims
//            >= nd unchanged, with ggml's IMROPE angle (:425-427): theta_0 =
//            (float)pos, theta_{i+1} = theta_i * theta_scale rounded to fp32,
//            theta_scale = powf(base, -2/nd) -- the running product ggml's
//            rope cache builds, one factor per pair --; cos / sin of that
//            fp32 angle evaluated in fp64 and rounded to fp32.  IMROPE gives
//            each pair the position of its section (t, h, w interleaved); the
//            reference fills every section of a block's position with the
//            block's first position b * bt (src/qwfn_engine.cpp:741-743, 926,
//            934), so every pair takes pos = b * bt.
//   store  : rounded to fp16 (the reference's F16 pool cache).
template <int D>
__device__ __forceinline__ void pool_idx_block(const Geo &g, const IdxGeo &ig, const uint16_t *m,
                                               const float *__restrict__ k_norm, float *ys, uint16_t *dst, int t0,
                                               int lane) {
    float cc[D / 64], sn[D / 64];
    idx_rot_cs<D>(ig, t0, lane, cc, sn);
    pool_idx_rows<D>(g, ig, [&](int r, int k) { return h2f(m[(int64_t)r * D + lane + 64 * k]); }, k_norm, ys, dst,
                     lane, cc, sn);
}

// One wave per block, four blocks a workgroup: the blocks of rows (seq_ids[i]
// or 0, pos[i] / bt) when pos != NULL (a run of rows in one block pools it
// once, at its last row), else blocks blk0 + [0, n_items) of sequence seq_const.
template <int D>
__global__ void __launch_bounds__(256)
k_idx_pool(Geo g, qwfn_kv_view v, IdxGeo ig, const uint16_t *__restrict__ raw, uint16_t *__restrict__ pooled,
           const float *__restrict__ k_norm, const int32_t *seq_ids, const int32_t *pos, int32_t n_items,
           int32_t seq_const, int32_t blk0) {
    __shared__ float ys[4][D];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int item = blockIdx.x * 4 + w;
    if (item >= n_items) return;                   // whole waves: no barrier below spans waves
    int seq, b;
    if (pos) {
        seq = seq_ids ? seq_ids[item] : 0;
        const int t = pos[item];
        if (seq < 0 || seq >= g.n_seq_view || t < 0 || (int64_t)t >= (int64_t)g.pps * g.pt) return;   // reported by the write
        b = t / g.bt;
        if (item + 1 < n_items) {                  // the run's last row pools its block
            const int s2 = seq_ids ? seq_ids[item + 1] : 0, t2 = pos[item + 1];
            if (s2 == seq && t2 >= 0 && t2 / g.bt == b) return;
        }
    } else {
        seq = seq_const;
        b = blk0 + item;
    }
    const int t0 = b * g.bt;
    const int32_t pp = phys_page(g, v.page_table, seq, t0);
    if (pp < 0) { if (lane == 0) set_status(v.status, QWFN_STATUS_PAGE_RANGE); return; }
    pool_idx_block<D>(g, ig, raw + ((int64_t)pp * g.pt + t0 % g.pt) * D, k_norm, ys[w],
                      pooled + ((int64_t)seq * g.bps + b) * D, t0, lane);
}

// A call of at most kIdxFuseRows rows (a decode step) in one workgroup: the
// rows are range-checked into LDS; each is written unless a later row has the
// same (sequence, position) -- the last one is kept --, and after a barrier
// the last row touching each block pools it from the cache, one wave a block.
constexpr int kIdxFuseThreads = 1024;
template <int D>
__global__ void __launch_bounds__(kIdxFuseThreads)
k_idx_append_pool(Geo g, qwfn_kv_view v, IdxGeo ig, uint16_t *__restrict__ raw, uint16_t *__restrict__ pooled,
                  const float *__restrict__ k_norm, const void *src, int32_t f16, const int32_t *seq_ids,
                  const int32_t *pos, int32_t n_rows) {
    constexpr int NW = kIdxFuseThreads / 64, PER = D / 8;
    __shared__ int32_t s_seq[kIdxFuseRows], s_pos[kIdxFuseRows], s_pp[kIdxFuseRows];
    __shared__ uint8_t s_write[kIdxFuseRows], s_pool[kIdxFuseRows];
    __shared__ float ys[NW][D];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    if (tid < n_rows) {
        const int seq = seq_ids ? seq_ids[tid] : 0, t = pos[tid];
        int32_t pp = -1;
        if (seq < 0 || seq >= g.n_seq_view) set_status(v.status, QWFN_STATUS_SEQ_RANGE);
        else if (t < 0 || (int64_t)t >= (int64_t)g.pps * g.pt) set_status(v.status, QWFN_STATUS_POS_RANGE);
        else if ((pp = phys_page(g, v.page_table, seq, t)) < 0) set_status(v.status, QWFN_STATUS_PAGE_RANGE);
        s_seq[tid] = pp >= 0 ? seq : -1;
        s_pos[tid] = pp >= 0 ? t : -1;
        s_pp[tid] = pp;
    }
    __syncthreads();
    if (tid < n_rows) {
        const int seq = s_seq[tid], t = s_pos[tid];
        bool wr = seq >= 0, pl = seq >= 0;
        for (int r2 = tid + 1; r2 < n_rows; ++r2) {
            if (seq >= 0 && s_seq[r2] == seq) {
                wr = wr && s_pos[r2] != t;
                pl = pl && s_pos[r2] / g.bt != t / g.bt;
            }
        }
        s_write[tid] = wr;
        s_pool[tid] = pl;
    }
    __syncthreads();
    for (int i = tid; i < n_rows * PER; i += kIdxFuseThreads) {
        const int r = i / PER, c = i % PER;
        if (!s_write[r]) continue;
        uint4 out;
        if (f16) {
            out = reinterpret_cast<const uint4 *>((const uint16_t *)src + (int64_t)r * D)[c];
        } else {
            const float4 *s4 = reinterpret_cast<const float4 *>((const float *)src + (int64_t)r * D) + 2 * c;
            const float4 a = s4[0], b = s4[1];
            out.x = (uint32_t)f2h(a.x) | (uint32_t)f2h(a.y) << 16;
            out.y = (uint32_t)f2h(a.z) | (uint32_t)f2h(a.w) << 16;
            out.z = (uint32_t)f2h(b.x) | (uint32_t)f2h(b.y) << 16;
            out.w = (uint32_t)f2h(b.z) | (uint32_t)f2h(b.w) << 16;
        }
        reinterpret_cast<uint4 *>(raw + ((int64_t)s_pp[r] * g.pt + s_pos[r] % g.pt) * D)[c] = out;
    }
    __syncthreads();                               // the rows' stores, for this workgroup's pooling
    for (int r = w; r < n_rows; r += NW) {
        if (!s_pool[r]) continue;                  // (uniform over the wave)
        const int seq = s_seq[r], b = s_pos[r] / g.bt, t0 = b * g.bt;
        const int32_t pp = phys_page(g, v.page_table, seq, t0);
        if (pp < 0) { if (lane == 0) set_status(v.status, QWFN_STATUS_PAGE_RANGE); continue; }
        pool_idx_block<D>(g, ig, raw + ((int64_t)pp * g.pt + t0 % g.pt) * D, k_norm, ys[w],
                          pooled + ((int64_t)seq * g.bps + b) * D, t0, lane);
    }
}

// Part p of sequence s's cut for the attention's own selection (one of the
// kIdxCutParts workgroups a sequence of the fused decode step's append
// launch): the eligible blocks e_lo + j * n_eligible / kIdxCutSamples, j = p
// kIdxCutPer .. + kIdxCutPer - 1, are scored from the pool cache (16 lanes a
// block, dims 64 i + 4 lane .. + 3 a lane, the query heads' dots relu'd when
// set and summed); wave 0 then finds the ceil(rs / kIdxCutParts)-th largest
// of their keys by a bitwise search (the largest key T with that many sample
// keys at or above it: one compare and ballot count a bit) into cutk[s][p].
// The indexer takes every eligible key at or above the mean of the parts'
// threshold keys as a candidate, and the attention ranks them exactly when they
// number at least topk (the selection is exact for any threshold; this one
// makes that the usual case), so the samples need not match the indexer's
// scores bit for bit.  The block this launch re-pools (the row's last) is
// never a sample.
constexpr int kIdxCutPer = kIdxCutSamples / kIdxCutParts;     // samples a workgroup
constexpr int kIdxCutLanes = kIdxFuseThreads / kIdxCutPer;    // lanes a sample
static_assert(kIdxCutLanes == 16 && kIdxCutPer == 64, "16 lanes a sample; a key a lane of wave 0");
struct IdxCutShared {
    float q[kIdxMaxCutHeads * 128];
    uint32_t key[kIdxCutPer];
};
template <int D>
__device__ __forceinline__ void idx_sample_cut(const Geo &g, const uint16_t *pooled, const int32_t *len,
                                               const IdxCut &ct, int s, int part, IdxCutShared &sh) {
    constexpr int NT = kIdxFuseThreads, NL = kIdxCutLanes;
    static_assert(D % (4 * NL) == 0, "whole 4-dim pieces a lane");
    const int tid = threadIdx.x, jl = tid % NL;
    const int L = len[s];
    int rs = 0;
    Ranges r{0, 0, 0, 0};
    if (L >= 1 && L <= ct.max_seq_len && s < g.n_seq_view) {
        r = qsa_ranges(g, L);
        const int topk = eff_topk(g, r);
        if (g.topk > 0 && r.e_hi - r.e_lo > topk) rs = sample_rank<kIdxCutSamples>(r, topk);
    }
    uint32_t tk = 0u;                              // no cut: every key a candidate
    if (rs > 0) {                                  // (uniform)
        const int nq = ct.n_head * D;
        const int j = part * kIdxCutPer + tid / NL;
        const uint16_t *P =
            pooled + ((int64_t)s * g.bps + r.e_lo + (int)((int64_t)j * (r.e_hi - r.e_lo) / kIdxCutSamples)) * D;
        uint2 pk[D / (4 * NL)];
#pragma unroll
        for (int i = 0; i < D / (4 * NL); ++i) pk[i] = *reinterpret_cast<const uint2 *>(P + 4 * NL * i + 4 * jl);
        for (int i = tid; i < nq; i += NT) sh.q[i] = ct.q_idx[(int64_t)s * nq + i];
        __syncthreads();
        float score = 0.0f;
        for (int h = 0; h < ct.n_head; ++h) {
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < D / (4 * NL); ++i) {
                const float4 q4 = *reinterpret_cast<const float4 *>(&sh.q[h * D + 4 * NL * i + 4 * jl]);
                acc = fmaf(q4.x, h2f((uint16_t)pk[i].x), acc);
                acc = fmaf(q4.y, h2f((uint16_t)(pk[i].x >> 16)), acc);
                acc = fmaf(q4.z, h2f((uint16_t)pk[i].y), acc);
                acc = fmaf(q4.w, h2f((uint16_t)(pk[i].y >> 16)), acc);
            }
            acc += __shfl_xor(acc, 1);
            acc += __shfl_xor(acc, 2);
            acc += __shfl_xor(acc, 4);
            acc += __shfl_xor(acc, 8);
            score += g.relu && !(acc > 0.0f) ? 0.0f : acc;
        }
        if (jl == 0) sh.key[tid / NL] = score_key(score);
        __syncthreads();
        if (tid < 64) {                            // wave 0: a sample key a lane
            const uint32_t k1 = sh.key[tid];
            const int need = (rs + kIdxCutParts - 1) / kIdxCutParts;
#pragma unroll 1
            for (int bit = 31; bit >= 0; --bit) {
                const uint32_t t = tk | (1u << bit);
                tk = __builtin_popcountll(__ballot(k1 >= t)) >= need ? t : tk;
            }
        }
    }
    if (tid == 0) ct.cutk[(int64_t)s * kIdxCutParts + part] = tk;
}

// The fused decode step's rows (at most kIdxFuseRows sequences, one row
// each): sequence r's raw key written at position len[r] - 1 and its block
// re-pooled by wave r mod 16, the block's other members read from the cache
// and the new row taken from registers, the rotation's cos / sin computed
// while the page-table load is in flight.  No barrier: each wave owns its
// sequences and its slice of LDS.  kv (when enabled): the rows' K and V
// appended as k_append does, lane i on thread i ^ 512.  Results equal
// k_idx_append_pool's on the same rows.
template <int D>
__global__ void __launch_bounds__(kIdxFuseThreads)
k_idx_decode_append(Geo g, qwfn_kv_view v, IdxGeo ig, uint16_t *__restrict__ raw, uint16_t *__restrict__ pooled,
                    const float *__restrict__ k_norm, const void *src, int32_t f16, const int32_t *len,
                    int32_t n_rows, FusedAppend kv, IdxCut ct) {
    constexpr int NW = kIdxFuseThreads / 64, K = D / 64;
    __shared__ union {
        float ys[NW][D];
        IdxCutShared cut;
    } shu;
    float (&ys)[NW][D] = shu.ys;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    if (blockIdx.x > 0) {                          // workgroup 1 + p + kIdxCutParts s: part p of sequence s's cut
        if constexpr (D <= 128)
            idx_sample_cut<D>(g, pooled, len, ct, (blockIdx.x - 1) / kIdxCutParts, (blockIdx.x - 1) % kIdxCutParts,
                              shu.cut);
        return;
    }
    if (kv.enabled) {
        const int64_t total = (int64_t)n_rows * 2 * g.Hkv * (g.hd / 32) * 8;
        for (int64_t i = tid ^ (kIdxFuseThreads / 2); i < total; i += kIdxFuseThreads)
            append_lane(g, v, kv.k_new, kv.v_new, kv.src_f16, i, [&](int r, int &seq, int &t) {
                seq = r;
                t = len[r] - 1;
            });
    }
    for (int s = w; s < n_rows; s += NW) {
        const int L = len[s];
        uint16_t nh[K];
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int64_t e = (int64_t)s * D + lane + 64 * k;
            nh[k] = f16 ? reinterpret_cast<const uint16_t *>(src)[e] : f2h(reinterpret_cast<const float *>(src)[e]);
        }
        const int t = L - 1;
        if (s >= g.n_seq_view) { if (lane == 0) set_status(v.status, QWFN_STATUS_SEQ_RANGE); continue; }
        if (t < 0 || (int64_t)t >= (int64_t)g.pps * g.pt) { if (lane == 0) set_status(v.status, QWFN_STATUS_POS_RANGE); continue; }
        const int32_t pp = phys_page(g, v.page_table, s, t);
        const int b = t / g.bt, t0 = b * g.bt, rn = t - t0;
        float cc[K], sn[K];
        idx_rot_cs<D>(ig, t0, lane, cc, sn);
        if (pp < 0) { if (lane == 0) set_status(v.status, QWFN_STATUS_PAGE_RANGE); continue; }
        uint16_t *row = raw + ((int64_t)pp * g.pt + t % g.pt) * D;
#pragma unroll
        for (int k = 0; k < K; ++k) row[lane + 64 * k] = nh[k];
        const uint16_t *m = raw + ((int64_t)pp * g.pt + t0 % g.pt) * D;   // a block never straddles pages
        pool_idx_rows<D>(g, ig,
                         [&](int r, int k) { return h2f(r == rn ? nh[k] : m[(int64_t)r * D + lane + 64 * k]); },
                         k_norm, ys[w], pooled + ((int64_t)s * g.bps + b) * D, lane, cc, sn);
    }
}

hipError_t launch_idx_append_pool(const Geo &g, const qwfn_kv_view &v, const IdxGeo &ig, uint16_t *raw,
                                  uint16_t *pooled, const float *k_norm, const void *src, int32_t src_f16,
                                  const int32_t *seq_ids, const int32_t *pos, int32_t n_rows, hipStream_t st,
                                  const FusedAppend &kv, const int32_t *len, const IdxCut &cut) {
    if (n_rows > kIdxFuseRows || (kv.enabled && !len) || (!len && !pos)) return hipErrorInvalidValue;
    if (cut.q_idx && (!len || ig.dim > 128 || cut.n_head < 1 || cut.n_head * ig.dim > kIdxMaxCutHeads * 128))
        return hipErrorInvalidValue;
#define QWFN_IDX_AP(D_)                                                                                        \
    if (len)                                                                                                   \
        hipLaunchKernelGGL(k_idx_decode_append<D_>, dim3(1 + (cut.q_idx ? n_rows * kIdxCutParts : 0)),          \
                           dim3(kIdxFuseThreads), 0,                                                            \
                           st, g, v, ig, raw, pooled, k_norm, src, src_f16, len, n_rows, kv, cut);              \
    else                                                                                                       \
        hipLaunchKernelGGL(k_idx_append_pool<D_>, dim3(1), dim3(kIdxFuseThreads), 0, st, g, v, ig, raw, pooled, \
                           k_norm, src, src_f16, seq_ids, pos, n_rows)
    switch (ig.dim) {
    case 64:  QWFN_IDX_AP(64); break;
    case 128: QWFN_IDX_AP(128); break;
    case 256: QWFN_IDX_AP(256); break;
    default: return hipErrorInvalidValue;
    }
#undef QWFN_IDX_AP
    return hipGetLastError();
}

hipError_t launch_idx_pool(const Geo &g, const qwfn_kv_view &v, const IdxGeo &ig, const uint16_t *raw,
                           uint16_t *pooled, const float *k_norm, const int32_t *seq_ids, const int32_t *pos,
                           int32_t n_items, int32_t seq_const, int32_t blk0, hipStream_t st) {
    if (n_items <= 0) return hipSuccess;
    const dim3 grid((unsigned)((n_items + 3) / 4));
    switch (ig.dim) {
    case 64:  hipLaunchKernelGGL(k_idx_pool<64>, grid, dim3(256), 0, st, g, v, ig, raw, pooled, k_norm, seq_ids, pos, n_items, seq_const, blk0); break;
    case 128: hipLaunchKernelGGL(k_idx_pool<128>, grid, dim3(256), 0, st, g, v, ig, raw, pooled, k_norm, seq_ids, pos, n_items, seq_const, blk0); break;
    case 256: hipLaunchKernelGGL(k_idx_pool<256>, grid, dim3(256), 0, st, g, v, ig, raw, pooled, k_norm, seq_ids, pos, n_items, seq_const, blk0); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace qwfn_qsa
