// qsa_idx_pool.h -- the checkpoint indexer's one-block pooling by one wave
// (the arithmetic pool_idx_block in qsa_idx.hip documents: mean, RMSNorm *
// k_norm, ggml's rotation, fp16 store; src/qwfn_graph.cpp:410-429), shared by
// the indexer-key launches of qsa_idx.hip and by the indexer's own append
// workgroup in qsa_kernels.hip (the fused checkpoint decode step up to 8,192
// blocks), with the score of the block it completes.
#pragma once
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include "qsa_append.h"
#include "qsa_device.h"
#include "qsa_internal.h"

namespace qwfn_qsa {

// cos / sin of the rotation of dims lane + 64 k (pool_idx_block's arithmetic) for a
// block at position t0: 1, 0 for the dims past nd.
template <int D>
__device__ __forceinline__ void idx_rot_cs(const IdxGeo &ig, int t0, int lane, float (&cc)[D / 64],
                                           float (&sn)[D / 64]) {
    const int half = ig.nd / 2;
#pragma unroll
    for (int k = 0; k < D / 64; ++k) {
        const int d = lane + 64 * k;
        cc[k] = 1.0f;
        sn[k] = 0.0f;
        if (d < ig.nd) {
            const int i = d < half ? d : d - half;
            // ggml's angle of pair i: the block position times theta_scale, i
            // times over, each product rounded to fp32
            float th = (float)t0;
            for (int e = 0; e < i; ++e) th = __fmul_rn(th, ig.theta_scale);
            cc[k] = (float)cos((double)th);
            sn[k] = (float)sin((double)th);
        }
    }
}

// The pooled key of one block from its bt members (row(r, k): member r's dim
// lane + 64 k as fp32, position order) and its rotation's cos / sin, by one
// wave (pool_idx_block's arithmetic).
template <int D, class Row>
__device__ __forceinline__ void pool_idx_rows(const Geo &g, const IdxGeo &ig, Row row, const float *__restrict__ k_norm,
                                              float *ys, uint16_t *dst, int lane, const float (&cc)[D / 64],
                                              const float (&sn)[D / 64], float *yo = nullptr) {
#pragma clang fp contract(off)
    constexpr int K = D / 64, U = 8;
    float x[K];
    for (int r0 = 0; r0 < g.bt; r0 += U) {
        float y[U][K];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int r = min(r0 + u, g.bt - 1);
#pragma unroll
            for (int k = 0; k < K; ++k) y[u][k] = row(r, k);
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int k = 0; k < K; ++k)
                if (r0 + u < g.bt) x[k] = r0 + u == 0 ? y[u][k] : x[k] + y[u][k];
    }
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        x[k] = x[k] * g.inv_bt;
        const float sq = x[k] * x[k];
        ss = ss + (double)sq;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss = ss + __shfl_xor(ss, off);
    const float mean = (float)(ss / (double)D);
    const float scale = 1.0f / sqrtf(mean + ig.eps);
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int d = lane + 64 * k;
        ys[d] = (x[k] * scale) * k_norm[d];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    const int half = ig.nd / 2;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int d = lane + 64 * k;
        float o = ys[d];
        if (d < ig.nd) {
            const int i = d < half ? d : d - half;
            const float c = cc[k], s = sn[k];
            const float x0 = ys[i], x1 = ys[i + half];
            o = d < half ? x0 * c - x1 * s : x0 * s + x1 * c;
        }
        const uint16_t h = f2h(o);
        dst[d] = h;
        if (yo) yo[d] = h2f(h);                    // the stored key, widened exactly
    }
}

// The query values lane (h, j) = (lane / 4, lane % 4) of a wave needs for
// one block's score: head h's dims 16 i + 4 j .. + 3, i < D / 16 (lanes past
// 4 G repeat the last head).
template <int D, int G>
__device__ __forceinline__ void idx_score_q(const float *__restrict__ q, int lane, float4 (&qr)[D / 16]) {
    const int h = min(lane >> 2, G - 1), j = lane & 3;
#pragma unroll
    for (int i = 0; i < D / 16; ++i) qr[i] = *reinterpret_cast<const float4 *>(&q[h * D + 16 * i + 4 * j]);
}

// The score of one pooled block (fp32 key yo [D] in LDS, the stored fp16 values
// widened) against G query heads, in the indexer's order exactly (k_indexer:
// lane j of four holds dims 16 i + 4 j .. + 3, one fmaf chain a head over
// them, (c0+c1)+(c2+c3) across the four lanes, relu per head when set, the
// heads summed in order).  Here lane (h, j) runs head h's chain j (its query
// values qr from idx_score_q), so the four heads' chains run side by side;
// the wave's lanes 0, 4, .. hold the heads' dots.
template <int D, int G>
__device__ __forceinline__ float idx_block_score(const float *yo, const float4 (&qr)[D / 16], bool relu, int lane) {
#pragma clang fp contract(off)
    static_assert(4 * G <= 64, "a head's four chains a lane each");
    const int j = lane & 3;
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < D / 16; ++i) {
        const float4 p = *reinterpret_cast<const float4 *>(&yo[16 * i + 4 * j]);
        acc = fmaf(qr[i].x, p.x, acc);
        acc = fmaf(qr[i].y, p.y, acc);
        acc = fmaf(qr[i].z, p.z, acc);
        acc = fmaf(qr[i].w, p.w, acc);
    }
    const float t01 = acc + __shfl_xor(acc, 1);   // (c0+c1) / (c2+c3)
    float dot = t01 + __shfl_xor(t01, 2);         // (c0+c1)+(c2+c3)
    if (relu) dot = dot > 0.0f ? dot : 0.0f;
    float score = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dot), 0));
#pragma unroll
    for (int h = 1; h < G; ++h) score = score + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dot), 4 * h));
    return score;
}

// The indexer's append workgroup of sequence s (the fused checkpoint decode
// step with the attention selecting from the indexer's row): the token's K and
// V rows into the attention's pages (append_lane, waves 1 ..), its raw key
// into the raw cache and its block re-pooled from the members and the new row
// (wave 0, as k_idx_decode_append); when the token completes the block, wave
// 0 also scores it from the stored key (idx_block_score) into the sequence's
// score row, which the scoring workgroups leave to it.  With the cut placed in
// the same launch (ia.slots), that score's key + 1 also goes to the slot after
// the sequence's part keys, whenever the scoring workgroup of that block
// expects it (the key 0 when an error ends the append first).  scratch: 2 D
// floats.
template <int D, int G, int NT>
__device__ __forceinline__ void idx_append_wg(const Geo &gi, const IdxAppend &ia, const float *__restrict__ q,
                                              const int32_t *len, int s, uint16_t *pooled, float *sc,
                                              float *scratch) {
    static_assert(NT > 64, "wave 0 keys, the others K / V");
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const Geo &g = ia.ga;
    if (w != 0) {                                  // the K / V rows; wave 0 starts the key's chain at once
        if (ia.kv.enabled) {
            const int64_t per = (int64_t)2 * g.Hkv * (g.hd / 32) * 8;
            for (int64_t i = tid - 64; i < per; i += NT - 64)
                append_lane(g, ia.va, ia.kv.k_new, ia.kv.v_new, ia.kv.src_f16, (int64_t)s * per + i,
                            [&](int r, int &seq, int &t) {
                                seq = r;
                                t = len[r] - 1;
                            });
        }
        return;
    }
    constexpr int K = D / 64;
    const int L = len[s];
    uint16_t nh[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int64_t e = (int64_t)s * D + lane + 64 * k;
        nh[k] = ia.f16 ? reinterpret_cast<const uint16_t *>(ia.src)[e] : f2h(reinterpret_cast<const float *>(ia.src)[e]);
    }
    float4 qr[D / 16];                             // the block score's query values, loaded early
    idx_score_q<D, G>(q + (int64_t)s * gi.H * D, lane, qr);
    // the block this token completes, when it is eligible: its chunk's scoring
    // workgroup waits for its key in the slot (the same test on that side);
    // tested once the loads above are out
    bool expect = false;
    if (ia.slots && L >= 1 && L % g.bt == 0 && gi.topk > 0) {
        const Ranges r = qsa_ranges(gi, L);
        const int bc = (L - 1) / g.bt;
        expect = r.e_hi - r.e_lo > eff_topk(gi, r) && bc >= r.e_lo && bc < r.e_hi;
    }
    uint32_t *slot = ia.slots ? ia.slots + (int64_t)s * kCutSlots + kIdxCutParts : nullptr;
    auto publish = [&](uint32_t key1) {
        if (expect && lane == 0) __hip_atomic_store(slot, key1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    const int t = L - 1;
    if (s >= g.n_seq_view) { if (lane == 0) set_status(ia.va.status, QWFN_STATUS_SEQ_RANGE); publish(1u); return; }
    if (t < 0 || (int64_t)t >= (int64_t)g.pps * g.pt) {
        if (lane == 0) set_status(ia.va.status, QWFN_STATUS_POS_RANGE);
        publish(1u);
        return;
    }
    const int32_t pp = phys_page(g, ia.va.page_table, s, t);
    const int b = t / g.bt, t0 = b * g.bt, rn = t - t0;
    float cc[K], sn[K];
    idx_rot_cs<D>(ia.ig, t0, lane, cc, sn);
    if (pp < 0) { if (lane == 0) set_status(ia.va.status, QWFN_STATUS_PAGE_RANGE); publish(1u); return; }
    uint16_t *row = ia.raw + ((int64_t)pp * g.pt + t % g.pt) * D;
#pragma unroll
    for (int k = 0; k < K; ++k) row[lane + 64 * k] = nh[k];
    const uint16_t *m = ia.raw + ((int64_t)pp * g.pt + t0 % g.pt) * D;   // a block never straddles pages
    float *ys = scratch, *yo = scratch + D;
    pool_idx_rows<D>(g, ia.ig, [&](int r, int k) { return h2f(r == rn ? nh[k] : m[(int64_t)r * D + lane + 64 * k]); },
                     ia.k_norm, ys, pooled + ((int64_t)s * g.bps + b) * D, lane, cc, sn, yo);
    if (rn != g.bt - 1) return;                    // (uniform) a partial block is forced, not scored
    const Ranges r = qsa_ranges(gi, L);
    if (!(gi.topk > 0 && r.e_hi - r.e_lo > eff_topk(gi, r) && b >= r.e_lo && b < r.e_hi)) return;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    const float score = idx_block_score<D, G>(yo, qr, gi.relu, lane);
    if (lane == 0) sc[b] = score;
    publish(score_key(score) + 1u);
}

}  // namespace qwfn_qsa
