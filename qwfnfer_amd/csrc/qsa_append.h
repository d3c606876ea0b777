// qsa_append.h -- device helpers shared by the kernels that write the cache
// (q8_0 / q4_0 / fp16 rows, pooled keys) and by the decode launches that do
// it as one of their workgroups: the split-reduction completion protocol,
// ggml's q8_0 and q4_0 quantizers, member staging and the pooled-key chain,
// and the decode token's append + pool.
#pragma once

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include "qsa_device.h"

namespace qwfn_qsa {

// Completion protocol of a split reduction, called by EVERY thread of a
// workgroup that has finished writing its share (the barriers inside must be
// reached from one call site by all waves).  Each thread waits for its own
// stores, the barrier orders them before thread 0's agent-scope release fence
// and the counter increment; only the workgroup that arrives last takes the
// acquire fence before reading the others' results.  One fence pair per
// workgroup rather than per wave: on gfx950 an agent-scope fence writes back
// and invalidates the XCD's L2.  Returns true in the last workgroup.
//
// ACQ = false skips the acquire fence (an L2 invalidate, ~0.5 us): the last
// workgroup must then read the others' results only through device-coherent
// loads (buffer loads with kCpolSc1), or take the fence itself before plain
// loads.
template <bool ACQ = true>
__device__ __forceinline__ bool arrive_last(int32_t *counter, int expected, int *flag) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        const int old = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = old == expected - 1;
        if (ACQ && last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        *flag = last;
    }
    __syncthreads();
    return *flag != 0;
}

// Exclusive prefix sum over the NT threads of a workgroup; *total = the sum.
template <int NT>
__device__ __forceinline__ int block_excl_sum(int v, int *tmp, int *total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int x = wave_incl_scan(v);
    if (lane == 63) tmp[w] = x;
    __syncthreads();
    int base = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < NT / 64; ++i) {
        const int t = tmp[i];
        if (i < w) base += t;
        tot += t;
    }
    __syncthreads();
    *total = tot;
    return base + x - v;
}

// One q8_0 block is quantized by 8 consecutive lanes holding 4 values each:
// amax over the 32 values, d = amax/127 -> fp16, then the variant's id and
// rounding (ggml's q8_0 algorithm).  Returns the 4 quants packed little-endian
// and the fp16 scale; dq (if set) receives the dequantized values.
__device__ __forceinline__ uint32_t quant4(const float x[4], int variant, uint16_t *dh_out,
                                           float *dq) {
#pragma clang fp contract(off)
    float a = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float ax = fabsf(x[k]);
        a = ax > a ? ax : a;
    }
    // max over the block's 8 lanes (aligned groups of 8): quad xor 1, quad
    // xor 2, then the half-row mirror pairs the two quads
    a = fmaxf(a, dppf<kDppQuadXor1>(a, a));
    a = fmaxf(a, dppf<kDppQuadXor2>(a, a));
    a = fmaxf(a, dppf<kDppRowHalfMirror>(a, a));
    const float d = a / 127.0f;
    const uint16_t dh = f2h(d);
    float id;
    if (variant == QWFN_Q8_X86_RNE) id = a != 0.0f ? 127.0f / a : 0.0f;
    else                            id = d != 0.0f ? 1.0f / d : 0.0f;
    uint32_t pk = 0;
    const float df = h2f(dh);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        float r = x[k] * id;
        r = (variant == QWFN_Q8_X86_RNE) ? __builtin_rintf(r) : roundf(r);
        const int8_t qi = to_i8(r);
        pk |= (uint32_t)(uint8_t)qi << (8 * k);
        if (dq) dq[k] = df * (float)qi;
    }
    *dh_out = dh;
    return pk;
}

// Four quants (dims d..d+3 of one row, packed little-endian) into a K or V page.
__device__ __forceinline__ void store_q4(const Geo &g, uint8_t *page, bool is_v, int gh, int row, int d,
                                         uint32_t pk) {
    if (is_v && g.vdim) {
        const int64_t o = vquant_off(g, gh, row, d);
        page[o] = (uint8_t)pk;
        page[o + 64] = (uint8_t)(pk >> 8);
        page[o + 128] = (uint8_t)(pk >> 16);
        page[o + 192] = (uint8_t)(pk >> 24);
    } else {
        *reinterpret_cast<uint32_t *>(page + quant_off(g, gh, row, d)) = pk;
    }
}

__device__ __forceinline__ void load2(const void *src, int32_t f16, int64_t idx, float x[2]) {
    if (f16) {
        const uint32_t u = *reinterpret_cast<const uint32_t *>((const uint16_t *)src + idx);
        x[0] = h2f((uint16_t)(u & 0xFFFF)); x[1] = h2f((uint16_t)(u >> 16));
    } else {
        const float2 f = *reinterpret_cast<const float2 *>((const float *)src + idx);
        x[0] = f.x; x[1] = f.y;
    }
}

__device__ __forceinline__ void load4(const void *src, int32_t f16, int64_t idx, float x[4]) {
    if (f16) {
        const uint2 u = *reinterpret_cast<const uint2 *>((const uint16_t *)src + idx);
        x[0] = h2f((uint16_t)(u.x & 0xFFFF)); x[1] = h2f((uint16_t)(u.x >> 16));
        x[2] = h2f((uint16_t)(u.y & 0xFFFF)); x[3] = h2f((uint16_t)(u.y >> 16));
    } else {
        const float4 f = *reinterpret_cast<const float4 *>((const float *)src + idx);
        x[0] = f.x; x[1] = f.y; x[2] = f.z; x[3] = f.w;
    }
}

// One q4_0 block by 8 consecutive lanes, lane e holding values 2e, 2e+1,
// 16+2e, 17+2e (x[0..3]): ggml's quantize_row_q4_0_ref -- m = the element of
// largest magnitude (the first one on ties; +0 when every |x| is 0 or NaN),
// d = m / -8 stored as fp16, id = 1/d (0 when d == 0), q = min(15,
// trunc(x*id + 8.5)) (0 for a NaN), qs[j] = q[j] | q[j+16] << 4.  Returns this
// lane's two qs bytes (2e, 2e+1) packed little-endian and the fp16 scale.
__device__ __forceinline__ uint32_t quant_q4(const float x[4], int e, uint16_t *dh_out) {
#pragma clang fp contract(off)
    float a = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) a = fmaxf(a, fabsf(x[k]));
    a = fmaxf(a, dppf<kDppQuadXor1>(a, a));
    a = fmaxf(a, dppf<kDppQuadXor2>(a, a));
    a = fmaxf(a, dppf<kDppRowHalfMirror>(a, a));
    // the first index holding the largest magnitude, and its value
    const int idx[4] = {2 * e, 2 * e + 1, 16 + 2 * e, 17 + 2 * e};
    int bi = 32;
    float bv = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (a > 0.0f && fabsf(x[k]) == a && idx[k] < bi) { bi = idx[k]; bv = x[k]; }
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) {
        const int oi = __shfl_xor(bi, off, 8);
        const float ov = __shfl_xor(bv, off, 8);
        if (oi < bi) { bi = oi; bv = ov; }
    }
    const float d = bv / -8.0f;
    *dh_out = f2h(d);
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint32_t q[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float r = x[k] * id + 8.5f;
        const int t = r != r ? 0 : (int)r;          // truncation; |x*id| <= 8 keeps it in 0 .. 16
        q[k] = (uint32_t)(t < 15 ? t : 15);
    }
    return (q[0] | q[2] << 4) | ((q[1] | q[3] << 4) << 8);
}

// One lane of a K/V row append (k_append, and the decode step's append in
// k_idx_append_pool): lane i quantizes (q8_0, q4_0) or converts (F16) 4 values
// of one 32-value block and stores them with the block's scale.  Blocks
// enumerate (row, K|V, KV head, j), 8 lanes a block, which must be active
// together (the quantizers' DPP and shuffles span them); row r is sequence
// seq's token at position t, row_at(r, seq, t).  A bad sequence, position or
// page skips the block and is reported once a row.
template <class RowAt>
__device__ __forceinline__ void append_lane(const Geo &g, const qwfn_kv_view &v, const void *ksrc, const void *vsrc,
                                            int32_t f16, int64_t i, RowAt row_at) {
    const int nj = g.hd / 32;
    const int e4 = (int)(i & 7);
    int64_t qb = i >> 3;
    const int j = (int)(qb % nj); qb /= nj;
    const int gh = (int)(qb % g.Hkv); qb /= g.Hkv;
    const int which = (int)(qb & 1);
    const int r = (int)(qb >> 1);
    int seq, t;
    row_at(r, seq, t);
    const bool report = (e4 == 0 && j == 0 && gh == 0 && which == 0);
    // the lanes of one block stay together past the checks: they are uniform per block
    if (seq < 0 || seq >= g.n_seq_view) { if (report) set_status(v.status, QWFN_STATUS_SEQ_RANGE); return; }
    if (t < 0 || (int64_t)t >= (int64_t)g.pps * g.pt) { if (report) set_status(v.status, QWFN_STATUS_POS_RANGE); return; }
    const int32_t pp = phys_page(g, v.page_table, seq, t);
    if (pp < 0) { if (report) set_status(v.status, QWFN_STATUS_PAGE_RANGE); return; }
    const void *src = which ? vsrc : ksrc;
    const int64_t base = ((int64_t)r * g.Hkv + gh) * g.hd + 32 * j;
    uint8_t *page = (uint8_t *)(which ? v.v_pages : v.k_pages) + (int64_t)pp * g.page_bytes;
    const int row = t % g.pt;
    float x[4];
    if (g.kt == QWFN_KV_Q4_0) {
        float a[2], b[2];
        load2(src, f16, base + 2 * e4, a);
        load2(src, f16, base + 16 + 2 * e4, b);
        x[0] = a[0]; x[1] = a[1]; x[2] = b[0]; x[3] = b[1];
        uint16_t dh;
        const uint32_t qs = quant_q4(x, e4, &dh);
        *reinterpret_cast<uint16_t *>(page + chunk_off(g, gh, row, j) + 2 * e4) = (uint16_t)qs;
        if (e4 == 0) *reinterpret_cast<uint16_t *>(page + scale_off(g, gh, row, j)) = dh;
    } else if (g.kt == QWFN_KV_F16) {
        load4(src, f16, base + 4 * e4, x);
        const uint32_t lo = (uint32_t)f2h(x[0]) | (uint32_t)f2h(x[1]) << 16;
        const uint32_t hi = (uint32_t)f2h(x[2]) | (uint32_t)f2h(x[3]) << 16;
        const int d = 32 * j + 4 * e4;
        *reinterpret_cast<uint2 *>(page + chunk_off(g, gh, row, d / 8) + (d % 8) * 2) = make_uint2(lo, hi);
    } else {
        load4(src, f16, base + 4 * e4, x);
        uint16_t dh;
        const uint32_t pk = quant4(x, g.variant, &dh, nullptr);
        store_q4(g, page, which, gh, row, 32 * j + 4 * e4, pk);
        if (e4 == 0) *reinterpret_cast<uint16_t *>(page + scale_off(g, gh, row, j)) = dh;
    }
}

// One dequantized value straight from global memory (gather path): q8_0
// d*q, q4_0 d*(nibble - 8) (dims 0..15 of a block in the low nibbles of its
// 16 bytes, dims 16..31 in the high ones), fp16 as stored.
__device__ __forceinline__ float member_k(const Geo &g, const uint8_t *page, int gh, int row, int d,
                                          bool is_v = false) {
    if (g.kt == QWFN_KV_F16)
        return h2f(*reinterpret_cast<const uint16_t *>(page + chunk_off(g, gh, row, d / 8) + (d % 8) * 2));
    const uint16_t s = *reinterpret_cast<const uint16_t *>(page + scale_off(g, gh, row, d / 32));
    if (g.kt == QWFN_KV_Q4_0) {
        const uint8_t b = page[chunk_off(g, gh, row, d / 32) + d % 16];
        return h2f(s) * (float)((d % 32 < 16 ? (b & 15) : (b >> 4)) - 8);
    }
    const int8_t q = (int8_t)page[(is_v && g.vdim) ? vquant_off(g, gh, row, d) : quant_off(g, gh, row, d)];
    return h2f(s) * (float)q;
}

constexpr int kStageRows = 64;   // member rows staged through LDS per round

// Head-row bytes of K/V of an element type (compile-time twin of kv_row_bytes).
template <int HD, int KT> constexpr int row_bytes_t() { return KT == QWFN_KV_Q4_0 ? HD / 2 : KT == QWFN_KV_F16 ? 2 * HD : HD; }
// Member rows one staging round holds in kStageRows * HD bytes of LDS.
template <int HD, int KT> constexpr int stage_max_t() { return kStageRows * HD / row_bytes_t<HD, KT>() < kStageRows ? kStageRows * HD / row_bytes_t<HD, KT>() : kStageRows; }

// Rows [row0, row0+n) (n <= stage_max_t) of KV head gh of one page, copied
// into LDS as their raw row bytes raw[n][row bytes] and fp16 sc[n][HD/32] (no
// scales for fp16) -- every load issued before any is consumed, so the copy
// costs one memory round trip.
template <int HD, int KT = QWFN_KV_Q8_0>
__device__ __forceinline__ void stage_rows(const Geo &g, const uint8_t *page, int gh, int row0, int n,
                                           int8_t *raw, uint16_t *sc, int tid, int nt) {
    constexpr int RB = row_bytes_t<HD, KT>(), CH = RB / 16;
#pragma unroll 4
    for (int k = tid; k < n * CH; k += nt) {
        const int r = k % n, c = k / n, row = row0 + r;
        const uint4 val = *reinterpret_cast<const uint4 *>(
            page + ((int64_t)(gh * (g.pt / 64) + row / 64) * CH + c) * 1024 + (row % 64) * 16);
        *reinterpret_cast<uint4 *>(raw + r * RB + c * 16) = val;
    }
    if (KT == QWFN_KV_F16) return;
    const uint16_t *s = reinterpret_cast<const uint16_t *>(page + scale_off(g, gh, row0, 0));
#pragma unroll 4
    for (int k = tid; k < n * (HD / 32); k += nt) sc[k] = s[k];
}

// Dimension d of staged row t.
template <int HD, int KT>
__device__ __forceinline__ float staged_value(const int8_t *raw, const uint16_t *sc, int t, int d) {
    constexpr int RB = row_bytes_t<HD, KT>();
    if (KT == QWFN_KV_F16) return h2f(reinterpret_cast<const uint16_t *>(raw + t * RB)[d]);
    const float s = h2f(sc[t * (HD / 32) + d / 32]);
    if (KT == QWFN_KV_Q4_0) {
        const uint8_t b = (uint8_t)raw[t * RB + (d / 32) * 16 + d % 16];
        return s * (float)((d % 32 < 16 ? (b & 15) : (b >> 4)) - 8);
    }
    return s * (float)raw[t * RB + d];
}

// Pooled key of one block of KV head gh: thread d < HD keeps dimension d's
// chain acc = m_0 + m_1 + ... + m_{bt-1}, then * (1/bt).  With `last` set the
// final member is taken from it (the decode token, still in LDS) instead of
// memory.  All nt threads must call (it synchronises).
// Dimension tid's chain over n staged rows: acc + m_0 + ... + m_{n-1}, or
// m_0 + ... when `first` (the block's first member starts the chain).
template <int HD, int KT = QWFN_KV_Q8_0>
__device__ __forceinline__ float pool_chain(const int8_t *raw, const uint16_t *sc, int n, int tid, float acc,
                                            bool first) {
#pragma clang fp contract(off)
#pragma unroll 8
    for (int t = 0; t < n; ++t) {
        const float m = staged_value<HD, KT>(raw, sc, t, tid);
        acc = (first && t == 0) ? m : acc + m;
    }
    return acc;
}

template <int HD, int KT = QWFN_KV_Q8_0>
__device__ void pool_block_dev(const Geo &g, const uint8_t *page, int gh, int row0, float *dst,
                               const float *last, int8_t *q8, uint16_t *sc, int tid, int nt) {
#pragma clang fp contract(off)
    constexpr int SM = stage_max_t<HD, KT>();
    const int from_mem = last ? g.bt - 1 : g.bt;
    float acc = 0.0f;
    for (int r0 = 0; r0 < from_mem; r0 += SM) {
        const int n = min(SM, from_mem - r0);
        stage_rows<HD, KT>(g, page, gh, row0 + r0, n, q8, sc, tid, nt);
        __syncthreads();
        if (tid < HD) acc = pool_chain<HD, KT>(q8, sc, n, tid, acc, r0 == 0);
        __syncthreads();
    }
    if (tid < HD) {
        if (last) acc = (g.bt == 1) ? last[tid] : acc + last[tid];
        dst[tid] = acc * g.inv_bt;
    }
}

// Append of the decode token (K and V rows of KV head gh) and, when it
// completes its block, the block's pooled key -- the decode writes of
// src/qwfn_graph.cpp:465-476, 520-528 as one workgroup.  The new K row is
// kept dequantized in LDS as the block's last member.  KT: the cache type;
// lane (which, j, e4) holds the 4 values k_append's lane holds (q4_0: dims
// 2e4, 2e4+1, 16+2e4, 17+2e4 of block j; otherwise 4e4 .. 4e4+3).  NT
// threads; SH provides u.st.q8 / u.st.sc (kStageRows rows) and newk[HD].
template <int HD, int KT, int NT, typename SH>
__device__ __forceinline__ void fused_append_pool(const Geo &g, const qwfn_kv_view &v, const FusedAppend &fa,
                                                  int s, int gh, const int32_t *seq_len, int32_t max_seq_len,
                                                  SH &sh) {
    const int tid = threadIdx.x, per = (HD / 32) * 8;   // lanes per row
    const int which = tid / per, j = (tid % per) / 8, e4 = tid % 8;
    // the new rows do not depend on the length: their loads go out first
    float x[4] = {0.0f, 0.0f, 0.0f, 0.0f}, dq[4];
    const void *src = which ? fa.v_new : fa.k_new;
    const int64_t base = ((int64_t)s * g.Hkv + gh) * HD + 32 * j;
    if (tid < 2 * per) {
        if (KT == QWFN_KV_Q4_0) {
            float a[2], b[2];
            load2(src, fa.src_f16, base + 2 * e4, a);
            load2(src, fa.src_f16, base + 16 + 2 * e4, b);
            x[0] = a[0]; x[1] = a[1]; x[2] = b[0]; x[3] = b[1];
        } else {
            load4(src, fa.src_f16, base + 4 * e4, x);
        }
    }
    const int L = seq_len[s];
    if (L < 1 || L > max_seq_len) return;
    const int p = L - 1;
    const int32_t pp = phys_page(g, v.page_table, s, p);
    if (pp < 0) { if (tid == 0 && gh == 0) set_status(v.status, QWFN_STATUS_PAGE_RANGE); return; }
    const int row = p % g.pt;
    // a completed block's older members go to LDS while the new row is quantized
    const bool complete = L % g.bt == 0;
    const bool early = complete && g.bt > 1 && g.bt - 1 <= stage_max_t<HD, KT>();
    const uint8_t *kpage = (const uint8_t *)v.k_pages + (int64_t)pp * g.page_bytes;
    if (early)
        stage_rows<HD, KT>(g, kpage, gh, row - (g.bt - 1), g.bt - 1, sh.u.st.q8, sh.u.st.sc, tid, NT);
    uint8_t *page = (uint8_t *)(which ? v.v_pages : v.k_pages) + (int64_t)pp * g.page_bytes;
    if (KT == QWFN_KV_Q4_0) {
        uint16_t dh;
        const uint32_t qs = quant_q4(x, e4, &dh);     // all lanes: the shuffles need full groups
        const float d = h2f(dh);
        dq[0] = d * (float)((int)(qs & 15) - 8);
        dq[2] = d * (float)((int)((qs >> 4) & 15) - 8);
        dq[1] = d * (float)((int)((qs >> 8) & 15) - 8);
        dq[3] = d * (float)((int)((qs >> 12) & 15) - 8);
        if (tid < 2 * per) {
            *reinterpret_cast<uint16_t *>(page + chunk_off(g, gh, row, j) + 2 * e4) = (uint16_t)qs;
            if (e4 == 0) *reinterpret_cast<uint16_t *>(page + scale_off(g, gh, row, j)) = dh;
            if (which == 0) {
                const int d0 = 32 * j + 2 * e4;
                sh.newk[d0] = dq[0]; sh.newk[d0 + 1] = dq[1]; sh.newk[d0 + 16] = dq[2]; sh.newk[d0 + 17] = dq[3];
            }
        }
    } else if (KT == QWFN_KV_F16) {
        uint16_t h[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) { h[k] = f2h(x[k]); dq[k] = h2f(h[k]); }
        if (tid < 2 * per) {
            const int d = 32 * j + 4 * e4;
            *reinterpret_cast<uint2 *>(page + chunk_off(g, gh, row, d / 8) + (d % 8) * 2) =
                make_uint2((uint32_t)h[0] | (uint32_t)h[1] << 16, (uint32_t)h[2] | (uint32_t)h[3] << 16);
            if (which == 0)
                for (int k = 0; k < 4; ++k) sh.newk[d + k] = dq[k];
        }
    } else {
        uint16_t dh;
        const uint32_t pk = quant4(x, g.variant, &dh, dq);   // all lanes: DPP needs full groups
        if (tid < 2 * per) {
            store_q4(g, page, which, gh, row, 32 * j + 4 * e4, pk);
            if (e4 == 0) *reinterpret_cast<uint16_t *>(page + scale_off(g, gh, row, j)) = dh;
            if (which == 0)
                for (int k = 0; k < 4; ++k) sh.newk[32 * j + 4 * e4 + k] = dq[k];
        }
    }
    __syncthreads();
    if (!complete) return;                         // the block is not complete yet
    const int b = p / g.bt;
    float *dst = v.pooled + (((int64_t)s * g.Hkv + gh) * g.bps + b) * HD;
    if (early) {
#pragma clang fp contract(off)
        if (tid < HD)
            dst[tid] = (pool_chain<HD, KT>(sh.u.st.q8, sh.u.st.sc, g.bt - 1, tid, 0.0f, true) + sh.newk[tid]) *
                       g.inv_bt;
        return;
    }
    pool_block_dev<HD, KT>(g, kpage, gh, row - (g.bt - 1), dst, sh.newk, sh.u.st.q8, sh.u.st.sc, tid, NT);
}

}  // namespace qwfn_qsa
