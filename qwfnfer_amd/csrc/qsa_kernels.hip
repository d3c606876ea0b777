// qsa_kernels.hip -- gfx950 (CDNA4) kernels of the q8_0 KV cache and the QSA
// decode path.  Wave64 throughout; every cross-lane reduction is a
// __shfl_xor / __shfl_up ladder inside one wave, every cross-wave step goes
// through LDS.  Kernels that must be bit-exact against the CPU oracle (append,
// pool, indexer scores and selection) are compiled with fp contraction off and
// spell every fused multiply-add as fmaf.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include "qsa_internal.h"

namespace qwfn_qsa {

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// Byte offsets inside a page (layout in include/qwfn_qsa.h).
__device__ __forceinline__ int64_t quant_off(const Geo &g, int gh, int row, int d) {
    return ((int64_t)(gh * (g.pt / 64) + row / 64) * (g.hd / 16) + d / 16) * 1024 +
           (row % 64) * 16 + d % 16;
}
__device__ __forceinline__ int64_t scale_off(const Geo &g, int gh, int row, int j) {
    return g.qbytes + ((int64_t)(gh * g.pt + row) * (g.hd / 32) + j) * 2;
}

__device__ __forceinline__ void set_status(int32_t *st, int32_t bits) {
    if (st) atomicOr(st, bits);
}

// Physical page of (seq, t) or -1.  Caller has range-checked seq and t.
__device__ __forceinline__ int32_t phys_page(const Geo &g, const int32_t *pt, int seq, int t) {
    const int32_t p = pt[(int64_t)seq * g.pps + t / g.pt];
    return (p >= 0 && p < g.n_phys) ? p : -1;
}

__device__ __forceinline__ int8_t to_i8(float r) {
    if (r != r) return 0;
    if (r > 127.0f) return 127;
    if (r < -128.0f) return -128;
    return (int8_t)(int)r;
}

// Orderable key of a score: larger key = larger score; NaN lowest; -0 == +0.
__device__ __forceinline__ uint32_t score_key(float x) {
    if (x != x) return 0u;
    if (x == 0.0f) return 0x80000000u;
    const uint32_t u = __float_as_uint(x);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// Exclusive prefix sum over the NT threads of a workgroup; *total = the sum.
template <int NT>
__device__ __forceinline__ int block_excl_sum(int v, int *tmp, int *total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o);
        if (lane >= o) x += y;
    }
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
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) {
        const float b = __shfl_xor(a, o);
        a = b > a ? b : a;
    }
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

// ---------------------------------------------------------------------------
// append: quantize rows to q8_0 and overwrite them in the paged cache
// ---------------------------------------------------------------------------

// Lane i: 4 values of one q8_0 block; blocks enumerate (row, K|V, head, j).
__global__ void __launch_bounds__(256)
k_append(Geo g, qwfn_kv_view v, const void *ksrc, const void *vsrc, int32_t f16,
         const int32_t *seq_ids, const int32_t *pos, int32_t n_rows) {
    const int nj = g.hd / 32;
    const int64_t total = (int64_t)n_rows * 2 * g.Hkv * nj * 8;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const int e4 = (int)(i & 7);
    int64_t qb = i >> 3;
    const int j = (int)(qb % nj); qb /= nj;
    const int gh = (int)(qb % g.Hkv); qb /= g.Hkv;
    const int which = (int)(qb & 1);
    const int r = (int)(qb >> 1);
    const int seq = seq_ids ? seq_ids[r] : 0;
    const int t = pos[r];
    const bool report = (e4 == 0 && j == 0 && gh == 0 && which == 0);
    if (seq < 0 || seq >= g.n_seq_view) { if (report) set_status(v.status, QWFN_STATUS_SEQ_RANGE); return; }
    if (t < 0 || (int64_t)t >= (int64_t)g.pps * g.pt) { if (report) set_status(v.status, QWFN_STATUS_POS_RANGE); return; }
    const int32_t pp = phys_page(g, v.page_table, seq, t);
    if (pp < 0) { if (report) set_status(v.status, QWFN_STATUS_PAGE_RANGE); return; }
    float x[4];
    load4(which ? vsrc : ksrc, f16, ((int64_t)r * g.Hkv + gh) * g.hd + 32 * j + 4 * e4, x);
    uint16_t dh;
    const uint32_t pk = quant4(x, g.variant, &dh, nullptr);
    uint8_t *page = (uint8_t *)(which ? v.v_pages : v.k_pages) + (int64_t)pp * g.page_bytes;
    const int row = t % g.pt;
    *reinterpret_cast<uint32_t *>(page + quant_off(g, gh, row, 32 * j + 4 * e4)) = pk;
    if (e4 == 0) *reinterpret_cast<uint16_t *>(page + scale_off(g, gh, row, j)) = dh;
}

hipError_t launch_append(const Geo &g, const qwfn_kv_view &v, const void *k, const void *vv,
                         int32_t src_f16, const int32_t *seq_ids, const int32_t *pos,
                         int32_t n_rows, hipStream_t st) {
    const int64_t total = (int64_t)n_rows * 2 * g.Hkv * (g.hd / 32) * 8;
    const int64_t blocks = (total + 255) / 256;
    hipLaunchKernelGGL(k_append, dim3((unsigned)blocks), dim3(256), 0, st, g, v, k, vv, src_f16,
                       seq_ids, pos, n_rows);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// pooled keys: sequential fp32 add chain over the block's members, * 1/bt
// ---------------------------------------------------------------------------

__device__ __forceinline__ float member_k(const Geo &g, const uint8_t *page, int gh, int row, int d) {
    const int8_t q = (int8_t)page[quant_off(g, gh, row, d)];
    const uint16_t s = *reinterpret_cast<const uint16_t *>(page + scale_off(g, gh, row, d / 32));
    return h2f(s) * (float)q;
}

// grid (n_blocks, Hkv), block = hd threads; thread d owns one dimension.
__global__ void __launch_bounds__(256)
k_pool(Geo g, qwfn_kv_view v, const int32_t *seq_ids, const int32_t *block_ids, int32_t seq_const) {
#pragma clang fp contract(off)
    const int bi = blockIdx.x, gh = blockIdx.y, d = threadIdx.x;
    const int seq = seq_ids ? seq_ids[bi] : seq_const;
    const int b = block_ids ? block_ids[bi] : bi;
    const bool report = (gh == 0 && d == 0);
    if (seq < 0 || seq >= g.n_seq_view) { if (report) set_status(v.status, QWFN_STATUS_SEQ_RANGE); return; }
    if (b < 0 || b >= g.bps) { if (report) set_status(v.status, QWFN_STATUS_BLOCK_RANGE); return; }
    const int t0 = b * g.bt;
    const int32_t pp = phys_page(g, v.page_table, seq, t0);   // a block never straddles pages
    if (pp < 0) { if (report) set_status(v.status, QWFN_STATUS_PAGE_RANGE); return; }
    const uint8_t *page = (const uint8_t *)v.k_pages + (int64_t)pp * g.page_bytes;
    const int row0 = t0 % g.pt;
    float acc = member_k(g, page, gh, row0, d);
    for (int t = 1; t < g.bt; ++t) acc = acc + member_k(g, page, gh, row0 + t, d);
    v.pooled[(((int64_t)seq * g.Hkv + gh) * g.bps + b) * g.hd + d] = acc * g.inv_bt;
}

hipError_t launch_pool(const Geo &g, const qwfn_kv_view &v, const int32_t *seq_ids,
                       const int32_t *block_ids, int32_t n_blocks, int32_t seq_const,
                       hipStream_t st) {
    hipLaunchKernelGGL(k_pool, dim3((unsigned)n_blocks, (unsigned)g.Hkv), dim3((unsigned)g.hd), 0, st,
                       g, v, seq_ids, block_ids, seq_const);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// indexer: scores of the eligible blocks, then top-k in the last workgroup
// ---------------------------------------------------------------------------

// Forced/eligible ranges of a sequence of length L (same rule as the oracle):
// F = [0, sink) U [fw, b_last], E = [sink, min(L/bt, fw)).
struct Ranges { int b_last, fw, e_lo, e_hi; };
__device__ __forceinline__ Ranges qsa_ranges(const Geo &g, int L) {
    Ranges r;
    const int last = L - 1, w0 = last - g.local + 1, nbw = L / g.bt;
    r.b_last = last / g.bt;
    r.fw = w0 > 0 ? w0 / g.bt : 0;
    r.e_lo = g.sink;
    r.e_hi = nbw < r.fw ? nbw : r.fw;
    if (r.e_hi < r.e_lo) r.e_hi = r.e_lo;
    return r;
}

constexpr int kIdxThreads = 256;
constexpr int kBlocksPerChunk = kIdxThreads / 4;   // 4 lanes share one block's dot

struct IdxShared {
    float q[16 * 256];            // the group's query heads, G <= 16, hd <= 256
    uint32_t hist[4096];
    float newk[256];
    int tmp[8];
    int flag, bin, need;
};

// Append of the decode token (K and V rows of KV head gh) and, when it
// completes its block, the block's pooled key -- the decode writes of
// src/qwfn_graph.cpp:465-476, 520-528 as one workgroup.  The new K row is
// also kept dequantized in LDS as the block's last member.
__device__ void fused_append_pool(const Geo &g, const qwfn_kv_view &v, const FusedAppend &fa,
                                  int s, int gh, int L, IdxShared &sh) {
#pragma clang fp contract(off)
    const int tid = threadIdx.x, nj = g.hd / 32, per = nj * 8;   // lanes per row
    const int p = L - 1;
    const int32_t pp = phys_page(g, v.page_table, s, p);
    if (pp < 0) { if (tid == 0 && gh == 0) set_status(v.status, QWFN_STATUS_PAGE_RANGE); return; }
    const int row = p % g.pt;
    if (tid < 2 * per) {
        const int which = tid / per, j = (tid % per) / 8, e4 = tid % 8;
        float x[4], dq[4];
        load4(which ? fa.v_new : fa.k_new, fa.src_f16, ((int64_t)s * g.Hkv + gh) * g.hd + 32 * j + 4 * e4, x);
        uint16_t dh;
        const uint32_t pk = quant4(x, g.variant, &dh, dq);
        uint8_t *page = (uint8_t *)(which ? v.v_pages : v.k_pages) + (int64_t)pp * g.page_bytes;
        *reinterpret_cast<uint32_t *>(page + quant_off(g, gh, row, 32 * j + 4 * e4)) = pk;
        if (e4 == 0) *reinterpret_cast<uint16_t *>(page + scale_off(g, gh, row, j)) = dh;
        if (which == 0)
            for (int k = 0; k < 4; ++k) sh.newk[32 * j + 4 * e4 + k] = dq[k];
    }
    __syncthreads();
    if (L % g.bt != 0) return;                     // the block is not complete yet
    const int b = p / g.bt, row0 = row - (g.bt - 1);
    const uint8_t *page = (const uint8_t *)v.k_pages + (int64_t)pp * g.page_bytes;
    for (int d = tid; d < g.hd; d += kIdxThreads) {
        float acc = sh.newk[d];
        if (g.bt > 1) {
            acc = member_k(g, page, gh, row0, d);
            for (int t = 1; t < g.bt - 1; ++t) acc = acc + member_k(g, page, gh, row0 + t, d);
            acc = acc + sh.newk[d];
        }
        v.pooled[(((int64_t)s * g.Hkv + gh) * g.bps + b) * g.hd + d] = acc * g.inv_bt;
    }
}

// One radix pass over the eligible keys that match `prefix` above bit
// shift+bits: histogram of the `bits`-bit digit at `shift`, then the digit of
// the need-th largest key.  Updates *prefix (appending the digit) and *need.
template <int BITS>
__device__ void radix_pass(const float *sc, int e_lo, int e_hi, int shift, uint32_t &prefix,
                           int &need, bool first, IdxShared &sh) {
    constexpr int NB = 1 << BITS, PER = NB / kIdxThreads > 0 ? NB / kIdxThreads : 1;
    const int tid = threadIdx.x;
    for (int i = tid; i < NB; i += kIdxThreads) sh.hist[i] = 0u;
    __syncthreads();
    for (int b = e_lo + tid; b < e_hi; b += kIdxThreads) {
        const uint32_t k = score_key(sc[b]);
        if (first || (k >> (shift + BITS)) == prefix) atomicAdd(&sh.hist[(k >> shift) & (NB - 1)], 1u);
    }
    __syncthreads();
    // suffix counts: thread t owns bins [t*PER, t*PER+PER) (all threads when
    // NB >= 256; threads >= NB own nothing)
    int own = 0;
    if (tid * PER < NB)
        for (int i = 0; i < PER; ++i) own += (int)sh.hist[tid * PER + i];
    int total;
    const int excl = block_excl_sum<kIdxThreads>(own, sh.tmp, &total);
    const int above = total - excl - own;        // keys in bins owned by higher threads
    if (tid * PER < NB && above < need && above + own >= need) {
        int run = above;
        for (int i = PER - 1; i >= 0; --i) {
            const int c = (int)sh.hist[tid * PER + i];
            if (run + c >= need) { sh.bin = tid * PER + i; sh.need = need - run; break; }
            run += c;
        }
    }
    __syncthreads();
    prefix = first ? (uint32_t)sh.bin : ((prefix << BITS) | (uint32_t)sh.bin);
    need = sh.need;
    __syncthreads();
}

// Selection of one (sequence, KV head) by the last scoring workgroup.
__device__ void select_blocks(const Geo &g, const float *sc, int L, int32_t *out, int32_t *nout,
                              IdxShared &sh) {
    const int tid = threadIdx.x;
    const Ranges r = qsa_ranges(g, L);
    const int ne = r.e_hi - r.e_lo;
    if (g.topk <= 0 || ne <= g.topk) {
        const int n = r.b_last + 1;
        for (int i = tid; i < n; i += kIdxThreads) out[i] = i;
        if (tid == 0) *nout = n;
        return;
    }
    uint32_t prefix = 0;
    int need = g.topk;
    radix_pass<12>(sc, r.e_lo, r.e_hi, 20, prefix, need, true, sh);
    radix_pass<12>(sc, r.e_lo, r.e_hi, 8, prefix, need, false, sh);
    radix_pass<8>(sc, r.e_lo, r.e_hi, 0, prefix, need, false, sh);
    const uint32_t T = prefix;
    // ordered compaction: thread t owns the contiguous range [b0, b1)
    const int per = (ne + kIdxThreads - 1) / kIdxThreads;
    const int b0 = r.e_lo + tid * per;
    const int b1 = min(b0 + per, r.e_hi);
    int eq = 0;
    for (int b = b0; b < b1; ++b) eq += (score_key(sc[b]) == T);
    int tot;
    int eqi = block_excl_sum<kIdxThreads>(eq, sh.tmp, &tot);
    int cnt = 0;
    {
        int e2 = eqi;
        for (int b = b0; b < b1; ++b) {
            const uint32_t k = score_key(sc[b]);
            bool take = k > T;
            if (k == T) take = (e2++ < need);
            cnt += take;
        }
    }
    int pos = g.sink + block_excl_sum<kIdxThreads>(cnt, sh.tmp, &tot);
    for (int b = b0; b < b1; ++b) {
        const uint32_t k = score_key(sc[b]);
        bool take = k > T;
        if (k == T) take = (eqi++ < need);
        if (take) out[pos++] = b;
    }
    for (int i = tid; i < g.sink; i += kIdxThreads) out[i] = i;
    const int nwin = r.b_last - r.fw + 1;
    for (int i = tid; i < nwin; i += kIdxThreads) out[g.sink + g.topk + i] = r.fw + i;
    if (tid == 0) *nout = g.sink + g.topk + nwin;
}

// grid (n_chunks [+1 with the fused append], Hkv, n_seq)
template <int G>
__global__ void __launch_bounds__(kIdxThreads)
k_indexer(Geo g, qwfn_kv_view v, const float *q, const int32_t *seq_len, int32_t max_seq_len,
          int32_t *sel, int32_t *nsel, int32_t max_sel, Ws ws, int32_t n_chunks, FusedAppend fa) {
#pragma clang fp contract(off)
    __shared__ IdxShared sh;
    const int tid = threadIdx.x, c = blockIdx.x, gh = blockIdx.y, s = blockIdx.z;
    const int L = seq_len[s];
    const bool ok = L >= 1 && L <= max_seq_len;
    if (fa.enabled && c == n_chunks) {             // the append workgroup
        if (ok) fused_append_pool(g, v, fa, s, gh, L, sh);
        return;
    }
    const int pair = s * g.Hkv + gh;
    float *sc = ws.scores + (int64_t)pair * ws.nb_cap;
    if (ok && g.topk > 0) {
        const Ranges r = qsa_ranges(g, L);
        const int ne = r.e_hi - r.e_lo;
        if (ne > g.topk && c * kBlocksPerChunk < ne) {
            const float *qg = q + ((int64_t)s * g.H + (int64_t)gh * G) * g.hd;
            for (int i = tid * 4; i < G * g.hd; i += kIdxThreads * 4)
                *reinterpret_cast<float4 *>(&sh.q[i]) = *reinterpret_cast<const float4 *>(qg + i);
            __syncthreads();
            const int bl = tid >> 2, j = tid & 3;
            const int bi = c * kBlocksPerChunk + bl;
            const bool act = bi < ne;
            const int b = r.e_lo + (act ? bi : 0);
            const float *P = v.pooled + (((int64_t)s * g.Hkv + gh) * g.bps + b) * g.hd;
            float acc[G];
#pragma unroll
            for (int h = 0; h < G; ++h) acc[h] = 0.0f;
            if (act) {
                for (int i = 0; i < g.hd / 16; ++i) {
                    const float4 p4 = *reinterpret_cast<const float4 *>(P + 16 * i + 4 * j);
#pragma unroll
                    for (int h = 0; h < G; ++h) {
                        const float4 q4 = *reinterpret_cast<const float4 *>(&sh.q[h * g.hd + 16 * i + 4 * j]);
                        acc[h] = fmaf(q4.x, p4.x, acc[h]);
                        acc[h] = fmaf(q4.y, p4.y, acc[h]);
                        acc[h] = fmaf(q4.z, p4.z, acc[h]);
                        acc[h] = fmaf(q4.w, p4.w, acc[h]);
                    }
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
        }
    }
    // completion count: the last workgroup of this (sequence, KV head) selects
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const int old = atomicAdd(&ws.cnt_idx[pair], 1);
        sh.flag = (old == n_chunks - 1);
    }
    __syncthreads();
    if (!sh.flag) return;
    __threadfence();
    if (tid == 0) ws.cnt_idx[pair] = 0;
    int32_t *out = sel + (int64_t)pair * max_sel;
    if (!ok) {
        if (tid == 0) { nsel[pair] = 0; if (gh == 0) set_status(v.status, QWFN_STATUS_LEN_RANGE); }
        return;
    }
    select_blocks(g, sc, L, out, nsel + pair, sh);
}

template <int G>
static void launch_indexer_g(const Geo &g, const qwfn_kv_view &v, const float *q,
                             const int32_t *seq_len, int32_t n_seq, int32_t max_seq_len,
                             int32_t *sel, int32_t *nsel, int32_t max_sel, const Ws &ws,
                             const FusedAppend &fa, hipStream_t st) {
    const int nb_max = max_seq_len / g.bt;
    int n_chunks = (nb_max + kBlocksPerChunk - 1) / kBlocksPerChunk;
    if (n_chunks < 1) n_chunks = 1;
    const dim3 grid((unsigned)(n_chunks + (fa.enabled ? 1 : 0)), (unsigned)g.Hkv, (unsigned)n_seq);
    hipLaunchKernelGGL(k_indexer<G>, grid, dim3(kIdxThreads), 0, st, g, v, q, seq_len, max_seq_len,
                       sel, nsel, max_sel, ws, n_chunks, fa);
}

// ---------------------------------------------------------------------------
// attention: one 64-cell tile per workgroup, partial softmax state per tile,
// the last workgroup of a (sequence, KV head) merges the partials
// ---------------------------------------------------------------------------

template <int HD, int G>
struct AttnCfg {
    static constexpr int NW = G >= 4 ? 4 : G;          // waves per workgroup
    static constexpr int HPW = G / NW;                 // query heads per wave
    static constexpr int NT = NW * 64;
    static constexpr int CH = HD / 16;                 // 16-byte chunks per head row
    static constexpr int ROWF = HD + 4;                // padded LDS row (floats)
    static constexpr int DPL = HD / 64;                // PV dims per lane
    static_assert(G % NW == 0, "group size");
    static_assert(HD % 64 == 0, "head_dim");
};

template <int HD, int G>
struct AttnShared {
    float kv[64 * AttnCfg<HD, G>::ROWF];
    float p[G][64];
    uint16_t ksc[64][HD / 32], vsc[64][HD / 32];
    int32_t kpage[64], row[64];
    float Mh[G], Lh[G];
    int flag;
};

template <int HD, int G>
__global__ void __launch_bounds__((AttnCfg<HD, G>::NT))
k_attn(Geo g, qwfn_kv_view v, const float *__restrict__ q, const int32_t *seq_len,
       int32_t max_seq_len, const int32_t *sel, const int32_t *nsel, int32_t max_sel,
       float *__restrict__ out, Ws ws, int32_t n_tiles) {
    using C = AttnCfg<HD, G>;
    __shared__ AttnShared<HD, G> sh;
    const int tid = threadIdx.x, tile = blockIdx.x, gh = blockIdx.y, s = blockIdx.z;
    const int pair = s * g.Hkv + gh;
    const int L = seq_len[s];
    const bool ok = L >= 1 && L <= max_seq_len;
    int n = 0;
    if (ok) {
        n = sel ? nsel[pair] : (L - 1) / g.bt + 1;
        n = n < max_sel ? n : max_sel;
    }
    const int tiles_act = (n * g.bt + 63) / 64;
    if (ok && tile < tiles_act) {
        // cells of this tile -> (token, K page, V page)
        if (tid < 64) {
            const int cidx = tile * 64 + tid, slot = cidx / g.bt;
            int kp = -1, rw = -1;
            if (slot < n) {
                const int blk = sel ? sel[(int64_t)pair * max_sel + slot] : slot;
                const int t = blk * g.bt + cidx % g.bt;
                if (blk >= 0 && t < L) {
                    kp = phys_page(g, v.page_table, s, t);
                    rw = t % g.pt;
                    if (kp < 0) { set_status(v.status, QWFN_STATUS_PAGE_RANGE); rw = -1; }
                }
            }
            sh.kpage[tid] = kp;
            sh.row[tid] = rw;
        }
        __syncthreads();
        // issue every global load of the tile before any use
        constexpr int PER = (64 * C::CH + C::NT - 1) / C::NT;
        uint4 kq[PER], vq[PER];
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int k = tid + i * C::NT;
            kq[i] = make_uint4(0, 0, 0, 0);
            vq[i] = make_uint4(0, 0, 0, 0);
            if (k < 64 * C::CH) {
                const int cell = k % 64, ch = k / 64, rw = sh.row[cell];
                if (rw >= 0) {
                    const int64_t off = (int64_t)sh.kpage[cell] * g.page_bytes +
                                        ((int64_t)(gh * (g.pt / 64) + rw / 64) * C::CH + ch) * 1024 +
                                        (rw % 64) * 16;
                    kq[i] = *reinterpret_cast<const uint4 *>((const uint8_t *)v.k_pages + off);
                    vq[i] = *reinterpret_cast<const uint4 *>((const uint8_t *)v.v_pages + off);
                }
            }
        }
        for (int k = tid; k < 128; k += C::NT) {
            const int cell = k % 64, rw = sh.row[cell];
            const bool isv = k >= 64;
            uint16_t *dst = isv ? sh.vsc[cell] : sh.ksc[cell];
            if (rw >= 0) {
                const uint8_t *base = (const uint8_t *)(isv ? v.v_pages : v.k_pages) +
                                      (int64_t)sh.kpage[cell] * g.page_bytes +
                                      g.qbytes + ((int64_t)(gh * g.pt + rw) * (HD / 32)) * 2;
#pragma unroll
                for (int jj = 0; jj < HD / 32; ++jj) dst[jj] = reinterpret_cast<const uint16_t *>(base)[jj];
            } else {
#pragma unroll
                for (int jj = 0; jj < HD / 32; ++jj) dst[jj] = 0;
            }
        }
        __syncthreads();
        // dequantize K into LDS (exact: fp16 scale times int8)
        auto dequant = [&](const uint4 *qv, uint16_t (*scl)[HD / 32]) {
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int k = tid + i * C::NT;
                if (k < 64 * C::CH) {
                    const int cell = k % 64, ch = k / 64;
                    const float sc = h2f(scl[cell][ch / 2]);
                    const uint32_t w[4] = {qv[i].x, qv[i].y, qv[i].z, qv[i].w};
                    float *dst = &sh.kv[cell * C::ROWF + ch * 16];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        float4 f;
                        f.x = sc * (float)(int8_t)(w[u] & 0xFF);
                        f.y = sc * (float)(int8_t)((w[u] >> 8) & 0xFF);
                        f.z = sc * (float)(int8_t)((w[u] >> 16) & 0xFF);
                        f.w = sc * (float)(int8_t)(w[u] >> 24);
                        *reinterpret_cast<float4 *>(dst + 4 * u) = f;
                    }
                }
            }
        };
        dequant(kq, sh.ksc);
        __syncthreads();
        // QK: lane = cell, wave w owns heads [w*HPW, (w+1)*HPW)
        const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
        const int h0 = w * C::HPW;
        const float *qg = q + ((int64_t)s * g.H + (int64_t)gh * G + h0) * HD;
        float sacc[C::HPW];
#pragma unroll
        for (int hh = 0; hh < C::HPW; ++hh) sacc[hh] = 0.0f;
        const float *krow = &sh.kv[lane * C::ROWF];
#pragma unroll 8
        for (int d4 = 0; d4 < HD / 4; ++d4) {
            const float4 kf = *reinterpret_cast<const float4 *>(krow + 4 * d4);
#pragma unroll
            for (int hh = 0; hh < C::HPW; ++hh) {
                const float4 qv = *reinterpret_cast<const float4 *>(qg + hh * HD + 4 * d4);
                sacc[hh] += qv.x * kf.x + qv.y * kf.y + qv.z * kf.z + qv.w * kf.w;
            }
        }
        const bool valid = sh.row[lane] >= 0;
        float m_h[C::HPW], l_h[C::HPW];
#pragma unroll
        for (int hh = 0; hh < C::HPW; ++hh) {
            const float s2 = valid ? sacc[hh] * g.scale_log2 : -INFINITY;
            const float m = wave_max(s2);
            const float p = valid ? exp2f(s2 - m) : 0.0f;
            m_h[hh] = m;
            l_h[hh] = wave_sum(p);
            sh.p[h0 + hh][lane] = p;
        }
        __syncthreads();                          // K reads done, p visible
        dequant(vq, sh.vsc);
        __syncthreads();
        // PV: lane owns DPL consecutive dims of each of the wave's heads
        float o[C::HPW][C::DPL];
#pragma unroll
        for (int hh = 0; hh < C::HPW; ++hh)
#pragma unroll
            for (int k = 0; k < C::DPL; ++k) o[hh][k] = 0.0f;
#pragma unroll 4
        for (int cell = 0; cell < 64; ++cell) {
            float vv[C::DPL];
#pragma unroll
            for (int k = 0; k < C::DPL; ++k) vv[k] = sh.kv[cell * C::ROWF + lane * C::DPL + k];
#pragma unroll
            for (int hh = 0; hh < C::HPW; ++hh) {
                const float p = sh.p[h0 + hh][cell];
#pragma unroll
                for (int k = 0; k < C::DPL; ++k) o[hh][k] += p * vv[k];
            }
        }
        const int64_t tb = ((int64_t)pair * n_tiles + tile) * G;
#pragma unroll
        for (int hh = 0; hh < C::HPW; ++hh) {
#pragma unroll
            for (int k = 0; k < C::DPL; ++k)
                ws.part_o[(tb + h0 + hh) * HD + lane * C::DPL + k] = o[hh][k];
            if (lane == 0) {
                ws.part_ml[(tb + h0 + hh) * 2 + 0] = m_h[hh];
                ws.part_ml[(tb + h0 + hh) * 2 + 1] = l_h[hh];
            }
        }
    }
    // completion count; the last workgroup of the pair merges
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const int old = atomicAdd(&ws.cnt_attn[pair], 1);
        sh.flag = (old == (int)gridDim.x - 1);
    }
    __syncthreads();
    if (!sh.flag) return;
    __threadfence();
    if (tid == 0) ws.cnt_attn[pair] = 0;
    float *og = out + ((int64_t)s * g.H + (int64_t)gh * G) * HD;
    if (!ok || tiles_act == 0) {
        for (int i = tid; i < G * HD; i += C::NT) og[i] = 0.0f;
        if (!ok && tid == 0 && gh == 0) set_status(v.status, QWFN_STATUS_LEN_RANGE);
        return;
    }
    // merge: M = max_i m_i, w_i = exp2(m_i - M), O = sum_i w_i O_i / sum_i w_i l_i,
    // the weights staged through LDS (the kv tile) one chunk of tiles at a time
    const int64_t pb = (int64_t)pair * n_tiles * G;
    if (tid < G) {
        float M = -INFINITY;
        for (int i = 0; i < tiles_act; ++i) M = fmaxf(M, ws.part_ml[(pb + (int64_t)i * G + tid) * 2]);
        sh.Mh[tid] = M;
        sh.Lh[tid] = 0.0f;
    }
    __syncthreads();
    constexpr int CHK = (64 * C::ROWF) / G;
    constexpr int OPT = (G * HD + C::NT - 1) / C::NT;
    float *wts = sh.kv;
    float acc[OPT];
#pragma unroll
    for (int r = 0; r < OPT; ++r) acc[r] = 0.0f;
    for (int i0 = 0; i0 < tiles_act; i0 += CHK) {
        const int ni = min(CHK, tiles_act - i0);
        for (int k = tid; k < ni * G; k += C::NT) {
            const int h = k % G;
            const float m = ws.part_ml[(pb + (int64_t)(i0 + k / G) * G + h) * 2];
            wts[k] = (m == -INFINITY) ? 0.0f : exp2f(m - sh.Mh[h]);
        }
        __syncthreads();
        if (tid < G) {
            float Ls = sh.Lh[tid];
            for (int i = 0; i < ni; ++i)
                Ls += wts[i * G + tid] * ws.part_ml[(pb + (int64_t)(i0 + i) * G + tid) * 2 + 1];
            sh.Lh[tid] = Ls;
        }
#pragma unroll
        for (int r = 0; r < OPT; ++r) {
            const int k = tid + r * C::NT;
            if (k < G * HD) {
                const int h = k / HD, d = k % HD;
                for (int i = 0; i < ni; ++i)
                    acc[r] += wts[i * G + h] * ws.part_o[(pb + (int64_t)(i0 + i) * G + h) * HD + d];
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < OPT; ++r) {
        const int k = tid + r * C::NT;
        if (k < G * HD) {
            const float Ls = sh.Lh[k / HD];
            og[k] = Ls > 0.0f ? acc[r] / Ls : 0.0f;
        }
    }
}

template <int HD, int G>
static void launch_attn_t(const Geo &g, const qwfn_kv_view &v, const float *q,
                          const int32_t *seq_len, int32_t n_seq, int32_t max_seq_len,
                          const int32_t *sel, const int32_t *nsel, int32_t max_sel, float *out,
                          const Ws &ws, hipStream_t st) {
    const dim3 grid((unsigned)ws.n_tiles, (unsigned)g.Hkv, (unsigned)n_seq);
    hipLaunchKernelGGL((k_attn<HD, G>), grid, dim3(AttnCfg<HD, G>::NT), 0, st, g, v, q, seq_len,
                       max_seq_len, sel, nsel, max_sel, out, ws, ws.n_tiles);
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
    v_out[o] = member_k(g, (const uint8_t *)v.v_pages + (int64_t)pp * g.page_bytes, gh, rw, d);
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
// dispatch over the instantiated (head_dim, group) pairs
// ---------------------------------------------------------------------------

#define QWFN_FOR_EACH_SHAPE(X) X(128, 8) X(128, 4) X(128, 2) X(64, 8) X(256, 12) X(256, 8)

bool kernels_for(int32_t hd, int32_t G) {
#define X(HD_, G_) if (hd == HD_ && G == G_) return true;
    QWFN_FOR_EACH_SHAPE(X)
#undef X
    return false;
}

hipError_t launch_indexer(const Geo &g, const qwfn_kv_view &v, const float *q,
                          const int32_t *seq_len, int32_t n_seq, int32_t max_seq_len,
                          int32_t *sel, int32_t *nsel, int32_t max_sel, const Ws &ws,
                          const FusedAppend &fa, hipStream_t st) {
    switch (g.G) {
    case 2:  launch_indexer_g<2>(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel, ws, fa, st); break;
    case 4:  launch_indexer_g<4>(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel, ws, fa, st); break;
    case 8:  launch_indexer_g<8>(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel, ws, fa, st); break;
    case 12: launch_indexer_g<12>(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel, ws, fa, st); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_attention(const Geo &g, const qwfn_kv_view &v, const float *q,
                            const int32_t *seq_len, int32_t n_seq, int32_t max_seq_len,
                            const int32_t *sel, const int32_t *nsel, int32_t max_sel,
                            float *out, const Ws &ws, hipStream_t st) {
#define X(HD_, G_)                                                                              \
    if (g.hd == HD_ && g.G == G_) {                                                             \
        launch_attn_t<HD_, G_>(g, v, q, seq_len, n_seq, max_seq_len, sel, nsel, max_sel, out, ws, st); \
        return hipGetLastError();                                                               \
    }
    QWFN_FOR_EACH_SHAPE(X)
#undef X
    return hipErrorInvalidValue;
}

}  // namespace qwfn_qsa
