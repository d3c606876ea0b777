// qsa_device.h -- device helpers shared by the gfx950 kernel sources.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "qsa_internal.h"

namespace qwfn_qsa {

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
// fp32 -> fp16, round to nearest even
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

__device__ __forceinline__ void set_status(int32_t *st, int32_t bits) {
    if (st) atomicOr(st, bits);
}

// Physical page of (seq, t) or -1.  Caller has range-checked seq and t.
__device__ __forceinline__ int32_t phys_page(const Geo &g, const int32_t *pt, int seq, int t) {
    const int32_t p = pt[(int64_t)seq * g.pps + t / g.pt];
    return (p >= 0 && p < g.n_phys) ? p : -1;
}


// ---------------------------------------------------------------------------
// page layout, score keys, wave reductions and buffer loads
// ---------------------------------------------------------------------------

// Byte offsets inside a page (layout in include/qwfn_qsa.h).
__device__ __forceinline__ int64_t quant_off(const Geo &g, int gh, int row, int d) {
    return ((int64_t)(gh * (g.pt / 64) + row / 64) * (g.hd / 16) + d / 16) * 1024 +
           (row % 64) * 16 + d % 16;
}
// V quants when the block size is a multiple of 64: per 64-token tile, each
// dimension's 64 cells are contiguous, so a lane owning a dimension reads its
// cells with wide loads for the dot2 products of the attention.
__device__ __forceinline__ int64_t vquant_off(const Geo &g, int gh, int row, int d) {
    return ((int64_t)(gh * (g.pt / 64) + row / 64) * g.hd + d) * 64 + row % 64;
}
__device__ __forceinline__ int64_t scale_off(const Geo &g, int gh, int row, int j) {
    return g.qbytes + ((int64_t)(gh * g.pt + row) * (g.hd / 32) + j) * 2;
}
// 16-byte chunk c of KV head gh's row `row` (the K layout, every element
// type; q8_0 chunks hold 16 dims, q4_0 chunks one ggml block's 16 qs bytes,
// fp16 chunks 8 dims).
__device__ __forceinline__ int64_t chunk_off(const Geo &g, int gh, int row, int c) {
    return ((int64_t)(gh * (g.pt / 64) + row / 64) * g.chunks + c) * 1024 + (row % 64) * 16;
}

// Cache sequence and length of launch sequence s (prefill: query s of one
// cache sequence, see Geo::pf).  `raw` is seq_len[s] as loaded.
__device__ __forceinline__ int cache_seq(const Geo &g, int s) { return g.pf ? g.pf_seq : s; }
__device__ __forceinline__ int seq_length(const Geo &g, int raw, int s) { return g.pf ? g.pf_pos0 + s + 1 : raw; }

__device__ __forceinline__ int8_t to_i8(float r) {
    if (r != r) return 0;
    if (r > 127.0f) return 127;
    if (r < -128.0f) return -128;
    return (int8_t)(int)r;
}

// Orderable key of a score: larger key = larger score; NaN lowest; -0 == +0.
__device__ __forceinline__ uint32_t score_key(float x) {
    const uint32_t u = __float_as_uint(x);
    uint32_t k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    k = x == 0.0f ? 0x80000000u : k;               // -0 == +0
    return x != x ? 0u : k;                        // NaN lowest
}

// Cross-lane steps on the DPP network (gfx9 encodings): a wave64 reduction
// is quad xor-1, quad xor-2, half-row mirror, row mirror, then row_bcast:15
// into rows 1/3 and row_bcast:31 into rows 2/3, leaving the total in lane 63;
// no LDS traffic, unlike ds_bpermute shuffles.
template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf, bool BOUND_ZERO = false>
__device__ __forceinline__ float dppf(float old, float src) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                                 __builtin_bit_cast(int, src), CTRL,
                                                                 ROW_MASK, BANK_MASK, BOUND_ZERO));
}
template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf, bool BOUND_ZERO = false>
__device__ __forceinline__ int dppi(int old, int src) {
    return __builtin_amdgcn_update_dpp(old, src, CTRL, ROW_MASK, BANK_MASK, BOUND_ZERO);
}
constexpr int kDppQuadXor1 = 0xB1, kDppQuadXor2 = 0x4E, kDppRowHalfMirror = 0x141, kDppRowMirror = 0x140;
constexpr int kDppRowShr = 0x110, kDppRowBcast15 = 0x142, kDppRowBcast31 = 0x143;
constexpr int kDppRowRor8 = 0x128;   // lane l of a 16-lane row takes lane l ^ 8's value

__device__ __forceinline__ float lane63(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Raw buffer loads: one descriptor per array, a per-lane byte offset and a
// uniform (SGPR) byte offset, so a run of loads costs one instruction each
// with no 64-bit address arithmetic.  Offsets at or past `bytes` read 0.
using BufRsrc = __amdgpu_buffer_rsrc_t;
__device__ __forceinline__ BufRsrc buf_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
// Cache policy of a load that must see other workgroups' released stores
// without an L2 invalidate: sc1, the agent-scope coherent load.
constexpr int kCpolSc1 = 16;
template <int VW, int CP = 0> struct BufLoad;
template <int CP> struct BufLoad<1, CP> {
    using T = float __attribute__((ext_vector_type(1)));
    static __device__ __forceinline__ T at(BufRsrc r, int voff, int soff) {
        T v; v[0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, CP)); return v;
    }
};
template <int CP> struct BufLoad<2, CP> {
    using T = float __attribute__((ext_vector_type(2)));
    static __device__ __forceinline__ T at(BufRsrc r, int voff, int soff) {
        return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, CP));
    }
};
template <int CP> struct BufLoad<4, CP> {
    using T = float __attribute__((ext_vector_type(4)));
    static __device__ __forceinline__ T at(BufRsrc r, int voff, int soff) {
        return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, CP));
    }
};

// Maximum over the wave, returned to every lane.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dppf<kDppQuadXor1>(v, v));
    v = fmaxf(v, dppf<kDppQuadXor2>(v, v));
    v = fmaxf(v, dppf<kDppRowHalfMirror>(v, v));
    v = fmaxf(v, dppf<kDppRowMirror>(v, v));
    v = fmaxf(v, dppf<kDppRowBcast15, 0xa>(v, v));
    v = fmaxf(v, dppf<kDppRowBcast31, 0xc>(v, v));
    return lane63(v);
}

// Sum over the wave, returned to every lane.
__device__ __forceinline__ float wave_sum(float v) {
    v += dppf<kDppQuadXor1>(0.0f, v);
    v += dppf<kDppQuadXor2>(0.0f, v);
    v += dppf<kDppRowHalfMirror>(0.0f, v);
    v += dppf<kDppRowMirror>(0.0f, v);
    v += dppf<kDppRowBcast15, 0xa>(0.0f, v);
    v += dppf<kDppRowBcast31, 0xc>(0.0f, v);
    return lane63(v);
}

// Inclusive prefix sum over the wave (Hillis-Steele inside each 16-lane row,
// then the row totals broadcast forward).
__device__ __forceinline__ int wave_incl_scan(int x) {
    x += dppi<kDppRowShr + 1, 0xf, 0xf, true>(0, x);
    x += dppi<kDppRowShr + 2, 0xf, 0xf, true>(0, x);
    x += dppi<kDppRowShr + 4, 0xf, 0xf, true>(0, x);
    x += dppi<kDppRowShr + 8, 0xf, 0xf, true>(0, x);
    x += dppi<kDppRowBcast15, 0xa>(0, x);
    x += dppi<kDppRowBcast31, 0xc>(0, x);
    return x;
}

// ---------------------------------------------------------------------------
// selection ranges
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

// Eligible blocks kept: top_k_blocks, less the forced ones (sink + window)
// when the count includes them.  Only meaningful past the short-context case
// (e_hi > e_lo, so the window starts after the sink blocks).
__device__ __forceinline__ int eff_topk(const Geo &g, const Ranges &r) {
    if (!g.keep_total) return g.topk;
    const int k = g.topk - g.sink - (r.b_last - r.fw + 1);
    return k > 0 ? k : 0;
}

// ---------------------------------------------------------------------------
// matrix-core operand types and helpers
// ---------------------------------------------------------------------------

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));
typedef int32_t i4v __attribute__((ext_vector_type(4)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));   // plain 16-byte load/store (no struct copy)

// Sum / max over the lanes l, l^16, l^32, l^48 (the four k-groups of one MFMA
// column), by the gfx950 row swaps: v_permlane32_swap pairs lane l with l^32
// and v_permlane16_swap pairs row 2r with 2r+1; both results are symmetric, so
// every lane of the column ends with the same value.
__device__ __forceinline__ unsigned opaque_copy(unsigned x) {
    unsigned y;
    asm volatile("v_mov_b32 %0, %1" : "=v"(y) : "v"(x));
    return y;
}
// Lane l with lane l ^ 32 (permlane32) or l ^ 16 (permlane16), combined by op.
// The swap gets two registers the compiler cannot prove equal: given one value
// twice it would take the two results as equal and keep only the first.
template <typename Op>
__device__ __forceinline__ float swap32_op(float v, Op op) {
    const unsigned b = __builtin_bit_cast(unsigned, v);
    const auto r = __builtin_amdgcn_permlane32_swap(b, opaque_copy(b), false, false);
    const unsigned r0 = r[0], r1 = r[1];                  // (bit_cast of r[i] reads element 0)
    return op(__builtin_bit_cast(float, r0), __builtin_bit_cast(float, r1));
}
template <typename Op>
__device__ __forceinline__ float swap16_op(float v, Op op) {
    const unsigned b = __builtin_bit_cast(unsigned, v);
    const auto r = __builtin_amdgcn_permlane16_swap(b, opaque_copy(b), false, false);
    const unsigned r0 = r[0], r1 = r[1];
    return op(__builtin_bit_cast(float, r0), __builtin_bit_cast(float, r1));
}
__device__ __forceinline__ float col_sum4(float v) {
    const auto add = [](float a, float b) { return a + b; };
    return swap16_op(swap32_op(v, add), add);
}
__device__ __forceinline__ float col_max4(float v) {
    const auto mx = [](float a, float b) { return fmaxf(a, b); };
    return swap16_op(swap32_op(v, mx), mx);
}

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// Four int8 quants of consecutive cells -> two exact fp16 pairs: bias to
// unsigned, splice under the fp16 exponent of 1024, subtract 1152.
__device__ __forceinline__ void q8x4_to_h2(uint32_t w, half2v &lo, half2v &hi) {
    const uint32_t u = w ^ 0x80808080u;
    const half2v bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    lo = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) + bias;
    hi = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) + bias;
}


// Two weights times their V scales as exact fp16 pairs: hi = f16(p * dv), lo
// = f16(p * dv - hi) (the fma's exact residual), packed two to a word (the
// second weight's in the high halves).  Each dv is the low (SEL 0) or high
// (SEL 1) half of its scale word; the mix instructions read the packed
// halves in place (op_sel), four instructions for the two pairs.
template <int SEL>
__device__ __forceinline__ void p_split2(float p0, uint32_t d0, float p1, uint32_t d1, uint32_t &hi, uint32_t &lo) {
    if constexpr (SEL == 0) {
        asm("v_fma_mixlo_f16 %0, %1, %2, 0 op_sel_hi:[0,1,0]" : "=v"(hi) : "v"(p0), "v"(d0));
        asm("v_fma_mixlo_f16 %0, %1, %2, -%3 op_sel_hi:[0,1,1]" : "=v"(lo) : "v"(p0), "v"(d0), "v"(hi));
        asm("v_fma_mixhi_f16 %0, %1, %2, 0 op_sel_hi:[0,1,0]" : "+v"(hi) : "v"(p1), "v"(d1));
        asm("v_fma_mixhi_f16 %0, %1, %2, -%3 op_sel:[0,0,1] op_sel_hi:[0,1,1]" : "+v"(lo) : "v"(p1), "v"(d1), "v"(hi));
    } else {
        asm("v_fma_mixlo_f16 %0, %1, %2, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "=v"(hi) : "v"(p0), "v"(d0));
        asm("v_fma_mixlo_f16 %0, %1, %2, -%3 op_sel:[0,1,0] op_sel_hi:[0,1,1]" : "=v"(lo) : "v"(p0), "v"(d0), "v"(hi));
        asm("v_fma_mixhi_f16 %0, %1, %2, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "+v"(hi) : "v"(p1), "v"(d1));
        asm("v_fma_mixhi_f16 %0, %1, %2, -%3 op_sel:[0,1,1] op_sel_hi:[0,1,1]" : "+v"(lo) : "v"(p1), "v"(d1), "v"(hi));
    }
}

// Eight int8 quants -> eight exact fp16 values, in order.
__device__ __forceinline__ h8v q8x8_to_h8(uint2 w) {
    half2v a, b, c, d;
    q8x4_to_h2(w.x, a, b);
    q8x4_to_h2(w.y, c, d);
    h8v r;
    r[0] = a[0]; r[1] = a[1]; r[2] = b[0]; r[3] = b[1];
    r[4] = c[0]; r[5] = c[1]; r[6] = d[0]; r[7] = d[1];
    return r;
}

// One 16-byte global -> LDS transfer per lane (global_load_lds_dwordx4): lane
// l's 16 bytes land at LDS byte address lds + 16 l.  Issued from asm so the
// compiler adds no wait of its own; the caller waits with wait_vmem_all()
// before reading the destination.  m0 (the LDS base operand) is restored.
__device__ __forceinline__ void lds_dma16(const void *gsrc, uint32_t lds) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "v"(gsrc), "s"(lds)
                 : "memory");
}
// The same transfer from a wave-uniform base (an SGPR pair) plus a 32-bit
// per-lane byte offset: no 64-bit address arithmetic in the lanes.
__device__ __forceinline__ void lds_dma16_sv(const void *sbase, uint32_t voff, uint32_t lds) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\tglobal_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "v"(voff), "s"(sbase), "s"(lds)
                 : "memory");
}

__device__ __forceinline__ void wait_vmem_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Wait until at most N of the wave's vector-memory operations are in flight
// (loads retire in issue order, so the oldest have landed); asm so that no
// memory access is moved across it.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is six bits");
    asm volatile("s_waitcnt vmcnt(%0)" ::"I"(N) : "memory");
}

// Matrix-core operand layouts (v_mfma_*_16x16x32_*, wave64), lane l = 16*lg + hn:
//   A: row hn, k = 8*lg .. 8*lg+7;  B: column hn, k = 8*lg .. 8*lg+7;
//   D: rows 4*lg .. 4*lg+3, column hn.

}  // namespace qwfn_qsa
