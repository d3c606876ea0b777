// qsa_device.h -- device helpers shared by the gfx950 kernel sources.
#pragma once

#include <hip/hip_runtime.h>
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

}  // namespace qwfn_qsa
