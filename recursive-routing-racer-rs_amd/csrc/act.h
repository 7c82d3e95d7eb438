// act.h -- activation sources shared by the GEMV kernels: how a GEMV builds
// its activation vector (plain, RMS-normalised, silu-gated, GQA-gathered).
#pragma once

#include "device_common.h"
#include "internal.h"

namespace rrr {

// Raw inputs of the 4 activations starting at k (k % 4 == 0) of a batch-1
// GEMV: x (or the gate / gathered V) in xa, gamma or up in xb.
template <int ACT>
__device__ __forceinline__ void src_load4(const GemvArgs &a, uint32_t k, float4 &xa, float4 &xb)
{
    if constexpr (ACT == ACT_GQA_V) {
        const uint32_t hd = a.head_dim, hpk = a.heads_per_kv;
        xa = *(const float4 *)(a.x + a.K + a.K / hpk + (k / (hd * hpk)) * hd + k % hd);
    } else {
        xa = *(const float4 *)(a.x + k);
    }
    if constexpr (ACT == ACT_RMSNORM) xb = *(const float4 *)(a.gamma + k);
    if constexpr (ACT == ACT_SILU) xb = *(const float4 *)(a.x + a.K + k);
}

template <int ACT>
__device__ __forceinline__ float4 xform4(const float4 &x, const float4 &y, float inv)
{
    if constexpr (ACT == ACT_RMSNORM)
        return make_float4(__fmul_rn(__fmul_rn(y.x, x.x), inv), __fmul_rn(__fmul_rn(y.y, x.y), inv),
                           __fmul_rn(__fmul_rn(y.z, x.z), inv), __fmul_rn(__fmul_rn(y.w, x.w), inv));
    else if constexpr (ACT == ACT_SILU)
        return make_float4(silu_fast(x.x) * y.x, silu_fast(x.y) * y.y, silu_fast(x.z) * y.z, silu_fast(x.w) * y.w);
    else
        return x;
}

}  // namespace rrr
