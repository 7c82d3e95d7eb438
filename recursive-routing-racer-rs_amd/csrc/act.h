// act.h -- activation sources shared by the GEMV kernels: how a GEMV builds
// its activation vector (plain, RMS-normalised, silu-gated, GQA-gathered),
// and the RoPE + f16 KV-cache store shared by rope_kv_store_kernel and the
// QKV GEMV's fused epilogue.
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

__device__ __forceinline__ uint32_t f16_bits(float v) { return __builtin_bit_cast(uint16_t, (_Float16)v); }

// apply_rope_cfg (phi4.rs:238-256) in f32, pair j of a head at position
// pos: the coefficients (cos and sin of the angle, scaled by attn_factor)
// and the rotation, applied in that order.
__device__ __forceinline__ void rope_coef(uint32_t j, uint32_t pos, const RopeArgs &r, float &cs, float &ss)
{
    const float base_freq = 1.0f / powf(r.theta, 2.0f * (float)j / (float)r.rope_dim);
    const float factor = j < r.n_factors ? r.factors[j] : 1.0f;
    const float freq = base_freq / factor;
    const float angle = (float)pos * freq;
    float sin_t, cos_t;
    sincosf(angle, &sin_t, &cos_t);
    cs = cos_t * r.attn_factor;
    ss = sin_t * r.attn_factor;
}

__device__ __forceinline__ void rope_rotate(float &x0, float &x1, float cs, float ss)
{
    const float a = x0, b = x1;
    x0 = a * cs - b * ss;
    x1 = a * ss + b * cs;
}

// rope_kv_store (rope_kv_store_kernel, attn.hip) of the qkv row pair (row,
// row + 1), row even, as the GEMV stores it: Q and K pairs in their heads'
// first rope_dim dims rotated (coefficients of pair j at coef[2j], coef[2j+1],
// from rope_coef at the launch's position), every value stored to y, the K
// and V pairs also as f16 into cache row pos.
__device__ __forceinline__ void rope_store_pair(const GemvArgs &a, uint32_t row, float v0, float v1,
                                                const float *coef)
{
    const RopeArgs &r = a.rope;
    if (row < r.q_dim) {
        if (row < r.n_heads * r.head_dim && row % r.head_dim < r.rope_dim) {
            const uint32_t j = (row % r.head_dim) / 2;
            rope_rotate(v0, v1, coef[2 * j], coef[2 * j + 1]);
        }
    } else if (row < r.q_dim + r.kv_stride) {
        const uint32_t e = row - r.q_dim;
        const uint32_t d = r.rope_dim ? e % r.head_dim : 0u;
        if (d < r.rope_dim) rope_rotate(v0, v1, coef[d], coef[d + 1]);
        a.kc[((size_t)r.pos * r.kv_stride + e) / 2] = f16_bits(v0) | (f16_bits(v1) << 16);
    } else {
        const uint32_t e = row - r.q_dim - r.kv_stride;
        a.vc[((size_t)r.pos * r.kv_stride + e) / 2] = f16_bits(v0) | (f16_bits(v1) << 16);
    }
    a.y[row] = v0;
    a.y[row + 1] = v1;
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
