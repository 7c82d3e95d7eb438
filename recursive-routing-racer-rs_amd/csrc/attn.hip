// attn.hip -- the decode glue around the weight sweep: RoPE with the f16
// KV-cache store (the rope_kv_store / kv_store pipelines, phi4.rs:1016-1017,
// :1666-1677) and decode attention over the cache (the attention pipeline,
// phi4.rs:1018, :1304-1312).
#include "device_common.h"
#include "internal.h"

namespace rrr {

__device__ __forceinline__ uint32_t f16_bits(float v) { return __builtin_bit_cast(uint16_t, (_Float16)v); }

// One rotation of apply_rope_cfg (phi4.rs:238-256) in f32: pair j of a head.
__device__ __forceinline__ void rope_pair(float &x0, float &x1, uint32_t j, const RopeArgs &r)
{
    const float base_freq = 1.0f / powf(r.theta, 2.0f * (float)j / (float)r.rope_dim);
    const float factor = j < r.n_factors ? r.factors[j] : 1.0f;
    const float freq = base_freq / factor;
    const float angle = (float)r.pos * freq;
    float sin_t, cos_t;
    sincosf(angle, &sin_t, &cos_t);
    const float cs = cos_t * r.attn_factor, ss = sin_t * r.attn_factor;
    const float a = x0, b = x1;
    x0 = a * cs - b * ss;
    x1 = a * ss + b * cs;
}

// Threads [0, nq): the Q rotation pairs (head i / (rope_dim/2), pair i %
// (rope_dim/2)), rotated in place.  Threads [nq, nq + kv_stride/2): element
// pair 2p of K (rotated in place when it lies in its head's first rope_dim
// dims) and of V, both stored as f16 into row pos of the caches.
__global__ __launch_bounds__(256) void rope_kv_store_kernel(float *__restrict__ qkv, RopeArgs r, uint32_t *__restrict__ kc,
                                                            uint32_t *__restrict__ vc)
{
    const uint32_t half_rope = r.rope_dim / 2;
    const uint32_t nq = r.n_heads * half_rope, nkv = r.kv_stride / 2;
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < nq) {
        const uint32_t h = i / half_rope, j = i - h * half_rope;
        float *p = qkv + (size_t)h * r.head_dim + 2 * j;
        float x0 = p[0], x1 = p[1];
        rope_pair(x0, x1, j, r);
        p[0] = x0;
        p[1] = x1;
    } else if (i < nq + nkv) {
        const uint32_t e = 2 * (i - nq);
        float *k = qkv + r.q_dim + e;
        const float *v = qkv + r.q_dim + r.kv_stride + e;
        float k0 = k[0], k1 = k[1];
        const uint32_t d = r.rope_dim ? e % r.head_dim : 0u;   // head_dim is 0 in the kv_store form
        if (d < r.rope_dim) {
            rope_pair(k0, k1, d / 2, r);
            k[0] = k0;
            k[1] = k1;
        }
        const size_t w = ((size_t)r.pos * r.kv_stride + e) / 2;
        kc[w] = f16_bits(k0) | (f16_bits(k1) << 16);
        vc[w] = f16_bits(v[0]) | (f16_bits(v[1]) << 16);
    }
}

hipError_t launch_rope_kv_store(float *qkv, const RopeArgs &r, uint16_t *kc, uint16_t *vc, hipStream_t s)
{
    const uint32_t n = r.n_heads * (r.rope_dim / 2) + r.kv_stride / 2;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(rope_kv_store_kernel, dim3((n + 255) / 256), dim3(256), 0, s, qkv, r, (uint32_t *)kc,
                       (uint32_t *)vc);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Decode attention, split over the sequence (flash-decoding).  Workgroup
// (g, sp) takes KV head g and cache rows [sp * per, sp * per + per): its 16
// lane groups of 16 lanes each take every 16th row, lane li owning dims
// 8 li .. 8 li + 7 of the row (one 16-byte f16 load of K and one of V).  The
// HPK query heads of the KV group share every K/V load.  Scores go through
// exp2 with the queries pre-scaled by log2(e) / sqrt(head_dim); each lane
// group keeps a running max, sum and output (online softmax), the 16 groups
// are merged in LDS, and the workgroup writes {output, max, sum} per query
// head; attn_merge_kernel combines the splits.  The row -> lane group and
// split assignment depend on seq_len only, so results are reproducible.
constexpr uint32_t ATT_PART = ATT_HD + 2;   // floats of one split's partial: output, max, sum

template <int HPK>
__global__ __launch_bounds__(256) void attn_split_kernel(const float *__restrict__ q, const uint16_t *__restrict__ kc,
                                                         const uint16_t *__restrict__ vc, float *__restrict__ part,
                                                         uint32_t seq, uint32_t per, uint32_t kv_stride, float qscale)
{
    __shared__ float sm[16][HPK][2];
    __shared__ float so[16][HPK][ATT_HD];
    const uint32_t g = blockIdx.x, sp = blockIdx.y, splits = gridDim.y;
    const uint32_t t = threadIdx.x, grp = t >> 4, li = t & 15;
    const uint32_t r0 = sp * per, r1 = min(seq, r0 + per);

    float qv[HPK][8];
#pragma unroll
    for (int h = 0; h < HPK; h++) {
        const float4 *qp = (const float4 *)(q + (size_t)(g * HPK + h) * ATT_HD + 8 * li);
        const float4 a = qp[0], b = qp[1];
        qv[h][0] = a.x * qscale; qv[h][1] = a.y * qscale; qv[h][2] = a.z * qscale; qv[h][3] = a.w * qscale;
        qv[h][4] = b.x * qscale; qv[h][5] = b.y * qscale; qv[h][6] = b.z * qscale; qv[h][7] = b.w * qscale;
    }
    float m[HPK], l[HPK], o[HPK][8];
#pragma unroll
    for (int h = 0; h < HPK; h++) {
        m[h] = -__builtin_inff();
        l[h] = 0.0f;
#pragma unroll
        for (int d = 0; d < 8; d++) o[h][d] = 0.0f;
    }
    for (uint32_t row = r0 + grp; row < r1; row += 16) {
        const size_t off = (size_t)row * kv_stride + (size_t)g * ATT_HD + 8 * li;
        const u32x4 kr = *(const u32x4 *)(kc + off);
        const u32x4 vr = *(const u32x4 *)(vc + off);
        float k[8], v[8];
#pragma unroll
        for (int w = 0; w < 4; w++) {
            k[2 * w] = h2f(kr[w] & 0xFFFFu);
            k[2 * w + 1] = h2f(kr[w] >> 16);
            v[2 * w] = h2f(vr[w] & 0xFFFFu);
            v[2 * w + 1] = h2f(vr[w] >> 16);
        }
#pragma unroll
        for (int h = 0; h < HPK; h++) {
            float s = 0.0f;
#pragma unroll
            for (int d = 0; d < 8; d++) s = fmaf(qv[h][d], k[d], s);
            s += __shfl_xor(s, 1, 16);
            s += __shfl_xor(s, 2, 16);
            s += __shfl_xor(s, 4, 16);
            s += __shfl_xor(s, 8, 16);
            const float mn = fmaxf(m[h], s);
            const float c = exp2f(m[h] - mn), p = exp2f(s - mn);
            l[h] = fmaf(l[h], c, p);
#pragma unroll
            for (int d = 0; d < 8; d++) o[h][d] = fmaf(o[h][d], c, p * v[d]);
            m[h] = mn;
        }
    }
#pragma unroll
    for (int h = 0; h < HPK; h++) {
        if (li == 0) {
            sm[grp][h][0] = m[h];
            sm[grp][h][1] = l[h];
        }
#pragma unroll
        for (int d = 0; d < 8; d++) so[grp][h][8 * li + d] = o[h][d];
    }
    __syncthreads();
    for (uint32_t i = t; i < HPK * ATT_HD; i += 256) {
        const uint32_t h = i / ATT_HD, d = i % ATT_HD;
        float M = -__builtin_inff();
        for (int gi = 0; gi < 16; gi++) M = fmaxf(M, sm[gi][h][0]);
        float L = 0.0f, O = 0.0f;
        for (int gi = 0; gi < 16; gi++) {
            const float c = exp2f(sm[gi][h][0] - M);   // 0 for a group without rows
            L = fmaf(sm[gi][h][1], c, L);
            O = fmaf(so[gi][h][d], c, O);
        }
        float *dst = part + ((size_t)(g * HPK + h) * splits + sp) * ATT_PART;
        dst[d] = O;
        if (d == 0) {
            dst[ATT_HD] = M;
            dst[ATT_HD + 1] = L;
        }
    }
}

__global__ __launch_bounds__(ATT_HD) void attn_merge_kernel(const float *__restrict__ part, float *__restrict__ out,
                                                            uint32_t splits)
{
    const uint32_t h = blockIdx.x, d = threadIdx.x;
    const float *p = part + (size_t)h * splits * ATT_PART;
    float M = -__builtin_inff();
    for (uint32_t s = 0; s < splits; s++) M = fmaxf(M, p[s * ATT_PART + ATT_HD]);
    float L = 0.0f, O = 0.0f;
    for (uint32_t s = 0; s < splits; s++) {
        const float c = exp2f(p[s * ATT_PART + ATT_HD] - M);
        L = fmaf(p[s * ATT_PART + ATT_HD + 1], c, L);
        O = fmaf(p[s * ATT_PART + d], c, O);
    }
    out[(size_t)h * ATT_HD + d] = O / L;
}

uint64_t attention_partials_bytes() { return (uint64_t)ATT_HEADS_MAX * ATT_SPLITS_MAX * ATT_PART * 4; }

// Rows per split: enough splits for about two workgroups per CU, at least 16
// rows (one per lane group) each, at most ATT_SPLITS_MAX splits.
void attention_plan(uint32_t seq, uint32_t n_kv_heads, uint32_t cus, uint32_t &splits, uint32_t &per)
{
    const uint32_t want = max(1u, min(ATT_SPLITS_MAX, (2 * cus + n_kv_heads - 1) / n_kv_heads));
    splits = max(1u, min(want, (seq + 15) / 16));
    per = (seq + splits - 1) / splits;
    splits = (seq + per - 1) / per;   // every split has at least one row
}

template <int HPK>
static void go_attn(const float *q, const uint16_t *kc, const uint16_t *vc, float *part, uint32_t seq, uint32_t per,
                    uint32_t kv_stride, float qscale, uint32_t n_kv_heads, uint32_t splits, hipStream_t s)
{
    hipLaunchKernelGGL(attn_split_kernel<HPK>, dim3(n_kv_heads, splits), dim3(256), 0, s, q, kc, vc, part, seq, per,
                       kv_stride, qscale);
}

hipError_t launch_attention(const float *q, const uint16_t *kc, const uint16_t *vc, float *out, void *partials,
                            uint32_t seq, uint32_t n_kv_heads, uint32_t heads_per_kv, uint32_t cus, hipStream_t s)
{
    uint32_t splits, per;
    attention_plan(seq, n_kv_heads, cus, splits, per);
    const uint32_t kv_stride = n_kv_heads * ATT_HD;
    const float qscale = (float)(1.4426950408889634 / sqrt((double)ATT_HD));   // log2(e) / sqrt(head_dim)
    float *part = (float *)partials;
    switch (heads_per_kv) {
    case 1: go_attn<1>(q, kc, vc, part, seq, per, kv_stride, qscale, n_kv_heads, splits, s); break;
    case 2: go_attn<2>(q, kc, vc, part, seq, per, kv_stride, qscale, n_kv_heads, splits, s); break;
    case 3: go_attn<3>(q, kc, vc, part, seq, per, kv_stride, qscale, n_kv_heads, splits, s); break;
    case 4: go_attn<4>(q, kc, vc, part, seq, per, kv_stride, qscale, n_kv_heads, splits, s); break;
    case 5: go_attn<5>(q, kc, vc, part, seq, per, kv_stride, qscale, n_kv_heads, splits, s); break;
    case 6: go_attn<6>(q, kc, vc, part, seq, per, kv_stride, qscale, n_kv_heads, splits, s); break;
    case 7: go_attn<7>(q, kc, vc, part, seq, per, kv_stride, qscale, n_kv_heads, splits, s); break;
    case 8: go_attn<8>(q, kc, vc, part, seq, per, kv_stride, qscale, n_kv_heads, splits, s); break;
    default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(attn_merge_kernel, dim3(n_kv_heads * heads_per_kv), dim3(ATT_HD), 0, s, part, out, splits);
    return hipGetLastError();
}

}  // namespace rrr
