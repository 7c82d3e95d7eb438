// gemv_mfma.hip -- batch-1 K-quant GEMV on the int8 matrix cores.
//
// y[n] = sum_k x[k] * W[n][k] for Q4_K / Q5_K / Q6_K rows (phi4.rs:628-630),
// with the multiply-accumulate on v_mfma_i32_16x16x64_i8 instead of VALU FMAs.
//
// Activation encoding.  Each 16-element group of x is written in block
// floating point with three signed int8 digits per element:
//     x ~= 2^E * (d0 + d1 / 128 + d2 / 16384),  |d_t| <= 64,
// where 2^E is chosen from the group maximum M so that M / 2^E lies in
// [32, 64).  Every step (scale by 2^-E, round, subtract, scale by 128) is
// exact in f32, so the encoding error is at most 2^(E-15) per element, i.e.
// below 2^-20 of the group maximum.
//
// Weights.  A K-quant super-block stores small integers q (Q4_K 0..15,
// Q5_K 0..31, Q6_K 0..63 with an offset of 32) and per-sub-block f32 scales.
// The raw q bytes go straight into the MFMA B operand; the integer dot
// products C_t = sum q * d_t (t = 0, 1, 2) are exact, and
//     sum_k q_k x_k = 2^(E-14) * (C_0 * 2^14 + C_1 * 2^7 + C_2)
// is recombined in int32 (no overflow: |C_t| < 2^16) and scaled once per
// 16 elements by (sub-block scale) * 2^(E-14).  The Q4_K / Q5_K min term
// uses the f32 16-element sums of x; the Q6_K offset uses the digit sums.
//
// MFMA mapping (16x16x64, lane l: A row l%16, B column l%16, k-group l/16;
// D rows 4*(l/16)+r of column l%16 in register r):
//   B[k][n]  = q of weight row n (16 rows per workgroup) at k-set K_g,
//   A[m][k]  = digit (m%4) of x at K_g when m/4 == g (and m%4 < 3), else 0,
// so lane (n, g) receives its own three partial dot products C_0..C_2 for row
// n and k-set K_g in registers 0..2.  Each lane's k-set is 16 consecutive
// elements with one scale, so the scale is applied per lane after the MFMA.
//
// Work split: one workgroup per 16-row tile; its W waves take super-blocks
// b = w, w + W, ... (split K) and issue all their weight loads before the
// activation staging; the per-wave partials are added in wave order.
#include "act.h"

namespace rrr {

// Q4_K (phi4.rs:481-510).  Lane group g takes qs pair g (bytes 32g..32g+31):
// low nibbles = sub-block 2g, high nibbles = sub-block 2g+1.
//   u = 0: low nibbles of bytes 0..15   (k-set 64g + 0..15)
//   u = 1: low nibbles of bytes 16..31  (64g + 16..31)
//   u = 2: high nibbles of bytes 0..15  (64g + 32..47)
//   u = 3: high nibbles of bytes 16..31 (64g + 48..63)
struct MqQ4K {
    static constexpr uint32_t BS = 144;
    static constexpr bool HAS_MIN = true, OFF32 = false;
    struct Raw { u32x4 hdr, qs0, qs1; };
    __device__ static uint32_t koff(uint32_t g, int u) { return 64 * g + 16 * u; }
    __device__ static void load(Raw &w, __amdgpu_buffer_rsrc_t rs, uint32_t boff, uint32_t g)
    {
        w.hdr = bload16(rs, boff);
        w.qs0 = bload16(rs, boff + 16 + 32 * g);
        w.qs1 = bload16(rs, boff + 32 + 32 * g);
    }
    __device__ static void decode(const Raw &w, uint32_t g, i32x4 *bq, float *sc, float *mn)
    {
        const float d = h2f(w.hdr.x), dmin = h2f(w.hdr.x >> 16);
        uint32_t s0, m0, s1, m1;
        scale_min_k4(2 * g, w.hdr.y, w.hdr.z, w.hdr.w, s0, m0);
        scale_min_k4(2 * g + 1, w.hdr.y, w.hdr.z, w.hdr.w, s1, m1);
        sc[0] = sc[1] = d * (float)s0;
        sc[2] = sc[3] = d * (float)s1;
        mn[0] = mn[1] = dmin * (float)m0;
        mn[2] = mn[3] = dmin * (float)m1;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            bq[0][i] = (int)(w.qs0[i] & 0x0F0F0F0Fu);
            bq[1][i] = (int)(w.qs1[i] & 0x0F0F0F0Fu);
            bq[2][i] = (int)((w.qs0[i] >> 4) & 0x0F0F0F0Fu);
            bq[3][i] = (int)((w.qs1[i] >> 4) & 0x0F0F0F0Fu);
        }
    }
};

// Q5_K (phi4.rs:512-542): Q4_K's nibbles plus bit s of qh[j] as bit 4.
struct MqQ5K {
    static constexpr uint32_t BS = 176;
    static constexpr bool HAS_MIN = true, OFF32 = false;
    struct Raw { u32x4 hdr, qh0, qh1, qs0, qs1; };
    __device__ static uint32_t koff(uint32_t g, int u) { return 64 * g + 16 * u; }
    __device__ static void load(Raw &w, __amdgpu_buffer_rsrc_t rs, uint32_t boff, uint32_t g)
    {
        w.hdr = bload16(rs, boff);
        w.qh0 = bload16(rs, boff + 16);
        w.qh1 = bload16(rs, boff + 32);
        w.qs0 = bload16(rs, boff + 48 + 32 * g);
        w.qs1 = bload16(rs, boff + 64 + 32 * g);
    }
    __device__ static void decode(const Raw &w, uint32_t g, i32x4 *bq, float *sc, float *mn)
    {
        const float d = h2f(w.hdr.x), dmin = h2f(w.hdr.x >> 16);
        uint32_t s0, m0, s1, m1;
        scale_min_k4(2 * g, w.hdr.y, w.hdr.z, w.hdr.w, s0, m0);
        scale_min_k4(2 * g + 1, w.hdr.y, w.hdr.z, w.hdr.w, s1, m1);
        sc[0] = sc[1] = d * (float)s0;
        sc[2] = sc[3] = d * (float)s1;
        mn[0] = mn[1] = dmin * (float)m0;
        mn[2] = mn[3] = dmin * (float)m1;
        const uint32_t lo = 2 * g, hi = 2 * g + 1;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            bq[0][i] = (int)((w.qs0[i] & 0x0F0F0F0Fu) | (((w.qh0[i] >> lo) & 0x01010101u) << 4));
            bq[1][i] = (int)((w.qs1[i] & 0x0F0F0F0Fu) | (((w.qh1[i] >> lo) & 0x01010101u) << 4));
            bq[2][i] = (int)(((w.qs0[i] >> 4) & 0x0F0F0F0Fu) | (((w.qh0[i] >> hi) & 0x01010101u) << 4));
            bq[3][i] = (int)(((w.qs1[i] >> 4) & 0x0F0F0F0Fu) | (((w.qh1[i] >> hi) & 0x01010101u) << 4));
        }
    }
};

// Q6_K (phi4.rs:444-479).  Lane group g takes half g6 = g/2 and positions
// l0 = 16 (g&1) .. l0+15; quad u of those positions (elements
// 128 g6 + 32 u + l) is MFMA u and uses scale sc[8 g6 + l0/16 + 2u], the
// is = g*8 + l/16 rule of phi4.rs:463.  Stored values q + 32 (0..63) enter the
// MFMA unsigned; the offset is removed with the digit sums.
struct MqQ6K {
    static constexpr uint32_t BS = 210;
    static constexpr bool HAS_MIN = false, OFF32 = true;
    struct Raw { u32x4 qa, qb, qh; u32x2 sc; uint32_t d; };
    __device__ static uint32_t koff(uint32_t g, int u) { return 128 * (g >> 1) + 32 * u + 16 * (g & 1); }
    __device__ static void load(Raw &w, __amdgpu_buffer_rsrc_t rs, uint32_t boff, uint32_t g)
    {
        const uint32_t g6 = g >> 1, l0 = 16 * (g & 1);
        w.qa = bload16(rs, boff + 64 * g6 + l0);
        w.qb = bload16(rs, boff + 64 * g6 + 32 + l0);
        w.qh = bload16(rs, boff + 128 + 32 * g6 + l0);
        w.sc = __builtin_amdgcn_raw_buffer_load_b64(rs, boff + 192 + 8 * g6, 0, 0);
        w.d = bload2(rs, boff + 208);
    }
    __device__ static void decode(const Raw &w, uint32_t g, i32x4 *bq, float *sc, float *)
    {
        const float d = h2f(w.d);
        const uint32_t h = g & 1;
        sc[0] = d * (float)(int8_t)byte_of(w.sc.x, h);
        sc[1] = d * (float)(int8_t)byte_of(w.sc.x, h + 2);
        sc[2] = d * (float)(int8_t)byte_of(w.sc.y, h);
        sc[3] = d * (float)(int8_t)byte_of(w.sc.y, h + 2);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t a = w.qa[i], b = w.qb[i], hh = w.qh[i];
            bq[0][i] = (int)((a & 0x0F0F0F0Fu) | ((hh & 0x03030303u) << 4));
            bq[1][i] = (int)((b & 0x0F0F0F0Fu) | ((hh & 0x0C0C0C0Cu) << 2));
            bq[2][i] = (int)(((a >> 4) & 0x0F0F0F0Fu) | (hh & 0x30303030u));
            bq[3][i] = (int)(((b >> 4) & 0x0F0F0F0Fu) | ((hh >> 2) & 0x30303030u));
        }
    }
};

// Digits of one float4 of activations: returns the three digit planes packed
// four int8 per dword, and the integer sum of d0*2^14 + d1*2^7 + d2.
__device__ __forceinline__ void encode4(const float4 &v, int e, uint32_t &p0, uint32_t &p1, uint32_t &p2, int &dsum)
{
    const float c[4] = {v.x, v.y, v.z, v.w};
    p0 = p1 = p2 = 0u;
    dsum = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float xs = ldexpf(c[i], -e);
        const float d0 = rintf(xs);
        float r = (xs - d0) * 128.0f;
        const float d1 = rintf(r);
        r = (r - d1) * 128.0f;
        const float d2 = rintf(r);
        const int i0 = (int)d0, i1 = (int)d1, i2 = (int)d2;
        p0 |= ((uint32_t)i0 & 255u) << (8 * i);
        p1 |= ((uint32_t)i1 & 255u) << (8 * i);
        p2 |= ((uint32_t)i2 & 255u) << (8 * i);
        dsum += i0 * 16384 + i1 * 128 + i2;
    }
}

template <class Q, int W, int NBW, int ACT>
__global__ __launch_bounds__(64 * W) void gemv_mq_kernel(GemvArgs a)
{
    extern __shared__ float smem[];
    const uint32_t K = a.K, B = K / 256, NF = K / 4, NG = K / 16;
    constexpr uint32_t NT = 64 * W;                 // threads per workgroup
    constexpr int JF = (NBW * W * 64 + NT - 1) / NT; // activation float4s per thread: K <= W * NBW * 256
    uint8_t *dg = (uint8_t *)smem;                       // 3 digit planes of K bytes + 16 zero bytes
    float *fac = (float *)(dg + 3 * K + 16);             // NG: 2^(E-14) per group
    float *gsum = fac + NG;                              // NG: f32 sums (Q4_K/Q5_K) or int digit sums (Q6_K)
    float *red = gsum + NG;                              // W
    float *part = red + W;                               // W x 16 per-wave row partials

    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint32_t n = lane & 15, g = lane >> 4;
    const uint32_t row0 = blockIdx.x * 16;
    const uint64_t row_bytes = (uint64_t)B * Q::BS;
    const uint64_t wg_off = (uint64_t)row0 * row_bytes;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.W + wg_off, a.w_bytes > wg_off ? a.w_bytes - wg_off : 0);

    // 1. activation inputs (NF is a multiple of 64: each guard is wave-uniform)
    float4 xa[JF], xb[JF];
#pragma unroll
    for (int j = 0; j < JF; j++)
        if (t + NT * j < NF) src_load4<ACT>(a, 4 * (t + NT * j), xa[j], xb[j]);

    // 2. all weight loads of this wave: blocks wave, wave + W, ...
    typename Q::Raw raw[NBW];
#pragma unroll
    for (int i = 0; i < NBW; i++) {
        const uint32_t b = wave + W * i;
        if (b < B) Q::load(raw[i], rs, (uint32_t)(n * row_bytes + (uint64_t)b * Q::BS), g);
    }

    // 3. activation staging: RMSNorm scale, transform, int8 digits
    float inv = 1.0f;
    if constexpr (ACT == ACT_RMSNORM) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < JF; j++)
            if (t + NT * j < NF) {
                acc = __builtin_fmaf(xa[j].x, xa[j].x, acc);
                acc = __builtin_fmaf(xa[j].y, xa[j].y, acc);
                acc = __builtin_fmaf(xa[j].z, xa[j].z, acc);
                acc = __builtin_fmaf(xa[j].w, xa[j].w, acc);
            }
        inv = rms_inv(block_sum_w<W>(acc, red), K, a.eps);
    }
    if (t < 4) ((uint32_t *)(dg + 3 * K))[t] = 0u;
#pragma unroll
    for (int j = 0; j < JF; j++) {
        const uint32_t f = t + NT * j;
        if (f < NF) {
            const float4 v = xform4<ACT>(xa[j], xb[j], inv);
            float mx = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
            mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
            int e = 0;
            if (mx > 0.0f && __builtin_isfinite(mx)) {
                int ex;
                (void)frexpf(mx, &ex);
                e = ex - 6;  // mx / 2^e in [32, 64)
            }
            uint32_t p0, p1, p2;
            int ds;
            encode4(v, e, p0, p1, p2, ds);
            ((uint32_t *)dg)[f] = p0;
            ((uint32_t *)(dg + K))[f] = p1;
            ((uint32_t *)(dg + 2 * K))[f] = p2;
            if constexpr (Q::OFF32) {
                ds = ds + __shfl_xor(ds, 1, 64);
                ds = ds + __shfl_xor(ds, 2, 64);
                if ((t & 3) == 0) ((int *)gsum)[f / 4] = ds;
            } else {
                float sv = (v.x + v.y) + (v.z + v.w);
                sv = sv + __shfl_xor(sv, 1, 64);
                sv = sv + __shfl_xor(sv, 2, 64);
                if ((t & 3) == 0) gsum[f / 4] = sv;
            }
            if ((t & 3) == 0)
                fac[f / 4] = __builtin_isfinite(mx) ? ldexpf(1.0f, e - 14) : __builtin_nanf("");
        }
    }
    __syncthreads();

    // 4. MFMAs: lane (n, g) supplies B = q of row n at k-set K_g and A = its
    // digit row (m = n: plane n%4 of group n/4) when n/4 == g
    const uint32_t m = n;
    const bool a_live = (m >> 2) == g && (m & 3) < 3;
    const uint32_t a_plane = (m & 3) * K;
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < NBW; i++) {
        const uint32_t b = wave + W * i;
        if (b < B) {
            i32x4 bq[4];
            float sc[4], mn[4];
            Q::decode(raw[i], g, bq, sc, mn);
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const uint32_t k0 = b * 256 + Q::koff(g, u);
                const uint32_t aoff = a_live ? a_plane + k0 : 3 * K;
                const i32x4 av = *(const i32x4 *)(dg + aoff);
                i32x4 c = {0, 0, 0, 0};
                c = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i8x16, av), __builtin_bit_cast(i8x16, bq[u]), c,
                                                          0, 0, 0);
                int T = c[0] * 16384 + c[1] * 128 + c[2];
                if constexpr (Q::OFF32) T -= 32 * ((const int *)gsum)[k0 / 16];
                acc = fmaf(sc[u] * fac[k0 / 16], (float)T, acc);
                if constexpr (Q::HAS_MIN) acc = fmaf(-mn[u], gsum[k0 / 16], acc);
            }
        }
    }

    // 5. reduce the 4 k-groups of a row (lanes n, n+16, n+32, n+48), then the
    // W waves in order
    acc = acc + __shfl_xor(acc, 16, 64);
    acc = acc + __shfl_xor(acc, 32, 64);
    if (lane < 16) part[wave * 16 + lane] = acc;
    __syncthreads();
    if (t < 16 && row0 + t < a.N) {
        float v = part[t];
#pragma unroll
        for (int w = 1; w < W; w++) v += part[16 * w + t];
        float *yp = a.y + row0 + t;
        *yp = a.residual ? *yp + v : v;
    }
}

template <class Q, int W, int NBW, int ACT>
static hipError_t go_mq(const GemvArgs &a, hipStream_t s)
{
    const size_t lds = 3 * (size_t)a.K + 16 + 2 * (size_t)(a.K / 16) * 4 + 17 * W * 4;
    hipLaunchKernelGGL((gemv_mq_kernel<Q, W, NBW, ACT>), dim3((a.N + 15) / 16), dim3(64 * W), lds, s, a);
    return hipGetLastError();
}

// Waves per 16-row tile: K is split across W waves (super-blocks w, w + W,
// ...), up to 16 waves so that small matrices still fill the SIMDs.
template <class Q, int ACT>
static hipError_t go_mq_k(const GemvArgs &a, hipStream_t s)
{
    const uint32_t B = a.K / 256;
    if (B <= 4) return go_mq<Q, 4, 1, ACT>(a, s);
    if (B <= 8) return go_mq<Q, 8, 1, ACT>(a, s);
    if (B <= 12) return go_mq<Q, 12, 1, ACT>(a, s);
    if (B <= 16) return go_mq<Q, 16, 1, ACT>(a, s);
    return go_mq<Q, 16, 2, ACT>(a, s);
}

template <class Q>
static hipError_t go_mq_act(const GemvArgs &a, uint32_t act, hipStream_t s)
{
    switch (act) {
    case ACT_PLAIN: return go_mq_k<Q, ACT_PLAIN>(a, s);
    case ACT_SILU: return go_mq_k<Q, ACT_SILU>(a, s);
    case ACT_GQA_V: return go_mq_k<Q, ACT_GQA_V>(a, s);
    case ACT_RMSNORM: return go_mq_k<Q, ACT_RMSNORM>(a, s);
    default: return hipErrorInvalidValue;
    }
}

bool gemv_mfma_supported(const GemvArgs &a)
{
    return a.M == 1 && (a.type == T_Q4_K || a.type == T_Q5_K || a.type == T_Q6_K) && a.K <= 8192;
}

hipError_t launch_gemv_mfma(const GemvArgs &a, uint32_t act, hipStream_t s)
{
    switch (a.type) {
    case T_Q4_K: return go_mq_act<MqQ4K>(a, act, s);
    case T_Q5_K: return go_mq_act<MqQ5K>(a, act, s);
    case T_Q6_K: return go_mq_act<MqQ6K>(a, act, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace rrr
