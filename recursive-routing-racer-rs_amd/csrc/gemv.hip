// gemv.hip -- fused dequant-in-kernel GEMV / batched GEMV on raw GGUF blocks.
//
// Y[m][n] = sum_k X[m][k] * W[n][k]  (phi4.rs:628-630; batch shape :1257-1268)
//
// Layout: W is the raw GGUF tensor, N rows of K/256 super-blocks, uploaded
// unchanged.  A 256-thread workgroup owns 4*R consecutive rows (R per wave)
// and MT activation rows.  The activation tile is staged once per K-chunk in
// LDS together with its 16-element partial sums; every lane then owns a fixed
// 16-byte slice of each super-block it visits (selected per type below),
// loads it with a bounds-checked buffer load, and multiplies it against the
// matching LDS spans for all R rows and MT tokens.  The per-sub-block scale
// and min are applied once per span:
//     sum_j x_j * (q_j * s - m) = s * sum_j q_j x_j - m * sum_j x_j
// so the inner loop is one conversion and one FMA per element.
#include "device_common.h"
#include "internal.h"

namespace rrr {

// ---------------------------------------------------------------------------
// Per-type lane decoders.  LPB lanes share one super-block, BPI blocks are in
// flight per wave iteration (LPB * BPI == 64).

// Q4_K block (phi4.rs:481-510): {f16 d; f16 dmin; u8 sc[12]; u8 qs[128]}.
// Lane c (0..7) takes qs bytes [16c, 16c+16): pair p = c/2, j0 = 16 (c&1);
// low nibbles are sub-block 2p, high nibbles sub-block 2p+1, positions j0..j0+15.
struct DecQ4K {
    static constexpr uint32_t BS = 144, LPB = 8, BPI = 8;
    struct Raw { u32x4 hdr, qs; };
    uint32_t c, p, j0;
    __device__ explicit DecQ4K(uint32_t lane) : c(lane & 7), p((lane & 7) >> 1), j0((lane & 1) * 16) {}
    __device__ static uint32_t slot(uint32_t lane) { return lane >> 3; }
    __device__ void load(Raw &w, __amdgpu_buffer_rsrc_t rs, uint32_t boff) const
    {
        w.hdr = bload16(rs, boff);
        w.qs = bload16(rs, boff + 16 + 16 * c);
    }
    template <int MT>
    __device__ void accum(const Raw &w, const float *xb, uint32_t xst, const float *gb, uint32_t gst,
                          float *acc) const
    {
        const float d = h2f(w.hdr.x), dmin = h2f(w.hdr.x >> 16);
        uint32_t sc0, mn0, sc1, mn1;
        scale_min_k4(2 * p, w.hdr.y, w.hdr.z, w.hdr.w, sc0, mn0);
        scale_min_k4(2 * p + 1, w.hdr.y, w.hdr.z, w.hdr.w, sc1, mn1);
        const float s0 = d * (float)sc0, n0 = dmin * (float)mn0;
        const float s1 = d * (float)sc1, n1 = dmin * (float)mn1;
        float ql[16], qh[16];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t v = w.qs[i];
            const uint32_t lo = v & 0x0F0F0F0Fu, hi = (v >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                ql[4 * i + b] = (float)byte_of(lo, b);
                qh[4 * i + b] = (float)byte_of(hi, b);
            }
        }
        const uint32_t xo = 64 * p + j0;
#pragma unroll
        for (int m = 0; m < MT; m++) {
            const float4 *xl = (const float4 *)(xb + m * xst + xo);
            const float4 *xh = (const float4 *)(xb + m * xst + xo + 32);
            float dl = 0.0f, dh = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 a = xl[i], b = xh[i];
                dl = fmaf(ql[4 * i + 0], a.x, dl); dl = fmaf(ql[4 * i + 1], a.y, dl);
                dl = fmaf(ql[4 * i + 2], a.z, dl); dl = fmaf(ql[4 * i + 3], a.w, dl);
                dh = fmaf(qh[4 * i + 0], b.x, dh); dh = fmaf(qh[4 * i + 1], b.y, dh);
                dh = fmaf(qh[4 * i + 2], b.z, dh); dh = fmaf(qh[4 * i + 3], b.w, dh);
            }
            const float gl = gb[m * gst + xo / 16], gh = gb[m * gst + xo / 16 + 2];
            float r = acc[m];
            r = fmaf(s0, dl, r); r = fmaf(-n0, gl, r);
            r = fmaf(s1, dh, r); r = fmaf(-n1, gh, r);
            acc[m] = r;
        }
    }
};

// Q5_K block (phi4.rs:512-542): {d; dmin; sc[12]; qh[32]; qs[128]}.
// Same lane split as Q4_K; the fifth bit of position j in sub-block s is bit s
// of qh[j], so the lane also loads qh[j0..j0+15].
struct DecQ5K {
    static constexpr uint32_t BS = 176, LPB = 8, BPI = 8;
    struct Raw { u32x4 hdr, qh, qs; };
    uint32_t c, p, j0;
    __device__ explicit DecQ5K(uint32_t lane) : c(lane & 7), p((lane & 7) >> 1), j0((lane & 1) * 16) {}
    __device__ static uint32_t slot(uint32_t lane) { return lane >> 3; }
    __device__ void load(Raw &w, __amdgpu_buffer_rsrc_t rs, uint32_t boff) const
    {
        w.hdr = bload16(rs, boff);
        w.qh = bload16(rs, boff + 16 + j0);
        w.qs = bload16(rs, boff + 48 + 16 * c);
    }
    template <int MT>
    __device__ void accum(const Raw &w, const float *xb, uint32_t xst, const float *gb, uint32_t gst,
                          float *acc) const
    {
        const float d = h2f(w.hdr.x), dmin = h2f(w.hdr.x >> 16);
        uint32_t sc0, mn0, sc1, mn1;
        scale_min_k4(2 * p, w.hdr.y, w.hdr.z, w.hdr.w, sc0, mn0);
        scale_min_k4(2 * p + 1, w.hdr.y, w.hdr.z, w.hdr.w, sc1, mn1);
        const float s0 = d * (float)sc0, n0 = dmin * (float)mn0;
        const float s1 = d * (float)sc1, n1 = dmin * (float)mn1;
        float ql[16], qh[16];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t v = w.qs[i], h = w.qh[i];
            const uint32_t lo = (v & 0x0F0F0F0Fu) | (((h >> (2 * p)) & 0x01010101u) << 4);
            const uint32_t hi = ((v >> 4) & 0x0F0F0F0Fu) | (((h >> (2 * p + 1)) & 0x01010101u) << 4);
#pragma unroll
            for (int b = 0; b < 4; b++) {
                ql[4 * i + b] = (float)byte_of(lo, b);
                qh[4 * i + b] = (float)byte_of(hi, b);
            }
        }
        const uint32_t xo = 64 * p + j0;
#pragma unroll
        for (int m = 0; m < MT; m++) {
            const float4 *xl = (const float4 *)(xb + m * xst + xo);
            const float4 *xh = (const float4 *)(xb + m * xst + xo + 32);
            float dl = 0.0f, dh = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 a = xl[i], b = xh[i];
                dl = fmaf(ql[4 * i + 0], a.x, dl); dl = fmaf(ql[4 * i + 1], a.y, dl);
                dl = fmaf(ql[4 * i + 2], a.z, dl); dl = fmaf(ql[4 * i + 3], a.w, dl);
                dh = fmaf(qh[4 * i + 0], b.x, dh); dh = fmaf(qh[4 * i + 1], b.y, dh);
                dh = fmaf(qh[4 * i + 2], b.z, dh); dh = fmaf(qh[4 * i + 3], b.w, dh);
            }
            const float gl = gb[m * gst + xo / 16], gh = gb[m * gst + xo / 16 + 2];
            float r = acc[m];
            r = fmaf(s0, dl, r); r = fmaf(-n0, gl, r);
            r = fmaf(s1, dh, r); r = fmaf(-n1, gh, r);
            acc[m] = r;
        }
    }
};

// Q6_K block (phi4.rs:444-479): {ql[128]; qh[64]; i8 sc[16]; f16 d}.
// Lane G (0..3) takes half g = G/2 and positions l0 = 16 (G&1) .. l0+15 of it:
// ql[64g + l0 ..], ql[64g + 32 + l0 ..] and qh[32g + l0 ..], i.e. all four
// quads of those 16 positions.  Element g*128 + 32u + l uses scale
// sc[8g + l/16 + 2u], which is the is = g*8 + l/16 rule of phi4.rs:463.
// Blocks are 210 bytes, so these 16-byte loads are 2-byte aligned.
struct DecQ6K {
    static constexpr uint32_t BS = 210, LPB = 4, BPI = 16;
    struct Raw { u32x4 qa, qb, qh; u32x2 sc; uint32_t d; };
    uint32_t g, l0;
    __device__ explicit DecQ6K(uint32_t lane) : g((lane & 3) >> 1), l0((lane & 1) * 16) {}
    __device__ static uint32_t slot(uint32_t lane) { return lane >> 2; }
    __device__ void load(Raw &w, __amdgpu_buffer_rsrc_t rs, uint32_t boff) const
    {
        w.qa = bload16(rs, boff + 64 * g + l0);
        w.qb = bload16(rs, boff + 64 * g + 32 + l0);
        w.qh = bload16(rs, boff + 128 + 32 * g + l0);
        w.sc = __builtin_amdgcn_raw_buffer_load_b64(rs, boff + 192 + 8 * g, 0, 0);
        w.d = bload2(rs, boff + 208);
    }
    template <int MT>
    __device__ void accum(const Raw &w, const float *xb, uint32_t xst, const float *gb, uint32_t gst,
                          float *acc) const
    {
        const float d = h2f(w.d);
        const uint32_t h = l0 >> 4;
        float ds[4];
        ds[0] = d * (float)(int8_t)byte_of(w.sc.x, h);
        ds[1] = d * (float)(int8_t)byte_of(w.sc.x, h + 2);
        ds[2] = d * (float)(int8_t)byte_of(w.sc.y, h);
        ds[3] = d * (float)(int8_t)byte_of(w.sc.y, h + 2);
        float q[4][16];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t a = w.qa[i], b = w.qb[i], hh = w.qh[i];
            const uint32_t q1 = (a & 0x0F0F0F0Fu) | ((hh & 0x03030303u) << 4);
            const uint32_t q2 = (b & 0x0F0F0F0Fu) | ((hh & 0x0C0C0C0Cu) << 2);
            const uint32_t q3 = ((a >> 4) & 0x0F0F0F0Fu) | (hh & 0x30303030u);
            const uint32_t q4 = ((b >> 4) & 0x0F0F0F0Fu) | ((hh >> 2) & 0x30303030u);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                q[0][4 * i + k] = (float)byte_of(q1, k);
                q[1][4 * i + k] = (float)byte_of(q2, k);
                q[2][4 * i + k] = (float)byte_of(q3, k);
                q[3][4 * i + k] = (float)byte_of(q4, k);
            }
        }
        const uint32_t xo = 128 * g + l0;
#pragma unroll
        for (int m = 0; m < MT; m++) {
            float r = acc[m];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const float4 *xv = (const float4 *)(xb + m * xst + xo + 32 * u);
                float dot = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float4 a = xv[i];
                    dot = fmaf(q[u][4 * i + 0], a.x, dot); dot = fmaf(q[u][4 * i + 1], a.y, dot);
                    dot = fmaf(q[u][4 * i + 2], a.z, dot); dot = fmaf(q[u][4 * i + 3], a.w, dot);
                }
                // stored values are q + 32 (0..63); remove the offset once per span
                dot = fmaf(-32.0f, gb[m * gst + (xo + 32 * u) / 16], dot);
                r = fmaf(ds[u], dot, r);
            }
            acc[m] = r;
        }
    }
};

// F32 rows (matmul_tiled with M=1 on untransposed weights, phi4.rs:641-646,
// and the row-major logits).  A "block" is 256 floats; lane c (0..15) takes
// floats 4c + 64i (i = 0..3) so each load instruction covers contiguous 256 B.
struct DecF32 {
    static constexpr uint32_t BS = 1024, LPB = 16, BPI = 4;
    struct Raw { u32x4 v[4]; };
    uint32_t c;
    __device__ explicit DecF32(uint32_t lane) : c(lane & 15) {}
    __device__ static uint32_t slot(uint32_t lane) { return lane >> 4; }
    __device__ void load(Raw &w, __amdgpu_buffer_rsrc_t rs, uint32_t boff) const
    {
#pragma unroll
        for (int i = 0; i < 4; i++) w.v[i] = bload16(rs, boff + 16 * c + 256 * i);
    }
    template <int MT>
    __device__ void accum(const Raw &w, const float *xb, uint32_t xst, const float *, uint32_t,
                          float *acc) const
    {
#pragma unroll
        for (int m = 0; m < MT; m++) {
            float r = acc[m];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 a = *(const float4 *)(xb + m * xst + 4 * c + 64 * i);
                r = fmaf(u2f(w.v[i].x), a.x, r);
                r = fmaf(u2f(w.v[i].y), a.y, r);
                r = fmaf(u2f(w.v[i].z), a.z, r);
                r = fmaf(u2f(w.v[i].w), a.w, r);
            }
            acc[m] = r;
        }
    }
};

// ---------------------------------------------------------------------------
// Activation staging: 16 consecutive values of token m starting at k.

template <int ACT>
__device__ __forceinline__ void stage16(const GemvArgs &a, uint32_t m, uint32_t k, float inv, float *v)
{
    if constexpr (ACT == ACT_PLAIN) {
        const float4 *s = (const float4 *)(a.x + (uint64_t)m * a.K + k);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 t = s[i];
            v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
        }
    } else if constexpr (ACT == ACT_RMSNORM) {
        const float4 *s = (const float4 *)(a.x + k);
        const float4 *g = (const float4 *)(a.gamma + k);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 t = s[i], w = g[i];
            v[4 * i + 0] = __fmul_rn(__fmul_rn(w.x, t.x), inv);
            v[4 * i + 1] = __fmul_rn(__fmul_rn(w.y, t.y), inv);
            v[4 * i + 2] = __fmul_rn(__fmul_rn(w.z, t.z), inv);
            v[4 * i + 3] = __fmul_rn(__fmul_rn(w.w, t.w), inv);
        }
    } else if constexpr (ACT == ACT_SILU) {
        const float4 *gt = (const float4 *)(a.x + k);
        const float4 *up = (const float4 *)(a.x + a.K + k);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 t = gt[i], u = up[i];
            v[4 * i + 0] = silu_f(t.x) * u.x;
            v[4 * i + 1] = silu_f(t.y) * u.y;
            v[4 * i + 2] = silu_f(t.z) * u.z;
            v[4 * i + 3] = silu_f(t.w) * u.w;
        }
    } else {  // ACT_GQA_V: 16 | head_dim, so the 16 values are contiguous
        const uint32_t hd = a.head_dim, hpk = a.heads_per_kv;
        const uint32_t src = a.K + a.K / hpk + (k / (hd * hpk)) * hd + k % hd;
        const float4 *s = (const float4 *)(a.x + src);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 t = s[i];
            v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
        }
    }
}

template <class Dec, int R, int MT, int ACT>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a, uint32_t KC)
{
    extern __shared__ float smem[];
    float *xs = smem;                    // MT * KC activations
    float *gs = xs + MT * KC;            // MT * KC/16 partial sums
    float *red = gs + MT * (KC / 16);    // 4 floats for the RMSNorm reduction

    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    // 1-D grid, token tile fastest: the workgroups that read the same weight
    // rows for different token tiles are dispatched back to back.
    const uint32_t m_tiles = (a.M + MT - 1) / MT;
    const uint32_t row_tile = blockIdx.x / m_tiles;
    const uint32_t m0 = (blockIdx.x - row_tile * m_tiles) * MT;
    const uint32_t mt = (a.M - m0) < (uint32_t)MT ? (a.M - m0) : (uint32_t)MT;
    const uint32_t wg_row0 = row_tile * (4 * R);
    const uint32_t row0 = wg_row0 + wave * R;
    const uint32_t B = a.K / 256;
    const uint64_t row_bytes = (uint64_t)B * Dec::BS;
    const uint64_t wg_off = (uint64_t)wg_row0 * row_bytes;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.W + wg_off, a.w_bytes > wg_off ? a.w_bytes - wg_off : 0);

    float inv = 1.0f;
    if constexpr (ACT == ACT_RMSNORM) inv = rms_inv(block_sumsq_256(a.x, a.K, red), a.K, a.eps);

    const Dec dec(lane);
    const uint32_t slot = Dec::slot(lane);
    float acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int m = 0; m < MT; m++) acc[r][m] = 0.0f;

    for (uint32_t kc0 = 0; kc0 < a.K; kc0 += KC) {
        const uint32_t kcn = (a.K - kc0) < KC ? (a.K - kc0) : KC;
        const uint32_t ng = kcn / 16;
        __syncthreads();
        for (uint32_t gi = t; gi < (uint32_t)MT * ng; gi += 256) {
            const uint32_t m = gi / ng, gg = gi - m * ng;
            float v[16];
            if (m < mt) {
                stage16<ACT>(a, m0 + m, kc0 + 16 * gg, inv, v);
            } else {
#pragma unroll
                for (int i = 0; i < 16; i++) v[i] = 0.0f;
            }
            float s = 0.0f;
            float4 *dst = (float4 *)(xs + m * KC + 16 * gg);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                dst[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
                s += (v[4 * i] + v[4 * i + 1]) + (v[4 * i + 2] + v[4 * i + 3]);
            }
            gs[m * (KC / 16) + gg] = s;
        }
        __syncthreads();

        const uint32_t CB = kcn / 256, bg0 = kc0 / 256;
        for (uint32_t it = 0; it < CB; it += Dec::BPI) {
            const uint32_t bl = it + slot;
            if (bl < CB) {
                typename Dec::Raw raw[R];
#pragma unroll
                for (int r = 0; r < R; r++)
                    if (row0 + r < a.N)
                        dec.load(raw[r], rs, (uint32_t)((uint64_t)(wave * R + r) * row_bytes + (uint64_t)(bg0 + bl) * Dec::BS));
#pragma unroll
                for (int r = 0; r < R; r++)
                    if (row0 + r < a.N)
                        dec.template accum<MT>(raw[r], xs + bl * 256, KC, gs + bl * 16, KC / 16, acc[r]);
            }
        }
    }

#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
        for (int m = 0; m < MT; m++) {
            const float v = wave_sum(acc[r][m]);
            if (lane == 0 && row0 + r < a.N && (uint32_t)m < mt) {
                float *yp = a.y + (uint64_t)(m0 + m) * a.N + row0 + r;
                *yp = a.residual ? *yp + v : v;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Host-side launch selection.

uint64_t block_bytes(uint32_t type)
{
    switch (type) {
    case T_Q4_K: return 144;
    case T_Q5_K: return 176;
    case T_Q6_K: return 210;
    case T_F32: return 1024;
    default: return 0;
    }
}

template <class Dec, int R, int MT, int ACT>
static hipError_t go(const GemvArgs &a, hipStream_t s)
{
    uint32_t kcmax = (MT == 1 ? 8192u : MT == 2 ? 4096u : 2048u);
    uint32_t KC = a.K < kcmax ? a.K : kcmax;
    size_t lds = ((size_t)MT * KC + (size_t)MT * (KC / 16) + 4) * sizeof(float);
    dim3 grid(((a.M + MT - 1) / MT) * ((a.N + 4 * R - 1) / (4 * R)));
    hipLaunchKernelGGL((gemv_kernel<Dec, R, MT, ACT>), grid, dim3(256), lds, s, a, KC);
    return hipGetLastError();
}

template <class Dec, int ACT>
static hipError_t go_rows(const GemvArgs &a, hipStream_t s)
{
    // Rows per wave: enough workgroups to cover 256 CUs twice where N allows.
    if (a.N >= 16384) return go<Dec, 4, 1, ACT>(a, s);
    if (a.N >= 2048) return go<Dec, 2, 1, ACT>(a, s);
    return go<Dec, 1, 1, ACT>(a, s);
}

template <class Dec>
static hipError_t go_type(const GemvArgs &a, uint32_t act, hipStream_t s)
{
    if (a.M > 1) {
        if (act != ACT_PLAIN) return hipErrorInvalidValue;
        if (a.M >= 4) return go<Dec, 2, 4, ACT_PLAIN>(a, s);
        return go<Dec, 2, 2, ACT_PLAIN>(a, s);
    }
    switch (act) {
    case ACT_PLAIN: return go_rows<Dec, ACT_PLAIN>(a, s);
    case ACT_SILU: return go_rows<Dec, ACT_SILU>(a, s);
    case ACT_GQA_V: return go_rows<Dec, ACT_GQA_V>(a, s);
    case ACT_RMSNORM: return go_rows<Dec, ACT_RMSNORM>(a, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv(const GemvArgs &a, uint32_t act, hipStream_t s)
{
    switch (a.type) {
    case T_Q4_K: return go_type<DecQ4K>(a, act, s);
    case T_Q5_K: return go_type<DecQ5K>(a, act, s);
    case T_Q6_K: return go_type<DecQ6K>(a, act, s);
    case T_F32: return go_type<DecF32>(a, act, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace rrr
