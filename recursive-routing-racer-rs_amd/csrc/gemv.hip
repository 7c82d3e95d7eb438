// gemv.hip -- fused dequant-in-kernel GEMV / batched GEMV on raw GGUF blocks.
//
// Y[m][n] = sum_k X[m][k] * W[n][k]  (phi4.rs:628-630; batch shape :1257-1268)
//
// W is the raw GGUF tensor, N rows of K/256 super-blocks, uploaded unchanged.
// A 256-thread workgroup owns 4*R consecutive rows (R per wave).  Within a
// wave, BPI super-blocks of a row are in flight per iteration and LPB lanes
// share each super-block; every lane owns a fixed 16-byte slice of the block
// (chosen per type below), loads it with a bounds-checked buffer load, and
// multiplies it against the NS activation spans that slice covers.  The
// sub-block scale and min are applied once per span:
//     sum_j x_j * (q_j * s - m) = s * sum_j q_j x_j - m * sum_j x_j
// with the 16-element activation sums precomputed at staging, so the inner
// loop is one int->float conversion and one FMA per weight.  A lane reads its
// activation spans once per iteration and reuses them for all R rows.
#include "act.h"

namespace rrr {

// ---------------------------------------------------------------------------
// Per-type lane decoders.  Lane = part * BPI + slot: `slot` picks the
// super-block within the iteration, `part` the 16-byte slice within it.
// span_off(j) is the offset of activation span j inside the 256-element block.
// STR is the float4 row stride of the interleaved LDS layout used by the
// batch-1 kernel (see gemv_pf_kernel).

// Q4_K block (phi4.rs:481-510): {f16 d; f16 dmin; u8 sc[12]; u8 qs[128]}.
// Part c (0..7) takes qs bytes [16c, 16c+16): pair p = c/2, j0 = 16 (c&1);
// its low nibbles are sub-block 2p (span 0), its high nibbles sub-block 2p+1
// (span 1), positions j0..j0+15.
struct DecQ4K {
    static constexpr uint32_t BS = 144, LPB = 8, BPI = 8, STR = 10;
    static constexpr int NS = 2, SPAN = 16;
    struct Raw { u32x4 hdr, qs; };
    uint32_t c, p, j0;
    __device__ explicit DecQ4K(uint32_t lane) : c(lane / BPI), p((lane / BPI) >> 1), j0(((lane / BPI) & 1) * 16) {}
    __device__ static uint32_t slot(uint32_t lane) { return lane % BPI; }
    __device__ uint32_t span_off(int j) const { return 64 * p + j0 + 32 * j; }
    __device__ void load(Raw &w, __amdgpu_buffer_rsrc_t rs, uint32_t boff) const
    {
        w.hdr = bload16(rs, boff);
        w.qs = bload16(rs, boff + 16 + 16 * c);
    }
    template <int MT>
    __device__ void accum(const Raw &w, const float (*xr)[NS * SPAN], const float (*gr)[NS], float *acc) const
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
#pragma unroll
        for (int m = 0; m < MT; m++) {
            float dl = 0.0f, dh = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                dl = fmaf(ql[i], xr[m][i], dl);
                dh = fmaf(qh[i], xr[m][16 + i], dh);
            }
            float r = acc[m];
            r = fmaf(s0, dl, r); r = fmaf(-n0, gr[m][0], r);
            r = fmaf(s1, dh, r); r = fmaf(-n1, gr[m][1], r);
            acc[m] = r;
        }
    }
};

// Q5_K block (phi4.rs:512-542): {d; dmin; sc[12]; qh[32]; qs[128]}.
// Same parts as Q4_K; the fifth bit of position j in sub-block s is bit s of
// qh[j], so each lane also loads qh[j0..j0+15].
struct DecQ5K {
    static constexpr uint32_t BS = 176, LPB = 8, BPI = 8, STR = 10;
    static constexpr int NS = 2, SPAN = 16;
    struct Raw { u32x4 hdr, qh, qs; };
    uint32_t c, p, j0;
    __device__ explicit DecQ5K(uint32_t lane) : c(lane / BPI), p((lane / BPI) >> 1), j0(((lane / BPI) & 1) * 16) {}
    __device__ static uint32_t slot(uint32_t lane) { return lane % BPI; }
    __device__ uint32_t span_off(int j) const { return 64 * p + j0 + 32 * j; }
    __device__ void load(Raw &w, __amdgpu_buffer_rsrc_t rs, uint32_t boff) const
    {
        w.hdr = bload16(rs, boff);
        w.qh = bload16(rs, boff + 16 + j0);
        w.qs = bload16(rs, boff + 48 + 16 * c);
    }
    template <int MT>
    __device__ void accum(const Raw &w, const float (*xr)[NS * SPAN], const float (*gr)[NS], float *acc) const
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
#pragma unroll
        for (int m = 0; m < MT; m++) {
            float dl = 0.0f, dh = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                dl = fmaf(ql[i], xr[m][i], dl);
                dh = fmaf(qh[i], xr[m][16 + i], dh);
            }
            float r = acc[m];
            r = fmaf(s0, dl, r); r = fmaf(-n0, gr[m][0], r);
            r = fmaf(s1, dh, r); r = fmaf(-n1, gr[m][1], r);
            acc[m] = r;
        }
    }
};

// Q6_K block (phi4.rs:444-479): {ql[128]; qh[64]; i8 sc[16]; f16 d}.
// Part G (0..3) takes half g = G/2 and positions l0 = 16 (G&1) .. l0+15:
// ql[64g + l0 ..], ql[64g + 32 + l0 ..] and qh[32g + l0 ..], i.e. all four
// quads u of those positions (span u).  Element g*128 + 32u + l uses scale
// sc[8g + l/16 + 2u], which is the is = g*8 + l/16 rule of phi4.rs:463.
// Blocks are 210 bytes, so these 16-byte loads are 2-byte aligned.
struct DecQ6K {
    static constexpr uint32_t BS = 210, LPB = 4, BPI = 16, STR = 17;
    static constexpr int NS = 4, SPAN = 16;
    struct Raw { u32x4 qa, qb, qh; u32x2 sc; uint32_t d; };
    uint32_t g, l0;
    __device__ explicit DecQ6K(uint32_t lane) : g((lane / BPI) >> 1), l0(((lane / BPI) & 1) * 16) {}
    __device__ static uint32_t slot(uint32_t lane) { return lane % BPI; }
    __device__ uint32_t span_off(int u) const { return 128 * g + l0 + 32 * u; }
    __device__ void load(Raw &w, __amdgpu_buffer_rsrc_t rs, uint32_t boff) const
    {
        w.qa = bload16(rs, boff + 64 * g + l0);
        w.qb = bload16(rs, boff + 64 * g + 32 + l0);
        w.qh = bload16(rs, boff + 128 + 32 * g + l0);
        w.sc = __builtin_amdgcn_raw_buffer_load_b64(rs, boff + 192 + 8 * g, 0, 0);
        w.d = bload2(rs, boff + 208);
    }
    template <int MT>
    __device__ void accum(const Raw &w, const float (*xr)[NS * SPAN], const float (*gr)[NS], float *acc) const
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
#pragma unroll
        for (int m = 0; m < MT; m++) {
            float r = acc[m];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                float dot = 0.0f;
#pragma unroll
                for (int i = 0; i < 16; i++) dot = fmaf(q[u][i], xr[m][16 * u + i], dot);
                // stored values are q + 32 (0..63); remove the offset once per span
                dot = fmaf(-32.0f, gr[m][u], dot);
                r = fmaf(ds[u], dot, r);
            }
            acc[m] = r;
        }
    }
};

// F32 rows (matmul_tiled with M=1 on untransposed weights, phi4.rs:641-646,
// and the row-major logits).  A "block" is 256 floats; part c (0..15) takes
// floats 4c + 64i (span i, i = 0..3), so each load instruction covers
// contiguous 256-byte runs.
struct DecF32 {
    static constexpr uint32_t BS = 1024, LPB = 16, BPI = 4, STR = 4;
    static constexpr int NS = 4, SPAN = 4;
    struct Raw { u32x4 v[4]; };
    uint32_t c;
    __device__ explicit DecF32(uint32_t lane) : c(lane / BPI) {}
    __device__ static uint32_t slot(uint32_t lane) { return lane % BPI; }
    __device__ uint32_t span_off(int i) const { return 4 * c + 64 * i; }
    __device__ void load(Raw &w, __amdgpu_buffer_rsrc_t rs, uint32_t boff) const
    {
#pragma unroll
        for (int i = 0; i < 4; i++) w.v[i] = bload16(rs, boff + 16 * c + 256 * i);
    }
    template <int MT>
    __device__ void accum(const Raw &w, const float (*xr)[NS * SPAN], const float (*)[NS], float *acc) const
    {
#pragma unroll
        for (int m = 0; m < MT; m++) {
            float r = acc[m];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                r = fmaf(u2f(w.v[i].x), xr[m][4 * i + 0], r);
                r = fmaf(u2f(w.v[i].y), xr[m][4 * i + 1], r);
                r = fmaf(u2f(w.v[i].z), xr[m][4 * i + 2], r);
                r = fmaf(u2f(w.v[i].w), xr[m][4 * i + 3], r);
            }
            acc[m] = r;
        }
    }
};

// ---------------------------------------------------------------------------
// Activation sources.  src_load fetches the raw inputs of 16 consecutive
// activations of token m at k; src_xform turns them into the activations.

struct Src16 {
    float4 a[4];  // x / gate / gathered V
    float4 b[4];  // gamma (ACT_RMSNORM) or up (ACT_SILU)
};

template <int ACT>
__device__ __forceinline__ void src_load(const GemvArgs &a, uint32_t m, uint32_t k, Src16 &s)
{
    const float4 *pa;
    if constexpr (ACT == ACT_GQA_V) {
        // 16 | head_dim, so the 16 gathered values are contiguous
        const uint32_t hd = a.head_dim, hpk = a.heads_per_kv;
        pa = (const float4 *)(a.x + a.K + a.K / hpk + (k / (hd * hpk)) * hd + k % hd);
    } else {
        pa = (const float4 *)(a.x + (uint64_t)m * a.K + k);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) s.a[i] = pa[i];
    if constexpr (ACT == ACT_RMSNORM) {
#pragma unroll
        for (int i = 0; i < 4; i++) s.b[i] = ((const float4 *)(a.gamma + k))[i];
    } else if constexpr (ACT == ACT_SILU) {
#pragma unroll
        for (int i = 0; i < 4; i++) s.b[i] = ((const float4 *)(a.x + a.K + k))[i];
    }
}

template <int ACT>
__device__ __forceinline__ void src_xform(const Src16 &s, float inv, float4 *v)
{
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 x = s.a[i];
        if constexpr (ACT == ACT_RMSNORM) {
            const float4 w = s.b[i];
            v[i] = make_float4(__fmul_rn(__fmul_rn(w.x, x.x), inv), __fmul_rn(__fmul_rn(w.y, x.y), inv),
                               __fmul_rn(__fmul_rn(w.z, x.z), inv), __fmul_rn(__fmul_rn(w.w, x.w), inv));
        } else if constexpr (ACT == ACT_SILU) {
            const float4 u = s.b[i];
            v[i] = make_float4(silu_fast(x.x) * u.x, silu_fast(x.y) * u.y, silu_fast(x.z) * u.z, silu_fast(x.w) * u.w);
        } else {
            v[i] = x;
        }
    }
}

__device__ __forceinline__ float sum16(const float4 *v)
{
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
    return s;
}

// ---------------------------------------------------------------------------
// General kernel: M >= 1 token rows in tiles of MT, K streamed through LDS in
// chunks of KC with a contiguous layout (xs[m*KC + k]).  Used for batched
// GEMV, rows longer than four wave iterations and the tall F32 logits.
template <class Dec, int R, int MT, int ACT>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a, uint32_t KC)
{
    extern __shared__ float smem[];
    float *xs = smem;                    // MT * KC activations
    float *gs = xs + MT * KC;            // MT * KC/16 partial sums
    float *red = gs + MT * (KC / 16);    // 16 floats for the RMSNorm reduction

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
            float4 v[4];
            if (m < mt) {
                Src16 sv;
                src_load<ACT>(a, m0 + m, kc0 + 16 * gg, sv);
                src_xform<ACT>(sv, inv, v);
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
            float4 *dst = (float4 *)(xs + m * KC + 16 * gg);
#pragma unroll
            for (int i = 0; i < 4; i++) dst[i] = v[i];
            gs[m * (KC / 16) + gg] = sum16(v);
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
                float xr[MT][Dec::NS * Dec::SPAN], gr[MT][Dec::NS];
#pragma unroll
                for (int m = 0; m < MT; m++)
#pragma unroll
                    for (int j = 0; j < Dec::NS; j++) {
                        const uint32_t o = bl * 256 + dec.span_off(j);
#pragma unroll
                        for (int i = 0; i < Dec::SPAN / 4; i++) {
                            const float4 f = *(const float4 *)(xs + m * KC + o + 4 * i);
                            xr[m][j * Dec::SPAN + 4 * i] = f.x; xr[m][j * Dec::SPAN + 4 * i + 1] = f.y;
                            xr[m][j * Dec::SPAN + 4 * i + 2] = f.z; xr[m][j * Dec::SPAN + 4 * i + 3] = f.w;
                        }
                        gr[m][j] = gs[m * (KC / 16) + o / 16];
                    }
#pragma unroll
                for (int r = 0; r < R; r++)
                    if (row0 + r < a.N) dec.template accum<MT>(raw[r], xr, gr, acc[r]);
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
// Batch-1 kernel for rows of at most IT wave iterations (every decode-path
// GEMV).  Order of work per workgroup:
//   1. each thread fetches the raw inputs of its activation float4s of the
//      canonical sum-of-squares split (runs of 64 float4s per wave:
//      coalesced; L2 hits after the first workgroup of an XCD);
//   2. every wave issues ALL of its weight loads, so HBM latency overlaps the
//      staging (vmcnt retires in order, which is why the activation loads go
//      first);
//   3. the fused RMSNorm reduces the sum of squares of those registers in the
//      canonical order; activations are transformed,
//      written to LDS, and their 16-element sums formed with two lane
//      shuffles ((f0 + f1) + (f2 + f3) over the four float4s of a group);
//   4. per iteration each lane reads its spans from LDS once and runs the dot
//      products for its R rows as the weight loads land.
// LDS layout: activations interleaved by block at float4 granularity,
//   xs4[(I * 64 + q) * STR + s]  for block b = I * BPI + s, elements 4q..4q+3,
// so the lanes of one LDS read (consecutive slots s) touch consecutive
// float4s; STR pads each row so that the staging writes (consecutive q) and
// the reads of different parts fall on different banks.
// Partial sums: gs[(I * 16 + o / 16) * BPI + s].

template <class Dec, int R, int IT, int ACT>
__global__ __launch_bounds__(256) void gemv_pf_kernel(GemvArgs a)
{
    extern __shared__ float smem[];
    constexpr uint32_t BPI = Dec::BPI, STR = Dec::STR;
    constexpr int JF = IT * BPI / 4;  // activation float4s per thread: K <= IT * BPI * 256
    const uint32_t K = a.K;
    float4 *xs4 = (float4 *)smem;                               // IT * 64 * STR float4
    float *gs = smem + 4 * IT * 64 * STR;                       // IT * 16 * BPI
    float *red = gs + IT * 16 * BPI;                            // 16

    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint32_t wg_row0 = blockIdx.x * (4 * R);
    const uint32_t row0 = wg_row0 + wave * R;
    const uint32_t B = K / 256, NF = K / 4;
    const uint64_t row_bytes = (uint64_t)B * Dec::BS;
    const uint64_t wg_off = (uint64_t)wg_row0 * row_bytes;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.W + wg_off, a.w_bytes > wg_off ? a.w_bytes - wg_off : 0);
    const Dec dec(lane);
    const uint32_t slot = Dec::slot(lane);

    // 1. activation inputs, the thread's float4s of the canonical
    // sum-of-squares split (NF is a multiple of 64, so each guard is
    // wave-uniform)
    uint32_t fo[JF], sl[JF];
    sumsq_slots<JF>(sumsq_parts(K), fo, sl);
    float4 xa[JF], xb[JF];
#pragma unroll
    for (int j = 0; j < JF; j++)
        if (fo[j] < NF) src_load4<ACT>(a, 4 * fo[j], xa[j], xb[j]);

    // 2. all weight loads of this wave
    typename Dec::Raw raw[IT][R];
#pragma unroll
    for (int it = 0; it < IT; it++) {
        const uint32_t bl = it * BPI + slot;
#pragma unroll
        for (int r = 0; r < R; r++)
            if (bl < B && row0 + r < a.N)
                dec.load(raw[it][r], rs, (uint32_t)((uint64_t)(wave * R + r) * row_bytes + (uint64_t)bl * Dec::BS));
    }

    // 3. RMSNorm scale, transform, stage
    float inv = 1.0f;
    if constexpr (ACT == ACT_RMSNORM) inv = rms_inv(sumsq_held_256<JF>(xa, fo, sl, NF, red), K, a.eps);
#pragma unroll
    for (int j = 0; j < JF; j++) {
        const uint32_t f = fo[j];
        if (f < NF) {
            const float4 v = xform4<ACT>(xa[j], xb[j], inv);
            const uint32_t b = f / 64, q = f % 64, I = b / BPI, s = b % BPI;
            xs4[(I * 64 + q) * STR + s] = v;
            float sv = (v.x + v.y) + (v.z + v.w);
            sv = sv + __shfl_xor(sv, 1, 64);
            sv = sv + __shfl_xor(sv, 2, 64);
            if ((t & 3) == 0) gs[(I * 16 + q / 4) * BPI + s] = sv;
        }
    }
    __syncthreads();

    // 4. dot products
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
#pragma unroll
    for (int it = 0; it < IT; it++) {
        const uint32_t bl = it * BPI + slot;
        if (bl < B) {
            float xr[1][Dec::NS * Dec::SPAN], gr[1][Dec::NS];
#pragma unroll
            for (int j = 0; j < Dec::NS; j++) {
                const uint32_t o = dec.span_off(j);
#pragma unroll
                for (int i = 0; i < Dec::SPAN / 4; i++) {
                    const float4 fv = xs4[(it * 64 + o / 4 + i) * STR + slot];
                    xr[0][j * Dec::SPAN + 4 * i] = fv.x; xr[0][j * Dec::SPAN + 4 * i + 1] = fv.y;
                    xr[0][j * Dec::SPAN + 4 * i + 2] = fv.z; xr[0][j * Dec::SPAN + 4 * i + 3] = fv.w;
                }
                gr[0][j] = gs[(it * 16 + o / 16) * BPI + slot];
            }
#pragma unroll
            for (int r = 0; r < R; r++)
                if (row0 + r < a.N) dec.template accum<1>(raw[it][r], xr, gr, &acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        const float v = wave_sum(acc[r]);
        if (lane == 0 && row0 + r < a.N) {
            float *yp = a.y + row0 + r;
            *yp = a.residual ? *yp + v : v;
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
    size_t lds = ((size_t)MT * KC + (size_t)MT * (KC / 16) + 16) * sizeof(float);
    dim3 grid(((a.M + MT - 1) / MT) * ((a.N + 4 * R - 1) / (4 * R)));
    hipLaunchKernelGGL((gemv_kernel<Dec, R, MT, ACT>), grid, dim3(256), lds, s, a, KC);
    return hipGetLastError();
}

template <class Dec, int R, int IT, int ACT>
static hipError_t go_pf(const GemvArgs &a, hipStream_t s)
{
    const size_t lds = ((size_t)4 * IT * 64 * Dec::STR + (size_t)IT * 16 * Dec::BPI + 16) * sizeof(float);
    const dim3 grid((a.N + 4 * R - 1) / (4 * R));
    hipLaunchKernelGGL((gemv_pf_kernel<Dec, R, IT, ACT>), grid, dim3(256), lds, s, a);
    return hipGetLastError();
}

template <class Dec, int R, int ACT>
static hipError_t go_pf_it(const GemvArgs &a, hipStream_t s)
{
    const uint32_t it = (a.K / 256 + Dec::BPI - 1) / Dec::BPI;
    if (it <= 1) return go_pf<Dec, R, 1, ACT>(a, s);
    if (it <= 2) return go_pf<Dec, R, 2, ACT>(a, s);
    return go_pf<Dec, R, 4, ACT>(a, s);
}

// Rows per wave: about two workgroups per CU where N allows.  Batch-1 shapes
// whose rows fit in at most four wave iterations (every decode-path GEMV)
// take the load-first kernel; longer rows and very tall F32 matrices (the
// logits) stream through the chunked loop kernel.
template <class Dec, int ACT>
static hipError_t go_rows(const GemvArgs &a, hipStream_t s)
{
    const uint32_t it = (a.K / 256 + Dec::BPI - 1) / Dec::BPI;
    const uint32_t it_inst = it <= 1 ? 1 : it <= 2 ? 2 : 4;
    const size_t lds = ((size_t)4 * it_inst * 64 * Dec::STR + (size_t)it_inst * 16 * Dec::BPI + 16) * sizeof(float);
    const bool f32 = Dec::BS == 1024;
    if (it <= 4 && lds <= 65536 && !(f32 && a.N > 16384)) {
        if (a.N >= 12288 && !f32) return go_pf_it<Dec, 4, ACT>(a, s);
        if (a.N >= 2048) return go_pf_it<Dec, 2, ACT>(a, s);
        return go_pf_it<Dec, 1, ACT>(a, s);
    }
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

// Batched K-quant rows above 16 tokens that the skinny kernel does not take
// (more than 32 rows, Q6_K, K > 3072) run on the prefill GEMM's fp16 matrix
// cores: the f32 rows become f16 block floating point (a power-of-two scale
// per row, undone exactly on the output), zero-padded to a multiple of 128
// rows inside the context workspace.
static bool batched_gemm_route(const GemvArgs &a, uint32_t act)
{
    return a.M > 16 && act == ACT_PLAIN && !a.residual && a.type != T_F32 && a.ws &&
           (((uintptr_t)a.x | (uintptr_t)a.y) & 15) == 0 && gemm_rows_supported(a.type, a.K, a.N, a.M, a.ws_bytes);
}

hipError_t launch_gemv(const GemvArgs &a, uint32_t act, hipStream_t s)
{
    if (gemv_mfma_supported(a)) return launch_gemv_mfma(a, act, s);
    if (a.M > 1 && act == ACT_PLAIN && gemv_mq_tokens_supported(a)) return launch_gemv_mq_tokens(a, s);
    if (a.M > 1 && act == ACT_PLAIN && skinny_supported(a)) return launch_skinny(a, s);
    if (batched_gemm_route(a, act)) return launch_gemm_f32_rows(a.x, a.W, a.type, a.y, a.K, a.N, a.M, a.ws, a.ws_bytes, s);
    switch (a.type) {
    case T_Q4_K: return go_type<DecQ4K>(a, act, s);
    case T_Q5_K: return go_type<DecQ5K>(a, act, s);
    case T_Q6_K: return go_type<DecQ6K>(a, act, s);
    case T_F32: return go_type<DecF32>(a, act, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace rrr
