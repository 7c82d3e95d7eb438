// skinny.hip -- batched GEMV / skinny GEMM on the fp16 matrix cores for
// 2 <= M <= 32 token rows and Q4_K / Q5_K weights (the batched shape of
// phi4.rs:1257-1268: Y[m][n] = sum_k X[m][k] * W[n][k], X and Y f32 row-major).
//
// Exact weights.  For super-block b of row n,
//     sum_k x_k w_k = d * sum_s sum_{k in s} (sc_s q_k) x_k - dmin * sum_s mn_s X_s
// (phi4.rs:481-542, w = d*sc*q - dmin*mn), X_s the sum of x over sub-block s.
// sc_s q_k <= 63 * 31 = 1953 < 2^11 is an integer, exact in fp16: the MFMA B
// operand carries it, the 8 sub-blocks of a block accumulate in the MFMA's f32
// accumulator, and d, dmin are applied once per block.  The min term is a
// second, small MFMA (16x16x16) of the sub-block sums X_s against mn_s.
//
// Activations.  A wave's K slice (one super-block) of token m is scaled by
// 2^-E (E from the slice maximum, so the values lie below 2^14) and split
// x = hi + lo, hi = fp16(x), lo = fp16(x - hi), relative error 2^-22 of the
// slice maximum.  M <= 16: A rows 2m+h (h = 0 hi, 1 lo), 8 tokens per 16-row A
// tile (the GEMV bar, 1e-4).  16 < M <= 32: A rows are 16 tokens of hi only
// (error 2^-12, the MFMA bar 2e-3).  The X_s are scaled by 2^-(E+5)
// (|X_s| <= 32 max) and split the same way; d and dmin take the 2^E back.
//
// MFMA layouts (lane l): 16x16x32 f16 -- A row l%16 / B column l%16 at
// k = 8(l/16) .. +7; 16x16x16 f16 -- the same at k = 4(l/16) .. +3; D rows
// 4(l/16)+r of column l%16 in register r.
//
// Encoding pass (M > 8: two A tiles).  The A operands depend only on X, so a
// small kernel (skinny_encode_kernel, one wave per A tile and super-block
// column) builds them once per call into the workspace, in the lane order of
// the MFMA:
//   av   [TOK][W][8][64] f16x8  lane's 8 values of sub-block s
//   amin [TOK][W][64]    f16x4  lane's 4 sub-block sums (min-term A operand)
//   ex   [TOK][W][16]    int    E of A row r
// (W = K/256 columns, TOK A tiles), 8,768 bytes per (tile, column).  Every
// workgroup of the main kernel then loads its operands with 16-byte loads
// instead of reading all of X in f32 and converting it again.  With one A
// tile (M <= 8) each wave encodes its own slice: there the pass's launch
// costs more than the staging it saves (gate+up 16384x3072 at M = 4:
// 16.5 us with it, 14.4 us without).
//
// Work split: a workgroup of K/256 waves, wave w owns super-block w of every
// row; it gets its A operands (its first tiles' weight loads in flight), then
// walks the workgroup's 16-row tiles b, b + G, ... (G = gridDim.x), staging the
// tile's 16 blocks of its column in its private LDS region by LDS DMA (the
// next tiles' loads in flight meanwhile).  Row partials of the waves are added
// in wave order per tile.
#include "device_common.h"
#include "internal.h"

namespace rrr {

typedef _Float16 f16x8s __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4s __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2s __attribute__((ext_vector_type(2)));

// Scalar offset past every weight byte (w_bytes + RRR_READ_SLACK must stay
// below it): such loads return zeros and move no data.
constexpr uint32_t SK_OOB = 0x80000000u;

__device__ __forceinline__ f16x2s sk_bits(uint32_t v) { return __builtin_bit_cast(f16x2s, v); }
__device__ __forceinline__ uint32_t sk_u32(f16x2s v) { return __builtin_bit_cast(uint32_t, v); }

// Four quant values (bytes < 64 of v) times the scale as exact fp16:
// v_perm places byte q under the exponent of 1024 (f16 0x64qq = 1024 + q),
// and fma(1024 + q, sc, -1024 sc) = sc * q, exact (< 2^11).
__device__ __forceinline__ void sk_scale4(uint32_t v, f16x2s sc2, f16x2s nb2, uint32_t &o01, uint32_t &o23)
{
    o01 = sk_u32(__builtin_elementwise_fma(sk_bits(__builtin_amdgcn_perm(0x64646464u, v, 0x04010400u)), sc2, nb2));
    o23 = sk_u32(__builtin_elementwise_fma(sk_bits(__builtin_amdgcn_perm(0x64646464u, v, 0x04030402u)), sc2, nb2));
}

// Q4_K (phi4.rs:481-510): element 32s + e of a block is nibble (s & 1) of
// qs[32 (s/2) + e].  Lane k-group kg takes e = 8kg .. 8kg+7 of every s.
struct SkQ4K {
    static constexpr uint32_t BS = 144;
    struct Raw { u32x4 hdr; u32x2 qs[4]; };
    __device__ static void load(Raw &r, const uint8_t *L, uint32_t o, uint32_t kg)
    {
        r.hdr = *(const u32x4 *)(L + o);
#pragma unroll
        for (int p = 0; p < 4; p++) r.qs[p] = *(const u32x2 *)(L + o + 16 + 32 * p + 8 * kg);
    }
    // quant values of sub-block s at the lane's 8 positions, one per byte
    __device__ static void quants(const Raw &r, int s, uint32_t &v0, uint32_t &v1)
    {
        v0 = (r.qs[s >> 1].x >> (4 * (s & 1))) & 0x0F0F0F0Fu;
        v1 = (r.qs[s >> 1].y >> (4 * (s & 1))) & 0x0F0F0F0Fu;
    }
};

// Q5_K (phi4.rs:512-542): Q4_K's nibbles plus bit s of qh[e] as bit 4.
struct SkQ5K {
    static constexpr uint32_t BS = 176;
    struct Raw { u32x4 hdr; u32x2 qh; u32x2 qs[4]; };
    __device__ static void load(Raw &r, const uint8_t *L, uint32_t o, uint32_t kg)
    {
        r.hdr = *(const u32x4 *)(L + o);
        r.qh = *(const u32x2 *)(L + o + 16 + 8 * kg);
#pragma unroll
        for (int p = 0; p < 4; p++) r.qs[p] = *(const u32x2 *)(L + o + 48 + 32 * p + 8 * kg);
    }
    __device__ static void quants(const Raw &r, int s, uint32_t &v0, uint32_t &v1)
    {
        v0 = ((r.qs[s >> 1].x >> (4 * (s & 1))) & 0x0F0F0F0Fu) | (((r.qh.x >> s) & 0x01010101u) << 4);
        v1 = ((r.qs[s >> 1].y >> (4 * (s & 1))) & 0x0F0F0F0Fu) | (((r.qh.y >> s) & 0x01010101u) << 4);
    }
};

// Staging geometry of one wave's 16 block pieces, loaded straight into LDS
// (16-byte LDS DMA: lane l of a load writes base + 16 l).  Load slot s covers
// rows s*RPS .. s*RPS+RPS-1 (lane l: unit l % UPB of row l / UPB) and has a
// 1 KB LDS slot of its own, so lanes past the slot's rows (which read nothing
// and write zeros) stay inside it.  A tile buffer is S slots.
template <class Q>
struct SkGeom {
    static constexpr uint32_t UPB = Q::BS / 16;
    static constexpr uint32_t RPS = 64 / UPB;
    static constexpr int S = (16 + RPS - 1) / RPS;
    static constexpr uint32_t BUF = 1024 * S;
    // LDS offset of row r inside a tile buffer
    __device__ static uint32_t row_off(uint32_t r) { return (r / RPS) * 1024 + (r % RPS) * Q::BS; }
};

// Workspace layout of the encoded activations (see the top of this file).
constexpr uint32_t SK_AV_UNIT = 8 * 64 * 16, SK_AMIN_UNIT = 64 * 8, SK_EX_UNIT = 16 * 4;
__host__ __device__ constexpr uint64_t sk_ws_bytes(uint32_t tok, uint32_t W)
{
    return (uint64_t)tok * W * (SK_AV_UNIT + SK_AMIN_UNIT + SK_EX_UNIT);
}
struct SkWs {
    u32x4 *av;
    u32x2 *amin;
    int *ex;
    __host__ __device__ SkWs(void *base, uint32_t tok, uint32_t W)
    {
        uint8_t *p = (uint8_t *)base;
        av = (u32x4 *)p;
        amin = (u32x2 *)(p + (uint64_t)tok * W * SK_AV_UNIT);
        ex = (int *)(p + (uint64_t)tok * W * (SK_AV_UNIT + SK_AMIN_UNIT));
    }
};

// A operands of A tile tt and super-block column w, built by one wave:
// lane (row r16, group kg) gets token tok's values k0 + 32 s + 8 kg + i
// (i < 8) of every sub-block s, its 4 sub-block sums (min-term A operand) and
// the block exponent E of its A row.  HILO: 8 tokens (hi, lo rows) per A
// tile, else 16 tokens (hi rows).  after_loads() runs once the activation
// loads are issued (the caller queues its weight loads behind them).
template <bool HILO, class F>
__device__ __forceinline__ void sk_encode(const float *__restrict__ x, uint32_t M, uint32_t K, uint32_t tt,
                                          uint32_t w, uint32_t lane, f16x8s (&av)[8], f16x4s &am, int &e,
                                          F &&after_loads)
{
    const uint32_t r16 = lane & 15, kg = lane >> 4;
    const uint32_t k0 = w * 256;
    const uint32_t tok = HILO ? tt * 8 + (r16 >> 1) : tt * 16 + r16;
    const bool lo = HILO && (r16 & 1);
    const bool live = tok < M;
    const float4 *xp = (const float4 *)(x + (uint64_t)min(tok, M - 1) * K + k0 + 8 * kg);
    float4 xv[16];
#pragma unroll
    for (int s = 0; s < 8; s++) {
        xv[2 * s] = xp[8 * s];
        xv[2 * s + 1] = xp[8 * s + 1];
    }
    after_loads();
    float mx = 0.0f, gs[8];
#pragma unroll
    for (int s = 0; s < 8; s++) {
        const float4 u = xv[2 * s], v = xv[2 * s + 1];
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(u.x), fabsf(u.y)), fmaxf(fabsf(u.z), fabsf(u.w))));
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        gs[s] = ((u.x + u.y) + (u.z + u.w)) + ((v.x + v.y) + (v.z + v.w));
    }
    // the token's four k-groups (lanes r16 + 16 kg)
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
#pragma unroll
    for (int s = 0; s < 8; s++) {
        gs[s] = gs[s] + __shfl_xor(gs[s], 16, 64);
        gs[s] = gs[s] + __shfl_xor(gs[s], 32, 64);
    }
    e = 0;
    if (mx > 0.0f && __builtin_isfinite(mx)) {
        int ex;
        (void)frexpf(mx, &ex);
        e = ex - 14;  // mx / 2^e in [2^13, 2^14)
    }
    const float sx = ldexpf(1.0f, -e), sg = ldexpf(1.0f, -e - 5);
#pragma unroll
    for (int s = 0; s < 8; s++) {
        const float4 u = xv[2 * s], v = xv[2 * s + 1];
        const float f[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
        f16x8s h;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float y = f[i] * sx;
            const _Float16 hi = (_Float16)y;
            h[i] = live ? (lo ? (_Float16)(y - (float)hi) : hi) : (_Float16)0.0f;
        }
        av[s] = h;
    }
    // X_s of sub-blocks 4 kg .. 4 kg + 3 (k-groups 2, 3 are padding)
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float g = 0.0f;
#pragma unroll
        for (int s = 0; s < 8; s++)
            if (s == (int)(4 * kg) + i) g = gs[s];
        const float y = g * sg;
        const _Float16 hi = (_Float16)y;
        am[i] = live && kg < 2 ? (lo ? (_Float16)(y - (float)hi) : hi) : (_Float16)0.0f;
    }
}

// The encoding pass: one wave per (super-block column, A tile), grid (W, TOK).
template <bool HILO>
__global__ __launch_bounds__(64) void skinny_encode_kernel(const float *__restrict__ x, uint32_t M, uint32_t K,
                                                           void *ws, uint32_t tok_tiles)
{
    const uint32_t W = K / 256, w = blockIdx.x, tt = blockIdx.y, lane = threadIdx.x;
    const SkWs o(ws, tok_tiles, W);
    f16x8s av[8];
    f16x4s am;
    int e;
    sk_encode<HILO>(x, M, K, tt, w, lane, av, am, e, [] {});
    u32x4 *ap = o.av + (uint64_t)(tt * W + w) * 8 * 64 + lane;
#pragma unroll
    for (int s = 0; s < 8; s++) ap[s * 64] = __builtin_bit_cast(u32x4, av[s]);
    o.amin[(uint64_t)(tt * W + w) * 64 + lane] = __builtin_bit_cast(u32x2, am);
    if (lane < 16) o.ex[(tt * W + w) * 16 + lane] = e;
}

// TOK A tiles (TPT tokens each); DPT = tokens of a tile per lane in the D
// layout.  NB tile buffers per wave: tiles i+1 .. i+NB-1 stream in while
// tile i is multiplied.  PRE: the A operands come from the encoding pass,
// else each wave builds its own (one A tile: the f32 activations are no more
// bytes than their encoding, and the pass would cost a launch).
template <class Q, bool HILO, int TOK, int NB, bool PRE>
__global__ __launch_bounds__(TOK == 1 ? 1024 : 768) void skinny_kernel(GemvArgs a, uint32_t ntiles)
{
    using G = SkGeom<Q>;
    constexpr int TPT = HILO ? 8 : 16, DPT = HILO ? 2 : 4, MP = TOK * TPT;
    extern __shared__ float smem[];
    const uint32_t K = a.K, M = a.M, N = a.N, W = K / 256;
    const uint32_t t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t r16 = lane & 15, kg = lane >> 4;
    const uint32_t GR = gridDim.x, tile0 = blockIdx.x;
    const uint32_t ntl = tile0 < ntiles ? (ntiles - tile0 + GR - 1) / GR : 0u;
    uint8_t *L = (uint8_t *)smem + wave * NB * G::BUF;            // this wave's tile buffers
    float *part = (float *)((uint8_t *)smem + W * NB * G::BUF);  // [2][W][MP][16]

    const uint32_t row_bytes = W * Q::BS;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.W, a.w_bytes + RRR_READ_SLACK);

    // weight units: lane-fixed offsets, a uniform offset per load slot; rows
    // past 16 in the last slot read nothing
    const uint32_t rsel = min(lane / G::UPB, G::RPS - 1), vl = lane - (lane / G::UPB) * G::UPB;
    const bool lane_ok = lane < G::RPS * G::UPB;
    const uint32_t voff = lane_ok ? rsel * row_bytes + wave * Q::BS + 16 * vl : SK_OOB;
    const uint32_t voff_last = (G::S - 1) * G::RPS + rsel < 16 ? voff : SK_OOB;
    const uint32_t tile_bytes = 16 * row_bytes;
    // tile tl into buffer tl % NB (S loads; past the last tile: zeros)
    auto dma = [&](uint32_t tl) {
        const uint32_t tb = tl < ntl ? (tile0 + tl * GR) * tile_bytes : SK_OOB;
        uint8_t *dst = L + (tl % NB) * G::BUF;
#pragma unroll
        for (int s = 0; s < G::S; s++)
            lds_dma16<RRR_CPOL_NT>(rs, dst + 1024 * s, s == G::S - 1 ? voff_last : voff, tb + s * G::RPS * row_bytes);
    };

    // 1. A operands, the first tiles' weights streaming in meanwhile (queued
    // after the loads of the encoded operands, and after those of f32
    // activations, which the encoding needs first: loads return in order, so
    // tile 0 waits for the A operands and its own weights only, while the
    // next tiles' weights arrive under its MFMAs)
    f16x8s av[TOK][8];
    f16x4s amin[TOK];
    int eexp[TOK][DPT];   // E of the lane's D-layout tokens
    // D row 4 kg + j holds A row 4 kg + j: the token of A row 4 kg + 2 j
    // (HILO: rows 2t, 2t+1 are token t's hi and lo) or 4 kg + j
    if constexpr (PRE) {
        const SkWs o(a.ws, TOK, W);
#pragma unroll
        for (int tt = 0; tt < TOK; tt++) {
            const u32x4 *ap = o.av + (uint64_t)(tt * W + wave) * 8 * 64 + lane;
#pragma unroll
            for (int s = 0; s < 8; s++) av[tt][s] = __builtin_bit_cast(f16x8s, ap[s * 64]);
            amin[tt] = __builtin_bit_cast(f16x4s, o.amin[(uint64_t)(tt * W + wave) * 64 + lane]);
#pragma unroll
            for (int j = 0; j < DPT; j++)
                eexp[tt][j] = o.ex[(tt * W + wave) * 16 + (HILO ? 4 * kg + 2 * j : 4 * kg + j)];
        }
        __builtin_amdgcn_sched_barrier(0);
        for (uint32_t i = 0; i + 1 < NB; i++) dma(i);
    } else {
#pragma unroll
        for (int tt = 0; tt < TOK; tt++) {
            int e;
            sk_encode<HILO>(a.x, M, K, tt, wave, lane, av[tt], amin[tt], e, [&] {
                if (tt == 0)
                    for (uint32_t i = 0; i + 1 < NB; i++) dma(i);
            });
#pragma unroll
            for (int j = 0; j < DPT; j++) eexp[tt][j] = __shfl(e, HILO ? 4 * kg + 2 * j : 4 * kg + j, 64);
        }
    }

    // 2^E of the lane's D-layout tokens (the same for every tile)
    float pe[TOK][DPT];
#pragma unroll
    for (int tt = 0; tt < TOK; tt++)
#pragma unroll
        for (int j = 0; j < DPT; j++) pe[tt][j] = ldexpf(1.0f, eexp[tt][j]);
    // 2. tiles: tile tl + NB - 1 into the buffer tile tl - 1 used, wait for
    // tile tl, MFMAs, row partials
    uint32_t buf = 0;
    const uint32_t roff = G::row_off(r16);
    for (uint32_t tl = 0; tl < ntl; tl++) {
        dma(tl + NB - 1);
        wait_vm<(NB - 1) * G::S>();
        typename Q::Raw raw;
        Q::load(raw, L + (tl % NB) * G::BUF, roff, kg);
        const float d = h2f(raw.hdr.x), dmin = h2f(raw.hdr.x >> 16);
        uint32_t scb[2], mnb[2];
        scale_min_bytes_k4(raw.hdr.y, raw.hdr.z, raw.hdr.w, scb, mnb);
        // min term B operand: mn of sub-blocks 4 kg .. 4 kg + 3 (k-groups 2, 3 padding)
        const uint32_t mk = kg == 0 ? mnb[0] : mnb[1];
        const f16x2s m01 = sk_bits(__builtin_amdgcn_perm(0x64646464u, mk, 0x04010400u)) - f16x2s{(_Float16)1024.0f, (_Float16)1024.0f};
        const f16x2s m23 = sk_bits(__builtin_amdgcn_perm(0x64646464u, mk, 0x04030402u)) - f16x2s{(_Float16)1024.0f, (_Float16)1024.0f};
        const f16x4s bmin = kg < 2 ? f16x4s{m01[0], m01[1], m23[0], m23[1]} : f16x4s{(_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f};
        f32x4 acc[TOK], accm[TOK];
#pragma unroll
        for (int tt = 0; tt < TOK; tt++) acc[tt] = accm[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 8; s++) {
            // {sc_s, sc_s} exactly: byte s under the exponent of 1024, minus 1024
            const f16x2s sc2 = sk_bits(__builtin_amdgcn_perm(0x64646464u, scb[s >> 2], 0x04000400u + 0x00010001u * (s & 3))) -
                               f16x2s{(_Float16)1024.0f, (_Float16)1024.0f};
            const f16x2s nb2 = sc2 * f16x2s{(_Float16)-1024.0f, (_Float16)-1024.0f};
            uint32_t v0, v1, b[4];
            Q::quants(raw, s, v0, v1);
            sk_scale4(v0, sc2, nb2, b[0], b[1]);
            sk_scale4(v1, sc2, nb2, b[2], b[3]);
            const f16x8s bv = __builtin_bit_cast(f16x8s, u32x4{b[0], b[1], b[2], b[3]});
#pragma unroll
            for (int tt = 0; tt < TOK; tt++) acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[tt][s], bv, acc[tt], 0, 0, 0);
            // one sub-block's B operand live at a time
            if constexpr (TOK > 1) __builtin_amdgcn_sched_barrier(0);
        }
        // the row partials of this wave: d * 2^E * S - dmin * 2^(E+5) * S_min
        float *pp = part + (size_t)buf * W * MP * 16 + (size_t)wave * MP * 16 + r16;
#pragma unroll
        for (int tt = 0; tt < TOK; tt++) {
            accm[tt] = __builtin_amdgcn_mfma_f32_16x16x16f16(amin[tt], bmin, accm[tt], 0, 0, 0);
#pragma unroll
            for (int j = 0; j < DPT; j++) {
                const float sv = HILO ? acc[tt][2 * j] + acc[tt][2 * j + 1] : acc[tt][j];
                const float sm = HILO ? accm[tt][2 * j] + accm[tt][2 * j + 1] : accm[tt][j];
                const float v = pe[tt][j] * fmaf(d, sv, -(32.0f * dmin) * sm);
                const uint32_t tok = tt * TPT + (HILO ? 2 * kg + j : 4 * kg + j);
                pp[tok * 16] = v;
            }
        }
        __syncthreads();
        // the waves' partials in order
        for (uint32_t i = t; i < MP * 16; i += 64 * W) {   // the launch's 64 W threads
            const uint32_t m = i >> 4, c = i & 15, row = (tile0 + tl * GR) * 16 + c;
            if (m < M && row < N) {
                // the W <= 16 waves' partials in wave order
                float v = ordered_sum<16>(part + (size_t)buf * W * MP * 16 + i, W, MP * 16);
                float *yp = a.y + (uint64_t)m * N + row;
                if (a.residual) v = *yp + v;
                *yp = v;
            }
        }
        buf ^= 1u;
    }
}

static uint32_t sk_cus()
{
    static uint32_t cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
        cus[dev] = (uint32_t)v;
    }
    return cus[dev];
}

template <class Q, bool HILO, int TOK, int NB>
static size_t sk_lds(uint32_t W)
{
    constexpr int MP = TOK * (HILO ? 8 : 16);
    return (size_t)W * NB * SkGeom<Q>::BUF + 2ull * W * MP * 16 * 4;
}

template <class Q, bool HILO, int TOK, int NB>
static hipError_t go_skinny_nb(const GemvArgs &a, hipStream_t s)
{
    const uint32_t W = a.K / 256, ntiles = (a.N + 15) / 16;
    constexpr bool PRE = TOK > 1;
    if (PRE)
        hipLaunchKernelGGL(skinny_encode_kernel<HILO>, dim3(W, TOK), dim3(64), 0, s, a.x, a.M, a.K, a.ws, (uint32_t)TOK);
    // up to one workgroup per CU, the tiles spread evenly over them
    const uint32_t per = (ntiles + sk_cus() - 1) / sk_cus();
    const uint32_t grid = (ntiles + per - 1) / per;
    const size_t lds = sk_lds<Q, HILO, TOK, NB>(W);
    hipLaunchKernelGGL((skinny_kernel<Q, HILO, TOK, NB, PRE>), dim3(grid), dim3(64 * W), lds, s, a, ntiles);
    return hipGetLastError();
}

// the deepest tile ring that fits in LDS (160 KB)
template <class Q, bool HILO, int TOK>
static hipError_t go_skinny(const GemvArgs &a, hipStream_t s)
{
    const uint32_t W = a.K / 256;
    constexpr size_t LDS_MAX = 160 * 1024;
    if (sk_lds<Q, HILO, TOK, 4>(W) <= LDS_MAX) return go_skinny_nb<Q, HILO, TOK, 4>(a, s);
    if (sk_lds<Q, HILO, TOK, 3>(W) <= LDS_MAX) return go_skinny_nb<Q, HILO, TOK, 3>(a, s);
    if (sk_lds<Q, HILO, TOK, 2>(W) <= LDS_MAX) return go_skinny_nb<Q, HILO, TOK, 2>(a, s);
    return hipErrorNotSupported;
}

bool skinny_supported(const GemvArgs &a)
{
    if (a.type != T_Q4_K && a.type != T_Q5_K) return false;
    if (a.M < 2 || a.M > 32 || a.K % 256 || a.K == 0) return false;
    // waves per workgroup: up to 16 with one A tile (M <= 8), up to 12 with
    // two, whose A operands need more registers
    if (a.K > (a.M <= 8 ? 4096u : 3072u)) return false;
    if (!a.ws || a.ws_bytes < sk_ws_bytes(2, a.K / 256)) return false;
    return a.w_bytes + RRR_READ_SLACK < SK_OOB;
}

template <class Q>
static hipError_t go_skinny_m(const GemvArgs &a, hipStream_t s)
{
    if (a.M <= 8) return go_skinny<Q, true, 1>(a, s);
    if (a.M <= 16) return go_skinny<Q, true, 2>(a, s);
    return go_skinny<Q, false, 2>(a, s);
}

hipError_t launch_skinny(const GemvArgs &a, hipStream_t s)
{
    if (!skinny_supported(a)) return hipErrorNotSupported;
    return a.type == T_Q4_K ? go_skinny_m<SkQ4K>(a, s) : go_skinny_m<SkQ5K>(a, s);
}

}  // namespace rrr
