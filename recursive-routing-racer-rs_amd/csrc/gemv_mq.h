// gemv_mq.h -- batch-1 K-quant GEMV on the int8 matrix cores: quant unit
// decoders, activation encoding and the per-workgroup body of the launch
// (gemv_mfma.hip).
//
// y[n] = sum_k x[k] * W[n][k] for Q4_K / Q5_K / Q6_K rows (phi4.rs:628-630),
// with the multiply-accumulate on v_mfma_i32_16x16x64_i8 instead of VALU FMAs.
//
// Activation encoding.  Each 16-element group of x is written in block
// floating point: the fixed-point value Q = rint(x * 2^(14-E)), with 2^E
// chosen from the group maximum M so that M / 2^E lies in [32, 64)
// (|Q| < 2^20), split into three signed int8 radix-256 digits
//     Q = d0 + 2^8 d1 + 2^16 d2.
// The encoding error is at most 2^(E-15) per element, i.e. below 2^-20 of
// the group maximum.
//
// Weights.  A K-quant super-block stores small integers q (Q4_K 0..15,
// Q5_K 0..31, Q6_K 0..63 with an offset of 32) and per-sub-block scales.
// The raw q values go straight into the MFMA B operand; the integer dot
// products C_t = sum q * d_t (t = 0, 1, 2) are exact, and
//     sum_k q_k x_k = 2^(E-14) * (C_0 + C_1 * 2^8 + C_2 * 2^16)
// is recombined in int32 (|C_2| < 2^14, |C_0|, |C_1| < 2^17) and scaled once
// per 16 elements.  The Q6_K offset (q - 32) is folded into the MFMA
// accumulator input as -32 * (sum of Q over the group); the Q4_K / Q5_K min
// term uses the f32 16-element sums of x.
//
// MFMA mapping (16x16x64, lane l: A row l%16, B column l%16, k-group l/16;
// C/D rows 4*(l/16)+r of column l%16 in register r):
//   B[k][n]  = q of weight row n (16 rows per workgroup) at k-set K_g,
//   A[m][k]  = digit (m%4) of x at K_g when m/4 == g (and m%4 < 3), else 0,
//   C[4g+r][n] = group constants of K_g: r = 0 the offset term, r = 3 the
//                group factor 2^(E-14) (bit pattern; A row 4g+3 is zero, so
//                it comes back unchanged in D),
// so lane (n, g) receives its own three partial dot products for row n and
// k-set K_g in registers 0..2 and the factor in register 3.  Each lane's
// k-set is 16 consecutive elements with one scale, applied after the MFMA.
//
// Work split: one workgroup per 16-row tile; wave w owns super-blocks
// [w*BPW, w*BPW + BPW) of the 16 rows.  A wave streams its 16 row pieces
// with 16-byte loads on consecutive lanes (contiguous runs of BPW blocks per
// row), encodes its own slice of x, stages both in its private LDS region and
// runs its MFMAs as soon as its own data has landed -- no workgroup barrier
// until the final cross-wave sum (plus one for the fused RMSNorm scale).
#pragma once

#include "act.h"

namespace rrr {

__device__ __forceinline__ u32x4 lds16(const uint8_t *L, uint32_t o)
{
    return *(const u32x4 *)(L + o);
}

// Q4_K (phi4.rs:481-510).  Lane group g takes qs pair g (bytes 32g..32g+31):
// low nibbles = sub-block 2g, high nibbles = sub-block 2g+1.
//   u = 0: low nibbles of bytes 0..15   (k-set 64g + 0..15)
//   u = 1: low nibbles of bytes 16..31  (64g + 16..31)
//   u = 2: high nibbles of bytes 0..15  (64g + 32..47)
//   u = 3: high nibbles of bytes 16..31 (64g + 48..63)
// Block value = d * sum_u sc[u] * S_u - dmin * sum_u mn[u] * X_u.
struct MqQ4K {
    static constexpr uint32_t BS = 144;
    static constexpr bool HAS_MIN = true, OFF32 = false;
    struct Raw { u32x4 hdr, qs0, qs1; };
    __device__ static uint32_t koff(uint32_t g, int u) { return 64 * g + 16 * u; }
    // o: LDS offset of the 16-byte aligned block piece
    __device__ static void load(Raw &w, const uint8_t *L, uint32_t o, uint32_t g)
    {
        w.hdr = lds16(L, o);
        w.qs0 = lds16(L, o + 16 + 32 * g);
        w.qs1 = lds16(L, o + 32 + 32 * g);
    }
    __device__ static void decode(const Raw &w, uint32_t g, i32x4 *bq, float *sc, float *mn, float &d, float &dmin)
    {
        d = h2f(w.hdr.x);
        dmin = h2f(w.hdr.x >> 16);
        uint32_t s0, m0, s1, m1;
        scale_min_pair_k4(g, w.hdr.y, w.hdr.z, w.hdr.w, s0, m0, s1, m1);
        sc[0] = sc[1] = (float)s0;
        sc[2] = sc[3] = (float)s1;
        mn[0] = mn[1] = (float)m0;
        mn[2] = mn[3] = (float)m1;
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
    __device__ static void load(Raw &w, const uint8_t *L, uint32_t o, uint32_t g)
    {
        w.hdr = lds16(L, o);
        w.qh0 = lds16(L, o + 16);
        w.qh1 = lds16(L, o + 32);
        w.qs0 = lds16(L, o + 48 + 32 * g);
        w.qs1 = lds16(L, o + 64 + 32 * g);
    }
    __device__ static void decode(const Raw &w, uint32_t g, i32x4 *bq, float *sc, float *mn, float &d, float &dmin)
    {
        d = h2f(w.hdr.x);
        dmin = h2f(w.hdr.x >> 16);
        uint32_t s0, m0, s1, m1;
        scale_min_pair_k4(g, w.hdr.y, w.hdr.z, w.hdr.w, s0, m0, s1, m1);
        sc[0] = sc[1] = (float)s0;
        sc[2] = sc[3] = (float)s1;
        mn[0] = mn[1] = (float)m0;
        mn[2] = mn[3] = (float)m1;
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
// MFMA unsigned; the offset comes in through the accumulator input.
struct MqQ6K {
    static constexpr uint32_t BS = 210;
    static constexpr bool HAS_MIN = false, OFF32 = true;
    struct Raw { u32x4 qa, qb, qh; u32x2 sc; uint32_t d; };
    __device__ static uint32_t koff(uint32_t g, int u) { return 128 * (g >> 1) + 32 * u + 16 * (g & 1); }
    // o: LDS offset of the block piece, staged 16-byte aligned
    __device__ static void load(Raw &w, const uint8_t *L, uint32_t o, uint32_t g)
    {
        const uint32_t g6 = g >> 1, l0 = 16 * (g & 1);
        w.qa = lds16(L, o + 64 * g6 + l0);
        w.qb = lds16(L, o + 64 * g6 + 32 + l0);
        w.qh = lds16(L, o + 128 + 32 * g6 + l0);
        w.sc = *(const u32x2 *)(L + o + 192 + 8 * g6);
        w.d = *(const uint16_t *)(L + o + 208);
    }
    __device__ static void decode(const Raw &w, uint32_t g, i32x4 *bq, float *sc, float *, float &d, float &)
    {
        d = h2f(w.d);
        const uint32_t h = g & 1;
        sc[0] = (float)(int8_t)byte_of(w.sc.x, h);
        sc[1] = (float)(int8_t)byte_of(w.sc.x, h + 2);
        sc[2] = (float)(int8_t)byte_of(w.sc.y, h);
        sc[3] = (float)(int8_t)byte_of(w.sc.y, h + 2);
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

// Fixed-point form of one float4 of activations: Q = rint(x * 2^(14-E))
// (|Q| < 2^20) as three signed radix-256 digits Q = d0 + 2^8 d1 + 2^16 d2.
// fma(x, 2^(14-E), 1.5 * 2^23) lands in [2^23, 2^24), where the f32 spacing
// is 1, so it is the exactly rounded 1.5 * 2^23 + Q and its bit pattern is
// 0x4B400000 + Q.  Adding the bias 0x808080 makes every byte c_t of
// Qb = Q + 0x808080 (< 2^24) the digit d_t = c_t - 128, i.e. the int8 byte
// c_t ^ 0x80.  Returns the digit planes (four int8 per dword, plane t = byte
// t) and the sum of the four biased values.
__device__ __forceinline__ void encode4(const float4 &v, float scale, uint32_t &p0, uint32_t &p1, uint32_t &p2,
                                        uint32_t &qbsum)
{
    constexpr float MAGIC = 12582912.0f;                       // 1.5 * 2^23
    constexpr uint32_t REBIAS = 0x00808080u - 0x4B400000u;     // mod 2^32
    const uint32_t q0 = __float_as_uint(__builtin_fmaf(v.x, scale, MAGIC)) + REBIAS;
    const uint32_t q1 = __float_as_uint(__builtin_fmaf(v.y, scale, MAGIC)) + REBIAS;
    const uint32_t q2 = __float_as_uint(__builtin_fmaf(v.z, scale, MAGIC)) + REBIAS;
    const uint32_t q3 = __float_as_uint(__builtin_fmaf(v.w, scale, MAGIC)) + REBIAS;
    qbsum = (q0 + q1) + (q2 + q3);
    // v_perm: selector bytes 0..3 take bytes of the second operand, 4..7 of
    // the first, 0x0c gives 0
    p0 = (__builtin_amdgcn_perm(q1, q0, 0x0c0c0400u) | __builtin_amdgcn_perm(q3, q2, 0x04000c0cu)) ^ 0x80808080u;
    p1 = (__builtin_amdgcn_perm(q1, q0, 0x0c0c0501u) | __builtin_amdgcn_perm(q3, q2, 0x05010c0cu)) ^ 0x80808080u;
    p2 = (__builtin_amdgcn_perm(q1, q0, 0x0c0c0602u) | __builtin_amdgcn_perm(q3, q2, 0x06020c0cu)) ^ 0x80808080u;
}

// Butterflies within a quad of lanes (DPP quad_perm, no LDS traffic).
__device__ __forceinline__ float quad_max(float v)
{
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false)));
    return fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false)));
}
__device__ __forceinline__ float quad_sum(float v)
{
    v = v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));
    return v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));
}
__device__ __forceinline__ uint32_t quad_sum_u32(uint32_t v)
{
    v = v + (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);
    return v + (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);
}

// Wave-private LDS layout of one wave (BPW super-blocks of 16 rows):
//   weights: 16 rows x RS bytes, block j of row r at r*RS + j*LB (16-byte
//            aligned pieces of UPB units; Q6_K pieces carry 14 bytes of the
//            next block in their last unit).  The loads are block by block:
//            load slot s of block j covers rows s*RPS .. s*RPS + RPS-1 of
//            that block (lane l: unit l % UPB of row l / UPB), so a lane's
//            offsets are fixed and only a uniform per-slot offset moves, and
//            a block's MFMAs can start while the next block is still landing.
//   digits:  per token m, 3 planes x DG bytes (plane p, local element e at
//            (3 m + p) * DG + e)
//   aux:     per token and 16-element group 16 bytes = MFMA accumulator
//            input {-32 * sum Q (Q6_K only, else 0), 0, 0, bits of 2^(E-14)}
//   gsum:    per token and group the f32 sum of x (Q4_K / Q5_K min term)
//   zero:    (MT > 1) 16 zero bytes, the A operand of the lanes that supply
//            no digit row when A is read from LDS before each MFMA (one read
//            for every lane, no branch)
// MT tokens (rows of x) share every weight block: the multi-token form
// (MT > 1) encodes each token's slice and runs one MFMA per token and k-set
// on the same B operand.
// Waves of a workgroup for K columns at BPW super-blocks per wave (at least
// 4, one per SIMD).  The launchers size the workgroup with it and the kernel
// derives its wave count from it: reading blockDim.x would cost a dependent
// load of the dispatch's hidden arguments at kernel entry.
__host__ __device__ constexpr uint32_t mq_waves(uint32_t K, uint32_t BPW)
{
    return (K / 256 + BPW - 1) / BPW > 4u ? (K / 256 + BPW - 1) / BPW : 4u;
}

template <class Q, int BPW, int MT = 1>
struct MwGeom {
    static constexpr uint32_t UPB = (Q::BS + 15) / 16;            // 16-byte units per block piece
    static constexpr uint32_t LB = 16 * UPB;
    static constexpr uint32_t RS = (BPW * LB) % 32 == 0 ? BPW * LB + 16 : BPW * LB;  // odd multiple of 16
    static constexpr uint32_t RPS = 64 / UPB;                      // rows per load slot
    static constexpr uint32_t DG = BPW * 256;
    static constexpr uint32_t NGW = BPW * 16;
    static constexpr uint32_t D_OFF = 16 * RS;
    static constexpr uint32_t A_OFF = D_OFF + MT * 3 * DG;
    static constexpr uint32_t G_OFF = A_OFF + MT * 16 * NGW;
    static constexpr uint32_t Z_OFF = G_OFF + MT * 4 * NGW;       // 16 zero bytes (A of the lanes without a digit row)
    static constexpr uint32_t BYTES = Z_OFF + (MT > 1 ? 16 : 0);  // multiple of 16
};

// Odd Q6_K blocks (210 bytes) start 2 bytes past a 4-byte boundary, and
// 16-byte loads that are only 2-byte aligned take a slow path (~1.5 us more
// per 20 MB).  Such a block's units are loaded from 2 bytes earlier and moved
// down by 2 bytes in registers, the top 2 bytes coming from the next lane
// (the block's next unit; for the last unit they fall past byte 222 of the
// block, which is never read).  `sh` is 0 or 2; every lane of the wave
// calls it.
__device__ __forceinline__ u32x4 q6_realign(const u32x4 &v, uint32_t sh)
{
    const uint32_t nx = (uint32_t)__builtin_amdgcn_mov_dpp((int)v.x, 0x130, 0xF, 0xF, false);   // wave_shl:1
    return u32x4{__builtin_amdgcn_alignbyte(v.y, v.x, sh), __builtin_amdgcn_alignbyte(v.z, v.y, sh),
                 __builtin_amdgcn_alignbyte(v.w, v.z, sh), __builtin_amdgcn_alignbyte(nx, v.w, sh)};
}

__device__ __forceinline__ void wave_lds_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Scalar offset of a load past every weight byte (the path requires
// w_bytes + RRR_READ_SLACK < MQ_OOB): such loads return zeros and move no data.
constexpr uint32_t MQ_OOB = 0x80000000u;

// A tile is tr <= 16 rows (the MFMA's 16 columns, the rest idle), chosen by
// the launcher so that the tiles spread evenly over the CUs (K <= 4096,
// N = 3072: 256 tiles of 12 rows rather than 192 of 16).
// Persistent form (MULTI): workgroup b takes the tiles b, b + G, ...
// (G = gridDim.x) with the same wave <-> K-slice split for every tile, so the
// activation slice is encoded once per workgroup and, with one super-block per
// wave, the MFMA A operands and accumulator inputs stay in registers.  A
// block's registers take the next tile's loads of that block as soon as the
// block is staged in LDS, before it is multiplied.  The single-tile form (one
// tile per workgroup) issues no prefetch: even loads past the buffer end cost
// texture-addresser time.  Row sums are added over the waves in wave order,
// so results depend on neither form, G nor the number of waves.
// TR: the most rows a tile of the launch has (tr <= TR <= 16); a wave issues
// the load slots that cover TR rows, so a launch of shorter tiles issues no
// empty slots.
// PAIR (a.pair, MULTI, tr = 16): W holds 2N rows, N gate rows then N up rows
// (the ffn_up matmul into the 2F gate_up buffer that silu_gate reads,
// phi4.rs:1025-1029); ntiles counts 16-row pairs, and the workgroup's tile
// 2q is gate rows 16P .. 16P+15 of its q-th pair P, tile 2q+1 the matching up
// rows (each a contiguous run of rows, as in a plain launch).  It writes
// y[16P + r] = silu(gate) * up with the RRR_ACT_SILU_GATE formula, on the
// same row sums a plain launch computes: the result is bitwise what a GEMV
// into 2N rows followed by that activation gives.
// ROPE (a.rope_on, tr even): the rows go out in pairs through
// rope_store_pair (act.h), the rope_kv_store of the token's qkv row; each
// row's value is the sum a plain launch stores.  The rope_dim rotation
// coefficients sit in LDS past the row partials (the launcher adds their
// rope_dim floats).
// Sum of the W <= 16 wave partials p[0], p[16], ..., p[16 (W - 1)] in wave
// order (all requested before the first add).
__device__ __forceinline__ float waves_sum(const float *p, uint32_t W) { return ordered_sum<16>(p, W, 16); }

// Phase timestamps (the STAMPS instantiation only, rrr_probe_gemv_phases):
// the 100 MHz constant clock read once `dep` is available, kept in scalar
// registers and stored at the end, so that no store enters the memory queue
// between the phases.  Slot k of a wave (a.stamps[(block * W + wave) * 16 + k]):
// 0 start, 1 activations landed, 2 after the fused RMSNorm scale, 3
// activations encoded, 4 / 6 first tile's block 0 / 1 staged, 5 / 7 its
// MFMAs done, 8-11 the same for the last tile (several tiles per workgroup),
// 12 the wave's partials written, 13 past the final barrier, 14 end.
__device__ __forceinline__ uint64_t phase_stamp(float dep)
{
    uint64_t t;
    asm volatile("s_memrealtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t) : "v"(dep) : "memory");
    return t;
}

// MT > 1: the multi-token form (plain activations; a.M <= MT tokens, rows m
// of x at x + m K, outputs at y + m N; tokens past a.M read the last row and
// store nothing).
template <class Q, int BPW, int ACT, bool MULTI, int TR = 16, bool PAIR = false, bool ROPE = false,
          bool STAMPS = false, int MT = 1>
__device__ __forceinline__ void mq_body(const GemvArgs &a, uint32_t ntiles, uint32_t tr)
{
    extern __shared__ float smem[];
    using G = MwGeom<Q, BPW, MT>;
    static_assert(TR >= 1 && TR <= 16, "tile rows");
    static_assert(MT == 1 || (ACT == ACT_PLAIN && !PAIR && !ROPE && !STAMPS), "multi-token form: plain rows");
    constexpr int SB = (TR + (int)G::RPS - 1) / (int)G::RPS;     // load slots of one block
    // A operands in registers, except in the persistent two-block form, whose
    // next-tile prefetch registers leave no room for them (it reads them from
    // LDS before each MFMA)
    constexpr bool AREG = (BPW == 1 || !MULTI) && MT == 1;
    constexpr int AJ = AREG ? BPW : 1;
    const uint32_t K = a.K, B = K / 256;
    const uint32_t W = mq_waves(K, BPW), NT = 64 * W;   // the launch's workgroup
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint32_t n = lane & 15, g = lane >> 4;
    uint64_t stamp[15] = {};
    auto mark = [&](int k, float dep) {
        if constexpr (STAMPS) stamp[k] = phase_stamp(dep);
    };
    auto mark_flush = [&]() {
        if constexpr (STAMPS) {
            if (lane == 0)
                for (int k = 0; k < 15; k++) a.stamps[((size_t)blockIdx.x * W + wave) * 16 + k] = stamp[k];
        }
    };
    mark(0, 0.0f);
    const uint32_t GR = gridDim.x, tile0 = blockIdx.x;
    static_assert(!PAIR || (MULTI && TR == 16), "a pair is a gate tile and an up tile of 16 rows");
    const uint32_t nown = tile0 < ntiles ? (ntiles - tile0 + GR - 1) / GR : 0u;   // tiles (PAIR: pairs) of this workgroup
    const uint32_t ntl = MULTI ? (PAIR ? 2 * nown : nown) : 1u;                    // tiles of this workgroup
    uint8_t *L = (uint8_t *)smem + wave * G::BYTES;              // this wave's region
    float *red = (float *)((uint8_t *)smem + W * G::BYTES);      // 16: RMSNorm slice sums
    float *part = red + 16;                                      // ntl x MT x W x 16 per-wave row partials

    const uint32_t row_bytes = B * Q::BS;
    // every buffer has RRR_READ_SLACK readable bytes past its end: a Q6_K
    // piece's last unit runs 14 bytes past its block
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.W, a.w_bytes + RRR_READ_SLACK);
    const uint32_t b0 = wave * BPW;                              // first super-block of this wave
    const uint32_t nb = b0 < B ? min((uint32_t)BPW, B - b0) : 0u;

    // weight units of this wave's blocks (layout above); lanes past RPS rows,
    // rows past the tile's tr rows and blocks past nb read nothing (an
    // out-of-range offset: no memory request)
    const uint32_t rsel = min(lane / G::UPB, G::RPS - 1), ul = lane - (lane / G::UPB) * G::UPB;
    const bool lane_ok = lane < G::RPS * G::UPB;
    constexpr bool REALIGN = Q::BS % 4 != 0;
    uint32_t voff[BPW], sh[BPW];
#pragma unroll
    for (int j = 0; j < BPW; j++) {
        const uint32_t blk = b0 + min((uint32_t)j, nb ? nb - 1 : 0u);
        sh[j] = REALIGN ? (blk * Q::BS) & 3u : 0u;             // 0 or 2 bytes (the same for every row)
        voff[j] = rsel * row_bytes + blk * Q::BS - sh[j] + 16 * ul;
    }
    const uint32_t loff = rsel * G::RS + 16 * ul;
    u32x4 wa[BPW][SB];
    // first row of this workgroup's tile tl in W, and its rows
    auto tile_row0 = [&](uint32_t tl) -> uint32_t {
        if constexpr (PAIR) return 16 * (tile0 + (tl >> 1) * GR) + ((tl & 1) ? a.N : 0u);
        return (tile0 + tl * GR) * tr;
    };
    auto tile_rows = [&](uint32_t tl) -> uint32_t {
        if constexpr (PAIR) return min(16u, a.N - 16 * (tile0 + (tl >> 1) * GR));
        return tr;
    };
    auto issue = [&](int j, uint32_t tl) {
        const uint32_t tb = tl < ntl ? tile_row0(tl) * row_bytes : MQ_OOB;
        const uint32_t rows = tl < ntl ? tile_rows(tl) : 0u;
#pragma unroll
        for (int s = 0; s < SB; s++)
            wa[j][s] = bload16_nt_so(rs, lane_ok && j < (int)nb && s * G::RPS + rsel < rows ? voff[j] : MQ_OOB,
                                     tb + s * G::RPS * row_bytes);
    };

    // The loads below are unconditional (clamped indices, out-of-range scalar
    // offsets): loads under a branch make the compiler wait for every
    // outstanding load at the join.
    // the residual of this thread's first output row, read now rather than
    // on the kernel's tail (a clamped row when there is none)
    const uint32_t row_first = PAIR ? 0u : min((tile0 + (t >> 4) * GR) * tr + (t & 15), a.N - 1);
    const float yres = PAIR || MT > 1 ? 0.0f : a.y[row_first];
    // 1. this wave's activation inputs: float4 lane + 64 j of its slice, of
    // each token
    float4 xa[MT][BPW], xb[MT][BPW];
#pragma unroll
    for (int j = 0; j < BPW; j++) {
        const uint32_t k4 = min(b0 * 256 + 4 * (lane + 64 * j), K - 4);
        if constexpr (MT == 1) {
            src_load4<ACT>(a, k4, xa[0][j], xb[0][j]);
        } else {
#pragma unroll
            for (int m = 0; m < MT; m++) xa[m][j] = *(const float4 *)(a.x + (size_t)min((uint32_t)m, a.M - 1) * K + k4);
        }
    }

    // every wave's activation loads enter the memory pipeline before any
    // weight load of the workgroup (a bare barrier: no wait on the loads)
    __builtin_amdgcn_s_barrier();
#pragma unroll
    for (int j = 0; j < BPW; j++) issue(j, 0);
    // the weight loads leave before any use of the activations: the
    // scheduler would otherwise hoist the sum of squares (or the encoding)
    // above them, behind a wait for the activation loads to land
    __builtin_amdgcn_sched_barrier(0);
    // 2. fused RMSNorm: the wave's slice of x is slice `wave` of the canonical
    // sum-of-squares split (BPW float4s per lane is its P = ceil(K / 4096)
    // for K <= 8192); the slice sums are added in wave order (waves without
    // a super-block add +0)
    float inv = 1.0f;
    mark(1, xa[0][0].x);
    if constexpr (ACT == ACT_RMSNORM) {
        float sq = 0.0f;
#pragma unroll
        for (int j = 0; j < BPW; j++)
            if (j < (int)nb) sq = sumsq4(xa[0][j], sq);
        sq = wave_sum(sq);
        if (lane == 0) red[wave] = sq;
        __syncthreads();
        // the W slice sums in order, all requested before the first add (a
        // runtime-length loop waits out one LDS round trip per wave)
        inv = rms_inv(ordered_sum<16>(red, W, 1), K, a.eps);
    }

    mark(2, xa[0][0].x + inv);
    // 3. activation staging of this wave's slice (of each token)
#pragma unroll
    for (int mj = 0; mj < MT * BPW; mj++) {
        const int m = mj / BPW, j = mj % BPW;
        const uint32_t f = lane + 64 * j;                        // local float4 index
        uint8_t *Lm = L + m * (3 * G::DG);                       // token m's digit planes
        const uint32_t am = m * (16 * G::NGW), gm = m * (4 * G::NGW);   // its aux and group sums
        const float4 v = xform4<ACT>(xa[m][j], xb[m][j], inv);
        const float mx = quad_max(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        int e = 0;
        if (mx > 0.0f && __builtin_isfinite(mx)) {
            int ex;
            (void)frexpf(mx, &ex);
            e = ex - 6;  // mx / 2^e in [32, 64)
        }
        uint32_t p0, p1, p2, qb;
        encode4(v, ldexpf(1.0f, 14 - e), p0, p1, p2, qb);
        *(uint32_t *)(Lm + G::D_OFF + 4 * f) = p0;
        *(uint32_t *)(Lm + G::D_OFF + G::DG + 4 * f) = p1;
        *(uint32_t *)(Lm + G::D_OFF + 2 * G::DG + 4 * f) = p2;
        i32x4 ax = {0, 0, 0, 0};
        if constexpr (Q::OFF32) {
            // sum (q - 32) Q = sum q Q - 32 sum Q: the second term enters the
            // weight-1 plane's accumulator (int32 wrap-around is harmless, the
            // recombined value is within +-2^29)
            ax[0] = -32 * (int)(quad_sum_u32(qb) - 16u * 0x00808080u);
        } else {
            const float sv = quad_sum((v.x + v.y) + (v.z + v.w));
            if ((lane & 3) == 0) *(float *)(L + G::G_OFF + gm + f) = sv;  // group f / 4
        }
        ax[3] = __float_as_int(__builtin_isfinite(mx) ? ldexpf(1.0f, e - 14) : __builtin_nanf(""));
        if ((lane & 3) == 0) *(i32x4 *)(L + G::A_OFF + am + 4 * f) = ax;
    }
    if constexpr (MT > 1) {
        if (lane == 0) *(i32x4 *)(L + G::Z_OFF) = i32x4{0, 0, 0, 0};
    }
    wave_lds_sync();
    mark(3, 0.0f);

    // A operands (zero in the non-live lanes), accumulator inputs and group
    // sums of the slice, into registers while the weights are in flight; lane
    // (n, g) supplies A = its digit row (m = n: plane n%4 of group n/4) when
    // n/4 == g
    const bool a_live = (n >> 2) == g && (n & 3) < 3;
    const uint32_t a_base = G::D_OFF + (n & 3) * G::DG;
    i32x4 av[AJ][4], aux[AJ][4];
    float gs[AJ][4];
#pragma unroll
    for (int j = 0; j < AJ; j++)
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const uint32_t grp = j * 16 + Q::koff(g, u) / 16;
            av[j][u] = i32x4{0, 0, 0, 0};
            aux[j][u] = *(const i32x4 *)(L + G::A_OFF + 16 * grp);
            gs[j][u] = Q::HAS_MIN ? *(const float *)(L + G::G_OFF + 4 * grp) : 0.0f;
        }
    if (a_live) {
#pragma unroll
        for (int j = 0; j < AJ; j++)
#pragma unroll
            for (int u = 0; u < 4; u++) av[j][u] = *(const i32x4 *)(L + a_base + j * 256 + Q::koff(g, u));
    }
    // multi-token form, one super-block a wave: every token's A operands in
    // registers for all tiles (the group factors or accumulator inputs and
    // the group sums are read from LDS per MFMA: kept in registers too, they
    // would not fit)
    constexpr bool AREGT = MT > 1 && BPW == 1;
    i32x4 avt[AREGT ? MT : 1][4];
    if constexpr (AREGT) {
#pragma unroll
        for (int m = 0; m < MT; m++)
#pragma unroll
            for (int u = 0; u < 4; u++)
                avt[m][u] = *(const i32x4 *)(L + (a_live ? m * (3 * G::DG) + a_base + Q::koff(g, u) : G::Z_OFF));
    }

    // ROPE: the position's rotation coefficients (pair j by thread j, j + NT,
    // ...; read after the final barrier), here where the wave would wait for
    // its first weight block anyway: computed before the RMSNorm barrier, they
    // held every wave back by their latency
    float *coef = part + ntl * W * 16;
    if constexpr (ROPE) {
        for (uint32_t j = t; j < a.rope.rope_dim / 2; j += NT) rope_coef(j, a.rope.pos, a.rope, coef[2 * j], coef[2 * j + 1]);
    }

    // 4. per tile, block by block: the block's units to LDS (its registers
    // then take the next tile's loads of the block), its MFMAs; row partials
    // to part[]
    auto process = [&](uint32_t tl) {
        float acc[MT];
#pragma unroll
        for (int m = 0; m < MT; m++) acc[m] = 0.0f;
#pragma unroll
        for (int j = 0; j < BPW; j++) {
            wave_lds_sync();
#pragma unroll
            for (int s = 0; s < SB; s++) {
                u32x4 v = wa[j][s];
                if constexpr (REALIGN) v = q6_realign(v, sh[j]);
                if (lane_ok && j < (int)nb && s * G::RPS + rsel < tr)
                    *(u32x4 *)(L + loff + s * G::RPS * G::RS + j * G::LB) = v;
            }
            if constexpr (MULTI) issue(j, tl + 1);
            wave_lds_sync();
            if (tl == 0) mark(4 + 2 * j, 0.0f);
            else if (tl + 1 == ntl) mark(8 + 2 * j, 0.0f);
            if (j < (int)nb) {
                typename Q::Raw raw;
                Q::load(raw, L, n * G::RS + j * G::LB, g);
                i32x4 bq[4];
                float sc[4], mn[4], d, dmin;
                Q::decode(raw, g, bq, sc, mn, d, dmin);
#pragma unroll
                for (int m = 0; m < MT; m++) {
                    float acc_s = 0.0f, acc_m = 0.0f;
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        i32x4 A, C;
                        float gsum, fac = 0.0f;
                        if constexpr (AREG) {
                            A = av[j][u];
                            C = aux[j][u];
                            gsum = gs[j][u];
                        } else {
                            const uint32_t grp = j * 16 + Q::koff(g, u) / 16;
                            if constexpr (AREGT) {
                                A = avt[m][u];
                            } else if constexpr (MT == 1) {
                                A = i32x4{0, 0, 0, 0};
                                if (a_live) A = *(const i32x4 *)(L + a_base + j * 256 + Q::koff(g, u));
                            } else {
                                A = *(const i32x4 *)(L + (a_live ? m * (3 * G::DG) + a_base + j * 256 + Q::koff(g, u)
                                                                 : G::Z_OFF));
                            }
                            const uint8_t *cp = L + G::A_OFF + m * (16 * G::NGW) + 16 * grp;
                            // Q4_K / Q5_K: the accumulator input {0, 0, 0, factor}
                            // becomes the constant 0 and the factor a plain
                            // read (the value the MFMA would pass through)
                            if constexpr (Q::OFF32)
                                C = *(const i32x4 *)cp;
                            else {
                                C = i32x4{0, 0, 0, 0};
                                fac = *(const float *)(cp + 12);
                            }
                            gsum = Q::HAS_MIN ? *(const float *)(L + G::G_OFF + m * (4 * G::NGW) + 4 * grp) : 0.0f;
                        }
                        const i32x4 cc = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                            __builtin_bit_cast(i8x16, A), __builtin_bit_cast(i8x16, bq[u]), C, 0, 0, 0);
                        const int T = cc[0] + cc[1] * 256 + cc[2] * 65536;
                        if (AREG || Q::OFF32) fac = __int_as_float(cc[3]);
                        acc_s = fmaf(sc[u], fac * (float)T, acc_s);
                        if constexpr (Q::HAS_MIN) acc_m = fmaf(mn[u], gsum, acc_m);
                    }
                    acc[m] = fmaf(d, acc_s, acc[m]);
                    if constexpr (Q::HAS_MIN) acc[m] = fmaf(-dmin, acc_m, acc[m]);
                }
            }
            if (tl == 0) mark(5 + 2 * j, acc[0]);
            else if (tl + 1 == ntl) mark(9 + 2 * j, acc[0]);
        }
        // the 4 k-groups of a row (lanes n, n+16, n+32, n+48), by lane swaps
#pragma unroll
        for (int m = 0; m < MT; m++) {
            acc[m] = lanes4_sum(acc[m]);
            if (lane < 16) part[((tl * MT + m) * W + wave) * 16 + lane] = acc[m];
        }
        if (tl + 1 == ntl) mark(12, acc[0]);
    };
    if constexpr (MULTI) {
        for (uint32_t tl = 0; tl < ntl; tl++) process(tl);
    } else {
        process(0);
    }

    // 5. rows of every tile of this workgroup: the W waves' partials in order
    __syncthreads();
    mark(13, 0.0f);
    if constexpr (PAIR) {
        for (uint32_t i = t; i < nown * 16; i += NT) {
            const uint32_t q = i >> 4, r = i & 15, row = (tile0 + q * GR) * 16 + r;
            if (row < a.N) {
                const float *pg = part + 2 * q * W * 16 + r, *pu = pg + W * 16;
                a.y[row] = silu_fast(waves_sum(pg, W)) * waves_sum(pu, W);
            }
        }
        if constexpr (STAMPS) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            mark(14, 0.0f);
            mark_flush();
        }
        return;
    }
    if constexpr (ROPE) {
        static_assert(!PAIR, "rope epilogue on a plain row layout");
        for (uint32_t i = t; i < ntl * 8; i += NT) {
            const uint32_t tl = i >> 3, r = 2 * (i & 7), row = (tile0 + tl * GR) * tr + r;
            if (r < tr && row < a.N) {
                rope_store_pair(a, row, waves_sum(part + tl * W * 16 + r, W), waves_sum(part + tl * W * 16 + r + 1, W),
                                coef);
            }
        }
        if constexpr (STAMPS) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            mark(14, 0.0f);
            mark_flush();
        }
        return;
    }
    for (uint32_t i = t; i < ntl * MT * 16; i += NT) {
        const uint32_t tm = i >> 4, tl = tm / MT, m = tm % MT, r = i & 15, row = (tile0 + tl * GR) * tr + r;
        if (r < tr && row < a.N && (MT == 1 || m < a.M)) {
            float *yo = a.y + (size_t)m * a.N + row;
            float v = waves_sum(part + tm * W * 16 + r, W);
            if (a.residual) v = (MT == 1 && i == t ? yres : *yo) + v;
            *yo = v;
        }
    }
    if constexpr (STAMPS) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        mark(14, 0.0f);
        mark_flush();
    }
}

// Rows per tile and tiles per workgroup for `wgs` workgroups: the fewest
// tiles per workgroup (k, at most per_max) that cover N with tiles of at most
// 16 rows, then the smallest tile (tr rows, at least min_tr) that still does,
// so that the tiles split evenly.
inline void mq_tiles(uint32_t N, uint32_t wgs, uint32_t per_max, uint32_t min_tr, uint32_t &tr, uint32_t &ntiles,
                     uint32_t &per)
{
    uint32_t k = (N + 16 * wgs - 1) / (16 * wgs);
    k = max(1u, min(k, per_max));
    tr = max(min_tr, min(16u, (N + k * wgs - 1) / (k * wgs)));
    ntiles = (N + tr - 1) / tr;
    per = min((ntiles + wgs - 1) / wgs, per_max);
}

inline uint32_t device_cus()
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

}  // namespace rrr
