// gemm.hip -- prefill dequant-GEMM: Y[M][N] = X[M][K] . W[N][K]^T (or Y +=, the
// residual of the layer folded in) with X in f16 (bf16 activations are
// converted to f16 rows once per call, below) and W in raw Q4_K / Q5_K / Q6_K
// super-blocks (the batched shape of phi4.rs:1257-1268 at prompt length; the
// reference has no MFMA kernel for it).
//
// Workgroup: 512 threads.  Waves 0-3 (2 x 2) each own a (BM/2) x (BN/2)
// block of 32x32 v_mfma_f32_32x32x16_f16 tiles with fp32 accumulators, and
// load X: 16-byte LDS DMA straight from global memory, GEMM_NA - 1 steps
// ahead, into a ring of GEMM_NA X buffers.  Waves 4-7 stage the weights.
//
// K steps of BK elements.  Per step each staging thread dequantizes 32
// elements (two runs of 16) of one weight row into an fp16 LDS tile.  The
// dequant runs in packed fp16: v_perm places each quant byte q under the
// exponent of 1024 (f16 0x64qq = 1024 + q), an exact v_pk_add removes the 1024
// (1056 for Q6_K's offset), and one v_pk_fma / v_pk_mul applies the sub-block
// scale and min (phi4.rs:444-542: w = d*sc*q - dmin*m, w = d*sc*(q - 32)) with
// one rounding to fp16; fp16 weights keep the product error near 2^-11 per
// weight (bf16 would be 2^-8).  The weight tile is double-buffered in LDS:
// step s+1 is staged while the MFMA waves work on step s; a ring of four
// register sets keeps the weight loads of the next three steps in flight.
//
// Tile order: the M/BM tiles of one N tile get workgroup ids congruent mod 8,
// so they run on the same XCD and the weight tile is fetched from HBM once.
//
// Split K: when the BM x BN tiles are too few to fill the CUs (a 512-token
// prompt against N = 3072 or 5120), workgroup (tile, ks) of S splits takes
// super-blocks [ks * q + min(ks, r), (ks + 1) * q + min(ks + 1, r)) of the
// B = K / 256 (q = B / S, r = B % S: the first r splits one more) and
// writes its fp32 partial to a workspace; gemm_splitk_reduce then adds the S partials of each output in
// split order (deterministic), applies the row scale and stores or adds to Y.
#include "device_common.h"
#include "internal.h"

namespace rrr {

typedef _Float16 f16x8v __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));

// Scalar offset past every input byte (the launcher requires smaller buffers):
// loads of the step after the last return zeros and move no data.
constexpr uint32_t GM_OOB = 0x80000000u;

// X (A) buffers of the ring the MFMA waves load X into, GEMM_NA - 1 steps
// ahead
constexpr int GEMM_NA = 3;
// LDS of a BM x BN tile with K steps of BK: GEMM_NA X buffers and two weight
// (B) buffers, fp16
template <int BM, int BN, int BK>
constexpr size_t gemm_lds_bytes = (GEMM_NA * (size_t)BM + 2 * BN) * BK * 2;

__device__ __forceinline__ uint32_t pk_f16(float a, float b)
{
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
}
// f16 with round-to-nearest-even for the dequantized weights
__device__ __forceinline__ uint32_t pk_f16_rn(float a, float b)
{
    const f16x2v h = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, h);
}

__device__ __forceinline__ f16x2v f16x2_bits(uint32_t v) { return __builtin_bit_cast(f16x2v, v); }
__device__ __forceinline__ uint32_t bits_f16x2(f16x2v v) { return __builtin_bit_cast(uint32_t, v); }

// Four quant bytes (each < 1024) of one dword -> two fp16 pairs (1024 + q)
__device__ __forceinline__ void q4_to_f16(uint32_t v, f16x2v &p01, f16x2v &p23)
{
    p01 = f16x2_bits(__builtin_amdgcn_perm(0x64646464u, v, 0x04010400u));
    p23 = f16x2_bits(__builtin_amdgcn_perm(0x64646464u, v, 0x04030402u));
}

// Units of 32 * NP elements of one super-block row: part p (0 or 1) of
// 64-element chunk c holds the two runs of 16 elements 64c + 16p + (0..15)
// and 64c + 32 + 16p + (0..15), which come from the same 16 quant bytes (low
// and high nibbles), so the two parts of a chunk load disjoint bytes.  A unit
// is parts p0 .. p0 + NP - 1 of one chunk (the kernel below takes NP = 1: two
// staging threads per chunk; NP = 2 is the whole chunk with one header load).
// Loads take the row and in-block offset in voff and the block start in the
// scalar offset blk.  dequant() writes 16 dwords of fp16 pairs per part: run 0
// in element order, then run 1.

// Q4_K (phi4.rs:481-510): element 64g + 32h + l is the h-th nibble of qs[32g + l]
// of sub-block 2g + h; w = (d*sc)*q - dmin*m.
template <int NP>
struct GqQ4K {
    static constexpr uint32_t BS = 144;
    struct Raw { u32x4 hdr, q[NP]; };
    __device__ static void load(Raw &r, __amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t blk, uint32_t c, uint32_t p0)
    {
        r.hdr = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, blk, 0);
#pragma unroll
        for (int k = 0; k < NP; k++)
            r.q[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + 16 + 32 * c + 16 * (p0 + k), blk, 0);
    }
    __device__ static void dequant(const Raw &r, uint32_t c, uint32_t, uint32_t *out)
    {
        const f16x2v K2 = {(_Float16)1024.0f, (_Float16)1024.0f};
#pragma unroll
        for (int h = 0; h < 2; h++) {
            uint32_t sc, mn;
            scale_min_k4(2 * c + h, r.hdr.y, r.hdr.z, r.hdr.w, sc, mn);
            const _Float16 A = (_Float16)__fmul_rn(h2f(r.hdr.x), (float)sc);
            const _Float16 Bn = (_Float16)(-__fmul_rn(h2f(r.hdr.x >> 16), (float)mn));
            const f16x2v A2 = {A, A}, B2 = {Bn, Bn};
#pragma unroll
            for (int k = 0; k < NP; k++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t v = (r.q[k][i] >> (4 * h)) & 0x0F0F0F0Fu;
                    f16x2v p01, p23;
                    q4_to_f16(v, p01, p23);
                    out[16 * k + 8 * h + 2 * i] = bits_f16x2(__builtin_elementwise_fma(A2, p01 - K2, B2));
                    out[16 * k + 8 * h + 2 * i + 1] = bits_f16x2(__builtin_elementwise_fma(A2, p23 - K2, B2));
                }
        }
    }
};

// Q5_K (phi4.rs:512-542): Q4_K plus bit sb of qh[l] as bit 4.
template <int NP>
struct GqQ5K {
    static constexpr uint32_t BS = 176;
    struct Raw { u32x4 hdr, qh[NP], q[NP]; };
    __device__ static void load(Raw &r, __amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t blk, uint32_t c, uint32_t p0)
    {
        r.hdr = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, blk, 0);
#pragma unroll
        for (int k = 0; k < NP; k++) {
            r.qh[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + 16 + 16 * (p0 + k), blk, 0);
            r.q[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + 48 + 32 * c + 16 * (p0 + k), blk, 0);
        }
    }
    __device__ static void dequant(const Raw &r, uint32_t c, uint32_t, uint32_t *out)
    {
        const f16x2v K2 = {(_Float16)1024.0f, (_Float16)1024.0f};
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t sb = 2 * c + h;
            uint32_t sc, mn;
            scale_min_k4(sb, r.hdr.y, r.hdr.z, r.hdr.w, sc, mn);
            const _Float16 A = (_Float16)__fmul_rn(h2f(r.hdr.x), (float)sc);
            const _Float16 Bn = (_Float16)(-__fmul_rn(h2f(r.hdr.x >> 16), (float)mn));
            const f16x2v A2 = {A, A}, B2 = {Bn, Bn};
#pragma unroll
            for (int k = 0; k < NP; k++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t v = ((r.q[k][i] >> (4 * h)) & 0x0F0F0F0Fu) | (((r.qh[k][i] >> sb) & 0x01010101u) << 4);
                    f16x2v p01, p23;
                    q4_to_f16(v, p01, p23);
                    out[16 * k + 8 * h + 2 * i] = bits_f16x2(__builtin_elementwise_fma(A2, p01 - K2, B2));
                    out[16 * k + 8 * h + 2 * i + 1] = bits_f16x2(__builtin_elementwise_fma(A2, p23 - K2, B2));
                }
        }
    }
};

// Q6_K (phi4.rs:444-479): element 128h6 + 32Qd + l is ql[64h6 + 32(Qd&1) + l]
// (high nibble when Qd >= 2) with qh[32h6 + l] bits 2Qd; scale sc[e/16] (the
// is = g*8 + l/16 rule, phi4.rs:463); w = (d*sc)*(q - 32).  Chunk c is
// h6 = c/2 with Qd = 2(c&1) + j for run j, so l = 16p + (0..15) in both runs.
template <int NP>
struct GqQ6K {
    static constexpr uint32_t BS = 210;
    // d: the block's last dword (scales 14, 15 and the f16 d in its high
    // half), a 32-bit register with no 16-bit value to widen in the loop
    struct Raw { u32x4 ql[NP][2], qh[NP]; uint32_t sc, d; };
    __device__ static void load(Raw &r, __amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t blk, uint32_t c, uint32_t p0)
    {
        const uint32_t h6 = c >> 1;
#pragma unroll
        for (int k = 0; k < NP; k++) {
#pragma unroll
            for (int j = 0; j < 2; j++)
                r.ql[k][j] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + 64 * h6 + 32 * j + 16 * (p0 + k), blk, 0);
            r.qh[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + 128 + 32 * h6 + 16 * (p0 + k), blk, 0);
        }
        r.sc = __builtin_amdgcn_raw_buffer_load_b32(rs, voff + 192 + 4 * c, blk, 0);
        r.d = __builtin_amdgcn_raw_buffer_load_b32(rs, voff + 206, blk, 0);
    }
    __device__ static void dequant(const Raw &r, uint32_t c, uint32_t p0, uint32_t *out)
    {
        const uint32_t hi = c & 1;
        const float d = h2f(r.d >> 16);
        const f16x2v K2 = {(_Float16)1056.0f, (_Float16)1056.0f};
#pragma unroll
        for (int k = 0; k < NP; k++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const uint32_t qd = 2 * hi + j;
                // scale of elements 64c + 32j + 16p .. +15: sc[4c + 2j + p]
                const _Float16 A = (_Float16)__fmul_rn(d, (float)(int8_t)byte_of(r.sc, 2 * j + p0 + k));
                const f16x2v A2 = {A, A};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t v = ((r.ql[k][j][i] >> (4 * hi)) & 0x0F0F0F0Fu) |
                                       (((r.qh[k][i] >> (2 * qd)) & 0x03030303u) << 4);
                    f16x2v p01, p23;
                    q4_to_f16(v, p01, p23);
                    out[16 * k + 8 * j + 2 * i] = bits_f16x2(A2 * (p01 - K2));
                    out[16 * k + 8 * j + 2 * i + 1] = bits_f16x2(A2 * (p23 - K2));
                }
            }
    }
};

// Every dword of v counts as used here, so the registers a load fills stay
// reserved until this point.  Otherwise a dword the dequant never reads (a
// Q4_K header's last word when the chunk's scales sit in the first two) is
// dead from the load on, and the register allocator reuses its register for
// a temporary right after the load issues: a write that must first wait for
// that load to land.
template <class T>
__device__ __forceinline__ void keep_live(const T &v)
{
    constexpr int N = sizeof(T) / 4;
    struct A {
        uint32_t w[N];
    };
    const A a = __builtin_bit_cast(A, v);
#pragma unroll
    for (int i = 0; i < N; i++) asm volatile("" ::"v"(a.w[i]));
}

// Warp-specialised form: waves 0-3 run the MFMAs of a BM x BN tile (2 x 2,
// each (BM/2) x (BN/2)) and send X into LDS by DMA, waves 4-7 load and
// dequantize the next step's weights into the other LDS buffer, so every SIMD
// holds one wave of each kind and the staging VALU fills the matrix core's
// gaps.  Both roles pass one barrier per step (plus one after the prologue)
// on separate straight-line paths.
// silu_f(gate) * up of row block i (32 rows) of MFMA wave cw's 32 outputs of
// tile nt into Y (M x F), the D layout of the 32x32 MFMAs (lane l: column
// l % 32, rows 8 (r / 4) + 4 (l / 32) + r % 4 in register r)
template <int BM>
__device__ __forceinline__ void silu_rows_store(float *Y, uint32_t F, uint32_t nt, uint32_t m0, uint32_t cw,
                                                uint32_t lane, int i, const float *g, const float *u)
{
    const uint32_t wm = cw >> 1, wn = cw & 1, n = nt * 64 + wn * 32 + (lane & 31);
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const uint32_t m = m0 + wm * (BM / 2) + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        __builtin_nontemporal_store(silu_f(g[r]) * u[r], Y + (uint64_t)m * F + n);
    }
}

// SILU (gate/up with silu(gate) * up in the epilogue): W holds N = 2F rows,
// F gate rows then F up rows; tile nt takes outputs 64 nt .. 64 nt + 63, its
// B rows 0-31 / 32-63 / 64-95 / 96-127 being gate / up / gate / up rows of
// outputs 64 nt + 0-31, + 0-31, + 32-63, + 32-63, so an MFMA wave's two
// 32-column accumulators hold the gate and the up sums of the same outputs;
// Y (M x F) gets silu_f(gate) * up of the sums the plain GEMM stores.  The
// MFMA waves hand row blocks 2 and 3 of their sums to the staging waves
// through the (then idle) LDS, so the eight waves share the silu work.
template <template <int> class QT, int BM, int BN, int BK, bool ACC, bool SPLIT, bool SILU = false>
__global__ __launch_bounds__(512) void gemm_dq_kernel(const uint16_t *X, const uint8_t *W, float *Y, uint32_t K,
                                                      uint32_t N, uint32_t M, uint32_t tiles_n, const float *rscale,
                                                      uint32_t S, float *ws, uint32_t mrows)
{
    // LDS rows of BK f16, unpadded; 16-byte chunk c of row r sits at chunk
    // c ^ swz(r), swz(r) = g((r / RPL) % CPR) with RPL rows per 64-bank line,
    // CPR chunks per row and g swapping bits 1 and 2.  Any 16 consecutive
    // lanes then hit 64 distinct banks both when they read one chunk of 16
    // consecutive rows (g is a bijection) and when the staging waves write
    // chunks c and c ^ 2 of each of 16 / TPW consecutive rows (those rows'
    // g values fall in distinct classes {x, x ^ 2}, bit 3 aside); with g
    // the identity, those writes pair up two to a bank within 16 lanes.
    // swz depends on r % 16 only; every tile base and row stride below is a
    // multiple of 16.
    constexpr int LDK = BK, CPR = BK / 8, RPL = 128 / BK;
    static_assert(RPL * CPR == 16, "swizzle period");
    auto swz = [](uint32_t r) {
        const uint32_t x = (r / RPL) % CPR;
        return (x & ~6u) | ((x & 2u) << 1) | ((x & 4u) >> 1);
    };
    constexpr int UE = BN * BK / 256, TPW = BK / UE;       // weight elements per producer thread, threads per row
    constexpr int NPW = UE / 32;                           // 32-element parts per producer thread
    static_assert((UE == 32 || UE == 64) && BK % 64 == 0, "tile shape");
    using Q = QT<NPW>;
    // register sets of the producer's load ring (loads issued four steps
    // ahead, three sets in flight while one is staged)
    constexpr int NSET = 4;
    extern __shared__ float smem[];
    _Float16 *As = (_Float16 *)smem;                       // [GEMM_NA][BM][LDK]
    _Float16 *Bs = As + GEMM_NA * BM * LDK;                // [2][BN][LDK]

    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    // tile of this workgroup (same XCD for the M tiles of one N tile) and its
    // K split (the tile count is a multiple of 8 when K is split)
    const uint32_t tiles_m = M / BM, ntile = tiles_n * tiles_m;
    const uint32_t ks = SPLIT ? blockIdx.x / ntile : 0u, id = blockIdx.x - ks * ntile;
    uint32_t nt, mt;
    if (tiles_n % 8 == 0) {
        nt = (id / (8 * tiles_m)) * 8 + id % 8;
        mt = (id / 8) % tiles_m;
    } else {
        nt = id / tiles_m;
        mt = id % tiles_m;
    }
    const uint32_t m0 = mt * BM, n0 = nt * BN;
    // this split's K steps and its first step
    const uint32_t B = K / 256, bq = B / S, br = B % S;
    const uint32_t nsteps = SPLIT ? (bq + (ks < br ? 1u : 0u)) * (256 / BK) : K / BK;
    const uint32_t s0 = SPLIT ? (ks * bq + min(ks, br)) * (256 / BK) : 0u;

    if (wave >= 4) {
        // ---- producer: loads, dequant, conversion --------------------------
        const uint32_t tp = t - 256;
        // weight row, the step's 64-element chunk (its start lb) and the first
        // part wp of it (two parts a thread: the whole chunk, wp = 0)
        const uint32_t ur = tp / TPW, lb = 64 * ((tp % TPW) * NPW / 2), wp = (tp % TPW) * NPW % 2;
        const __amdgpu_buffer_rsrc_t wrs = make_rsrc(W, (uint64_t)N * B * Q::BS);
        const uint32_t wrow = SILU ? ((ur & 32u) ? N / 2 : 0u) + nt * (BN / 2) + (ur & 31u) + ((ur >> 6) << 5) : n0 + ur;
        const uint32_t wvoff = wrow * B * Q::BS;
        typename Q::Raw S0, S1, S2, S3;
        // element e0 of the step's unit inside its super-block: chunk e0/64, lane part e0%64
        auto issue = [&](typename Q::Raw &st, uint32_t s) {
            const bool ok = s < nsteps;   // past the end: out-of-range offsets, zeros
            const uint32_t sg = s0 + s, e0 = (sg * BK) % 256 + lb;
            Q::load(st, wrs, wvoff, ok ? (sg * BK / 256) * Q::BS : GM_OOB, e0 >> 6, wp);
            __builtin_amdgcn_sched_barrier(0);   // the sets' loads in program order
        };
        auto stage = [&](const typename Q::Raw &st, uint32_t s) {
            // the dequant stays after the previous barrier: hoisted above
            // it, it would wait for loads issued only a step earlier
            __builtin_amdgcn_sched_barrier(0);
            keep_live(st);
            const uint32_t buf = s & 1, e0 = ((s0 + s) * BK) % 256 + lb;
            uint32_t o[16 * NPW];
            Q::dequant(st, e0 >> 6, wp, o);
            // part k: runs at chunks c0 + 2k + (0, 1) and c0 + 2k + (4, 5)
            _Float16 *dst = Bs + (buf * BN + ur) * LDK;
            const uint32_t c0 = (lb + 16 * wp) / 8, gu = swz(ur);
#pragma unroll
            for (int i = 0; i < 4 * NPW; i++)
                *(u32x4 *)(dst + 8 * ((c0 + 2 * (i >> 2) + (i & 1) + 4 * ((i >> 1) & 1)) ^ gu)) =
                    u32x4{o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]};
        };
        // Each stage finds the loads of the other NSET - 1 sets issued after
        // its own, on the first pass as on every later one, so the compiler's
        // wait before it lets those stay in flight (a prologue that staged
        // step 0 and re-issued its set first would leave the loop-entry state
        // differently ordered, and the merged wait covers nearly every load).
        issue(S0, 0);
        issue(S1, 1);
        issue(S2, 2);
        issue(S3, 3);
        // stage s (its set then takes the loads of s+NSET) before barrier s;
        // steps past the end (nsteps rounded up to NSET) stage zeros
        for (uint32_t s = 0; s < nsteps; s += NSET) {
            stage(S0, s);
            issue(S0, s + NSET);
            __syncthreads();
            stage(S1, s + 1);
            issue(S1, s + 1 + NSET);
            __syncthreads();
            stage(S2, s + 2);
            issue(S2, s + 2 + NSET);
            __syncthreads();
            stage(S3, s + 3);
            issue(S3, s + 3 + NSET);
            __syncthreads();
        }
        // the barrier that ends the MFMA waves' last step
        __syncthreads();
        if constexpr (SILU) {
            // the MFMA waves' zeros past the end have landed; then row blocks
            // 2, 3 of MFMA wave t / 64 - 4, once it has handed them over
            __syncthreads();
            __syncthreads();
            const uint32_t cw = wave - 4;
            const float *hs = (const float *)smem + cw * 64 * 64 + lane;
#pragma unroll
            for (int i = 2; i < 4; i++) {
                float g[16], u[16];
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    g[r] = hs[((i - 2) * 32 + 2 * r) * 64];
                    u[r] = hs[((i - 2) * 32 + 2 * r + 1) * 64];
                }
                silu_rows_store<BM>(Y, N / 2, nt, m0, cw, lane, i, g, u);
            }
        }
        return;
    }

    // ---- consumer: MFMAs on LDS buffer s&1 ----------------------------------
    // 32x32x16 f16 MFMAs (the matrix core's best rate at one wave per SIMD);
    // lane l holds A row l % 32 and B column l % 32 at k = 8 (l / 32) + 0..7
    // of the 16-wide slice, and D column l % 32, rows 8 (r / 4) + 4 (l / 32)
    // + r % 4 in accumulator register r.
    constexpr int UI = BM / 64, UJ = BN / 64;   // 32x32 tiles per wave
    const uint32_t wm = wave >> 1, wn = wave & 1;
    f32x16 acc[UI][UJ];
#pragma unroll
    for (int i = 0; i < UI; i++)
#pragma unroll
        for (int j = 0; j < UJ; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;
    const uint32_t fr = lane & 31, fk = 8 * (lane >> 5);
    // The fragments of one 16-wide k slice; two sets alternate so that the
    // LDS reads of slice kq + 1 are in flight while the MFMAs of slice kq
    // run.  The scheduling fences keep that order: left to itself the
    // compiler reloads one fragment register per row of tiles and waits out
    // the LDS latency before each row's MFMAs.
    struct Frag {
        f16x8v a[UI], b[UJ];
    };
    auto frag_load = [&](Frag &f, uint32_t abuf, uint32_t bbuf, int kq) {
        const uint32_t ch = 8 * (((fk / 8) + 2 * kq) ^ swz(fr));
        const _Float16 *Ab = As + (abuf * BM + wm * (BM / 2) + fr) * LDK + ch;
        const _Float16 *Bb = Bs + (bbuf * BN + wn * (BN / 2) + fr) * LDK + ch;
#pragma unroll
        for (int i = 0; i < UI; i++) f.a[i] = *(const f16x8v *)(Ab + 32 * i * LDK);
#pragma unroll
        for (int j = 0; j < UJ; j++) f.b[j] = *(const f16x8v *)(Bb + 32 * j * LDK);
    };
    auto frag_mfma = [&](const Frag &f) {
#pragma unroll
        for (int i = 0; i < UI; i++)
#pragma unroll
            for (int j = 0; j < UJ; j++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
    };
    constexpr int KQ = BK / 16;   // even
    // X goes from global memory straight into LDS, issued by these waves
    // (whose vector memory path is otherwise idle) NA - 1 steps ahead into a
    // ring of NA A buffers: 16-byte LDS DMA, lane l of a load writing
    // base + 16 l, so load i of wave w covers tile rows XRP (XI w + i) ..
    // + XRP - 1, lane l row l / CPR and the chunk whose swizzled place is
    // l % CPR.  Steps past nsteps load zeros (out-of-range offsets).
    constexpr int NA = GEMM_NA, XRP = 512 / BK, XI = BM / (4 * XRP), XPQ = XI / (KQ / 2);
    static_assert(XI * 4 * XRP == BM && XPQ * (KQ / 2) == XI && (NA - 2) * XI < 32 && NA >= 3 && NA <= 4,
                  "X loads per wave and step");
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(X, (uint64_t)M * K * 2);
    const uint32_t wu = __builtin_amdgcn_readfirstlane(wave);   // wave-uniform: LDS bases in scalar registers
    auto x_dma = [&](uint32_t s, uint32_t abuf, int i) {
        const uint32_t rb = XRP * (XI * wu + i), r = rb + lane / CPR;
        const uint32_t voff = ((m0 + r) * K + 8 * ((lane % CPR) ^ swz(r))) * 2;
        lds_dma16<0>(xrs, As + (abuf * BM + rb) * LDK, voff, s < nsteps ? (s0 + s) * BK * 2 : GM_OOB);
    };
    // one barrier per step, as many steps as the producer stages (nsteps
    // rounded up to NSET, at least NA - 1); the barrier of step s comes once this
    // wave's reads of step s have landed and its X loads of step s + 1 have
    // (those of the later steps stay in flight), and the first slice of step
    // s + 1 is read while the last slice of step s multiplies
    static_assert(NSET >= NA - 1, "the prologue's X steps exist");
    const uint32_t steps3 = (nsteps + NSET - 1) / NSET * NSET;
#pragma unroll
    for (int p = 0; p < NA - 1; p++)
#pragma unroll
        for (int i = 0; i < XI; i++) x_dma(p, p, i);
    wait_vm<(NA - 2) * XI>();
    Frag f0, f1;
    barrier_lds();
    frag_load(f0, 0, 0, 0);
    uint32_t ca = 0;   // A buffer of step s (s % NA)
    for (uint32_t s = 0; s < steps3; s++) {
        const uint32_t cb = s & 1, na = ca == NA - 1 ? 0u : ca + 1, pa = ca == 0 ? NA - 1 : ca - 1;
#pragma unroll
        for (int kq = 0; kq < KQ; kq += 2) {
            frag_load(f1, ca, cb, kq + 1);
            __builtin_amdgcn_sched_barrier(0);
            frag_mfma(f0);
            __builtin_amdgcn_sched_barrier(0);
            // X of step s + NA - 1 into the buffer step s - 1 used, issued on
            // every step (one straight-line loop body with no branch): in the
            // last NA - 1 steps it is a step past nsteps, whose zeros land in
            // a buffer no later step reads
#pragma unroll
            for (int i = 0; i < XPQ; i++) x_dma(s + NA - 1, pa, XPQ * (kq / 2) + i);
            if (kq + 2 < KQ) {
                frag_load(f0, ca, cb, kq + 2);
            } else {
                // X of steps s + 2 .. s + NA - 1 stay in flight
                wait_vm<(NA - 2) * XI>();
                barrier_lds();
                frag_load(f0, na, cb ^ 1u, 0);   // past the last step: stale, unused
            }
            __builtin_amdgcn_sched_barrier(0);
            frag_mfma(f1);
            __builtin_amdgcn_sched_barrier(0);
        }
        ca = na;
    }
    // the zeros of the steps past the end have landed before the epilogue
    // reuses the LDS (SILU: every wave's, a barrier later)
    wait_vm<0>();

    if constexpr (SILU) {
        static_assert(!SPLIT && !ACC && BN == 128 && BM == 256, "gate/up tiles of 64 outputs, whole K");
        // row blocks 2, 3 to the staging wave t / 64 + 4 (LDS past the last
        // step's barrier and the zeros' landing: only this wave's stale
        // fragment read touches it)
        __syncthreads();
        float *hs = (float *)smem + wave * 64 * 64 + lane;
#pragma unroll
        for (int i = 2; i < 4; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                hs[((i - 2) * 32 + 2 * r) * 64] = acc[i][0][r];
                hs[((i - 2) * 32 + 2 * r + 1) * 64] = acc[i][1][r];
            }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 2; i++) {
            float g[16], u[16];
#pragma unroll
            for (int r = 0; r < 16; r++) {
                g[r] = acc[i][0][r];
                u[r] = acc[i][1][r];
            }
            silu_rows_store<BM>(Y, N / 2, nt, m0, wave, lane, i, g, u);
        }
        return;
    }
    if constexpr (SPLIT) {
#pragma unroll
        for (int i = 0; i < UI; i++)
#pragma unroll
            for (int j = 0; j < UJ; j++) {
                const uint32_t n = n0 + wn * (BN / 2) + 32 * j + fr;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const uint32_t m = m0 + wm * (BM / 2) + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    __builtin_nontemporal_store(acc[i][j][r], ws + ((uint64_t)ks * M + m) * N + n);
                }
            }
        return;
    }
    // Outputs (here, the split partials above and the silu * up rows) leave
    // as non-temporal stores: every CU writes its whole tile at the end at
    // once, and the stream gets through faster without allocating in the
    // caches on its way (gate+up at 512 rows: 33.5 MB of f32).
    // The row scales (powers of two) are exact.  Per row tile, its rows'
    // scales and (ACC) the Y values it adds to are requested at once, rows
    // past mrows (zero padding of a row chunk, not the caller's: never
    // stored) reading row mrows - 1: loaded under the row test, each would
    // wait for the one before.
    // (no row scale: a resource of no bytes, whose loads return zeros
    // without a memory request, and the product is not taken)
    const __amdgpu_buffer_rsrc_t rsr = make_rsrc(rscale, rscale ? (uint64_t)mrows * 4 : 0u);
#pragma unroll
    for (int i = 0; i < UI; i++) {
        float sc[16], yo[UJ][16];
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const uint32_t m = m0 + wm * (BM / 2) + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            const uint32_t mc = min(m, mrows - 1);
            sc[r] = __uint_as_float(bload4(rsr, 4 * mc));
            if constexpr (ACC) {
#pragma unroll
                for (int j = 0; j < UJ; j++) yo[j][r] = Y[(uint64_t)mc * N + n0 + wn * (BN / 2) + 32 * j + fr];
            }
        }
#pragma unroll
        for (int j = 0; j < UJ; j++) {
            const uint32_t n = n0 + wn * (BN / 2) + 32 * j + fr;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const uint32_t m = m0 + wm * (BM / 2) + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m >= mrows) continue;
                const float v = rscale ? acc[i][j][r] * sc[r] : acc[i][j][r];
                if constexpr (ACC)
                    Y[(uint64_t)m * N + n] = yo[j][r] + v;
                else
                    __builtin_nontemporal_store(v, Y + (uint64_t)m * N + n);
            }
        }
    }
}

// Y (+)= rscale[m] * sum over the SS partials of ws (in split order, all
// requested before the first add), four outputs per thread (N % 4 == 0), for
// the first mrows of the M partial rows
template <bool ACC, int SS>
__global__ __launch_bounds__(256) void gemm_splitk_reduce(const float *__restrict__ ws, uint32_t M, uint32_t N,
                                                          float *__restrict__ Y, const float *__restrict__ rscale,
                                                          uint32_t mrows)
{
    const uint64_t q = (uint64_t)blockIdx.x * 256 + threadIdx.x, mn = (uint64_t)M * N;
    if (4 * q >= (uint64_t)mrows * N) return;
    float4 p[SS];
#pragma unroll
    for (int k = 0; k < SS; k++) p[k] = ((const float4 *)(ws + k * mn))[q];
    float4 v = p[0];
#pragma unroll
    for (int k = 1; k < SS; k++) {
        v.x += p[k].x; v.y += p[k].y; v.z += p[k].z; v.w += p[k].w;
    }
    if (rscale) {
        const float r = rscale[(4 * q) / N];
        v.x *= r; v.y *= r; v.z *= r; v.w *= r;
    }
    float4 *y = (float4 *)Y + q;
    if constexpr (ACC) {
        const float4 o = *y;
        v.x = o.x + v.x; v.y = o.y + v.y; v.z = o.z + v.z; v.w = o.w + v.w;
    }
    *y = v;
}

template <template <int> class QT, int BM, int BN, int BK, bool ACC>
static hipError_t go_gemm(const uint16_t *X, const float *rscale, const uint8_t *W, float *Y, uint32_t K, uint32_t N,
                          uint32_t M, uint32_t mrows, uint32_t S, float *ws, const GemmNorm *nrm, const GemmRope *rp,
                          hipStream_t s)
{
    constexpr size_t lds = gemm_lds_bytes<BM, BN, BK>;
    static_assert(lds <= 160 * 1024, "LDS per workgroup");
    // the fused reductions take every one of the M rows
    if ((nrm || rp) && mrows != M) return hipErrorInvalidValue;
    const uint32_t tiles_n = N / BN, tiles = tiles_n * (M / BM);
    if (S > 1)
        hipLaunchKernelGGL((gemm_dq_kernel<QT, BM, BN, BK, ACC, true>), dim3(tiles * S), dim3(512), lds, s, X, W, Y, K,
                           N, M, tiles_n, rscale, S, ws, mrows);
    else
        hipLaunchKernelGGL((gemm_dq_kernel<QT, BM, BN, BK, ACC, false>), dim3(tiles), dim3(512), lds, s, X, W, Y, K,
                           N, M, tiles_n, rscale, 1u, nullptr, mrows);
    if (S > 1 && rp) {
        // the reduction is the rope_kv_store's first step
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        return launch_splitk_rope_kv_store(ws, S, M, Y, rp->r, rp->rows, rp->kc, rp->vc, s);
    }
    if (rp) {
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        return launch_rope_kv_store(Y, rp->r, rp->kc, rp->vc, s, rp->rows);
    }
    if (S > 1 && nrm) {
        // the reduction also writes the rows' RMSNorm
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        return launch_splitk_reduce_rmsnorm(ws, S, M, N, Y, rscale, ACC, nrm->gamma, nrm->eps, nrm->out, s);
    }
    if (S > 1) {
        const uint64_t quads = (uint64_t)mrows * N / 4;
        const dim3 grid((unsigned)((quads + 255) / 256));
#define RRR_SKR_CASE(K)                                                                                         \
    case K:                                                                                                     \
        hipLaunchKernelGGL((gemm_splitk_reduce<ACC, K>), grid, dim3(256), 0, s, ws, M, N, Y, rscale, mrows); \
        break;
        switch (S) {
            RRR_SKR_CASE(2) RRR_SKR_CASE(3) RRR_SKR_CASE(4) RRR_SKR_CASE(5)
            RRR_SKR_CASE(6) RRR_SKR_CASE(7) RRR_SKR_CASE(8)
        default: return hipErrorInvalidValue;
        }
#undef RRR_SKR_CASE
    }
    if (nrm) {
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        return launch_rmsnorm_f16(Y, nrm->gamma, nrm->out, M, N, nrm->eps, s);
    }
    return hipGetLastError();
}

// Splits of K for a grid of `tiles` tiles: at most as many as keep every
// workgroup in the first round over the MI355X's 256 CUs (a second round
// costs a whole tile's time) and at most 8, each a whole number of
// super-blocks (the first B % S splits one more), their partials within the
// workspace; of those, the fewest that give the shortest longest split
// (K = 8192, 48 tiles: 5 splits of 7/7/6/6/6 super-blocks rather than 4 of
// 8; K = 3072: 4 splits of 3 rather than 5 of 3/3/2/2/2); 1 when the tiles
// already fill half of the CUs.
static uint32_t gemm_splits(uint32_t tiles, uint32_t K, uint32_t M, uint32_t N, size_t ws_bytes)
{
    const uint32_t cus = 256, B = K / 256;
    if (tiles >= cus / 2 || tiles % 8) return 1;
    uint32_t best = 1;
    for (uint32_t S = 2; S <= min(min(8u, cus / tiles), B); S++) {
        if ((uint64_t)S * M * N * 4 > ws_bytes) break;
        if ((B + S - 1) / S < (B + best - 1) / best) best = S;
    }
    return best;
}

template <template <int> class QT, bool ACC>
static hipError_t go_gemm_t(const uint16_t *X, const float *rscale, const uint8_t *W, float *Y, uint32_t K,
                            uint32_t N, uint32_t M, uint32_t mrows, float *ws, size_t ws_bytes, const GemmNorm *nrm,
                            const GemmRope *rp, hipStream_t s)
{
    // 256 x 128 tiles when they cover at least half of the CUs, or with K
    // split to do so; else 128 x 64 (with K steps of 128 so each barrier
    // covers as much MFMA work), K split the same way when those tiles are few
    if (M % 256 == 0 && N % 128 == 0) {
        const uint32_t tiles = (N / 128) * (M / 256);
        const uint32_t S = ws ? gemm_splits(tiles, K, M, N, ws_bytes) : 1u;
        if (tiles * S >= 128)
            return go_gemm<QT, 256, 128, 64, ACC>(X, rscale, W, Y, K, N, M, mrows, S, ws, nrm, rp, s);
    }
    const uint32_t S = ws ? gemm_splits((N / 64) * (M / 128), K, M, N, ws_bytes) : 1u;
    return go_gemm<QT, 128, 64, 128, ACC>(X, rscale, W, Y, K, N, M, mrows, S, ws, nrm, rp, s);
}

bool gemm_supported(uint32_t type, uint32_t K, uint32_t N, uint32_t M, uint64_t x_bytes)
{
    return (type == T_Q4_K || type == T_Q5_K || type == T_Q6_K) && K % 256 == 0 && N % 64 == 0 && M % 128 == 0 &&
           (uint64_t)N * (K / 256) * 210 + RRR_READ_SLACK < GM_OOB && x_bytes + RRR_READ_SLACK < GM_OOB;
}

template <bool ACC>
static hipError_t go_gemm_q(const uint16_t *X, const float *rscale, const uint8_t *W, uint32_t type, float *Y,
                            uint32_t K, uint32_t N, uint32_t M, uint32_t mrows, float *ws, size_t ws_bytes,
                            hipStream_t s, const GemmNorm *nrm = nullptr, const GemmRope *rp = nullptr)
{
    if (!gemm_supported(type, K, N, M, (uint64_t)M * K * 2) || mrows == 0 || mrows > M) return hipErrorNotSupported;
    switch (type) {
    case T_Q4_K: return go_gemm_t<GqQ4K, ACC>(X, rscale, W, Y, K, N, M, mrows, ws, ws_bytes, nrm, rp, s);
    case T_Q5_K: return go_gemm_t<GqQ5K, ACC>(X, rscale, W, Y, K, N, M, mrows, ws, ws_bytes, nrm, rp, s);
    case T_Q6_K: return go_gemm_t<GqQ6K, ACC>(X, rscale, W, Y, K, N, M, mrows, ws, ws_bytes, nrm, rp, s);
    default: return hipErrorNotSupported;
    }
}

// The activations of rrr_gemm_bf16 and of the batched GEMV above 16 rows,
// converted to f16 rows once per call (so the N / BN column tiles read them
// as they are), into the context workspace, a chunk of rows at a time; a
// chunk is padded with zero rows to a multiple of 128 (which the GEMM computes
// and does not store).
//
// bf16 -> f16, 8 elements a thread: exact for |x| in f16's normal range.
__global__ __launch_bounds__(256) void bf16_rows_to_f16_kernel(const uint16_t *__restrict__ X, uint32_t K,
                                                               uint32_t rows, u32x4 *__restrict__ Xh, uint64_t n8)
{
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n8) return;
    const uint64_t e = 8 * i;   // K % 256 == 0: a thread's 8 elements sit in one row
    u32x4 h = {0u, 0u, 0u, 0u};
    if (e / K < rows) {
        const u32x4 v = *(const u32x4 *)(X + e);
#pragma unroll
        for (int c = 0; c < 4; c++) h[c] = pk_f16(__uint_as_float(v[c] << 16), __uint_as_float(v[c] & 0xFFFF0000u));
    }
    Xh[i] = h;
}

// f32 rows -> f16 block floating point, one workgroup per row: row m is
// scaled by 2^(15 - e) (max|x_m| = f * 2^e, f in [0.5, 1); exact in f32), so
// its largest value lands in [2^14, 2^15), rounded to nearest even, and
// rscale[m] = 2^(e - 15) undoes the scale on the GEMM's output (exact).
// A zero row keeps scale 1; a row holding inf or NaN is converted unscaled,
// so the non-finite values reach the products.  Rows past `rows` are zeros.
__global__ __launch_bounds__(256) void f32_rows_to_f16_kernel(const float *__restrict__ X, uint32_t K, uint32_t rows,
                                                              uint16_t *__restrict__ Xh, float *__restrict__ rscale)
{
    __shared__ float wmax[4];
    const uint32_t m = blockIdx.x, t = threadIdx.x;
    uint16_t *out = Xh + (uint64_t)m * K;
    if (m >= rows) {
        for (uint32_t k = 8 * t; k < K; k += 8 * 256) *(u32x4 *)(out + k) = u32x4{0u, 0u, 0u, 0u};
        if (t == 0) rscale[m] = 1.0f;
        return;
    }
    const float *row = X + (uint64_t)m * K;
    float mx = 0.0f;
    for (uint32_t k = 4 * t; k < K; k += 4 * 256) {
        const float4 v = *(const float4 *)(row + k);
        // fmaxf drops NaN: a NaN anywhere is kept by the isnan test below
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        if (__builtin_isnan(v.x + v.y + v.z + v.w)) mx = __builtin_inff();
    }
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if ((t & 63) == 0) wmax[t >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    int e = 15;
    if (mx > 0.0f && __builtin_isfinite(mx)) (void)frexpf(mx, &e);
    e = max(e, -110);   // 2^(15 - e) stays a normal f32
    const float sc = ldexpf(1.0f, 15 - e);
    if (t == 0) rscale[m] = ldexpf(1.0f, e - 15);
    for (uint32_t k = 8 * t; k < K; k += 8 * 256) {
        const float4 a = *(const float4 *)(row + k), b = *(const float4 *)(row + k + 4);
        *(u32x4 *)(out + k) = u32x4{pk_f16_rn(a.x * sc, a.y * sc), pk_f16_rn(a.z * sc, a.w * sc),
                                    pk_f16_rn(b.x * sc, b.y * sc), pk_f16_rn(b.z * sc, b.w * sc)};
    }
}

// Rows per chunk: all M rows (rounded up to 128) when their f16 copy and
// row scales take at most half of the workspace (the other half holds split
// partials), else the most multiples of 256 that do; 0 when not even 128 do.
static uint32_t gemm_chunk_rows(uint32_t M, uint32_t K, size_t ws_bytes)
{
    const uint64_t per_row = 2ull * K + 4, cap = (uint64_t)(ws_bytes / 2) / per_row;
    const uint64_t mp = (M + 127ull) / 128 * 128;
    if (mp <= cap) return (uint32_t)mp;
    if (cap >= 256) return (uint32_t)(cap / 256 * 256);
    return cap >= 128 ? 128u : 0u;
}

// X (bf16 or f32, M x K) . W^T in row chunks through the f16 GEMM.
static hipError_t gemm_rows(const void *X, bool f32, const uint8_t *W, uint32_t type, float *Y, uint32_t K,
                            uint32_t N, uint32_t M, void *ws, size_t ws_bytes, hipStream_t s)
{
    const uint32_t mc = ws ? gemm_chunk_rows(M, K, ws_bytes) : 0u;
    if (!mc || !gemm_supported(type, K, N, mc, (uint64_t)mc * K * 2)) return hipErrorNotSupported;
    // workspace: f16 rows | row scales | split partials (256-byte aligned)
    const uint64_t xh_bytes = ((uint64_t)mc * K * 2 + 255) & ~255ull, rs_bytes = ((uint64_t)mc * 4 + 255) & ~255ull;
    uint16_t *Xh = (uint16_t *)ws;
    float *rscale = (float *)((uint8_t *)ws + xh_bytes);
    float *part = (float *)((uint8_t *)ws + xh_bytes + rs_bytes);
    const size_t part_bytes = ws_bytes - xh_bytes - rs_bytes;
    for (uint32_t m0 = 0; m0 < M; m0 += mc) {
        const uint32_t rows = min(mc, M - m0), mp = (rows + 127) / 128 * 128;
        if (f32) {
            hipLaunchKernelGGL(f32_rows_to_f16_kernel, dim3(mp), dim3(256), 0, s, (const float *)X + (uint64_t)m0 * K,
                               K, rows, Xh, rscale);
        } else {
            const uint64_t n8 = (uint64_t)mp * K / 8;
            hipLaunchKernelGGL(bf16_rows_to_f16_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, s,
                               (const uint16_t *)X + (uint64_t)m0 * K, K, rows, (u32x4 *)Xh, n8);
        }
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        e = go_gemm_q<false>(Xh, f32 ? rscale : nullptr, W, type, Y + (uint64_t)m0 * N, K, N, mp, rows, part,
                             part_bytes, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_gemm_bf16(const uint16_t *X, const uint8_t *W, uint32_t type, float *Y, uint32_t K, uint32_t N,
                            uint32_t M, float *ws, size_t ws_bytes, hipStream_t s)
{
    return gemm_rows(X, false, W, type, Y, K, N, M, ws, ws_bytes, s);
}

bool gemm_rows_supported(uint32_t type, uint32_t K, uint32_t N, uint32_t M, size_t ws_bytes)
{
    const uint32_t mc = gemm_chunk_rows(M, K, ws_bytes);
    return M > 0 && mc && gemm_supported(type, K, N, mc, (uint64_t)mc * K * 2);
}

hipError_t launch_gemm_f32_rows(const float *X, const uint8_t *W, uint32_t type, float *Y, uint32_t K, uint32_t N,
                                uint32_t M, void *ws, size_t ws_bytes, hipStream_t s)
{
    return gemm_rows(X, true, W, type, Y, K, N, M, ws, ws_bytes, s);
}

hipError_t launch_gemm_f16(const uint16_t *X, const float *rscale, const uint8_t *W, uint32_t type, float *Y,
                           uint32_t K, uint32_t N, uint32_t M, bool accumulate, float *ws, size_t ws_bytes,
                           hipStream_t s)
{
    return accumulate ? go_gemm_q<true>(X, rscale, W, type, Y, K, N, M, M, ws, ws_bytes, s)
                      : go_gemm_q<false>(X, rscale, W, type, Y, K, N, M, M, ws, ws_bytes, s);
}

hipError_t launch_gemm_f16_rmsnorm(const uint16_t *X, const float *rscale, const uint8_t *W, uint32_t type, float *Y,
                                   uint32_t K, uint32_t N, uint32_t M, bool accumulate, const float *gamma, float eps,
                                   uint16_t *out16, float *ws, size_t ws_bytes, hipStream_t s)
{
    if (!splitk_reduce_rmsnorm_supported(N)) return hipErrorNotSupported;
    const GemmNorm nrm{gamma, eps, out16};
    return accumulate ? go_gemm_q<true>(X, rscale, W, type, Y, K, N, M, M, ws, ws_bytes, s, &nrm)
                      : go_gemm_q<false>(X, rscale, W, type, Y, K, N, M, M, ws, ws_bytes, s, &nrm);
}

// The gate/up GEMM with silu(gate) * up in its epilogue into ws (M x F
// f32), then the f16 block-floating-point rows of silu_gate_f16 from it:
// whole K on 256 x 128 tiles that cover half of the CUs, else not supported.
hipError_t launch_gemm_f16_silu_f16(const uint16_t *X, const uint8_t *W, uint32_t type, uint16_t *mid, float *rscale,
                                    uint32_t K, uint32_t F, uint32_t M, float *ws, size_t ws_bytes, hipStream_t s)
{
    const uint32_t N = 2 * F;
    if (!gemm_supported(type, K, N, M, (uint64_t)M * K * 2) || M % 256 || N % 128) return hipErrorNotSupported;
    const uint32_t tiles_n = N / 128, tiles = tiles_n * (M / 256);
    if (tiles < 128 || (uint64_t)M * F * 4 > ws_bytes) return hipErrorNotSupported;
    constexpr size_t lds = gemm_lds_bytes<256, 128, 64>;
#define RRR_SILU_CASE(T, QT)                                                                                          \
    case T:                                                                                                            \
        hipLaunchKernelGGL((gemm_dq_kernel<QT, 256, 128, 64, false, false, true>), dim3(tiles), dim3(512), lds, s, X, \
                           W, ws, K, N, M, tiles_n, nullptr, 1u, nullptr, M);                                          \
        break;
    switch (type) {
        RRR_SILU_CASE(T_Q4_K, GqQ4K)
        RRR_SILU_CASE(T_Q5_K, GqQ5K)
        RRR_SILU_CASE(T_Q6_K, GqQ6K)
    default: return hipErrorNotSupported;
    }
#undef RRR_SILU_CASE
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_f16_rows_scaled(ws, mid, rscale, M, F, s);
}

hipError_t launch_gemm_f16_rope_kv(const uint16_t *X, const uint8_t *W, uint32_t type, float *Y, uint32_t K,
                                   uint32_t N, uint32_t M, const RopeArgs &r, uint32_t rows, uint16_t *kc,
                                   uint16_t *vc, float *ws, size_t ws_bytes, hipStream_t s)
{
    if (!splitk_rope_kv_store_supported(r) || r.row_stride != N || rows > M) return hipErrorNotSupported;
    const GemmRope rp{r, rows, kc, vc};
    return go_gemm_q<false>(X, nullptr, W, type, Y, K, N, M, M, ws, ws_bytes, s, nullptr, &rp);
}

}  // namespace rrr
