// sweep.hip -- the decode weight sweep as one persistent launch: the list of
// fused GEMV ops that the reference replays per token through
// dispatch_batch_persistent_v2 (engine.rs:317-370, table built at
// phi4.rs:972-1064) runs inside one kernel of one workgroup per CU.
//
// Roles inside a workgroup (13 waves):
//   compute waves 0..11  each owns a K slice of every op (one super-block of
//                        K = 3072, two or three of K = 8192) and streams its
//                        slice of the workgroup's tiles of the NEXT op into a
//                        private 9 KB LDS ring by LDS DMA while the current op
//                        waits for its inputs and runs; at the start of an op
//                        it moves its slice from the ring into registers,
//                        which frees the ring for the next op's weights.
//   sync wave 12         waits until every workgroup has finished the
//                        previous op, releases the op to the compute waves,
//                        adds their row partials (and the residual), stores
//                        the rows and publishes the workgroup's completion.
// A compute wave issues only weight DMAs and its activation loads, in that
// order, so waiting for its activations (in-order vmcnt) also waits for the
// op's own weights and never for the next op's; the sync wave issues no DMA,
// so its polls and stores are not queued behind weight traffic.
//
// Completion records: after op i, workgroup b stores one 8-byte record
// {epoch, sum of squares of the rows it wrote} through to the coherent level
// (after its rows).  Op i starts when every record has reached op i-1's
// epoch; an RMSNorm op takes the sum of squares of its input (the previous
// op's output) as the sum of the records' partials in workgroup order, so
// the norm needs no pass of its own.  Epochs come from a per-workgroup run
// counter in device memory (so the launch can be recorded in a graph and
// replayed) and are compared modulo 2^32.
//
// Waits are bounded (~2 s of the 100 MHz real-time clock): on expiry the
// error word is set, the workgroup abandons the run and rrr_sweep_check
// reports it.
#include "gemv_mq.h"

namespace rrr {

constexpr uint32_t SW_CW = 12;                                  // compute waves
constexpr uint32_t SW_THREADS = 64 * (SW_CW + 1);               // + the sync wave
constexpr uint32_t SW_REGION = 12 * 1024;                       // LDS of a compute wave: ring, then staging
constexpr uint32_t SW_DMA_MAX = 10;                             // 1 KB ring slots (one DMA load each)
constexpr uint32_t SW_DMA_EARLY = 2;                            // next-op loads a wave issues before its MFMAs
constexpr uint32_t SW_NB_MAX = 3;                               // super-blocks per compute wave
constexpr uint32_t SW_NT_MAX = 4;                               // tiles per workgroup in one op
constexpr uint32_t SW_PART_OFF = SW_CW * SW_REGION;
constexpr uint32_t SW_CTL_OFF = SW_PART_OFF + SW_NT_MAX * SW_CW * 16 * 4;
constexpr uint32_t SW_LDS_BYTES = SW_CTL_OFF + 64;
constexpr uint32_t SW_G_MAX = 256;                              // records: 4 per lane of one wave
constexpr uint32_t SW_ABORT = 0xFFFFFFFFu;
constexpr uint64_t SW_SPIN_TICKS = 200000000ull;                // ~2 s at 100 MHz
constexpr uint32_t SW_OOB = 0x80000000u;                        // offset past every weight byte
static_assert(SW_LDS_BYTES <= 160 * 1024, "LDS");
static_assert(SW_DMA_MAX * 1024 <= SW_REGION, "ring");

// device memory of a sweep: records (2 words each), run counters, error word
constexpr uint32_t SW_REC_WORDS = 2 * SW_G_MAX, SW_RUNC_OFF = SW_REC_WORDS, SW_ERR_OFF = SW_RUNC_OFF + SW_G_MAX;
constexpr uint32_t SW_STATE_WORDS = SW_ERR_OFF + 4;

// The decode layer's op forms (weight type, activation, super-blocks per
// compute wave, most tiles per workgroup).
enum SwForm : uint32_t { SWF_Q5K_RMS = 0, SWF_Q4K_RMS = 1, SWF_Q4K_GQA = 2, SWF_Q4K_SILU = 3, SWF_Q6K_SILU = 4,
                         SWF_NONE = 7 /* no next op */ };

template <uint32_t F> struct SwF;
template <> struct SwF<SWF_Q5K_RMS> { using Q = MqQ5K; static constexpr int ACT = ACT_RMSNORM, NB = 1, NT = 2; };
template <> struct SwF<SWF_Q4K_RMS> { using Q = MqQ4K; static constexpr int ACT = ACT_RMSNORM, NB = 1, NT = 4; };
template <> struct SwF<SWF_Q4K_GQA> { using Q = MqQ4K; static constexpr int ACT = ACT_GQA_V, NB = 1, NT = 2; };
template <> struct SwF<SWF_Q4K_SILU> { using Q = MqQ4K; static constexpr int ACT = ACT_SILU, NB = 3, NT = 1; };
template <> struct SwF<SWF_Q6K_SILU> { using Q = MqQ6K; static constexpr int ACT = ACT_SILU, NB = 3, NT = 1; };

// Ring layout.  A piece is one row's super-block: UPB 16-byte units (a Q6_K
// block is loaded as the 224-byte window from the 16-byte boundary at or
// below its start).  A DMA load (64 lanes x 16 bytes, one 1 KB ring slot)
// carries one block of PPI consecutive rows of the workgroup (lane l: row
// l / UPB, unit l % UPB), so a lane's byte offset is the same for every load
// and the load's own part (rows, block) is a scalar offset.  Slot i holds
// row group i / NB, block i % NB.
template <class Q> struct SwPiece;
template <> struct SwPiece<MqQ4K> { static constexpr uint32_t UPB = 9, PPI = 7; };
template <> struct SwPiece<MqQ5K> { static constexpr uint32_t UPB = 11, PPI = 5; };
template <> struct SwPiece<MqQ6K> { static constexpr uint32_t UPB = 14, PPI = 4; };

struct __attribute__((aligned(16))) SwOpDev {
    const uint8_t *W;
    const float *x;
    const float *gamma;
    float *y;
    uint32_t w_bytes, row_bytes;
    uint32_t K, N;
    uint32_t tr, ntiles, per;   // rows per tile, tiles, tiles per workgroup (workgroup b: tiles b*per ..)
    uint32_t form, residual;
    uint32_t gqa;               // head_dim | heads_per_kv << 16
    float eps;
    uint32_t stage;             // staging bytes of this op (at the end of each compute wave's region)
};

__device__ __forceinline__ uint32_t sw_lds_load(const uint32_t *p)
{
    return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void sw_lds_store(uint32_t *p, uint32_t v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// 16-byte LDS DMA: lane l's 16 bytes at voff + soff go to LDS dst + 16 l.
// Only the device pass sees the builtin.
__device__ __forceinline__ void sw_dma16(__amdgpu_buffer_rsrc_t rs, uint8_t *dst, uint32_t voff, uint32_t soff)
{
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)dst, 16, voff, soff, 0,
                                             RRR_CPOL_NT);
#endif
}

__device__ __forceinline__ void sw_wait_vm0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// The super-blocks [j0, j0 + nb) of a compute wave in an op of B blocks.
template <int NB>
__device__ __forceinline__ void sw_slice(uint32_t w, uint32_t B, uint32_t &j0, uint32_t &nb)
{
    if constexpr (NB == 1) {
        j0 = w;
        nb = w < B ? 1u : 0u;
    } else {
        const uint32_t base = B / SW_CW, extra = B % SW_CW;
        j0 = w * base + min(w, extra);
        nb = base + (w < extra ? 1u : 0u);
    }
}

// Workgroup b's tiles b*per .. (ntl of them) and its rows [r0, r0 + nrows).
struct SwRows {
    uint32_t ntl, r0, nrows;
};
__device__ __forceinline__ SwRows sw_rows(const SwOpDev &o, uint32_t b)
{
    const uint32_t t0 = b * o.per;
    const uint32_t ntl = o.ntiles > t0 ? min(o.per, o.ntiles - t0) : 0u;
    const uint32_t r0 = t0 * o.tr;
    return {ntl, r0, ntl ? min(ntl * o.tr, o.N - r0) : 0u};
}

// Ring slots an op fills: row groups of PPI rows, NB blocks each.
template <uint32_t F>
__device__ __forceinline__ uint32_t sw_slots(uint32_t nrows)
{
    using P = SwPiece<typename SwF<F>::Q>;
    return (nrows + P::PPI - 1) / P::PPI * SwF<F>::NB;
}

// LDS DMA of this wave's slice of the workgroup's rows of op o into its ring
// slots [lo, hi).
template <uint32_t F>
__device__ __forceinline__ void sw_dma(const SwOpDev &o, uint32_t w, uint32_t b, uint32_t lane, uint8_t *ring,
                                       uint32_t lo, uint32_t hi)
{
    using S = SwF<F>;
    using Q = typename S::Q;
    using P = SwPiece<Q>;
    constexpr uint32_t NB = S::NB;
    uint32_t j0, nb;
    sw_slice<NB>(w, o.K / 256, j0, nb);
    const SwRows R = sw_rows(o, b);
    hi = min(hi, sw_slots<F>(R.nrows));
    const uint32_t lr = lane / P::UPB, uk = lane - lr * P::UPB;
    const uint32_t lane_off = lr * o.row_bytes + 16 * uk;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(o.W, (uint64_t)o.w_bytes + RRR_READ_SLACK);
#pragma unroll
    for (uint32_t i = 0; i < SW_DMA_MAX; i++) {
        if (i >= lo && i < hi) {
            const uint32_t rg = i / NB, jj = i % NB;
            const bool ok = lr < P::PPI && rg * P::PPI + lr < R.nrows && jj < nb;
            const uint32_t soff = (R.r0 + rg * P::PPI) * o.row_bytes + (((j0 + jj) * Q::BS) & ~15u);
            sw_dma16(rs, ring + 1024 * i, ok ? lane_off : SW_OOB, soff);
        }
    }
}

template <uint32_t F>
__device__ __forceinline__ uint32_t sw_slots_of(const SwOpDev &o, uint32_t b)
{
    return sw_slots<F>(sw_rows(o, b).nrows);
}

// 16 bytes at LDS byte address a (even): five aligned dwords, shifted by
// a % 4 bytes (0 or 2).
__device__ __forceinline__ u32x4 sw_lds16_u2(const uint8_t *L, uint32_t a)
{
    const uint32_t *p = (const uint32_t *)(L + (a & ~3u));
    const uint32_t s = a & 3u;
    const uint32_t w0 = p[0], w1 = p[1], w2 = p[2], w3 = p[3], w4 = p[4];
    return u32x4{__builtin_amdgcn_alignbyte(w1, w0, s), __builtin_amdgcn_alignbyte(w2, w1, s),
                 __builtin_amdgcn_alignbyte(w3, w2, s), __builtin_amdgcn_alignbyte(w4, w3, s)};
}

// MqQ6K::load for a block at any even LDS offset o (a Q6_K block of 210
// bytes starts 0..14 bytes into its 16-byte aligned window).
__device__ __forceinline__ void sw_load_q6k(MqQ6K::Raw &w, const uint8_t *L, uint32_t o, uint32_t g)
{
    const uint32_t g6 = g >> 1, l0 = 16 * (g & 1);
    w.qa = sw_lds16_u2(L, o + 64 * g6 + l0);
    w.qb = sw_lds16_u2(L, o + 64 * g6 + 32 + l0);
    w.qh = sw_lds16_u2(L, o + 128 + 32 * g6 + l0);
    const uint32_t a = o + 192 + 8 * g6, s = a & 3u;
    const uint32_t *p = (const uint32_t *)(L + (a & ~3u));
    const uint32_t w0 = p[0], w1 = p[1], w2 = p[2];
    w.sc = u32x2{__builtin_amdgcn_alignbyte(w1, w0, s), __builtin_amdgcn_alignbyte(w2, w1, s)};
    const uint32_t ad = o + 208;
    w.d = (*(const uint32_t *)(L + (ad & ~3u)) >> (8 * (ad & 3u))) & 0xFFFFu;
}

// Compute-wave body of one op of form F (next op of form FN): activations,
// weights from the ring into registers, the next op's DMA into the freed
// ring, MFMAs, row partials to LDS.
template <uint32_t F, uint32_t FN>
__device__ __forceinline__ void sw_compute_op(const SwOpDev &o, uint32_t w, uint32_t b, uint32_t lane, uint8_t *ring,
                                              float *part, float inv, const SwOpDev *next)
{
    using S = SwF<F>;
    using Q = typename S::Q;
    using P = SwPiece<Q>;
    constexpr int NB = S::NB, NT = S::NT, ACT = S::ACT;
    constexpr bool AREG = NB == 1;
    constexpr uint32_t DG = NB * 256, D_OFF = 0, A_OFF = 3 * DG, G_OFF = A_OFF + 16 * NB * 16;
    uint8_t *stage = ring + SW_REGION - o.stage;
    const uint32_t K = o.K, B = K / 256, tr = o.tr;
    const SwRows R = sw_rows(o, b);
    const uint32_t n = lane & 15, g = lane >> 4;
    uint32_t j0, nb;
    sw_slice<NB>(w, B, j0, nb);

    // 1. activation inputs of this wave's blocks (coherent loads: written by
    // other workgroups in this launch)
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(o.x, 0xFFFFFFFFull);
    float4 xa[NB], xb[NB];
#pragma unroll
    for (int jj = 0; jj < NB; jj++) {
        const uint32_t k = jj < (int)nb ? (j0 + jj) * 256 + 4 * lane : 0u;
        uint32_t i = k;
        if constexpr (ACT == ACT_GQA_V) {
            const uint32_t hd = o.gqa & 0xFFFFu, hpk = o.gqa >> 16;
            i = K + K / hpk + (k / (hd * hpk)) * hd + k % hd;
        }
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rx, 4 * i, 0, RRR_CPOL_SC1);
        xa[jj] = make_float4(u2f(v.x), u2f(v.y), u2f(v.z), u2f(v.w));
        if constexpr (ACT == ACT_SILU) {
            const u32x4 u = __builtin_amdgcn_raw_buffer_load_b128(rx, 4 * (K + k), 0, RRR_CPOL_SC1);
            xb[jj] = make_float4(u2f(u.x), u2f(u.y), u2f(u.z), u2f(u.w));
        }
        if constexpr (ACT == ACT_RMSNORM) xb[jj] = *(const float4 *)(o.gamma + k);   // read-only
    }
    // the op's weights (DMA issued earlier) and the activations have landed
    sw_wait_vm0();

    // 2. this op's weights from the ring into registers: lane (n, g) holds the
    // pieces of row n of every tile (rows past the tile repeat its last row)
    typename Q::Raw raw[NT][NB];
    const uint32_t nn = min(n, tr - 1);
#pragma unroll
    for (int tl = 0; tl < NT; tl++) {
        const uint32_t rho = min(tl * tr + nn, R.nrows ? R.nrows - 1 : 0u);   // row within the workgroup's rows
        const uint32_t rg = rho / P::PPI, rp = rho - rg * P::PPI;
#pragma unroll
        for (int jj = 0; jj < NB; jj++) {
            if (tl < (int)R.ntl) {
                const uint32_t o16 = 1024 * (rg * NB + jj) + 16 * P::UPB * rp;
                if constexpr (Q::BS % 16 == 0) {
                    Q::load(raw[tl][jj], ring, o16, g);
                } else {
                    // Q6_K: the block starts sh bytes into its window (the same
                    // for every row: rows are whole 16-byte units)
                    const uint32_t sh = ((j0 + jj) * Q::BS) & 15u;
                    sw_load_q6k(raw[tl][jj], ring, o16 + sh, g);
                }
            }
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the ring has been read
    // 3. the first of the next op's weights into the freed ring; the rest
    // after the MFMAs (a wave's load issue stalls once its CU holds some
    // 40 loads, and the MFMAs must not wait behind them)
    if constexpr (FN != SWF_NONE) sw_dma<FN>(*next, w, b, lane, ring, 0u, SW_DMA_EARLY);

    // 4. activation encoding of this wave's slice (the batch-1 GEMV's block
    // floating point, gemv_mq.h)
#pragma unroll
    for (int jj = 0; jj < NB; jj++) {
        const uint32_t f = lane + 64 * jj;
        float4 v = xform4<ACT>(xa[jj], xb[jj], inv);
        if (jj >= (int)nb) v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        const float mx = quad_max(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        int e = 0;
        if (mx > 0.0f && __builtin_isfinite(mx)) {
            int ex;
            (void)frexpf(mx, &ex);
            e = ex - 6;
        }
        uint32_t p0, p1, p2, qb;
        encode4(v, ldexpf(1.0f, 14 - e), p0, p1, p2, qb);
        *(uint32_t *)(stage + D_OFF + 4 * f) = p0;
        *(uint32_t *)(stage + D_OFF + DG + 4 * f) = p1;
        *(uint32_t *)(stage + D_OFF + 2 * DG + 4 * f) = p2;
        i32x4 ax = {0, 0, 0, 0};
        if constexpr (Q::OFF32) {
            ax[0] = -32 * (int)(quad_sum_u32(qb) - 16u * 0x00808080u);
        } else {
            const float sv = quad_sum((v.x + v.y) + (v.z + v.w));
            if ((lane & 3) == 0) *(float *)(stage + G_OFF + f) = sv;
        }
        ax[3] = __float_as_int(__builtin_isfinite(mx) ? ldexpf(1.0f, e - 14) : __builtin_nanf(""));
        if ((lane & 3) == 0) *(i32x4 *)(stage + A_OFF + 4 * f) = ax;
    }
    wave_lds_sync();
    const bool a_live = (n >> 2) == g && (n & 3) < 3;
    const uint32_t a_base = D_OFF + (n & 3) * DG;
    // one super-block a wave: A operands, group factors (the accumulator input
    // is {0, 0, 0, factor} for Q4_K / Q5_K) and group sums in registers
    i32x4 av[AREG ? 4 : 1];
    int fb[AREG ? 4 : 1];
    float gs[AREG ? 4 : 1];
    if constexpr (AREG) {
        static_assert(!Q::OFF32, "one-block forms are Q4_K / Q5_K");
#pragma unroll
        for (int u = 0; u < 4; u++) {
            av[u] = i32x4{0, 0, 0, 0};
            fb[u] = *(const int *)(stage + A_OFF + Q::koff(g, u) + 12);
            gs[u] = *(const float *)(stage + G_OFF + Q::koff(g, u) / 4);
        }
        if (a_live) {
#pragma unroll
            for (int u = 0; u < 4; u++) av[u] = *(const i32x4 *)(stage + a_base + Q::koff(g, u));
        }
    }

    // 5. MFMAs per tile; the 4 k-groups of a row, then row partials to LDS
#pragma unroll
    for (int tl = 0; tl < NT; tl++) {
        if (tl < (int)R.ntl) {
            float acc = 0.0f;
#pragma unroll
            for (int jj = 0; jj < NB; jj++) {
                i32x4 bq[4];
                float sc[4], mn[4], d, dmin;
                Q::decode(raw[tl][jj], g, bq, sc, mn, d, dmin);
                float acc_s = 0.0f, acc_m = 0.0f;
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    i32x4 A, C;
                    float gsum;
                    if constexpr (AREG) {
                        A = av[u];
                        C = i32x4{0, 0, 0, fb[u]};
                        gsum = gs[u];
                    } else {
                        const uint32_t ko = Q::koff(g, u);
                        A = i32x4{0, 0, 0, 0};
                        if (a_live) A = *(const i32x4 *)(stage + a_base + jj * 256 + ko);
                        C = *(const i32x4 *)(stage + A_OFF + 256 * jj + ko);
                        gsum = Q::HAS_MIN ? *(const float *)(stage + G_OFF + 64 * jj + ko / 4) : 0.0f;
                    }
                    const i32x4 cc = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i8x16, A),
                                                                           __builtin_bit_cast(i8x16, bq[u]), C, 0, 0, 0);
                    const int T = cc[0] + cc[1] * 256 + cc[2] * 65536;
                    acc_s = fmaf(sc[u], __int_as_float(cc[3]) * (float)T, acc_s);
                    if constexpr (Q::HAS_MIN) acc_m = fmaf(mn[u], gsum, acc_m);
                }
                acc = fmaf(d, acc_s, acc);
                if constexpr (Q::HAS_MIN) acc = fmaf(-dmin, acc_m, acc);
            }
            acc = lanes4_sum(acc);
            if (lane < 16) part[(tl * SW_CW + w) * 16 + lane] = acc;
        }
    }
}

// The rest of the next op's weights, after this op's partials are counted.
template <uint32_t F, uint32_t FN>
__device__ __forceinline__ void sw_dma_rest(uint32_t w, uint32_t b, uint32_t lane, uint8_t *ring, const SwOpDev *next)
{
    if constexpr (FN != SWF_NONE) sw_dma<FN>(*next, w, b, lane, ring, SW_DMA_EARLY, SW_DMA_MAX);
}

// Sync wave: waits for every workgroup's record of op i-1, releases op i
// (with the RMSNorm factor), then adds the compute waves' row partials and
// the residual, stores the rows and publishes this workgroup's record.
__device__ __forceinline__ bool sw_sync_wave(const SwOpDev *ops, uint32_t nops, uint32_t *state, uint32_t base,
                                             uint32_t lane, uint32_t *ctl, const float *part)
{
    const uint32_t b = blockIdx.x, G = gridDim.x;
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(state, 4ull * SW_STATE_WORDS);
    for (uint32_t i = 0; i < nops; i++) {
        const SwOpDev o = ops[i];
        const bool rms = o.form == SWF_Q5K_RMS || o.form == SWF_Q4K_RMS;
        float sumsq = 0.0f;
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        if (i > 0) {
            // every workgroup's record of op i-1: lane l holds records 4l .. 4l+3
            const uint32_t target = base + i + 1, q = 4 * lane;
            // two polls in flight, issued ~0.2 us apart, so a record is seen
            // about one round trip after it lands
            auto done = [&](const u32x4 &r0, const u32x4 &r1) {
                return __all((q >= G || (int)(r0.x - target) >= 0) && (q + 1 >= G || (int)(r0.z - target) >= 0) &&
                             (q + 2 >= G || (int)(r1.x - target) >= 0) && (q + 3 >= G || (int)(r1.z - target) >= 0));
            };
            auto partial = [&](const u32x4 &r0, const u32x4 &r1) {
                return ((q < G ? u2f(r0.y) : 0.0f) + (q + 1 < G ? u2f(r0.w) : 0.0f)) +
                       ((q + 2 < G ? u2f(r1.y) : 0.0f) + (q + 3 < G ? u2f(r1.w) : 0.0f));
            };
            u32x4 a0 = __builtin_amdgcn_raw_buffer_load_b128(rr, 32 * lane, 0, RRR_CPOL_SC1);
            u32x4 a1 = __builtin_amdgcn_raw_buffer_load_b128(rr, 32 * lane + 16, 0, RRR_CPOL_SC1);
            float ps;
            for (;;) {
                __builtin_amdgcn_s_sleep(8);
                const u32x4 b0 = __builtin_amdgcn_raw_buffer_load_b128(rr, 32 * lane, 0, RRR_CPOL_SC1);
                const u32x4 b1 = __builtin_amdgcn_raw_buffer_load_b128(rr, 32 * lane + 16, 0, RRR_CPOL_SC1);
                if (done(a0, a1)) {
                    ps = partial(a0, a1);
                    break;
                }
                __builtin_amdgcn_s_sleep(8);
                a0 = __builtin_amdgcn_raw_buffer_load_b128(rr, 32 * lane, 0, RRR_CPOL_SC1);
                a1 = __builtin_amdgcn_raw_buffer_load_b128(rr, 32 * lane + 16, 0, RRR_CPOL_SC1);
                if (done(b0, b1)) {
                    ps = partial(b0, b1);
                    break;
                }
                if (__builtin_amdgcn_s_memrealtime() - t0 > SW_SPIN_TICKS) return false;
            }
            sumsq = wave_sum(ps);
        } else if (rms) {
            // op 0's input was written before the launch: its sum of squares here
            const __amdgpu_buffer_rsrc_t rx = make_rsrc(o.x, 4ull * o.K);
            float ps = 0.0f;
            for (uint32_t f = lane; f < o.K / 4; f += 64) {
                const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rx, 16 * f, 0, RRR_CPOL_SC1);
                ps = __builtin_fmaf(u2f(v.x), u2f(v.x), ps);
                ps = __builtin_fmaf(u2f(v.y), u2f(v.y), ps);
                ps = __builtin_fmaf(u2f(v.z), u2f(v.z), ps);
                ps = __builtin_fmaf(u2f(v.w), u2f(v.w), ps);
            }
            sumsq = wave_sum(ps);
        }
        if (lane == 0) {
            if (rms) ctl[1] = __float_as_uint(rms_inv(sumsq, o.K, o.eps));
            sw_lds_store(ctl, i + 1);                      // go
        }
        // this workgroup's rows: lane q = 16 * tile + row
        const SwRows R = sw_rows(o, b);
        const uint32_t tl = lane >> 4, r = lane & 15, row = R.r0 + tl * o.tr + r;
        const bool mine = tl < R.ntl && r < o.tr && row < o.N;
        const __amdgpu_buffer_rsrc_t ry = make_rsrc(o.y, 4ull * o.N);
        float res = 0.0f;
        if (o.residual && mine) res = u2f(__builtin_amdgcn_raw_buffer_load_b32(ry, 4 * row, 0, RRR_CPOL_SC1));
        // the compute waves' partials of op i
        while (sw_lds_load(ctl + 2) < (i + 1) * SW_CW) {
            if (__builtin_amdgcn_s_memrealtime() - t0 > SW_SPIN_TICKS) return false;
            __builtin_amdgcn_s_sleep(1);
        }
        float sq = 0.0f;
        if (mine) {
            float v = part[(tl * SW_CW) * 16 + r];
#pragma unroll
            for (uint32_t w = 1; w < SW_CW; w++) v += part[(tl * SW_CW + w) * 16 + r];
            if (o.residual) v = res + v;
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), ry, 4 * row, 0, RRR_CPOL_SC1);
            sq = v * v;
        }
        sq = wave_sum(sq);
        // rows through to the coherent level, then the record
        sw_wait_vm0();
        if (lane == 0) {
            const u32x2 rec = {base + i + 2, __float_as_uint(sq)};
            __builtin_amdgcn_raw_buffer_store_b64(rec, rr, 8 * b, 0, RRR_CPOL_SC1);
        }
    }
    return true;
}

// Form pairs the decode layer runs: (form of op i, form of op i+1).
#define RRR_SW_FORM_PAIRS(X)                                                                        \
    X(SWF_Q5K_RMS, SWF_Q4K_GQA) X(SWF_Q4K_GQA, SWF_Q4K_RMS) X(SWF_Q4K_RMS, SWF_Q6K_SILU)          \
    X(SWF_Q4K_RMS, SWF_Q4K_SILU) X(SWF_Q6K_SILU, SWF_Q5K_RMS) X(SWF_Q4K_SILU, SWF_Q5K_RMS)
// every form, as the last op of a sweep (no next op)
#define RRR_SW_FORMS(X) X(SWF_Q5K_RMS) X(SWF_Q4K_RMS) X(SWF_Q4K_GQA) X(SWF_Q4K_SILU) X(SWF_Q6K_SILU)

__device__ __forceinline__ uint32_t sw_pair(uint32_t f, uint32_t fn) { return 8 * f + fn; }

__global__ __launch_bounds__(SW_THREADS) void sweep_kernel(const SwOpDev *ops, uint32_t nops, uint32_t *state)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t sw_lds[];
    const uint32_t t = threadIdx.x, lane = t & 63, w = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t b = blockIdx.x;
    uint32_t *ctl = (uint32_t *)(sw_lds + SW_CTL_OFF);   // go, RMSNorm factor, done count, epoch base, runs
    float *part = (float *)(sw_lds + SW_PART_OFF);
    if (t == 0) {
        const uint32_t runs = state[SW_RUNC_OFF + b];
        ctl[0] = 0;
        ctl[1] = 0;
        ctl[2] = 0;
        ctl[3] = runs * (nops + 2);
        ctl[4] = runs;
    }
    __syncthreads();
    const uint32_t base = ctl[3];

    if (w == SW_CW) {
        const bool ok = sw_sync_wave(ops, nops, state, base, lane, ctl, part);
        if (!ok) {
            if (lane == 0) {
                sw_lds_store(ctl, SW_ABORT);
                __hip_atomic_store(state + SW_ERR_OFF, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        } else if (lane == 0) {
            state[SW_RUNC_OFF + b] = ctl[4] + 1;
        }
        return;
    }

    // compute wave w: op 0's weights stream in right away
    uint8_t *ring = sw_lds + w * SW_REGION;
    {
        const SwOpDev o0 = ops[0];
        switch (o0.form) {
        case SWF_Q5K_RMS: sw_dma<SWF_Q5K_RMS>(o0, w, b, lane, ring, 0u, SW_DMA_MAX); break;
        case SWF_Q4K_RMS: sw_dma<SWF_Q4K_RMS>(o0, w, b, lane, ring, 0u, SW_DMA_MAX); break;
        case SWF_Q4K_GQA: sw_dma<SWF_Q4K_GQA>(o0, w, b, lane, ring, 0u, SW_DMA_MAX); break;
        case SWF_Q4K_SILU: sw_dma<SWF_Q4K_SILU>(o0, w, b, lane, ring, 0u, SW_DMA_MAX); break;
        default: sw_dma<SWF_Q6K_SILU>(o0, w, b, lane, ring, 0u, SW_DMA_MAX); break;
        }
    }
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (uint32_t i = 0; i < nops; i++) {
        // the lane index is redefined every op, so nothing derived from it
        // is hoisted out of the loop (held across ops, it would not fit the
        // 128 registers and be spilled to scratch)
        uint32_t ln = lane;
        asm volatile("" : "+v"(ln));
        const SwOpDev o = ops[i];
        const SwOpDev *next = i + 1 < nops ? ops + i + 1 : nullptr;
        const uint32_t fn = next ? next->form : (uint32_t)SWF_NONE;
        // released by the sync wave once the previous op is done everywhere
        uint32_t go;
        while ((go = sw_lds_load(ctl)) < i + 1) {
            if (__builtin_amdgcn_s_memrealtime() - t0 > 4 * SW_SPIN_TICKS) go = SW_ABORT;
            if (go == SW_ABORT) break;
            __builtin_amdgcn_s_sleep(1);
        }
        if (go == SW_ABORT) break;
        const float inv = u2f(ctl[1]);
        switch (sw_pair(o.form, fn)) {
#define RRR_SW_CASE(F, FN) \
        case 8 * F + FN: \
            sw_compute_op<F, FN>(o, w, b, ln, ring, part, inv, next); \
            if (ln == 0) __hip_atomic_fetch_add(ctl + 2, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP); \
            sw_dma_rest<F, FN>(w, b, ln, ring, next); \
            break;
#define RRR_SW_CASE_LAST(F) RRR_SW_CASE(F, SWF_NONE)
            RRR_SW_FORM_PAIRS(RRR_SW_CASE)
            RRR_SW_FORMS(RRR_SW_CASE_LAST)
#undef RRR_SW_CASE_LAST
#undef RRR_SW_CASE
        default: break;   // not reached: rrr_sweep_create admits only the pairs above
        }
    }
    // no DMA may still be writing this workgroup's LDS when its waves end
    sw_wait_vm0();
}

// ---- host side ----------------------------------------------------------

static uint32_t sw_form_nb(uint32_t form) { return form == SWF_Q4K_SILU || form == SWF_Q6K_SILU ? SW_NB_MAX : 1u; }

static uint32_t sw_form_nt(uint32_t form)
{
    switch (form) {
    case SWF_Q5K_RMS: return SwF<SWF_Q5K_RMS>::NT;
    case SWF_Q4K_RMS: return SwF<SWF_Q4K_RMS>::NT;
    case SWF_Q4K_GQA: return SwF<SWF_Q4K_GQA>::NT;
    case SWF_Q4K_SILU: return SwF<SWF_Q4K_SILU>::NT;
    default: return SwF<SWF_Q6K_SILU>::NT;
    }
}

static uint32_t sw_form_ppi(uint32_t form)
{
    switch (form) {
    case SWF_Q5K_RMS: return SwPiece<MqQ5K>::PPI;
    case SWF_Q6K_SILU: return SwPiece<MqQ6K>::PPI;
    default: return SwPiece<MqQ4K>::PPI;
    }
}

// ring slots (1 KB) of the largest workgroup share and staging bytes of an op
static uint32_t sw_form_slots(uint32_t form, uint32_t per, uint32_t tr)
{
    const uint32_t ppi = sw_form_ppi(form);
    return (per * tr + ppi - 1) / ppi * sw_form_nb(form);
}
static uint32_t sw_form_stage(uint32_t form) { return 1088u * sw_form_nb(form); }

// Per-op set-up: the form and the tiling over `grid` workgroups; false if the
// sweep cannot run the op.
bool sweep_plan_op(const GemvArgs &a, uint32_t act, uint32_t grid, uint32_t &variant, uint32_t &ntiles, uint32_t &tr,
                   size_t &lds)
{
    if (a.M != 1 || a.K % 256 || a.K == 0 || a.w_bytes + RRR_READ_SLACK >= SW_OOB || grid == 0 || grid > SW_G_MAX)
        return false;
    const uint32_t B = a.K / 256;
    const bool small = B <= SW_CW, large = B > SW_CW && B <= SW_CW * SW_NB_MAX;
    if (a.type == T_Q5_K && act == ACT_RMSNORM && small) variant = SWF_Q5K_RMS;
    else if (a.type == T_Q4_K && act == ACT_RMSNORM && small) variant = SWF_Q4K_RMS;
    else if (a.type == T_Q4_K && act == ACT_GQA_V && small) variant = SWF_Q4K_GQA;
    else if (a.type == T_Q4_K && act == ACT_SILU && large) variant = SWF_Q4K_SILU;
    else if (a.type == T_Q6_K && act == ACT_SILU && large && (B * 210) % 16 == 0) variant = SWF_Q6K_SILU;
    else return false;
    const uint32_t nt = sw_form_nt(variant);
    uint32_t per;
    mq_tiles(a.N, grid, nt, 1u, tr, ntiles, per);
    // (an op's ring is read into registers before its staging is written;
    // the next op's ring beside this op's staging is checked pairwise)
    if ((uint64_t)ntiles > (uint64_t)per * grid || per > nt || sw_form_slots(variant, per, tr) > SW_DMA_MAX)
        return false;
    lds = SW_LDS_BYTES;
    return true;
}

// Whether op `next` may follow op `cur` (a form pair the kernel carries, and
// the next op's ring slots fit beside the current op's staging).
bool sweep_pair_ok(uint32_t cur, uint32_t cur_ntiles, uint32_t cur_tr, uint32_t next, uint32_t next_ntiles,
                   uint32_t next_tr, uint32_t grid)
{
    (void)cur_ntiles;
    (void)cur_tr;
    bool known = false;
#define RRR_SW_PAIR_OK(F, FN) known = known || (cur == F && next == FN);
    RRR_SW_FORM_PAIRS(RRR_SW_PAIR_OK)
#undef RRR_SW_PAIR_OK
    const uint32_t per_next = (next_ntiles + grid - 1) / grid;
    return known && sw_form_slots(next, per_next, next_tr) * 1024 + sw_form_stage(cur) <= SW_REGION;
}

size_t sweep_op_bytes() { return sizeof(SwOpDev); }

void sweep_pack_op(void *dst, const GemvArgs &a, uint32_t variant, uint32_t ntiles, uint32_t tr, uint32_t grid)
{
    SwOpDev o{};
    o.W = a.W;
    o.x = a.x;
    o.gamma = a.gamma;
    o.y = a.y;
    o.w_bytes = (uint32_t)a.w_bytes;
    o.row_bytes = (a.K / 256) * (uint32_t)block_bytes(a.type);
    o.K = a.K;
    o.N = a.N;
    o.tr = tr;
    o.ntiles = ntiles;
    o.per = (ntiles + grid - 1) / grid;
    o.form = variant;
    o.residual = a.residual;
    o.gqa = a.head_dim | (a.heads_per_kv << 16);
    o.eps = a.eps;
    o.stage = sw_form_stage(variant);
    *(SwOpDev *)dst = o;
}

uint32_t sweep_cus() { return device_cus(); }

// Workgroups of the sweep: one per CU (at most SW_G_MAX) when the workgroup
// fits there, else 0.
uint32_t sweep_grid(size_t)
{
    int per = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, sweep_kernel, SW_THREADS, SW_LDS_BYTES) != hipSuccess ||
        per < 1)
        return 0;
    return min(device_cus(), SW_G_MAX);
}

size_t sweep_state_words() { return SW_STATE_WORDS; }
size_t sweep_err_word() { return SW_ERR_OFF; }

hipError_t launch_sweep(const void *ops, uint32_t nops, uint32_t *state, uint32_t grid, hipStream_t s)
{
    hipLaunchKernelGGL(sweep_kernel, dim3(grid), dim3(SW_THREADS), SW_LDS_BYTES, s, (const SwOpDev *)ops, nops, state);
    return hipGetLastError();
}

}  // namespace rrr
