// gemm.hip -- prefill dequant-GEMM: Y[M][N] = X_bf16[M][K] . W[N][K]^T with W
// in raw Q4_K / Q5_K / Q6_K super-blocks (the batched shape of phi4.rs:1257-1268
// at prompt length; the reference has no MFMA kernel for it).
//
// Workgroup: 256 threads = 2 x 2 waves over a BM x BN output tile, each wave a
// (BM/2) x (BN/2) block of 16x16 v_mfma_f32_16x16x32_f16 tiles with fp32
// accumulators (lane l: A row l%16 and B column l%16 at k-group l/16, 8 f16
// each; D rows 4*(l/16)+r of column l%16 in register r).
//
// K steps of BK = 128 (half a super-block).  Per step every weight row of the
// tile contributes two 64-element units ("pairs": elements 64g..64g+63 of a
// super-block, one scale pair for Q4_K/Q5_K, four scales for Q6_K); a thread
// dequantizes one unit with the reference's formulas (phi4.rs:444-542) in f32
// and rounds to f16 into LDS.  X rows are converted bf16 -> f16, exact for
// |x| in f16's normal range.  LDS is double-buffered: the MFMAs of step s read
// one buffer while the raw data of step s+1, loaded into registers during
// step s-1, is dequantized into the other.  fp16 weights keep the product
// error at 2^-12 per weight (bf16 weights would be 2^-9).
//
// Tile order: the M/BM tiles of one N tile get workgroup ids congruent mod 8,
// so they run on the same XCD and the weight tile is fetched from HBM once.
#include "device_common.h"
#include "internal.h"

namespace rrr {

typedef _Float16 f16x8v __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));

// Scalar offset past every input byte (the launcher requires smaller buffers):
// loads of the step after the last return zeros and move no data.
constexpr uint32_t GM_OOB = 0x80000000u;

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

// Raw bytes of one 64-element unit (pair g of a super-block) and its dequant.
// Q4_K (phi4.rs:481-510): qs bytes 32g..32g+31, low nibbles = sub-block 2g,
// high nibbles = 2g+1; w = (d*sc)*q - (dmin*m).
struct GqQ4K {
    static constexpr uint32_t BS = 144;
    struct Raw { u32x4 hdr, q0, q1; };
    __device__ static void load(Raw &r, __amdgpu_buffer_rsrc_t rs, uint32_t boff, uint32_t g, uint32_t so)
    {
        r.hdr = __builtin_amdgcn_raw_buffer_load_b128(rs, boff, so, RRR_CPOL_NT);
        r.q0 = __builtin_amdgcn_raw_buffer_load_b128(rs, boff + 16 + 32 * g, so, RRR_CPOL_NT);
        r.q1 = __builtin_amdgcn_raw_buffer_load_b128(rs, boff + 32 + 32 * g, so, RRR_CPOL_NT);
    }
    // out[j] packs elements 2j, 2j+1 of the unit (32 dwords)
    __device__ static void dequant(const Raw &r, uint32_t g, uint32_t *out)
    {
        const float d = h2f(r.hdr.x), dmin = h2f(r.hdr.x >> 16);
        uint32_t s0, m0, s1, m1;
        scale_min_k4(2 * g, r.hdr.y, r.hdr.z, r.hdr.w, s0, m0);
        scale_min_k4(2 * g + 1, r.hdr.y, r.hdr.z, r.hdr.w, s1, m1);
        const float a0 = __fmul_rn(d, (float)s0), b0 = __fmul_rn(dmin, (float)m0);
        const float a1 = __fmul_rn(d, (float)s1), b1 = __fmul_rn(dmin, (float)m1);
        const u32x4 q[2] = {r.q0, r.q1};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t w = q[i >> 2][i & 3];  // bytes 4i..4i+3 of the 32
#pragma unroll
            for (int h = 0; h < 2; h++) {        // h=0: low nibbles (sub-block 2g), h=1: high (2g+1)
                const uint32_t v = (w >> (4 * h)) & 0x0F0F0F0Fu;
                const float A = h ? a1 : a0, B = h ? b1 : b0;
                const float e0 = __fsub_rn(__fmul_rn(A, (float)(v & 255u)), B);
                const float e1 = __fsub_rn(__fmul_rn(A, (float)((v >> 8) & 255u)), B);
                const float e2 = __fsub_rn(__fmul_rn(A, (float)((v >> 16) & 255u)), B);
                const float e3 = __fsub_rn(__fmul_rn(A, (float)(v >> 24)), B);
                out[16 * h + 2 * i] = pk_f16_rn(e0, e1);
                out[16 * h + 2 * i + 1] = pk_f16_rn(e2, e3);
            }
        }
    }
};

// Q5_K (phi4.rs:512-542): Q4_K plus bit (2g / 2g+1) of qh[l] as bit 4.
struct GqQ5K {
    static constexpr uint32_t BS = 176;
    struct Raw { u32x4 hdr, h0, h1, q0, q1; };
    __device__ static void load(Raw &r, __amdgpu_buffer_rsrc_t rs, uint32_t boff, uint32_t g, uint32_t so)
    {
        r.hdr = __builtin_amdgcn_raw_buffer_load_b128(rs, boff, so, RRR_CPOL_NT);
        r.h0 = __builtin_amdgcn_raw_buffer_load_b128(rs, boff + 16, so, RRR_CPOL_NT);
        r.h1 = __builtin_amdgcn_raw_buffer_load_b128(rs, boff + 32, so, RRR_CPOL_NT);
        r.q0 = __builtin_amdgcn_raw_buffer_load_b128(rs, boff + 48 + 32 * g, so, RRR_CPOL_NT);
        r.q1 = __builtin_amdgcn_raw_buffer_load_b128(rs, boff + 64 + 32 * g, so, RRR_CPOL_NT);
    }
    __device__ static void dequant(const Raw &r, uint32_t g, uint32_t *out)
    {
        const float d = h2f(r.hdr.x), dmin = h2f(r.hdr.x >> 16);
        uint32_t s0, m0, s1, m1;
        scale_min_k4(2 * g, r.hdr.y, r.hdr.z, r.hdr.w, s0, m0);
        scale_min_k4(2 * g + 1, r.hdr.y, r.hdr.z, r.hdr.w, s1, m1);
        const float a0 = __fmul_rn(d, (float)s0), b0 = __fmul_rn(dmin, (float)m0);
        const float a1 = __fmul_rn(d, (float)s1), b1 = __fmul_rn(dmin, (float)m1);
        const u32x4 q[2] = {r.q0, r.q1}, qh[2] = {r.h0, r.h1};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t w = q[i >> 2][i & 3], hb = qh[i >> 2][i & 3];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint32_t v = ((w >> (4 * h)) & 0x0F0F0F0Fu) | (((hb >> (2 * g + h)) & 0x01010101u) << 4);
                const float A = h ? a1 : a0, B = h ? b1 : b0;
                const float e0 = __fsub_rn(__fmul_rn(A, (float)(v & 255u)), B);
                const float e1 = __fsub_rn(__fmul_rn(A, (float)((v >> 8) & 255u)), B);
                const float e2 = __fsub_rn(__fmul_rn(A, (float)((v >> 16) & 255u)), B);
                const float e3 = __fsub_rn(__fmul_rn(A, (float)(v >> 24)), B);
                out[16 * h + 2 * i] = pk_f16_rn(e0, e1);
                out[16 * h + 2 * i + 1] = pk_f16_rn(e2, e3);
            }
        }
    }
};

// Q6_K (phi4.rs:444-479): pair g = quadrants 2(g&1), 2(g&1)+1 of half g/2:
// element 64g + 32u + l (u = 0, 1) is ql[64(g/2) + 32u + l] (low nibble for even
// g, high for odd) with qh[32(g/2) + l] bits 2(2(g&1)+u); scale index
// is = (64g + 32u + l) / 16; w = (d*sc[is]) * (q - 32).
struct GqQ6K {
    static constexpr uint32_t BS = 210;
    struct Raw { u32x4 l0, l1, l2, l3, h0, h1; uint32_t sc, d; };
    __device__ static void load(Raw &r, __amdgpu_buffer_rsrc_t rs, uint32_t boff, uint32_t g, uint32_t so)
    {
        const uint32_t g6 = g >> 1;
        r.l0 = __builtin_amdgcn_raw_buffer_load_b128(rs, boff + 64 * g6, so, RRR_CPOL_NT);
        r.l1 = __builtin_amdgcn_raw_buffer_load_b128(rs, boff + 64 * g6 + 16, so, RRR_CPOL_NT);
        r.l2 = __builtin_amdgcn_raw_buffer_load_b128(rs, boff + 64 * g6 + 32, so, RRR_CPOL_NT);
        r.l3 = __builtin_amdgcn_raw_buffer_load_b128(rs, boff + 64 * g6 + 48, so, RRR_CPOL_NT);
        r.h0 = __builtin_amdgcn_raw_buffer_load_b128(rs, boff + 128 + 32 * g6, so, RRR_CPOL_NT);
        r.h1 = __builtin_amdgcn_raw_buffer_load_b128(rs, boff + 128 + 32 * g6 + 16, so, RRR_CPOL_NT);
        r.sc = __builtin_amdgcn_raw_buffer_load_b32(rs, boff + 192 + 4 * g, so, RRR_CPOL_NT);
        r.d = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, boff + 208, so, RRR_CPOL_NT);
    }
    __device__ static void dequant(const Raw &r, uint32_t g, uint32_t *out)
    {
        const float d = h2f(r.d);
        const uint32_t hi = g & 1;
        float ds[4];
#pragma unroll
        for (int s = 0; s < 4; s++) ds[s] = __fmul_rn(d, (float)(int8_t)byte_of(r.sc, s));
        const u32x4 ql[4] = {r.l0, r.l1, r.l2, r.l3}, qh[2] = {r.h0, r.h1};
#pragma unroll
        for (int u = 0; u < 2; u++) {
#pragma unroll
            for (int i = 0; i < 8; i++) {                          // positions l = 4i..4i+3
                const uint32_t w = ql[2 * u + (i >> 2)][i & 3], hb = qh[i >> 2][i & 3];
                const uint32_t shift = 2 * (2 * hi + u);
                const uint32_t v = ((w >> (4 * hi)) & 0x0F0F0F0Fu) | (((hb >> shift) & 0x03030303u) << 4);
                const float A = ds[2 * u + (i >= 4)];              // is = 4g + 2u + l/16
                const float e0 = __fmul_rn(A, (float)((int)(v & 255u) - 32));
                const float e1 = __fmul_rn(A, (float)((int)((v >> 8) & 255u) - 32));
                const float e2 = __fmul_rn(A, (float)((int)((v >> 16) & 255u) - 32));
                const float e3 = __fmul_rn(A, (float)((int)(v >> 24) - 32));
                out[16 * u + 2 * i] = pk_f16_rn(e0, e1);
                out[16 * u + 2 * i + 1] = pk_f16_rn(e2, e3);
            }
        }
    }
};

template <class Q, int BM, int BN>
__global__ __launch_bounds__(256) void gemm_dq_kernel(const uint16_t *X, const uint8_t *W, float *Y, uint32_t K,
                                                      uint32_t N, uint32_t M, uint32_t tiles_n)
{
    constexpr int BK = 128, LDK = BK + 8;                  // f16 per LDS row (16-byte pad)
    constexpr int TI = BM / 32, TJ = BN / 32;              // 16x16 tiles per wave
    constexpr int UNITS = BN * 2;                          // weight units per step
    constexpr int XPT = BM * BK / 256 / 8;                 // X 16-byte loads per thread
    extern __shared__ float smem[];
    _Float16 *As = (_Float16 *)smem;                       // [2][BM][LDK]
    _Float16 *Bs = As + 2 * BM * LDK;                      // [2][BN][LDK]

    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1;
    // tile of this workgroup (same XCD for the M tiles of one N tile)
    const uint32_t id = blockIdx.x, tiles_m = M / BM;
    uint32_t nt, mt;
    if (tiles_n % 8 == 0) {
        nt = (id / (8 * tiles_m)) * 8 + id % 8;
        mt = (id / 8) % tiles_m;
    } else {
        nt = id / tiles_m;
        mt = id % tiles_m;
    }
    const uint32_t m0 = mt * BM, n0 = nt * BN;
    const uint32_t nsteps = K / BK, B = K / 256;

    // weight unit of this thread: row n0 + ur, pair 2*(step%2) + up
    const bool u_ok = t < UNITS;
    const uint32_t ur = (t >> 1) % BN, up = t & 1;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(W, (uint64_t)N * B * Q::BS);
    const uint32_t wrow = (n0 + ur) * B * Q::BS;
    // X: thread covers row m0 + xr, 8 * XPT consecutive k of the step
    const uint32_t xr = t / (256 / BM), xk = (t % (256 / BM)) * 8 * XPT;
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(X, (uint64_t)M * K * 2);
    const uint32_t xrow = ((m0 + xr) * K + xk) * 2;

    typename Q::Raw raw;
    u32x4 xv[XPT];
    auto issue = [&](uint32_t s) {
        const uint32_t so_w = s < nsteps ? (s >> 1) * Q::BS : GM_OOB;
        const uint32_t so_x = s < nsteps ? s * BK * 2 : GM_OOB;
        Q::load(raw, wrs, wrow, 2 * (s & 1) + up, so_w);
#pragma unroll
        for (int i = 0; i < XPT; i++)
            xv[i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xrow + 16 * i, so_x, 0);  // reused by every N tile: cached
    };
    auto stage = [&](uint32_t s, int buf) {
        if (u_ok) {
            uint32_t o[32];
            Q::dequant(raw, 2 * (s & 1) + up, o);
            _Float16 *dst = Bs + (buf * BN + ur) * LDK + 64 * up;
#pragma unroll
            for (int i = 0; i < 8; i++) *(u32x4 *)(dst + 8 * i) = u32x4{o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]};
        }
        _Float16 *xd = As + (buf * BM + xr) * LDK + xk;
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const u32x4 v = xv[i];
            u32x4 h;
#pragma unroll
            for (int c = 0; c < 4; c++) h[c] = pk_f16(__uint_as_float(v[c] << 16), __uint_as_float(v[c] & 0xFFFF0000u));
            *(u32x4 *)(xd + 8 * i) = h;
        }
    };

    f32x4 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; i++)
#pragma unroll
        for (int j = 0; j < TJ; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    issue(0);
    stage(0, 0);
    issue(1);
    __syncthreads();
    const uint32_t fr = lane & 15, fk = 8 * (lane >> 4);
    for (uint32_t s = 0; s < nsteps; s++) {
        const int cur = s & 1;
        const _Float16 *Ab = As + (cur * BM + wm * (BM / 2) + fr) * LDK + fk;
        const _Float16 *Bb = Bs + (cur * BN + wn * (BN / 2) + fr) * LDK + fk;
#pragma unroll
        for (int kk = 0; kk < BK / 32; kk++) {
            f16x8v a[TI], b[TJ];
#pragma unroll
            for (int i = 0; i < TI; i++) a[i] = *(const f16x8v *)(Ab + 16 * i * LDK + 32 * kk);
#pragma unroll
            for (int j = 0; j < TJ; j++) b[j] = *(const f16x8v *)(Bb + 16 * j * LDK + 32 * kk);
#pragma unroll
            for (int i = 0; i < TI; i++)
#pragma unroll
                for (int j = 0; j < TJ; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        // next step's data into the other buffer, then the loads two steps ahead
        stage(s + 1, cur ^ 1);
        issue(s + 2);
        __syncthreads();
    }

    // D rows 4*(l/16)+r of column l%16 in register r
#pragma unroll
    for (int i = 0; i < TI; i++)
#pragma unroll
        for (int j = 0; j < TJ; j++) {
            const uint32_t n = n0 + wn * (BN / 2) + 16 * j + fr;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t m = m0 + wm * (BM / 2) + 16 * i + 4 * (lane >> 4) + r;
                Y[(uint64_t)m * N + n] = acc[i][j][r];
            }
        }
}

template <class Q, int BM, int BN>
static hipError_t go_gemm(const uint16_t *X, const uint8_t *W, float *Y, uint32_t K, uint32_t N, uint32_t M,
                          hipStream_t s)
{
    constexpr size_t lds = 2 * (size_t)(BM + BN) * (128 + 8) * 2;
    static_assert(lds <= 160 * 1024, "LDS per workgroup");
    const uint32_t tiles_n = N / BN, tiles = tiles_n * (M / BM);
    hipLaunchKernelGGL((gemm_dq_kernel<Q, BM, BN>), dim3(tiles), dim3(256), lds, s, X, W, Y, K, N, M, tiles_n);
    return hipGetLastError();
}

template <class Q>
static hipError_t go_gemm_t(const uint16_t *X, const uint8_t *W, float *Y, uint32_t K, uint32_t N, uint32_t M,
                            hipStream_t s)
{
    // 128 x 128 tiles when they fill the CUs, else 128 x 64
    if (N % 128 == 0 && (N / 128) * (M / 128) >= 256) return go_gemm<Q, 128, 128>(X, W, Y, K, N, M, s);
    return go_gemm<Q, 128, 64>(X, W, Y, K, N, M, s);
}

bool gemm_bf16_supported(uint32_t type, uint32_t K, uint32_t N, uint32_t M, uint64_t w_bytes, uint64_t x_bytes)
{
    (void)w_bytes;
    return (type == T_Q4_K || type == T_Q5_K || type == T_Q6_K) && K % 256 == 0 && N % 64 == 0 && M % 128 == 0 &&
           (uint64_t)N * (K / 256) * 210 + RRR_READ_SLACK < GM_OOB && x_bytes + RRR_READ_SLACK < GM_OOB;
}

hipError_t launch_gemm_bf16(const uint16_t *X, const uint8_t *W, uint64_t w_bytes, uint32_t type, float *Y,
                            uint32_t K, uint32_t N, uint32_t M, hipStream_t s)
{
    if (!gemm_bf16_supported(type, K, N, M, w_bytes, (uint64_t)M * K * 2)) return hipErrorNotSupported;
    switch (type) {
    case T_Q4_K: return go_gemm_t<GqQ4K>(X, W, Y, K, N, M, s);
    case T_Q5_K: return go_gemm_t<GqQ5K>(X, W, Y, K, N, M, s);
    case T_Q6_K: return go_gemm_t<GqQ6K>(X, W, Y, K, N, M, s);
    default: return hipErrorNotSupported;
    }
}

}  // namespace rrr
