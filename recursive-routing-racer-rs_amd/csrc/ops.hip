// ops.hip -- dequant, RMSNorm, SwiGLU glue, residual add, fill, transposed
// logits and argmax kernels of the decode path.
#include "device_common.h"
#include "internal.h"

namespace rrr {

// ---------------------------------------------------------------------------
// Standalone dequant to f32: bit-exact with phi4.rs:444-542.  One thread per
// 16 consecutive output elements.  Every product below is exact in f32
// (11-bit d times a 6-bit scale times a 6-bit quant), so each output carries
// at most the single rounding of `q*s - m` that the Rust code performs.
template <uint32_t TYPE>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t *__restrict__ W, uint64_t w_bytes,
                                                       float *__restrict__ out, uint64_t n_groups)
{
    const uint64_t gid = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= n_groups) return;
    const uint64_t blk = gid >> 4;
    const uint32_t e0 = (uint32_t)(gid & 15) * 16;
    float v[16];
    if constexpr (TYPE == T_Q4_K || TYPE == T_Q5_K) {
        const uint32_t BS = TYPE == T_Q4_K ? 144 : 176;
        const uint8_t *b = W + blk * BS;
        const float d = h2f(b[0] | (b[1] << 8)), dmin = h2f(b[2] | (b[3] << 8));
        const uint32_t sub = e0 / 32, j0 = e0 % 32, pair = sub / 2;
        uint32_t sc, mn;
        const uint8_t *q = b + 4;
        if (sub < 4) {
            sc = q[sub] & 63u;
            mn = q[sub + 4] & 63u;
        } else {
            const uint32_t i = sub - 4;
            sc = (q[8 + i] & 0x0Fu) | ((uint32_t)(q[i] >> 6) << 4);
            mn = (q[8 + i] >> 4) | ((uint32_t)(q[4 + i] >> 6) << 4);
        }
        const float s = __fmul_rn(d, (float)sc), m = __fmul_rn(dmin, (float)mn);
        const uint8_t *qs = b + (TYPE == T_Q4_K ? 16 : 48);
        for (int i = 0; i < 16; i++) {
            const uint32_t j = j0 + i;
            const uint8_t qb = qs[pair * 32 + j];
            uint32_t qi = (sub & 1) ? (qb >> 4) : (qb & 0xFu);
            if constexpr (TYPE == T_Q5_K) qi |= ((uint32_t)(b[16 + j] >> sub) & 1u) << 4;
            v[i] = __fsub_rn(__fmul_rn((float)qi, s), m);
        }
    } else if constexpr (TYPE == T_Q6_K) {
        const uint8_t *b = W + blk * 210;
        const float d = h2f(b[208] | (b[209] << 8));
        const uint32_t g = e0 / 128, quad = (e0 % 128) / 32, l0 = e0 % 32;
        const uint32_t is = g * 8 + l0 / 16 + 2 * quad;
        const float ds = __fmul_rn(d, (float)(int8_t)b[192 + is]);
        for (int i = 0; i < 16; i++) {
            const uint32_t l = l0 + i;
            const uint8_t qlb = b[g * 64 + l + (quad & 1) * 32];
            const uint32_t lo = (quad < 2) ? (qlb & 0xFu) : (qlb >> 4);
            const uint32_t hi = (b[128 + g * 32 + l] >> (2 * quad)) & 3u;
            v[i] = __fmul_rn(ds, (float)((int)(lo | (hi << 4)) - 32));
        }
    } else {
        const float *f = (const float *)W + gid * 16;
        for (int i = 0; i < 16; i++) v[i] = f[i];
    }
    float4 *o = (float4 *)(out + gid * 16);
    for (int i = 0; i < 4; i++) o[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
}

hipError_t launch_dequant(uint32_t type, const uint8_t *W, uint64_t w_bytes, float *out, uint64_t n,
                          hipStream_t s)
{
    const uint64_t ng = n / 16;
    const dim3 grid((unsigned)((ng + 255) / 256));
    switch (type) {
    case T_Q4_K: hipLaunchKernelGGL(dequant_kernel<T_Q4_K>, grid, dim3(256), 0, s, W, w_bytes, out, ng); break;
    case T_Q5_K: hipLaunchKernelGGL(dequant_kernel<T_Q5_K>, grid, dim3(256), 0, s, W, w_bytes, out, ng); break;
    case T_Q6_K: hipLaunchKernelGGL(dequant_kernel<T_Q6_K>, grid, dim3(256), 0, s, W, w_bytes, out, ng); break;
    case T_F32: hipLaunchKernelGGL(dequant_kernel<T_F32>, grid, dim3(256), 0, s, W, w_bytes, out, ng); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// An f32 result as output type TO: itself, or its f16 rounding (nearest
// even).  The asm keeps the f32 value: without it the compiler may fold the
// last multiply into one mixed-precision op that rounds the exact product to
// f16 once, which is not the f32 result's rounding.
template <typename TO>
__device__ __forceinline__ TO to_out(float v)
{
    if constexpr (sizeof(TO) == 2) asm volatile("" : "+v"(v));
    return (TO)v;
}
// Four outputs at float4 index f of a row: f32, or f16 rounded to nearest
// even (the prefill GEMMs' activations).
__device__ __forceinline__ void store4(float *y, uint32_t f, float4 v) { ((float4 *)y)[f] = v; }
__device__ __forceinline__ void store4(_Float16 *y, uint32_t f, float4 v)
{
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    ((h4 *)y)[f] = h4{to_out<_Float16>(v.x), to_out<_Float16>(v.y), to_out<_Float16>(v.z), to_out<_Float16>(v.w)};
}

// ---------------------------------------------------------------------------
// RMSNorm (phi4.rs:593-599): one 256-thread workgroup per row; the sum of
// squares uses the same fixed-order reduction as the fused GEMV staging, so
// rmsnorm -> gemv and the fused gemv_rmsnorm produce identical bits.  TO =
// _Float16 rounds the same f32 results to f16.
template <typename TO>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *__restrict__ x, const float *__restrict__ g,
                                                      TO *__restrict__ y, uint32_t d, float eps)
{
    __shared__ float red[16];
    const float *xr = x + (uint64_t)blockIdx.x * d;
    TO *yr = y + (uint64_t)blockIdx.x * d;
    const uint32_t t = threadIdx.x;
    if (d % 4 == 0 && d <= 8 * 4 * 256) {
        // the row stays in registers (one pass over x); the thread holds its
        // float4s of the canonical sum-of-squares split
        // x and gamma requested at once (buffer loads; a slot past the row
        // takes an out-of-range offset: no request, zeros), not each under
        // its slot test, which would wait for the one before
        const uint32_t nf = d / 4;
        uint32_t f[8], sl[8];
        sumsq_slots<8>(sumsq_parts(d), f, sl);
        const __amdgpu_buffer_rsrc_t rx = make_rsrc(xr, (uint64_t)d * 4), rg = make_rsrc(g, (uint64_t)d * 4);
        float4 v[8];
        u32x4 gw[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t off = f[j] < nf ? 16 * f[j] : RRR_OOB;
            v[j] = u2f4(bload16_so(rx, off, 0));
            gw[j] = bload16_so(rg, off, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        const float inv = rms_inv(sumsq_held_256<8>(v, f, sl, nf, red), d, eps);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            if (f[j] < nf) {
                const float4 w = u2f4(gw[j]);
                store4(yr, f[j], make_float4(__fmul_rn(__fmul_rn(w.x, v[j].x), inv), __fmul_rn(__fmul_rn(w.y, v[j].y), inv),
                                          __fmul_rn(__fmul_rn(w.z, v[j].z), inv), __fmul_rn(__fmul_rn(w.w, v[j].w), inv)));
            }
        }
        return;
    }
    const float inv = rms_inv(block_sumsq_256(xr, d, red), d, eps);
    for (uint32_t i = t; i < d; i += 256) yr[i] = to_out<TO>(__fmul_rn(__fmul_rn(g[i], xr[i]), inv));
}

hipError_t launch_rmsnorm(const float *x, const float *g, float *y, uint32_t rows, uint32_t d, float eps,
                          hipStream_t s)
{
    hipLaunchKernelGGL(rmsnorm_kernel<float>, dim3(rows), dim3(256), 0, s, x, g, y, d, eps);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_f16(const float *x, const float *g, uint16_t *y, uint32_t rows, uint32_t d, float eps,
                              hipStream_t s)
{
    hipLaunchKernelGGL(rmsnorm_kernel<_Float16>, dim3(rows), dim3(256), 0, s, x, g, (_Float16 *)y, d, eps);
    return hipGetLastError();
}

// The split-K reduction of a GEMM whose output feeds an RMSNorm (the prefill
// layer's O-proj and FFN-down, each adding to the residual rows that the next
// norm reads): one 256-thread workgroup per row m adds the S partials
// ws[k][m][:] in split order, applies the row scale, adds the row of Y when
// `acc`, stores it to Y (what gemm_splitk_reduce stores) and writes the
// row's RMSNorm with gamma in f16, the arithmetic and canonical sum-of-squares
// order of rmsnorm_kernel<_Float16> over the stored row, so both outputs are
// bitwise the two launches'.  d % 4 == 0, d <= 8192.
// SS: the split count (2..8); P = ceil(d / 4096), the slots a thread holds
// being 4 P.  Every slot's partials, residual and gamma are requested at once
// (buffer loads; a slot past the row, or the residual without acc, takes an
// out-of-range offset: no request, zeros), before the first add: a load under
// a branch would make the compiler wait for it at the join, one round trip
// per slot.
template <int SS, int P>
__global__ __launch_bounds__(256) void splitk_reduce_rmsnorm_kernel(const float *__restrict__ ws, uint32_t M,
                                                                    uint32_t d, float *__restrict__ Y,
                                                                    const float *__restrict__ rscale, uint32_t acc,
                                                                    const float *__restrict__ g, float eps,
                                                                    _Float16 *__restrict__ out)
{
    constexpr int NS = 4 * P;
    __shared__ float red[16];
    const uint32_t m = blockIdx.x, nf = d / 4;
    const uint32_t mn4 = M * d * 4;                               // bytes of one split's partials
    float4 *yr = (float4 *)(Y + (uint64_t)m * d);
    const float r = rscale ? rscale[m] : 1.0f;
    uint32_t f[8], sl[8];
    sumsq_slots<8>(P, f, sl);
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(ws, (uint64_t)SS * mn4);
    const __amdgpu_buffer_rsrc_t ry = make_rsrc(Y, (uint64_t)mn4);
    const __amdgpu_buffer_rsrc_t rg = make_rsrc(g, (uint64_t)d * 4);
    u32x4 pw[NS][SS], py[NS], pg[NS];
#pragma unroll
    for (int j = 0; j < NS; j++) {
        const bool ok = f[j] < nf;
        const uint32_t off = ok ? (m * d + 4 * f[j]) * 4 : RRR_OOB;
#pragma unroll
        for (int k = 0; k < SS; k++) pw[j][k] = bload16_so(rw, off, k * mn4);
        py[j] = bload16_so(ry, acc ? off : RRR_OOB, 0);
        pg[j] = bload16_so(rg, ok ? 16 * f[j] : RRR_OOB, 0);
    }
    float4 v[8];
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < NS; j++) {
        if (f[j] < nf) {
            float4 a = u2f4(pw[j][0]);
#pragma unroll
            for (int k = 1; k < SS; k++) {
                const float4 q = u2f4(pw[j][k]);
                a.x += q.x; a.y += q.y; a.z += q.z; a.w += q.w;
            }
            if (rscale) {
                a.x *= r; a.y *= r; a.z *= r; a.w *= r;
            }
            if (acc) {
                const float4 o = u2f4(py[j]);
                a.x = o.x + a.x; a.y = o.y + a.y; a.z = o.z + a.z; a.w = o.w + a.w;
            }
            yr[f[j]] = a;
            v[j] = a;
        }
    }
    const float inv = rms_inv(sumsq_held_256<8>(v, f, sl, nf, red), d, eps);
    _Float16 *orow = out + (uint64_t)m * d;
#pragma unroll
    for (int j = 0; j < NS; j++) {
        if (f[j] < nf) {
            const float4 w = u2f4(pg[j]);
            store4(orow, f[j], make_float4(__fmul_rn(__fmul_rn(w.x, v[j].x), inv), __fmul_rn(__fmul_rn(w.y, v[j].y), inv),
                                           __fmul_rn(__fmul_rn(w.z, v[j].z), inv), __fmul_rn(__fmul_rn(w.w, v[j].w), inv)));
        }
    }
}

bool splitk_reduce_rmsnorm_supported(uint32_t d) { return d % 4 == 0 && d <= 8 * 4 * 256; }

hipError_t launch_splitk_reduce_rmsnorm(const float *ws, uint32_t S, uint32_t M, uint32_t d, float *Y,
                                        const float *rscale, bool acc, const float *g, float eps, uint16_t *out,
                                        hipStream_t s)
{
#define RRR_SRR_CASE(N)                                                                                          \
    case N:                                                                                                       \
        if (d <= 4096)                                                                                            \
            hipLaunchKernelGGL((splitk_reduce_rmsnorm_kernel<N, 1>), dim3(M), dim3(256), 0, s, ws, M, d, Y, rscale, \
                               acc ? 1u : 0u, g, eps, (_Float16 *)out);                                            \
        else                                                                                                      \
            hipLaunchKernelGGL((splitk_reduce_rmsnorm_kernel<N, 2>), dim3(M), dim3(256), 0, s, ws, M, d, Y, rscale, \
                               acc ? 1u : 0u, g, eps, (_Float16 *)out);                                            \
        break;
    switch (S) {
        RRR_SRR_CASE(2) RRR_SRR_CASE(3) RRR_SRR_CASE(4) RRR_SRR_CASE(5)
        RRR_SRR_CASE(6) RRR_SRR_CASE(7) RRR_SRR_CASE(8)
    default: return hipErrorInvalidValue;
    }
#undef RRR_SRR_CASE
    return hipGetLastError();
}

// silu_gate (phi4.rs:1369-1373): rows of [gate(F) | up(F)] -> rows of F (f32,
// or the same values rounded to f16).
template <typename TO>
__global__ __launch_bounds__(256) void silu_gate_kernel(const float *__restrict__ gu, TO *__restrict__ mid,
                                                        uint32_t F, uint64_t total)
{
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const uint64_t r = i / F, c = i - r * F;
    const float *row = gu + r * 2 * F;
    mid[i] = to_out<TO>(silu_f(row[c]) * row[F + c]);
}

hipError_t launch_silu_gate(const float *gu, float *mid, uint32_t rows, uint32_t F, hipStream_t s)
{
    const uint64_t total = (uint64_t)rows * F;
    hipLaunchKernelGGL(silu_gate_kernel<float>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, gu, mid, F,
                       total);
    return hipGetLastError();
}

// silu_gate rows in f16 block floating point: one 256-thread workgroup per
// row computes v = silu(gate) * up (the f32 values of silu_gate_kernel), the
// row's largest |v| = f * 2^e (f in [0.5, 1)), and stores f16(v * 2^(15 - e))
// (the scaling is exact, so the row's largest magnitude lands in [2^14,
// 2^15) and every value keeps f16's 11 significant bits however large the
// activations grow); rscale[row] = 2^(e - 15) undoes it.  A row with no
// finite nonzero maximum is stored unscaled (rscale 1).
// NV > 0: the row's values stay in registers (F <= 256 * NV, one read of
// gate / up); NV == 0: any F, gate / up read twice.  PRE: gu holds the
// values v themselves (rows of F: the gate/up GEMM's silu epilogue).
template <int NV, bool PRE = false>
__global__ __launch_bounds__(256) void silu_gate_f16_rows_kernel(const float *__restrict__ gu,
                                                                 _Float16 *__restrict__ mid,
                                                                 float *__restrict__ rscale, uint32_t F)
{
    __shared__ float red[4];
    const float *row = gu + (uint64_t)blockIdx.x * (PRE ? 1 : 2) * F;
    _Float16 *out = mid + (uint64_t)blockIdx.x * F;
    const uint32_t t = threadIdx.x;
    float m = 0.0f;
    float v[NV > 0 ? NV : 1];
    if constexpr (NV > 0) {
        // thread t holds elements 4 (t + 256 j) .. +3 (F % 4 == 0: 16-byte loads)
#pragma unroll
        for (int j = 0; j < NV / 4; j++) {
            const uint32_t i = 4 * (t + 256u * j);
            float4 g = make_float4(0.f, 0.f, 0.f, 0.f), u = g;
            if constexpr (PRE) {
                if (i < F) g = *(const float4 *)(row + i);
                v[4 * j] = g.x;
                v[4 * j + 1] = g.y;
                v[4 * j + 2] = g.z;
                v[4 * j + 3] = g.w;
            } else {
                if (i < F) {
                    g = *(const float4 *)(row + i);
                    u = *(const float4 *)(row + F + i);
                }
                v[4 * j] = silu_f(g.x) * u.x;
                v[4 * j + 1] = silu_f(g.y) * u.y;
                v[4 * j + 2] = silu_f(g.z) * u.z;
                v[4 * j + 3] = silu_f(g.w) * u.w;
            }
#pragma unroll
            for (int c = 0; c < 4; c++) m = fmaxf(m, fabsf(v[4 * j + c]));
        }
    } else {
        for (uint32_t i = t; i < F; i += 256) m = fmaxf(m, fabsf(PRE ? row[i] : silu_f(row[i]) * row[F + i]));
    }
    m = wave_max(m);
    if ((t & 63) == 0) red[t >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int e = 15;
    if (m > 0.0f && __builtin_isfinite(m)) (void)frexpf(m, &e);
    const float sc = ldexpf(1.0f, 15 - e);
    if constexpr (NV > 0) {
        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int j = 0; j < NV / 4; j++) {
            const uint32_t i = 4 * (t + 256u * j);
            if (i < F)
                *(h4 *)(out + i) = h4{to_out<_Float16>(v[4 * j] * sc), to_out<_Float16>(v[4 * j + 1] * sc),
                                      to_out<_Float16>(v[4 * j + 2] * sc), to_out<_Float16>(v[4 * j + 3] * sc)};
        }
    } else {
        for (uint32_t i = t; i < F; i += 256) out[i] = to_out<_Float16>((PRE ? row[i] : silu_f(row[i]) * row[F + i]) * sc);
    }
    if (t == 0) rscale[blockIdx.x] = ldexpf(1.0f, e - 15);
}

hipError_t launch_silu_gate_f16(const float *gu, uint16_t *mid, float *rscale, uint32_t rows, uint32_t F,
                                hipStream_t s)
{
    if (F <= 256 * 32 && F % 4 == 0)
        hipLaunchKernelGGL(silu_gate_f16_rows_kernel<32>, dim3(rows), dim3(256), 0, s, gu, (_Float16 *)mid, rscale, F);
    else
        hipLaunchKernelGGL(silu_gate_f16_rows_kernel<0>, dim3(rows), dim3(256), 0, s, gu, (_Float16 *)mid, rscale, F);
    return hipGetLastError();
}

// The same rows from precomputed values v (rows of F floats).
hipError_t launch_f16_rows_scaled(const float *v, uint16_t *mid, float *rscale, uint32_t rows, uint32_t F,
                                  hipStream_t s)
{
    if (F <= 256 * 32 && F % 4 == 0)
        hipLaunchKernelGGL((silu_gate_f16_rows_kernel<32, true>), dim3(rows), dim3(256), 0, s, v, (_Float16 *)mid,
                           rscale, F);
    else
        hipLaunchKernelGGL((silu_gate_f16_rows_kernel<0, true>), dim3(rows), dim3(256), 0, s, v, (_Float16 *)mid,
                           rscale, F);
    return hipGetLastError();
}

// residual_add (phi4.rs:608-610); out may alias a.
__global__ __launch_bounds__(256) void residual_add_kernel(const float *a, const float *b, float *out, uint32_t n)
{
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = a[i] + b[i];
}

hipError_t launch_residual_add(const float *a, const float *b, float *out, uint32_t n, hipStream_t s)
{
    hipLaunchKernelGGL(residual_add_kernel, dim3((n + 255) / 256), dim3(256), 0, s, a, b, out, n);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void fill_u32_kernel(uint32_t *p, uint64_t n, uint32_t v)
{
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256) p[i] = v;
}

hipError_t launch_fill_u32(uint32_t *p, uint64_t n, uint32_t v, hipStream_t s)
{
    uint64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)blocks), dim3(256), 0, s, p, n, v);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Logits over the reference's transposed chunks (phi4.rs:874-893):
// chunk c holds n_c = min(chunk, V - c*chunk) vocab rows as B_c[d*n_c + v].
// A workgroup owns 64 consecutive vocab entries of one chunk, so the ~3,100
// workgroups of the 200,064-entry vocabulary spread evenly over the CUs
// (with 256 entries, 782 workgroups left 14 CUs a fourth 3 MB workgroup at
// the end).  Wave w sums d in [w*K/4, (w+1)*K/4) as four interleaved row
// streams (a lane: 4 entries of every 4th row, one 16-byte load per row), the
// streams are added by a fixed butterfly and the waves in order through LDS.
// The activation (optionally RMS-normalised in place) sits in LDS.
__global__ __launch_bounds__(256) void logits_chunked_kernel(const float *__restrict__ x, const float *__restrict__ gamma,
                                                             float eps, const float *__restrict__ E,
                                                             float *__restrict__ y, uint32_t K, uint32_t V,
                                                             uint32_t chunk)
{
    extern __shared__ float sm[];
    float *xs = sm;             // K
    float *part = xs + K;       // 4 waves x 64 entries
    float *red = part + 256;    // 16
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    float inv = 1.0f;
    if (gamma) inv = rms_inv(block_sumsq_256(x, K, red), K, eps);
    for (uint32_t i = t; i < K; i += 256) xs[i] = gamma ? __fmul_rn(__fmul_rn(gamma[i], x[i]), inv) : x[i];
    __syncthreads();

    // 64 vocab entries per workgroup (chunks are multiples of 64 entries when
    // there are several): lane (q, g) = (lane % 16, lane / 16) reads entries
    // 4q .. 4q+3 of the rows d = d0 + 4i + g of its wave's quarter of K
    const uint32_t v0 = blockIdx.x * 64;
    const uint32_t c = v0 / chunk, cstart = c * chunk;
    const uint32_t n = (V - cstart) < chunk ? (V - cstart) : chunk;
    const uint32_t q = lane & 15, g = lane >> 4;
    const uint32_t vin = v0 - cstart + 4 * q;     // index inside the chunk
    const uint64_t cbase = (uint64_t)cstart * K;  // chunk c starts after c full chunks
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(E + cbase, (uint64_t)n * K * 4);
    const uint32_t dq = K / 4, d0 = wave * dq;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    if (vin < n) {
        const uint32_t step = 4 * n * 4;          // 4 rows
        uint32_t off = ((d0 + g) * n + vin) * 4;
        uint32_t dd = 0;
        for (; dd + 32 <= dq; dd += 32) {
            u32x4 w[8];
#pragma unroll
            for (int u = 0; u < 8; u++) w[u] = bload16_nt(rs, off + u * step);
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const float xv = xs[d0 + dd + 4 * u + g];
                a0 = fmaf(xv, u2f(w[u].x), a0);
                a1 = fmaf(xv, u2f(w[u].y), a1);
                a2 = fmaf(xv, u2f(w[u].z), a2);
                a3 = fmaf(xv, u2f(w[u].w), a3);
            }
            off += 8 * step;
        }
        for (; dd + g < dq; dd += 4) {
            const u32x4 w = bload16_nt(rs, off);
            const float xv = xs[d0 + dd + g];
            a0 = fmaf(xv, u2f(w.x), a0);
            a1 = fmaf(xv, u2f(w.y), a1);
            a2 = fmaf(xv, u2f(w.z), a2);
            a3 = fmaf(xv, u2f(w.w), a3);
            off += step;
        }
    }
    // the 4 row streams of a wave (lanes q, q+16, q+32, q+48), then the waves
    // in order
    a0 = a0 + __shfl_xor(a0, 16, 64); a0 = a0 + __shfl_xor(a0, 32, 64);
    a1 = a1 + __shfl_xor(a1, 16, 64); a1 = a1 + __shfl_xor(a1, 32, 64);
    a2 = a2 + __shfl_xor(a2, 16, 64); a2 = a2 + __shfl_xor(a2, 32, 64);
    a3 = a3 + __shfl_xor(a3, 16, 64); a3 = a3 + __shfl_xor(a3, 32, 64);
    if (g == 0) ((float4 *)part)[wave * 16 + q] = make_float4(a0, a1, a2, a3);
    __syncthreads();
    if (t < 64 && v0 - cstart + t < n) {
        const float r = ((part[t] + part[64 + t]) + part[128 + t]) + part[192 + t];
        y[cstart + (v0 - cstart) + t] = r;
    }
}

hipError_t launch_logits_chunked(const float *x, const float *gamma, float eps, const float *E, float *y,
                                 uint32_t K, uint32_t V, uint32_t chunk, hipStream_t s)
{
    const size_t lds = ((size_t)K + 256 + 16) * sizeof(float);
    // 64-entry groups of each chunk (a partial last chunk may leave a
    // partial group)
    uint32_t nwg = 0;
    for (uint32_t c0 = 0; c0 < V; c0 += chunk) nwg += ((V - c0 < chunk ? V - c0 : chunk) + 63) / 64;
    hipLaunchKernelGGL(logits_chunked_kernel, dim3(nwg), dim3(256), lds, s, x, gamma, eps, E, y, K, V, chunk);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Argmax with the semantics of the sequential loop at phi4.rs:1172-1183:
// start from (value -inf, index 0), replace only on strictly greater, so the
// first maximal index wins and NaN never wins.  Pass 1: one candidate per
// workgroup; pass 2: one workgroup reduces the candidates in index order.
struct Cand { float v; uint32_t i; };

__device__ __forceinline__ Cand better(Cand a, Cand b)
{
    // a precedes b in index order whenever both are live candidates
    if (b.v > a.v || (b.v == a.v && b.i < a.i)) return b;
    return a;
}

__device__ __forceinline__ Cand wave_best(Cand c)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        Cand d;
        d.v = __shfl_xor(c.v, o, 64);
        d.i = __shfl_xor(c.i, o, 64);
        c = better(c, d);
    }
    return c;
}

__device__ Cand block_best(Cand c, Cand *sm)
{
    c = wave_best(c);
    if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = c;
    __syncthreads();
    Cand r = sm[0];
    for (int w = 1; w < 4; w++) r = better(r, sm[w]);
    return r;
}

// Split-K form of the transposed-chunk logits.  Workgroup (slab, h) takes
// the 256 vocab entries of one slab of a chunk and rows [h*K/NS, (h+1)*K/NS)
// of the chunk's [d][n] matrix, i.e. row pieces of 1 KB: lane l of a wave
// reads entries 4l .. 4l+3 of one row per load, so each load instruction is
// 1 KB of whole cache lines, and the 8 d-ranges make 6,256 workgroups of
// 384 KB for the 200,064 x 3072 logits (balanced over the CUs).  Wave w
// takes the rows w, w+4, ... of the range (U loads in flight), the waves'
// sums are added in wave order, and the NS partial sums of an entry are
// written through to the coherent level; the last workgroup of the slab to
// arrive (an agent-scope counter, reset by that workgroup for the next call)
// adds them in order h = 0, 1, ..., NS-1 and writes the logits.
// AM: that workgroup also reduces its 256 logits to the slab's (max, first
// index), writes it through to the coherent level and counts on one more
// counter; the last slab to arrive reduces the slabs' candidates in index
// order (the argmax rule above) and writes the token.
constexpr uint32_t LOGITS_SPLITS = 8, LOGITS_SLAB = 256, LOGITS_COUNTER_STRIDE = 64, LOGITS_U = 8;
// scalar+vector offset past every chunk byte (a chunk is below 2 GiB on this
// path): such loads return zeros and move no data
constexpr uint32_t MQ_OOB_LOGITS = 0x80000000u;

template <int U, bool AM>
__global__ __launch_bounds__(256) void logits_split_kernel(const float *__restrict__ x, const float *__restrict__ gamma,
                                                           float eps, const float *__restrict__ E, float *__restrict__ y,
                                                           uint32_t K, uint32_t V, uint32_t chunk, float *part,
                                                           uint32_t *counters, Cand *cand, uint32_t *token)
{
    constexpr uint32_t NS = LOGITS_SPLITS;
    extern __shared__ float sm[];
    const uint32_t Dr = K / NS;
    float *xs = sm;                 // Dr
    float *wsum = xs + Dr;          // 4 waves x 256 entries
    float *red = wsum + 4 * 256;    // 16
    __shared__ uint32_t last;
    __shared__ Cand amsm[4];
    // wave-uniform: the weight loads' scalar offsets derive from it (else each
    // load is wrapped in a readfirstlane loop)
    const uint32_t t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t sb = blockIdx.x / NS, h = blockIdx.x % NS;
    const uint32_t spc = chunk / LOGITS_SLAB;                 // slabs per full chunk
    const uint32_t c = sb / spc, j = sb - c * spc;
    const uint32_t cstart = c * chunk;
    const uint32_t n = (V - cstart) < chunk ? (V - cstart) : chunk;
    const uint32_t d0 = h * Dr;

    const uint32_t vin = j * LOGITS_SLAB + 4 * lane;          // entry inside the chunk
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(E + (uint64_t)cstart * K, (uint64_t)n * K * 4);
    const uint32_t voff = vin < n ? 4 * vin : MQ_OOB_LOGITS;
    const uint32_t rstep = 4 * n * 4;                          // 4 rows
    uint32_t soff = (d0 + wave) * n * 4;
    const uint32_t nr = Dr / 4;                                // rows of this wave (a multiple of U)
    // the first U rows are requested before the RMSNorm prologue, which then
    // runs while they are in flight
    u32x4 w[U];
#pragma unroll
    for (int u = 0; u < U; u++) w[u] = bload16_nt_so(rs, voff, soff + u * rstep);
    soff += U * rstep;

    float inv = 1.0f;
    if (gamma) inv = rms_inv(block_sumsq_256(x, K, red), K, eps);
    for (uint32_t i = t; i < Dr; i += 256) xs[i] = gamma ? __fmul_rn(__fmul_rn(gamma[d0 + i], x[d0 + i]), inv) : x[d0 + i];
    __syncthreads();

    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    for (uint32_t r = 0; r < nr; r += U) {
        u32x4 wn[U];
        const bool more = r + U < nr;
#pragma unroll
        for (int u = 0; u < U; u++) wn[u] = bload16_nt_so(rs, more ? voff : MQ_OOB_LOGITS, soff + u * rstep);
        soff += U * rstep;
#pragma unroll
        for (int u = 0; u < U; u++) {
            const float xv = xs[wave + 4 * (r + u)];
            a0 = fmaf(xv, u2f(w[u].x), a0);
            a1 = fmaf(xv, u2f(w[u].y), a1);
            a2 = fmaf(xv, u2f(w[u].z), a2);
            a3 = fmaf(xv, u2f(w[u].w), a3);
        }
#pragma unroll
        for (int u = 0; u < U; u++) w[u] = wn[u];
    }
    ((float4 *)wsum)[wave * 64 + lane] = make_float4(a0, a1, a2, a3);
    __syncthreads();
    const float p = ((wsum[t] + wsum[256 + t]) + wsum[512 + t]) + wsum[768 + t];
    const uint32_t v = cstart + j * LOGITS_SLAB + t;          // this thread's entry
    const bool live = j * LOGITS_SLAB + t < n;
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(part, (uint64_t)NS * V * 4);
    if (live) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(p), rp, 4 * (h * V + v), 0, RRR_CPOL_SC1);
    // publish: this workgroup's partials are at the coherent level, then count
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (t == 0)
        last = __hip_atomic_fetch_add(counters + sb * LOGITS_COUNTER_STRIDE, 1u, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == NS - 1;
    __syncthreads();
    if (!last) return;
    float r = -__builtin_inff();
    if (live) {
        float q[NS];
#pragma unroll
        for (uint32_t k = 0; k < NS; k++)
            q[k] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rp, 4 * (k * V + v), 0, RRR_CPOL_SC1));
        r = q[0];
#pragma unroll
        for (uint32_t k = 1; k < NS; k++) r = r + q[k];
        y[v] = r;
    }
    if (t == 0) __hip_atomic_store(counters + sb * LOGITS_COUNTER_STRIDE, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if constexpr (AM) {
        const uint32_t slabs = gridDim.x / NS;
        const __amdgpu_buffer_rsrc_t rc = make_rsrc(cand, (uint64_t)slabs * sizeof(Cand));
        Cand c = {-__builtin_inff(), 0u};
        if (live && r > c.v) c = Cand{r, v};   // NaN and -inf never win
        c = block_best(c, amsm);
        if (t == 0) {
            __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(c.v), c.i}, rc, 8 * sb, 0, RRR_CPOL_SC1);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            last = __hip_atomic_fetch_add(counters + LOGITS_MAX_SLABS * LOGITS_COUNTER_STRIDE, 1u, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT) == slabs - 1;
        }
        __syncthreads();
        if (!last) return;
        Cand b = {-__builtin_inff(), 0u};
        for (uint32_t i = t; i < slabs; i += 256) {
            const u32x2 u = __builtin_amdgcn_raw_buffer_load_b64(rc, 8 * i, 0, RRR_CPOL_SC1);
            b = better(b, Cand{__uint_as_float(u.x), u.y});
        }
        b = block_best(b, amsm);
        if (t == 0) {
            token[0] = b.i;
            __hip_atomic_store(counters + LOGITS_MAX_SLABS * LOGITS_COUNTER_STRIDE, 0u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// one counter line per slab, then the argmax counter's line
uint64_t logits_counter_bytes() { return (uint64_t)(LOGITS_MAX_SLABS + 1) * LOGITS_COUNTER_STRIDE * 4; }

// the slab candidates follow the split partials in the workspace
static uint64_t logits_cand_offset(uint32_t V) { return ((uint64_t)LOGITS_SPLITS * V * 4 + 255) & ~255ull; }

bool logits_split_supported(uint32_t K, uint32_t V, uint32_t chunk, uint64_t ws_bytes)
{
    if (K % (4 * LOGITS_SPLITS * LOGITS_U) || K > 12288 || chunk % LOGITS_SLAB) return false;
    if ((uint64_t)(chunk < V ? chunk : V) * K * 4 >= MQ_OOB_LOGITS) return false;
    uint64_t slabs = 0;
    for (uint64_t c0 = 0; c0 < V; c0 += chunk) slabs += ((V - c0 < chunk ? V - c0 : chunk) + LOGITS_SLAB - 1) / LOGITS_SLAB;
    return slabs <= LOGITS_MAX_SLABS && logits_cand_offset(V) + slabs * sizeof(Cand) <= ws_bytes;
}

hipError_t launch_logits_split(const float *x, const float *gamma, float eps, const float *E, float *y, uint32_t K,
                               uint32_t V, uint32_t chunk, float *part, uint32_t *counters, uint32_t *token,
                               hipStream_t s)
{
    uint32_t slabs = 0;
    for (uint32_t c0 = 0; c0 < V; c0 += chunk) slabs += ((V - c0 < chunk ? V - c0 : chunk) + LOGITS_SLAB - 1) / LOGITS_SLAB;
    const size_t lds = ((size_t)K / LOGITS_SPLITS + 4 * 256 + 16) * sizeof(float);
    Cand *cand = (Cand *)((uint8_t *)part + logits_cand_offset(V));
    if (token)
        hipLaunchKernelGGL((logits_split_kernel<LOGITS_U, true>), dim3(slabs * LOGITS_SPLITS), dim3(256), lds, s, x, gamma,
                           eps, E, y, K, V, chunk, part, counters, cand, token);
    else
        hipLaunchKernelGGL((logits_split_kernel<LOGITS_U, false>), dim3(slabs * LOGITS_SPLITS), dim3(256), lds, s, x,
                           gamma, eps, E, y, K, V, chunk, part, counters, cand, token);
    return hipGetLastError();
}

constexpr uint32_t ARGMAX_WG = 1024;

__global__ __launch_bounds__(256) void argmax_pass1(const float *__restrict__ v, uint32_t n, Cand *part)
{
    __shared__ Cand sm[4];
    Cand c = {-__builtin_inff(), 0u};
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
        const float x = v[i];
        if (x > c.v) { c.v = x; c.i = i; }
    }
    c = block_best(c, sm);
    if (threadIdx.x == 0) part[blockIdx.x] = c;
}

__global__ __launch_bounds__(256) void argmax_pass2(const Cand *part, uint32_t np, uint32_t *out)
{
    __shared__ Cand sm[4];
    Cand c = {-__builtin_inff(), 0u};
    for (uint32_t i = threadIdx.x; i < np; i += 256) c = better(c, part[i]);
    c = block_best(c, sm);
    if (threadIdx.x == 0) out[0] = c.i;
}

uint64_t argmax_partials_bytes() { return ARGMAX_WG * sizeof(Cand); }

hipError_t launch_argmax(const float *v, uint32_t n, void *partials, uint32_t *out, hipStream_t s)
{
    uint32_t wg = (n + 255) / 256;
    if (wg > ARGMAX_WG) wg = ARGMAX_WG;
    if (wg == 0) wg = 1;
    hipLaunchKernelGGL(argmax_pass1, dim3(wg), dim3(256), 0, s, v, n, (Cand *)partials);
    hipLaunchKernelGGL(argmax_pass2, dim3(1), dim3(256), 0, s, (const Cand *)partials, wg, out);
    return hipGetLastError();
}

}  // namespace rrr
