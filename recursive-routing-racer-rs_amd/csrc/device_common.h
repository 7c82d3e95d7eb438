// device_common.h -- gfx950 device helpers shared by the decode-path kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef char i8x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define RRR_WAVE 64

// Buffer resource descriptor (V#) for raw byte addressing on gfx9: stride 0,
// num_records = bytes, DST_SEL/format word 0x00020000.  Loads past
// num_records return zero instead of faulting, which bounds every weight read
// to the tensor the caller passed.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint64_t bytes)
{
    uint32_t n = bytes > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)n, 0x00020000);
}

// 16-byte load at any byte offset (the hardware runs in unaligned-access mode
// under ROCm, so Q6_K's 2-byte-aligned 210-byte blocks need no realignment).
__device__ __forceinline__ u32x4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
// Streaming (non-temporal) variant for data read exactly once, such as
// weight matrices: keeps activations and outputs resident in the caches.
constexpr int RRR_CPOL_NT = 2;
// agent-scope coherent access (sc1): goes through to the level shared by
// every XCD, for data exchanged between workgroups of one launch
constexpr int RRR_CPOL_SC1 = 16;
__device__ __forceinline__ u32x4 bload16_nt(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, RRR_CPOL_NT);
}
// ... with a wave-uniform part of the offset in the scalar offset operand
__device__ __forceinline__ u32x4 bload16_nt_so(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff)
{
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, RRR_CPOL_NT);
}
// ... plain policy, with a wave-uniform part of the offset in the scalar operand
__device__ __forceinline__ u32x4 bload16_so(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff)
{
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
}
// An offset past every buffer a kernel addresses this way (each below 2 GB):
// a buffer load there moves no data and returns zeros, so a load can be
// issued unconditionally instead of under a branch.
constexpr uint32_t RRR_OOB = 0x80000000u;
__device__ __forceinline__ float4 u2f4(const u32x4 &v)
{
    return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}
__device__ __forceinline__ uint32_t bload4(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t bload2(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

// 16-byte LDS DMA load: lane l's 16 bytes at `voff + soff` go to LDS
// dst + 16 l (dst wave-uniform; out-of-range lanes write zeros).  Only the
// device pass sees the builtin (the host pass would otherwise drop the
// kernels' launch stubs).
template <int CPOL>
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t rs, void *dst, uint32_t voff, uint32_t soff)
{
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)dst, 16, voff, soff, 0,
                                             CPOL);
#endif
}

// Wait until at most N vector memory operations of this wave are in flight
// (they retire in order).  The compiler does not track LDS DMA, so LDS reads
// of DMA-written data wait here (and, for other waves, behind a barrier
// after it); the memory clobber keeps them after the wait.
template <int N>
__device__ __forceinline__ void wait_vm()
{
    static_assert(N >= 0 && N < 64, "vmcnt");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier that waits for this wave's LDS (and scalar) operations
// only.  __syncthreads' release fence also waits for every vector memory
// operation once LDS DMA is in flight, which would wait out DMA issued for a
// later step; the memory clobber keeps the compiler's memory accesses on
// their side of the barrier.
__device__ __forceinline__ void barrier_lds()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// IEEE binary16 -> binary32 (exact; v_cvt_f32_f16).
__device__ __forceinline__ float h2f(uint32_t bits16)
{
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(bits16 & 0xFFFFu));
}

// u32 bits -> f32.  Take the argument by value: applying __builtin_bit_cast
// directly to an ext-vector swizzle such as v.y reads element 0 instead.
__device__ __forceinline__ float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

__device__ __forceinline__ uint32_t byte_of(uint32_t w, uint32_t i) { return (w >> (8u * i)) & 0xFFu; }

// 6-bit scale/min pair j (0..7) from the 12 packed bytes held in three
// little-endian dwords (bytes 4..15 of a Q4_K/Q5_K block).  Restates the
// get_scale_min step of phi4.rs:492-498.
__device__ __forceinline__ void scale_min_k4(uint32_t j, uint32_t s0, uint32_t s1, uint32_t s2,
                                             uint32_t &sc, uint32_t &mn)
{
    // q[i] for i in 0..11 is byte (i & 3) of dword s[i >> 2].  With i = j % 4
    // and h = j / 4, q0 = q[i], q4 = q[4 + i], q8 = q[8 + i]:
    //   h = 0: sc = q0 & 63,                     mn = q4 & 63
    //   h = 1: sc = (q8 & 15) | (q0 >> 6) << 4,  mn = (q8 >> 4) | (q4 >> 6) << 4
    // Both cases are a 4-bit and a 2-bit field of u = q8 | q0 << 8 (sc) or
    // v = q8 | q4 << 8 (mn) at offsets that depend on h only:
    //   sc = u[8 - 8h .. +3] | u[12 + 2h .. +1] << 4
    //   mn = v[8 - 4h .. +3] | v[12 + 2h .. +1] << 4
    // so there is no select (which the compiler turns into branches around
    // the header loads when j is the same on every lane).
    const uint32_t i = j & 3u, h = (j >> 2) & 1u;
    const uint32_t q0 = byte_of(s0, i), q4 = byte_of(s1, i), q8 = byte_of(s2, i);
    const uint32_t u = q8 | (q0 << 8), v = q8 | (q4 << 8);
    sc = ((u >> (8u - 8u * h)) & 15u) | (((u >> (12u + 2u * h)) & 3u) << 4);
    mn = ((v >> (8u - 4u * h)) & 15u) | (((v >> (12u + 2u * h)) & 3u) << 4);
}

// The 6-bit scales (sc) and mins (mn) of sub-blocks 0..3 (index 0) and 4..7
// (index 1) as the four bytes of a dword each, from the 12 packed bytes in y,
// z, w (bytes 4..15 of a Q4_K / Q5_K block): the get_scale_min step of
// phi4.rs:492-498 for every j at once.  j < 4: sc = q[j] & 63, mn = q[j+4] &
// 63; j >= 4: sc = (q[j+4] & 15) | (q[j-4] >> 6) << 4, mn = (q[j+4] >> 4) |
// (q[j] >> 6) << 4.  The shifts by 2 move bits 6..7 of each byte to bits 4..5;
// the 0x30 mask drops what the next byte shifts in.
__device__ __forceinline__ void scale_min_bytes_k4(uint32_t y, uint32_t z, uint32_t w, uint32_t (&sc)[2],
                                                   uint32_t (&mn)[2])
{
    sc[0] = y & 0x3F3F3F3Fu;
    mn[0] = z & 0x3F3F3F3Fu;
    sc[1] = (w & 0x0F0F0F0Fu) | ((y >> 2) & 0x30303030u);
    mn[1] = ((w >> 4) & 0x0F0F0F0Fu) | ((z >> 2) & 0x30303030u);
}

// Scale / min pairs of sub-blocks 2g and 2g + 1 (g = 0..3) from the packed
// bytes: the four 6-bit scales (mins) of sub-blocks 0..3 are the bytes of
// y & 0x3F3F3F3F (z & ...), those of 4..7 the low nibbles of w (its high
// nibbles) with bits 6..7 of the bytes of y (z) on top.
__device__ __forceinline__ void scale_min_pair_k4(uint32_t g, uint32_t y, uint32_t z, uint32_t w, uint32_t &s0,
                                                  uint32_t &m0, uint32_t &s1, uint32_t &m1)
{
    const uint32_t scw = g < 2 ? y & 0x3F3F3F3Fu : (w & 0x0F0F0F0Fu) | ((y >> 2) & 0x30303030u);
    const uint32_t mnw = g < 2 ? z & 0x3F3F3F3Fu : ((w >> 4) & 0x0F0F0F0Fu) | ((z >> 2) & 0x30303030u);
    const uint32_t sh = 16u * (g & 1u);
    s0 = (scw >> sh) & 0xFFu;
    s1 = (scw >> (sh + 8u)) & 0xFFu;
    m0 = (mnw >> sh) & 0xFFu;
    m1 = (mnw >> (sh + 8u)) & 0xFFu;
}

// The values of v in lane (lane & ~X) and in lane (lane | X), X = 16 or 32,
// by the gfx950 lane swaps (VALU, no LDS round trip): v_permlane16_swap
// exchanges the odd 16-lane rows of its first operand with the even rows of
// its second, v_permlane32_swap the upper half of the first with the lower
// half of the second, so with both operands v the results are v of the
// lower and of the upper partner.
template <int X>
__device__ __forceinline__ void lane_pair(float v, float &lo, float &hi)
{
    const uint32_t u = __float_as_uint(v);
    if constexpr (X == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        lo = __uint_as_float(r[0]);
        hi = __uint_as_float(r[1]);
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        lo = __uint_as_float(r[0]);
        hi = __uint_as_float(r[1]);
    }
}

// Maximum / sum of v over the lanes l, l ^ 16, l ^ 32, l ^ 48 by the lane
// swaps (VALU, no LDS round trip); every lane of the four gets the same
// value, and the sum is the one the xor-16 then xor-32 butterfly gives.
__device__ __forceinline__ float lanes4_max(float v)
{
    float a, b;
    lane_pair<16>(v, a, b);
    lane_pair<32>(fmaxf(a, b), a, b);
    return fmaxf(a, b);
}
__device__ __forceinline__ float lanes4_sum(float v)
{
    float a, b;
    lane_pair<16>(v, a, b);
    lane_pair<32>(a + b, a, b);
    return a + b;
}

// Sum of the n <= NMAX values p[0], p[stride], ..., p[(n - 1) stride] (LDS)
// in index order, every one requested before the first add (one LDS wait
// instead of one per value); n >= 1.
template <int NMAX>
__device__ __forceinline__ float ordered_sum(const float *p, uint32_t n, uint32_t stride)
{
    float q[NMAX];
#pragma unroll
    for (uint32_t k = 0; k < NMAX; k++) q[k] = p[stride * min(k, n - 1)];
    float v = q[0];
#pragma unroll
    for (uint32_t k = 1; k < NMAX; k++) v = k < n ? v + q[k] : v;
    return v;
}

// Deterministic full-wave sum: the xor butterfly over lane distances 32, 16,
// 8, 4, 2, 1 in that order (each step adds a lane's value and its partner's,
// so every lane ends with the same bits), entirely in VALU: the 32 and 16
// steps by the gfx950 lane swaps, 8 by a row rotation, 4 by two row shifts
// each writing the banks (groups of 4 lanes) whose partner it reaches, 2 and
// 1 by quad permutes.  No LDS round trip.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_sum(float v)
{
    float a, b;
    lane_pair<32>(v, a, b);
    v = a + b;
    lane_pair<16>(v, a, b);
    v = a + b;
    v = v + dpp_f<0x128>(v);                                             // row_ror:8 = lane ^ 8
    const int u = __float_as_int(v);
    int p = __builtin_amdgcn_update_dpp(u, u, 0x104, 0xF, 0x5, false);   // row_shl:4 on lanes with bit 2 clear
    p = __builtin_amdgcn_update_dpp(p, u, 0x114, 0xF, 0xA, false);       // row_shr:4 on lanes with bit 2 set
    v = v + __int_as_float(p);
    v = v + dpp_f<0x4E>(v);                                              // quad_perm [2,3,0,1] = lane ^ 2
    v = v + dpp_f<0xB1>(v);                                              // quad_perm [1,0,3,2] = lane ^ 1
    return v;
}

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, RRR_WAVE));
    return v;
}

// Workgroup (256 threads) sum of per-thread partials: a fixed wave butterfly,
// then waves 0..3 in order.  `red` is 4 floats of LDS.  Every thread returns
// the same value.
__device__ __forceinline__ float block_sum_256(float acc, float *red)
{
    acc = wave_sum(acc);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    const float s = ((red[0] + red[1]) + red[2]) + red[3];
    __syncthreads();
    return s;
}

// Same for a workgroup of W waves (waves summed in order).  `red` holds W floats.
template <int W>
__device__ __forceinline__ float block_sum_w(float acc, float *red)
{
    acc = wave_sum(acc);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    float s = red[0];
#pragma unroll
    for (int w = 1; w < W; w++) s = s + red[w];
    __syncthreads();
    return s;
}

// Canonical sum-of-squares order shared by every RMSNorm on the path
// (standalone and fused), so that they agree bit for bit.  It is the
// activation split of the batch-1 MFMA GEMV, whose waves then square the x
// they already hold.  For d % 4 == 0 the float4s of the vector fall into at
// most 16 slices of 64 P float4s, P = ceil(d / 4096); lane l of slice s
// accumulates x^2 with fmaf over the float4s 64 P s + l + 64 j (j < P, those
// below d / 4), component by component; the 64 lane sums of a slice are added
// by the wave butterfly, and the slice sums in slice order 0, 1, ..., 15
// (slices past the end add +0, which changes no sum).  For d % 4 != 0 thread
// t of a 256-thread workgroup accumulates the elements t, t + 256, ..., and
// the four wave butterflies are added in wave order.
__device__ __forceinline__ uint32_t sumsq_parts(uint32_t d) { return (d + 4095) / 4096; }

// A 256-thread workgroup takes the slices wave, wave + 4, wave + 8, wave + 12
// in each wave.  The k-th of the NV float4s a thread holds is part k % P of
// slice wave + 4 (k / P): f[k] is its float4 index in the vector, sl[k] =
// k / P (counted, not divided).  Every float4 of a vector of d <= NV * 1024
// elements is held by some thread.
template <int NV>
__device__ __forceinline__ void sumsq_slots(uint32_t P, uint32_t (&f)[NV], uint32_t (&sl)[NV])
{
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t i = 0, j = 0;
#pragma unroll
    for (int k = 0; k < NV; k++) {
        sl[k] = i;
        f[k] = 64 * P * (wave + 4 * i) + lane + 64 * j;
        if (++j == P) {
            j = 0;
            ++i;
        }
    }
}

__device__ __forceinline__ float sumsq4(const float4 &v, float acc)
{
    acc = __builtin_fmaf(v.x, v.x, acc);
    acc = __builtin_fmaf(v.y, v.y, acc);
    acc = __builtin_fmaf(v.z, v.z, acc);
    acc = __builtin_fmaf(v.w, v.w, acc);
    return acc;
}

// The total of a 256-thread workgroup's slice sums: sq[i] of wave w is the
// (wave-summed) slice w + 4 i.  `red` is 16 floats of LDS.  Every thread
// returns the same value.
__device__ __forceinline__ float slices_total_256(const float (&sq)[4], float *red)
{
    const uint32_t wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
        for (int i = 0; i < 4; i++) red[wave + 4 * i] = sq[i];
    }
    __syncthreads();
    float s = red[0];
#pragma unroll
    for (int w = 1; w < 16; w++) s = s + red[w];
    __syncthreads();
    return s;
}

// Canonical sum of squares from the float4s a thread of a 256-thread
// workgroup holds, v[k] = float4 f[k] of the vector (sumsq_slots; those at or
// past nf = d / 4 are not used).
template <int NV>
__device__ __forceinline__ float sumsq_held_256(const float4 *v, const uint32_t (&f)[NV], const uint32_t (&sl)[NV],
                                                uint32_t nf, float *red)
{
    float sq[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < NV; k++)
            if (sl[k] == (uint32_t)i && f[k] < nf) acc = sumsq4(v[k], acc);
        sq[i] = wave_sum(acc);
    }
    return slices_total_256(sq, red);
}

// Canonical sum of squares of x[0..d) by a 256-thread workgroup, read from
// memory.  `red` is 16 floats of LDS.
// The canonical sum of squares of block_sumsq_256 in two halves, for
// d % 4 == 0 and d <= 4096 (one float4 per slice and thread): the loads, all
// issued at once and unconditionally (clamped addresses; past d the value is
// not used), then the sums.  A load under a branch makes the compiler wait
// for every load in flight at the join -- also for loads issued before the
// call, such as a weight stream -- and it serialises the x loads.
struct SumsqX {
    float4 v[4];
};
__device__ __forceinline__ SumsqX sumsq_load_256(const float *__restrict__ x, uint32_t d)
{
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nf = d / 4;
    const float4 *p = (const float4 *)x;
    SumsqX r;
#pragma unroll
    for (int i = 0; i < 4; i++) r.v[i] = p[min(64 * (wave + 4 * i) + lane, nf - 1)];
    return r;
}
__device__ __forceinline__ float sumsq_finish_256(const SumsqX &xv, uint32_t d, float *red)
{
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nf = d / 4;
    float sq[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float acc = 64 * (wave + 4 * i) + lane < nf ? sumsq4(xv.v[i], 0.0f) : 0.0f;
        sq[i] = wave_sum(acc);
    }
    return slices_total_256(sq, red);
}

__device__ __forceinline__ float block_sumsq_256(const float *__restrict__ x, uint32_t d, float *red)
{
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    if (d % 4 == 0 && d > 0 && d <= 4096) return sumsq_finish_256(sumsq_load_256(x, d), d, red);
    if (d % 4 != 0) {
        float acc = 0.0f;
        for (uint32_t i = t; i < d; i += 256) acc = __builtin_fmaf(x[i], x[i], acc);
        return block_sum_256(acc, red);
    }
    const uint32_t nf = d / 4, P = sumsq_parts(d);
    const float4 *p = (const float4 *)x;
    float sq[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float acc = 0.0f;
        const uint32_t f0 = 64 * P * (wave + 4 * i) + lane;
        for (uint32_t j = 0; j < P; j++)
            if (f0 + 64 * j < nf) acc = sumsq4(p[f0 + 64 * j], acc);
        sq[i] = wave_sum(acc);
    }
    return slices_total_256(sq, red);
}

// 1 / sqrt(sumsq / d + eps) with correctly rounded divide and square root,
// the evaluation order of rms_norm (phi4.rs:596).
__device__ __forceinline__ float rms_inv(float sumsq, uint32_t d, float eps)
{
    float mean = __fdiv_rn(sumsq, (float)d);
    return __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(mean, eps)));
}

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + expf(-g)); }

// silu from the hardware exp2 and reciprocal (a few ulp): the activation of
// the fused silu-gate GEMV, whose 1e-4 bar leaves room, where the exact
// form's ~30 instructions per element sit on the path before the MFMAs (the
// reference's GPU shader uses a relaxed exp as well).  The standalone
// silu_gate keeps silu_f.
__device__ __forceinline__ float silu_fast(float g) { return __fdividef(g, 1.0f + __expf(-g)); }
