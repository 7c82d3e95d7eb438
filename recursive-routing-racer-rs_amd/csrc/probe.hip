// probe.hip -- platform probes for the measurements: a streaming read of a
// device buffer (the read that flushes the Infinity Cache before a timed
// region), a read of one share per CU with every load in flight (the floor
// one launch of a GEMV's byte count can reach) and loops of independent MFMAs
// (the matrix cores' dense rate).
#include "rrr_probe.h"

#include <hip/hip_runtime.h>

#include "device_common.h"
#include "internal.h"

namespace rrr {

// Every thread reads 16-byte units i, i + T, ... (T threads in the grid),
// one non-temporal load per iteration: each pass of the grid sweeps T * 16
// contiguous bytes, a wave 1 KB of whole cache lines, with eight workgroups
// of 256 threads on every CU keeping the loads in flight.  (Four loads per
// thread and iteration, T * 16 bytes apart, read ~13 % slower on this
// device: each wave then has four distant streams open.)  The XOR of what a
// thread read goes to out[] only if it equals a value no sane input
// produces, which keeps the loads without a write per thread.
__global__ __launch_bounds__(256) void probe_read_kernel(const u32x4 *p, uint64_t n16, uint32_t *out)
{
    const uint64_t T = (uint64_t)gridDim.x * blockDim.x;
    uint32_t acc = 0;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += T) {
        const u32x4 a = __builtin_nontemporal_load(p + i);
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    if (acc == 0x9E3779B9u) out[0] = acc;
}

// One workgroup of 1024 threads per CU reads a contiguous share of NL * 16 KB
// (a GEMV's per-CU share of its weight bytes): lane t of workgroup b loads
// the 16-byte units b * NL * 1024 + t + 1024 j, j < NL, all NL loads issued
// before the first is used (a wave load covers 1 KB of whole cache lines),
// non-temporal; buffer loads past `bytes` return zeros and move no data.
template <int NL>
__global__ __launch_bounds__(1024) void probe_share_kernel(const void *p, uint32_t bytes, uint32_t *out)
{
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(p, bytes);
    const uint32_t base = blockIdx.x * (uint32_t)(NL * 16384) + 16u * threadIdx.x;
    u32x4 v[NL];
#pragma unroll
    for (int j = 0; j < NL; j++) v[j] = bload16_nt(rs, base + 16384u * j);
    uint32_t acc = 0;
#pragma unroll
    for (int j = 0; j < NL; j++) acc ^= (v[j].x ^ v[j].y) ^ (v[j].z ^ v[j].w);
    if (acc == 0x9E3779B9u) out[0] = acc;
}

// Each wave runs `iters` rounds of 4 independent MFMAs (no dependence between
// the 4 accumulators of a round); the accumulators go to out[] only under the
// same never-taken condition.  The accumulators are one array, each started
// from its own lane-dependent value: written as four named vectors, the
// 16x16 forms compiled to eight accumulator-register moves per round between
// the MFMAs, which the probe would then have measured instead.
template <int KIND>
__global__ __launch_bounds__(256) void probe_mfma_kernel(uint32_t iters, uint32_t *out)
{
    const uint32_t lane = threadIdx.x & 63;
    if constexpr (KIND == RRR_PROBE_MFMA_F16_16X16X32) {
        f16x8 a, b;
        for (int k = 0; k < 8; k++) {
            a[k] = (_Float16)(float)((lane + k) & 7);
            b[k] = (_Float16)(float)((lane * 3 + k) & 7);
        }
        f32x4 c[4];
#pragma unroll
        for (int j = 0; j < 4; j++) c[j] = (f32x4){(float)(lane + j), 0, 0, 0};
        for (uint32_t it = 0; it < iters; it++) {
#pragma unroll
            for (int j = 0; j < 4; j++) c[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c[j], 0, 0, 0);
        }
        const f32x4 t = (c[0] + c[1]) + (c[2] + c[3]);
        const float s = (t[0] + t[1]) + (t[2] + t[3]);
        if (s == -1.0f) out[0] = __float_as_uint(s);
    } else if constexpr (KIND == RRR_PROBE_MFMA_F16_32X32X16) {
        f16x8 a, b;
        for (int k = 0; k < 8; k++) {
            a[k] = (_Float16)(float)((lane + k) & 7);
            b[k] = (_Float16)(float)((lane * 3 + k) & 7);
        }
        const float l = (float)lane;
        f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
        c0[0] = l;
        c1[1] = l;
        c2[2] = l;
        c3[3] = l;
        for (uint32_t it = 0; it < iters; it++) {
            c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c3, 0, 0, 0);
        }
        const float s = (c0[0] + c1[1]) + (c2[2] + c3[3]);
        if (s == -1.0f) out[0] = __float_as_uint(s);
    } else {
        i32x4 a, b;
        for (int k = 0; k < 4; k++) {
            a[k] = (int)(0x01010101u * ((lane + k) & 7));
            b[k] = (int)(0x01010101u * ((lane * 3 + k) & 7));
        }
        i32x4 c[4];
#pragma unroll
        for (int j = 0; j < 4; j++) c[j] = (i32x4){(int)lane + j, 0, 0, 0};
        for (uint32_t it = 0; it < iters; it++) {
#pragma unroll
            for (int j = 0; j < 4; j++)
                c[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i8x16, a), __builtin_bit_cast(i8x16, b),
                                                             c[j], 0, 0, 0);
        }
        const i32x4 t = (c[0] + c[1]) + (c[2] + c[3]);
        const int s = (t[0] + t[1]) + (t[2] + t[3]);
        if (s == -1) out[0] = (uint32_t)s;
    }
}

hipError_t launch_probe_read(const void *p, uint64_t bytes, uint32_t *out, hipStream_t s)
{
    const uint32_t grid = 8 * device_cu_count();
    hipLaunchKernelGGL(probe_read_kernel, dim3(grid), dim3(256), 0, s, (const u32x4 *)p, bytes / 16, out);
    return hipGetLastError();
}

bool probe_shares_supported(uint64_t bytes) { return bytes > 0 && bytes <= (uint64_t)device_cu_count() * 16 * 16384; }

hipError_t launch_probe_shares(const void *p, uint64_t bytes, uint32_t *out, hipStream_t s)
{
    const uint32_t cus = device_cu_count();
    const uint64_t per = (bytes + cus - 1) / cus, nl = (per + 16383) / 16384;
#define RRR_SHARE_CASE(N)                                                                                         \
    if (nl <= N) {                                                                                                \
        hipLaunchKernelGGL(probe_share_kernel<N>, dim3(cus), dim3(1024), 0, s, p, (uint32_t)bytes, out);         \
        return hipGetLastError();                                                                                 \
    }
    RRR_SHARE_CASE(1) RRR_SHARE_CASE(2) RRR_SHARE_CASE(3) RRR_SHARE_CASE(4) RRR_SHARE_CASE(5) RRR_SHARE_CASE(6)
    RRR_SHARE_CASE(7) RRR_SHARE_CASE(8) RRR_SHARE_CASE(10) RRR_SHARE_CASE(12) RRR_SHARE_CASE(16)
#undef RRR_SHARE_CASE
    return hipErrorInvalidValue;
}

hipError_t launch_probe_mfma(uint32_t kind, uint32_t waves_per_cu, uint32_t iters, uint32_t *out, hipStream_t s)
{
    // 4 waves a workgroup, waves_per_cu / 4 workgroups per CU
    const uint32_t grid = device_cu_count() * (waves_per_cu / 4);
    switch (kind) {
    case RRR_PROBE_MFMA_F16_16X16X32:
        hipLaunchKernelGGL(probe_mfma_kernel<RRR_PROBE_MFMA_F16_16X16X32>, dim3(grid), dim3(256), 0, s, iters, out);
        break;
    case RRR_PROBE_MFMA_F16_32X32X16:
        hipLaunchKernelGGL(probe_mfma_kernel<RRR_PROBE_MFMA_F16_32X32X16>, dim3(grid), dim3(256), 0, s, iters, out);
        break;
    default:
        hipLaunchKernelGGL(probe_mfma_kernel<RRR_PROBE_MFMA_I8_16X16X64>, dim3(grid), dim3(256), 0, s, iters, out);
        break;
    }
    return hipGetLastError();
}

}  // namespace rrr
