// attn.hip -- the decode glue around the weight sweep: RoPE with the f16
// KV-cache store (the rope_kv_store / kv_store pipelines, phi4.rs:1016-1017,
// :1666-1677) and decode attention over the cache (the attention pipeline,
// phi4.rs:1018, :1304-1312).
#include "act.h"

namespace rrr {

// Token blockIdx.y (position pos + blockIdx.y, its qkv row_stride floats
// after the previous one's).  Work items [0, nq): the Q rotation pairs (head
// i / (rope_dim/2), pair i % (rope_dim/2)), rotated in place.  Items [nq, nq +
// kv_stride/2): element pair 2p of K (rotated in place when it lies in its
// head's first rope_dim dims) and of V, both stored as f16 into the token's
// row of the caches.  The position's rope_dim/2 coefficient pairs (shared by
// every Q and K head) are computed once per workgroup into LDS when `lds_coef`
// (rope_coef, the same values), else per item.
__global__ __launch_bounds__(256) void rope_kv_store_kernel(float *__restrict__ qkv, RopeArgs r, uint32_t *__restrict__ kc,
                                                            uint32_t *__restrict__ vc, uint32_t lds_coef)
{
    extern __shared__ float cf[];   // pair j at cf[2j], cf[2j + 1]
    const uint32_t half_rope = r.rope_dim / 2;
    const uint32_t nq = r.n_heads * half_rope, nkv = r.kv_stride / 2;
    const uint32_t pos = r.pos + blockIdx.y;
    qkv += (size_t)blockIdx.y * r.row_stride;
    if (lds_coef) {
        for (uint32_t j = threadIdx.x; j < half_rope; j += 256) rope_coef(j, pos, r, cf[2 * j], cf[2 * j + 1]);
        __syncthreads();
    }
    auto coef = [&](uint32_t j, float &cs, float &ss) {
        if (lds_coef) {
            cs = cf[2 * j];
            ss = cf[2 * j + 1];
        } else {
            rope_coef(j, pos, r, cs, ss);
        }
    };
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < nq + nkv; i += gridDim.x * 256) {
        if (i < nq) {
            const uint32_t h = i / half_rope, j = i - h * half_rope;
            float *p = qkv + (size_t)h * r.head_dim + 2 * j;
            float x0 = p[0], x1 = p[1], cs, ss;
            coef(j, cs, ss);
            rope_rotate(x0, x1, cs, ss);
            p[0] = x0;
            p[1] = x1;
        } else {
            const uint32_t e = 2 * (i - nq);
            float *k = qkv + r.q_dim + e;
            const float *v = qkv + r.q_dim + r.kv_stride + e;
            float k0 = k[0], k1 = k[1];
            const uint32_t d = r.rope_dim ? e % r.head_dim : 0u;   // head_dim is 0 in the kv_store form
            if (d < r.rope_dim) {
                float cs, ss;
                coef(d / 2, cs, ss);
                rope_rotate(k0, k1, cs, ss);
                k[0] = k0;
                k[1] = k1;
            }
            const size_t w = ((size_t)pos * r.kv_stride + e) / 2;
            kc[w] = f16_bits(k0) | (f16_bits(k1) << 16);
            vc[w] = f16_bits(v[0]) | (f16_bits(v[1]) << 16);
        }
    }
}

// Rows of many tokens: one workgroup per token walking its items (its
// coefficients computed once); a few tokens: a workgroup per 256 items.
hipError_t launch_rope_kv_store(float *qkv, const RopeArgs &r, uint16_t *kc, uint16_t *vc, hipStream_t s,
                                uint32_t rows)
{
    const uint32_t n = r.n_heads * (r.rope_dim / 2) + r.kv_stride / 2;
    if (n == 0 || rows == 0) return hipSuccess;
    const size_t lds = (size_t)r.rope_dim * 4;
    const uint32_t lds_coef = lds <= 32 * 1024 ? 1u : 0u;
    const uint32_t bx = rows >= 64 ? 1u : (n + 255) / 256;
    hipLaunchKernelGGL(rope_kv_store_kernel, dim3(bx, rows), dim3(256), lds_coef ? lds : 0, s, qkv, r, (uint32_t *)kc,
                       (uint32_t *)vc, lds_coef);
    return hipGetLastError();
}

// The prompt's QKV rows from the K-split GEMM's partials: element (m, c) is
// the sum of ws[k][m][c] over the S splits in split order (as
// gemm_splitk_reduce adds them), then the rope_kv_store of the row: every
// element of qkv, and the caches, end bit for bit as after the reduction
// followed by rope_kv_store_kernel.  Rows m >= rows (the GEMM's padding rows)
// get the plain sums (SS = S, 2..8: a quad's partials are all requested
// before the first add).  Four elements (two pairs) a thread; the launcher
// requires q_dim, kv_stride and row_stride (= the GEMM's N) % 4 == 0, so a
// quad never straddles the Q, K and V parts.
template <int SS>
__global__ __launch_bounds__(256) void splitk_rope_kv_store_kernel(const float *__restrict__ ws, uint32_t M,
                                                                   float *__restrict__ qkv, RopeArgs r, uint32_t rows,
                                                                   uint32_t *__restrict__ kc, uint32_t *__restrict__ vc,
                                                                   uint32_t lds_coef)
{
    extern __shared__ float cf[];   // pair j at cf[2j], cf[2j + 1]
    const uint32_t N = r.row_stride, m = blockIdx.y, half_rope = r.rope_dim / 2;
    const uint32_t pos = r.pos + m, qh = r.n_heads * r.head_dim;
    const bool live = m < rows;
    const uint64_t mn = (uint64_t)M * N;
    const float *src = ws + (uint64_t)m * N;
    float *dst = qkv + (uint64_t)m * N;
    if (lds_coef && live) {
        for (uint32_t j = threadIdx.x; j < half_rope; j += 256) rope_coef(j, pos, r, cf[2 * j], cf[2 * j + 1]);
        __syncthreads();
    }
    auto coef = [&](uint32_t j, float &cs, float &ss) {
        if (lds_coef) {
            cs = cf[2 * j];
            ss = cf[2 * j + 1];
        } else {
            rope_coef(j, pos, r, cs, ss);
        }
    };
    for (uint32_t c = 4 * (blockIdx.x * 256 + threadIdx.x); c < N; c += 4 * gridDim.x * 256) {
        float4 p[SS];
#pragma unroll
        for (int k = 0; k < SS; k++) p[k] = *(const float4 *)(src + k * mn + c);
        float4 v = p[0];
#pragma unroll
        for (int k = 1; k < SS; k++) {
            v.x += p[k].x; v.y += p[k].y; v.z += p[k].z; v.w += p[k].w;
        }
        if (live) {
            float x[4] = {v.x, v.y, v.z, v.w};
            if (c < r.q_dim) {
                // Q: pair j of a head rotated for j < rope_dim / 2
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const uint32_t e = c + 2 * h;
                    if (e < qh) {
                        const uint32_t j = (e % r.head_dim) / 2;
                        if (j < half_rope) {
                            float cs, ss;
                            coef(j, cs, ss);
                            rope_rotate(x[2 * h], x[2 * h + 1], cs, ss);
                        }
                    }
                }
            } else if (c < r.q_dim + r.kv_stride) {
                // K: rotated dims below rope_dim of each head, stored in row pos
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const uint32_t e = c - r.q_dim + 2 * h;
                    const uint32_t d = r.rope_dim ? e % r.head_dim : 0u;
                    if (d < r.rope_dim) {
                        float cs, ss;
                        coef(d / 2, cs, ss);
                        rope_rotate(x[2 * h], x[2 * h + 1], cs, ss);
                    }
                    kc[((size_t)pos * r.kv_stride + e) / 2] = f16_bits(x[2 * h]) | (f16_bits(x[2 * h + 1]) << 16);
                }
            } else {
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const uint32_t e = c - r.q_dim - r.kv_stride + 2 * h;
                    vc[((size_t)pos * r.kv_stride + e) / 2] = f16_bits(x[2 * h]) | (f16_bits(x[2 * h + 1]) << 16);
                }
            }
            v = make_float4(x[0], x[1], x[2], x[3]);
        }
        *(float4 *)(dst + c) = v;
    }
}

bool splitk_rope_kv_store_supported(const RopeArgs &r)
{
    return r.q_dim % 4 == 0 && r.kv_stride % 4 == 0 && r.row_stride % 4 == 0 &&
           r.row_stride == r.q_dim + 2 * r.kv_stride;
}

// One workgroup per row (M rows: the GEMM's, padding included).
hipError_t launch_splitk_rope_kv_store(const float *ws, uint32_t S, uint32_t M, float *qkv, const RopeArgs &r,
                                       uint32_t rows, uint16_t *kc, uint16_t *vc, hipStream_t s)
{
    if (!splitk_rope_kv_store_supported(r)) return hipErrorNotSupported;
    const size_t lds = (size_t)r.rope_dim * 4;
    const uint32_t lds_coef = lds <= 32 * 1024 ? 1u : 0u;
#define RRR_SRK_CASE(K)                                                                                          \
    case K:                                                                                                       \
        hipLaunchKernelGGL(splitk_rope_kv_store_kernel<K>, dim3(1, M), dim3(256), lds_coef ? lds : 0, s, ws, M, qkv, \
                           r, rows, (uint32_t *)kc, (uint32_t *)vc, lds_coef);                                      \
        break;
    switch (S) {
        RRR_SRK_CASE(2) RRR_SRK_CASE(3) RRR_SRK_CASE(4) RRR_SRK_CASE(5)
        RRR_SRK_CASE(6) RRR_SRK_CASE(7) RRR_SRK_CASE(8)
    default: return hipErrorInvalidValue;
    }
#undef RRR_SRK_CASE
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Decode attention, split over the sequence (flash-decoding), one launch.
// Workgroup (g, sp) takes KV head g and cache rows [sp * per, sp * per + per),
// at most 16 * ATT_ROWS_PER_GROUP of them: its 16 lane groups of 16 lanes each
// take every 16th row (all of their K and V loads in flight at once), lane li
// owning dims 8 li .. 8 li + 7 of a row (one 16-byte f16 load of K and one of
// V; a score is one DPP row sum).  The HPK query heads of the KV group share
// every K/V load.  Scores go through exp2 with the queries pre-scaled by
// log2(e) / sqrt(head_dim).  A wave's 4 lane groups take one maximum per head
// (lane swaps), so their sums and outputs add without rescaling; the 4 waves
// are merged in LDS, and the workgroup's {output, max, sum} per query head is
// written through the coherent level; the last workgroup of KV head g to
// arrive (an agent-scope counter) merges the splits and writes the output,
// then resets the counter for the next call.  Every merge runs in a fixed
// order, so the result depends on seq_len only.

__device__ __forceinline__ float safe_scale(float m, float M) { return m == -__builtin_inff() ? 0.0f : exp2f(m - M); }

// exp2(m - M), 0 for m = -inf (a part without rows), without a branch: the
// hardware exp2 runs for every lane and the select follows (results below
// 2^-126 flush to zero, against a largest weight of 1).
__device__ __forceinline__ float scale_exp2(float m, float M)
{
    const float e = __builtin_amdgcn_exp2f(m - M);
    return m == -__builtin_inff() ? 0.0f : e;
}

// Sum over the 16 lanes of a DPP row (butterfly: xor 1, xor 2, then the
// half-row and row mirrors); every lane of the row gets the sum.
__device__ __forceinline__ float row16_sum(float v)
{
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false));  // row_half_mirror
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false));  // row_mirror
    return v;
}

// Online-softmax state {m, l, o[8]} of lanes (lane & ~X) and (lane | X)
// merged, lower partner first: both lanes end with the same state.
template <int X>
__device__ __forceinline__ void merge_pair(float &m, float &l, float (&o)[8])
{
    float m0, m1, l0, l1;
    lane_pair<X>(m, m0, m1);
    lane_pair<X>(l, l0, l1);
    const float M = fmaxf(m0, m1), c0 = safe_scale(m0, M), c1 = safe_scale(m1, M);
    l = l0 * c0 + l1 * c1;
#pragma unroll
    for (int d = 0; d < 8; d++) {
        float o0, o1;
        lane_pair<X>(o[d], o0, o1);
        o[d] = o0 * c0 + o1 * c1;
    }
    m = M;
}

template <int HPK>
__global__ __launch_bounds__(256) void attn_kernel(const float *__restrict__ q, const uint16_t *__restrict__ kc,
                                                   const uint16_t *__restrict__ vc, float *part, uint32_t *counters,
                                                   float *__restrict__ out, uint32_t seq, uint32_t per,
                                                   uint32_t kv_stride, float qscale)
{
    __shared__ float gml[4][HPK][2];
    __shared__ __attribute__((aligned(16))) float go[4][HPK][ATT_HD];
    __shared__ uint32_t last;
    const uint32_t g = blockIdx.x, sp = blockIdx.y, splits = gridDim.y;
    const uint32_t t = threadIdx.x, grp = t >> 4, li = t & 15;
    const uint32_t r0 = sp * per, r1 = min(seq, r0 + per);

    // this lane group's rows r0 + grp + 16 k (k < ATT_ROWS_PER_GROUP), all
    // requested first; a row past the split repeats the split's last row
    // (already fetched by another lane group: no extra memory traffic)
    u32x4 kr[ATT_ROWS_PER_GROUP], vr[ATT_ROWS_PER_GROUP];
#pragma unroll
    for (int k = 0; k < (int)ATT_ROWS_PER_GROUP; k++) {
        const uint32_t row = min(r0 + grp + 16 * k, r1 - 1);
        const size_t off = (size_t)row * kv_stride + (size_t)g * ATT_HD + 8 * li;
        kr[k] = *(const u32x4 *)(kc + off);
        vr[k] = *(const u32x4 *)(vc + off);
    }
    float qv[HPK][8];
#pragma unroll
    for (int h = 0; h < HPK; h++) {
        const float4 *qp = (const float4 *)(q + (size_t)(g * HPK + h) * ATT_HD + 8 * li);
        const float4 a = qp[0], b = qp[1];
        qv[h][0] = a.x * qscale; qv[h][1] = a.y * qscale; qv[h][2] = a.z * qscale; qv[h][3] = a.w * qscale;
        qv[h][4] = b.x * qscale; qv[h][5] = b.y * qscale; qv[h][6] = b.z * qscale; qv[h][7] = b.w * qscale;
    }
    // the lane group's ATT_ROWS_PER_GROUP rows at once: their scores
    // (independent dot products and row sums), the wave's maximum per head,
    // then the sum and output; rows past the split add nothing (uniform in the
    // row of 16 lanes)
    constexpr int R = (int)ATT_ROWS_PER_GROUP;
    float kf[R][8], v[R][8];
    bool live[R];
#pragma unroll
    for (int k = 0; k < R; k++) {
        live[k] = r0 + grp + 16 * k < r1;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            kf[k][2 * w] = h2f(kr[k][w] & 0xFFFFu);
            kf[k][2 * w + 1] = h2f(kr[k][w] >> 16);
            v[k][2 * w] = h2f(vr[k][w] & 0xFFFFu);
            v[k][2 * w + 1] = h2f(vr[k][w] >> 16);
        }
    }
    const uint32_t wv = t >> 6;
#pragma unroll
    for (int h = 0; h < HPK; h++) {
        float sc[R];
#pragma unroll
        for (int k = 0; k < R; k++) {
            float s = 0.0f;
#pragma unroll
            for (int d = 0; d < 8; d++) s = fmaf(qv[h][d], kf[k][d], s);
            sc[k] = row16_sum(s);
        }
        float mx = -__builtin_inff();
#pragma unroll
        for (int k = 0; k < R; k++)
            if (live[k]) mx = fmaxf(mx, sc[k]);
        mx = lanes4_max(mx);   // the wave's maximum: -inf only for a wave without rows
        float ps = 0.0f, p[R];
#pragma unroll
        for (int k = 0; k < R; k++) {
            const float e = __builtin_amdgcn_exp2f(sc[k] - mx);
            p[k] = live[k] ? e : 0.0f;
            ps += p[k];
        }
        float od[8];
#pragma unroll
        for (int d = 0; d < 8; d++) {
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < R; k++) acc = fmaf(p[k], v[k][d], acc);
            od[d] = lanes4_sum(acc);
        }
        ps = lanes4_sum(ps);
        if ((t & 63) < 16) {
            if (li == 0) {
                gml[wv][h][0] = mx;
                gml[wv][h][1] = ps;
            }
            float4 *dst = (float4 *)&go[wv][h][8 * li];
            dst[0] = make_float4(od[0], od[1], od[2], od[3]);
            dst[1] = make_float4(od[4], od[5], od[6], od[7]);
        }
    }
    __syncthreads();
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(part, (uint64_t)gridDim.x * HPK * splits * ATT_PART * 4);
    for (uint32_t i = t; i < HPK * ATT_HD; i += 256) {
        const uint32_t h = i / ATT_HD, d = i % ATT_HD;
        const float M = fmaxf(fmaxf(gml[0][h][0], gml[1][h][0]), fmaxf(gml[2][h][0], gml[3][h][0]));
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int wi = 0; wi < 4; wi++) {
            const float c = scale_exp2(gml[wi][h][0], M);   // 0 for a wave without rows
            L = fmaf(gml[wi][h][1], c, L);
            O = fmaf(go[wi][h][d], c, O);
        }
        if (splits == 1) {
            out[(size_t)(g * HPK + h) * ATT_HD + d] = O / L;
        } else {
            // partial of (g, sp, h): [output 128 | max | sum]
            const uint32_t base = (((g * splits + sp) * HPK + h) * ATT_PART) * 4;
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(O), rp, base + 4 * d, 0, RRR_CPOL_SC1);
            if (d == 0) {
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(M), rp, base + 4 * ATT_HD, 0, RRR_CPOL_SC1);
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(L), rp, base + 4 * ATT_HD + 4, 0, RRR_CPOL_SC1);
            }
        }
    }
    if (splits == 1) return;
    // publish: this workgroup's partials are at the coherent level, then count
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (t == 0)
        last = __hip_atomic_fetch_add(counters + g * ATT_COUNTER_STRIDE, 1u, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == splits - 1;
    __syncthreads();
    if (!last) return;
    // the last workgroup of KV head g merges its splits: wave w takes query
    // heads w, w + 4, ...; lane (dq, hf) = (lane % 32, lane / 32) takes dims
    // 4 dq .. 4 dq + 3 of splits 16 hf .. 16 hf + 15.  All of a head's loads
    // (output quads, maxima and sums) are in flight at once; the two halves
    // meet by lane swaps (both lanes compute the same max and the same
    // lower + upper sum), and everything is added in split order.
    static_assert(ATT_SPLITS_MAX <= 32, "two halves of at most 16 splits");
    const uint32_t lane = t & 63, dq = lane & 31, hf = lane >> 5;
    for (uint32_t h = wv; h < (uint32_t)HPK; h += 4) {
        u32x4 ov[16];
        float ms[16], ls[16];
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const uint32_t s = min(16 * hf + j, splits - 1);   // past the last split: a valid record, weight 0
            const uint32_t base = (((g * splits + s) * HPK + h) * ATT_PART) * 4;
            ov[j] = __builtin_amdgcn_raw_buffer_load_b128(rp, base + 16 * dq, 0, RRR_CPOL_SC1);
            const auto u = __builtin_amdgcn_raw_buffer_load_b64(rp, base + 4 * ATT_HD, 0, RRR_CPOL_SC1);
            ms[j] = __uint_as_float(u[0]);
            ls[j] = __uint_as_float(u[1]);
        }
        __builtin_amdgcn_sched_barrier(0);   // keep every load ahead of the first use
        float M = -__builtin_inff();
#pragma unroll
        for (int j = 0; j < 16; j++)
            if (16 * hf + j < splits) M = fmaxf(M, ms[j]);
        float lo, hi;
        lane_pair<32>(M, lo, hi);
        M = fmaxf(lo, hi);
        float L = 0.0f, O[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const float e = scale_exp2(ms[j], M);
            const float w = 16 * hf + j < splits ? e : 0.0f;
            L = fmaf(ls[j], w, L);
            O[0] = fmaf(__uint_as_float(ov[j].x), w, O[0]);
            O[1] = fmaf(__uint_as_float(ov[j].y), w, O[1]);
            O[2] = fmaf(__uint_as_float(ov[j].z), w, O[2]);
            O[3] = fmaf(__uint_as_float(ov[j].w), w, O[3]);
        }
        lane_pair<32>(L, lo, hi);
        L = lo + hi;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            lane_pair<32>(O[c], lo, hi);
            O[c] = lo + hi;
        }
        if (hf == 0)
            *(float4 *)(out + (size_t)(g * HPK + h) * ATT_HD + 4 * dq) =
                make_float4(O[0] / L, O[1] / L, O[2] / L, O[3] / L);
    }
    __syncthreads();
    if (t == 0) __hip_atomic_store(counters + g * ATT_COUNTER_STRIDE, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

uint64_t attention_scratch_bytes() { return ATT_SCRATCH_BYTES; }

// Rows per split: as many as the 16 lane groups take (16 * ATT_ROWS_PER_GROUP),
// so the fewest splits: below that the cross-workgroup merge (partials
// through the coherent level, a counter, the last workgroup's loads, ~2.5 us)
// costs more than the longer splits' load phase (64 rows: 4.3 us in one split
// against 6.9 us in four; 512 rows 7.45 against 8.1 us in 32 splits).  At
// most ATT_SPLITS_MAX splits, which holds for seq <= ATT_SEQ_MAX.
void attention_plan(uint32_t seq, uint32_t n_kv_heads, uint32_t heads_per_kv, uint32_t cus, uint32_t &splits,
                    uint32_t &per)
{
    (void)n_kv_heads;
    (void)heads_per_kv;
    (void)cus;
    splits = min(ATT_SPLITS_MAX, max(1u, (seq + 16 * ATT_ROWS_PER_GROUP - 1) / (16 * ATT_ROWS_PER_GROUP)));
    per = (seq + splits - 1) / splits;
    splits = (seq + per - 1) / per;   // every split has at least one row
}

template <int HPK>
static void go_attn(const float *q, const uint16_t *kc, const uint16_t *vc, float *part, uint32_t *counters, float *out,
                    uint32_t seq, uint32_t per, uint32_t kv_stride, float qscale, uint32_t n_kv_heads, uint32_t splits,
                    hipStream_t s)
{
    hipLaunchKernelGGL(attn_kernel<HPK>, dim3(n_kv_heads, splits), dim3(256), 0, s, q, kc, vc, part, counters, out, seq,
                       per, kv_stride, qscale);
}

hipError_t launch_attention(const float *q, const uint16_t *kc, const uint16_t *vc, float *out, void *scratch,
                            uint32_t seq, uint32_t n_kv_heads, uint32_t heads_per_kv, uint32_t cus, hipStream_t s)
{
    uint32_t splits, per;
    attention_plan(seq, n_kv_heads, heads_per_kv, cus, splits, per);
    const uint32_t kv_stride = n_kv_heads * ATT_HD;
    const float qscale = (float)(1.4426950408889634 / sqrt((double)ATT_HD));   // log2(e) / sqrt(head_dim)
    uint32_t *counters = (uint32_t *)scratch;
    float *part = (float *)((char *)scratch + ATT_COUNTER_BYTES);
#define RRR_ATT_CASE(H) \
    case H: go_attn<H>(q, kc, vc, part, counters, out, seq, per, kv_stride, qscale, n_kv_heads, splits, s); break;
    switch (heads_per_kv) {
        RRR_ATT_CASE(1) RRR_ATT_CASE(2) RRR_ATT_CASE(3) RRR_ATT_CASE(4)
        RRR_ATT_CASE(5) RRR_ATT_CASE(6) RRR_ATT_CASE(7) RRR_ATT_CASE(8)
    default: return hipErrorInvalidValue;
    }
#undef RRR_ATT_CASE
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Causal prefill attention (the per-token attention dispatches of
// forward_prefill_batched, phi4.rs:1304-1312, for all prompt tokens in one
// launch).  Workgroup (g, tok) takes KV head g for token tok at position
// pos0 + tok, over cache rows 0 .. pos0 + tok.  The lane layout, scores and
// online softmax are the decode kernel's; the rows are walked in chunks of
// 16 * ATT_ROWS_PER_GROUP (lane group grp takes rows grp, grp + 16, ... of a
// chunk), the next chunk's K/V loads issued before the current chunk is
// scored (rows past the end repeat the last row: no branch around the loads).
// The 16 lane groups are merged in LDS in a fixed order.
template <int HPK, bool F16OUT>
__global__ __launch_bounds__(256) void attn_prefill_kernel(const float *__restrict__ qkv, uint32_t row_stride,
                                                           const uint16_t *__restrict__ kc,
                                                           const uint16_t *__restrict__ vc, void *__restrict__ out,
                                                           uint32_t pos0, uint32_t kv_stride, float qscale)
{
    constexpr uint32_t CH = 16 * ATT_ROWS_PER_GROUP;
    __shared__ float gml[16][HPK][2];
    __shared__ __attribute__((aligned(16))) float go[16][HPK][ATT_HD];
    const uint32_t g = blockIdx.x, tok = blockIdx.y;
    const uint32_t t = threadIdx.x, grp = t >> 4, li = t & 15;
    const uint32_t L = pos0 + tok + 1, nch = (L + CH - 1) / CH;

    u32x4 kr[ATT_ROWS_PER_GROUP], vr[ATT_ROWS_PER_GROUP], kn[ATT_ROWS_PER_GROUP], vn[ATT_ROWS_PER_GROUP];
    auto load = [&](u32x4 *kd, u32x4 *vd, uint32_t c) {
#pragma unroll
        for (int k = 0; k < (int)ATT_ROWS_PER_GROUP; k++) {
            const uint32_t row = min(c * CH + grp + 16 * k, L - 1);
            const size_t off = (size_t)row * kv_stride + (size_t)g * ATT_HD + 8 * li;
            kd[k] = *(const u32x4 *)(kc + off);
            vd[k] = *(const u32x4 *)(vc + off);
        }
    };
    load(kr, vr, 0);
    const float *q = qkv + (size_t)tok * row_stride;
    float qv[HPK][8];
#pragma unroll
    for (int h = 0; h < HPK; h++) {
        const float4 *qp = (const float4 *)(q + (size_t)(g * HPK + h) * ATT_HD + 8 * li);
        const float4 a = qp[0], b = qp[1];
        qv[h][0] = a.x * qscale; qv[h][1] = a.y * qscale; qv[h][2] = a.z * qscale; qv[h][3] = a.w * qscale;
        qv[h][4] = b.x * qscale; qv[h][5] = b.y * qscale; qv[h][6] = b.z * qscale; qv[h][7] = b.w * qscale;
    }
    float m[HPK], l[HPK], o[HPK][8];
#pragma unroll
    for (int h = 0; h < HPK; h++) {
        m[h] = -__builtin_inff();
        l[h] = 0.0f;
#pragma unroll
        for (int d = 0; d < 8; d++) o[h][d] = 0.0f;
    }
    for (uint32_t c = 0; c < nch; c++) {
        load(kn, vn, min(c + 1, nch - 1));
#pragma unroll
        for (int k = 0; k < (int)ATT_ROWS_PER_GROUP; k++) {
            const bool live = c * CH + grp + 16 * k < L;
            float kf[8], v[8];
#pragma unroll
            for (int w = 0; w < 4; w++) {
                kf[2 * w] = h2f(kr[k][w] & 0xFFFFu);
                kf[2 * w + 1] = h2f(kr[k][w] >> 16);
                v[2 * w] = h2f(vr[k][w] & 0xFFFFu);
                v[2 * w + 1] = h2f(vr[k][w] >> 16);
            }
#pragma unroll
            for (int h = 0; h < HPK; h++) {
                float sc = 0.0f;
#pragma unroll
                for (int d = 0; d < 8; d++) sc = fmaf(qv[h][d], kf[d], sc);
                sc = row16_sum(sc);
                if (live) {
                    const float mn = fmaxf(m[h], sc);
                    const float cf = exp2f(m[h] - mn), p = exp2f(sc - mn);
                    l[h] = fmaf(l[h], cf, p);
#pragma unroll
                    for (int d = 0; d < 8; d++) o[h][d] = fmaf(o[h][d], cf, p * v[d]);
                    m[h] = mn;
                }
            }
        }
#pragma unroll
        for (int k = 0; k < (int)ATT_ROWS_PER_GROUP; k++) {
            kr[k] = kn[k];
            vr[k] = vn[k];
        }
    }
#pragma unroll
    for (int h = 0; h < HPK; h++) {
        if (li == 0) {
            gml[grp][h][0] = m[h];
            gml[grp][h][1] = l[h];
        }
        float4 *dst = (float4 *)&go[grp][h][8 * li];
        dst[0] = make_float4(o[h][0], o[h][1], o[h][2], o[h][3]);
        dst[1] = make_float4(o[h][4], o[h][5], o[h][6], o[h][7]);
    }
    __syncthreads();
    const size_t orow = (size_t)tok * gridDim.x * HPK * ATT_HD;
    for (uint32_t i = t; i < HPK * ATT_HD; i += 256) {
        const uint32_t h = i / ATT_HD, d = i % ATT_HD;
        float M = -__builtin_inff();
#pragma unroll
        for (int gi = 0; gi < 16; gi++) M = fmaxf(M, gml[gi][h][0]);
        float Ls = 0.0f, O = 0.0f;
#pragma unroll
        for (int gi = 0; gi < 16; gi++) {
            const float c = safe_scale(gml[gi][h][0], M);   // 0 for a group without rows
            Ls = fmaf(gml[gi][h][1], c, Ls);
            O = fmaf(go[gi][h][d], c, O);
        }
        const size_t oi = orow + (size_t)(g * HPK + h) * ATT_HD + d;
        if constexpr (F16OUT)
            ((_Float16 *)out)[oi] = (_Float16)(O / Ls);
        else
            ((float *)out)[oi] = O / Ls;
    }
}

// Causal prefill attention on the matrix cores.  Workgroup (g, tb): query
// heads g*HPK .. g*HPK+HPK-1, of KV head g / hsplit (hsplit workgroups share
// a KV group's heads_per_kv = hsplit * HPK heads; hsplit 1: all of them),
// tokens tb*16 .. tb*16+15 (lane l's token is l % 16); its ATTM_WAVES
// waves take every ATTM_WAVES-th block of 32 cache rows and merge their
// (max, sum, output) at the end in a fixed order.  Per block and per query
// head h of the group:
//   S^T = K . Q^T    (v_mfma_f32_16x16x32_f16, keys x tokens, K from the f16
//                     cache as A operands, Q^T as B operands in f16 hi + lo,
//                     so the scores carry ~2^-22 of Q's rounding)
//   online softmax per token (exp2, queries pre-scaled by log2(e)/sqrt(128)),
//                    its reference max moved lazily (P <= 8)
//   O^T += V^T . P^T (dims x tokens; P in f16 hi + lo, V exact in f16)
// In the MFMA layouts (lane l: A row / B column l % 16 at k slots
// 8 (l / 16) .. +7; D rows 4 (l / 16) + r of column l % 16) lane l's D
// registers of the two S^T key tiles hold keys 4 (l/16) + r and
// 16 + 4 (l/16) + r of its token: exactly the 8 k slots it supplies as P^T's
// B operand when V^T's A operand takes the same keys in the same order (the
// k order inside one MFMA only has to agree between A and B).  V^T comes
// from a transposed LDS copy of the block.  A token's scores of a block sit
// in the 4 lanes l % 16 + 16 j: its max and sum are two cross-lane steps.
// The hi + lo splits are taken of Q * 2^(14 - e) (per token and head, the
// scaled query's largest component f * 2^e, f in [0.5, 1): it lands in
// [2^13, 2^14), inside f16's range whatever the activations' size) and of
// P * 2^12 (P <= 8), undone exactly on the scores and at the end; the lo
// parts then stay in f16's normal range, where they keep their precision.
// The Q^T operands sit in LDS (one head's are read per block), so the
// accumulators need no moves between register files.
constexpr uint32_t ATTM_LD = 36;   // f16 per V^T row in LDS (32 keys + pad; 72-byte rows)
constexpr float ATTM_PS = 4096.0f;
constexpr uint32_t ATTM_WAVES = 4, ATTM_OLD = ATT_HD + 4;   // waves; floats per merged output row (padded)

__device__ __forceinline__ void wave_lds_order()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int HPK>
struct AttmLds {
    static constexpr size_t VT = (size_t)ATTM_WAVES * ATT_HD * ATTM_LD * 2;            // V^T per wave
    static constexpr size_t O = (size_t)ATTM_WAVES * HPK * 16 * ATTM_OLD * 4;          // merge: outputs
    static constexpr size_t ML = (size_t)ATTM_WAVES * HPK * 16 * 2 * 4;                // merge: max, sum
    static constexpr size_t Q = (size_t)HPK * 4 * 2 * 64 * 16;                        // Q^T operands, hi + lo
    // the loop's V^T and Q^T share their bytes with the merge's outputs
    static constexpr size_t CW = (size_t)HPK * 16 * (ATTM_WAVES + 1) * 4;             // merge: weights, scale
    static constexpr size_t LOOP = VT + Q, MAIN = LOOP > O ? LOOP : O;
    static constexpr size_t BYTES = MAIN + ML + CW;
};

template <int HPK, bool F16OUT>
__global__ __launch_bounds__(64 * ATTM_WAVES) void attn_prefill_mfma_kernel(const float *__restrict__ qkv, uint32_t row_stride,
                                                               const uint16_t *__restrict__ kc,
                                                               const uint16_t *__restrict__ vc,
                                                               void *__restrict__ out, uint32_t rows, uint32_t pos0,
                                                               uint32_t kv_stride, float qscale, uint32_t hsplit)
{
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    typedef float f4 __attribute__((ext_vector_type(4)));
    using LD = AttmLds<HPK>;
    __shared__ __attribute__((aligned(16))) uint8_t sm[LD::BYTES];
    const uint32_t wv = threadIdx.x >> 6;
    _Float16 *vt = (_Float16 *)sm + (size_t)wv * ATT_HD * ATTM_LD;   // this wave's V^T
    float *mo = (float *)sm;                                        // merge outputs (after the loop)
    float *mml = (float *)(sm + LD::MAIN);                          // merge max / sum
    float *mcw = (float *)(sm + LD::MAIN + LD::ML);                 // merge weights and scale per (head, token)
    h8 *qop = (h8 *)(sm + LD::VT);                                  // Q^T operands [h][kk][hi, lo][lane]
    const uint32_t g = blockIdx.x, tb = blockIdx.y, l = threadIdx.x & 63, n = l & 15, grp = l >> 4;
    const uint32_t tok = tb * 16 + n, tq = min(tok, rows - 1), tpos = pos0 + tq;
    const uint32_t last = pos0 + min(tb * 16 + 15, rows - 1);      // the last cache row the block's tokens see
    const uint32_t nblk = last / 32 + 1;
    const uint16_t *kbase = kc + (size_t)(g / hsplit) * ATT_HD, *vbase = vc + (size_t)(g / hsplit) * ATT_HD;

    // K and V of block blk (rows past `last` repeat it): the next block of
    // this wave is requested before the current one is multiplied
    auto load_blk = [&](uint32_t blk, h8 (&ka)[2][4], h8 (&vr)[2][4]) {
        const uint32_t c0 = 32 * blk;
        // K A operands: key tile kt (rows c0 + 16 kt + n), dims 32 kk + 8 grp
#pragma unroll
        for (int kt = 0; kt < 2; kt++) {
            const uint32_t row = min(c0 + 16 * kt + n, last);
#pragma unroll
            for (int kk = 0; kk < 4; kk++)
                ka[kt][kk] = *(const h8 *)(kbase + (size_t)row * kv_stride + 32 * kk + 8 * grp);
        }
        // V rows c0 + 4 grp + {0..3} and c0 + 16 + 4 grp + {0..3}, dims 8 n .. 8 n + 7
#pragma unroll
        for (int half = 0; half < 2; half++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t row = min(c0 + 16 * half + 4 * grp + j, last);
                vr[half][j] = *(const h8 *)(vbase + (size_t)row * kv_stride + 8 * n);
            }
    };
    // this wave's first block is requested before the Q^T operands are built
    h8 kaA[2][4], vrA[2][4];
    if (wv < nblk) load_blk(wv, kaA, vrA);

    // Q^T operands of each head: token tq, dims 32 kk + 8 grp .. +7, scaled,
    // hi + lo; every wave computes them, wave 0 keeps them in LDS (the block
    // loop reads one head's at a time, so the accumulators fit the VGPRs)
    float qs[HPK];   // the scale of head h's scores (undoes the query's power of two)
    const float *q = qkv + (size_t)tq * row_stride;
#pragma unroll
    for (int h = 0; h < HPK; h++) {
        float x[4][8], mx = 0.0f;
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            const float4 *qp = (const float4 *)(q + (size_t)(g * HPK + h) * ATT_HD + 32 * kk + 8 * grp);
            const float4 a = qp[0], b = qp[1];
            x[kk][0] = a.x; x[kk][1] = a.y; x[kk][2] = a.z; x[kk][3] = a.w;
            x[kk][4] = b.x; x[kk][5] = b.y; x[kk][6] = b.z; x[kk][7] = b.w;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                x[kk][i] *= qscale;
                mx = fmaxf(mx, fabsf(x[kk][i]));
            }
        }
        mx = lanes4_max(mx);   // the token's 128 dims sit in lanes n + 16 j
        int e = 0;
        if (mx > 0.0f && __builtin_isfinite(mx)) (void)frexpf(mx, &e);
        const float up = ldexpf(1.0f, 14 - e);
        qs[h] = ldexpf(1.0f, e - 14);
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            h8 qh, ql;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float v = x[kk][i] * up;
                const _Float16 hi = (_Float16)v;
                qh[i] = hi;
                ql[i] = (_Float16)(v - (float)hi);
            }
            if (wv == 0) {
                qop[((h * 4 + kk) * 2) * 64 + l] = qh;
                qop[((h * 4 + kk) * 2 + 1) * 64 + l] = ql;
            }
        }
    }
    __syncthreads();   // the Q^T operands are in LDS
    f4 o[HPK][8];
    float m[HPK], ls[HPK];
#pragma unroll
    for (int h = 0; h < HPK; h++) {
        m[h] = -__builtin_inff();
        ls[h] = 0.0f;
#pragma unroll
        for (int dt = 0; dt < 8; dt++) o[h][dt] = f4{0.f, 0.f, 0.f, 0.f};
    }
    auto process = [&](uint32_t blk, const h8 (&ka)[2][4], const h8 (&vr)[2][4]) {
        const uint32_t c0 = 32 * blk;
        // this wave's V^T (the wave's LDS operations run in order: the
        // previous block's reads come before these writes)
        wave_lds_order();
#pragma unroll
        for (int half = 0; half < 2; half++)
#pragma unroll
            for (int d = 0; d < 8; d++)
                *(h4 *)(vt + (8 * n + d) * ATTM_LD + 16 * half + 4 * grp) =
                    h4{vr[half][0][d], vr[half][1][d], vr[half][2][d], vr[half][3][d]};
        wave_lds_order();
#pragma unroll
        for (int h = 0; h < HPK; h++) {
            h8 qh[4], ql[4];
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                qh[kk] = qop[((h * 4 + kk) * 2) * 64 + l];
                ql[kk] = qop[((h * 4 + kk) * 2 + 1) * 64 + l];
            }
            f4 sc[2];
#pragma unroll
            for (int kt = 0; kt < 2; kt++) {
                sc[kt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kk = 0; kk < 4; kk++) {
                    sc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[kt][kk], qh[kk], sc[kt], 0, 0, 0);
                    sc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[kt][kk], ql[kk], sc[kt], 0, 0, 0);
                }
            }
            // lane l: sc[kt][r] = score of key c0 + 16 kt + 4 grp + r for its token
            float bm = -__builtin_inff();
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    sc[kt][r] *= qs[h];
                    if (c0 + 16 * kt + 4 * grp + r > tpos) sc[kt][r] = -__builtin_inff();
                    bm = fmaxf(bm, sc[kt][r]);
                }
            bm = lanes4_max(bm);
            // Lazy reference max: it moves only when the block's max passes it
            // by more than 3 (so P <= 8 and P * 2^12 stays inside f16), which
            // after the first blocks is rare, and the accumulators are then
            // rescaled in a branch the whole wave skips otherwise.  -inf while
            // none of this wave's blocks so far holds a key of the token's
            // range (a wave's first block may lie past the token).
            const float mo = m[h];
            const bool upd = bm > mo + 3.0f;   // -inf + 3 = -inf: a first finite block moves it
            const float mn = upd ? bm : mo;
            const bool none = mn == -__builtin_inff();
            const float cf = upd && mo != -__builtin_inff() ? exp2f(mo - mn) : 1.0f;
            if (__builtin_amdgcn_ballot_w64(cf != 1.0f)) {
#pragma unroll
                for (int dt = 0; dt < 8; dt++) o[h][dt] = o[h][dt] * cf;
            }
            float ps = 0.0f;
            h8 pb, pl;
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float p = none ? 0.0f : exp2f(sc[kt][r] - mn), pp = p * ATTM_PS;
                    ps += p;
                    const _Float16 hi = (_Float16)pp;
                    pb[4 * kt + r] = hi;
                    pl[4 * kt + r] = (_Float16)(pp - (float)hi);
                }
            ps = lanes4_sum(ps);
            ls[h] = fmaf(ls[h], cf, ps);
            m[h] = mn;
            // V^T operands of the 8 dim tiles read first, then the 8 P-hi
            // MFMAs and the 8 P-lo MFMAs (each accumulator takes hi then lo)
            h8 av[8];
#pragma unroll
            for (int dt = 0; dt < 8; dt++) {
                const _Float16 *vrow = vt + (16 * dt + n) * ATTM_LD;
                const h4 a0 = *(const h4 *)(vrow + 4 * grp), a1 = *(const h4 *)(vrow + 16 + 4 * grp);
                av[dt] = h8{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
            }
#pragma unroll
            for (int dt = 0; dt < 8; dt++) o[h][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[dt], pb, o[h][dt], 0, 0, 0);
#pragma unroll
            for (int dt = 0; dt < 8; dt++) o[h][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[dt], pl, o[h][dt], 0, 0, 0);
        }
    };
    if constexpr (HPK <= 3) {
        // two register sets (HPK = 4 would spill: its accumulators take 32
        // registers more)
        h8 kaB[2][4], vrB[2][4];
        uint32_t blk = wv;
        while (blk < nblk) {
            load_blk(min(blk + ATTM_WAVES, nblk - 1), kaB, vrB);   // past the last block: a repeat, unused
            process(blk, kaA, vrA);
            blk += ATTM_WAVES;
            if (blk >= nblk) break;
            load_blk(min(blk + ATTM_WAVES, nblk - 1), kaA, vrA);
            process(blk, kaB, vrB);
            blk += ATTM_WAVES;
        }
    } else {
        for (uint32_t blk = wv; blk < nblk; blk += ATTM_WAVES) {
            if (blk != wv) load_blk(blk, kaA, vrA);
            process(blk, kaA, vrA);
        }
    }
    // merge the waves: wave w's output rows (token, dims) and its max / sum
    // per (head, token); a wave without blocks holds max -inf, sum 0
    __syncthreads();   // every wave is done with its V^T
#pragma unroll
    for (int h = 0; h < HPK; h++) {
        float *orow = mo + ((size_t)(wv * HPK + h) * 16 + n) * ATTM_OLD;
#pragma unroll
        for (int dt = 0; dt < 8; dt++)
            *(float4 *)(orow + 16 * dt + 4 * grp) = make_float4(o[h][dt][0], o[h][dt][1], o[h][dt][2], o[h][dt][3]);
        if (grp == 0) {
            mml[((wv * HPK + h) * 16 + n) * 2] = m[h];
            mml[((wv * HPK + h) * 16 + n) * 2 + 1] = ls[h];
        }
    }
    __syncthreads();
    // per (head, token): the waves' weights exp2(m_w - M) and the output
    // scale 1 / (PS L), once (L summed over the waves in order)
    if (threadIdx.x < HPK * 16) {
        const uint32_t ht = threadIdx.x, h = ht % HPK, t = ht / HPK;
        float M = -__builtin_inff();
#pragma unroll
        for (uint32_t w = 0; w < ATTM_WAVES; w++) M = fmaxf(M, mml[((w * HPK + h) * 16 + t) * 2]);
        float L = 0.0f;
#pragma unroll
        for (uint32_t w = 0; w < ATTM_WAVES; w++) {
            const float c = safe_scale(mml[((w * HPK + h) * 16 + t) * 2], M);   // 0 for a wave without rows
            L = fmaf(mml[((w * HPK + h) * 16 + t) * 2 + 1], c, L);
            mcw[ht * (ATTM_WAVES + 1) + w] = c;
        }
        mcw[ht * (ATTM_WAVES + 1) + ATTM_WAVES] = (1.0f / ATTM_PS) / L;
    }
    __syncthreads();
    // four dims a thread: the waves' outputs weighted and added in wave order
    const size_t qd = (size_t)gridDim.x * HPK * ATT_HD;
    for (uint32_t i = threadIdx.x; i < HPK * 16 * ATT_HD / 4; i += 64 * ATTM_WAVES) {
        const uint32_t d = 4 * (i % (ATT_HD / 4)), ht = i / (ATT_HD / 4), h = ht % HPK, t = ht / HPK;   // dims fastest
        const uint32_t tk = tb * 16 + t;
        const float *cw = mcw + ht * (ATTM_WAVES + 1);
        f4 O = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (uint32_t w = 0; w < ATTM_WAVES; w++) {
            const float c = cw[w];
            const f4 ow = *(const f4 *)(mo + ((size_t)(w * HPK + h) * 16 + t) * ATTM_OLD + d);
#pragma unroll
            for (int e = 0; e < 4; e++) O[e] = fmaf(ow[e], c, O[e]);
        }
        if (tk < rows) {
            const size_t oi = (size_t)tk * qd + (size_t)(g * HPK + h) * ATT_HD + d;
            const float sc = cw[ATTM_WAVES];
            f4 v;
#pragma unroll
            for (int e = 0; e < 4; e++) v[e] = O[e] * sc;
            if constexpr (F16OUT) {
                asm volatile("" : "+v"(v));   // the f32 results, then their rounding (no mixed-precision fold)
                *(h4 *)((_Float16 *)out + oi) = h4{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
            } else {
                *(f4 *)((float *)out + oi) = v;
            }
        }
    }
}

template <int HPK>
static void go_attn_prefill(const float *qkv, uint32_t row_stride, uint32_t rows, const uint16_t *kc,
                            const uint16_t *vc, void *out, bool out_f16, uint32_t pos0, uint32_t n_kv_heads,
                            float qscale, hipStream_t s, uint32_t hsplit = 1)
{
    const uint32_t kv_stride = n_kv_heads * ATT_HD;
    if constexpr (HPK <= 4) {   // the matrix-core form (its accumulators take 32 registers per head)
        const dim3 grid(n_kv_heads * hsplit, (rows + 15) / 16);
        static_assert(AttmLds<4>::BYTES <= 160 * 1024, "LDS per workgroup");
        if (out_f16)
            hipLaunchKernelGGL((attn_prefill_mfma_kernel<HPK, true>), grid, dim3(64 * ATTM_WAVES), 0, s, qkv,
                               row_stride, kc, vc, out, rows, pos0, kv_stride, qscale, hsplit);
        else
            hipLaunchKernelGGL((attn_prefill_mfma_kernel<HPK, false>), grid, dim3(64 * ATTM_WAVES), 0, s, qkv,
                               row_stride, kc, vc, out, rows, pos0, kv_stride, qscale, hsplit);
        return;
    }
    if (out_f16)
        hipLaunchKernelGGL((attn_prefill_kernel<HPK, true>), dim3(n_kv_heads, rows), dim3(256), 0, s, qkv, row_stride,
                           kc, vc, out, pos0, kv_stride, qscale);
    else
        hipLaunchKernelGGL((attn_prefill_kernel<HPK, false>), dim3(n_kv_heads, rows), dim3(256), 0, s, qkv,
                           row_stride, kc, vc, out, pos0, kv_stride, qscale);
}

hipError_t launch_attention_prefill(const float *qkv, uint32_t row_stride, uint32_t rows, const uint16_t *kc,
                                    const uint16_t *vc, void *out, bool out_f16, uint32_t pos0, uint32_t n_kv_heads,
                                    uint32_t heads_per_kv, hipStream_t s)
{
    if (rows == 0) return hipSuccess;
    const float qscale = (float)(1.4426950408889634 / sqrt((double)ATT_HD));   // log2(e) / sqrt(head_dim)
    // a short prompt's workgroups (KV head, 16 tokens) leave CUs idle: then
    // one workgroup per query head (the same arithmetic per head, bitwise
    // the grouped form; 128 rows x 8 x 3 heads: 7.6 instead of 12.2 us),
    // else the KV group's heads share every K/V block in one workgroup
    // (512 rows: 22.4 against 30.8 us split)
    const uint64_t tgroups = (rows + 15) / 16;
    if (heads_per_kv > 1 && heads_per_kv <= 4 && (uint64_t)n_kv_heads * heads_per_kv * tgroups <= device_cu_count()) {
        go_attn_prefill<1>(qkv, row_stride, rows, kc, vc, out, out_f16, pos0, n_kv_heads, qscale, s, heads_per_kv);
        return hipGetLastError();
    }
#define RRR_ATTP_CASE(H) \
    case H: go_attn_prefill<H>(qkv, row_stride, rows, kc, vc, out, out_f16, pos0, n_kv_heads, qscale, s); break;
    switch (heads_per_kv) {
        RRR_ATTP_CASE(1) RRR_ATTP_CASE(2) RRR_ATTP_CASE(3) RRR_ATTP_CASE(4)
        RRR_ATTP_CASE(5) RRR_ATTP_CASE(6) RRR_ATTP_CASE(7) RRR_ATTP_CASE(8)
    default: return hipErrorInvalidValue;
    }
#undef RRR_ATTP_CASE
    return hipGetLastError();
}

}  // namespace rrr
