// gemv_mfma.hip -- the standalone launch of the batch-1 int8-MFMA GEMV
// (y[n] = sum_k x[k] * W[n][k] for Q4_K / Q5_K / Q6_K rows, phi4.rs:628-630;
// the design is described in gemv_mq.h).
#include "gemv_mq.h"

namespace rrr {

template <class Q, int BPW, int ACT, bool MULTI, int TR, bool PAIR = false, bool ROPE = false, bool ST = false>
__global__ __launch_bounds__(1024) void gemv_mq_kernel(GemvArgs a, uint32_t ntiles, uint32_t tr)
{
    mq_body<Q, BPW, ACT, MULTI, TR, PAIR, ROPE, ST>(a, ntiles, tr);
}

// The multi-token form, MT rows of x per weight stream, in workgroups of at
// most NTH threads (768 = 12 waves leaves 168 registers a lane where 1024
// threads leave 128, which MT = 4 and 8 exceed).
template <class Q, int BPW, bool MULTI, int MT, int NTH>
__global__ __launch_bounds__(NTH) void gemv_mq_tokens_kernel(GemvArgs a, uint32_t ntiles, uint32_t tr)
{
    mq_body<Q, BPW, ACT_PLAIN, MULTI, 16, false, false, false, MT>(a, ntiles, tr);
}

// The launch's grid and waves per workgroup (reported to the stamped launch).
struct MqShape {
    uint32_t grid, waves;
};

// Super-blocks per wave and waves per workgroup (at least 4; waves past the
// last super-block only encode).
// Up to one workgroup per CU, each taking its tiles as far as its row
// partials fit in LDS.  Tiles split evenly over the CUs (a wave issues only
// the load slots its tile height needs, so short tiles cost no empty loads).
template <class Q, int BPW>
static void mq_plan(const GemvArgs &a, uint32_t &W, uint32_t &grid, size_t &lds, uint32_t &tr, uint32_t &ntiles)
{
    using G = MwGeom<Q, BPW>;
    W = mq_waves(a.K, BPW);
    const size_t fixed = W * G::BYTES + 64;
    const uint32_t per_max = (uint32_t)((160 * 1024 - fixed) / (W * 64));
    uint32_t per;
    mq_tiles(a.N, device_cus(), per_max, 1u, tr, ntiles, per);
    grid = (ntiles + per - 1) / per;
    lds = fixed + (size_t)per * W * 64;
}

template <class Q, int BPW, int ACT, int TR, bool ST>
static void launch_mq(const GemvArgs &a, uint32_t W, uint32_t grid, size_t lds, uint32_t tr, uint32_t ntiles,
                      hipStream_t s)
{
    if (grid == ntiles)
        hipLaunchKernelGGL((gemv_mq_kernel<Q, BPW, ACT, false, TR, false, false, ST>), dim3(grid), dim3(64 * W), lds, s,
                           a, ntiles, tr);
    else
        hipLaunchKernelGGL((gemv_mq_kernel<Q, BPW, ACT, true, TR, false, false, ST>), dim3(grid), dim3(64 * W), lds, s,
                           a, ntiles, tr);
}

// The silu pair form (a.pair): per 16 output rows a gate tile and its up
// tile, fused RMSNorm; always the persistent form (a workgroup holds both
// tiles of a pair).
template <class Q, int BPW, bool ST = false>
static hipError_t go_mq_pair(const GemvArgs &a, hipStream_t s, MqShape *sh = nullptr)
{
    using G = MwGeom<Q, BPW>;
    const uint32_t W = mq_waves(a.K, BPW);
    const size_t fixed = W * G::BYTES + 64;
    const uint32_t per_max = (uint32_t)((160 * 1024 - fixed) / (W * 64)) / 2;   // pairs: two tiles each
    if (per_max == 0) return hipErrorInvalidValue;
    const uint32_t npairs = (a.N + 15) / 16, cus = device_cus();
    const uint32_t per = min((npairs + cus - 1) / cus, per_max);
    const uint32_t grid = (npairs + per - 1) / per;
    const size_t lds = fixed + (size_t)2 * per * W * 64;
    hipLaunchKernelGGL((gemv_mq_kernel<Q, BPW, ACT_RMSNORM, true, 16, true, false, ST>), dim3(grid), dim3(64 * W), lds,
                       s, a, npairs, 16u);
    if (sh) *sh = MqShape{grid, W};
    return hipGetLastError();
}

template <class Q, int BPW, int ACT, bool ST = false>
static hipError_t go_mq(const GemvArgs &a, hipStream_t s, MqShape *sh = nullptr)
{
    static_assert(16 * MwGeom<Q, BPW>::BYTES + 64 + 16 * 64 <= 160 * 1024, "LDS per workgroup");
    uint32_t W, grid, tr, ntiles;
    size_t lds;
    mq_plan<Q, BPW>(a, W, grid, lds, tr, ntiles);
    // slot sets for the tile heights of the decode shapes (N = 5120: 10 rows,
    // N = 3072: 12 rows, larger N: 16 rows)
    if (tr <= 10)
        launch_mq<Q, BPW, ACT, 10, ST>(a, W, grid, lds, tr, ntiles, s);
    else if (tr <= 12)
        launch_mq<Q, BPW, ACT, 12, ST>(a, W, grid, lds, tr, ntiles, s);
    else
        launch_mq<Q, BPW, ACT, 16, ST>(a, W, grid, lds, tr, ntiles, s);
    if (sh) *sh = MqShape{grid, W};
    return hipGetLastError();
}

// The QKV GEMV with rope_kv_store in its epilogue (fused RMSNorm): plain
// tiles of an even height, so that a RoPE pair never straddles two tiles.
template <class Q, int BPW>
static hipError_t go_mq_rope(const GemvArgs &a, hipStream_t s)
{
    uint32_t W, grid, tr, ntiles;
    size_t lds;
    mq_plan<Q, BPW>(a, W, grid, lds, tr, ntiles);
    if (tr % 2) return hipErrorNotSupported;
    lds += 4 * (size_t)a.rope.rope_dim;   // the rotation coefficients
    if (lds > 160 * 1024) return hipErrorNotSupported;
    const bool multi = grid != ntiles;
    if (tr <= 10) {
        if (multi)
            hipLaunchKernelGGL((gemv_mq_kernel<Q, BPW, ACT_RMSNORM, true, 10, false, true>), dim3(grid), dim3(64 * W),
                               lds, s, a, ntiles, tr);
        else
            hipLaunchKernelGGL((gemv_mq_kernel<Q, BPW, ACT_RMSNORM, false, 10, false, true>), dim3(grid), dim3(64 * W),
                               lds, s, a, ntiles, tr);
    } else {
        if (multi)
            hipLaunchKernelGGL((gemv_mq_kernel<Q, BPW, ACT_RMSNORM, true, 16, false, true>), dim3(grid), dim3(64 * W),
                               lds, s, a, ntiles, tr);
        else
            hipLaunchKernelGGL((gemv_mq_kernel<Q, BPW, ACT_RMSNORM, false, 16, false, true>), dim3(grid), dim3(64 * W),
                               lds, s, a, ntiles, tr);
    }
    return hipGetLastError();
}

template <class Q, int ACT, bool ST>
static hipError_t go_mq_k(const GemvArgs &a, hipStream_t s, MqShape *sh)
{
    return a.K <= 16 * 256 ? go_mq<Q, 1, ACT, ST>(a, s, sh) : go_mq<Q, 2, ACT, ST>(a, s, sh);
}

template <class Q, bool ST = false>
static hipError_t go_mq_act(const GemvArgs &a, uint32_t act, hipStream_t s, MqShape *sh = nullptr)
{
    switch (act) {
    case ACT_PLAIN: return go_mq_k<Q, ACT_PLAIN, ST>(a, s, sh);
    case ACT_SILU: return go_mq_k<Q, ACT_SILU, ST>(a, s, sh);
    case ACT_GQA_V: return go_mq_k<Q, ACT_GQA_V, ST>(a, s, sh);
    case ACT_RMSNORM: return go_mq_k<Q, ACT_RMSNORM, ST>(a, s, sh);
    default: return hipErrorInvalidValue;
    }
}

// The multi-token form: a.M <= MT rows of x through the same weight stream
// (plain activations, optional residual).  Tiles of up to 16 rows; each
// workgroup's LDS holds MT encoded slices and MT row partials per tile.
template <class Q, int BPW, int MT>
static bool mq_tokens_plan(const GemvArgs &a, uint32_t &W, uint32_t &grid, size_t &lds, uint32_t &tr,
                           uint32_t &ntiles)
{
    using G = MwGeom<Q, BPW, MT>;
    W = mq_waves(a.K, BPW);
    const size_t fixed = W * G::BYTES + 64, per_tile = (size_t)W * 64 * MT;
    if (fixed + per_tile > 160 * 1024) return false;
    const uint32_t per_max = (uint32_t)((160 * 1024 - fixed) / per_tile);
    uint32_t per;
    mq_tiles(a.N, device_cus(), per_max, 1u, tr, ntiles, per);
    grid = (ntiles + per - 1) / per;
    lds = fixed + (size_t)per * per_tile;
    return true;
}

template <class Q, int BPW, int MT, int NTH>
static hipError_t go_mq_tokens_b(const GemvArgs &a, hipStream_t s, bool launch)
{
    uint32_t W, grid, tr, ntiles;
    size_t lds;
    if (!mq_tokens_plan<Q, BPW, MT>(a, W, grid, lds, tr, ntiles) || 64 * W > NTH) return hipErrorNotSupported;
    if (!launch) return hipSuccess;
    if (grid == ntiles)
        hipLaunchKernelGGL((gemv_mq_tokens_kernel<Q, BPW, false, MT, NTH>), dim3(grid), dim3(64 * W), lds, s, a, ntiles,
                           tr);
    else
        hipLaunchKernelGGL((gemv_mq_tokens_kernel<Q, BPW, true, MT, NTH>), dim3(grid), dim3(64 * W), lds, s, a, ntiles,
                           tr);
    return hipGetLastError();
}

// K <= 3072 (at most 12 waves): 2 or 4 tokens a launch (8 ran slower than
// the skinny kernel: every token's A and C operands are LDS reads per
// MFMA); K <= 8192 (16 waves of two super-blocks): 2 (more tokens would
// spill at 128 registers)
template <class Q>
static hipError_t go_mq_tokens(const GemvArgs &a, hipStream_t s, bool launch)
{
    if (a.K <= 12 * 256) {
        if (a.M <= 2) return go_mq_tokens_b<Q, 1, 2, 768>(a, s, launch);
        return go_mq_tokens_b<Q, 1, 4, 768>(a, s, launch);
    }
    if (a.M <= 2) return go_mq_tokens_b<Q, 2, 2, 1024>(a, s, launch);
    return hipErrorNotSupported;
}

static hipError_t mq_tokens(const GemvArgs &a, hipStream_t s, bool launch)
{
    if (a.M < 2 || a.M > MQ_TOKENS_MAX || a.K > 8192 || a.w_bytes + RRR_READ_SLACK >= MQ_OOB) return hipErrorNotSupported;
    switch (a.type) {
    case T_Q4_K: return go_mq_tokens<MqQ4K>(a, s, launch);
    case T_Q5_K: return go_mq_tokens<MqQ5K>(a, s, launch);
    case T_Q6_K: return go_mq_tokens<MqQ6K>(a, s, launch);
    default: return hipErrorNotSupported;
    }
}

bool gemv_mq_tokens_supported(const GemvArgs &a) { return mq_tokens(a, nullptr, false) == hipSuccess; }

hipError_t launch_gemv_mq_tokens(const GemvArgs &a, hipStream_t s) { return mq_tokens(a, s, true); }

uint32_t device_cu_count() { return device_cus(); }

bool gemv_mfma_supported(const GemvArgs &a)
{
    if (a.M != 1 || (a.type != T_Q4_K && a.type != T_Q5_K && a.type != T_Q6_K) || a.K > 8192) return false;
    return a.w_bytes + RRR_READ_SLACK < MQ_OOB;
}

hipError_t launch_gemv_mfma(const GemvArgs &a, uint32_t act, hipStream_t s)
{
    if (a.rope_on) {
        if (act != ACT_RMSNORM || a.pair || a.residual || a.N % 2) return hipErrorNotSupported;
        const bool one = a.K <= 16 * 256;
        switch (a.type) {
        case T_Q4_K: return one ? go_mq_rope<MqQ4K, 1>(a, s) : go_mq_rope<MqQ4K, 2>(a, s);
        case T_Q5_K: return one ? go_mq_rope<MqQ5K, 1>(a, s) : go_mq_rope<MqQ5K, 2>(a, s);
        case T_Q6_K: return one ? go_mq_rope<MqQ6K, 1>(a, s) : go_mq_rope<MqQ6K, 2>(a, s);
        default: return hipErrorNotSupported;
        }
    }
    if (a.pair) {
        if (act != ACT_RMSNORM || a.residual) return hipErrorInvalidValue;
        const bool one = a.K <= 16 * 256;
        switch (a.type) {
        case T_Q4_K: return one ? go_mq_pair<MqQ4K, 1>(a, s) : go_mq_pair<MqQ4K, 2>(a, s);
        case T_Q5_K: return one ? go_mq_pair<MqQ5K, 1>(a, s) : go_mq_pair<MqQ5K, 2>(a, s);
        case T_Q6_K: return one ? go_mq_pair<MqQ6K, 1>(a, s) : go_mq_pair<MqQ6K, 2>(a, s);
        default: return hipErrorInvalidValue;
        }
    }
    switch (a.type) {
    case T_Q4_K: return go_mq_act<MqQ4K>(a, act, s);
    case T_Q5_K: return go_mq_act<MqQ5K>(a, act, s);
    case T_Q6_K: return go_mq_act<MqQ6K>(a, act, s);
    default: return hipErrorInvalidValue;
    }
}

// The launch launch_gemv_mfma makes for `a` (plain and pair forms; not the
// RoPE epilogue), instantiated with phase timestamps into a.stamps.
hipError_t launch_gemv_mfma_stamped(const GemvArgs &a, uint32_t act, hipStream_t s, uint32_t &grid, uint32_t &waves)
{
    if (a.rope_on || !a.stamps) return hipErrorNotSupported;
    MqShape sh{0, 0};
    hipError_t e;
    if (a.pair) {
        if (act != ACT_RMSNORM || a.residual) return hipErrorInvalidValue;
        const bool one = a.K <= 16 * 256;
        switch (a.type) {
        case T_Q4_K: e = one ? go_mq_pair<MqQ4K, 1, true>(a, s, &sh) : go_mq_pair<MqQ4K, 2, true>(a, s, &sh); break;
        case T_Q5_K: e = one ? go_mq_pair<MqQ5K, 1, true>(a, s, &sh) : go_mq_pair<MqQ5K, 2, true>(a, s, &sh); break;
        case T_Q6_K: e = one ? go_mq_pair<MqQ6K, 1, true>(a, s, &sh) : go_mq_pair<MqQ6K, 2, true>(a, s, &sh); break;
        default: return hipErrorInvalidValue;
        }
    } else {
        switch (a.type) {
        case T_Q4_K: e = go_mq_act<MqQ4K, true>(a, act, s, &sh); break;
        case T_Q5_K: e = go_mq_act<MqQ5K, true>(a, act, s, &sh); break;
        case T_Q6_K: e = go_mq_act<MqQ6K, true>(a, act, s, &sh); break;
        default: return hipErrorInvalidValue;
        }
    }
    grid = sh.grid;
    waves = sh.waves;
    return e;
}

}  // namespace rrr
