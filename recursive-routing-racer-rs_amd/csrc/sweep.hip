// sweep.hip -- the decode weight sweep as one persistent launch: the list of
// fused GEMV ops that the reference replays per token through
// dispatch_batch_persistent_v2 (engine.rs:317-370, table built at
// phi4.rs:972-1064) runs inside a single cooperative kernel, one workgroup per
// CU.  Each op is the batch-1 int8-MFMA GEMV body (gemv_mq.h) over the
// workgroup's 16-row tiles; between ops a workgroup publishes a progress flag
// (after its rows are written through to the coherent level) and the next op
// waits until every workgroup's flag has reached it.  The wait comes after
// the op's first tile of weights has been requested, so HBM keeps streaming
// while the previous op's last rows land.  Results are bit-identical to the
// same ops launched one by one (row sums are added in wave order whatever the
// number of waves or workgroups).
#include "gemv_mq.h"

namespace rrr {

struct SweepOpDev {
    GemvArgs a;
    uint32_t variant;
    uint32_t ntiles;
    uint32_t tr;        // rows per tile
    uint32_t pad;
};

// variant = 8 * type index (Q4_K 0, Q5_K 1, Q6_K 2) + 4 * (BPW - 1) + activation
constexpr uint32_t sweep_variant_of(uint32_t type_index, uint32_t bpw, uint32_t act)
{
    return 8 * type_index + 4 * (bpw - 1) + act;
}

// ops[0..nops) in order; epoch = the value every flag is known to be below at
// launch (op i done -> flag = epoch + i + 1)
// flags: gridDim.x rounded up to a multiple of 4, then the error word, then
// the go words (SWEEP_GO_COPIES x SWEEP_GO_STRIDE)
__global__ __launch_bounds__(1024) void sweep_kernel(const SweepOpDev *ops, uint32_t nops, uint32_t *flags,
                                                     uint32_t epoch)
{
    __shared__ uint32_t bail;
    const uint32_t t = threadIdx.x;
    const uint32_t nf = (gridDim.x + 3) & ~3u;
    uint32_t *err = flags + nf, *go = flags + nf + 4;
    if (t == 0) bail = 0;
    __syncthreads();
    for (uint32_t op = 0; op < nops; op++) {
        const SweepOpDev o = ops[op];
        SweepWait sw{flags, go, op ? epoch + op : 0u, err, &bail};
        bool ok;
        const uint32_t v = o.variant;
        switch (v) {
        case sweep_variant_of(1, 1, ACT_RMSNORM): ok = mq_body<MqQ5K, 1, ACT_RMSNORM, true, true>(o.a, o.ntiles, o.tr, sw); break;
        case sweep_variant_of(0, 1, ACT_GQA_V): ok = mq_body<MqQ4K, 1, ACT_GQA_V, true, true>(o.a, o.ntiles, o.tr, sw); break;
        case sweep_variant_of(0, 1, ACT_RMSNORM): ok = mq_body<MqQ4K, 1, ACT_RMSNORM, true, true>(o.a, o.ntiles, o.tr, sw); break;
        case sweep_variant_of(2, 2, ACT_SILU): ok = mq_body<MqQ6K, 2, ACT_SILU, true, true>(o.a, o.ntiles, o.tr, sw); break;
        default: ok = mq_body<MqQ4K, 2, ACT_SILU, true, true>(o.a, o.ntiles, o.tr, sw); break;
        }
        if (!ok) return;
        // this workgroup's rows of the op have been written through: publish
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (t == 0) __hip_atomic_store(flags + blockIdx.x, epoch + op + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Per-op set-up: the variant, the tile count and the LDS the op needs with
// `grid` workgroups of 16 waves; false if the sweep cannot run it.
bool sweep_plan_op(const GemvArgs &a, uint32_t act, uint32_t grid, uint32_t &variant, uint32_t &ntiles, uint32_t &tr,
                   size_t &lds)
{
    if (a.M != 1 || a.K % 256 || a.K == 0 || a.K > 8192 || a.w_bytes + RRR_READ_SLACK >= MQ_OOB) return false;
    const uint32_t ti = a.type == T_Q4_K ? 0 : a.type == T_Q5_K ? 1 : a.type == T_Q6_K ? 2 : 3;
    if (ti == 3 || act > ACT_RMSNORM) return false;
    const uint32_t bpw = a.K <= 16 * 256 ? 1 : 2;
    size_t bytes;
    switch (ti * 2 + bpw - 1) {
    case 0: bytes = MwGeom<MqQ4K, 1>::BYTES; break;
    case 1: bytes = MwGeom<MqQ4K, 2>::BYTES; break;
    case 2: bytes = MwGeom<MqQ5K, 1>::BYTES; break;
    case 3: bytes = MwGeom<MqQ5K, 2>::BYTES; break;
    case 4: bytes = MwGeom<MqQ6K, 1>::BYTES; break;
    default: bytes = MwGeom<MqQ6K, 2>::BYTES; break;
    }
    variant = sweep_variant_of(ti, bpw, act);
    // the kernel carries the decode layer's five forms only (each further form
    // adds register pressure to the one fused kernel)
    if (variant != sweep_variant_of(1, 1, ACT_RMSNORM) && variant != sweep_variant_of(0, 1, ACT_GQA_V) &&
        variant != sweep_variant_of(0, 1, ACT_RMSNORM) && variant != sweep_variant_of(2, 2, ACT_SILU) &&
        variant != sweep_variant_of(0, 2, ACT_SILU))
        return false;
    uint32_t per;
    mq_tiles(a.N, grid, 64, bpw == 1 ? 1u : 16u, tr, ntiles, per);
    lds = 16 * bytes + 16 + (size_t)per * 16 * 64;
    return lds <= 160 * 1024;
}

size_t sweep_op_bytes() { return sizeof(SweepOpDev); }

void sweep_pack_op(void *dst, const GemvArgs &a, uint32_t variant, uint32_t ntiles, uint32_t tr)
{
    SweepOpDev o{a, variant, ntiles, tr, 0u};
    *(SweepOpDev *)dst = o;
}

// Workgroups of the sweep: one per CU when a 1024-thread workgroup with `lds`
// bytes fits there, else 0.
uint32_t sweep_grid(size_t lds)
{
    int per = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, sweep_kernel, 1024, lds) != hipSuccess || per < 1) return 0;
    return device_cus();
}

uint32_t sweep_cus() { return device_cus(); }

size_t sweep_flag_words(uint32_t grid) { return ((grid + 3) & ~3u) + 4 + SWEEP_GO_COPIES * SWEEP_GO_STRIDE; }
size_t sweep_err_word(uint32_t grid) { return (grid + 3) & ~3u; }

hipError_t launch_sweep(const void *ops, uint32_t nops, uint32_t *flags, uint32_t epoch, uint32_t grid, size_t lds,
                        hipStream_t s)
{
    const SweepOpDev *o = (const SweepOpDev *)ops;
    void *args[] = {(void *)&o, (void *)&nops, (void *)&flags, (void *)&epoch};
    return hipLaunchCooperativeKernel((const void *)sweep_kernel, dim3(grid), dim3(1024), args, (unsigned)lds, s);
}

}  // namespace rrr
