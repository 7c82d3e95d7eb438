// attn_static.hip -- decode attention that allocates nothing: its split
// partials and arrival counters live in a file-scope device array instead of
// a buffer the context allocates.  For callers that may not allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc).  Same kernels and launch plan as rrr_attention, so the
// results are the same bits for the same seq_len.
#include "rrr_hip.h"

#include <hip/hip_runtime.h>

#include <mutex>

#include "internal.h"

namespace rrr {

// Held by every device the library runs on until the process ends.  In host
// code `scratch` names a host-side stand-in, not the device copy: host code
// uses only the address hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) uint8_t scratch[ATT_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[MAX_DEVICES];   // device address of `scratch`, per device
}  // namespace

// The device address of this device's `scratch`, looked up once per device
// with that device current (rrr_init calls it for its device; the entry
// point on its first call on a device).
int attention_static_setup(int dev, void **out)
{
    *out = nullptr;
    if (dev < 0 || dev >= MAX_DEVICES) return set_error(RRR_ERR_NO_DEVICE, "attention scratch: device index out of range");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return set_error(RRR_ERR_HIP, "attention scratch: hipGetSymbolAddress failed");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return RRR_OK;
}

}  // namespace rrr

using namespace rrr;

extern "C" int rrr_attention_noalloc(const float *q, const uint16_t *k_cache, const uint16_t *v_cache, float *out,
                                     uint32_t seq_len, uint32_t n_kv_heads, uint32_t heads_per_kv, uint32_t head_dim,
                                     void *stream)
{
    if (!q || !k_cache || !v_cache || !out) return set_error(RRR_ERR_NULL, "rrr_attention_noalloc: null pointer");
    if (head_dim != ATT_HD) return set_error(RRR_ERR_UNSUPPORTED, "rrr_attention_noalloc: head_dim must be 128");
    if (seq_len == 0 || n_kv_heads == 0 || heads_per_kv == 0)
        return set_error(RRR_ERR_BAD_SHAPE, "rrr_attention_noalloc: seq_len, n_kv_heads and heads_per_kv must be positive");
    // the scratch array holds the partials of ATT_SPLITS_MAX splits of
    // ATT_HEADS_MAX query heads: larger problems are refused
    if (seq_len > ATT_SEQ_MAX)
        return set_error(RRR_ERR_UNSUPPORTED, "rrr_attention_noalloc: seq_len exceeds 2048 (the scratch array's limit)");
    if (heads_per_kv > 8 || (uint64_t)n_kv_heads * heads_per_kv > ATT_HEADS_MAX)
        return set_error(RRR_ERR_UNSUPPORTED,
                         "rrr_attention_noalloc: at most 8 query heads per KV head and 64 query heads "
                         "(the scratch array's limit)");
    if (((uintptr_t)q | (uintptr_t)out | (uintptr_t)k_cache | (uintptr_t)v_cache) & 15)
        return set_error(RRR_ERR_INVALID_ARG, "rrr_attention_noalloc: q, out and the caches must be 16-byte aligned");
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return set_error(RRR_ERR_HIP, "rrr_attention_noalloc: hipGetDevice failed");
    void *ptr = nullptr;
    if (int rc = attention_static_setup(dev, &ptr)) return rc;
    hipStream_t s = (hipStream_t)stream;
    // the arrival counters must start at zero (a fill kernel: no memset
    // node, so the call may be captured into a graph)
    hipError_t e = launch_fill_u32((uint32_t *)ptr, ATT_COUNTER_BYTES / 4, 0u, s);
    if (e == hipSuccess)
        e = launch_attention(q, k_cache, v_cache, out, ptr, seq_len, n_kv_heads, heads_per_kv, device_cu_count(), s);
    if (e != hipSuccess) return set_error(RRR_ERR_HIP, hipGetErrorString(e));
    return set_error(RRR_OK, "");
}
