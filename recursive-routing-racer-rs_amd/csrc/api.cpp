// api.cpp -- the C ABI of librrr_hip.so (declared in include/rrr_hip.h).
//
// Every entry point validates its arguments completely before the first HIP
// call, so a validation-only context (RRR_DEVICE_NONE) exercises all error
// paths on a machine without a GPU.
#include "rrr_hip.h"
#include "rrr_gguf.h"
#include "rrr_probe.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_set>
#include <vector>

#include "internal.h"

using namespace rrr;

namespace {

constexpr uint32_t CTX_MAGIC = 0x52525243u, BUF_MAGIC = 0x52525242u, GRAPH_MAGIC = 0x52525247u;

thread_local std::string g_err;
std::mutex g_mu;
std::unordered_set<rrr_ctx *> g_ctxs;

int fail(int code, const char *fmt, ...)
{
    char msg[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(msg, sizeof msg, fmt, ap);
    va_end(ap);
    g_err = msg;
    return code;
}

int ok()
{
    g_err.clear();
    return RRR_OK;
}

}  // namespace

namespace rrr {
int set_error(int code, const char *msg)
{
    if (code == RRR_OK) return ok();
    g_err = msg;
    return code;
}
}  // namespace rrr

struct rrr_buf {
    uint32_t magic;
    rrr_ctx *ctx;
    void *ptr;        // device pointer (nullptr in a validation-only context)
    uint64_t bytes;
    rrr_buf *parent;  // non-null for views
};

struct rrr_graph {
    uint32_t magic;
    rrr_ctx *ctx;
    hipGraph_t graph;
    hipGraphExec_t exec;
};

struct rrr_ctx {
    uint32_t magic;
    int device;
    bool nodevice;
    bool async;
    bool capturing;
    bool timer_started;
    hipStream_t stream;
    hipEvent_t ev0, ev1;
    void *scratch;      // argmax partial candidates
    void *att_scratch;  // attention: per-KV-head counters (zero between calls) and split partials
    void *gemm_ws;      // GEMM_WS_BYTES: prefill GEMM partials of split K; the skinny GEMV's encoded
                        // activations; the split-K logits' partials (stream order keeps the users apart)
    void *logits_cnt;   // split-K logits: per-slab counters (zero between calls)
    std::unordered_set<rrr_buf *> bufs;
    std::unordered_set<rrr_graph *> graphs;
};

namespace {

int check_ctx(rrr_ctx *ctx)
{
    if (!ctx) return fail(RRR_ERR_NULL, "null context");
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_ctxs.count(ctx) || ctx->magic != CTX_MAGIC) return fail(RRR_ERR_STALE, "context already destroyed");
    return RRR_OK;
}

int check_buf(rrr_ctx *ctx, const rrr_buf *b, const char *what)
{
    if (!b) return fail(RRR_ERR_NULL, "%s: null buffer", what);
    if (!ctx->bufs.count(const_cast<rrr_buf *>(b)) || b->magic != BUF_MAGIC)
        return fail(RRR_ERR_STALE, "%s: buffer already freed or not owned by this context", what);
    return RRR_OK;
}

int need(const rrr_buf *b, uint64_t bytes, const char *what)
{
    if (b->bytes < bytes)
        return fail(RRR_ERR_SHORT_BUFFER, "%s: buffer holds %llu bytes, the op needs %llu", what,
                    (unsigned long long)b->bytes, (unsigned long long)bytes);
    return RRR_OK;
}

int need_f32(const rrr_buf *b, uint64_t count, const char *what)
{
    if (int rc = need(b, count * 4, what)) return rc;
    if (b->ptr && ((uintptr_t)b->ptr & 15))
        return fail(RRR_ERR_INVALID_ARG, "%s: f32 vector buffers must be 16-byte aligned", what);
    return RRR_OK;
}

bool valid_type(uint32_t t) { return t == RRR_TYPE_F32 || t == RRR_TYPE_Q4_K || t == RRR_TYPE_Q5_K || t == RRR_TYPE_Q6_K; }

int check_shape(uint32_t type, uint32_t K, uint32_t N)
{
    if (!valid_type(type)) return fail(RRR_ERR_BAD_TYPE, "ggml type %u is not one of 0, 12, 13, 14", type);
    if (K == 0 || N == 0) return fail(RRR_ERR_BAD_SHAPE, "K and N must be positive (K=%u N=%u)", K, N);
    if (K % 256) return fail(RRR_ERR_BAD_SHAPE, "K=%u is not a multiple of the 256-element super-block", K);
    if (K > 65536) return fail(RRR_ERR_UNSUPPORTED, "K=%u exceeds 65536", K);
    return RRR_OK;
}

// Launch epilogue: report launch errors, then wait unless async or capturing.
int finish(rrr_ctx *ctx, hipError_t e, const char *what)
{
    if (e != hipSuccess) return fail(RRR_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    if (!ctx->async && !ctx->capturing) {
        e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) return fail(RRR_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    }
    return ok();
}

int device_ready(rrr_ctx *ctx)
{
    if (ctx->nodevice) return fail(RRR_ERR_NO_DEVICE, "validation-only context has no device");
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return fail(RRR_ERR_HIP, "hipSetDevice: %s", hipGetErrorString(e));
    return RRR_OK;
}

#define TRY(x)                     \
    do {                           \
        int rc_ = (x);             \
        if (rc_ != RRR_OK) return rc_; \
    } while (0)

}  // namespace

extern "C" {

int rrr_abi_version(void) { return RRR_ABI_VERSION; }

const char *rrr_last_error(void) { return g_err.c_str(); }

int rrr_device_count(void)
{
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

uint64_t rrr_tensor_bytes(uint32_t type, uint32_t K, uint32_t N)
{
    if (!valid_type(type) || K == 0 || K % 256) return 0;
    return (uint64_t)N * (K / 256) * block_bytes(type);
}

int rrr_init(int device, rrr_ctx **out)
{
    if (!out) return fail(RRR_ERR_NULL, "rrr_init: null output pointer");
    *out = nullptr;
    if (device < RRR_DEVICE_NONE) return fail(RRR_ERR_INVALID_ARG, "rrr_init: device %d", device);
    rrr_ctx *ctx = new rrr_ctx();
    ctx->magic = CTX_MAGIC;
    ctx->device = device;
    ctx->nodevice = device == RRR_DEVICE_NONE;
    ctx->async = ctx->capturing = ctx->timer_started = false;
    ctx->stream = nullptr;
    ctx->ev0 = ctx->ev1 = nullptr;
    ctx->scratch = ctx->att_scratch = ctx->gemm_ws = ctx->logits_cnt = nullptr;
    if (!ctx->nodevice) {
        int n = rrr_device_count();
        if (device >= n) {
            delete ctx;
            return fail(RRR_ERR_NO_DEVICE, "rrr_init: device %d requested, %d visible", device, n);
        }
        hipError_t e = hipSetDevice(device);
        if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
        if (e == hipSuccess) e = hipEventCreate(&ctx->ev0);
        if (e == hipSuccess) e = hipEventCreate(&ctx->ev1);
        if (e == hipSuccess) e = hipMalloc(&ctx->scratch, argmax_partials_bytes());
        if (e == hipSuccess) e = hipMalloc(&ctx->att_scratch, attention_scratch_bytes());
        if (e == hipSuccess) e = hipMemset(ctx->att_scratch, 0, attention_scratch_bytes());
        if (e == hipSuccess) e = hipMalloc(&ctx->gemm_ws, GEMM_WS_BYTES);
        if (e == hipSuccess) e = hipMalloc(&ctx->logits_cnt, logits_counter_bytes());
        if (e == hipSuccess) e = hipMemset(ctx->logits_cnt, 0, logits_counter_bytes());
        if (e == hipSuccess) e = hipDeviceSynchronize();
        void *static_scratch = nullptr;   // rrr_attention_noalloc's array on this device
        if (e == hipSuccess && attention_static_setup(device, &static_scratch) != RRR_OK) e = hipErrorInvalidSymbol;
        if (e != hipSuccess) {
            if (ctx->logits_cnt) (void)hipFree(ctx->logits_cnt);
            if (ctx->gemm_ws) (void)hipFree(ctx->gemm_ws);
            if (ctx->att_scratch) (void)hipFree(ctx->att_scratch);
            if (ctx->scratch) (void)hipFree(ctx->scratch);
            if (ctx->ev1) (void)hipEventDestroy(ctx->ev1);
            if (ctx->ev0) (void)hipEventDestroy(ctx->ev0);
            if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
            delete ctx;
            return fail(RRR_ERR_HIP, "rrr_init: %s", hipGetErrorString(e));
        }
    }
    {
        std::lock_guard<std::mutex> lk(g_mu);
        g_ctxs.insert(ctx);
    }
    *out = ctx;
    return ok();
}

int rrr_destroy(rrr_ctx *ctx)
{
    TRY(check_ctx(ctx));
    if (!ctx->nodevice) {
        (void)hipSetDevice(ctx->device);
        if (ctx->capturing) {
            hipGraph_t g = nullptr;
            (void)hipStreamEndCapture(ctx->stream, &g);
            if (g) (void)hipGraphDestroy(g);
        }
        (void)hipStreamSynchronize(ctx->stream);
        for (rrr_graph *g : ctx->graphs) {
            (void)hipGraphExecDestroy(g->exec);
            (void)hipGraphDestroy(g->graph);
            g->magic = 0;
            delete g;
        }
        for (rrr_buf *b : ctx->bufs)
            if (!b->parent && b->ptr) (void)hipFree(b->ptr);
        (void)hipFree(ctx->scratch);
        (void)hipFree(ctx->att_scratch);
        (void)hipFree(ctx->gemm_ws);
        (void)hipFree(ctx->logits_cnt);
        (void)hipEventDestroy(ctx->ev0);
        (void)hipEventDestroy(ctx->ev1);
        (void)hipStreamDestroy(ctx->stream);
    } else {
        for (rrr_graph *g : ctx->graphs) delete g;
    }
    for (rrr_buf *b : ctx->bufs) {
        b->magic = 0;
        delete b;
    }
    {
        std::lock_guard<std::mutex> lk(g_mu);
        g_ctxs.erase(ctx);
    }
    ctx->magic = 0;
    delete ctx;
    return ok();
}

// ---- buffers ---------------------------------------------------------------

int rrr_buf_alloc(rrr_ctx *ctx, uint64_t bytes, rrr_buf **out)
{
    TRY(check_ctx(ctx));
    if (!out) return fail(RRR_ERR_NULL, "rrr_buf_alloc: null output pointer");
    *out = nullptr;
    if (bytes == 0) return fail(RRR_ERR_INVALID_ARG, "rrr_buf_alloc: zero bytes");
    if (ctx->capturing) return fail(RRR_ERR_STATE, "rrr_buf_alloc: not allowed during graph capture");
    void *p = nullptr;
    if (!ctx->nodevice) {
        TRY(device_ready(ctx));
        // read slack for kernels, rounded to whole 256-byte lines
        const uint64_t alloc = (bytes + RRR_READ_SLACK + 255) & ~255ull;
        hipError_t e = hipMalloc(&p, alloc);
        if (e != hipSuccess) return fail(RRR_ERR_HIP, "hipMalloc(%llu): %s", (unsigned long long)bytes, hipGetErrorString(e));
    }
    rrr_buf *b = new rrr_buf{BUF_MAGIC, ctx, p, bytes, nullptr};
    ctx->bufs.insert(b);
    *out = b;
    return ok();
}

int rrr_buf_view(rrr_ctx *ctx, rrr_buf *parent, uint64_t offset, uint64_t bytes, rrr_buf **out)
{
    TRY(check_ctx(ctx));
    if (!out) return fail(RRR_ERR_NULL, "rrr_buf_view: null output pointer");
    *out = nullptr;
    TRY(check_buf(ctx, parent, "rrr_buf_view"));
    if (bytes == 0 || offset > parent->bytes || bytes > parent->bytes - offset)
        return fail(RRR_ERR_INVALID_ARG, "rrr_buf_view: range [%llu, +%llu) outside a %llu-byte buffer",
                    (unsigned long long)offset, (unsigned long long)bytes, (unsigned long long)parent->bytes);
    if (offset % 4) return fail(RRR_ERR_INVALID_ARG, "rrr_buf_view: offset must be a multiple of 4");
    rrr_buf *root = parent->parent ? parent->parent : parent;
    void *p = parent->ptr ? (void *)((char *)parent->ptr + offset) : nullptr;
    rrr_buf *b = new rrr_buf{BUF_MAGIC, ctx, p, bytes, root};
    ctx->bufs.insert(b);
    *out = b;
    return ok();
}

int rrr_buf_free(rrr_ctx *ctx, rrr_buf *buf)
{
    TRY(check_ctx(ctx));
    TRY(check_buf(ctx, buf, "rrr_buf_free"));
    if (ctx->capturing) return fail(RRR_ERR_STATE, "rrr_buf_free: not allowed during graph capture");
    if (!buf->parent) {
        for (rrr_buf *b : ctx->bufs)
            if (b->parent == buf) return fail(RRR_ERR_STATE, "rrr_buf_free: free the views of this buffer first");
    }
    if (!ctx->nodevice && !buf->parent && buf->ptr) {
        TRY(device_ready(ctx));
        (void)hipStreamSynchronize(ctx->stream);
        hipError_t e = hipFree(buf->ptr);
        if (e != hipSuccess) return fail(RRR_ERR_HIP, "hipFree: %s", hipGetErrorString(e));
    }
    ctx->bufs.erase(buf);
    buf->magic = 0;
    delete buf;
    return ok();
}

uint64_t rrr_buf_size(const rrr_buf *buf) { return buf && buf->magic == BUF_MAGIC ? buf->bytes : 0; }

static int copy_check(rrr_ctx *ctx, const rrr_buf *buf, uint64_t offset, const void *host, uint64_t bytes,
                      const char *what)
{
    TRY(check_ctx(ctx));
    TRY(check_buf(ctx, buf, what));
    if (!host && bytes) return fail(RRR_ERR_NULL, "%s: null host pointer", what);
    if (offset > buf->bytes || bytes > buf->bytes - offset)
        return fail(RRR_ERR_SHORT_BUFFER, "%s: range [%llu, +%llu) outside a %llu-byte buffer", what,
                    (unsigned long long)offset, (unsigned long long)bytes, (unsigned long long)buf->bytes);
    if (ctx->capturing) return fail(RRR_ERR_STATE, "%s: host copies are not allowed during graph capture", what);
    return RRR_OK;
}

int rrr_buf_upload(rrr_ctx *ctx, rrr_buf *buf, uint64_t offset, const void *src, uint64_t bytes)
{
    TRY(copy_check(ctx, buf, offset, src, bytes, "rrr_buf_upload"));
    if (bytes == 0) return ok();
    TRY(device_ready(ctx));
    hipError_t e = hipMemcpyAsync((char *)buf->ptr + offset, src, bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return fail(RRR_ERR_HIP, "rrr_buf_upload: %s", hipGetErrorString(e));
    return ok();
}

int rrr_buf_download(rrr_ctx *ctx, const rrr_buf *buf, uint64_t offset, void *dst, uint64_t bytes)
{
    TRY(copy_check(ctx, buf, offset, dst, bytes, "rrr_buf_download"));
    if (bytes == 0) return ok();
    TRY(device_ready(ctx));
    hipError_t e = hipMemcpyAsync(dst, (const char *)buf->ptr + offset, bytes, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return fail(RRR_ERR_HIP, "rrr_buf_download: %s", hipGetErrorString(e));
    return ok();
}

int rrr_buf_fill_u32(rrr_ctx *ctx, rrr_buf *buf, uint64_t offset, uint64_t bytes, uint32_t value)
{
    TRY(check_ctx(ctx));
    TRY(check_buf(ctx, buf, "rrr_buf_fill_u32"));
    if (offset % 4 || bytes % 4) return fail(RRR_ERR_INVALID_ARG, "rrr_buf_fill_u32: offset and bytes must be multiples of 4");
    if (offset > buf->bytes || bytes > buf->bytes - offset)
        return fail(RRR_ERR_SHORT_BUFFER, "rrr_buf_fill_u32: range outside the buffer");
    TRY(device_ready(ctx));
    return finish(ctx, launch_fill_u32((uint32_t *)((char *)buf->ptr + offset), bytes / 4, value, ctx->stream),
                  "rrr_buf_fill_u32");
}

// ---- weights ---------------------------------------------------------------

int rrr_weight_upload(rrr_ctx *ctx, uint32_t type, uint32_t K, uint32_t N, const void *raw, uint64_t bytes,
                      rrr_buf **out)
{
    TRY(check_ctx(ctx));
    if (!out) return fail(RRR_ERR_NULL, "rrr_weight_upload: null output pointer");
    *out = nullptr;
    if (!raw) return fail(RRR_ERR_NULL, "rrr_weight_upload: null source");
    TRY(check_shape(type, K, N));
    const uint64_t need_bytes = rrr_tensor_bytes(type, K, N);
    if (bytes < need_bytes)
        return fail(RRR_ERR_SHORT_BUFFER, "rrr_weight_upload: %llu bytes given, a %ux%u type-%u tensor has %llu",
                    (unsigned long long)bytes, N, K, type, (unsigned long long)need_bytes);
    rrr_buf *b = nullptr;
    TRY(rrr_buf_alloc(ctx, need_bytes, &b));
    int rc = rrr_buf_upload(ctx, b, 0, raw, need_bytes);
    if (rc != RRR_OK) {
        std::string msg = g_err;
        rrr_buf_free(ctx, b);
        return fail(rc, "%s", msg.c_str());
    }
    *out = b;
    return ok();
}

int rrr_gguf_upload(rrr_ctx *ctx, const rrr_gguf *g, const char *name, rrr_buf **out)
{
    TRY(check_ctx(ctx));
    if (!out) return fail(RRR_ERR_NULL, "rrr_gguf_upload: null output pointer");
    *out = nullptr;
    rrr_gguf_tensor t;
    TRY(rrr_gguf_find_tensor(g, name, &t));
    if (!valid_type(t.type))
        return fail(RRR_ERR_BAD_TYPE, "tensor '%s' has ggml type %u; the kernels read types 0, 12, 13, 14", name,
                    t.type);
    if (t.dims[0] == 0 || t.n_elements == 0) return fail(RRR_ERR_BAD_SHAPE, "tensor '%s' is empty", name);
    const uint64_t rows = t.n_elements / t.dims[0];
    if (t.dims[0] > UINT32_MAX || rows > UINT32_MAX)
        return fail(RRR_ERR_BAD_SHAPE, "tensor '%s': %llu rows of %llu elements exceed 32-bit sizes", name,
                    (unsigned long long)rows, (unsigned long long)t.dims[0]);
    const int rc = rrr_weight_upload(ctx, t.type, (uint32_t)t.dims[0], (uint32_t)rows, t.data, t.bytes, out);
    if (rc != RRR_OK) {
        std::string msg = g_err;
        return fail(rc, "tensor '%s': %s", name, msg.c_str());
    }
    return ok();
}

// ---- typed ops ---------------------------------------------------------------

int rrr_dequant(rrr_ctx *ctx, uint32_t type, const rrr_buf *W, rrr_buf *out, uint64_t n)
{
    TRY(check_ctx(ctx));
    TRY(check_buf(ctx, W, "rrr_dequant W"));
    TRY(check_buf(ctx, out, "rrr_dequant out"));
    if (!valid_type(type)) return fail(RRR_ERR_BAD_TYPE, "rrr_dequant: ggml type %u", type);
    if (n == 0 || n % 256) return fail(RRR_ERR_BAD_SHAPE, "rrr_dequant: n_elements=%llu is not a positive multiple of 256", (unsigned long long)n);
    TRY(need(W, n / 256 * block_bytes(type), "rrr_dequant W"));
    TRY(need_f32(out, n, "rrr_dequant out"));
    TRY(device_ready(ctx));
    return finish(ctx, launch_dequant(type, (const uint8_t *)W->ptr, W->bytes, (float *)out->ptr, n, ctx->stream),
                  "rrr_dequant");
}

// Checks of one GEMV-family call and its launch arguments.
static int gemv_prepare(rrr_ctx *ctx, const rrr_buf *X, uint64_t x_floats, const rrr_buf *gamma, float eps,
                        uint32_t act, uint32_t hd, uint32_t hpk, const rrr_buf *W, uint32_t type, rrr_buf *Y,
                        uint32_t K, uint32_t N, uint32_t M, uint32_t residual, const char *what, GemvArgs &a,
                        uint64_t y_floats = 0)   // 0: M * N
{
    TRY(check_buf(ctx, X, what));
    TRY(check_buf(ctx, W, what));
    TRY(check_buf(ctx, Y, what));
    if (gamma) TRY(check_buf(ctx, gamma, what));
    TRY(check_shape(type, K, N));
    if (M == 0) return fail(RRR_ERR_BAD_SHAPE, "%s: M must be positive", what);
    if (M > 65535) return fail(RRR_ERR_UNSUPPORTED, "%s: M=%u exceeds 65535", what, M);
    TRY(need(W, rrr_tensor_bytes(type, K, N), what));
    TRY(need_f32(X, x_floats, what));
    TRY(need_f32(Y, y_floats ? y_floats : (uint64_t)M * N, what));
    if (gamma) TRY(need_f32(gamma, K, what));
    if (act == ACT_RMSNORM && !(std::isfinite(eps) && eps >= 0.0f)) return fail(RRR_ERR_INVALID_ARG, "%s: eps", what);
    a = GemvArgs{};
    a.type = type;
    a.x = (const float *)X->ptr;
    a.gamma = gamma ? (const float *)gamma->ptr : nullptr;
    a.eps = eps;
    a.head_dim = hd;
    a.heads_per_kv = hpk;
    a.W = (const uint8_t *)W->ptr;
    a.w_bytes = W->bytes;
    a.y = (float *)Y->ptr;
    a.K = K;
    a.N = N;
    a.M = M;
    a.residual = residual;
    a.ws = ctx->gemm_ws;
    a.ws_bytes = GEMM_WS_BYTES;
    return RRR_OK;
}

static int gemv_common(rrr_ctx *ctx, const rrr_buf *X, uint64_t x_floats, const rrr_buf *gamma, float eps,
                       uint32_t act, uint32_t hd, uint32_t hpk, const rrr_buf *W, uint32_t type, rrr_buf *Y,
                       uint32_t K, uint32_t N, uint32_t M, uint32_t residual, const char *what)
{
    GemvArgs a;
    TRY(gemv_prepare(ctx, X, x_floats, gamma, eps, act, hd, hpk, W, type, Y, K, N, M, residual, what, a));
    TRY(device_ready(ctx));
    return finish(ctx, launch_gemv(a, act, ctx->stream), what);
}

// The operand set of rrr_gemv_residual's activation kinds (x floats, act).
static int residual_act(uint32_t act_kind, uint32_t act_param, uint32_t K, uint64_t &x_floats, uint32_t &act,
                        uint32_t &hd, uint32_t &hpk, const char *what)
{
    hd = hpk = 0;
    switch (act_kind) {
    case RRR_ACT_IDENTITY: x_floats = K; act = ACT_PLAIN; return RRR_OK;
    case RRR_ACT_SILU_GATE: x_floats = 2ull * K; act = ACT_SILU; return RRR_OK;
    case RRR_ACT_GQA_V:
        hd = act_param & 0xFFFFu;
        hpk = act_param >> 16;
        if (hd == 0 || hpk == 0 || hd % 16 || K % (hd * hpk) || (K / hpk) % 16)
            return fail(RRR_ERR_INVALID_ARG, "%s: GQA params head_dim=%u heads_per_kv=%u do not tile K=%u", what, hd,
                        hpk, K);
        x_floats = (uint64_t)K + 2ull * (K / hpk);
        act = ACT_GQA_V;
        return RRR_OK;
    default:
        return fail(RRR_ERR_INVALID_ARG, "%s: act_kind %u", what, act_kind);
    }
}

int rrr_gemv(rrr_ctx *ctx, const rrr_buf *X, const rrr_buf *W, uint32_t type, rrr_buf *Y, uint32_t K, uint32_t N,
             uint32_t M)
{
    TRY(check_ctx(ctx));
    return gemv_common(ctx, X, (uint64_t)M * K, nullptr, 0.0f, ACT_PLAIN, 0, 0, W, type, Y, K, N, M, 0, "rrr_gemv");
}

int rrr_gemv_rmsnorm(rrr_ctx *ctx, const rrr_buf *x, const rrr_buf *gamma, float eps, const rrr_buf *W, uint32_t type,
                     rrr_buf *Y, uint32_t K, uint32_t N)
{
    TRY(check_ctx(ctx));
    if (!gamma) return fail(RRR_ERR_NULL, "rrr_gemv_rmsnorm: null gamma");
    return gemv_common(ctx, x, K, gamma, eps, ACT_RMSNORM, 0, 0, W, type, Y, K, N, 1, 0, "rrr_gemv_rmsnorm");
}

int rrr_gemv_rmsnorm_silu(rrr_ctx *ctx, const rrr_buf *x, const rrr_buf *gamma, float eps, const rrr_buf *W,
                          uint32_t type, rrr_buf *Y, uint32_t K, uint32_t F)
{
    TRY(check_ctx(ctx));
    const char *what = "rrr_gemv_rmsnorm_silu";
    if (!gamma) return fail(RRR_ERR_NULL, "%s: null gamma", what);
    if (F == 0 || F > 0x7FFFFFFFu) return fail(RRR_ERR_BAD_SHAPE, "%s: F=%u", what, F);
    if (type != RRR_TYPE_Q4_K && type != RRR_TYPE_Q5_K && type != RRR_TYPE_Q6_K)
        return fail(RRR_ERR_UNSUPPORTED, "%s: type %u (Q4_K, Q5_K or Q6_K rows)", what, type);
    if (K > 8192) return fail(RRR_ERR_UNSUPPORTED, "%s: K=%u exceeds 8192", what, K);
    // the checks of a GEMV into all 2F rows, with an output of F floats
    GemvArgs a;
    TRY(gemv_prepare(ctx, x, K, gamma, eps, ACT_RMSNORM, 0, 0, W, type, Y, K, 2 * F, 1, 0, what, a, F));
    a.N = F;
    a.pair = 1;
    if (!gemv_mfma_supported(a)) return fail(RRR_ERR_UNSUPPORTED, "%s: shape", what);
    TRY(device_ready(ctx));
    return finish(ctx, launch_gemv(a, ACT_RMSNORM, ctx->stream), what);
}

int rrr_gemv_residual(rrr_ctx *ctx, const rrr_buf *x, uint32_t act_kind, uint32_t act_param, const rrr_buf *W,
                      uint32_t type, rrr_buf *hidden, uint32_t K, uint32_t N)
{
    TRY(check_ctx(ctx));
    const char *what = "rrr_gemv_residual";
    uint64_t x_floats;
    uint32_t act, hd, hpk;
    TRY(residual_act(act_kind, act_param, K, x_floats, act, hd, hpk, what));
    return gemv_common(ctx, x, x_floats, nullptr, 0.0f, act, hd, hpk, W, type, hidden, K, N, 1, 1, what);
}

int rrr_gemm_bf16(rrr_ctx *ctx, const rrr_buf *X, const rrr_buf *W, uint32_t type, rrr_buf *Y, uint32_t K, uint32_t N,
                  uint32_t M)
{
    TRY(check_ctx(ctx));
    const char *what = "rrr_gemm_bf16";
    TRY(check_buf(ctx, X, what));
    TRY(check_buf(ctx, W, what));
    TRY(check_buf(ctx, Y, what));
    TRY(check_shape(type, K, N));
    if (type == RRR_TYPE_F32) return fail(RRR_ERR_UNSUPPORTED, "%s: F32 weights are not a prefill shape", what);
    if (M == 0) return fail(RRR_ERR_BAD_SHAPE, "%s: M must be positive", what);
    TRY(need(W, rrr_tensor_bytes(type, K, N), what));
    TRY(need(X, (uint64_t)M * K * 2, what));
    TRY(need_f32(Y, (uint64_t)M * N, what));
    if (!gemm_rows_supported(type, K, N, M, GEMM_WS_BYTES))
        return fail(RRR_ERR_UNSUPPORTED, "%s: needs N %% 64 == 0 (N=%u)", what, N);
    if (((uintptr_t)X->ptr | (uintptr_t)Y->ptr) & 15)
        return fail(RRR_ERR_INVALID_ARG, "%s: X and Y must be 16-byte aligned", what);
    TRY(device_ready(ctx));
    hipError_t e = launch_gemm_bf16((const uint16_t *)X->ptr, (const uint8_t *)W->ptr, type, (float *)Y->ptr, K, N, M,
                                    (float *)ctx->gemm_ws, GEMM_WS_BYTES, ctx->stream);
    if (e == hipErrorNotSupported) return fail(RRR_ERR_UNSUPPORTED, "%s: shape not supported by the kernels", what);
    return finish(ctx, e, what);
}

int rrr_rmsnorm(rrr_ctx *ctx, const rrr_buf *x, const rrr_buf *gamma, rrr_buf *y, uint32_t rows, uint32_t d, float eps)
{
    TRY(check_ctx(ctx));
    const char *what = "rrr_rmsnorm";
    TRY(check_buf(ctx, x, what));
    TRY(check_buf(ctx, gamma, what));
    TRY(check_buf(ctx, y, what));
    if (rows == 0 || d == 0) return fail(RRR_ERR_BAD_SHAPE, "%s: rows and d must be positive", what);
    if (!(std::isfinite(eps) && eps >= 0.0f)) return fail(RRR_ERR_INVALID_ARG, "%s: eps must be finite and >= 0", what);
    TRY(need_f32(x, (uint64_t)rows * d, what));
    TRY(need_f32(gamma, d, what));
    TRY(need_f32(y, (uint64_t)rows * d, what));
    TRY(device_ready(ctx));
    return finish(ctx, launch_rmsnorm((const float *)x->ptr, (const float *)gamma->ptr, (float *)y->ptr, rows, d, eps,
                                      ctx->stream),
                  what);
}

int rrr_silu_gate(rrr_ctx *ctx, const rrr_buf *gu, rrr_buf *mid, uint32_t rows, uint32_t F)
{
    TRY(check_ctx(ctx));
    const char *what = "rrr_silu_gate";
    TRY(check_buf(ctx, gu, what));
    TRY(check_buf(ctx, mid, what));
    if (rows == 0 || F == 0) return fail(RRR_ERR_BAD_SHAPE, "%s: rows and F must be positive", what);
    TRY(need_f32(gu, 2ull * rows * F, what));
    TRY(need_f32(mid, (uint64_t)rows * F, what));
    TRY(device_ready(ctx));
    return finish(ctx, launch_silu_gate((const float *)gu->ptr, (float *)mid->ptr, rows, F, ctx->stream), what);
}

int rrr_residual_add(rrr_ctx *ctx, const rrr_buf *a, const rrr_buf *b, rrr_buf *out, uint32_t n)
{
    TRY(check_ctx(ctx));
    const char *what = "rrr_residual_add";
    TRY(check_buf(ctx, a, what));
    TRY(check_buf(ctx, b, what));
    TRY(check_buf(ctx, out, what));
    if (n == 0) return fail(RRR_ERR_BAD_SHAPE, "%s: n must be positive", what);
    TRY(need_f32(a, n, what));
    TRY(need_f32(b, n, what));
    TRY(need_f32(out, n, what));
    TRY(device_ready(ctx));
    return finish(ctx, launch_residual_add((const float *)a->ptr, (const float *)b->ptr, (float *)out->ptr, n, ctx->stream),
                  what);
}

static int logits_common(rrr_ctx *ctx, const rrr_buf *x, const rrr_buf *gamma, float eps, const rrr_buf *E,
                         rrr_buf *y, uint32_t K, uint32_t V, uint32_t layout, uint32_t chunk, const char *what,
                         rrr_buf *index = nullptr)
{
    TRY(check_buf(ctx, x, what));
    TRY(check_buf(ctx, E, what));
    TRY(check_buf(ctx, y, what));
    if (gamma) TRY(check_buf(ctx, gamma, what));
    if (index) {
        TRY(check_buf(ctx, index, what));
        TRY(need(index, 4, what));
    }
    uint32_t *token = index ? (uint32_t *)index->ptr : nullptr;
    // the logits, then (forms without the fused argmax) the argmax launch
    auto then_argmax = [&](hipError_t e) {
        if (e == hipSuccess && token) e = launch_argmax((const float *)y->ptr, V, ctx->scratch, token, ctx->stream);
        return e;
    };
    if (K == 0 || V == 0) return fail(RRR_ERR_BAD_SHAPE, "%s: K and V must be positive", what);
    if (layout > RRR_LOGITS_Q6K) return fail(RRR_ERR_INVALID_ARG, "%s: layout %u", what, layout);
    if (gamma && !(std::isfinite(eps) && eps >= 0.0f)) return fail(RRR_ERR_INVALID_ARG, "%s: eps", what);
    TRY(need_f32(x, K, what));
    TRY(need_f32(y, V, what));
    if (gamma) TRY(need_f32(gamma, K, what));
    if (layout == RRR_LOGITS_Q6K) {
        if (K % 256) return fail(RRR_ERR_BAD_SHAPE, "%s: Q6_K rows need K %% 256 == 0 (K=%u)", what, K);
        TRY(need(E, rrr_tensor_bytes(RRR_TYPE_Q6_K, K, V), what));
    } else {
        TRY(need(E, (uint64_t)V * K * 4, what));
    }
    if (layout != RRR_LOGITS_CHUNKED) {
        if (K % 256) return fail(RRR_ERR_BAD_SHAPE, "%s: row layout needs K %% 256 == 0 (K=%u)", what, K);
        TRY(device_ready(ctx));
        GemvArgs a{};
        a.type = layout == RRR_LOGITS_Q6K ? T_Q6_K : T_F32;
        a.x = (const float *)x->ptr;
        a.gamma = gamma ? (const float *)gamma->ptr : nullptr;
        a.eps = eps;
        a.W = (const uint8_t *)E->ptr;
        a.w_bytes = E->bytes;
        a.y = (float *)y->ptr;
        a.K = K;
        a.N = V;
        a.M = 1;
        return finish(ctx, then_argmax(launch_gemv(a, gamma ? ACT_RMSNORM : ACT_PLAIN, ctx->stream)), what);
    }
    if (chunk == 0) return fail(RRR_ERR_INVALID_ARG, "%s: chunk must be positive", what);
    if (chunk % 256 && chunk < V) return fail(RRR_ERR_UNSUPPORTED, "%s: chunk=%u must be a multiple of 256", what, chunk);
    if (K % 4) return fail(RRR_ERR_BAD_SHAPE, "%s: chunked layout needs K %% 4 == 0", what);
    if (K > 12288) return fail(RRR_ERR_UNSUPPORTED, "%s: K=%u exceeds 12288", what, K);
    const uint64_t cn = chunk < V ? chunk : V;
    if (cn * K * 4 > 0xFFFFFFFFull) return fail(RRR_ERR_UNSUPPORTED, "%s: one chunk exceeds 4 GiB", what);
    TRY(device_ready(ctx));
    const float *g = gamma ? (const float *)gamma->ptr : nullptr;
    if (logits_split_supported(K, V, (uint32_t)cn, GEMM_WS_BYTES))
        return finish(ctx, launch_logits_split((const float *)x->ptr, g, eps, (const float *)E->ptr, (float *)y->ptr, K, V,
                                               (uint32_t)cn, (float *)ctx->gemm_ws, (uint32_t *)ctx->logits_cnt, token,
                                               ctx->stream),
                      what);
    return finish(ctx, then_argmax(launch_logits_chunked((const float *)x->ptr, g, eps, (const float *)E->ptr,
                                                         (float *)y->ptr, K, V, (uint32_t)cn, ctx->stream)),
                  what);
}

int rrr_logits_f32(rrr_ctx *ctx, const rrr_buf *x, const rrr_buf *E, rrr_buf *logits, uint32_t K, uint32_t V,
                   uint32_t layout, uint32_t chunk)
{
    TRY(check_ctx(ctx));
    return logits_common(ctx, x, nullptr, 0.0f, E, logits, K, V, layout, chunk, "rrr_logits_f32");
}

int rrr_logits_rmsnorm(rrr_ctx *ctx, const rrr_buf *x, const rrr_buf *gamma, float eps, const rrr_buf *E,
                       rrr_buf *logits, uint32_t K, uint32_t V, uint32_t layout, uint32_t chunk)
{
    TRY(check_ctx(ctx));
    if (!gamma) return fail(RRR_ERR_NULL, "rrr_logits_rmsnorm: null gamma");
    return logits_common(ctx, x, gamma, eps, E, logits, K, V, layout, chunk, "rrr_logits_rmsnorm");
}

int rrr_logits_rmsnorm_argmax(rrr_ctx *ctx, const rrr_buf *x, const rrr_buf *gamma, float eps, const rrr_buf *E,
                              rrr_buf *logits, uint32_t K, uint32_t V, uint32_t layout, uint32_t chunk,
                              rrr_buf *out_index)
{
    TRY(check_ctx(ctx));
    const char *what = "rrr_logits_rmsnorm_argmax";
    if (!gamma) return fail(RRR_ERR_NULL, "%s: null gamma", what);
    if (!out_index) return fail(RRR_ERR_NULL, "%s: null out_index", what);
    return logits_common(ctx, x, gamma, eps, E, logits, K, V, layout, chunk, what, out_index);
}

int rrr_argmax_f32(rrr_ctx *ctx, const rrr_buf *logits, uint32_t V, rrr_buf *out_index)
{
    TRY(check_ctx(ctx));
    const char *what = "rrr_argmax_f32";
    TRY(check_buf(ctx, logits, what));
    TRY(check_buf(ctx, out_index, what));
    if (V == 0) return fail(RRR_ERR_BAD_SHAPE, "%s: V must be positive", what);
    TRY(need_f32(logits, V, what));
    TRY(need(out_index, 4, what));
    TRY(device_ready(ctx));
    return finish(ctx, launch_argmax((const float *)logits->ptr, V, ctx->scratch, (uint32_t *)out_index->ptr, ctx->stream),
                  what);
}

// ---- decode glue: RoPE + f16 KV store, decode attention --------------------

// rows consecutive tokens at positions pos .. pos + rows - 1, their qkv rows
// back to back
// The checks of the rope_kv_store pipeline; fills its RopeArgs.
static int rope_check(rrr_ctx *ctx, rrr_buf *qkv, uint32_t rows, const rrr_buf *rope_factors, uint32_t n_factors,
                      rrr_buf *k_cache, rrr_buf *v_cache, uint32_t pos, uint32_t n_heads, uint32_t n_kv_heads,
                      uint32_t head_dim, uint32_t rope_dim, uint32_t q_dim, uint32_t kv_stride, float theta,
                      float attn_factor, const char *what, RopeArgs &r)
{
    TRY(check_buf(ctx, qkv, what));
    TRY(check_buf(ctx, k_cache, what));
    TRY(check_buf(ctx, v_cache, what));
    if (n_factors) TRY(check_buf(ctx, rope_factors, what));
    if (kv_stride == 0 || kv_stride % 2) return fail(RRR_ERR_BAD_SHAPE, "%s: kv_stride=%u must be even and positive", what, kv_stride);
    if (rope_dim) {
        if (head_dim == 0 || head_dim % 2 || rope_dim % 2 || rope_dim > head_dim)
            return fail(RRR_ERR_BAD_SHAPE, "%s: need even head_dim >= even rope_dim (head_dim=%u rope_dim=%u)", what,
                        head_dim, rope_dim);
        if ((uint64_t)n_heads * head_dim > q_dim)
            return fail(RRR_ERR_BAD_SHAPE, "%s: %u Q heads of %u do not fit q_dim=%u", what, n_heads, head_dim, q_dim);
        if ((uint64_t)n_kv_heads * head_dim != kv_stride)
            return fail(RRR_ERR_BAD_SHAPE, "%s: kv_stride=%u is not n_kv_heads * head_dim", what, kv_stride);
        if (!(theta > 0.0f)) return fail(RRR_ERR_INVALID_ARG, "%s: theta must be positive", what);
    }
    if (rows == 0) return fail(RRR_ERR_BAD_SHAPE, "%s: rows must be positive", what);
    if ((uint64_t)pos + rows > 0xFFFFFFFFull) return fail(RRR_ERR_BAD_SHAPE, "%s: positions past 2^32", what);
    const uint64_t row = (uint64_t)q_dim + 2ull * kv_stride;
    if (rows > 1 && row > 0xFFFFFFFFull) return fail(RRR_ERR_BAD_SHAPE, "%s: qkv row too long", what);
    TRY(need(qkv, 4 * row * rows, what));
    TRY(need(k_cache, 2 * ((uint64_t)pos + rows) * kv_stride, what));
    TRY(need(v_cache, 2 * ((uint64_t)pos + rows) * kv_stride, what));
    if (n_factors) TRY(need(rope_factors, 4ull * n_factors, what));
    if (((uintptr_t)qkv->ptr | (uintptr_t)k_cache->ptr | (uintptr_t)v_cache->ptr) & 3)
        return fail(RRR_ERR_INVALID_ARG, "%s: buffers must be 4-byte aligned", what);
    r = RopeArgs{n_factors ? (const float *)rope_factors->ptr : nullptr, n_factors, pos, rope_dim ? n_heads : 0u,
                 head_dim, rope_dim, q_dim, kv_stride, theta, attn_factor, (uint32_t)row};
    return RRR_OK;
}

static int rope_common(rrr_ctx *ctx, rrr_buf *qkv, uint32_t rows, const rrr_buf *rope_factors, uint32_t n_factors,
                       rrr_buf *k_cache, rrr_buf *v_cache, uint32_t pos, uint32_t n_heads, uint32_t n_kv_heads,
                       uint32_t head_dim, uint32_t rope_dim, uint32_t q_dim, uint32_t kv_stride, float theta,
                       float attn_factor, const char *what)
{
    RopeArgs r;
    TRY(rope_check(ctx, qkv, rows, rope_factors, n_factors, k_cache, v_cache, pos, n_heads, n_kv_heads, head_dim,
                   rope_dim, q_dim, kv_stride, theta, attn_factor, what, r));
    TRY(device_ready(ctx));
    return finish(ctx, launch_rope_kv_store((float *)qkv->ptr, r, (uint16_t *)k_cache->ptr, (uint16_t *)v_cache->ptr,
                                            ctx->stream, rows),
                  what);
}

int rrr_gemv_rmsnorm_rope_kv(rrr_ctx *ctx, const rrr_buf *x, const rrr_buf *gamma, float eps, const rrr_buf *W,
                             uint32_t type, rrr_buf *qkv, uint32_t K, const rrr_buf *rope_factors, uint32_t n_factors,
                             rrr_buf *k_cache, rrr_buf *v_cache, uint32_t pos, uint32_t n_heads, uint32_t n_kv_heads,
                             uint32_t head_dim, uint32_t rope_dim, uint32_t q_dim, uint32_t kv_stride, float theta,
                             float attn_factor)
{
    TRY(check_ctx(ctx));
    const char *what = "rrr_gemv_rmsnorm_rope_kv";
    if (!gamma) return fail(RRR_ERR_NULL, "%s: null gamma", what);
    const uint64_t n64 = (uint64_t)q_dim + 2ull * kv_stride;
    if (n64 == 0 || n64 > 0xFFFFFFFFull) return fail(RRR_ERR_BAD_SHAPE, "%s: qkv row of %llu floats", what,
                                                     (unsigned long long)n64);
    const uint32_t N = (uint32_t)n64;
    RopeArgs r;
    TRY(rope_check(ctx, qkv, 1, rope_factors, n_factors, k_cache, v_cache, pos, n_heads, n_kv_heads, head_dim,
                   rope_dim, q_dim, kv_stride, theta, attn_factor, what, r));
    GemvArgs a;
    TRY(gemv_prepare(ctx, x, K, gamma, eps, ACT_RMSNORM, 0, 0, W, type, qkv, K, N, 1, 0, what, a));
    TRY(device_ready(ctx));
    if (N % 2 == 0 && gemv_mfma_supported(a)) {
        a.rope_on = 1;
        a.rope = r;
        a.kc = (uint32_t *)k_cache->ptr;
        a.vc = (uint32_t *)v_cache->ptr;
        const hipError_t e = launch_gemv_mfma(a, ACT_RMSNORM, ctx->stream);
        if (e != hipErrorNotSupported) return finish(ctx, e, what);
        a.rope_on = 0;
    }
    // the two launches (a shape the fused epilogue does not take)
    const hipError_t e = launch_gemv(a, ACT_RMSNORM, ctx->stream);
    if (e != hipSuccess) return finish(ctx, e, what);
    return finish(ctx, launch_rope_kv_store((float *)qkv->ptr, r, (uint16_t *)k_cache->ptr, (uint16_t *)v_cache->ptr,
                                            ctx->stream, 1),
                  what);
}

int rrr_rope_kv_store(rrr_ctx *ctx, rrr_buf *qkv, const rrr_buf *rope_factors, uint32_t n_factors, rrr_buf *k_cache,
                      rrr_buf *v_cache, uint32_t pos, uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                      uint32_t rope_dim, uint32_t q_dim, uint32_t kv_stride, float theta, float attn_factor)
{
    TRY(check_ctx(ctx));
    return rope_common(ctx, qkv, 1, rope_factors, n_factors, k_cache, v_cache, pos, n_heads, n_kv_heads, head_dim,
                       rope_dim, q_dim, kv_stride, theta, attn_factor, "rrr_rope_kv_store");
}

int rrr_rope_kv_store_rows(rrr_ctx *ctx, rrr_buf *qkv, uint32_t rows, const rrr_buf *rope_factors, uint32_t n_factors,
                           rrr_buf *k_cache, rrr_buf *v_cache, uint32_t pos0, uint32_t n_heads, uint32_t n_kv_heads,
                           uint32_t head_dim, uint32_t rope_dim, uint32_t q_dim, uint32_t kv_stride, float theta,
                           float attn_factor)
{
    TRY(check_ctx(ctx));
    return rope_common(ctx, qkv, rows, rope_factors, n_factors, k_cache, v_cache, pos0, n_heads, n_kv_heads, head_dim,
                       rope_dim, q_dim, kv_stride, theta, attn_factor, "rrr_rope_kv_store_rows");
}

int rrr_attention(rrr_ctx *ctx, const rrr_buf *q, const rrr_buf *k_cache, const rrr_buf *v_cache, rrr_buf *out,
                  uint32_t seq_len, uint32_t n_kv_heads, uint32_t heads_per_kv, uint32_t head_dim)
{
    TRY(check_ctx(ctx));
    const char *what = "rrr_attention";
    TRY(check_buf(ctx, q, what));
    TRY(check_buf(ctx, k_cache, what));
    TRY(check_buf(ctx, v_cache, what));
    TRY(check_buf(ctx, out, what));
    if (head_dim != ATT_HD) return fail(RRR_ERR_UNSUPPORTED, "%s: head_dim=%u (the kernels take %u)", what, head_dim, ATT_HD);
    if (seq_len == 0 || n_kv_heads == 0 || heads_per_kv == 0)
        return fail(RRR_ERR_BAD_SHAPE, "%s: seq_len, n_kv_heads and heads_per_kv must be positive", what);
    if (seq_len > ATT_SEQ_MAX) return fail(RRR_ERR_UNSUPPORTED, "%s: seq_len=%u exceeds %u", what, seq_len, ATT_SEQ_MAX);
    if (heads_per_kv > 8 || (uint64_t)n_kv_heads * heads_per_kv > ATT_HEADS_MAX)
        return fail(RRR_ERR_UNSUPPORTED, "%s: at most 8 query heads per KV head and %u query heads", what, ATT_HEADS_MAX);
    const uint64_t nq = (uint64_t)n_kv_heads * heads_per_kv * head_dim, kv = (uint64_t)seq_len * n_kv_heads * head_dim;
    TRY(need_f32(q, nq, what));
    TRY(need_f32(out, nq, what));
    TRY(need(k_cache, 2 * kv, what));
    TRY(need(v_cache, 2 * kv, what));
    if (((uintptr_t)q->ptr | (uintptr_t)out->ptr | (uintptr_t)k_cache->ptr | (uintptr_t)v_cache->ptr) & 15)
        return fail(RRR_ERR_INVALID_ARG, "%s: q, out and the caches must be 16-byte aligned", what);
    TRY(device_ready(ctx));
    return finish(ctx, launch_attention((const float *)q->ptr, (const uint16_t *)k_cache->ptr,
                                        (const uint16_t *)v_cache->ptr, (float *)out->ptr, ctx->att_scratch, seq_len,
                                        n_kv_heads, heads_per_kv, device_cu_count(), ctx->stream),
                  what);
}

// ---- prefill: causal attention over the prompt, f16-activation GEMMs --------

int rrr_attention_prefill(rrr_ctx *ctx, const rrr_buf *qkv, uint32_t rows, const rrr_buf *k_cache,
                          const rrr_buf *v_cache, rrr_buf *out, uint32_t out_type, uint32_t pos0, uint32_t n_kv_heads,
                          uint32_t heads_per_kv, uint32_t head_dim)
{
    TRY(check_ctx(ctx));
    const char *what = "rrr_attention_prefill";
    TRY(check_buf(ctx, qkv, what));
    TRY(check_buf(ctx, k_cache, what));
    TRY(check_buf(ctx, v_cache, what));
    TRY(check_buf(ctx, out, what));
    if (head_dim != ATT_HD) return fail(RRR_ERR_UNSUPPORTED, "%s: head_dim=%u (the kernels take %u)", what, head_dim, ATT_HD);
    if (rows == 0 || n_kv_heads == 0 || heads_per_kv == 0)
        return fail(RRR_ERR_BAD_SHAPE, "%s: rows, n_kv_heads and heads_per_kv must be positive", what);
    if (out_type != RRR_TYPE_F32 && out_type != RRR_TYPE_F16)
        return fail(RRR_ERR_BAD_TYPE, "%s: out_type %u (F32 or F16)", what, out_type);
    if ((uint64_t)pos0 + rows > ATT_SEQ_MAX)
        return fail(RRR_ERR_UNSUPPORTED, "%s: positions up to %llu exceed %u", what,
                    (unsigned long long)pos0 + rows, ATT_SEQ_MAX);
    if (heads_per_kv > 8 || (uint64_t)n_kv_heads * heads_per_kv > ATT_HEADS_MAX)
        return fail(RRR_ERR_UNSUPPORTED, "%s: at most 8 query heads per KV head and %u query heads", what, ATT_HEADS_MAX);
    const uint64_t nq = (uint64_t)n_kv_heads * heads_per_kv * head_dim, kvs = (uint64_t)n_kv_heads * head_dim;
    const uint64_t row = nq + 2 * kvs;
    TRY(need_f32(qkv, row * rows, what));
    TRY(need(out, nq * rows * (out_type == RRR_TYPE_F16 ? 2 : 4), what));
    TRY(need(k_cache, 2 * ((uint64_t)pos0 + rows) * kvs, what));
    TRY(need(v_cache, 2 * ((uint64_t)pos0 + rows) * kvs, what));
    if (((uintptr_t)qkv->ptr | (uintptr_t)k_cache->ptr | (uintptr_t)v_cache->ptr) & 15)
        return fail(RRR_ERR_INVALID_ARG, "%s: qkv and caches must be 16-byte aligned", what);
    TRY(device_ready(ctx));
    return finish(ctx, launch_attention_prefill((const float *)qkv->ptr, (uint32_t)row, rows,
                                                (const uint16_t *)k_cache->ptr, (const uint16_t *)v_cache->ptr,
                                                out->ptr, out_type == RRR_TYPE_F16, pos0, n_kv_heads, heads_per_kv,
                                                ctx->stream),
                  what);
}

int rrr_gemm_f16(rrr_ctx *ctx, const rrr_buf *X, const rrr_buf *row_scale, const rrr_buf *W, uint32_t type, rrr_buf *Y,
                 uint32_t K, uint32_t N, uint32_t M, uint32_t accumulate)
{
    TRY(check_ctx(ctx));
    const char *what = "rrr_gemm_f16";
    TRY(check_buf(ctx, X, what));
    if (row_scale) {
        TRY(check_buf(ctx, row_scale, what));
        TRY(need_f32(row_scale, M, what));
    }
    TRY(check_buf(ctx, W, what));
    TRY(check_buf(ctx, Y, what));
    TRY(check_shape(type, K, N));
    if (type == RRR_TYPE_F32) return fail(RRR_ERR_UNSUPPORTED, "%s: F32 weights are not a prefill shape", what);
    if (M == 0) return fail(RRR_ERR_BAD_SHAPE, "%s: M must be positive", what);
    TRY(need(W, rrr_tensor_bytes(type, K, N), what));
    TRY(need(X, (uint64_t)M * K * 2, what));
    TRY(need_f32(Y, (uint64_t)M * N, what));
    if (!gemm_supported(type, K, N, M, (uint64_t)M * K * 2))
        return fail(RRR_ERR_UNSUPPORTED, "%s: needs M %% 128 == 0 and N %% 64 == 0 (M=%u N=%u)", what, M, N);
    TRY(device_ready(ctx));
    return finish(ctx, launch_gemm_f16((const uint16_t *)X->ptr, row_scale ? (const float *)row_scale->ptr : nullptr,
                                       (const uint8_t *)W->ptr, type, (float *)Y->ptr, K, N, M, accumulate != 0,
                                       (float *)ctx->gemm_ws, GEMM_WS_BYTES, ctx->stream),
                  what);
}

int rrr_gemm_f16_rmsnorm(rrr_ctx *ctx, const rrr_buf *X, const rrr_buf *row_scale, const rrr_buf *W, uint32_t type,
                         rrr_buf *Y, uint32_t K, uint32_t N, uint32_t M, uint32_t accumulate, const rrr_buf *gamma,
                         float eps, rrr_buf *y16)
{
    TRY(check_ctx(ctx));
    const char *what = "rrr_gemm_f16_rmsnorm";
    TRY(check_buf(ctx, X, what));
    if (row_scale) {
        TRY(check_buf(ctx, row_scale, what));
        TRY(need_f32(row_scale, M, what));
    }
    TRY(check_buf(ctx, W, what));
    TRY(check_buf(ctx, Y, what));
    TRY(check_buf(ctx, gamma, what));
    TRY(check_buf(ctx, y16, what));
    TRY(check_shape(type, K, N));
    if (type == RRR_TYPE_F32) return fail(RRR_ERR_UNSUPPORTED, "%s: F32 weights are not a prefill shape", what);
    if (M == 0) return fail(RRR_ERR_BAD_SHAPE, "%s: M must be positive", what);
    if (!(std::isfinite(eps) && eps >= 0.0f)) return fail(RRR_ERR_INVALID_ARG, "%s: eps must be finite and >= 0", what);
    TRY(need(W, rrr_tensor_bytes(type, K, N), what));
    TRY(need(X, (uint64_t)M * K * 2, what));
    TRY(need_f32(Y, (uint64_t)M * N, what));
    TRY(need_f32(gamma, N, what));
    TRY(need(y16, 2ull * M * N, what));
    if (!gemm_supported(type, K, N, M, (uint64_t)M * K * 2) || !splitk_reduce_rmsnorm_supported(N))
        return fail(RRR_ERR_UNSUPPORTED, "%s: needs M %% 128 == 0, N %% 64 == 0 and N <= 8192 (M=%u N=%u)", what, M,
                    N);
    TRY(device_ready(ctx));
    return finish(ctx,
                  launch_gemm_f16_rmsnorm((const uint16_t *)X->ptr, row_scale ? (const float *)row_scale->ptr : nullptr,
                                          (const uint8_t *)W->ptr, type, (float *)Y->ptr, K, N, M, accumulate != 0,
                                          (const float *)gamma->ptr, eps, (uint16_t *)y16->ptr, (float *)ctx->gemm_ws,
                                          GEMM_WS_BYTES, ctx->stream),
                  what);
}

int rrr_gemm_f16_rope_kv_rows(rrr_ctx *ctx, const rrr_buf *X, const rrr_buf *W, uint32_t type, rrr_buf *qkv,
                              uint32_t K, uint32_t M, uint32_t rows, const rrr_buf *rope_factors, uint32_t n_factors,
                              rrr_buf *k_cache, rrr_buf *v_cache, uint32_t pos0, uint32_t n_heads,
                              uint32_t n_kv_heads, uint32_t head_dim, uint32_t rope_dim, uint32_t q_dim,
                              uint32_t kv_stride, float theta, float attn_factor)
{
    TRY(check_ctx(ctx));
    const char *what = "rrr_gemm_f16_rope_kv_rows";
    if (rows > M) return fail(RRR_ERR_BAD_SHAPE, "%s: rows=%u exceeds M=%u", what, rows, M);
    RopeArgs r;
    TRY(rope_check(ctx, qkv, rows, rope_factors, n_factors, k_cache, v_cache, pos0, n_heads, n_kv_heads, head_dim,
                   rope_dim, q_dim, kv_stride, theta, attn_factor, what, r));
    const uint32_t N = r.row_stride;
    TRY(check_buf(ctx, X, what));
    TRY(check_buf(ctx, W, what));
    TRY(check_shape(type, K, N));
    if (type == RRR_TYPE_F32) return fail(RRR_ERR_UNSUPPORTED, "%s: F32 weights are not a prefill shape", what);
    TRY(need(W, rrr_tensor_bytes(type, K, N), what));
    TRY(need(X, (uint64_t)M * K * 2, what));
    TRY(need_f32(qkv, (uint64_t)M * N, what));
    if ((uintptr_t)qkv->ptr & 15) return fail(RRR_ERR_INVALID_ARG, "%s: qkv must be 16-byte aligned", what);
    if (!gemm_supported(type, K, N, M, (uint64_t)M * K * 2) || !splitk_rope_kv_store_supported(r))
        return fail(RRR_ERR_UNSUPPORTED, "%s: needs M %% 128 == 0, N %% 64 == 0, q_dim and kv_stride %% 4 == 0 "
                    "(M=%u N=%u)", what, M, N);
    TRY(device_ready(ctx));
    return finish(ctx,
                  launch_gemm_f16_rope_kv((const uint16_t *)X->ptr, (const uint8_t *)W->ptr, type, (float *)qkv->ptr, K,
                                          N, M, r, rows, (uint16_t *)k_cache->ptr, (uint16_t *)v_cache->ptr,
                                          (float *)ctx->gemm_ws, GEMM_WS_BYTES, ctx->stream),
                  what);
}

int rrr_rmsnorm_f16(rrr_ctx *ctx, const rrr_buf *x, const rrr_buf *gamma, rrr_buf *y, uint32_t rows, uint32_t d,
                    float eps)
{
    TRY(check_ctx(ctx));
    const char *what = "rrr_rmsnorm_f16";
    TRY(check_buf(ctx, x, what));
    TRY(check_buf(ctx, gamma, what));
    TRY(check_buf(ctx, y, what));
    if (rows == 0 || d == 0) return fail(RRR_ERR_BAD_SHAPE, "%s: rows and d must be positive", what);
    if (!(std::isfinite(eps) && eps >= 0.0f)) return fail(RRR_ERR_INVALID_ARG, "%s: eps must be finite and >= 0", what);
    TRY(need_f32(x, (uint64_t)rows * d, what));
    TRY(need_f32(gamma, d, what));
    TRY(need(y, 2ull * rows * d, what));
    TRY(device_ready(ctx));
    return finish(ctx, launch_rmsnorm_f16((const float *)x->ptr, (const float *)gamma->ptr, (uint16_t *)y->ptr, rows, d,
                                          eps, ctx->stream),
                  what);
}

int rrr_silu_gate_f16(rrr_ctx *ctx, const rrr_buf *gate_up, rrr_buf *mid, rrr_buf *row_scale, uint32_t rows,
                      uint32_t F)
{
    TRY(check_ctx(ctx));
    const char *what = "rrr_silu_gate_f16";
    TRY(check_buf(ctx, gate_up, what));
    TRY(check_buf(ctx, mid, what));
    TRY(check_buf(ctx, row_scale, what));
    if (rows == 0 || F == 0) return fail(RRR_ERR_BAD_SHAPE, "%s: rows and F must be positive", what);
    TRY(need_f32(gate_up, 2ull * rows * F, what));
    TRY(need(mid, 2ull * rows * F, what));
    TRY(need_f32(row_scale, rows, what));
    TRY(device_ready(ctx));
    return finish(ctx, launch_silu_gate_f16((const float *)gate_up->ptr, (uint16_t *)mid->ptr,
                                            (float *)row_scale->ptr, rows, F, ctx->stream),
                  what);
}

int rrr_gemm_f16_silu_gate_f16(rrr_ctx *ctx, const rrr_buf *X, const rrr_buf *W, uint32_t type, rrr_buf *mid,
                               rrr_buf *row_scale, uint32_t K, uint32_t F, uint32_t M)
{
    TRY(check_ctx(ctx));
    const char *what = "rrr_gemm_f16_silu_gate_f16";
    TRY(check_buf(ctx, X, what));
    TRY(check_buf(ctx, W, what));
    TRY(check_buf(ctx, mid, what));
    TRY(check_buf(ctx, row_scale, what));
    if (M == 0 || F == 0 || F > 0x7FFFFFFFu) return fail(RRR_ERR_BAD_SHAPE, "%s: M and F must be positive", what);
    const uint32_t N = 2 * F;
    TRY(check_shape(type, K, N));
    if (type == RRR_TYPE_F32) return fail(RRR_ERR_UNSUPPORTED, "%s: F32 weights are not a prefill shape", what);
    TRY(need(W, rrr_tensor_bytes(type, K, N), what));
    TRY(need(X, (uint64_t)M * K * 2, what));
    TRY(need(mid, 2ull * M * F, what));
    TRY(need_f32(row_scale, M, what));
    if (!gemm_supported(type, K, N, M, (uint64_t)M * K * 2) || M % 256 || F % 64 || (uint64_t)M * F * 4 > GEMM_WS_BYTES ||
        (uint64_t)(N / 128) * (M / 256) < 128)
        return fail(RRR_ERR_UNSUPPORTED, "%s: needs M %% 256 == 0, F %% 64 == 0, (F / 64) * (M / 256) >= 128 and "
                    "M * F * 4 <= %llu (M=%u F=%u); use rrr_gemm_f16 and rrr_silu_gate_f16", what,
                    (unsigned long long)GEMM_WS_BYTES, M, F);
    TRY(device_ready(ctx));
    return finish(ctx,
                  launch_gemm_f16_silu_f16((const uint16_t *)X->ptr, (const uint8_t *)W->ptr, type,
                                           (uint16_t *)mid->ptr, (float *)row_scale->ptr, K, F, M,
                                           (float *)ctx->gemm_ws, GEMM_WS_BYTES, ctx->stream),
                  what);
}

// ---- name-keyed dispatch shim ----------------------------------------------

static int push_u32(const void *push, uint32_t push_bytes, uint32_t n, uint32_t *out, const char *name)
{
    if (push_bytes != 4 * n) return fail(RRR_ERR_INVALID_ARG, "%s: expects %u push bytes, got %u", name, 4 * n, push_bytes);
    if (!push) return fail(RRR_ERR_NULL, "%s: null push constants", name);
    const unsigned char *p = (const unsigned char *)push;
    for (uint32_t i = 0; i < n; i++)
        out[i] = (uint32_t)p[4 * i] | ((uint32_t)p[4 * i + 1] << 8) | ((uint32_t)p[4 * i + 2] << 16) |
                 ((uint32_t)p[4 * i + 3] << 24);
    return RRR_OK;
}

static int want_bufs(uint32_t n_bufs, uint32_t n, rrr_buf *const *bufs, const char *name)
{
    if (n_bufs != n) return fail(RRR_ERR_INVALID_ARG, "%s: expects %u buffers, got %u", name, n, n_bufs);
    if (!bufs) return fail(RRR_ERR_NULL, "%s: null buffer list", name);
    return RRR_OK;
}

static int want_grid(const uint32_t *g, uint32_t x, uint32_t y, uint32_t z, const char *name)
{
    if (!g) return fail(RRR_ERR_NULL, "%s: null grid", name);
    if (g[0] != x || g[1] != y || g[2] != z)
        return fail(RRR_ERR_INVALID_ARG, "%s: grid [%u,%u,%u] does not match the push constants (expected [%u,%u,%u])",
                    name, g[0], g[1], g[2], x, y, z);
    return RRR_OK;
}

static int dispatch_one(rrr_ctx *ctx, const char *name, rrr_buf *const *bufs, uint32_t n_bufs, const void *push,
                        uint32_t push_bytes, const uint32_t *groups)
{
    if (!name) return fail(RRR_ERR_NULL, "rrr_dispatch: null pipeline name");
    uint32_t pc[3];
    struct KQ { const char *name; uint32_t type; bool batch; };
    static const KQ kq[] = {
        {"matmul_q4k", RRR_TYPE_Q4_K, false},        {"matmul_q5k", RRR_TYPE_Q5_K, false},
        {"matmul_q6k", RRR_TYPE_Q6_K, false},        {"matmul_gpuq4", RRR_TYPE_Q4_K, false},
        {"matmul_gpuq5", RRR_TYPE_Q5_K, false},      {"matmul_gpuq6", RRR_TYPE_Q6_K, false},
        {"matmul_gpuq4_batch", RRR_TYPE_Q4_K, true}, {"matmul_gpuq5_batch", RRR_TYPE_Q5_K, true},
        {"matmul_gpuq6_batch", RRR_TYPE_Q6_K, true},
    };
    for (const KQ &q : kq) {
        if (strcmp(name, q.name)) continue;
        TRY(want_bufs(n_bufs, 3, bufs, name));
        if (!q.batch) {
            TRY(push_u32(push, push_bytes, 2, pc, name));
            TRY(want_grid(groups, pc[1], 1, 1, name));
            return gemv_common(ctx, bufs[0], pc[0], nullptr, 0.0f, ACT_PLAIN, 0, 0, bufs[1], q.type, bufs[2], pc[0], pc[1],
                               1, 0, name);
        }
        TRY(push_u32(push, push_bytes, 3, pc, name));
        TRY(want_grid(groups, pc[1], pc[2], 1, name));
        return gemv_common(ctx, bufs[0], (uint64_t)pc[2] * pc[0], nullptr, 0.0f, ACT_PLAIN, 0, 0, bufs[1], q.type,
                           bufs[2], pc[0], pc[1], pc[2], 0, name);
    }
    if (!strcmp(name, "matmul_tiled")) {
        TRY(want_bufs(n_bufs, 3, bufs, name));
        TRY(push_u32(push, push_bytes, 3, pc, name));  // [M, K, N]
        const uint32_t M = pc[0], K = pc[1], N = pc[2];
        TRY(want_grid(groups, (N + 15) / 16, (M + 15) / 16, 1, name));
        if (M != 1) return fail(RRR_ERR_UNSUPPORTED, "%s: only M = 1 (the logit shape) is supported", name);
        return logits_common(ctx, bufs[0], nullptr, 0.0f, bufs[1], bufs[2], K, N, RRR_LOGITS_CHUNKED, N, name);
    }
    if (!strcmp(name, "rmsnorm")) {
        TRY(want_bufs(n_bufs, 3, bufs, name));
        TRY(push_u32(push, push_bytes, 2, pc, name));
        TRY(want_grid(groups, 1, 1, 1, name));
        return rrr_rmsnorm(ctx, bufs[0], bufs[1], bufs[2], pc[0], pc[1], 1e-5f);
    }
    if (!strcmp(name, "silu_gate")) {
        TRY(want_bufs(n_bufs, 2, bufs, name));
        TRY(push_u32(push, push_bytes, 1, pc, name));
        TRY(want_grid(groups, (pc[0] + 255) / 256, 1, 1, name));
        return rrr_silu_gate(ctx, bufs[0], bufs[1], 1, pc[0]);
    }
    if (!strcmp(name, "residual_add")) {
        TRY(want_bufs(n_bufs, 3, bufs, name));
        TRY(push_u32(push, push_bytes, 1, pc, name));
        TRY(want_grid(groups, (pc[0] + 255) / 256, 1, 1, name));
        return rrr_residual_add(ctx, bufs[0], bufs[1], bufs[2], pc[0]);
    }
    if (!strcmp(name, "rope_kv_store")) {
        // bufs [qkv, rope_factors, k_cache, v_cache], push [pos, n_heads, n_kv_heads, head_dim, rope_dim, q_dim,
        // kv_stride] (phi4.rs:1016-1017, :1115-1117); theta and the attention factor are baked in, as in the
        // reference's shader (the legacy constants, phi4.rs:114-116)
        uint32_t p7[7];
        TRY(want_bufs(n_bufs, 4, bufs, name));
        TRY(push_u32(push, push_bytes, 7, p7, name));
        const uint32_t rp = (p7[1] + p7[2]) * (p7[4] / 2), hkv = p7[6] / 2;
        TRY(want_grid(groups, (std::max(rp, hkv) + 63) / 64, 1, 1, name));
        // A model without rope factors binds a one-float placeholder that is
        // never uploaded (rope_factor_len = 1, phi4.rs:965-967); like
        // apply_rope_cfg's empty list (phi4.rs:243) it means factor 1 for
        // every pair, so a single float is read only when there is a single pair.
        uint32_t nf = bufs[1] ? (uint32_t)std::min<uint64_t>(bufs[1]->bytes / 4, p7[4] / 2) : 0u;
        if (nf == 1 && p7[4] / 2 > 1) nf = 0;
        return rrr_rope_kv_store(ctx, bufs[0], bufs[1], nf, bufs[2], bufs[3], p7[0], p7[1], p7[2], p7[3], p7[4], p7[5],
                                 p7[6], 10000.0f, 1.190238f);
    }
    if (!strcmp(name, "kv_store")) {
        // bufs [qkv, k_cache, v_cache], push [pos, q_dim, kv_stride] (phi4.rs:1670-1677)
        TRY(want_bufs(n_bufs, 3, bufs, name));
        TRY(push_u32(push, push_bytes, 3, pc, name));
        TRY(want_grid(groups, (pc[2] / 2 + 255) / 256, 1, 1, name));
        return rrr_rope_kv_store(ctx, bufs[0], nullptr, 0, bufs[1], bufs[2], pc[0], 0, 0, 0, 0, pc[1], pc[2], 0.0f, 0.0f);
    }
    if (!strcmp(name, "attention")) {
        // bufs [q, k_cache, v_cache, out], push [seq_len, n_kv_heads, heads_per_kv, head_dim], grid [n_heads, 1, 1]
        // (phi4.rs:1018, :1304-1312)
        uint32_t p4[4];
        TRY(want_bufs(n_bufs, 4, bufs, name));
        TRY(push_u32(push, push_bytes, 4, p4, name));
        TRY(want_grid(groups, p4[1] * p4[2], 1, 1, name));
        return rrr_attention(ctx, bufs[0], bufs[1], bufs[2], bufs[3], p4[0], p4[1], p4[2], p4[3]);
    }
    static const char *out_of_scope[] = {"rope", "fused_norm_matmul_q4k", "fused_norm_matmul_q5k",
                                         "fused_norm_matmul_q6k"};
    for (const char *o : out_of_scope)
        if (!strcmp(name, o))
            return fail(RRR_ERR_UNSUPPORTED, "rrr_dispatch: pipeline '%s' is outside the weight-heavy decode path", name);
    return fail(RRR_ERR_UNSUPPORTED, "rrr_dispatch: unknown pipeline '%s'", name);
}

int rrr_dispatch(rrr_ctx *ctx, const char *name, rrr_buf *const *bufs, uint32_t n_bufs, const void *push,
                 uint32_t push_bytes, const uint32_t groups[3])
{
    TRY(check_ctx(ctx));
    return dispatch_one(ctx, name, bufs, n_bufs, push, push_bytes, groups);
}

int rrr_dispatch_batch(rrr_ctx *ctx, const rrr_dispatch_desc *descs, uint32_t n)
{
    TRY(check_ctx(ctx));
    if (!descs && n) return fail(RRR_ERR_NULL, "rrr_dispatch_batch: null descriptor list");
    const bool was_async = ctx->async;
    ctx->async = true;
    for (uint32_t i = 0; i < n; i++) {
        const rrr_dispatch_desc &d = descs[i];
        int rc = dispatch_one(ctx, d.name, d.bufs, d.n_bufs, d.push, d.push_bytes, d.groups);
        if (rc != RRR_OK) {
            ctx->async = was_async;
            std::string msg = g_err;
            return fail(rc, "rrr_dispatch_batch entry %u: %s", i, msg.c_str());
        }
    }
    ctx->async = was_async;
    if (ctx->nodevice || ctx->capturing || ctx->async) return ok();
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return fail(RRR_ERR_HIP, "rrr_dispatch_batch: %s", hipGetErrorString(e));
    return ok();
}

// ---- graphs ------------------------------------------------------------------

int rrr_graph_begin(rrr_ctx *ctx)
{
    TRY(check_ctx(ctx));
    if (ctx->capturing) return fail(RRR_ERR_STATE, "rrr_graph_begin: already capturing");
    TRY(device_ready(ctx));
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e == hipSuccess) e = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return fail(RRR_ERR_HIP, "rrr_graph_begin: %s", hipGetErrorString(e));
    ctx->capturing = true;
    return ok();
}

int rrr_graph_end(rrr_ctx *ctx, rrr_graph **out)
{
    TRY(check_ctx(ctx));
    if (!out) return fail(RRR_ERR_NULL, "rrr_graph_end: null output pointer");
    *out = nullptr;
    if (!ctx->capturing) return fail(RRR_ERR_STATE, "rrr_graph_end: no capture in progress");
    ctx->capturing = false;
    hipGraph_t g = nullptr;
    hipGraphExec_t ex = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->stream, &g);
    if (e == hipSuccess) e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return fail(RRR_ERR_HIP, "rrr_graph_end: %s", hipGetErrorString(e));
    }
    rrr_graph *gr = new rrr_graph{GRAPH_MAGIC, ctx, g, ex};
    ctx->graphs.insert(gr);
    *out = gr;
    return ok();
}

static int check_graph(rrr_ctx *ctx, rrr_graph *g, const char *what)
{
    if (!g) return fail(RRR_ERR_NULL, "%s: null graph", what);
    if (!ctx->graphs.count(g) || g->magic != GRAPH_MAGIC) return fail(RRR_ERR_STALE, "%s: graph already destroyed", what);
    return RRR_OK;
}

int rrr_graph_launch(rrr_ctx *ctx, rrr_graph *g)
{
    TRY(check_ctx(ctx));
    TRY(check_graph(ctx, g, "rrr_graph_launch"));
    if (ctx->capturing) return fail(RRR_ERR_STATE, "rrr_graph_launch: not allowed during capture");
    TRY(device_ready(ctx));
    return finish(ctx, hipGraphLaunch(g->exec, ctx->stream), "rrr_graph_launch");
}

int rrr_graph_destroy(rrr_ctx *ctx, rrr_graph *g)
{
    TRY(check_ctx(ctx));
    TRY(check_graph(ctx, g, "rrr_graph_destroy"));
    if (!ctx->nodevice) {
        (void)hipSetDevice(ctx->device);
        (void)hipStreamSynchronize(ctx->stream);
        (void)hipGraphExecDestroy(g->exec);
        (void)hipGraphDestroy(g->graph);
    }
    ctx->graphs.erase(g);
    g->magic = 0;
    delete g;
    return ok();
}

// ---- sync and timing ----------------------------------------------------------

int rrr_set_async(rrr_ctx *ctx, int async)
{
    TRY(check_ctx(ctx));
    ctx->async = async != 0;
    return ok();
}

int rrr_sync(rrr_ctx *ctx)
{
    TRY(check_ctx(ctx));
    if (ctx->capturing) return fail(RRR_ERR_STATE, "rrr_sync: not allowed during capture");
    TRY(device_ready(ctx));
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return fail(RRR_ERR_HIP, "rrr_sync: %s", hipGetErrorString(e));
    return ok();
}

int rrr_timer_start(rrr_ctx *ctx)
{
    TRY(check_ctx(ctx));
    if (ctx->capturing) return fail(RRR_ERR_STATE, "rrr_timer_start: not allowed during capture");
    TRY(device_ready(ctx));
    hipError_t e = hipEventRecord(ctx->ev0, ctx->stream);
    if (e != hipSuccess) return fail(RRR_ERR_HIP, "rrr_timer_start: %s", hipGetErrorString(e));
    ctx->timer_started = true;
    return ok();
}

int rrr_timer_stop(rrr_ctx *ctx, float *ms)
{
    TRY(check_ctx(ctx));
    if (!ms) return fail(RRR_ERR_NULL, "rrr_timer_stop: null output");
    if (!ctx->timer_started) return fail(RRR_ERR_STATE, "rrr_timer_stop: timer not started");
    TRY(device_ready(ctx));
    hipError_t e = hipEventRecord(ctx->ev1, ctx->stream);
    if (e == hipSuccess) e = hipEventSynchronize(ctx->ev1);
    if (e == hipSuccess) e = hipEventElapsedTime(ms, ctx->ev0, ctx->ev1);
    if (e != hipSuccess) return fail(RRR_ERR_HIP, "rrr_timer_stop: %s", hipGetErrorString(e));
    ctx->timer_started = false;
    return ok();
}

// ---- platform probes ------------------------------------------------------------

int rrr_probe_read(rrr_ctx *ctx, const rrr_buf *buf, uint64_t bytes, rrr_buf *sink)
{
    TRY(check_ctx(ctx));
    const char *what = "rrr_probe_read";
    TRY(check_buf(ctx, buf, what));
    TRY(check_buf(ctx, sink, what));
    if (bytes == 0 || bytes % 16) return fail(RRR_ERR_INVALID_ARG, "%s: bytes must be a positive multiple of 16", what);
    TRY(need(buf, bytes, what));
    TRY(need(sink, 4, what));
    TRY(device_ready(ctx));
    return finish(ctx, launch_probe_read(buf->ptr, bytes, (uint32_t *)sink->ptr, ctx->stream), what);
}

int rrr_probe_read_shares(rrr_ctx *ctx, const rrr_buf *buf, uint64_t bytes, rrr_buf *sink)
{
    TRY(check_ctx(ctx));
    const char *what = "rrr_probe_read_shares";
    TRY(check_buf(ctx, buf, what));
    TRY(check_buf(ctx, sink, what));
    if (bytes == 0 || bytes % 16) return fail(RRR_ERR_INVALID_ARG, "%s: bytes must be a positive multiple of 16", what);
    TRY(need(buf, bytes, what));
    TRY(need(sink, 4, what));
    TRY(device_ready(ctx));
    if (!probe_shares_supported(bytes))
        return fail(RRR_ERR_UNSUPPORTED, "%s: %llu bytes exceed 256 KB per CU", what, (unsigned long long)bytes);
    return finish(ctx, launch_probe_shares(buf->ptr, bytes, (uint32_t *)sink->ptr, ctx->stream), what);
}

int rrr_probe_gemv_phases(rrr_ctx *ctx, uint32_t op, uint32_t act_kind, uint32_t act_param, const rrr_buf *x,
                          const rrr_buf *gamma, float eps, const rrr_buf *W, uint32_t type, rrr_buf *y, uint32_t K,
                          uint32_t N, rrr_buf *stamps, uint32_t *grid_out, uint32_t *waves_out)
{
    TRY(check_ctx(ctx));
    const char *what = "rrr_probe_gemv_phases";
    if (!grid_out || !waves_out) return fail(RRR_ERR_NULL, "%s: null grid / waves output", what);
    TRY(check_buf(ctx, stamps, what));
    GemvArgs a;
    uint32_t act = ACT_PLAIN;
    switch (op) {
    case RRR_PHASES_PLAIN:
        TRY(gemv_prepare(ctx, x, K, nullptr, 0.0f, ACT_PLAIN, 0, 0, W, type, y, K, N, 1, 0, what, a));
        break;
    case RRR_PHASES_RMSNORM:
        if (!gamma) return fail(RRR_ERR_NULL, "%s: null gamma", what);
        act = ACT_RMSNORM;
        TRY(gemv_prepare(ctx, x, K, gamma, eps, ACT_RMSNORM, 0, 0, W, type, y, K, N, 1, 0, what, a));
        break;
    case RRR_PHASES_RESIDUAL: {
        uint64_t x_floats;
        uint32_t hd, hpk;
        TRY(residual_act(act_kind, act_param, K, x_floats, act, hd, hpk, what));
        TRY(gemv_prepare(ctx, x, x_floats, nullptr, 0.0f, act, hd, hpk, W, type, y, K, N, 1, 1, what, a));
        break;
    }
    case RRR_PHASES_RMSNORM_SILU:
        if (!gamma) return fail(RRR_ERR_NULL, "%s: null gamma", what);
        if (N == 0 || N > 0x7FFFFFFFu) return fail(RRR_ERR_BAD_SHAPE, "%s: F=%u", what, N);
        act = ACT_RMSNORM;
        TRY(gemv_prepare(ctx, x, K, gamma, eps, ACT_RMSNORM, 0, 0, W, type, y, K, 2 * N, 1, 0, what, a, N));
        a.N = N;
        a.pair = 1;
        break;
    default:
        return fail(RRR_ERR_INVALID_ARG, "%s: op %u", what, op);
    }
    if (!gemv_mfma_supported(a))
        return fail(RRR_ERR_UNSUPPORTED, "%s: not a shape of the int8-MFMA GEMV (Q4_K/Q5_K/Q6_K, K <= 8192)", what);
    TRY(device_ready(ctx));
    TRY(need(stamps, (uint64_t)device_cu_count() * 16 * 16 * 8, what));
    a.stamps = (uint64_t *)stamps->ptr;
    uint32_t grid = 0, waves = 0;
    const hipError_t e = launch_gemv_mfma_stamped(a, act, ctx->stream, grid, waves);
    *grid_out = grid;
    *waves_out = waves;
    return finish(ctx, e, what);
}

int rrr_probe_mfma(rrr_ctx *ctx, uint32_t kind, uint32_t waves_per_cu, uint32_t iters, rrr_buf *sink)
{
    TRY(check_ctx(ctx));
    const char *what = "rrr_probe_mfma";
    TRY(check_buf(ctx, sink, what));
    if (kind > RRR_PROBE_MFMA_I8_16X16X64) return fail(RRR_ERR_INVALID_ARG, "%s: kind %u", what, kind);
    if (waves_per_cu == 0 || waves_per_cu % 4 || waves_per_cu > 32)
        return fail(RRR_ERR_INVALID_ARG, "%s: waves_per_cu must be a multiple of 4 up to 32", what);
    if (iters == 0) return fail(RRR_ERR_INVALID_ARG, "%s: iters must be positive", what);
    TRY(need(sink, 4, what));
    TRY(device_ready(ctx));
    return finish(ctx, launch_probe_mfma(kind, waves_per_cu, iters, (uint32_t *)sink->ptr, ctx->stream), what);
}

uint32_t rrr_probe_cus(rrr_ctx *ctx)
{
    if (check_ctx(ctx) != RRR_OK || ctx->nodevice || device_ready(ctx) != RRR_OK) return 0;
    return device_cu_count();
}

// ---- one-call helper ------------------------------------------------------------

int rrr_matmul_kquant(rrr_ctx *ctx, rrr_buf *buf_a, const rrr_buf *weight_buf, rrr_buf *buf_c, uint32_t type,
                      const float *a, float *c, uint32_t K, uint32_t N)
{
    TRY(check_ctx(ctx));
    const char *what = "rrr_matmul_kquant";
    if (!a || !c) return fail(RRR_ERR_NULL, "%s: null host vector", what);
    TRY(check_buf(ctx, buf_a, what));
    TRY(check_buf(ctx, buf_c, what));
    TRY(check_buf(ctx, weight_buf, what));
    TRY(check_shape(type, K, N));
    TRY(need(weight_buf, rrr_tensor_bytes(type, K, N), what));
    TRY(need_f32(buf_a, K, what));
    TRY(need_f32(buf_c, N, what));
    if (ctx->capturing) return fail(RRR_ERR_STATE, "%s: not allowed during capture", what);
    TRY(rrr_buf_upload(ctx, buf_a, 0, a, (uint64_t)K * 4));
    const bool was_async = ctx->async;
    ctx->async = false;
    int rc = rrr_gemv(ctx, buf_a, weight_buf, type, buf_c, K, N, 1);
    ctx->async = was_async;
    TRY(rc);
    return rrr_buf_download(ctx, buf_c, 0, c, (uint64_t)N * 4);
}

}  // extern "C"
