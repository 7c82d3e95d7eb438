// internal.h -- launch interface between the C ABI (api.cpp) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rrr {

enum GgmlType : uint32_t { T_F32 = 0, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14 };

// How a GEMV builds its activation vector before the dot products.
enum ActKind : uint32_t {
    ACT_PLAIN = 0,    // x as given (M rows of K)
    ACT_SILU = 1,     // x[k] = silu(src[k]) * src[K + k]   (silu_gate)
    ACT_GQA_V = 2,    // x[k] = src[K + K/hpk + (k / (hd*hpk)) * hd + k % hd]
    ACT_RMSNORM = 3   // x[k] = (gamma[k] * src[k]) * inv_rms(src)
};

struct RopeArgs {
    const float *factors;   // LongRoPE divisors of the first n_factors pairs
    uint32_t n_factors;
    uint32_t pos, n_heads, head_dim, rope_dim, q_dim, kv_stride;
    float theta, attn_factor;
    uint32_t row_stride;    // floats from one token's qkv row to the next (rows > 1)
};

struct GemvArgs {
    uint32_t type;        // GgmlType of W
    const float *x;       // activation source
    const float *gamma;   // ACT_RMSNORM weights
    float eps;
    uint32_t head_dim, heads_per_kv;  // ACT_GQA_V
    const uint8_t *W;
    uint64_t w_bytes;
    float *y;
    uint32_t K, N, M;
    uint32_t residual;    // y += result instead of y = result
    void *ws;             // device workspace of the skinny path's encoded activations
    uint64_t ws_bytes;
    uint32_t pair;        // W holds 2N rows [gate | up]; y[n] = silu(gate row n) * (up row n)
    // rope_kv_store in the epilogue (y = qkv of one token at rope.pos): RoPE
    // pairs rotated before they are stored, K and V also stored as f16 into
    // row rope.pos of kc / vc (rrr_gemv_rmsnorm_rope_kv)
    uint32_t rope_on;
    RopeArgs rope;
    uint32_t *kc, *vc;
    uint64_t *stamps;     // phase timestamps of the stamped launch (rrr_probe_gemv_phases), else unused
};

// Every device buffer is allocated with at least this many bytes past its
// requested size.  Kernels may READ (never write) up to this far past the end
// of a tensor, e.g. a whole 16-byte unit that straddles the end of a Q6_K
// matrix (210-byte blocks).  A view ends inside its parent, so it inherits it.
constexpr uint64_t RRR_READ_SLACK = 16;

uint64_t block_bytes(uint32_t type);  // 144/176/210 per 256 elements, 1024 for F32

hipError_t launch_gemv(const GemvArgs &a, uint32_t act, hipStream_t s);
// int8-MFMA batch-1 K-quant GEMV (gemv_mfma.hip)
bool gemv_mfma_supported(const GemvArgs &a);
hipError_t launch_gemv_mfma(const GemvArgs &a, uint32_t act, hipStream_t s);
// the same launch with phase timestamps into a.stamps (16 u64 per wave of
// each workgroup); returns the grid and the waves per workgroup
hipError_t launch_gemv_mfma_stamped(const GemvArgs &a, uint32_t act, hipStream_t s, uint32_t &grid, uint32_t &waves);
// the same int8-MFMA GEMV for 2 <= M <= MQ_TOKENS_MAX rows of x sharing each
// weight block (plain activations; gemv_mfma.hip)
constexpr uint32_t MQ_TOKENS_MAX = 4;
bool gemv_mq_tokens_supported(const GemvArgs &a);
hipError_t launch_gemv_mq_tokens(const GemvArgs &a, hipStream_t s);
// fp16-MFMA batched GEMV for 2 <= M <= 32, Q4_K / Q5_K (skinny.hip)
bool skinny_supported(const GemvArgs &a);
hipError_t launch_skinny(const GemvArgs &a, hipStream_t s);
// CUs of the current device (cached per device)
uint32_t device_cu_count();
hipError_t launch_dequant(uint32_t type, const uint8_t *W, uint64_t w_bytes, float *out,
                          uint64_t n_elements, hipStream_t s);
hipError_t launch_rmsnorm(const float *x, const float *g, float *y, uint32_t rows, uint32_t d,
                          float eps, hipStream_t s);
hipError_t launch_silu_gate(const float *gu, float *mid, uint32_t rows, uint32_t F, hipStream_t s);
hipError_t launch_residual_add(const float *a, const float *b, float *out, uint32_t n, hipStream_t s);
hipError_t launch_fill_u32(uint32_t *p, uint64_t n_words, uint32_t v, hipStream_t s);
// Transposed-chunk logits (layout 1).  gamma != nullptr fuses the RMSNorm.
hipError_t launch_logits_chunked(const float *x, const float *gamma, float eps, const float *E,
                                 float *y, uint32_t K, uint32_t V, uint32_t chunk, hipStream_t s);
// Split-K transposed-chunk logits (K % 32 == 0, chunk % 256 == 0): `part`
// holds 8 V floats and the slab candidates of the argmax, `counters`
// logits_counter_bytes() zeroed once before the first call (they return to
// zero after every call; calls on one counter area must not overlap).
// token != nullptr: the argmax of the logits is written there too.
constexpr uint32_t LOGITS_MAX_SLABS = 4096;
uint64_t logits_counter_bytes();
bool logits_split_supported(uint32_t K, uint32_t V, uint32_t chunk, uint64_t ws_bytes);
hipError_t launch_logits_split(const float *x, const float *gamma, float eps, const float *E, float *y, uint32_t K,
                               uint32_t V, uint32_t chunk, float *part, uint32_t *counters, uint32_t *token,
                               hipStream_t s);
// Argmax: `partials` holds at least argmax_partials_bytes() bytes.
uint64_t argmax_partials_bytes();
hipError_t launch_argmax(const float *v, uint32_t n, void *partials, uint32_t *out, hipStream_t s);
// RoPE + f16 KV store (attn.hip): the rope_kv_store / kv_store pipelines.
// rows consecutive tokens at positions pos .. pos + rows - 1
hipError_t launch_rope_kv_store(float *qkv, const RopeArgs &r, uint16_t *kc, uint16_t *vc, hipStream_t s,
                                uint32_t rows = 1);
// Decode attention (attn.hip): head_dim ATT_HD, up to ATT_HEADS_MAX query
// heads (ATT_HEADS_MAX KV heads), `scratch` of attention_scratch_bytes()
// zeroed once before the first call (its counters return to zero after
// every call; calls on one scratch area must not overlap).
constexpr uint32_t ATT_HD = 128, ATT_HEADS_MAX = 64, ATT_SPLITS_MAX = 32, ATT_ROWS_PER_GROUP = 4;
constexpr uint32_t ATT_SEQ_MAX = ATT_SPLITS_MAX * 16 * ATT_ROWS_PER_GROUP;   // 2048 cache rows (MAX_SEQ)
// scratch layout: one u32 arrival counter per KV head, each on its own
// 256-byte line, then the split partials (per split and query head: the
// unnormalised output, max and sum, ATT_PART floats)
constexpr uint32_t ATT_PART = ATT_HD + 4;
constexpr uint32_t ATT_COUNTER_STRIDE = 64;   // u32 words between two KV heads' counters
constexpr uint64_t ATT_COUNTER_BYTES = (uint64_t)ATT_HEADS_MAX * ATT_COUNTER_STRIDE * 4;
constexpr uint64_t ATT_SCRATCH_BYTES = ATT_COUNTER_BYTES + (uint64_t)ATT_HEADS_MAX * ATT_SPLITS_MAX * ATT_PART * 4;
uint64_t attention_scratch_bytes();
// The device address of the library's own attention scratch array on device
// `dev` (current), looked up once per device (attn_static.hip).
int attention_static_setup(int dev, void **out);
// Records the thread's error message (RRR_OK clears it); returns code (api.cpp).
int set_error(int code, const char *msg);
void attention_plan(uint32_t seq, uint32_t n_kv_heads, uint32_t heads_per_kv, uint32_t cus, uint32_t &splits,
                    uint32_t &per);
hipError_t launch_attention(const float *q, const uint16_t *kc, const uint16_t *vc, float *out, void *scratch,
                            uint32_t seq, uint32_t n_kv_heads, uint32_t heads_per_kv, uint32_t cus, hipStream_t s);
// Causal prefill attention (attn.hip): token t (< rows) of qkv rows of
// row_stride floats, at position pos0 + t, attends over cache rows
// 0 .. pos0 + t; out rows of n_kv_heads * heads_per_kv * ATT_HD, f32 or f16.
hipError_t launch_attention_prefill(const float *qkv, uint32_t row_stride, uint32_t rows, const uint16_t *kc,
                                    const uint16_t *vc, void *out, bool out_f16, uint32_t pos0, uint32_t n_kv_heads,
                                    uint32_t heads_per_kv, hipStream_t s);
// Prefill dequant-GEMM (gemm.hip): X is M x K bf16 or f16 bits; Y = X . W^T,
// or Y += X . W^T with accumulate; with rscale, row m of the product is
// multiplied by rscale[m] (a power of two: exact) first.  ws (ws_bytes, may
// be null) holds the fp32 partials when K is split.
constexpr size_t GEMM_WS_BYTES = 48ull << 20;
bool gemm_supported(uint32_t type, uint32_t K, uint32_t N, uint32_t M, uint64_t x_bytes);
// bf16 X (any M >= 1, X and Y 16-byte aligned): converted to f16 in row
// chunks inside ws, each chunk zero-padded to a multiple of 128 rows
hipError_t launch_gemm_bf16(const uint16_t *X, const uint8_t *W, uint32_t type, float *Y, uint32_t K, uint32_t N,
                            uint32_t M, float *ws, size_t ws_bytes, hipStream_t s);
// f32 X (the batched GEMV above 16 rows): each row chunk as f16 block floating
// point (row m scaled by a power of two, undone exactly on Y's row) in ws
bool gemm_rows_supported(uint32_t type, uint32_t K, uint32_t N, uint32_t M, size_t ws_bytes);
hipError_t launch_gemm_f32_rows(const float *X, const uint8_t *W, uint32_t type, float *Y, uint32_t K, uint32_t N,
                                uint32_t M, void *ws, size_t ws_bytes, hipStream_t s);
hipError_t launch_gemm_f16(const uint16_t *X, const float *rscale, const uint8_t *W, uint32_t type, float *Y,
                           uint32_t K, uint32_t N, uint32_t M, bool accumulate, float *ws, size_t ws_bytes,
                           hipStream_t s);
// the same GEMM, then the RMSNorm (gamma, eps) of Y's rows in f16 into out16:
// with K split, inside the split reduction (splitk_reduce_rmsnorm_kernel),
// else the rmsnorm launch after the GEMM; N % 4 == 0, N <= 8192
struct GemmNorm {
    const float *gamma;
    float eps;
    uint16_t *out;
};
hipError_t launch_gemm_f16_rmsnorm(const uint16_t *X, const float *rscale, const uint8_t *W, uint32_t type, float *Y,
                                   uint32_t K, uint32_t N, uint32_t M, bool accumulate, const float *gamma, float eps,
                                   uint16_t *out16, float *ws, size_t ws_bytes, hipStream_t s);
// the QKV GEMM (accumulate 0, no row scale) of the prompt's M rows into the
// qkv rows Y, then the rope_kv_store of its first `rows` rows at positions
// r.pos ..: with K split, inside the split reduction
// (splitk_rope_kv_store_kernel), else the rope launch after the GEMM
struct GemmRope {
    RopeArgs r;
    uint32_t rows;
    uint16_t *kc, *vc;
};
hipError_t launch_gemm_f16_rope_kv(const uint16_t *X, const uint8_t *W, uint32_t type, float *Y, uint32_t K,
                                   uint32_t N, uint32_t M, const RopeArgs &r, uint32_t rows, uint16_t *kc,
                                   uint16_t *vc, float *ws, size_t ws_bytes, hipStream_t s);
// the gate/up GEMM (N = 2F: F gate rows, F up rows) with silu(gate) * up in
// its epilogue into ws (M x F f32), then silu_gate_f16's block floating
// point rows from those values (launch_f16_rows_scaled)
hipError_t launch_gemm_f16_silu_f16(const uint16_t *X, const uint8_t *W, uint32_t type, uint16_t *mid, float *rscale,
                                    uint32_t K, uint32_t F, uint32_t M, float *ws, size_t ws_bytes, hipStream_t s);
hipError_t launch_f16_rows_scaled(const float *v, uint16_t *mid, float *rscale, uint32_t rows, uint32_t F,
                                  hipStream_t s);
bool splitk_rope_kv_store_supported(const RopeArgs &r);
hipError_t launch_splitk_rope_kv_store(const float *ws, uint32_t S, uint32_t M, float *qkv, const RopeArgs &r,
                                       uint32_t rows, uint16_t *kc, uint16_t *vc, hipStream_t s);
bool splitk_reduce_rmsnorm_supported(uint32_t d);
hipError_t launch_splitk_reduce_rmsnorm(const float *ws, uint32_t S, uint32_t M, uint32_t d, float *Y,
                                        const float *rscale, bool acc, const float *g, float eps, uint16_t *out,
                                        hipStream_t s);
// f16 (round to nearest even) outputs of RMSNorm rows and of silu_gate rows
// (the latter scaled per row by a power of two, rscale undoing it), the
// activations of the prefill GEMMs (ops.hip)
hipError_t launch_rmsnorm_f16(const float *x, const float *g, uint16_t *y, uint32_t rows, uint32_t d, float eps,
                              hipStream_t s);
hipError_t launch_silu_gate_f16(const float *gu, uint16_t *mid, float *rscale, uint32_t rows, uint32_t F,
                                hipStream_t s);

// Platform probes (probe.hip)
hipError_t launch_probe_read(const void *p, uint64_t bytes, uint32_t *out, hipStream_t s);
bool probe_shares_supported(uint64_t bytes);
hipError_t launch_probe_shares(const void *p, uint64_t bytes, uint32_t *out, hipStream_t s);
hipError_t launch_probe_mfma(uint32_t kind, uint32_t waves_per_cu, uint32_t iters, uint32_t *out, hipStream_t s);

}  // namespace rrr
