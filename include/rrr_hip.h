/*
 * rrr_hip.h -- C ABI of librrr_hip.so, the MI355X (gfx950) replacement for the
 * reference's Vulkan compute engine on the weight-heavy decode path.
 *
 * The reference host (src/model/phi4.rs) reaches the GPU only through
 * ComputeEngine / GpuBuffer / DescSetHandle (src/gpu/mod.rs:3).  Every entry
 * point below names the reference interface it replaces.  All functions:
 *   - return an int status (RRR_OK = 0, negative on error) and never abort;
 *   - validate every argument before any HIP call, so the error paths run on a
 *     machine without a GPU;
 *   - record a human-readable message retrievable with rrr_last_error()
 *     (thread-local).
 *
 * Weights are the raw GGUF bytes uploaded unchanged (no host repack):
 * N rows of K/256 super-blocks, row n's blocks contiguous (GGUF ne0 = K inner,
 * ne1 = N rows; phi4.rs:748-749).  Activations and outputs are f32 row-major
 * per token, as in phi4.rs:1236-1238.
 *
 * Threading: one context = one HIP stream.  A context must not be used from
 * two threads at once (the reference engine has the same restriction: one
 * shared command buffer and fence, engine.rs:21-23).  By default every call
 * that launches work waits for it before returning, matching the reference's
 * submit + wait_for_fences on every dispatch (engine.rs:312, :369, :470,
 * :550).  rrr_set_async(ctx, 1) turns that off; rrr_sync() then waits.
 */
#ifndef RRR_HIP_H
#define RRR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RRR_ABI_VERSION 1

typedef enum rrr_status {
    RRR_OK = 0,
    RRR_ERR_INVALID_ARG = -1,  /* bad size, count, flag or range */
    RRR_ERR_BAD_TYPE = -2,     /* ggml type not in {0, 12, 13, 14} */
    RRR_ERR_BAD_SHAPE = -3,    /* K % 256 != 0 for a K-quant, zero dims, ... */
    RRR_ERR_SHORT_BUFFER = -4, /* a buffer is smaller than the op reads/writes */
    RRR_ERR_NULL = -5,         /* null handle or pointer */
    RRR_ERR_HIP = -6,          /* a HIP runtime call failed */
    RRR_ERR_UNSUPPORTED = -7,  /* pipeline name or shape the library does not run */
    RRR_ERR_NO_DEVICE = -8,    /* no such HIP device */
    RRR_ERR_STATE = -9,        /* call not allowed in the context's state */
    RRR_ERR_STALE = -10        /* handle already destroyed */
} rrr_status;

/* GGUF tensor types on the path (gguf.rs:179, :187-189). */
typedef enum rrr_ggml_type {
    RRR_TYPE_F32 = 0,
    RRR_TYPE_F16 = 1,    /* activations only (prefill attention output) */
    RRR_TYPE_Q4_K = 12,
    RRR_TYPE_Q5_K = 13,
    RRR_TYPE_Q6_K = 14
} rrr_ggml_type;

/* Logits weight layouts. */
typedef enum rrr_logits_layout {
    RRR_LOGITS_ROWS = 0,    /* E[v][d], V rows of K f32 (token_embd order) */
    RRR_LOGITS_CHUNKED = 1, /* reference chunks: B_c[d*n + v] = E[(c*chunk+v)*K + d]
                               (phi4.rs:874-893), chunks back to back */
    RRR_LOGITS_Q6K = 2      /* the tied token_embd as stored: V rows of K/256 raw
                               Q6_K super-blocks, the tensor the reference
                               dequantizes to build its F32 copy (phi4.rs:709,
                               :866-893); chunk is unused */
} rrr_logits_layout;

typedef struct rrr_ctx rrr_ctx;
typedef struct rrr_buf rrr_buf;
typedef struct rrr_graph rrr_graph;

/* ---- engine lifetime ------------------------------------------------- */

/* Replaces ComputeEngine::new (engine.rs:49-128): picks HIP device `device`
 * (the reference always takes pdevices[0], engine.rs:62-63) and creates the
 * context's stream.  device == RRR_DEVICE_NONE creates a validation-only
 * context: buffers are placeholders with a size and no memory, every call
 * validates its arguments as usual and then returns RRR_ERR_NO_DEVICE instead
 * of touching a GPU. */
#define RRR_DEVICE_NONE (-1)
int rrr_init(int device, rrr_ctx **out);
/* Replaces Drop for ComputeEngine (engine.rs:557-579): waits for the device,
 * frees every buffer and graph still owned by the context. */
int rrr_destroy(rrr_ctx *ctx);
/* Thread-local text of the last error ("" if none). */
const char *rrr_last_error(void);
int rrr_abi_version(void);
/* Number of HIP devices visible (0 when there is no GPU); never fails. */
int rrr_device_count(void);

/* ---- buffers --------------------------------------------------------- */

/* Replaces ComputeEngine::alloc_buffer (engine.rs:200-229).  The reference
 * allocates host-visible mapped memory; here buffers live in device HBM,
 * 256-byte aligned, and data moves with rrr_buf_upload / rrr_buf_download. */
int rrr_buf_alloc(rrr_ctx *ctx, uint64_t bytes, rrr_buf **out);
/* A view of [offset, offset+bytes) of `parent`; it shares the parent's memory
 * and must not outlive it.  Used where the reference binds sub-ranges. */
int rrr_buf_view(rrr_ctx *ctx, rrr_buf *parent, uint64_t offset, uint64_t bytes, rrr_buf **out);
/* Frees a buffer or view (the reference only frees pooled buffers at Drop,
 * engine.rs:557-566). */
int rrr_buf_free(rrr_ctx *ctx, rrr_buf *buf);
/* Size in bytes (GpuBuffer.capacity, engine.rs:42); 0 for a null handle. */
uint64_t rrr_buf_size(const rrr_buf *buf);
/* Replaces upload / upload_bytes (phi4.rs:616-622): memcpy into .mapped. */
int rrr_buf_upload(rrr_ctx *ctx, rrr_buf *buf, uint64_t offset, const void *src, uint64_t bytes);
/* Replaces download (phi4.rs:624-626) and the zero-copy reads of mapped
 * logits (phi4.rs:1178, :1190). */
int rrr_buf_download(rrr_ctx *ctx, const rrr_buf *buf, uint64_t offset, void *dst, uint64_t bytes);
/* Fills bytes [offset, offset+bytes) with a 32-bit pattern (offset and bytes
 * multiples of 4).  Uses a kernel, never hipMemset, so it may be captured. */
int rrr_buf_fill_u32(rrr_ctx *ctx, rrr_buf *buf, uint64_t offset, uint64_t bytes, uint32_t value);

/* ---- weights --------------------------------------------------------- */

/* Bytes of an N x K tensor of `type`: N * (K/256) * {144,176,210} for the
 * K-quants (gguf.rs:187-189), N * K * 4 for F32.  Returns 0 for an invalid
 * type or K. */
uint64_t rrr_tensor_bytes(uint32_t type, uint32_t K, uint32_t N);
/* Replaces load_weight_gpu (phi4.rs:744-771) without its repack step
 * (phi4.rs:752-755): the raw GGUF bytes are copied to HBM unchanged.
 * Checks type, K % 256 == 0 for K-quants and bytes >= rrr_tensor_bytes(). */
int rrr_weight_upload(rrr_ctx *ctx, uint32_t type, uint32_t K, uint32_t N, const void *raw,
                      uint64_t bytes, rrr_buf **out);

/* ---- typed ops (each a single kernel launch on the context stream) --- */

/* Dequantize n_elements (multiple of 256) of raw `type` blocks to f32,
 * bit-exact with dequant_q4_k / dequant_q5_k / dequant_q6_k
 * (phi4.rs:444-542) and dequant_tensor_f32 (phi4.rs:572-587). */
int rrr_dequant(rrr_ctx *ctx, uint32_t type, const rrr_buf *W, rrr_buf *out, uint64_t n_elements);

/* Y[m][n] = sum_k X[m][k] * W[n][k] for m < M, n < N.
 * M == 1 replaces matmul_q{4,5,6}k / matmul_gpuq{4,5,6} (push [K, N], grid
 * [N,1,1]; phi4.rs:631-658, :1081-1096) and matmul_tiled for F32 weights
 * (phi4.rs:641-646).  M > 1 replaces matmul_gpuq*_batch (push [K, N, M],
 * grid [N, M, 1]; phi4.rs:1257-1268, :1346-1391), which the reference's
 * prefill calls with M = the prompt length.  type 0 means F32 W stored
 * row-major N x K.  Accuracy: within 1e-4 normwise of the exact product per
 * row up to M = 16; above 16 rows the K-quant rows run on the fp16 matrix
 * cores (Q4_K / Q5_K with K <= 3072 up to 32 rows, every K-quant shape with
 * N % 64 == 0, X and Y 16-byte aligned, beyond: X as f16 rows with a
 * power-of-two scale per row, zero-padded to 128 rows in the context
 * workspace) within 2e-3. */
int rrr_gemv(rrr_ctx *ctx, const rrr_buf *X, const rrr_buf *W, uint32_t type, rrr_buf *Y,
             uint32_t K, uint32_t N, uint32_t M);

/* Y[m][n] = sum_k float(X_bf16[m][k]) * W[n][k]: the prefill dequant-GEMM
 * (MFMA, fp16 tiles, fp32 accumulate).  No reference counterpart exists for the
 * MFMA kernel; its call shape is the batched one above with X in bf16.  Any
 * M >= 1: X is converted to f16 (exact in f16's normal range) in row chunks
 * inside the context workspace, each padded with zero rows to a multiple of
 * 128.  K-quant W with N % 64 == 0 (else RRR_ERR_UNSUPPORTED); X and Y
 * 16-byte aligned. */
int rrr_gemm_bf16(rrr_ctx *ctx, const rrr_buf *X_bf16, const rrr_buf *W, uint32_t type,
                  rrr_buf *Y, uint32_t K, uint32_t N, uint32_t M);

/* y[r] = (gamma * x[r]) / sqrt(mean(x[r]^2) + eps) for r < rows.
 * Replaces the rmsnorm pipeline (push [rows, d]; phi4.rs:1006, :1043-1047;
 * CPU twin rms_norm phi4.rs:593-599 with eps RMS_EPS = 1e-5, :111). */
int rrr_rmsnorm(rrr_ctx *ctx, const rrr_buf *x, const rrr_buf *gamma, rrr_buf *y,
                uint32_t rows, uint32_t d, float eps);

/* mid[r][i] = silu(gu[r][i]) * gu[r][F + i]: replaces silu_gate (push [F];
 * phi4.rs:1028-1029; CPU twin :1369-1373). */
int rrr_silu_gate(rrr_ctx *ctx, const rrr_buf *gate_up, rrr_buf *mid, uint32_t rows, uint32_t F);

/* out = a + b over n floats (out may alias a): replaces residual_add
 * (push [d]; phi4.rs:1023, :1033; CPU twin elemwise_add :608-610). */
int rrr_residual_add(rrr_ctx *ctx, const rrr_buf *a, const rrr_buf *b, rrr_buf *out, uint32_t n);

/* logits[v] = sum_d x[d] * E[v][d] for v < V in one launch.  Replaces the
 * chunked matmul_tiled logit dispatches (phi4.rs:1049-1064, :1416-1434):
 * layout RRR_LOGITS_CHUNKED accepts the reference's transposed chunks of
 * `chunk` rows (8192 in the reference) back to back, RRR_LOGITS_ROWS the
 * untransposed E.  RRR_LOGITS_Q6K reads the raw Q6_K token_embd instead of
 * its F32 expansion: E[v][d] = dequant_q6_k (phi4.rs:444-479) of row v, the
 * same values the F32 layouts hold, from 4.9x fewer bytes (K % 256 == 0). */
int rrr_logits_f32(rrr_ctx *ctx, const rrr_buf *x, const rrr_buf *E, rrr_buf *logits, uint32_t K,
                   uint32_t V, uint32_t layout, uint32_t chunk);

/* Index of the largest logit (first on ties, NaN never wins), written as a
 * u32 to out_index: replaces the CPU argmax over the mapped logit chunks
 * (phi4.rs:1172-1183). */
int rrr_argmax_f32(rrr_ctx *ctx, const rrr_buf *logits, uint32_t V, rrr_buf *out_index);

/* ---- decode glue: RoPE + f16 KV cache, decode attention -------------- */

/* The rope_kv_store pipeline (phi4.rs:1016-1017; push [pos, n_heads,
 * n_kv_heads, head_dim, rope_dim, q_dim, kv_stride], :1115-1117).  qkv holds
 * [q(q_dim) | k(kv_stride) | v(kv_stride)] f32.  RoPE as apply_rope_cfg
 * (phi4.rs:238-256) rotates pairs (2i, 2i+1), i < rope_dim/2, of every Q
 * head and every K head in place: freq_i = theta^(-2i/rope_dim) / f_i
 * (f_i = rope_factors[i] for i < n_factors, else 1), angle = pos * freq_i,
 * cos and sin scaled by attn_factor.  Then K and V are stored as f16 (round
 * to nearest even) into row pos of k_cache / v_cache (rows of kv_stride f16,
 * the MAX_SEQ x kv_stride caches of phi4.rs:894-903).  rope_dim = 0 skips the
 * rotation: the kv_store pipeline (phi4.rs:1666-1677).  Phi-4-mini:
 * theta 10000, attn_factor 1.190238, rope_dim 96 (phi4.rs:114-116). */
int rrr_rope_kv_store(rrr_ctx *ctx, rrr_buf *qkv, const rrr_buf *rope_factors, uint32_t n_factors,
                      rrr_buf *k_cache, rrr_buf *v_cache, uint32_t pos, uint32_t n_heads,
                      uint32_t n_kv_heads, uint32_t head_dim, uint32_t rope_dim, uint32_t q_dim,
                      uint32_t kv_stride, float theta, float attn_factor);

/* The layer's first three dispatches, rmsnorm -> matmul (QKV) ->
 * rope_kv_store (phi4.rs:1006-1017), as one launch: rrr_gemv_rmsnorm of x
 * (K floats, gamma, eps) against W (type, K x N, N = q_dim + 2 * kv_stride)
 * into qkv, with the rope_kv_store of that row at position pos in the GEMV's
 * epilogue (same arguments and checks as rrr_rope_kv_store).  qkv, k_cache
 * and v_cache end bit for bit as after rrr_gemv_rmsnorm followed by
 * rrr_rope_kv_store; shapes the fused epilogue does not take run those two
 * launches. */
int rrr_gemv_rmsnorm_rope_kv(rrr_ctx *ctx, const rrr_buf *x, const rrr_buf *gamma, float eps,
                             const rrr_buf *W, uint32_t type, rrr_buf *qkv, uint32_t K,
                             const rrr_buf *rope_factors, uint32_t n_factors, rrr_buf *k_cache,
                             rrr_buf *v_cache, uint32_t pos, uint32_t n_heads, uint32_t n_kv_heads,
                             uint32_t head_dim, uint32_t rope_dim, uint32_t q_dim, uint32_t kv_stride,
                             float theta, float attn_factor);

/* The attention pipeline (phi4.rs:1018, :1304-1312; push [seq_len,
 * n_kv_heads, heads_per_kv, head_dim], one workgroup per query head in the
 * reference): for query head h (h < n_kv_heads * heads_per_kv) and KV head
 * g = h / heads_per_kv, out[h] = sum_t softmax_t(q_h . k_t / sqrt(head_dim))
 * v_t over cache rows t < seq_len (f16 K and V, f32 arithmetic).  q and out
 * are n_heads * head_dim f32 (16-byte aligned), the caches 16-byte aligned.
 * head_dim must be 128, heads_per_kv at most 8 and seq_len at most 2048
 * (the reference's MAX_SEQ, phi4.rs:181). */
int rrr_attention(rrr_ctx *ctx, const rrr_buf *q, const rrr_buf *k_cache, const rrr_buf *v_cache,
                  rrr_buf *out, uint32_t seq_len, uint32_t n_kv_heads, uint32_t heads_per_kv,
                  uint32_t head_dim);
/* rrr_attention that allocates nothing.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Plain
 * device pointers of the current device and a HIP stream (a hipStream_t;
 * NULL = the default stream); the launch is asynchronous on that stream.
 * The same kernels and plan as rrr_attention, so the output is the same bits
 * for the same inputs and seq_len.  The split partials and arrival counters
 * live in a 1,097,728-byte device array of the library (held by each device
 * it runs on until the process ends), not in a context: every call on one
 * device shares it, so calls that overlap on one device (two streams, two
 * threads) race; the counters are cleared by a fill kernel at the start of
 * each call.  Limits, checked before any launch (RRR_ERR_UNSUPPORTED beyond
 * them): seq_len <= 2048, heads_per_kv <= 8, n_kv_heads * heads_per_kv <= 64,
 * head_dim 128; q, out and the caches 16-byte aligned.  Calls no hipMalloc,
 * hipFree or allocating library routine. */
int rrr_attention_noalloc(const float *q, const uint16_t *k_cache, const uint16_t *v_cache, float *out,
                          uint32_t seq_len, uint32_t n_kv_heads, uint32_t heads_per_kv, uint32_t head_dim,
                          void *stream);

/* ---- prefill (forward_prefill_batched, phi4.rs:1200-1445, on the GPU) -- */

/* rope_kv_store for `rows` prompt tokens in one launch: token t's qkv row
 * (q_dim + 2 * kv_stride floats, rows back to back) at position pos0 + t,
 * rotated in place and its K/V stored into cache row pos0 + t (the
 * per-token rope_kv_store dispatches of phi4.rs:1285-1298).  Same arguments
 * and checks as rrr_rope_kv_store otherwise. */
int rrr_rope_kv_store_rows(rrr_ctx *ctx, rrr_buf *qkv, uint32_t rows, const rrr_buf *rope_factors,
                           uint32_t n_factors, rrr_buf *k_cache, rrr_buf *v_cache, uint32_t pos0,
                           uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim, uint32_t rope_dim,
                           uint32_t q_dim, uint32_t kv_stride, float theta, float attn_factor);
/* Causal attention of the prompt (the per-token attention dispatches of
 * phi4.rs:1304-1312 in one launch): token t's query (the first
 * n_kv_heads * heads_per_kv * head_dim floats of its qkv row, rows as in
 * rrr_rope_kv_store_rows) attends over cache rows 0 .. pos0 + t, as
 * rrr_attention with seq_len = pos0 + t + 1.  out: rows of n_heads * head_dim,
 * out_type RRR_TYPE_F32 or RRR_TYPE_F16 (rounded to nearest even, the input
 * of rrr_gemm_f16).  head_dim 128, heads_per_kv <= 8, pos0 + rows <= 2048;
 * qkv and the caches 16-byte aligned. */
int rrr_attention_prefill(rrr_ctx *ctx, const rrr_buf *qkv, uint32_t rows, const rrr_buf *k_cache,
                          const rrr_buf *v_cache, rrr_buf *out, uint32_t out_type, uint32_t pos0,
                          uint32_t n_kv_heads, uint32_t heads_per_kv, uint32_t head_dim);
/* Y = P (accumulate 0) or Y += P (accumulate 1, the residual adds of
 * phi4.rs:1321-1325 and :1396-1404 folded in), P = X . W^T with X an M x K
 * f16 matrix, row m of P multiplied by row_scale[m] when row_scale is given
 * (f32 powers of two, as rrr_silu_gate_f16 returns them; null: 1): the
 * batched prompt GEMMs of phi4.rs:1257-1268, :1346-1391 on the prefill MFMA
 * kernel (weights dequantized to f16 tiles, f32 accumulate).  Needs
 * M % 128 == 0 and N % 64 == 0 (pad the prompt with zero rows). */
int rrr_gemm_f16(rrr_ctx *ctx, const rrr_buf *X_f16, const rrr_buf *row_scale, const rrr_buf *W,
                 uint32_t type, rrr_buf *Y, uint32_t K, uint32_t N, uint32_t M, uint32_t accumulate);
/* rrr_rmsnorm (phi4.rs:593-599) with the same f32 results rounded to f16
 * (nearest even), the input of rrr_gemm_f16 (|y| <= sqrt(d) * max|gamma|). */
int rrr_rmsnorm_f16(rrr_ctx *ctx, const rrr_buf *x, const rrr_buf *gamma, rrr_buf *y_f16, uint32_t rows,
                    uint32_t d, float eps);
/* rrr_gemm_f16 into Y, then rrr_rmsnorm_f16(Y, gamma, y_f16, M, N, eps) of the
 * updated rows, as one call: the prefill layer's O-proj and FFN-down, whose
 * residual rows feed the next norm (phi4.rs:1321-1339, :1396-1404 then the
 * next layer's :1234-1246).  Results bitwise those of the two calls; when K
 * is split over workgroups the norm is taken inside the split reduction, so
 * the rows are not read again.  Needs N % 4 == 0 and N <= 8192 besides
 * rrr_gemm_f16's shape rules.  No counterpart call in the reference (it
 * runs these as separate dispatches). */
int rrr_gemm_f16_rmsnorm(rrr_ctx *ctx, const rrr_buf *X_f16, const rrr_buf *row_scale, const rrr_buf *W,
                         uint32_t type, rrr_buf *Y, uint32_t K, uint32_t N, uint32_t M, uint32_t accumulate,
                         const rrr_buf *gamma, float eps, rrr_buf *y_f16);
/* The prompt's QKV step (phi4.rs:1257-1268 batched matmul, then the
 * per-token rope_kv_store dispatches of :1285-1298): qkv = X . W^T as
 * rrr_gemm_f16 (accumulate 0, no row scale; N = q_dim + 2 * kv_stride, M
 * rows), then rrr_rope_kv_store_rows of its first `rows` rows at positions
 * pos0 .. (same RoPE arguments and checks).  With K split over workgroups
 * the split reduction and the RoPE + KV store are one launch.  qkv and the
 * caches end bit for bit as after those two calls.  q_dim and kv_stride
 * % 4 == 0, qkv 16-byte aligned.  No counterpart call in the reference. */
int rrr_gemm_f16_rope_kv_rows(rrr_ctx *ctx, const rrr_buf *X_f16, const rrr_buf *W, uint32_t type, rrr_buf *qkv,
                              uint32_t K, uint32_t M, uint32_t rows, const rrr_buf *rope_factors,
                              uint32_t n_factors, rrr_buf *k_cache, rrr_buf *v_cache, uint32_t pos0,
                              uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim, uint32_t rope_dim,
                              uint32_t q_dim, uint32_t kv_stride, float theta, float attn_factor);
/* rrr_silu_gate (phi4.rs:1369-1373) in f16 block floating point: row r's f32
 * results v, with max|v| = f * 2^e (f in [0.5, 1)), stored as
 * f16(v * 2^(15 - e)) (nearest even; the scaling is exact) and
 * row_scale[r] = 2^(e - 15) (f32); a row without a finite nonzero maximum
 * is stored unscaled (row_scale 1).  Keeps f16's 11 significant bits for
 * activations of any size; pass row_scale to rrr_gemm_f16. */
int rrr_silu_gate_f16(rrr_ctx *ctx, const rrr_buf *gate_up, rrr_buf *mid_f16, rrr_buf *row_scale,
                      uint32_t rows, uint32_t F);

/* The prompt's gate/up step (phi4.rs:1346-1373: the batched ffn_up matmul
 * into the 2F gate_up rows, then silu_gate): rrr_gemm_f16 of X (M x K f16)
 * against W (N = 2F rows: F gate rows, then F up rows; accumulate 0, no row
 * scale) followed by rrr_silu_gate_f16 of its rows, with silu(gate) * up
 * taken in the GEMM's epilogue, so no M x 2F gate_up rows are written or
 * read back.  mid_f16 and row_scale end bit for bit as after the two calls.
 * Needs M % 256 == 0, F % 64 == 0, (F / 64) * (M / 256) >= 128 (the GEMM
 * covers the CUs without a K split) and M * F * 4 bytes of the context's
 * GEMM workspace (48 MiB); RRR_ERR_UNSUPPORTED otherwise, and the two calls
 * do the step.  No counterpart call in the reference. */
int rrr_gemm_f16_silu_gate_f16(rrr_ctx *ctx, const rrr_buf *X_f16, const rrr_buf *W, uint32_t type,
                               rrr_buf *mid_f16, rrr_buf *row_scale, uint32_t K, uint32_t F, uint32_t M);

/* ---- fused decode-sweep ops (the four launches per layer) ------------ */

/* Y = W . rmsnorm(x, gamma, eps): RMSNorm folded into the GEMV's activation
 * staging (the reference registers fused_norm_matmul_q{4,5,6}k, phi4.rs:725-727,
 * but never dispatches them).  Y is bit-identical to rrr_rmsnorm followed by
 * rrr_gemv. */
int rrr_gemv_rmsnorm(rrr_ctx *ctx, const rrr_buf *x, const rrr_buf *gamma, float eps,
                     const rrr_buf *W, uint32_t type, rrr_buf *Y, uint32_t K, uint32_t N);
/* Y[f] = silu(g[f]) * u[f] for f < F, where [g | u] = W . rmsnorm(x, gamma,
 * eps) over W's 2F rows (F gate rows, then F up rows): the ffn_up matmul into
 * the 2F gate_up buffer followed by silu_gate (phi4.rs:1025-1029) as one
 * launch, so the down GEMV reads F activations instead of 2F.  The silu is
 * RRR_ACT_SILU_GATE's, on the row sums rrr_gemv_rmsnorm computes: Y is
 * bitwise that activation of rrr_gemv_rmsnorm's 2F outputs.  Q4_K, Q5_K and
 * Q6_K rows, K % 256 == 0, K <= 8192 (RRR_ERR_UNSUPPORTED otherwise). */
int rrr_gemv_rmsnorm_silu(rrr_ctx *ctx, const rrr_buf *x, const rrr_buf *gamma, float eps,
                          const rrr_buf *W, uint32_t type, rrr_buf *Y, uint32_t K, uint32_t F);
/* hidden[n] += sum_k act(x)[k] * W[n][k] (residual_add folded into the GEMV's
 * epilogue, phi4.rs:1020-1023 and :1030-1033).  act_kind:
 *   RRR_ACT_IDENTITY  act(x) = x[0..K)
 *   RRR_ACT_SILU_GATE act(x)[k] = silu(x[k]) * x[K + k]   (silu_gate, :1028-1029)
 *   RRR_ACT_GQA_V     act(x)[k] = x[K + K/hpk + (k / (hd*hpk))*hd + k % hd], the
 *                     output of single-query GQA attention at position 0 (the
 *                     softmax over one key is 1, so head h returns V of kv head
 *                     h / hpk); x is the fused QKV vector [q(K) | k(K/hpk) | v(K/hpk)].
 *                     act_param = hd | (hpk << 16), hd % 16 == 0.
 * act_param is ignored for the other kinds. */
enum { RRR_ACT_IDENTITY = 0, RRR_ACT_SILU_GATE = 1, RRR_ACT_GQA_V = 2 };
int rrr_gemv_residual(rrr_ctx *ctx, const rrr_buf *x, uint32_t act_kind, uint32_t act_param,
                      const rrr_buf *W, uint32_t type, rrr_buf *hidden, uint32_t K, uint32_t N);
/* logits = E . rmsnorm(x, gamma, eps), E in any rrr_logits_layout. */
int rrr_logits_rmsnorm(rrr_ctx *ctx, const rrr_buf *x, const rrr_buf *gamma, float eps,
                       const rrr_buf *E, rrr_buf *logits, uint32_t K, uint32_t V, uint32_t layout,
                       uint32_t chunk);
/* rrr_logits_rmsnorm, then the index of the largest logit as rrr_argmax_f32
 * defines it (first on ties, NaN never wins), written as a u32 to out_index:
 * the final logits dispatches (phi4.rs:1049-1064) and the host argmax over
 * the mapped chunks (phi4.rs:1172-1183) in one call.  On the transposed-chunk
 * layout the argmax runs inside the logits launch (the last workgroup of each
 * 256-entry slab reduces the slab, the last slab reduces the slabs); the
 * logits are bit-identical to rrr_logits_rmsnorm's. */
int rrr_logits_rmsnorm_argmax(rrr_ctx *ctx, const rrr_buf *x, const rrr_buf *gamma, float eps,
                              const rrr_buf *E, rrr_buf *logits, uint32_t K, uint32_t V,
                              uint32_t layout, uint32_t chunk, rrr_buf *out_index);

/* ---- name-keyed dispatch shim ---------------------------------------- */

/* Replaces dispatch_by_name (engine.rs:476-486) for the reference's pipelines,
 * with their exact binding order and little-endian u32 push layouts:
 *   matmul_q4k/q5k/q6k, matmul_gpuq4/5/6  bufs [x, W, y],  push [K, N]
 *   matmul_gpuq{4,5,6}_batch              bufs [X, W, Y],  push [K, N, M]
 *   matmul_tiled                          bufs [A, B, C],  push [M, K, N]
 *     (B is K x N row-major, as the logit chunks are; phi4.rs:886)
 *   rmsnorm                               bufs [x, g, y],  push [rows, d]
 *   silu_gate                             bufs [gu, mid],  push [F]
 *   residual_add                          bufs [a, b, out], push [d]
 *   rope_kv_store   bufs [qkv, rope_factors, k_cache, v_cache],
 *                   push [pos, n_heads, n_kv_heads, head_dim, rope_dim, q_dim, kv_stride]
 *   kv_store        bufs [qkv, k_cache, v_cache], push [pos, q_dim, kv_stride]
 *   attention       bufs [q, k_cache, v_cache, out],
 *                   push [seq_len, n_kv_heads, heads_per_kv, head_dim]
 * The matmul_gpuq* names take RAW GGUF bytes here (the repack is gone) with
 * the type implied by the name.  The grid argument is accepted for call-shape
 * compatibility and checked against the push constants; launch geometry is
 * chosen by the library.  Unknown names and the out-of-scope pipelines
 * (rope, fused_norm_matmul_q*k) return RRR_ERR_UNSUPPORTED.  rmsnorm uses
 * eps = 1e-5 and rope_kv_store theta 10000 / attention factor 1.190238, baked
 * in as the reference's shaders do; rope_kv_store takes the first
 * min(size / 4, rope_dim / 2) floats of rope_factors as the LongRoPE
 * factors. */
int rrr_dispatch(rrr_ctx *ctx, const char *name, rrr_buf *const *bufs, uint32_t n_bufs,
                 const void *push, uint32_t push_bytes, const uint32_t groups[3]);

/* One entry of a dispatch batch: replaces the tuples of
 * dispatch_batch_persistent_v2 (engine.rs:317-370) / dispatch_batch
 * (engine.rs:380-386).  `barrier` is accepted for shape compatibility; every
 * launch on the context stream is ordered after the previous one. */
typedef struct rrr_dispatch_desc {
    const char *name;
    rrr_buf *const *bufs;
    uint32_t n_bufs;
    const void *push;
    uint32_t push_bytes;
    uint32_t groups[3];
    uint32_t barrier;
} rrr_dispatch_desc;
/* Launches all entries in order, then waits once (one "submit"). */
int rrr_dispatch_batch(rrr_ctx *ctx, const rrr_dispatch_desc *descs, uint32_t n);

/* ---- HIP graphs (replace the pre-built mega-batch table) ------------- */

/* Between rrr_graph_begin and rrr_graph_end every op above is recorded into a
 * HIP graph instead of run (no waits inside).  rrr_graph_launch replays it,
 * the MI355X counterpart of replaying mega_dispatches through
 * dispatch_batch_persistent_v2 (phi4.rs:972-1064, :1163-1168). */
int rrr_graph_begin(rrr_ctx *ctx);
int rrr_graph_end(rrr_ctx *ctx, rrr_graph **out);
int rrr_graph_launch(rrr_ctx *ctx, rrr_graph *g);
int rrr_graph_destroy(rrr_ctx *ctx, rrr_graph *g);

/* ---- synchronisation and timing -------------------------------------- */

int rrr_set_async(rrr_ctx *ctx, int async);
int rrr_sync(rrr_ctx *ctx);
/* HIP events recorded on the context stream; elapsed milliseconds between the
 * last rrr_timer_start and rrr_timer_stop (waits for the stop event). */
int rrr_timer_start(rrr_ctx *ctx);
int rrr_timer_stop(rrr_ctx *ctx, float *ms);

/* ---- one-call helper ---------------------------------------------------- */

/* Mirror of gpu_matmul_kquant (phi4.rs:631-658): upload a[K] into buf_a, run
 * the GEMV against weight_buf, download c[N] from buf_c. */
int rrr_matmul_kquant(rrr_ctx *ctx, rrr_buf *buf_a, const rrr_buf *weight_buf, rrr_buf *buf_c,
                      uint32_t type, const float *a, float *c, uint32_t K, uint32_t N);

#ifdef __cplusplus
}
#endif
#endif
