/*
 * rrr_oracle.h -- CPU oracle for the weight-heavy decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference's
 * CPU formulas (src/model/phi4.rs, src/model/gguf.rs) and is used exclusively
 * to check results against, by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py.  Nothing in the product library links or calls
 * it.
 *
 * Build: oracle/Makefile, with -O2 -ffp-contract=off and no -ffast-math, so
 * that every `a * b + c` below rounds twice exactly as the Rust code does.
 *
 * Parity pins (what checks each function independently of this restatement):
 *   rrr_o_f16_to_f32      exhaustive over all 65,536 patterns vs numpy's IEEE
 *                         binary16 widening (tests/test_oracle_pins.py)
 *   rrr_o_scale_min_k4    exhaustive bijection 96 bits <-> 16 six-bit fields
 *   rrr_o_dequant_q4_k    hand-built known-answer blocks + repack cross-check
 *   rrr_o_dequant_q5_k    hand-built known-answer blocks + repack cross-check
 *   rrr_o_dequant_q6_k    distinct-scale KAT pinning is = g*8 + l/16, single
 *                         qh-bit KATs + repack cross-check
 *   rrr_o_rms_norm        closed form in fp64 + gamma=1 and scale invariants
 *   rrr_o_silu_gate       closed form in fp64 (math.exp)
 *   rrr_o_gemv*           one-hot x gives the dequantized column bit-exactly,
 *                         all-ones x gives row sums; fp64 evaluation bound
 *   rrr_o_logits_*        chunk layout round trip (phi4.rs:877-893) and
 *                         row-major == chunked on the same data
 *   rrr_o_f32_to_f16      numpy's IEEE round-to-nearest-even binary16 cast on
 *                         every binary16 value, every tie between neighbours,
 *                         overflow / subnormal / NaN edges and 2^20 randoms
 *   rrr_o_rope            pos 0 = exact scaling by the attention factor,
 *                         dims past rope_dim untouched, pair norms scaled by
 *                         the factor, rotations compose (pos a then b = a + b),
 *                         and an fp64 complex-rotation evaluation
 *   rrr_o_attention_f64   closed forms: one position gives V, equal keys give
 *                         the mean of V, one dominant key gives its V; heads
 *                         of one KV group with equal queries agree
 */
#ifndef RRR_ORACLE_H
#define RRR_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF tensor type ids, gguf.rs:183-189 */
enum { RRR_O_F32 = 0, RRR_O_Q4_K = 12, RRR_O_Q5_K = 13, RRR_O_Q6_K = 14 };

/* Bytes per 256-element super-block (gguf.rs:187-189); 1024 for F32. */
uint32_t rrr_o_block_bytes(uint32_t type);

/* phi4.rs:442: half::f16::from_bits(bits).to_f32() (half 2.7.1). */
float rrr_o_f16_to_f32(uint16_t bits);

/* The 6-bit scale/min unpack inlined at phi4.rs:492-498 (and :522-528,
 * :293-301, :355-363).  j in 0..7, q points at the 12 scale bytes. */
void rrr_o_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *mn);

/* phi4.rs:481-510 */
void rrr_o_dequant_q4_k(const uint8_t *data, size_t n_elements, float *out);
/* phi4.rs:512-542 */
void rrr_o_dequant_q5_k(const uint8_t *data, size_t n_elements, float *out);
/* phi4.rs:444-479 */
void rrr_o_dequant_q6_k(const uint8_t *data, size_t n_elements, float *out);
/* phi4.rs:572-587 restricted to the path's types {0,12,13,14}; returns 0 on
 * success, -1 for any other type. */
int rrr_o_dequant(uint32_t type, const uint8_t *data, size_t n_elements, float *out);

/* The host repackers phi4.rs:278-436 (second statement of the bit layouts)
 * and a reader of each repacked layout, used only as a cross-check. */
void rrr_o_repack_q4k(const uint8_t *raw, size_t n_elements, uint8_t *out); /* 192 B/block */
void rrr_o_repack_q5k(const uint8_t *raw, size_t n_elements, uint8_t *out); /* 320 B/block */
void rrr_o_repack_q6k(const uint8_t *raw, size_t n_elements, uint8_t *out); /* 320 B/block */
void rrr_o_dequant_gpuq4(const uint8_t *rep, size_t n_elements, float *out);
void rrr_o_dequant_gpuq5(const uint8_t *rep, size_t n_elements, float *out);
void rrr_o_dequant_gpuq6(const uint8_t *rep, size_t n_elements, float *out);

/* phi4.rs:593-599; eps is RMS_EPS = 1e-5 (phi4.rs:111) at every call site. */
void rrr_o_rms_norm(const float *x, const float *w, float *out, size_t n, float eps);
/* rows independent RMSNorms of length d (the prefill loop, phi4.rs:1242-1255) */
void rrr_o_rms_norm_rows(const float *x, const float *w, float *out, size_t rows, size_t d, float eps);
/* phi4.rs:1369-1373: mid[i] = silu(gu[i]) * gu[F + i], rows of 2F. */
void rrr_o_silu_gate(const float *gate_up, float *mid, size_t rows, size_t F);
/* phi4.rs:608-610 */
void rrr_o_residual_add(const float *a, const float *b, float *out, size_t n);

/* Quantised GEMV / batched GEMV, Y[m,n] = sum_k X[m,k] * W[n,k]
 * (phi4.rs:628-630, batch shape :1257-1268).  The reference has no CPU GEMV;
 * this is the composed "rayon dequant+dot" path: per output row, dequantize
 * each 256-element block with the restated dequant_q*_k into a stack buffer,
 * then a sequential f32 dot.  Rows are split into contiguous chunks over
 * `threads` threads (par_chunks equivalent).  type 0 = F32 row-major W. */
int rrr_o_gemv(uint32_t type, const uint8_t *W, const float *X, float *Y,
               uint32_t K, uint32_t N, uint32_t M, int threads);
/* Same sums evaluated in double from the exact f32 dequantized weights. */
int rrr_o_gemv_f64(uint32_t type, const uint8_t *W, const float *X, double *Y,
                   uint32_t K, uint32_t N, uint32_t M, int threads);

/* F32 logits.  layout 0: E row-major [V][K] (token_embd order, phi4.rs:886
 * source side).  layout 1: the reference's transposed chunks
 * B_c[d*n + v] = E[(c*chunk + v)*K + d] (phi4.rs:874-893), chunks stored
 * back to back.  Sequential f32 sum over d in both layouts. */
int rrr_o_logits_f32(const float *x, const float *E, float *y, uint32_t K,
                     uint32_t V, uint32_t layout, uint32_t chunk, int threads);
int rrr_o_logits_f64(const float *x, const float *E, double *y, uint32_t K,
                     uint32_t V, uint32_t layout, uint32_t chunk, int threads);
/* Build the transposed chunk layout from row-major E (phi4.rs:877-893). */
void rrr_o_logits_chunk_build(const float *E, uint32_t K, uint32_t V,
                              uint32_t chunk, float *out);

/* bf16 -> f32 widening (exact) used for the prefill activations. */
float rrr_o_bf16_to_f32(uint16_t bits);

/* ---- decode glue (the rows after the weight sweep) ---- */

/* binary32 -> binary16, round to nearest even (the f16 KV caches, phi4.rs:898). */
uint16_t rrr_o_f32_to_f16(float f);
void rrr_o_f32_to_f16_n(const float *x, uint16_t *out, size_t n);

/* phi4.rs:238-256 (apply_rope_cfg) in f32, in place over n_heads heads. */
void rrr_o_rope(float *x, uint32_t pos, uint32_t n_heads, uint32_t head_dim, uint32_t rope_dim, float theta,
                float attn_factor, const float *factors, uint32_t n_factors);

/* The rope_kv_store / kv_store pipelines (phi4.rs:1016-1017, :1666-1677). */
void rrr_o_rope_kv_store(float *qkv, const float *factors, uint32_t n_factors, uint16_t *k_cache, uint16_t *v_cache,
                         uint32_t pos, uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim, uint32_t rope_dim,
                         uint32_t q_dim, uint32_t kv_stride, float theta, float attn_factor);

/* The attention pipeline (phi4.rs:1018, :1304-1312) in double. */
void rrr_o_attention_f64(const float *q, const uint16_t *k_cache, const uint16_t *v_cache, double *out,
                         uint32_t seq_len, uint32_t n_kv_heads, uint32_t heads_per_kv, uint32_t head_dim);

#ifdef __cplusplus
}
#endif
#endif
