/*
 * rrr_oracle.c -- CPU oracle (test infrastructure only; see rrr_oracle.h).
 *
 * Every function restates the reference's Rust CPU code with the same
 * evaluation order.  Rust never contracts a*b+c into an FMA, so this file is
 * compiled with -ffp-contract=off.  Citations are to the reference tree.
 */
#include "rrr_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

uint32_t rrr_o_block_bytes(uint32_t type)
{
    /* gguf.rs:187-189 (K-quants) and gguf.rs:179 (F32, 4 B per element). */
    switch (type) {
    case RRR_O_Q4_K: return 144;
    case RRR_O_Q5_K: return 176;
    case RRR_O_Q6_K: return 210;
    case RRR_O_F32:  return 1024;
    default:         return 0;
    }
}

static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* phi4.rs:442 calls half::f16::from_bits(bits).to_f32() (half 2.7.1,
 * Cargo.lock:178-187; the crate is not vendored).  Its published behaviour is
 * the exact IEEE 754 binary16 -> binary32 widening: zeros and normals map
 * exactly, subnormals are normalised, +-inf map to +-inf and NaNs keep their
 * payload with the quiet bit set. */
float rrr_o_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    if (exp == 0) {
        if (man == 0) return bits_f32(sign);
        int e = -1;
        do { e++; man <<= 1; } while (!(man & 0x400u));
        man &= 0x3FFu;
        return bits_f32(sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13));
    }
    if (exp == 31) {
        if (man == 0) return bits_f32(sign | 0x7F800000u);
        return bits_f32(sign | 0x7FC00000u | (man << 13));
    }
    return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

float rrr_o_bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

/* phi4.rs:492-498 (identical at :522-528, :293-301, :355-363). */
void rrr_o_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *mn)
{
    if (j < 4) {
        *sc = q[j] & 0x3F;
        *mn = q[j + 4] & 0x3F;
    } else {
        int i = j - 4;
        *sc = (uint8_t)((q[8 + i] & 0x0F) | ((q[i] >> 6) << 4));
        *mn = (uint8_t)((q[8 + i] >> 4) | ((q[4 + i] >> 6) << 4));
    }
}

static inline float le_f16(const uint8_t *b) { return rrr_o_f16_to_f32((uint16_t)(b[0] | (b[1] << 8))); }

/* phi4.rs:481-510: block {f16 d; f16 dmin; u8 sc[12]; u8 qs[128]}. */
static void dq_q4k_block(const uint8_t *b, float *out)
{
    float d = le_f16(b), dmin = le_f16(b + 2);
    const uint8_t *sc = b + 4, *qs = b + 16;
    for (int sub = 0; sub < 8; sub++) {
        uint8_t sv, mv;
        rrr_o_scale_min_k4(sub, sc, &sv, &mv);
        float s = d * (float)sv;
        float m = dmin * (float)mv;
        int pair = sub / 2;
        for (int j = 0; j < 32; j++) {
            uint8_t qb = qs[pair * 32 + j];
            uint8_t qi = (sub % 2 == 0) ? (qb & 0xF) : ((qb >> 4) & 0xF);
            out[sub * 32 + j] = (float)qi * s - m;
        }
    }
}

/* phi4.rs:512-542: block {d; dmin; sc[12]; qh[32]; qs[128]}. */
static void dq_q5k_block(const uint8_t *b, float *out)
{
    float d = le_f16(b), dmin = le_f16(b + 2);
    const uint8_t *sc = b + 4, *qh = b + 16, *qs = b + 48;
    for (int sub = 0; sub < 8; sub++) {
        uint8_t sv, mv;
        rrr_o_scale_min_k4(sub, sc, &sv, &mv);
        float s = d * (float)sv;
        float m = dmin * (float)mv;
        int pair = sub / 2;
        for (int j = 0; j < 32; j++) {
            uint8_t qb = qs[pair * 32 + j];
            uint32_t lo = (sub % 2 == 0) ? (qb & 0xF) : ((qb >> 4) & 0xF);
            uint32_t hb = (qh[j] >> sub) & 1;
            uint32_t qi = lo | (hb << 4);
            out[sub * 32 + j] = (float)qi * s - m;
        }
    }
}

/* phi4.rs:444-479: block {ql[128]; qh[64]; i8 sc[16]; f16 d}; scale index
 * is = g*8 + l/16 (phi4.rs:463), product order (d * sc) * q. */
static void dq_q6k_block(const uint8_t *b, float *out)
{
    const uint8_t *ql = b, *qh = b + 128, *scales = b + 192;
    float d = le_f16(b + 208);
    for (int g = 0; g < 2; g++) {
        for (int l = 0; l < 32; l++) {
            uint8_t ql_lo = ql[g * 64 + l];
            uint8_t ql_hi = ql[g * 64 + l + 32];
            uint8_t qhb = qh[g * 32 + l];
            int is = g * 8 + l / 16;
            int q1 = (int)((ql_lo & 0x0F) | (((qhb >> 0) & 3) << 4)) - 32;
            int q2 = (int)((ql_hi & 0x0F) | (((qhb >> 2) & 3) << 4)) - 32;
            int q3 = (int)((ql_lo >> 4) | (((qhb >> 4) & 3) << 4)) - 32;
            int q4 = (int)((ql_hi >> 4) | (((qhb >> 6) & 3) << 4)) - 32;
            float *o = out + g * 128;
            o[l]      = d * (float)(int8_t)scales[is]     * (float)q1;
            o[l + 32] = d * (float)(int8_t)scales[is + 2] * (float)q2;
            o[l + 64] = d * (float)(int8_t)scales[is + 4] * (float)q3;
            o[l + 96] = d * (float)(int8_t)scales[is + 6] * (float)q4;
        }
    }
}

void rrr_o_dequant_q4_k(const uint8_t *data, size_t n, float *out)
{
    for (size_t bi = 0; bi < n / 256; bi++) dq_q4k_block(data + bi * 144, out + bi * 256);
}
void rrr_o_dequant_q5_k(const uint8_t *data, size_t n, float *out)
{
    for (size_t bi = 0; bi < n / 256; bi++) dq_q5k_block(data + bi * 176, out + bi * 256);
}
void rrr_o_dequant_q6_k(const uint8_t *data, size_t n, float *out)
{
    for (size_t bi = 0; bi < n / 256; bi++) dq_q6k_block(data + bi * 210, out + bi * 256);
}

/* phi4.rs:572-587, restricted to the path's types. */
int rrr_o_dequant(uint32_t type, const uint8_t *data, size_t n, float *out)
{
    switch (type) {
    case RRR_O_F32: memcpy(out, data, n * 4); return 0;
    case RRR_O_Q4_K: rrr_o_dequant_q4_k(data, n, out); return 0;
    case RRR_O_Q5_K: rrr_o_dequant_q5_k(data, n, out); return 0;
    case RRR_O_Q6_K: rrr_o_dequant_q6_k(data, n, out); return 0;
    default: return -1;
    }
}

/* ---- repackers (phi4.rs:278-436), a second statement of the layouts ---- */

static void put_f32(uint8_t *p, float v) { memcpy(p, &v, 4); }
static float get_f32(const uint8_t *p) { float v; memcpy(&v, p, 4); return v; }

/* phi4.rs:278-328: f32[8] scales, f32[8] mins, u32[32] nibble words with
 * element e at word[e/8] bits (e%8)*4. */
void rrr_o_repack_q4k(const uint8_t *raw, size_t n, uint8_t *out)
{
    for (size_t bi = 0; bi < n / 256; bi++) {
        const uint8_t *b = raw + bi * 144;
        uint8_t *ob = out + bi * 192;
        memset(ob, 0, 192);
        float d = le_f16(b), dmin = le_f16(b + 2);
        for (int sub = 0; sub < 8; sub++) {
            uint8_t sv, mv;
            rrr_o_scale_min_k4(sub, b + 4, &sv, &mv);
            put_f32(ob + sub * 4, d * (float)sv);
            put_f32(ob + 32 + sub * 4, dmin * (float)mv);
        }
        for (int e = 0; e < 256; e++) {
            int sub = e / 32, j = e % 32, pair = sub / 2;
            uint8_t qb = b[16 + pair * 32 + j];
            uint32_t nib = (sub % 2 == 0) ? (qb & 0xF) : ((qb >> 4) & 0xF);
            uint32_t w;
            memcpy(&w, ob + 64 + (e / 8) * 4, 4);
            w |= nib << ((e % 8) * 4);
            memcpy(ob + 64 + (e / 8) * 4, &w, 4);
        }
    }
}

/* phi4.rs:339-384: f32[8], f32[8], u8[256] 5-bit values at byte 64 + e. */
void rrr_o_repack_q5k(const uint8_t *raw, size_t n, uint8_t *out)
{
    for (size_t bi = 0; bi < n / 256; bi++) {
        const uint8_t *b = raw + bi * 176;
        uint8_t *ob = out + bi * 320;
        float d = le_f16(b), dmin = le_f16(b + 2);
        for (int sub = 0; sub < 8; sub++) {
            uint8_t sv, mv;
            rrr_o_scale_min_k4(sub, b + 4, &sv, &mv);
            put_f32(ob + sub * 4, d * (float)sv);
            put_f32(ob + 32 + sub * 4, dmin * (float)mv);
        }
        for (int e = 0; e < 256; e++) {
            int sub = e / 32, j = e % 32, pair = sub / 2;
            uint8_t qb = b[48 + pair * 32 + j];
            uint8_t lo = (sub % 2 == 0) ? (qb & 0xF) : ((qb >> 4) & 0xF);
            uint8_t hb = (b[16 + j] >> sub) & 1;
            ob[64 + e] = (uint8_t)(lo | (hb << 4));
        }
    }
}

/* phi4.rs:396-436: f32[16] scales (d * i8 sc), u8[256] 6-bit unsigned values
 * at byte 64 + e, indexed by (g, quad, l) instead of (g, l, is). */
void rrr_o_repack_q6k(const uint8_t *raw, size_t n, uint8_t *out)
{
    for (size_t bi = 0; bi < n / 256; bi++) {
        const uint8_t *b = raw + bi * 210;
        uint8_t *ob = out + bi * 320;
        float d = le_f16(b + 208);
        for (int s = 0; s < 16; s++) put_f32(ob + s * 4, d * (float)(int8_t)b[192 + s]);
        for (int e = 0; e < 256; e++) {
            int g = e / 128, pos = e % 128, quad = pos / 32, l = pos % 32;
            int ql_idx = g * 64 + l + ((quad & 1) * 32);
            uint8_t qlb = b[ql_idx];
            uint8_t ql_val = (quad < 2) ? (qlb & 0x0F) : ((qlb >> 4) & 0x0F);
            uint8_t qh_val = (b[128 + g * 32 + l] >> (quad * 2)) & 0x03;
            ob[64 + e] = (uint8_t)(ql_val | (qh_val << 4));
        }
    }
}

/* Readers of the repacked layouts: what matmul_gpuq{4,5,6} consume. */
void rrr_o_dequant_gpuq4(const uint8_t *rep, size_t n, float *out)
{
    for (size_t bi = 0; bi < n / 256; bi++) {
        const uint8_t *ob = rep + bi * 192;
        for (int e = 0; e < 256; e++) {
            uint32_t w;
            memcpy(&w, ob + 64 + (e / 8) * 4, 4);
            uint32_t q = (w >> ((e % 8) * 4)) & 0xF;
            out[bi * 256 + e] = (float)q * get_f32(ob + (e / 32) * 4) - get_f32(ob + 32 + (e / 32) * 4);
        }
    }
}
void rrr_o_dequant_gpuq5(const uint8_t *rep, size_t n, float *out)
{
    for (size_t bi = 0; bi < n / 256; bi++) {
        const uint8_t *ob = rep + bi * 320;
        for (int e = 0; e < 256; e++)
            out[bi * 256 + e] = (float)ob[64 + e] * get_f32(ob + (e / 32) * 4) - get_f32(ob + 32 + (e / 32) * 4);
    }
}
void rrr_o_dequant_gpuq6(const uint8_t *rep, size_t n, float *out)
{
    for (size_t bi = 0; bi < n / 256; bi++) {
        const uint8_t *ob = rep + bi * 320;
        for (int e = 0; e < 256; e++)
            out[bi * 256 + e] = get_f32(ob + (e / 16) * 4) * (float)((int)ob[64 + e] - 32);
    }
}

/* ---- elementwise ops ---- */

/* phi4.rs:593-599 */
void rrr_o_rms_norm(const float *x, const float *w, float *out, size_t n, float eps)
{
    float sum_sq = 0.0f;
    for (size_t i = 0; i < n; i++) sum_sq += x[i] * x[i];
    float inv_rms = 1.0f / sqrtf(sum_sq / (float)n + eps);
    for (size_t i = 0; i < n; i++) out[i] = w[i] * x[i] * inv_rms;
}

void rrr_o_rms_norm_rows(const float *x, const float *w, float *out, size_t rows, size_t d, float eps)
{
    for (size_t r = 0; r < rows; r++) rrr_o_rms_norm(x + r * d, w, out + r * d, d, eps);
}

/* phi4.rs:1369-1373 (cpu_silu :601-606 has the same expression) */
void rrr_o_silu_gate(const float *gu, float *mid, size_t rows, size_t F)
{
    for (size_t r = 0; r < rows; r++) {
        const float *g = gu + r * 2 * F;
        for (size_t i = 0; i < F; i++) {
            float gate = g[i];
            float silu = gate / (1.0f + expf(-gate));
            mid[r * F + i] = silu * g[F + i];
        }
    }
}

/* phi4.rs:608-610 */
void rrr_o_residual_add(const float *a, const float *b, float *out, size_t n)
{
    for (size_t i = 0; i < n; i++) out[i] = a[i] + b[i];
}

/* ---- GEMV: the composed rayon dequant+dot path ---- */

typedef void (*dq_block_fn)(const uint8_t *, float *);

static void dq_f32_block(const uint8_t *b, float *out) { memcpy(out, b, 1024); }

static dq_block_fn block_fn(uint32_t type)
{
    switch (type) {
    case RRR_O_F32: return dq_f32_block;
    case RRR_O_Q4_K: return dq_q4k_block;
    case RRR_O_Q5_K: return dq_q5k_block;
    case RRR_O_Q6_K: return dq_q6k_block;
    default: return NULL;
    }
}

#define MAX_M 1024

typedef struct {
    uint32_t type, K, N, M;
    const uint8_t *W;
    const float *X;
    float *Y;
    double *Yd;
    uint32_t n0, n1;
} gemv_job;

static void *gemv_worker(void *p)
{
    gemv_job *j = (gemv_job *)p;
    dq_block_fn fn = block_fn(j->type);
    uint32_t bs = rrr_o_block_bytes(j->type), nb = j->K / 256;
    float tmp[256];
    float *acc = (float *)malloc(sizeof(float) * j->M);
    double *accd = (double *)malloc(sizeof(double) * j->M);
    for (uint32_t n = j->n0; n < j->n1; n++) {
        for (uint32_t m = 0; m < j->M; m++) { acc[m] = 0.0f; accd[m] = 0.0; }
        const uint8_t *row = j->W + (size_t)n * nb * bs;
        for (uint32_t b = 0; b < nb; b++) {
            fn(row + (size_t)b * bs, tmp);
            for (uint32_t m = 0; m < j->M; m++) {
                const float *x = j->X + (size_t)m * j->K + (size_t)b * 256;
                if (j->Y) {
                    float a = acc[m];
                    for (int i = 0; i < 256; i++) a += tmp[i] * x[i];
                    acc[m] = a;
                } else {
                    double a = accd[m];
                    for (int i = 0; i < 256; i++) a += (double)tmp[i] * (double)x[i];
                    accd[m] = a;
                }
            }
        }
        for (uint32_t m = 0; m < j->M; m++) {
            if (j->Y) j->Y[(size_t)m * j->N + n] = acc[m];
            else j->Yd[(size_t)m * j->N + n] = accd[m];
        }
    }
    free(acc);
    free(accd);
    return NULL;
}

static int run_rows(gemv_job base, int threads, void *(*fn)(void *), uint32_t N)
{
    if (threads < 1) threads = 1;
    if ((uint32_t)threads > N) threads = N ? (int)N : 1;
    gemv_job *jobs = (gemv_job *)malloc(sizeof(gemv_job) * threads);
    pthread_t *tid = (pthread_t *)malloc(sizeof(pthread_t) * threads);
    uint32_t per = (N + threads - 1) / threads;
    for (int t = 0; t < threads; t++) {
        jobs[t] = base;
        jobs[t].n0 = (uint32_t)t * per < N ? (uint32_t)t * per : N;
        jobs[t].n1 = jobs[t].n0 + per < N ? jobs[t].n0 + per : N;
    }
    for (int t = 1; t < threads; t++) pthread_create(&tid[t], NULL, fn, &jobs[t]);
    fn(&jobs[0]);
    for (int t = 1; t < threads; t++) pthread_join(tid[t], NULL);
    free(jobs);
    free(tid);
    return 0;
}

static int gemv_common(uint32_t type, const uint8_t *W, const float *X, float *Y, double *Yd,
                       uint32_t K, uint32_t N, uint32_t M, int threads)
{
    if (!block_fn(type) || K % 256 || M == 0 || M > MAX_M) return -1;
    gemv_job base = {type, K, N, M, W, X, Y, Yd, 0, 0};
    return run_rows(base, threads, gemv_worker, N);
}

int rrr_o_gemv(uint32_t type, const uint8_t *W, const float *X, float *Y,
               uint32_t K, uint32_t N, uint32_t M, int threads)
{
    return gemv_common(type, W, X, Y, NULL, K, N, M, threads);
}

int rrr_o_gemv_f64(uint32_t type, const uint8_t *W, const float *X, double *Y,
                   uint32_t K, uint32_t N, uint32_t M, int threads)
{
    return gemv_common(type, W, X, NULL, Y, K, N, M, threads);
}

/* ---- F32 logits (phi4.rs:866-893 layout, :1049-1064 dispatch) ---- */

void rrr_o_logits_chunk_build(const float *E, uint32_t K, uint32_t V, uint32_t chunk, float *out)
{
    size_t base = 0;
    for (uint32_t start = 0; start < V; start += chunk) {
        uint32_t end = start + chunk < V ? start + chunk : V;
        uint32_t n = end - start;
        for (uint32_t d = 0; d < K; d++)
            for (uint32_t v = 0; v < n; v++)
                out[base + (size_t)d * n + v] = E[(size_t)(start + v) * K + d];
        base += (size_t)n * K;
    }
}

typedef struct {
    const float *x, *E;
    float *y;
    double *yd;
    uint32_t K, V, layout, chunk;
    uint32_t n0, n1;
} logit_job;

static void *logit_worker(void *p)
{
    logit_job *j = (logit_job *)p;
    for (uint32_t v = j->n0; v < j->n1; v++) {
        const float *e;
        size_t stride;
        if (j->layout == 0) {
            e = j->E + (size_t)v * j->K;
            stride = 1;
        } else {
            uint32_t c = v / j->chunk, vin = v % j->chunk;
            uint32_t start = c * j->chunk;
            uint32_t n = start + j->chunk < j->V ? j->chunk : j->V - start;
            e = j->E + (size_t)start * j->K + vin;
            stride = n;
        }
        if (j->y) {
            float a = 0.0f;
            for (uint32_t d = 0; d < j->K; d++) a += j->x[d] * e[(size_t)d * stride];
            j->y[v] = a;
        } else {
            double a = 0.0;
            for (uint32_t d = 0; d < j->K; d++) a += (double)j->x[d] * (double)e[(size_t)d * stride];
            j->yd[v] = a;
        }
    }
    return NULL;
}

static int logits_common(const float *x, const float *E, float *y, double *yd, uint32_t K,
                         uint32_t V, uint32_t layout, uint32_t chunk, int threads)
{
    if (layout > 1 || (layout == 1 && chunk == 0)) return -1;
    if (threads < 1) threads = 1;
    if ((uint32_t)threads > V) threads = V ? (int)V : 1;
    logit_job *jobs = (logit_job *)malloc(sizeof(logit_job) * threads);
    pthread_t *tid = (pthread_t *)malloc(sizeof(pthread_t) * threads);
    uint32_t per = (V + threads - 1) / threads;
    for (int t = 0; t < threads; t++) {
        logit_job jb = {x, E, y, yd, K, V, layout, chunk, 0, 0};
        jb.n0 = (uint32_t)t * per < V ? (uint32_t)t * per : V;
        jb.n1 = jb.n0 + per < V ? jb.n0 + per : V;
        jobs[t] = jb;
    }
    for (int t = 1; t < threads; t++) pthread_create(&tid[t], NULL, logit_worker, &jobs[t]);
    logit_worker(&jobs[0]);
    for (int t = 1; t < threads; t++) pthread_join(tid[t], NULL);
    free(jobs);
    free(tid);
    return 0;
}

int rrr_o_logits_f32(const float *x, const float *E, float *y, uint32_t K, uint32_t V,
                     uint32_t layout, uint32_t chunk, int threads)
{
    return logits_common(x, E, y, NULL, K, V, layout, chunk, threads);
}

int rrr_o_logits_f64(const float *x, const float *E, double *y, uint32_t K, uint32_t V,
                     uint32_t layout, uint32_t chunk, int threads)
{
    return logits_common(x, E, NULL, y, K, V, layout, chunk, threads);
}

/* ---- decode glue: RoPE, the f16 KV-cache store, decode attention ---- */

/* IEEE binary32 -> binary16, round to nearest, ties to even; overflow gives
 * +-inf, NaNs stay NaN (quiet).  The reference keeps K and V in f16 caches
 * (kv_size = MAX_SEQ * kv_stride * 2 bytes, phi4.rs:898) written by its
 * kv_store / rope_kv_store shaders (dispatched at :1016-1017 and :1676; the
 * SPIR-V is not in the tree), whose conversion is the default round-to-
 * nearest-even of a float -> half conversion. */
uint16_t rrr_o_f32_to_f16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, e = (x >> 23) & 0xFFu;
    uint32_t m = x & 0x7FFFFFu;
    if (e == 0xFFu) return (uint16_t)(sign | 0x7C00u | (m ? 0x200u | (m >> 13) : 0u));
    const int32_t E = (int32_t)e - 127 + 15;
    if (E >= 31) return (uint16_t)(sign | 0x7C00u);
    if (E <= 0) {
        if (E < -10) return (uint16_t)sign;
        m |= 0x800000u;                            /* 24-bit significand */
        const uint32_t shift = (uint32_t)(14 - E); /* value / 2^-24 = m >> shift */
        const uint32_t half = 1u << (shift - 1), rest = m & ((1u << shift) - 1u);
        uint32_t r = m >> shift;
        if (rest > half || (rest == half && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((uint32_t)E << 10) | (m >> 13);
    const uint32_t rest = m & 0x1FFFu;
    if (rest > 0x1000u || (rest == 0x1000u && (r & 1u))) r++;  /* a carry may reach the exponent / inf */
    return (uint16_t)(sign | r);
}

void rrr_o_f32_to_f16_n(const float *x, uint16_t *out, size_t n)
{
    for (size_t i = 0; i < n; i++) out[i] = rrr_o_f32_to_f16(x[i]);
}

/* phi4.rs:238-256 (apply_rope_cfg), step for step in f32: pairs (2i, 2i+1)
 * of the first rope_dim dims of each head, base_freq = 1 / theta^(2i /
 * rope_dim) (powf), divided by the LongRoPE factor (1 past the factor list),
 * angle = pos * freq, sin/cos scaled by the attention factor.  Rust's f32
 * powf / sin_cos call the platform libm powf / sinf / cosf, as this does. */
void rrr_o_rope(float *x, uint32_t pos, uint32_t n_heads, uint32_t head_dim, uint32_t rope_dim, float theta,
                float attn_factor, const float *factors, uint32_t n_factors)
{
    for (uint32_t h = 0; h < n_heads; h++) {
        const size_t base = (size_t)h * head_dim;
        for (uint32_t i = 0; i < rope_dim / 2; i++) {
            const float base_freq = 1.0f / powf(theta, 2.0f * (float)i / (float)rope_dim);
            const float factor = i < n_factors ? factors[i] : 1.0f;
            const float freq = base_freq / factor;
            const float angle = (float)pos * freq;
            const float sin_t = sinf(angle), cos_t = cosf(angle);
            const float cos_scaled = cos_t * attn_factor;
            const float sin_scaled = sin_t * attn_factor;
            const float x0 = x[base + 2 * i], x1 = x[base + 2 * i + 1];
            x[base + 2 * i] = x0 * cos_scaled - x1 * sin_scaled;
            x[base + 2 * i + 1] = x0 * sin_scaled + x1 * cos_scaled;
        }
    }
}

/* The rope_kv_store pipeline (phi4.rs:1016-1017; push [pos, n_heads,
 * n_kv_heads, head_dim, rope_dim, q_dim, kv_stride], :1115-1117): RoPE on the
 * Q heads (qkv[0, q_dim)) and the K heads (qkv[q_dim, q_dim + kv_stride)) in
 * place, as the CPU path does before its store (:1656-1657), then K and V as
 * f16 into row pos of the caches (row stride kv_stride).  rope_dim = 0 skips
 * the rotation: the kv_store pipeline (:1666-1677). */
void rrr_o_rope_kv_store(float *qkv, const float *factors, uint32_t n_factors, uint16_t *k_cache, uint16_t *v_cache,
                         uint32_t pos, uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim, uint32_t rope_dim,
                         uint32_t q_dim, uint32_t kv_stride, float theta, float attn_factor)
{
    if (rope_dim) {
        rrr_o_rope(qkv, pos, n_heads, head_dim, rope_dim, theta, attn_factor, factors, n_factors);
        rrr_o_rope(qkv + q_dim, pos, n_kv_heads, head_dim, rope_dim, theta, attn_factor, factors, n_factors);
    }
    for (uint32_t i = 0; i < kv_stride; i++) {
        k_cache[(size_t)pos * kv_stride + i] = rrr_o_f32_to_f16(qkv[q_dim + i]);
        v_cache[(size_t)pos * kv_stride + i] = rrr_o_f32_to_f16(qkv[q_dim + kv_stride + i]);
    }
}

/* Decode attention of the attention pipeline (phi4.rs:1018, :1304-1312;
 * push [seq_len, n_kv_heads, heads_per_kv, head_dim], one workgroup per
 * query head; the shader is not in the tree).  The textbook definition, in
 * double: query head h reads kv head g = h / heads_per_kv;
 * s_t = (q_h . k_t) / sqrt(head_dim) over the f16 cache rows t < seq_len,
 * p = softmax(s), out_h = sum_t p_t v_t. */
void rrr_o_attention_f64(const float *q, const uint16_t *k_cache, const uint16_t *v_cache, double *out,
                         uint32_t seq_len, uint32_t n_kv_heads, uint32_t heads_per_kv, uint32_t head_dim)
{
    const size_t kv_stride = (size_t)n_kv_heads * head_dim;
    const double scale = 1.0 / sqrt((double)head_dim);
    double *s = (double *)malloc(sizeof(double) * (seq_len ? seq_len : 1));
    for (uint32_t h = 0; h < n_kv_heads * heads_per_kv; h++) {
        const size_t g = h / heads_per_kv;
        double mx = -INFINITY;
        for (uint32_t t = 0; t < seq_len; t++) {
            double acc = 0.0;
            for (uint32_t d = 0; d < head_dim; d++)
                acc += (double)q[(size_t)h * head_dim + d] *
                       (double)rrr_o_f16_to_f32(k_cache[t * kv_stride + g * head_dim + d]);
            s[t] = acc * scale;
            if (s[t] > mx) mx = s[t];
        }
        double den = 0.0;
        for (uint32_t t = 0; t < seq_len; t++) {
            s[t] = exp(s[t] - mx);
            den += s[t];
        }
        for (uint32_t d = 0; d < head_dim; d++) {
            double acc = 0.0;
            for (uint32_t t = 0; t < seq_len; t++)
                acc += s[t] * (double)rrr_o_f16_to_f32(v_cache[t * kv_stride + g * head_dim + d]);
            out[(size_t)h * head_dim + d] = acc / den;
        }
    }
    free(s);
}
