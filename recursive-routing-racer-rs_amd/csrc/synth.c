/*
 * synth.c -- seeded synthetic inputs for the five decode-path workloads.
 *
 * Counter-based splitmix64: word i of stream s under seed S is
 * splitmix64's (i+1)-th output starting from state S ^ mix(s), so any range of
 * words can be produced independently (threads split ranges; the result does
 * not depend on the thread count).  Normals come from Box-Muller in double,
 * rounded to f32; f16 values are f32 -> f16 round-to-nearest-even.
 *
 * Block recipes (one 256-element super-block uses 32 consecutive words):
 *   Q4_K  d = f16(|n0|*0.01), dmin = f16(|n1|*0.005), 12 scale bytes and
 *         128 qs bytes uniform.
 *   Q5_K  as Q4_K plus 32 uniform qh bytes.
 *   Q6_K  ql/qh uniform, int8 scales uniform in -32..31, d = f16(|n0|*0.005).
 * Words 0..26 supply the random bytes, words 30/31 the two normals.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define GOLDEN 0x9E3779B97F4A7C15ull

static inline uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline uint64_t stream_state(uint64_t seed, uint64_t stream) { return seed ^ mix64(stream * GOLDEN + 1); }

uint64_t rrr_synth_word(uint64_t seed, uint64_t stream, uint64_t i)
{
    return mix64(stream_state(seed, stream) + (i + 1) * GOLDEN);
}

static inline double u01(uint64_t w) { return (double)(w >> 11) * (1.0 / 9007199254740992.0); }

/* Box-Muller on words (2i, 2i+1) gives normals (2i, 2i+1) of a stream. */
static inline void normal_pair(uint64_t st, uint64_t pair, double *a, double *b)
{
    double u1 = u01(mix64(st + (2 * pair + 1) * GOLDEN));
    double u2 = u01(mix64(st + (2 * pair + 2) * GOLDEN));
    double r = sqrt(-2.0 * log(1.0 - u1));
    double t = 6.283185307179586476925286766559 * u2;
    *a = r * cos(t);
    *b = r * sin(t);
}

/* f32 -> f16 bits, round to nearest even, with subnormals, overflow to inf
 * and NaN preserved as a quiet NaN. */
uint16_t rrr_synth_f32_to_f16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFF) return (uint16_t)(sign | 0x7C00u | (man ? 0x200u | (man >> 13) : 0));
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        int shift = 14 - e;
        uint32_t half = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1);
        uint32_t mid = 1u << (shift - 1);
        if (rem > mid || (rem == mid && (half & 1))) half++;
        return (uint16_t)(sign | half);
    }
    uint32_t h = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) h++;
    return (uint16_t)(sign | h);
}

typedef struct {
    int kind; /* 0 f32 normals, 1 q4k, 2 q5k, 3 q6k, 4 bf16 normals */
    uint64_t st;
    float mean, std;
    void *out;
    uint64_t i0, i1;
} synth_job;

static void gen_block(int kind, uint64_t st, uint64_t bi, uint8_t *b)
{
    uint64_t w[32];
    for (int i = 0; i < 32; i++) w[i] = mix64(st + (bi * 32 + (uint64_t)i + 1) * GOLDEN);
    uint8_t bytes[216];
    memcpy(bytes, w, 216);
    double u1 = u01(w[30]), u2 = u01(w[31]);
    double r = sqrt(-2.0 * log(1.0 - u1));
    double t = 6.283185307179586476925286766559 * u2;
    float n0 = (float)(r * cos(t)), n1 = (float)(r * sin(t));
    if (kind == 1 || kind == 2) {
        uint16_t d = rrr_synth_f32_to_f16(fabsf(n0) * 0.01f);
        uint16_t dmin = rrr_synth_f32_to_f16(fabsf(n1) * 0.005f);
        b[0] = (uint8_t)d; b[1] = (uint8_t)(d >> 8);
        b[2] = (uint8_t)dmin; b[3] = (uint8_t)(dmin >> 8);
        if (kind == 1) memcpy(b + 4, bytes, 140);        /* sc[12] + qs[128] */
        else memcpy(b + 4, bytes, 172);                  /* sc[12] + qh[32] + qs[128] */
    } else {
        memcpy(b, bytes, 192);                           /* ql[128] + qh[64] */
        for (int s = 0; s < 16; s++) b[192 + s] = (uint8_t)(int8_t)((int)(bytes[192 + s] & 63) - 32);
        uint16_t d = rrr_synth_f32_to_f16(fabsf(n0) * 0.005f);
        b[208] = (uint8_t)d; b[209] = (uint8_t)(d >> 8);
    }
}

static void *synth_worker(void *p)
{
    synth_job *j = (synth_job *)p;
    if (j->kind == 0 || j->kind == 4) {
        for (uint64_t i = j->i0; i < j->i1; i += 2) {
            double a, b;
            normal_pair(j->st, i / 2, &a, &b);
            float fa = (float)a * j->std + j->mean, fb = (float)b * j->std + j->mean;
            if (j->kind == 0) {
                float *o = (float *)j->out;
                o[i] = fa;
                if (i + 1 < j->i1) o[i + 1] = fb;
            } else {
                uint16_t *o = (uint16_t *)j->out;
                uint32_t ua, ub;
                memcpy(&ua, &fa, 4);
                memcpy(&ub, &fb, 4);
                /* f32 -> bf16 round to nearest even (finite inputs only) */
                o[i] = (uint16_t)((ua + 0x7FFFu + ((ua >> 16) & 1)) >> 16);
                if (i + 1 < j->i1) o[i + 1] = (uint16_t)((ub + 0x7FFFu + ((ub >> 16) & 1)) >> 16);
            }
        }
    } else {
        static const int bs[4] = {0, 144, 176, 210};
        uint8_t *o = (uint8_t *)j->out;
        for (uint64_t bi = j->i0; bi < j->i1; bi++) gen_block(j->kind, j->st, bi, o + bi * bs[j->kind]);
    }
    return NULL;
}

static void run(int kind, uint64_t seed, uint64_t stream, float mean, float std, void *out,
                uint64_t count, int threads)
{
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    synth_job jobs[256];
    pthread_t tid[256];
    /* even split boundaries keep normal pairs inside one job */
    uint64_t per = (count + (uint64_t)threads - 1) / (uint64_t)threads;
    per = (per + 1) & ~1ull;
    int used = 0;
    for (int t = 0; t < threads; t++) {
        uint64_t i0 = (uint64_t)t * per, i1 = i0 + per;
        if (i0 >= count) break;
        if (i1 > count) i1 = count;
        synth_job jb = {kind, stream_state(seed, stream), mean, std, out, i0, i1};
        jobs[used++] = jb;
    }
    for (int t = 1; t < used; t++) pthread_create(&tid[t], NULL, synth_worker, &jobs[t]);
    if (used) synth_worker(&jobs[0]);
    for (int t = 1; t < used; t++) pthread_join(tid[t], NULL);
}

/* n f32 values ~ N(mean, std^2) */
void rrr_synth_normal_f32(uint64_t seed, uint64_t stream, float mean, float std, float *out,
                          uint64_t n, int threads)
{
    run(0, seed, stream, mean, std, out, n, threads);
}

/* n bf16 values ~ N(mean, std^2) */
void rrr_synth_normal_bf16(uint64_t seed, uint64_t stream, float mean, float std, uint16_t *out,
                           uint64_t n, int threads)
{
    run(4, seed, stream, mean, std, out, n, threads);
}

/* n_blocks K-quant super-blocks of GGUF type 12, 13 or 14; returns -1 for
 * any other type. */
int rrr_synth_kquant(uint64_t seed, uint64_t stream, uint32_t type, uint8_t *out, uint64_t n_blocks,
                     int threads)
{
    int kind = type == 12 ? 1 : type == 13 ? 2 : type == 14 ? 3 : 0;
    if (!kind) return -1;
    run(kind, seed, stream, 0.0f, 0.0f, out, n_blocks, threads);
    return 0;
}
