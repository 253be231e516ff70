/*
 * oracle.c -- CPU restatement of the reference's MXFP4 decode path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  Built with -ffp-contract=off and
 * no fast-math so every f32 expression rounds exactly as the reference's Rust
 * CPU loops do.  Citations are file:line under botBehavior/rust-fp4-blackwell.
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ======================================================================
 * threads: deterministic row partitioning
 * ====================================================================== */
static int g_threads = 1;

void orc_set_threads(int n)
{
    if (n <= 0) {
        long c = sysconf(_SC_NPROCESSORS_ONLN);
        n = c > 0 ? (int)c : 1;
    }
    if (n > 256) n = 256;
    g_threads = n;
}

int orc_get_threads(void) { return g_threads; }

typedef void (*row_fn)(void *ctx, size_t r0, size_t r1);
typedef struct {
    row_fn fn;
    void *ctx;
    size_t r0, r1;
} par_job;

static void *par_trampoline(void *p)
{
    par_job *j = (par_job *)p;
    j->fn(j->ctx, j->r0, j->r1);
    return NULL;
}

/* Run fn over [0, rows) split into contiguous chunks, one per thread. */
static void parallel_rows(size_t rows, row_fn fn, void *ctx)
{
    int nt = g_threads;
    if ((size_t)nt > rows) nt = (int)(rows ? rows : 1);
    if (nt <= 1) {
        fn(ctx, 0, rows);
        return;
    }
    pthread_t th[256];
    par_job jobs[256];
    size_t per = rows / (size_t)nt, rem = rows % (size_t)nt, at = 0;
    for (int t = 0; t < nt; t++) {
        size_t cnt = per + ((size_t)t < rem ? 1 : 0);
        jobs[t].fn = fn;
        jobs[t].ctx = ctx;
        jobs[t].r0 = at;
        jobs[t].r1 = at + cnt;
        at += cnt;
    }
    for (int t = 1; t < nt; t++) pthread_create(&th[t], NULL, par_trampoline, &jobs[t]);
    par_trampoline(&jobs[0]);
    for (int t = 1; t < nt; t++) pthread_join(th[t], NULL);
}

/* ======================================================================
 * RNG
 * ====================================================================== */
/* fp4_gemv/src/main.rs:101-107: s ^= s<<13; s ^= s>>17; s ^= s<<5 */
uint32_t orc_xorshift32_next(uint32_t *state)
{
    uint32_t s = *state;
    s ^= s << 13;
    s ^= s >> 17;
    s ^= s << 5;
    *state = s;
    return s;
}

void orc_xorshift32_fill(uint32_t *state, uint32_t *out, size_t n)
{
    for (size_t i = 0; i < n; i++) out[i] = orc_xorshift32_next(state);
}

/* SplitMix64 finalizer (Steele, Lea & Flood 2014) over a counter that mixes
 * seed, stream and index.  Pure u64 arithmetic: identical on every device. */
uint64_t orc_mix64(uint64_t seed, uint64_t stream, uint64_t index)
{
    uint64_t z = seed + 0x9E3779B97F4A7C15ull * (index + 1ull) + 0xD1342543DE82EF95ull * stream;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

#define IH4_STD 37837.22723720648 /* sqrt((65536^2 - 1) / 3) */

float orc_ih4_coef(float sigma) { return (float)((double)sigma / IH4_STD); }

float orc_ih4_normal(uint64_t r, float coef)
{
    int32_t s = (int32_t)(r & 0xFFFF) + (int32_t)((r >> 16) & 0xFFFF) +
                (int32_t)((r >> 32) & 0xFFFF) + (int32_t)((r >> 48) & 0xFFFF) - 2 * 65535;
    return (float)s * coef;
}

/* ======================================================================
 * codecs
 * ====================================================================== */
static const float E2M1_MAG[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
/* The same values with the sign applied ("if c & 8 { -m } else { m }"), as one
 * table so the GEMV loop has no data-dependent branch. */
static const float E2M1_VAL[16] = {0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,  4.0f,  6.0f,
                                   -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

/* fp4_gemv/src/main.rs:130-134 */
float orc_e2m1_decode(uint8_t code) { return E2M1_VAL[code & 15]; }

/* llama_run/src/main.rs:21-32 (fp4_val) */
float orc_e2m1_decode_arith(uint32_t code)
{
    uint32_t e = (code >> 1) & 3;
    float m = (float)(code & 1);
    float mag;
    if (e == 0) {
        mag = 0.5f * m;
    } else {
        float base = (float)(1u << (e - 1));
        mag = base + base * 0.5f * m;
    }
    return (code & 8) ? -mag : mag;
}

/* trackb/FP4_M16N8K64_LAYOUT.md:20: value = 2^(b-127); OCP MX: 0xFF = NaN */
float orc_e8m0_decode(uint8_t b)
{
    if (b == 0xFF) return NAN;
    return ldexpf(1.0f, (int)b - 127);
}

/* trackb/fp4_scale_test.cu:12 */
uint8_t orc_e8m0_encode_pow2(float s)
{
    int e = (int)lroundf(log2f(s));
    return (uint8_t)(127 + e);
}

/* Round-to-nearest-even onto {0,.5,1,1.5,2,3,4,6}, saturating at 6.
 * Ties go to the code with an even mantissa bit (bit 0 of the code). */
uint8_t orc_e2m1_rne(float v)
{
    float a = fabsf(v);
    /* Count the decision thresholds a lies above; '>' at a tie rounds down to
     * the even neighbour, '>=' rounds up to it:
     *   0.25 tie -> 0, 0.75 -> 1.0, 1.25 -> 1.0, 1.75 -> 2, 2.5 -> 2,
     *   3.5 -> 4, 5 -> 4; above 5 -> 6 (saturating); NaN -> code 7. */
    uint8_t c = (uint8_t)((a > 0.25f) + (a >= 0.75f) + (a > 1.25f) + (a >= 1.75f) + (a > 2.5f) + (a >= 3.5f) +
                          (a > 5.0f));
    if (isnan(a)) c = 7;
    if (signbit(v)) c |= 8;
    return c;
}

/* llama_run/src/main.rs:591-614 */
float orc_f16_to_f32(uint16_t h)
{
    uint32_t sign = (h >> 15) & 1u, exp = (h >> 10) & 0x1Fu, mant = h & 0x3FFu, f;
    if (exp == 0) {
        if (mant == 0) {
            f = sign << 31;
        } else {
            int e = -14;
            uint32_t m = mant;
            while ((m & 0x400u) == 0) {
                m <<= 1;
                e -= 1;
            }
            m &= 0x3FFu;
            f = (sign << 31) | ((uint32_t)(e + 127) << 23) | (m << 13);
        }
    } else if (exp == 0x1F) {
        f = (sign << 31) | (0xFFu << 23) | (mant << 13);
    } else {
        f = (sign << 31) | ((exp - 15 + 127) << 23) | (mant << 13);
    }
    float out;
    memcpy(&out, &f, 4);
    return out;
}

/* IEEE binary32 -> binary16, round to nearest even, overflow to inf. */
uint16_t orc_f32_to_f16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) { /* inf / nan */
        return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u | ((ax >> 13) & 0x3FFu) : 0));
    }
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to >= 65520 -> inf */
    if (ax < 0x38800000u) {                                    /* result subnormal or zero */
        if (ax < 0x33000000u) return (uint16_t)sign;            /* < 2^-25: rounds to 0 */
        uint32_t e = ax >> 23;                                  /* 102..112 */
        uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e;                              /* 14..24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((ax - 0x38000000u) >> 13); /* rebias 127->15 */
    uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

/* llama_run/src/main.rs:425: bf16 -> f32 is a 16-bit shift */
float orc_bf16_to_f32(uint16_t h)
{
    uint32_t f = (uint32_t)h << 16;
    float out;
    memcpy(&out, &f, 4);
    return out;
}

uint16_t orc_f32_to_bf16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
    uint32_t lsb = (x >> 16) & 1u;
    x += 0x7FFFu + lsb;
    return (uint16_t)(x >> 16);
}

/* fp4_gemv/src/main.rs:113-120: low nibble first */
void orc_pack_codes(const uint8_t *codes, size_t n, uint8_t *packed)
{
    for (size_t i = 0; i < n / 2; i++)
        packed[i] = (uint8_t)((codes[2 * i] & 0xF) | ((codes[2 * i + 1] & 0xF) << 4));
}

void orc_unpack_codes(const uint8_t *packed, size_t n, uint8_t *codes)
{
    for (size_t i = 0; i < n / 2; i++) {
        codes[2 * i] = packed[i] & 0xF;
        codes[2 * i + 1] = packed[i] >> 4;
    }
}

/* ======================================================================
 * quantizers
 * ====================================================================== */
/* llama_run/src/main.rs:334-376 */
void orc_quant_fp4_absmax(const float *w, int outd, int ind, uint8_t *packed, float *scales)
{
    int nb = ind / 32;
    uint8_t *codes = (uint8_t *)malloc((size_t)outd * (size_t)ind);
    for (int r = 0; r < outd; r++) {
        for (int b = 0; b < nb; b++) {
            size_t base = (size_t)r * (size_t)ind + (size_t)b * 32;
            float amax = 0.0f;
            for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(w[base + i]));
            float scale = amax > 0.0f ? amax / 6.0f : 1.0f;
            scales[(size_t)r * nb + b] = scale;
            for (int i = 0; i < 32; i++) {
                float v = w[base + i] / scale;
                float a = fabsf(v);
                int bc = 0;
                float bd = 3.40282347e38f; /* f32::MAX */
                for (int ci = 0; ci < 8; ci++) {
                    float d = fabsf(a - E2M1_MAG[ci]);
                    if (d < bd) {
                        bd = d;
                        bc = ci;
                    }
                }
                uint8_t code = (uint8_t)bc;
                if (v < 0.0f) code |= 8;
                codes[base + i] = code;
            }
        }
    }
    orc_pack_codes(codes, (size_t)outd * (size_t)ind, packed);
    free(codes);
}

/* floor(log2(a)) for finite a > 0, from the exponent bits (exact). */
static int floor_log2f(float a)
{
    int e;
    frexpf(a, &e); /* a = m * 2^e, m in [0.5, 1) */
    return e - 1;
}

/* One 32-element OCP MX block: scale byte and 32 codes. */
static uint8_t quant_mx_block(const float *v, uint8_t *codes)
{
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    if (amax == 0.0f) {
        for (int i = 0; i < 32; i++) codes[i] = orc_e2m1_rne(v[i]);
        return 0;
    }
    int se = floor_log2f(amax) - 2; /* E2M1 emax = 2 */
    if (se < -127) se = -127;
    if (se > 127) se = 127;
    /* v * 2^-se == ldexpf(v, -se): the factor is a normal float for every
     * se in [-127, 125], so the product rounds exactly like ldexpf. */
    uint32_t fb = (uint32_t)(127 - se) << 23;
    float f;
    memcpy(&f, &fb, 4);
    for (int i = 0; i < 32; i++) codes[i] = orc_e2m1_rne(v[i] * f);
    return (uint8_t)(se + 127);
}

void orc_quant_mx(const float *w, size_t rows, size_t ind, uint8_t *packed, uint8_t *scales)
{
    size_t nb = ind / 32;
    uint8_t codes[32];
    for (size_t r = 0; r < rows; r++) {
        for (size_t b = 0; b < nb; b++) {
            const float *v = w + r * ind + b * 32;
            scales[r * nb + b] = quant_mx_block(v, codes);
            orc_pack_codes(codes, 32, packed + (r * ind + b * 32) / 2);
        }
    }
}

typedef struct {
    uint64_t seed, stream;
    float coef;
    size_t K, r0;
    uint8_t *packed, *scales;
} synth_w_ctx;

static void synth_w_rows(void *p, size_t a, size_t b)
{
    synth_w_ctx *c = (synth_w_ctx *)p;
    size_t nb = c->K / 32;
    float v[32];
    uint8_t codes[32];
    for (size_t rr = a; rr < b; rr++) {
        size_t r = c->r0 + rr;
        for (size_t blk = 0; blk < nb; blk++) {
            for (int i = 0; i < 32; i++)
                v[i] = orc_ih4_normal(orc_mix64(c->seed, c->stream, r * c->K + blk * 32 + (size_t)i),
                                      c->coef);
            c->scales[rr * nb + blk] = quant_mx_block(v, codes);
            orc_pack_codes(codes, 32, c->packed + (rr * c->K + blk * 32) / 2);
        }
    }
}

void orc_synth_mx_weight(uint64_t seed, uint64_t stream, float sigma, size_t K, size_t r0,
                         size_t nrows, uint8_t *packed, uint8_t *scales)
{
    synth_w_ctx c = {seed, stream, orc_ih4_coef(sigma), K, r0, packed, scales};
    parallel_rows(nrows, synth_w_rows, &c);
}

void orc_synth_f16(uint64_t seed, uint64_t stream, float sigma, float offset, size_t n,
                   uint16_t *out)
{
    float coef = orc_ih4_coef(sigma);
    for (size_t i = 0; i < n; i++)
        out[i] = orc_f32_to_f16(offset + orc_ih4_normal(orc_mix64(seed, stream, i), coef));
}

/* ======================================================================
 * GEMV
 * ====================================================================== */
typedef struct {
    uint32_t k;
    const uint32_t *w;
    const uint8_t *codes;
    const float *fscales;
    const uint8_t *escales;
    const float *x;
    float *y;
    double *y64, *absy;
} gemv_ctx;

/* fp4_gemv/src/main.rs:136-142: acc += fp4(code) * scale * x[k] */
static void gemv_f32scale_rows(void *p, size_t a, size_t b)
{
    gemv_ctx *c = (gemv_ctx *)p;
    uint32_t K = c->k, nb = K / 32;
    for (size_t n = a; n < b; n++) {
        float acc = 0.0f;
        for (uint32_t kk = 0; kk < K; kk++) {
            uint32_t word = c->w[(n * K + kk) / 8];
            uint8_t code = (uint8_t)((word >> (4 * (kk % 8))) & 0xF);
            acc += orc_e2m1_decode(code) * c->fscales[n * nb + kk / 32] * c->x[kk];
        }
        c->y[n] = acc;
    }
}

void orc_gemv_f32scale(uint32_t n, uint32_t k, const uint32_t *w, const float *scales,
                       const float *x, float *y)
{
    gemv_ctx c = {k, w, NULL, scales, NULL, x, y, NULL, NULL};
    parallel_rows(n, gemv_f32scale_rows, &c);
}

static void gemv_e8m0_rows(void *p, size_t a, size_t b)
{
    gemv_ctx *c = (gemv_ctx *)p;
    uint32_t K = c->k, nb = K / 32;
    for (size_t n = a; n < b; n++) {
        const uint8_t *row = c->codes + n * (K / 2);
        float acc = 0.0f;
        for (uint32_t blk = 0; blk < nb; blk++) {
            float sc = orc_e8m0_decode(c->escales[n * nb + blk]);
            for (uint32_t i = 0; i < 32; i++) {
                uint32_t kk = blk * 32 + i;
                uint8_t code = (uint8_t)((row[kk / 2] >> (4 * (kk & 1))) & 0xF);
                acc += orc_e2m1_decode(code) * sc * c->x[kk];
            }
        }
        c->y[n] = acc;
    }
}

void orc_gemv_e8m0(uint32_t n, uint32_t k, const uint8_t *codes, const uint8_t *scales,
                   const float *x, float *y)
{
    gemv_ctx c = {k, NULL, codes, NULL, scales, x, y, NULL, NULL};
    parallel_rows(n, gemv_e8m0_rows, &c);
}

static void gemv_e8m0_f64_rows(void *p, size_t a, size_t b)
{
    gemv_ctx *c = (gemv_ctx *)p;
    uint32_t K = c->k, nb = K / 32;
    for (size_t n = a; n < b; n++) {
        const uint8_t *row = c->codes + n * (K / 2);
        double acc = 0.0, aacc = 0.0;
        for (uint32_t kk = 0; kk < K; kk++) {
            uint8_t code = (uint8_t)((row[kk / 2] >> (4 * (kk & 1))) & 0xF);
            double t = (double)orc_e2m1_decode(code) * (double)orc_e8m0_decode(c->escales[n * nb + kk / 32]) *
                       (double)c->x[kk];
            acc += t;
            aacc += fabs(t);
        }
        c->y64[n] = acc;
        if (c->absy) c->absy[n] = aacc;
    }
}

void orc_gemv_e8m0_f64(uint32_t n, uint32_t k, const uint8_t *codes, const uint8_t *scales,
                       const float *x, double *y, double *absy)
{
    gemv_ctx c = {k, NULL, codes, NULL, scales, x, NULL, y, absy};
    parallel_rows(n, gemv_e8m0_f64_rows, &c);
}

/* ======================================================================
 * MMA tile / GEMM
 * ====================================================================== */
/* trackb/fp4_scale_test.cu:37 */
void orc_mma_m16n8k64_ref(const float *A, const float *B, const float *SFA, const float *SFB,
                          float *D)
{
    for (int i = 0; i < 16; i++)
        for (int j = 0; j < 8; j++) {
            float s = 0.0f;
            for (int k = 0; k < 64; k++)
                s += A[i * 64 + k] * SFA[i * 2 + k / 32] * B[k * 8 + j] * SFB[(k / 32) * 8 + j];
            D[i * 8 + j] = s;
        }
}

typedef struct {
    uint32_t N, K;
    const uint8_t *ac, *as, *wc, *ws;
    double *c, *absc;
} gemm_ctx;

static void gemm_rows(void *p, size_t a, size_t b)
{
    gemm_ctx *g = (gemm_ctx *)p;
    uint32_t K = g->K, nb = K / 32;
    double *arow = (double *)malloc(sizeof(double) * K);
    for (size_t m = a; m < b; m++) {
        for (uint32_t kk = 0; kk < K; kk++) {
            uint8_t code = (uint8_t)((g->ac[(m * K + kk) / 2] >> (4 * (kk & 1))) & 0xF);
            arow[kk] = (double)orc_e2m1_decode(code) * (double)orc_e8m0_decode(g->as[m * nb + kk / 32]);
        }
        for (uint32_t n = 0; n < g->N; n++) {
            double acc = 0.0, aacc = 0.0;
            const uint8_t *wrow = g->wc + (size_t)n * (K / 2);
            for (uint32_t blk = 0; blk < nb; blk++) {
                double ws = (double)orc_e8m0_decode(g->ws[(size_t)n * nb + blk]);
                for (uint32_t i = 0; i < 32; i++) {
                    uint32_t kk = blk * 32 + i;
                    uint8_t code = (uint8_t)((wrow[kk / 2] >> (4 * (kk & 1))) & 0xF);
                    double t = arow[kk] * (double)orc_e2m1_decode(code) * ws;
                    acc += t;
                    aacc += fabs(t);
                }
            }
            g->c[m * g->N + n] = acc;
            if (g->absc) g->absc[m * g->N + n] = aacc;
        }
    }
    free(arow);
}

void orc_gemm_mx_f64(uint32_t M, uint32_t N, uint32_t K, const uint8_t *a_codes,
                     const uint8_t *a_scales, const uint8_t *w_codes, const uint8_t *w_scales,
                     double *c, double *absc)
{
    gemm_ctx g = {N, K, a_codes, a_scales, w_codes, w_scales, c, absc};
    parallel_rows(M, gemm_rows, &g);
}

/* ======================================================================
 * layers
 * ====================================================================== */
/* llama_rmsnorm/src/main.rs:75-77 */
void orc_rmsnorm(uint32_t dim, float eps, const float *x, const float *w, float *y)
{
    float ss = 0.0f;
    for (uint32_t i = 0; i < dim; i++) ss += x[i] * x[i];
    float rms = 1.0f / sqrtf(ss / (float)dim + eps);
    for (uint32_t i = 0; i < dim; i++) y[i] = x[i] * rms * w[i];
}

/* llama_run/src/main.rs:462-471 */
void orc_rope_table(uint32_t max_pos, uint32_t head_dim, double theta, float *cosv, float *sinv)
{
    uint32_t half = head_dim / 2;
    for (uint32_t pos = 0; pos < max_pos; pos++)
        for (uint32_t j = 0; j < half; j++) {
            double freq = 1.0 / pow(theta, 2.0 * (double)j / (double)head_dim);
            double a = (double)pos * freq;
            cosv[(size_t)pos * half + j] = (float)cos(a);
            sinv[(size_t)pos * half + j] = (float)sin(a);
        }
}

/* llama_rope/src/main.rs:75-84 */
void orc_rope(uint32_t num_heads, uint32_t head_dim, const float *cosp, const float *sinp, float *q)
{
    uint32_t half = head_dim / 2;
    for (uint32_t h = 0; h < num_heads; h++) {
        float *b = q + (size_t)h * head_dim;
        for (uint32_t j = 0; j < half; j++) {
            float x0 = b[j], x1 = b[j + half];
            b[j] = x0 * cosp[j] - x1 * sinp[j];
            b[j + half] = x1 * cosp[j] + x0 * sinp[j];
        }
    }
}

/* llama_attn_decode/src/main.rs:150-179, with K/V read through `ld`. */
typedef float (*kv_load)(const void *base, size_t idx);
static float ld_f32(const void *b, size_t i) { return ((const float *)b)[i]; }
static float ld_f16(const void *b, size_t i) { return orc_f16_to_f32(((const uint16_t *)b)[i]); }

typedef struct {
    uint32_t nh, nkv, hd, seq;
    const float *q;
    const void *kc, *vc;
    size_t ts, hs;
    kv_load ld;
    float *out;
} attn_ctx;

static void attn_heads(void *p, size_t a, size_t b)
{
    attn_ctx *c = (attn_ctx *)p;
    uint32_t group = c->nh / c->nkv;
    float scale = 1.0f / sqrtf((float)c->hd);
    float *sc = (float *)malloc(sizeof(float) * (c->seq ? c->seq : 1));
    for (size_t h = a; h < b; h++) {
        size_t kvh = h / group;
        float m = -3.40282347e38f; /* f32::MIN */
        for (uint32_t t = 0; t < c->seq; t++) {
            float d = 0.0f;
            size_t base = t * c->ts + kvh * c->hs;
            for (uint32_t i = 0; i < c->hd; i++) d += c->q[h * c->hd + i] * c->ld(c->kc, base + i);
            sc[t] = d * scale;
            if (sc[t] > m) m = sc[t];
        }
        float l = 0.0f;
        for (uint32_t t = 0; t < c->seq; t++) {
            sc[t] = expf(sc[t] - m);
            l += sc[t];
        }
        for (uint32_t i = 0; i < c->hd; i++) {
            float acc = 0.0f;
            for (uint32_t t = 0; t < c->seq; t++) acc += sc[t] * c->ld(c->vc, t * c->ts + kvh * c->hs + i);
            c->out[h * c->hd + i] = acc / l;
        }
    }
    free(sc);
}

void orc_attn_decode(uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim, uint32_t seq,
                     const float *q, const float *kc, const float *vc, size_t ts, size_t hs,
                     float *out)
{
    attn_ctx c = {n_heads, n_kv_heads, head_dim, seq, q, kc, vc, ts, hs, ld_f32, out};
    parallel_rows(n_heads, attn_heads, &c);
}

void orc_attn_decode_f16(uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim, uint32_t seq,
                         const float *q, const uint16_t *kc, const uint16_t *vc, size_t ts,
                         size_t hs, float *out)
{
    attn_ctx c = {n_heads, n_kv_heads, head_dim, seq, q, kc, vc, ts, hs, ld_f16, out};
    parallel_rows(n_heads, attn_heads, &c);
}

/* llama_run/src/main.rs:244-252 */
void orc_swiglu(uint32_t n, const float *gate, const float *up, float *out)
{
    for (uint32_t i = 0; i < n; i++) {
        float g = gate[i];
        float s = g / (1.0f + expf(-g));
        out[i] = s * up[i];
    }
}

/* llama_run/src/main.rs:254-261 */
void orc_residual(uint32_t n, const float *y, float *x)
{
    for (uint32_t i = 0; i < n; i++) x[i] = x[i] + y[i];
}

/* llama_run/src/main.rs:263-315: strict >, start -1e30 at index 0, ties to
 * the lowest index (the sequential scan keeps the first maximum). */
uint32_t orc_argmax(uint32_t n, const float *logits)
{
    float bv = -1e30f;
    uint32_t bi = 0;
    for (uint32_t i = 0; i < n; i++)
        if (logits[i] > bv) {
            bv = logits[i];
            bi = i;
        }
    return bi;
}

/* ======================================================================
 * decoder
 * ====================================================================== */
struct orc_model {
    orc_model_config c;
    uint8_t *codes[64][ORC_NPROJ];
    uint8_t *scales[64][ORC_NPROJ]; /* E8M0 bytes or f32, per scale_format */
    uint16_t *norm_attn[64], *norm_ffn[64], *norm_final;
    uint16_t *embed;
    uint8_t *lm_codes, *lm_scales;
    void *kc[64], *vc[64];     /* [kvh][max_seq][hd], fp16 bits or f32 per kv_format */
    int embed_bf16;            /* embeddings hold bf16 (1) or f16 (0) bits; norms are f16 */
    float *cosv, *sinv;
    float *x0;                 /* the harness's activation vector (f32-scale models) */
    /* scratch */
    float *x, *h, *q, *k, *v, *a, *ao, *g, *u, *sw, *d, *logits, *attn_f32_q, *tmpw;
};

static size_t scale_bytes(const orc_model_config *c) { return c->scale_format == ORC_SCALE_F32 ? 4u : 1u; }
static size_t kv_bytes(const orc_model_config *c) { return c->kv_format == ORC_KV_F32 ? 4u : 2u; }

/* y = W.x for one projection of the model, in its scale format. */
static void model_gemv(const orc_model *m, uint32_t n, uint32_t k, const uint8_t *codes, const uint8_t *scales,
                       const float *x, float *y)
{
    if (m->c.scale_format == ORC_SCALE_F32)
        orc_gemv_f32scale(n, k, (const uint32_t *)codes, (const float *)scales, x, y);
    else
        orc_gemv_e8m0(n, k, codes, scales, x, y);
}

/* llama_decode/src/main.rs:307-325 (mk_fp4): n*k/8 words, one xorshift32
 * output each, then n*k/32 scales 0.25 + (r % 8) * 0.03125. */
static void mk_fp4(uint32_t *s, size_t n, size_t k, uint8_t *codes, float *scales)
{
    uint32_t *w = (uint32_t *)codes;
    for (size_t i = 0; i < n * k / 8; i++) w[i] = orc_xorshift32_next(s);
    for (size_t i = 0; i < n * (k / 32); i++) scales[i] = 0.25f + (float)(orc_xorshift32_next(s) % 8u) * 0.03125f;
}

static void proj_shape(const orc_model_config *c, int p, uint32_t *N, uint32_t *K)
{
    uint32_t qd = c->n_heads * c->head_dim, kvd = c->n_kv_heads * c->head_dim;
    switch (p) {
    case ORC_WQ: *N = qd; *K = c->dim; break;
    case ORC_WK: *N = kvd; *K = c->dim; break;
    case ORC_WV: *N = kvd; *K = c->dim; break;
    case ORC_WO: *N = c->dim; *K = qd; break;
    case ORC_WG: *N = c->ffn; *K = c->dim; break;
    case ORC_WU: *N = c->ffn; *K = c->dim; break;
    default: *N = c->dim; *K = c->ffn; break;
    }
}

/* Stream ids of the synthetic init (shared with the device engine). */
#define STREAM_W(l, p) (((uint64_t)(l) << 8) | (uint64_t)(p))
#define STREAM_LM 0xFFFF00ull
#define STREAM_EMBED 0xE0000ull
#define STREAM_NORM(l, w) (0xA0000ull + ((uint64_t)(l) << 1) + (uint64_t)(w))
#define STREAM_NORM_FINAL 0xAFFFFull
#define STREAM_KV(l, isv) (0x4B560000ull + ((uint64_t)(l) << 1) + (uint64_t)(isv))

orc_model *orc_model_create(const orc_model_config *cfg, uint64_t seed)
{
    if (cfg->n_layers > 64 || cfg->scale_format > ORC_SCALE_F32 || cfg->kv_format > ORC_KV_F32) return NULL;
    orc_model *m = (orc_model *)calloc(1, sizeof(orc_model));
    m->c = *cfg;
    const orc_model_config *c = cfg;
    const int f32s = c->scale_format == ORC_SCALE_F32;
    const size_t sb = scale_bytes(c);
    uint32_t xs = (uint32_t)seed; /* mk_fp4 stream (f32 scales) */
    for (uint32_t l = 0; l < c->n_layers; l++) {
        for (int p = 0; p < ORC_NPROJ; p++) {
            uint32_t N, K;
            proj_shape(c, p, &N, &K);
            m->codes[l][p] = (uint8_t *)malloc((size_t)N * K / 2);
            m->scales[l][p] = (uint8_t *)malloc((size_t)N * K / 32 * sb);
            if (f32s)
                mk_fp4(&xs, N, K, m->codes[l][p], (float *)m->scales[l][p]);
            else
                orc_synth_mx_weight(seed, STREAM_W(l, p), 0.02f, K, 0, N, m->codes[l][p], m->scales[l][p]);
        }
        m->norm_attn[l] = (uint16_t *)malloc(sizeof(uint16_t) * c->dim);
        m->norm_ffn[l] = (uint16_t *)malloc(sizeof(uint16_t) * c->dim);
        if (f32s) {
            for (uint32_t i = 0; i < c->dim; i++) m->norm_attn[l][i] = m->norm_ffn[l][i] = 0x3C00u; /* 1.0 */
        } else {
            orc_synth_f16(seed, STREAM_NORM(l, 0), 0.02f, 1.0f, c->dim, m->norm_attn[l]);
            orc_synth_f16(seed, STREAM_NORM(l, 1), 0.02f, 1.0f, c->dim, m->norm_ffn[l]);
        }
        size_t kvn = (size_t)c->n_kv_heads * c->max_seq * c->head_dim;
        m->kc[l] = calloc(kvn, kv_bytes(c));
        m->vc[l] = calloc(kvn, kv_bytes(c));
    }
    m->norm_final = (uint16_t *)malloc(sizeof(uint16_t) * c->dim);
    if (f32s)
        for (uint32_t i = 0; i < c->dim; i++) m->norm_final[i] = 0x3C00u;
    else
        orc_synth_f16(seed, STREAM_NORM_FINAL, 0.02f, 1.0f, c->dim, m->norm_final);
    m->embed = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)c->vocab * c->dim);
    orc_synth_f16(seed, STREAM_EMBED, 0.02f, 0.0f, (size_t)c->vocab * c->dim, m->embed);
    m->lm_codes = (uint8_t *)malloc((size_t)c->vocab * c->dim / 2);
    m->lm_scales = (uint8_t *)malloc((size_t)c->vocab * c->dim / 32 * sb);
    if (f32s)
        mk_fp4(&xs, c->vocab, c->dim, m->lm_codes, (float *)m->lm_scales);
    else
        orc_synth_mx_weight(seed, STREAM_LM, 0.02f, c->dim, 0, c->vocab, m->lm_codes, m->lm_scales);
    /* the harness's activation vector (llama_decode/src/main.rs:421) */
    m->x0 = (float *)calloc(c->dim, sizeof(float));
    if (f32s)
        for (uint32_t i = 0; i < c->dim; i++) m->x0[i] = (float)(orc_xorshift32_next(&xs) % 2001u) / 1000.0f - 1.0f;
    uint32_t half = c->head_dim / 2;
    m->cosv = (float *)malloc(sizeof(float) * (size_t)c->max_seq * half);
    m->sinv = (float *)malloc(sizeof(float) * (size_t)c->max_seq * half);
    orc_rope_table(c->max_seq, c->head_dim, c->theta, m->cosv, m->sinv);
    uint32_t qd = c->n_heads * c->head_dim, kvd = c->n_kv_heads * c->head_dim;
    uint32_t big = c->dim > qd ? c->dim : qd;
    m->x = (float *)calloc(c->dim, sizeof(float));
    m->h = (float *)malloc(sizeof(float) * c->dim);
    m->q = (float *)malloc(sizeof(float) * qd);
    m->k = (float *)malloc(sizeof(float) * kvd);
    m->v = (float *)malloc(sizeof(float) * kvd);
    m->a = (float *)malloc(sizeof(float) * qd);
    m->ao = (float *)malloc(sizeof(float) * big);
    m->g = (float *)malloc(sizeof(float) * c->ffn);
    m->u = (float *)malloc(sizeof(float) * c->ffn);
    m->sw = (float *)malloc(sizeof(float) * c->ffn);
    m->d = (float *)malloc(sizeof(float) * c->dim);
    m->logits = (float *)malloc(sizeof(float) * c->vocab);
    m->tmpw = (float *)malloc(sizeof(float) * c->dim);
    return m;
}

void orc_model_destroy(orc_model *m)
{
    if (!m) return;
    for (uint32_t l = 0; l < m->c.n_layers; l++) {
        for (int p = 0; p < ORC_NPROJ; p++) {
            free(m->codes[l][p]);
            free(m->scales[l][p]);
        }
        free(m->norm_attn[l]);
        free(m->norm_ffn[l]);
        free(m->kc[l]);
        free(m->vc[l]);
    }
    free(m->norm_final);
    free(m->embed);
    free(m->lm_codes);
    free(m->lm_scales);
    free(m->cosv);
    free(m->sinv);
    free(m->x0);
    free(m->x); free(m->h); free(m->q); free(m->k); free(m->v); free(m->a); free(m->ao);
    free(m->g); free(m->u); free(m->sw); free(m->d); free(m->logits); free(m->tmpw);
    free(m);
}

uint8_t *orc_model_codes(orc_model *m, int layer, int proj, size_t *bytes)
{
    uint32_t N, K;
    if (layer < 0) {
        *bytes = (size_t)m->c.vocab * m->c.dim / 2;
        return m->lm_codes;
    }
    proj_shape(&m->c, proj, &N, &K);
    *bytes = (size_t)N * K / 2;
    return m->codes[layer][proj];
}

uint8_t *orc_model_scales(orc_model *m, int layer, int proj, size_t *bytes)
{
    uint32_t N, K;
    if (layer < 0) {
        *bytes = (size_t)m->c.vocab * m->c.dim / 32 * scale_bytes(&m->c);
        return m->lm_scales;
    }
    proj_shape(&m->c, proj, &N, &K);
    *bytes = (size_t)N * K / 32 * scale_bytes(&m->c);
    return m->scales[layer][proj];
}

uint16_t *orc_model_embed(orc_model *m, size_t *count)
{
    *count = (size_t)m->c.vocab * m->c.dim;
    return m->embed;
}

uint16_t *orc_model_norm(orc_model *m, int layer, int which, size_t *count)
{
    *count = m->c.dim;
    if (layer < 0) return m->norm_final;
    return which ? m->norm_ffn[layer] : m->norm_attn[layer];
}

void *orc_model_kcache(orc_model *m, int layer, size_t *count)
{
    *count = (size_t)m->c.n_kv_heads * m->c.max_seq * m->c.head_dim;
    return m->kc[layer];
}

void *orc_model_vcache(orc_model *m, int layer, size_t *count)
{
    *count = (size_t)m->c.n_kv_heads * m->c.max_seq * m->c.head_dim;
    return m->vc[layer];
}

typedef struct {
    orc_model *m;
    uint32_t upto;
    uint64_t seed;
} prefill_ctx;

static void prefill_layers(void *p, size_t a, size_t b)
{
    prefill_ctx *c = (prefill_ctx *)p;
    const orc_model_config *cf = &c->m->c;
    float coef = orc_ih4_coef(0.1f);
    for (size_t l = a; l < b; l++)
        for (int isv = 0; isv < 2; isv++) {
            void *dst = isv ? c->m->vc[l] : c->m->kc[l];
            for (uint32_t t = 0; t < c->upto; t++)
                for (uint32_t kvh = 0; kvh < cf->n_kv_heads; kvh++)
                    for (uint32_t d = 0; d < cf->head_dim; d++) {
                        uint64_t idx = ((uint64_t)t * cf->n_kv_heads + kvh) * cf->head_dim + d;
                        float v = orc_ih4_normal(orc_mix64(c->seed, STREAM_KV(l, isv), idx), coef);
                        size_t at = ((size_t)kvh * cf->max_seq + t) * cf->head_dim + d;
                        if (cf->kv_format == ORC_KV_F32)
                            ((float *)dst)[at] = v;
                        else
                            ((uint16_t *)dst)[at] = orc_f32_to_f16(v);
                    }
        }
}

void orc_model_prefill_kv(orc_model *m, uint64_t seed, uint32_t upto)
{
    prefill_ctx c = {m, upto, seed};
    parallel_rows(m->c.n_layers, prefill_layers, &c);
}

/* Norm weights (f16) and embedding rows (f16 for the synthetic init of
 * BASELINE config 3, or the bf16 bits of a real checkpoint), widened exactly
 * to f32 as the reference's loader does (llama_run/src/main.rs:425-427). */
static void widen_f16(const uint16_t *src, uint32_t n, float *dst)
{
    for (uint32_t i = 0; i < n; i++) dst[i] = orc_f16_to_f32(src[i]);
}

static void widen_embed(const orc_model *m, const uint16_t *src, uint32_t n, float *dst)
{
    for (uint32_t i = 0; i < n; i++) dst[i] = m->embed_bf16 ? orc_bf16_to_f32(src[i]) : orc_f16_to_f32(src[i]);
}

void orc_model_set_embed_bf16(orc_model *m, int bf16) { m->embed_bf16 = bf16 ? 1 : 0; }

void orc_model_fill_kv(orc_model *m, float value, uint32_t upto)
{
    const orc_model_config *c = &m->c;
    if (upto > c->max_seq) upto = c->max_seq;
    const uint16_t h = orc_f32_to_f16(value);
    for (uint32_t l = 0; l < c->n_layers; l++)
        for (int isv = 0; isv < 2; isv++) {
            void *dst = isv ? m->vc[l] : m->kc[l];
            for (uint32_t kvh = 0; kvh < c->n_kv_heads; kvh++)
                for (uint32_t t = 0; t < upto; t++)
                    for (uint32_t d = 0; d < c->head_dim; d++) {
                        size_t at = ((size_t)kvh * c->max_seq + t) * c->head_dim + d;
                        if (c->kv_format == ORC_KV_F32)
                            ((float *)dst)[at] = value;
                        else
                            ((uint16_t *)dst)[at] = h;
                    }
        }
}

void orc_model_harness_begin(orc_model *m) { memcpy(m->x, m->x0, sizeof(float) * m->c.dim); }

/* The layers and the LM head of one decode step on the activation m->x
 * (llama_run/src/main.rs:512-534, llama_decode/src/main.rs:445-466): per
 * layer rmsnorm -> q, k, v GEMVs -> RoPE of q and k -> K/V append at `pos`
 * -> attention over pos + 1 positions -> o GEMV -> residual -> rmsnorm ->
 * gate, up GEMVs -> SwiGLU -> down GEMV -> residual; then the final rmsnorm
 * and the LM-head GEMV into m->logits. */
static void model_layers(orc_model *m, uint32_t pos)
{
    const orc_model_config *c = &m->c;
    uint32_t half = c->head_dim / 2;
    uint32_t qd = c->n_heads * c->head_dim, kvd = c->n_kv_heads * c->head_dim;
    const float *cp = m->cosv + (size_t)pos * half, *sp = m->sinv + (size_t)pos * half;
    for (uint32_t l = 0; l < c->n_layers; l++) {
        widen_f16(m->norm_attn[l], c->dim, m->tmpw);
        orc_rmsnorm(c->dim, c->eps, m->x, m->tmpw, m->h);
        model_gemv(m, qd, c->dim, m->codes[l][ORC_WQ], m->scales[l][ORC_WQ], m->h, m->q);
        model_gemv(m, kvd, c->dim, m->codes[l][ORC_WK], m->scales[l][ORC_WK], m->h, m->k);
        model_gemv(m, kvd, c->dim, m->codes[l][ORC_WV], m->scales[l][ORC_WV], m->h, m->v);
        orc_rope(c->n_heads, c->head_dim, cp, sp, m->q);
        orc_rope(c->n_kv_heads, c->head_dim, cp, sp, m->k);
        for (uint32_t kvh = 0; kvh < c->n_kv_heads; kvh++)
            for (uint32_t d = 0; d < c->head_dim; d++) {
                size_t at = ((size_t)kvh * c->max_seq + pos) * c->head_dim + d;
                if (c->kv_format == ORC_KV_F32) {
                    ((float *)m->kc[l])[at] = m->k[kvh * c->head_dim + d];
                    ((float *)m->vc[l])[at] = m->v[kvh * c->head_dim + d];
                } else {
                    ((uint16_t *)m->kc[l])[at] = orc_f32_to_f16(m->k[kvh * c->head_dim + d]);
                    ((uint16_t *)m->vc[l])[at] = orc_f32_to_f16(m->v[kvh * c->head_dim + d]);
                }
            }
        if (c->kv_format == ORC_KV_F32)
            orc_attn_decode(c->n_heads, c->n_kv_heads, c->head_dim, pos + 1, m->q, (const float *)m->kc[l],
                            (const float *)m->vc[l], c->head_dim, (size_t)c->max_seq * c->head_dim, m->a);
        else
            orc_attn_decode_f16(c->n_heads, c->n_kv_heads, c->head_dim, pos + 1, m->q, (const uint16_t *)m->kc[l],
                                (const uint16_t *)m->vc[l], c->head_dim, (size_t)c->max_seq * c->head_dim, m->a);
        model_gemv(m, c->dim, qd, m->codes[l][ORC_WO], m->scales[l][ORC_WO], m->a, m->ao);
        orc_residual(c->dim, m->ao, m->x);
        widen_f16(m->norm_ffn[l], c->dim, m->tmpw);
        orc_rmsnorm(c->dim, c->eps, m->x, m->tmpw, m->h);
        model_gemv(m, c->ffn, c->dim, m->codes[l][ORC_WG], m->scales[l][ORC_WG], m->h, m->g);
        model_gemv(m, c->ffn, c->dim, m->codes[l][ORC_WU], m->scales[l][ORC_WU], m->h, m->u);
        orc_swiglu(c->ffn, m->g, m->u, m->sw);
        model_gemv(m, c->dim, c->ffn, m->codes[l][ORC_WD], m->scales[l][ORC_WD], m->sw, m->d);
        orc_residual(c->dim, m->d, m->x);
    }
    widen_f16(m->norm_final, c->dim, m->tmpw);
    orc_rmsnorm(c->dim, c->eps, m->x, m->tmpw, m->h);
    model_gemv(m, c->vocab, c->dim, m->lm_codes, m->lm_scales, m->h, m->logits);
}

/* llama_run/src/main.rs:492-536 */
uint32_t orc_model_step(orc_model *m, uint32_t tok, uint32_t pos, float *logits)
{
    const orc_model_config *c = &m->c;
    if (pos >= c->max_seq || tok >= c->vocab) return 0xFFFFFFFFu;
    widen_embed(m, m->embed + (size_t)tok * c->dim, c->dim, m->x);
    model_layers(m, pos);
    if (logits) memcpy(logits, m->logits, sizeof(float) * c->vocab);
    return orc_argmax(c->vocab, m->logits);
}

/* llama_decode/src/main.rs:428-477: the same layers on the carried x; the
 * host argmax scans from f32::MIN with strict > (:467-476). */
uint32_t orc_model_step_noembed(orc_model *m, uint32_t pos, float *logits)
{
    const orc_model_config *c = &m->c;
    if (pos >= c->max_seq) return 0xFFFFFFFFu;
    model_layers(m, pos);
    if (logits) memcpy(logits, m->logits, sizeof(float) * c->vocab);
    uint32_t best = 0;
    float bv = -3.40282347e38f;
    for (uint32_t i = 0; i < c->vocab; i++)
        if (m->logits[i] > bv) {
            bv = m->logits[i];
            best = i;
        }
    return best;
}

/* Batched prefill with MXFP4 activations (the "next" path of the decode
 * engine: the prompt through the MXFP4 GEMM instead of token by token,
 * llama_run/src/main.rs:550-556).  Per layer, every projection input row is
 * RMS-normalised (or taken as is for o and down), quantised with the OCP MX
 * rules (orc_quant_mx), multiplied by the MXFP4 weights exactly in f64
 * (orc_gemm_mx_f64, trackb/fp4_scale_test.cu:37) and rounded to f32; RoPE, the
 * fp16 KV append, attention (causal: row i sees positions < pos0 + i + 1),
 * SwiGLU and the residual adds are the decode step's own
 * (llama_run/src/main.rs:513-530).  The last row's logits come from the f32
 * LM-head GEMV, as in a decode step.  Returns the argmax, writes the logits
 * if asked. */
static void gemm_rows_f32(uint32_t M, uint32_t N, uint32_t K, const uint8_t *ac, const uint8_t *as,
                          const uint8_t *wc, const uint8_t *ws, float *out)
{
    double *c = (double *)malloc(sizeof(double) * (size_t)M * N);
    double *absc = (double *)malloc(sizeof(double) * (size_t)M * N);
    orc_gemm_mx_f64(M, N, K, ac, as, wc, ws, c, absc);
    for (size_t i = 0; i < (size_t)M * N; i++) out[i] = (float)c[i];
    free(c);
    free(absc);
}

uint32_t orc_model_prefill(orc_model *m, const uint32_t *prompt, uint32_t n, uint32_t pos0, float *logits)
{
    const orc_model_config *c = &m->c;
    const uint32_t half = c->head_dim / 2, hd = c->head_dim;
    const uint32_t qd = c->n_heads * hd, kvd = c->n_kv_heads * hd;
    if (n == 0 || pos0 + n > c->max_seq) return 0xFFFFFFFFu;
    if (c->scale_format != ORC_SCALE_E8M0 || c->kv_format != ORC_KV_F16) return 0xFFFFFFFFu; /* MXFP4 GEMM path */
    for (uint32_t i = 0; i < n; i++)
        if (prompt[i] >= c->vocab) return 0xFFFFFFFFu;
    const uint32_t kmax = c->dim > c->ffn ? (c->dim > qd ? c->dim : qd) : (c->ffn > qd ? c->ffn : qd);
    float *X = (float *)malloc(sizeof(float) * (size_t)n * c->dim);
    float *H = (float *)malloc(sizeof(float) * (size_t)n * kmax);
    uint8_t *hc = (uint8_t *)malloc((size_t)n * kmax / 2), *hs = (uint8_t *)malloc((size_t)n * kmax / 32);
    float *Q = (float *)malloc(sizeof(float) * (size_t)n * qd);
    float *Kr = (float *)malloc(sizeof(float) * (size_t)n * kvd), *Vr = (float *)malloc(sizeof(float) * (size_t)n * kvd);
    float *A = (float *)malloc(sizeof(float) * (size_t)n * qd);
    float *O = (float *)malloc(sizeof(float) * (size_t)n * c->dim);
    float *G = (float *)malloc(sizeof(float) * (size_t)n * c->ffn), *U = (float *)malloc(sizeof(float) * (size_t)n * c->ffn);
    for (uint32_t i = 0; i < n; i++) widen_embed(m, m->embed + (size_t)prompt[i] * c->dim, c->dim, X + (size_t)i * c->dim);
    for (uint32_t l = 0; l < c->n_layers; l++) {
        widen_f16(m->norm_attn[l], c->dim, m->tmpw);
        for (uint32_t i = 0; i < n; i++) orc_rmsnorm(c->dim, c->eps, X + (size_t)i * c->dim, m->tmpw, H + (size_t)i * c->dim);
        orc_quant_mx(H, n, c->dim, hc, hs);
        gemm_rows_f32(n, qd, c->dim, hc, hs, m->codes[l][ORC_WQ], m->scales[l][ORC_WQ], Q);
        gemm_rows_f32(n, kvd, c->dim, hc, hs, m->codes[l][ORC_WK], m->scales[l][ORC_WK], Kr);
        gemm_rows_f32(n, kvd, c->dim, hc, hs, m->codes[l][ORC_WV], m->scales[l][ORC_WV], Vr);
        for (uint32_t i = 0; i < n; i++) {
            const uint32_t pos = pos0 + i;
            const float *cp = m->cosv + (size_t)pos * half, *sp = m->sinv + (size_t)pos * half;
            orc_rope(c->n_heads, hd, cp, sp, Q + (size_t)i * qd);
            orc_rope(c->n_kv_heads, hd, cp, sp, Kr + (size_t)i * kvd);
            for (uint32_t kvh = 0; kvh < c->n_kv_heads; kvh++)
                for (uint32_t d = 0; d < hd; d++) {
                    size_t at = ((size_t)kvh * c->max_seq + pos) * hd + d;
                    ((uint16_t *)m->kc[l])[at] = orc_f32_to_f16(Kr[(size_t)i * kvd + kvh * hd + d]);
                    ((uint16_t *)m->vc[l])[at] = orc_f32_to_f16(Vr[(size_t)i * kvd + kvh * hd + d]);
                }
        }
        for (uint32_t i = 0; i < n; i++)
            orc_attn_decode_f16(c->n_heads, c->n_kv_heads, hd, pos0 + i + 1, Q + (size_t)i * qd, (const uint16_t *)m->kc[l],
                                (const uint16_t *)m->vc[l], hd,
                                (size_t)c->max_seq * hd, A + (size_t)i * qd);
        orc_quant_mx(A, n, qd, hc, hs);
        gemm_rows_f32(n, c->dim, qd, hc, hs, m->codes[l][ORC_WO], m->scales[l][ORC_WO], O);
        orc_residual(n * c->dim, O, X);
        widen_f16(m->norm_ffn[l], c->dim, m->tmpw);
        for (uint32_t i = 0; i < n; i++) orc_rmsnorm(c->dim, c->eps, X + (size_t)i * c->dim, m->tmpw, H + (size_t)i * c->dim);
        orc_quant_mx(H, n, c->dim, hc, hs);
        gemm_rows_f32(n, c->ffn, c->dim, hc, hs, m->codes[l][ORC_WG], m->scales[l][ORC_WG], G);
        gemm_rows_f32(n, c->ffn, c->dim, hc, hs, m->codes[l][ORC_WU], m->scales[l][ORC_WU], U);
        orc_swiglu(n * c->ffn, G, U, H);
        orc_quant_mx(H, n, c->ffn, hc, hs);
        gemm_rows_f32(n, c->dim, c->ffn, hc, hs, m->codes[l][ORC_WD], m->scales[l][ORC_WD], O);
        orc_residual(n * c->dim, O, X);
    }
    memcpy(m->x, X + (size_t)(n - 1) * c->dim, sizeof(float) * c->dim);
    widen_f16(m->norm_final, c->dim, m->tmpw);
    orc_rmsnorm(c->dim, c->eps, m->x, m->tmpw, m->h);
    orc_gemv_e8m0(c->vocab, c->dim, m->lm_codes, m->lm_scales, m->h, m->logits);
    if (logits) memcpy(logits, m->logits, sizeof(float) * c->vocab);
    free(X); free(H); free(hc); free(hs); free(Q); free(Kr); free(Vr); free(A); free(O); free(G); free(U);
    return orc_argmax(c->vocab, m->logits);
}

static float top2_margin(const float *v, uint32_t n)
{
    float b1 = -INFINITY, b2 = -INFINITY;
    for (uint32_t i = 0; i < n; i++) {
        if (v[i] > b1) {
            b2 = b1;
            b1 = v[i];
        } else if (v[i] > b2) {
            b2 = v[i];
        }
    }
    return b1 - b2;
}

/* llama_run/src/main.rs:544-570 with the EOS stop disabled (fixed horizon). */
void orc_model_generate(orc_model *m, const uint32_t *prompt, uint32_t n_prompt, uint32_t pos0,
                        uint32_t n_new, uint32_t *out, float *margins)
{
    uint32_t tok = prompt[0], produced = 0;
    for (uint32_t step = 0; produced < n_new; step++) {
        uint32_t next = orc_model_step(m, tok, pos0 + step, NULL);
        if (step + 1 < n_prompt) {
            tok = prompt[step + 1];
        } else {
            if (margins) margins[produced] = top2_margin(m->logits, m->c.vocab);
            out[produced++] = next;
            tok = next;
        }
    }
}
