/*
 * oracle.h -- CPU restatement of the reference's MXFP4 Llama decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker.
 * The product (rust-fp4-blackwell_amd/) never links, loads or calls it.
 *
 * Every function restates the reference algorithm it names (file:line under
 * botBehavior/rust-fp4-blackwell).  Arithmetic is plain IEEE f32 in the
 * reference's evaluation order: the library is built with -O2
 * -ffp-contract=off and without -ffast-math, so `a*b + c` stays two roundings
 * exactly as in the reference's Rust CPU loops.
 *
 * Multithreaded entry points partition work by output row; each row is
 * computed by exactly one thread in the reference's k-order, so results are
 * bit-identical for any thread count.
 */
#ifndef RFP4_ORACLE_H
#define RFP4_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- threads */
void orc_set_threads(int n);   /* 0 = all online cores */
int orc_get_threads(void);

/* ---------------------------------------------------------------- RNG */
/* xorshift32 13/17/5: fp4_gemv/src/main.rs:101-107, llama_decode/src/main.rs:300-305 */
uint32_t orc_xorshift32_next(uint32_t *state);
void orc_xorshift32_fill(uint32_t *state, uint32_t *out, size_t n);
/* Counter-based 64-bit hash (SplitMix64 finalizer) of (seed, stream, index). */
uint64_t orc_mix64(uint64_t seed, uint64_t stream, uint64_t index);
/* Irwin-Hall(4) approximate N(0,1): sum of the four 16-bit fields of r, centred,
 * divided by the exact std 37837.22723720648; returned as (float)s * c where
 * c = (float)(sigma / 37837.22723720648). Integer-exact up to one f32 multiply. */
float orc_ih4_coef(float sigma);
float orc_ih4_normal(uint64_t r, float coef);

/* ---------------------------------------------------------------- codecs */
/* E2M1 by table {0,.5,1,1.5,2,3,4,6}, bit3 = sign: fp4_gemv/src/main.rs:130-134 */
float orc_e2m1_decode(uint8_t code);
/* E2M1 by arithmetic (fp4_val): llama_run/src/main.rs:21-32 */
float orc_e2m1_decode_arith(uint32_t code);
/* E8M0: value 2^(b-127); 0xFF is NaN (OCP MX v1.0). trackb/FP4_M16N8K64_LAYOUT.md:20 */
float orc_e8m0_decode(uint8_t b);
/* ue8m0 = 127 + lround(log2(s)) for power-of-two s: trackb/fp4_scale_test.cu:12 */
uint8_t orc_e8m0_encode_pow2(float s);
/* E2M1 round-to-nearest-even with saturation to +-6 (OCP MX conversion). */
uint8_t orc_e2m1_rne(float v);
/* fp16 <-> f32. half_to_f32: llama_run/src/main.rs:591-614; f32->f16 is RNE. */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
float orc_bf16_to_f32(uint16_t h);          /* llama_run/src/main.rs:425 */
uint16_t orc_f32_to_bf16(float f);          /* RNE */

/* Packing: two E2M1 codes per byte, low nibble = lower k.  Equal to the
 * reference's little-endian u32 of 8 nibbles: fp4_gemv/src/main.rs:113-120 */
void orc_pack_codes(const uint8_t *codes, size_t n, uint8_t *packed);
void orc_unpack_codes(const uint8_t *packed, size_t n, uint8_t *codes);

/* ---------------------------------------------------------------- quantizers */
/* quant_fp4: absmax/6 f32 scale, nearest level with ties to the lower code,
 * sign iff v<0: llama_run/src/main.rs:334-376 */
void orc_quant_fp4_absmax(const float *w, int outd, int ind, uint8_t *packed, float *scales);
/* OCP MX v1.0 E2M1/E8M0: shared exp = floor(log2(amax)) - 2, elements RNE and
 * saturated; all-zero block -> scale byte 0. */
void orc_quant_mx(const float *w, size_t rows, size_t ind, uint8_t *packed, uint8_t *scales);

/* Synthetic MXFP4 weight: element (r,k) = ih4_normal(mix64(seed,stream,r*K+k)),
 * quantized with orc_quant_mx per 32-block.  Rows [r0, r0+nrows). */
void orc_synth_mx_weight(uint64_t seed, uint64_t stream, float sigma, size_t K,
                         size_t r0, size_t nrows, uint8_t *packed, uint8_t *scales);
/* Synthetic fp16 tensor: f16(offset + ih4_normal(mix64(seed,stream,i))). */
void orc_synth_f16(uint64_t seed, uint64_t stream, float sigma, float offset,
                   size_t n, uint16_t *out);

/* ---------------------------------------------------------------- GEMV */
/* fp4_gemv CPU reference, f32 scales: fp4_gemv/src/main.rs:130-143.
 * y[n] = sum_k (fp4(c)*scale)*x[k], accumulated in k order. */
void orc_gemv_f32scale(uint32_t n, uint32_t k, const uint32_t *w, const float *scales,
                       const float *x, float *y);
/* Same loop with E8M0 scales (BASELINE config 1 numerics). */
void orc_gemv_e8m0(uint32_t n, uint32_t k, const uint8_t *codes, const uint8_t *scales,
                   const float *x, float *y);
/* f64 accumulation of the same products, plus sum_k |w_k x_k| per row
 * (for condition-aware tolerances). */
void orc_gemv_e8m0_f64(uint32_t n, uint32_t k, const uint8_t *codes, const uint8_t *scales,
                       const float *x, double *y, double *absy);

/* ---------------------------------------------------------------- MMA / GEMM */
/* trackb Dref closed form: D[i][j] = sum_k A*SFA[i][k/32]*B*SFB[k/32][j]
 * (trackb/fp4_scale_test.cu:37), f32, k order. A 16x64, B 64x8 row-major. */
void orc_mma_m16n8k64_ref(const float *A, const float *B, const float *SFA,
                          const float *SFB, float *D);
/* Dual-quantized MXFP4 GEMM: C[m][n] = sum_k deq(A[m][k]) * deq(W[n][k]) in f64
 * (A: M x K codes+E8M0, W: N x K codes+E8M0), output as double. */
void orc_gemm_mx_f64(uint32_t M, uint32_t N, uint32_t K, const uint8_t *a_codes,
                     const uint8_t *a_scales, const uint8_t *w_codes, const uint8_t *w_scales,
                     double *c, double *absc);

/* ---------------------------------------------------------------- layers */
/* llama_rmsnorm/src/main.rs:75-77 */
void orc_rmsnorm(uint32_t dim, float eps, const float *x, const float *w, float *y);
/* rotary table [pos][hd/2], freq in f64: llama_run/src/main.rs:462-471 */
void orc_rope_table(uint32_t max_pos, uint32_t head_dim, double theta, float *cosv, float *sinv);
/* rotate-half, in place: llama_rope/src/main.rs:75-84 (cos/sin of one position) */
void orc_rope(uint32_t num_heads, uint32_t head_dim, const float *cosp, const float *sinp, float *q);
/* GQA single-query attention: llama_attn_decode/src/main.rs:150-179.
 * K/V element (t, kvh, i) at kc[t*ts + kvh*hs + i] (f32), i.e. any token/head
 * stride, so the reference [t][kvh][hd] layout and head-major layouts share it. */
void orc_attn_decode(uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim, uint32_t seq,
                     const float *q, const float *kc, const float *vc, size_t ts, size_t hs,
                     float *out);
/* Same, reading fp16 K/V (decoded with orc_f16_to_f32). */
void orc_attn_decode_f16(uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim, uint32_t seq,
                         const float *q, const uint16_t *kc, const uint16_t *vc, size_t ts,
                         size_t hs, float *out);
/* llama_run/src/main.rs:244-252 */
void orc_swiglu(uint32_t n, const float *gate, const float *up, float *out);
/* llama_run/src/main.rs:254-261 */
void orc_residual(uint32_t n, const float *y, float *x);
/* llama_run/src/main.rs:263-315: lowest index on ties, start -1e30, strict > */
uint32_t orc_argmax(uint32_t n, const float *logits);

/* ---------------------------------------------------------------- decoder */
typedef struct orc_model_config {
    uint32_t dim, n_layers, n_heads, n_kv_heads, head_dim, ffn, vocab, max_seq;
    double theta;
    float eps;
    uint16_t scale_format; /* ORC_SCALE_*: per-32 block scales of every projection */
    uint16_t kv_format;    /* ORC_KV_*: element type of the K/V caches */
} orc_model_config;

enum { ORC_SCALE_E8M0 = 0, ORC_SCALE_F32 = 1 };
enum { ORC_KV_F16 = 0, ORC_KV_F32 = 1 };

/* Projection order inside a layer (stream ids for the synthetic init). */
enum { ORC_WQ = 0, ORC_WK, ORC_WV, ORC_WO, ORC_WG, ORC_WU, ORC_WD, ORC_NPROJ };

typedef struct orc_model orc_model;

/* Allocate a model with synthetic weights generated on the CPU from `seed` --
 * the same generators the device engine uses, so packed bytes are identical.
 *  - E8M0 scales: weights N(0, 0.02^2) quantized by the OCP MX rules,
 *    embeddings N(0, 0.02^2) in f16, norms 1 + 0.02*N in f16.
 *  - f32 scales: the reference harness's mk_fp4 (llama_decode/src/main.rs:
 *    300-325,369-393): xorshift32 seeded with the low 32 bits of `seed`,
 *    per layer q, k, v, o, gate, up, down, then the LM head, each as all its
 *    packed words (uniform codes) followed by all its scales
 *    0.25 + (r % 8) * 0.03125; then the harness's activation vector
 *    (r % 2001) / 1000 - 1 (:421).  Norms 1.0 (:381-383,392); embeddings as
 *    the E8M0 model's (the harness has none). */
orc_model *orc_model_create(const orc_model_config *cfg, uint64_t seed);
void orc_model_destroy(orc_model *m);
/* Embeddings are bf16 bit patterns (a real checkpoint) instead of f16. */
void orc_model_set_embed_bf16(orc_model *m, int bf16);
/* Raw views for hashing / comparison against the device engine. */
uint8_t *orc_model_codes(orc_model *m, int layer, int proj, size_t *bytes);
uint8_t *orc_model_scales(orc_model *m, int layer, int proj, size_t *bytes);
uint16_t *orc_model_embed(orc_model *m, size_t *count);
uint16_t *orc_model_norm(orc_model *m, int layer, int which, size_t *count); /* which: 0 attn, 1 ffn; layer=-1 final */
/* K/V caches [kvh][max_seq][hd], fp16 bits or f32 per kv_format; count in elements */
void *orc_model_kcache(orc_model *m, int layer, size_t *count);
void *orc_model_vcache(orc_model *m, int layer, size_t *count);
/* Fill positions [0, upto) of every layer's K/V cache with f16(0.1*N) from
 * (seed, stream 0x4B560000 + 2*layer (+1 for V), index (t*NKV+kvh)*HD+d). */
void orc_model_prefill_kv(orc_model *m, uint64_t seed, uint32_t upto);
/* The reference harness's context (llama_decode/src/main.rs:375-376,388-389):
 * positions [0, upto) of every K/V cache set to `value` (rounded to fp16 for
 * fp16 caches); and its persistent activation x := the vector drawn after the
 * weights (f32-scale models only, else zeros). */
void orc_model_fill_kv(orc_model *m, float value, uint32_t upto);
void orc_model_harness_begin(orc_model *m);
/* One step of the harness (llama_decode/src/main.rs:428-477): no embedding
 * lookup, x carries over from the previous step; returns the argmax of the
 * logits (strict >, first maximum). */
uint32_t orc_model_step_noembed(orc_model *m, uint32_t pos, float *logits);
/* One decode step (llama_run/src/main.rs:492-536): token `tok` at position
 * `pos`; writes logits (vocab floats) if non-null; returns the argmax. */
uint32_t orc_model_step(orc_model *m, uint32_t tok, uint32_t pos, float *logits);
/* Prompt-then-greedy loop (llama_run/src/main.rs:544-570 without the EOS stop):
 * feeds prompt[0..n_prompt) from position pos0, then generates n_new tokens.
 * out[i] = token produced after step i (n_prompt + n_new - 1 entries after the
 * first prompt token); margins[i] = top1 - top2 logit at that step (optional). */
void orc_model_generate(orc_model *m, const uint32_t *prompt, uint32_t n_prompt, uint32_t pos0,
                        uint32_t n_new, uint32_t *out, float *margins);
/* Batched prefill of prompt[0..n) at positions pos0.. with MXFP4 activations
 * (every projection input quantised per 32 along K with the OCP rules, the
 * GEMM exact in f64 then rounded to f32); writes the K/V caches of those
 * positions; returns the argmax of the last row's logits (written to
 * `logits` if non-null).  No reference counterpart: the reference feeds the
 * prompt token by token (llama_run/src/main.rs:550-556). */
uint32_t orc_model_prefill(orc_model *m, const uint32_t *prompt, uint32_t n, uint32_t pos0, float *logits);

#ifdef __cplusplus
}
#endif
#endif
