// Elementwise kernels, argmax, decode-cursor bookkeeping, synthetic init and
// the OCP MX quantizer for gfx950.
#pragma once
#include "common.h"

// ---------------------------------------------------------------- fill (memset replacement)
RFP4_DEV void fill_body(const FillArgs &a)
{
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n_words;
         i += (uint64_t)gridDim.x * blockDim.x)
        a.p[i] = a.value;
}

// ---------------------------------------------------------------- copy_into (llama_run/src/main.rs:140-146)
template <int DST_F16>
RFP4_DEV void copy_into_body(const CopyArgs &a)
{
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= a.n) return;
    if (DST_F16)
        ((uint16_t *)a.dst)[(size_t)a.off + i] = f32_to_f16_bits(a.src[i]);
    else
        ((float *)a.dst)[(size_t)a.off + i] = a.src[i];
}

// ---------------------------------------------------------------- swiglu / residual (llama_run/src/main.rs:244-261)
RFP4_DEV void swiglu_body(const EltwiseArgs &a)
{
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= a.n) return;
    float g = a.a[i];
    float s = __fdiv_rn(g, __fadd_rn(1.0f, expf(-g)));
    a.out[i] = __fmul_rn(s, a.b[i]);
}

RFP4_DEV void residual_body(const EltwiseArgs &a)
{
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= a.n) return;
    a.out[i] = __fadd_rn(a.out[i], a.a[i]);
}

// ---------------------------------------------------------------- argmax (llama_run/src/main.rs:263-315)
// One workgroup; strict '>' scan from (-1e30, 0); ties resolve to the lowest
// index through the packed (value, ~index) key.
RFP4_DEV void argmax_body(const ArgmaxArgs &a)
{
    __shared__ unsigned long long red[16];
    unsigned long long best = pack_argmax(-1e30f, 0u);
    for (uint32_t i = threadIdx.x; i < a.n; i += blockDim.x) {
        float v = a.logits[i];
        if (v > -1e30f) {
            unsigned long long k = pack_argmax(v, i);
            best = k > best ? k : best;
        }
    }
    // wave reduce on the 64-bit key
    for (int off = 32; off >= 1; off >>= 1) {
        unsigned long long o = __shfl_xor(best, off, 64);
        best = o > best ? o : best;
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if (lane == 0) red[wave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long b = red[0];
        for (int w = 1; w < nw; w++) b = red[w] > b ? red[w] : b;
        *a.out = 0xFFFFFFFFu - (uint32_t)(b & 0xFFFFFFFFull);
    }
}

// ---------------------------------------------------------------- end of decode step
RFP4_DEV void step_body(const StepArgs &a)
{
    __shared__ unsigned long long red[16];
    unsigned long long best = 0ull;
    for (uint32_t i = threadIdx.x; i < a.n_best; i += blockDim.x) best = a.best[i] > best ? a.best[i] : best;
    for (int off = 32; off >= 1; off >>= 1) {
        unsigned long long o = __shfl_xor(best, off, 64);
        best = o > best ? o : best;
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if (lane == 0) red[wave] = best;
    __syncthreads();
    __shared__ uint32_t s_next;
    if (threadIdx.x == 0) {
        unsigned long long b = red[0];
        for (int w = 1; w < nw; w++) b = red[w] > b ? red[w] : b;
        uint32_t tok = 0xFFFFFFFFu - (uint32_t)(b & 0xFFFFFFFFull);
        StepState st = *a.state;
        *a.last_tok = tok;
        uint32_t nxt = (uint32_t)st.step + 1u;
        if (nxt >= st.n_prompt && nxt < st.ids_cap) a.ids[nxt] = tok;
        // the next step's input token: a prompt token, else this step's argmax
        s_next = nxt < st.n_prompt ? a.ids[nxt] : tok;
        st.step += 1;
        st.pos += 1;
        *a.state = st;
    }
    if (!a.embed) return;
    // the next step's embedding (rfp4_embed's gather, done here so the step
    // graph has one launch less)
    __syncthreads();
    uint32_t t = s_next;
    if (t >= a.vocab) t = 0;
    const uint16_t *row = a.embed + (size_t)t * a.dim;
    for (uint32_t i = threadIdx.x; i < a.dim; i += blockDim.x) a.x[i] = half_bits_to_f32(row[i], a.bf16 != 0);
}

// ---------------------------------------------------------------- OCP MX block quantizer
// Bit-exact twin of the host quantizer: shared exp = floor(log2(amax)) - 2,
// elements RNE onto E2M1 with saturation, all-zero block -> scale byte 0.
RFP4_DEV int floor_log2_pos(float a)
{
    uint32_t u = __float_as_uint(a);
    int e = (int)((u >> 23) & 0xFFu);
    if (e != 0) return e - 127;
    return -118 - (int)__builtin_clz(u & 0x7FFFFFu); // subnormal u*2^-149: msb at 31-clz
}

RFP4_DEV uint32_t e2m1_rne_code(float v)
{
    float a = fabsf(v);
    uint32_t c;
    if (a <= 0.25f) c = 0;
    else if (a < 0.75f) c = 1;
    else if (a <= 1.25f) c = 2;
    else if (a < 1.75f) c = 3;
    else if (a <= 2.5f) c = 4;
    else if (a < 3.5f) c = 5;
    else if (a <= 5.0f) c = 6;
    else c = 7;
    if (__float_as_uint(v) >> 31) c |= 8u;
    return c;
}

// e2m1_rne_code(ldexpf(v, -se)) for two values at once: the gfx950 packed
// conversion divides by its scale operand, here 2^se (se in [-127, 127];
// 2^-127 is subnormal and used as is), and writes a's code to the low nibble
// and b's to the high nibble of byte SEL of w.  Checked against
// e2m1_rne_code on every f32 bit pattern at every shared exponent -127 .. 125
// (signed zeros, subnormals, ties, saturation, infinities, NaNs): identical.
template <int SEL>
RFP4_DEV uint32_t fp4_pack2(uint32_t w, float a, float b, float scale)
{
    return __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, a, b, scale, SEL);
}

// Quantize 32 values; writes 16 code bytes and returns the scale byte.
RFP4_DEV uint32_t quant_block32(const float *v, uint8_t *out16)
{
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    int se = 0;
    uint32_t sbyte = 0;
    if (amax != 0.0f) {
        se = floor_log2_pos(amax) - 2;
        se = se < -127 ? -127 : (se > 127 ? 127 : se);
        sbyte = (uint32_t)(se + 127);
    }
    const float sc = ldexpf(1.0f, se); // 1 where amax is 0 (se = 0)
    uint32_t words[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float *u = v + 8 * j;
        uint32_t w = fp4_pack2<0>(0u, u[0], u[1], sc);
        w = fp4_pack2<1>(w, u[2], u[3], sc);
        w = fp4_pack2<2>(w, u[4], u[5], sc);
        words[j] = fp4_pack2<3>(w, u[6], u[7], sc);
    }
    *(uint4 *)out16 = make_uint4(words[0], words[1], words[2], words[3]);
    return sbyte;
}

// Byte offset of scale block `blk` (32 values along K) of row `row` in the
// step-blocked layout the tiled GEMM reads (GemmArgs::a_st): per 32-row block
// and K step of 256 values, 256 bytes holding, for h = 0, 1 and rows
// r = 0..31, the step's blocks 4h .. 4h + 3 of row r.
RFP4_DEV size_t mx_st_offset(uint32_t row, uint32_t blk, uint32_t nsuper)
{
    return ((size_t)(row >> 5) * nsuper + (blk >> 3)) * 256u + 128u * ((blk >> 2) & 1u) + 4u * (row & 31u) + (blk & 3u);
}

// quant_block32 spread over 8 consecutive lanes: lane part p = lane & 7 holds
// values 4p .. 4p+3 of the block in v, and every lane of the group is active.
// Same shared exponent (the maximum does not depend on the order) and the
// same element arithmetic; part 0 writes the scale byte (and, where scale_t
// is not null, the same byte there: the step-blocked copy), even parts one
// 32-bit word of the 16 code bytes each.
RFP4_DEV void quant_block32_x8(float4 v, uint8_t *codes16, uint8_t *scale, uint8_t *scale_t = nullptr)
{
    const uint32_t p = threadIdx.x & 7u;
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = fmaxf(amax, dpp_mov<DPP_QUAD_1032>(amax));
    amax = fmaxf(amax, dpp_mov<DPP_QUAD_2301>(amax));
    amax = fmaxf(amax, dpp_mov<DPP_ROW_HALF_MIRROR>(amax)); // lane i <-> 7 - i: the other quad of the 8
    int se = 0;
    uint32_t sbyte = 0;
    if (amax != 0.0f) {
        se = floor_log2_pos(amax) - 2;
        se = se < -127 ? -127 : (se > 127 ? 127 : se);
        sbyte = (uint32_t)(se + 127);
    }
    const float sc = ldexpf(1.0f, se); // 1 where amax is 0 (se = 0)
    const uint32_t h = fp4_pack2<1>(fp4_pack2<0>(0u, v.x, v.y, sc), v.z, v.w, sc);
    const uint32_t hn = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)h, DPP_QUAD_1032, 0xF, 0xF, false); // part p ^ 1
    if ((p & 1u) == 0) *(uint32_t *)(codes16 + 2u * p) = h | (hn << 16);
    if (p == 0) {
        *scale = (uint8_t)sbyte;
        if (scale_t) *scale_t = (uint8_t)sbyte;
    }
}

// One thread per 32-block of the synthetic weight.
RFP4_DEV void synth_weight_body(const SynthWeightArgs &a)
{
    const uint64_t nb = a.k / 32;
    const uint64_t total = a.nrows * nb;
    for (uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (uint64_t)gridDim.x * blockDim.x) {
        uint64_t rr = t / nb, blk = t % nb;
        uint64_t base = (a.r0 + rr) * a.k + blk * 32;
        float v[32];
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = ih4_normal(mix64(a.seed, a.stream, base + (uint64_t)i), a.coef);
        uint32_t sb = quant_block32(v, a.packed + (rr * a.k + blk * 32) / 2);
        a.scales[t] = (uint8_t)sb;
    }
}

RFP4_DEV void synth_f16_body(const SynthF16Args &a)
{
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += (uint64_t)gridDim.x * blockDim.x)
        a.out[i] = f32_to_f16_bits(__fadd_rn(a.offset, ih4_normal(mix64(a.seed, a.stream, i), a.coef)));
}

// KV prefill: logical index (t*NKV + kvh)*HD + d, stored at [kvh][t][d].
RFP4_DEV void synth_kv_body(const SynthKvArgs &a)
{
    const uint64_t total = (uint64_t)a.upto * a.n_kv_heads * a.head_dim;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (uint64_t)gridDim.x * blockDim.x) {
        uint64_t d = i % a.head_dim, r = i / a.head_dim, kvh = r % a.n_kv_heads, t = r / a.n_kv_heads;
        float v = ih4_normal(mix64(a.seed, a.stream, i), a.coef);
        const uint64_t at = (kvh * a.max_seq + t) * a.head_dim + d;
        if (a.kv_f32)
            ((float *)a.cache)[at] = v;
        else
            ((uint16_t *)a.cache)[at] = f32_to_f16_bits(v);
    }
}

// f32 (SRC_BF16=0) or bf16 rows -> MXFP4, one thread per block.
template <int SRC_BF16>
RFP4_DEV void quant_mx_body(const QuantMxArgs &a)
{
    // one float4 (or 4 bf16) per thread and step, 8 threads per 32-block:
    // k % 32 == 0 makes every 8-lane group lie inside one block of one row
    const uint64_t total4 = a.rows * a.k / 4u;
    for (uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total4; t += (uint64_t)gridDim.x * blockDim.x) {
        float4 v;
        if (SRC_BF16) {
            const uint2 b = ((const uint2 *)a.src)[t];
            v = make_float4(__uint_as_float(b.x << 16), __uint_as_float(b.x & 0xFFFF0000u), __uint_as_float(b.y << 16),
                            __uint_as_float(b.y & 0xFFFF0000u));
        } else {
            v = ((const float4 *)a.src)[t];
        }
        uint8_t *st = nullptr;
        if (a.scales_t) {
            const uint64_t k4 = a.k / 4u, row = t / k4;
            st = a.scales_t + mx_st_offset((uint32_t)row, (uint32_t)((t - row * k4) / 8u), (uint32_t)(a.k >> 8));
        }
        quant_block32_x8(v, a.packed + (t / 8u) * 16u, a.scales + t / 8u, st);
    }
}

// ---------------------------------------------------------------- self-tests
// out[2i], out[2i+1] = hardware E2M1 conversion of byte i&3 of in[i>>2]
// (pins the builtin's nibble order against the host codec).
RFP4_DEV void selftest_cvt_body(const SelftestArgs &a)
{
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= a.n) return;
    uint32_t w = a.in[i];
    f32x2 v0 = fp4x2_to_f32<0>(w), v1 = fp4x2_to_f32<1>(w), v2 = fp4x2_to_f32<2>(w), v3 = fp4x2_to_f32<3>(w);
    float *o = a.out + (size_t)i * 8;
    o[0] = v0.x; o[1] = v0.y; o[2] = v1.x; o[3] = v1.y;
    o[4] = v2.x; o[5] = v2.y; o[6] = v3.x; o[7] = v3.y;
}
