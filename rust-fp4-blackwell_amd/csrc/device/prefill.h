// Row kernels of the batched prefill (several prompt positions per launch;
// the projections themselves run on the MXFP4 GEMM).  Each restates, per
// row, a piece the decode step already has (embedding lookup, RMSNorm, RoPE,
// fp16 KV append, SwiGLU) and feeds the GEMM's MXFP4 activations with the
// OCP quantizer of the weights (quant_block32).
#pragma once
#include "common.h"
#include "gemv.h"
#include "misc.h"
#include "norm_rope.h"

// grid (rows): y[r] = widen(embed[ids[r]])  (llama_run/src/main.rs:509-510)
RFP4_DEV void embed_rows_body(const RowsArgs &a)
{
    const uint32_t r = blockIdx.x;
    uint32_t tok = a.ids[r];
    if (tok >= a.vocab) tok = 0;
    const uint16_t *row = a.embed + (size_t)tok * a.k;
    for (uint32_t i = threadIdx.x; i < a.k; i += blockDim.x) a.y[(size_t)r * a.k + i] = half_bits_to_f32(row[i], a.bf16 != 0);
}

// grid (rows): RMSNorm of row r with fp16 weights, in the order of
// rmsnorm_body ((x * rms) * w, llama_run/src/main.rs:79-116), then OCP MX
// quantisation per 32 values (8 threads per block, float4 loads).  With
// `add`, the layer's residual add comes first: x = x + add
// (llama_run/src/main.rs:254-261) is stored back and normalised; each
// thread re-reads only the elements it stored.
RFP4_DEV void rmsnorm_quant_rows_body(const RowsArgs &a)
{
    __shared__ float red[16];
    const uint32_t r = blockIdx.x, k4 = a.k / 4u;
    const float4 *x = (const float4 *)(a.x + (size_t)r * a.k);
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < k4; i += blockDim.x) {
        float4 v = x[i];
        if (a.add) {
            const float4 d = ((const float4 *)(a.add + (size_t)r * a.k))[i];
            v = make_float4(__fadd_rn(v.x, d.x), __fadd_rn(v.y, d.y), __fadd_rn(v.z, d.z), __fadd_rn(v.w, d.w));
            ((float4 *)(a.x_out + (size_t)r * a.k))[i] = v;
        }
        ss = __fadd_rn(ss, __fmul_rn(v.x, v.x));
        ss = __fadd_rn(ss, __fmul_rn(v.y, v.y));
        ss = __fadd_rn(ss, __fmul_rn(v.z, v.z));
        ss = __fadd_rn(ss, __fmul_rn(v.w, v.w));
    }
    const float total = block_sum(ss, red);
    const float rms = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(total, (float)a.k), a.eps)));
    const uint2 *w = (const uint2 *)a.w;
    uint8_t *codes = a.codes + (size_t)r * a.k / 2u, *scales = a.scales + (size_t)r * (a.k / 32u);
    for (uint32_t i = threadIdx.x; i < k4; i += blockDim.x) { // k % 32 == 0: whole 8-thread groups
        const float4 v = x[i];
        const uint2 wb = w[i];
        const float4 y = make_float4(__fmul_rn(__fmul_rn(v.x, rms), f16_bits_to_f32((uint16_t)(wb.x & 0xFFFFu))),
                                     __fmul_rn(__fmul_rn(v.y, rms), f16_bits_to_f32((uint16_t)(wb.x >> 16))),
                                     __fmul_rn(__fmul_rn(v.z, rms), f16_bits_to_f32((uint16_t)(wb.y & 0xFFFFu))),
                                     __fmul_rn(__fmul_rn(v.w, rms), f16_bits_to_f32((uint16_t)(wb.y >> 16))));
        quant_block32_x8(y, codes + (i / 8u) * 16u, scales + i / 8u);
    }
}

// grid (rows): s = silu(gate) * up (llama_run/src/main.rs:244-252) of row r
// (gate = columns [0, k), up = [k, 2k) of the stacked gate|up output), then
// OCP MX quantisation per 32 values (8 threads per block, float4 loads).
RFP4_DEV void swiglu_quant_rows_body(const RowsArgs &a)
{
    const uint32_t r = blockIdx.x, k4 = a.k / 4u;
    const float4 *g = (const float4 *)(a.x + (size_t)r * 2u * a.k), *u = g + k4;
    uint8_t *codes = a.codes + (size_t)r * a.k / 2u, *scales = a.scales + (size_t)r * (a.k / 32u);
    for (uint32_t i = threadIdx.x; i < k4; i += blockDim.x) { // k % 32 == 0: whole 8-thread groups
        const float4 gv = g[i], uv = u[i];
        const float4 y = make_float4(__fmul_rn(silu_ref(gv.x), uv.x), __fmul_rn(silu_ref(gv.y), uv.y),
                                     __fmul_rn(silu_ref(gv.z), uv.z), __fmul_rn(silu_ref(gv.w), uv.w));
        quant_block32_x8(y, codes + (i / 8u) * 16u, scales + i / 8u);
    }
}

// grid (rows): RoPE of row r's q and k heads in place at position pos0 + r
// (llama_run/src/main.rs:517-518), then fp16 k (rotated) and v into the
// caches at that position (:519-521).
RFP4_DEV void rope_kv_rows_body(const RopeRowsArgs &a)
{
    const uint32_t r = blockIdx.x, pos = a.pos0 + r, half = a.head_dim / 2u;
    float *row = a.qkv + (size_t)r * a.row_stride;
    const float *cp = a.cosv + (size_t)pos * half, *sp = a.sinv + (size_t)pos * half;
    const uint32_t qd = a.n_heads * a.head_dim, kvd = a.n_kv_heads * a.head_dim;
    for (uint32_t i = threadIdx.x; i < (a.n_heads + a.n_kv_heads) * half; i += blockDim.x) {
        const uint32_t hh = i / half, j = i % half;
        rope_pair(row + hh * a.head_dim, j, half, cp[j], sp[j]); // k heads follow the q heads
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < kvd; i += blockDim.x) {
        const uint32_t kvh = i / a.head_dim, d = i % a.head_dim;
        const size_t at = (size_t)pos * a.ts + (size_t)kvh * a.hs + d;
        a.kc[at] = f32_to_f16_bits(row[qd + i]);
        a.vc[at] = f32_to_f16_bits(row[qd + kvd + i]);
    }
}
