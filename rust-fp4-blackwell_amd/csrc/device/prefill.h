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

#define RQ_U 4 // elements per thread whose loads are issued together in the row kernels

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
    // each thread takes elements i, i + T, i + 2T, ... in that order; the
    // loads of RQ_U consecutive ones are issued before any is used (one
    // memory round trip per RQ_U instead of per element)
    constexpr int U = RQ_U;
    __shared__ float red[16];
    const uint32_t r = blockIdx.x, k4 = a.k / 4u, T = blockDim.x;
    const float4 *x = (const float4 *)(a.x + (size_t)r * a.k);
    const float4 *add = a.add ? (const float4 *)(a.add + (size_t)r * a.k) : nullptr;
    float4 *xo = (float4 *)(a.x_out + (size_t)r * a.k);
    const uint2 *w = (const uint2 *)a.w;
    uint8_t *codes = a.codes + (size_t)r * a.k / 2u, *scales = a.scales + (size_t)r * (a.k / 32u);
    float ss = 0.0f;
    if (k4 <= (uint32_t)U * T) {
        // the whole row in registers (one pass of U elements per thread): x,
        // the added row and the norm weights loaded together, the sum, then
        // the scaled values quantised without reloading anything; the same
        // operations in the same order as the two-pass loop below
        float4 v[U], d[U];
        uint2 wb[U];
#pragma unroll
        for (int j = 0; j < U; j++) {
            const uint32_t i = threadIdx.x + (uint32_t)j * T;
            if (i < k4) {
                v[j] = x[i];
                if (add) d[j] = add[i];
                wb[j] = w[i];
            }
        }
#pragma unroll
        for (int j = 0; j < U; j++) {
            const uint32_t i = threadIdx.x + (uint32_t)j * T;
            if (i >= k4) break;
            if (add) {
                v[j] = make_float4(__fadd_rn(v[j].x, d[j].x), __fadd_rn(v[j].y, d[j].y), __fadd_rn(v[j].z, d[j].z),
                                   __fadd_rn(v[j].w, d[j].w));
                xo[i] = v[j];
            }
            ss = __fadd_rn(ss, __fmul_rn(v[j].x, v[j].x));
            ss = __fadd_rn(ss, __fmul_rn(v[j].y, v[j].y));
            ss = __fadd_rn(ss, __fmul_rn(v[j].z, v[j].z));
            ss = __fadd_rn(ss, __fmul_rn(v[j].w, v[j].w));
        }
        const float total = block_sum(ss, red);
        const float rms = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(total, (float)a.k), a.eps)));
#pragma unroll
        for (int j = 0; j < U; j++) {
            const uint32_t i = threadIdx.x + (uint32_t)j * T;
            if (i >= k4) break;
            const float4 y = make_float4(__fmul_rn(__fmul_rn(v[j].x, rms), f16_bits_to_f32((uint16_t)(wb[j].x & 0xFFFFu))),
                                         __fmul_rn(__fmul_rn(v[j].y, rms), f16_bits_to_f32((uint16_t)(wb[j].x >> 16))),
                                         __fmul_rn(__fmul_rn(v[j].z, rms), f16_bits_to_f32((uint16_t)(wb[j].y & 0xFFFFu))),
                                         __fmul_rn(__fmul_rn(v[j].w, rms), f16_bits_to_f32((uint16_t)(wb[j].y >> 16))));
            quant_block32_x8(y, codes + (i / 8u) * 16u, scales + i / 8u,
                             a.scales_t ? a.scales_t + mx_st_offset(r, i / 8u, a.k >> 8) : nullptr);
        }
        return;
    }
    for (uint32_t i0 = threadIdx.x; i0 < k4; i0 += U * T) {
        float4 v[U], d[U];
#pragma unroll
        for (int j = 0; j < U; j++) {
            const uint32_t i = i0 + (uint32_t)j * T;
            if (i < k4) {
                v[j] = x[i];
                if (add) d[j] = add[i];
            }
        }
#pragma unroll
        for (int j = 0; j < U; j++) {
            const uint32_t i = i0 + (uint32_t)j * T;
            if (i >= k4) break;
            if (add) {
                v[j] = make_float4(__fadd_rn(v[j].x, d[j].x), __fadd_rn(v[j].y, d[j].y), __fadd_rn(v[j].z, d[j].z),
                                   __fadd_rn(v[j].w, d[j].w));
                xo[i] = v[j];
            }
            ss = __fadd_rn(ss, __fmul_rn(v[j].x, v[j].x));
            ss = __fadd_rn(ss, __fmul_rn(v[j].y, v[j].y));
            ss = __fadd_rn(ss, __fmul_rn(v[j].z, v[j].z));
            ss = __fadd_rn(ss, __fmul_rn(v[j].w, v[j].w));
        }
    }
    const float total = block_sum(ss, red);
    const float rms = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(total, (float)a.k), a.eps)));
    for (uint32_t i0 = threadIdx.x; i0 < k4; i0 += U * T) { // k % 32 == 0: whole 8-thread groups
        float4 v[U];
        uint2 wb[U];
#pragma unroll
        for (int j = 0; j < U; j++) {
            const uint32_t i = i0 + (uint32_t)j * T;
            if (i < k4) {
                v[j] = add ? xo[i] : x[i];
                wb[j] = w[i];
            }
        }
#pragma unroll
        for (int j = 0; j < U; j++) {
            const uint32_t i = i0 + (uint32_t)j * T;
            if (i >= k4) break;
            const float4 y = make_float4(__fmul_rn(__fmul_rn(v[j].x, rms), f16_bits_to_f32((uint16_t)(wb[j].x & 0xFFFFu))),
                                         __fmul_rn(__fmul_rn(v[j].y, rms), f16_bits_to_f32((uint16_t)(wb[j].x >> 16))),
                                         __fmul_rn(__fmul_rn(v[j].z, rms), f16_bits_to_f32((uint16_t)(wb[j].y & 0xFFFFu))),
                                         __fmul_rn(__fmul_rn(v[j].w, rms), f16_bits_to_f32((uint16_t)(wb[j].y >> 16))));
            quant_block32_x8(y, codes + (i / 8u) * 16u, scales + i / 8u,
                             a.scales_t ? a.scales_t + mx_st_offset(r, i / 8u, a.k >> 8) : nullptr);
        }
    }
}

// grid (rows, parts): s = silu(gate) * up (llama_run/src/main.rs:244-252) of
// row r (gate = columns [0, k), up = [k, 2k) of the stacked gate|up output),
// then OCP MX quantisation per 32 values (8 threads per block, float4 loads,
// the loads of RQ_U consecutive elements of a thread issued together).  Part
// p of the row takes the float4 range [p * per, (p + 1) * per), per a whole
// number of 32-value blocks: several workgroups per row keep more waves in
// flight for the exponentials and divisions.
RFP4_DEV void swiglu_quant_rows_body(const RowsArgs &a)
{
    constexpr int U = RQ_U;
    const uint32_t r = blockIdx.x, k4 = a.k / 4u, T = blockDim.x;
    const uint32_t per = (k4 / 8u + gridDim.y - 1u) / gridDim.y * 8u;
    const uint32_t lo = blockIdx.y * per, hi = min(k4, lo + per);
    const float4 *g = (const float4 *)(a.x + (size_t)r * 2u * a.k), *u = g + k4;
    uint8_t *codes = a.codes + (size_t)r * a.k / 2u, *scales = a.scales + (size_t)r * (a.k / 32u);
    for (uint32_t i0 = lo + threadIdx.x; i0 < hi; i0 += U * T) { // k % 32 == 0: whole 8-thread groups
        float4 gv[U], uv[U];
#pragma unroll
        for (int j = 0; j < U; j++) {
            const uint32_t i = i0 + (uint32_t)j * T;
            if (i < hi) {
                gv[j] = g[i];
                uv[j] = u[i];
            }
        }
#pragma unroll
        for (int j = 0; j < U; j++) {
            const uint32_t i = i0 + (uint32_t)j * T;
            if (i >= hi) break;
            const float4 y = make_float4(__fmul_rn(silu_ref(gv[j].x), uv[j].x), __fmul_rn(silu_ref(gv[j].y), uv[j].y),
                                         __fmul_rn(silu_ref(gv[j].z), uv[j].z), __fmul_rn(silu_ref(gv[j].w), uv[j].w));
            quant_block32_x8(y, codes + (i / 8u) * 16u, scales + i / 8u,
                             a.scales_t ? a.scales_t + mx_st_offset(r, i / 8u, a.k >> 8) : nullptr);
        }
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
