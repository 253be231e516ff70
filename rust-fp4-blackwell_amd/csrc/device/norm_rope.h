// RMSNorm, RoPE, fp16 KV append and embedding gather for gfx950.
// Elementwise arithmetic uses the _rn intrinsics so no multiply-add is fused:
// every element rounds exactly as the reference's CPU loops do.
#pragma once
#include "common.h"

// Block-wide sum of one float per thread (blockDim multiple of 64, <= 1024);
// every thread receives the total.  Waves are combined in fixed order.
RFP4_DEV float block_sum(float v, float *red /* >= 16 floats */)
{
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.0f;
    for (int w = 0; w < nw; w++) t += red[w];
    __syncthreads();
    return t;
}

// y = x * (1/sqrt(sum(x^2)/d + eps)) * w   (llama_run/src/main.rs:79-116,
// order (x*rms)*w as llama_rmsnorm/src/main.rs:77).  One workgroup.
template <int W_F16>
RFP4_DEV void rmsnorm_body(const RmsnormArgs &a)
{
    __shared__ float red[16];
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < a.dim; i += blockDim.x) ss = __fadd_rn(ss, __fmul_rn(a.x[i], a.x[i]));
    float total = block_sum(ss, red);
    float rms = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(total, (float)a.dim), a.eps)));
    for (uint32_t i = threadIdx.x; i < a.dim; i += blockDim.x) {
        float w = W_F16 ? f16_bits_to_f32(((const uint16_t *)a.w)[i]) : ((const float *)a.w)[i];
        a.y[i] = __fmul_rn(__fmul_rn(a.x[i], rms), w);
    }
}

// Rotate-half RoPE on one (head, j) pair: llama_run/src/main.rs:118-138.
RFP4_DEV void rope_pair(float *b, uint32_t j, uint32_t half, float c, float s)
{
    float x0 = b[j], x1 = b[j + half];
    b[j] = __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, s));
    b[j + half] = __fadd_rn(__fmul_rn(x1, c), __fmul_rn(x0, s));
}

RFP4_DEV void rope_body(const RopeArgs &a)
{
    uint32_t half = a.head_dim / 2;
    uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= a.num_heads * half) return;
    uint32_t head = gid / half, j = gid % half;
    rope_pair(a.q + (size_t)head * a.head_dim, j, half, a.cosv[a.cos_base + j], a.sinv[a.cos_base + j]);
}


// x[i] = embed[ids[step]][i] (fp16 or bf16 -> f32): llama_run/src/main.rs:509-510,
// but gathered on the device so no per-token host upload is needed.
RFP4_DEV void embed_body(const EmbedArgs &a)
{
    uint32_t tok = a.ids[a.state->step];
    if (tok >= a.vocab) tok = 0;
    const uint16_t *row = a.embed + (size_t)tok * a.dim;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < a.dim; i += gridDim.x * blockDim.x)
        a.x[i] = half_bits_to_f32(row[i], a.bf16 != 0);
}
