// Split-K flash-decode GQA attention for one query token (gfx950).
//
// Semantics: llama_run/src/main.rs:148-242 / llama_attn_decode/src/main.rs:150-179:
//   out[h] = softmax((q_h . k_t) * 1/sqrt(HD)) . v_t  over t < seq, kvh = h / (NH/NKV).
//
// Grid (n_kv_heads, splits).  A workgroup owns one KV head and `chunk` tokens,
// and serves every query head of its GQA group, so each K/V byte is read from
// HBM once.  Each split keeps a local online-softmax state (m, l, acc[HD]);
// the last workgroup of a KV head to finish (agent-scope counter) merges the
// splits: M = max m_i, L = sum l_i e^(m_i-M), out = sum acc_i e^(m_i-M) / L.
#pragma once
#include "common.h"

#define ATTN_MAX_GROUP 8
#define ATTN_MAX_CHUNK 256

template <typename KT>
RFP4_DEV float kv_ld(const KT *p, size_t i);
template <>
RFP4_DEV float kv_ld<float>(const float *p, size_t i) { return p[i]; }
template <>
RFP4_DEV float kv_ld<uint16_t>(const uint16_t *p, size_t i) { return f16_bits_to_f32(p[i]); }

template <int HD, typename KT>
RFP4_DEV void attn_body(const AttnArgs &a)
{
    constexpr int DPL = HD / 64; // dims per lane in the V pass
    __shared__ float qs[ATTN_MAX_GROUP][HD];
    __shared__ float ps[ATTN_MAX_GROUP][ATTN_MAX_CHUNK];
    __shared__ float vred[4][ATTN_MAX_GROUP][HD];
    __shared__ float s_m[ATTN_MAX_GROUP], s_l[ATTN_MAX_GROUP];
    __shared__ int s_last;

    const uint32_t kvh = blockIdx.x, split = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t chunk = a.chunk;
    uint32_t seq = a.pos_ptr ? (uint32_t)(*a.pos_ptr + 1) : a.seq;
    seq = min(seq, chunk * a.max_splits); // never read past the planned splits
    const uint32_t nsplit = (seq + chunk - 1) / chunk;
    if (split >= nsplit) return;
    const uint32_t G = a.n_heads / a.n_kv_heads;
    const uint32_t t0 = split * chunk;
    const uint32_t nt = min(seq, t0 + chunk) - t0;
    const KT *kc = (const KT *)a.kc + (size_t)kvh * a.hs;
    const KT *vc = (const KT *)a.vc + (size_t)kvh * a.hs;
    const float scale = __fdiv_rn(1.0f, __fsqrt_rn((float)HD));

    for (uint32_t i = tid; i < G * HD; i += blockDim.x) qs[i / HD][i % HD] = a.q[(size_t)(kvh * G) * HD + i];
    __syncthreads();

    // ---- scores: one token per lane, q broadcast from LDS
    for (uint32_t tl = tid; tl < nt; tl += blockDim.x) {
        const KT *krow = kc + (size_t)(t0 + tl) * a.ts;
        float s[ATTN_MAX_GROUP];
#pragma unroll
        for (int g = 0; g < ATTN_MAX_GROUP; g++) s[g] = 0.0f;
#pragma unroll 4
        for (int d = 0; d < HD; d++) {
            float kd = kv_ld<KT>(krow, d);
#pragma unroll
            for (int g = 0; g < ATTN_MAX_GROUP; g++)
                if ((uint32_t)g < G) s[g] = fmaf(qs[g][d], kd, s[g]);
        }
#pragma unroll
        for (int g = 0; g < ATTN_MAX_GROUP; g++)
            if ((uint32_t)g < G) ps[g][tl] = s[g] * scale;
    }
    __syncthreads();

    // ---- local softmax per head: wave w handles heads w, w+4
    for (uint32_t g = wave; g < G; g += 4) {
        float m = -3.402823466e38f;
        for (uint32_t t = lane; t < nt; t += 64) m = fmaxf(m, ps[g][t]);
        m = wave_max(m);
        float l = 0.0f;
        for (uint32_t t = lane; t < nt; t += 64) {
            float p = expf(ps[g][t] - m);
            ps[g][t] = p;
            l += p;
        }
        l = wave_sum(l);
        if (lane == 0) {
            s_m[g] = m;
            s_l[g] = l;
        }
    }
    __syncthreads();

    // ---- P.V: wave w takes tokens t = w (mod 4); lane owns DPL dims
    float acc[ATTN_MAX_GROUP][DPL];
#pragma unroll
    for (int g = 0; g < ATTN_MAX_GROUP; g++)
#pragma unroll
        for (int j = 0; j < DPL; j++) acc[g][j] = 0.0f;
    for (uint32_t t = wave; t < nt; t += 4) {
        const KT *vrow = vc + (size_t)(t0 + t) * a.ts + lane * DPL;
        float v[DPL];
#pragma unroll
        for (int j = 0; j < DPL; j++) v[j] = kv_ld<KT>(vrow, j);
#pragma unroll
        for (int g = 0; g < ATTN_MAX_GROUP; g++)
            if ((uint32_t)g < G) {
                float p = ps[g][t];
#pragma unroll
                for (int j = 0; j < DPL; j++) acc[g][j] = fmaf(p, v[j], acc[g][j]);
            }
    }
#pragma unroll
    for (int g = 0; g < ATTN_MAX_GROUP; g++)
        if ((uint32_t)g < G)
#pragma unroll
            for (int j = 0; j < DPL; j++) vred[wave][g][lane * DPL + j] = acc[g][j];
    __syncthreads();

    // ---- write this split's partial state
    const uint32_t stride = HD + 2;
    for (uint32_t i = tid; i < G * HD; i += blockDim.x) {
        uint32_t g = i / HD, d = i % HD;
        float v = vred[0][g][d] + vred[1][g][d] + vred[2][g][d] + vred[3][g][d];
        size_t base = ((size_t)(kvh * G + g) * a.max_splits + split) * stride;
        a.part[base + 2 + d] = v;
        if (d == 0) {
            a.part[base] = s_m[g];
            a.part[base + 1] = s_l[g];
        }
    }

    // ---- last workgroup of this KV head merges all splits
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        uint32_t prev = atomicAdd(&a.counters[kvh], 1u);
        s_last = (prev == nsplit - 1) ? 1 : 0;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    for (uint32_t i = tid; i < G * HD; i += blockDim.x) {
        uint32_t g = i / HD, d = i % HD;
        size_t hbase = (size_t)(kvh * G + g) * a.max_splits * stride;
        float M = -3.402823466e38f;
        for (uint32_t sp = 0; sp < nsplit; sp++) M = fmaxf(M, a.part[hbase + sp * stride]);
        float L = 0.0f, o = 0.0f;
        for (uint32_t sp = 0; sp < nsplit; sp++) {
            const float *pp = a.part + hbase + sp * stride;
            float e = expf(pp[0] - M);
            L = fmaf(pp[1], e, L);
            o = fmaf(pp[2 + d], e, o);
        }
        a.out[(size_t)(kvh * G + g) * HD + d] = __fdiv_rn(o, L);
    }
    if (tid == 0) a.counters[kvh] = 0u;
}
