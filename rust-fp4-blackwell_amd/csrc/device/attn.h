// Split-K flash-decode GQA attention for one query token (gfx950).
//
// Semantics: llama_run/src/main.rs:148-242 / llama_attn_decode/src/main.rs:150-179:
//   out[h] = softmax((q_h . k_t) * 1/sqrt(HD)) . v_t  over t < seq, kvh = h / (NH/NKV).
//
// Grid (n_kv_heads, splits).  A workgroup owns one KV head and `chunk` tokens
// and serves every query head of its GQA group, so each K/V byte is read from
// HBM once.  A token row is split over LPT lanes, 16 bytes each, and every
// thread issues the K and V loads of all its tokens before any arithmetic, so
// a workgroup costs one memory round trip.  Each split keeps a local softmax
// state (m, l, acc[HD]); the last workgroup of a KV head to finish (agent-scope
// counter) merges the splits: M = max m_i, L = sum l_i e^(m_i-M),
// out = sum acc_i e^(m_i-M) / L.
//
// Optional fusion (engine): with rope tables given, q and the current token's
// k are rotated here (llama_run/src/main.rs:517-518) and the split owning
// position seq-1 appends fp16 k, v to the caches (:519-521); that split uses
// the new row directly instead of its own load of the not-yet-written row.
#pragma once
#include "common.h"
#include "norm_rope.h"

#define ATTN_MAX_GROUP 8
#define ATTN_MAX_STEPS 8

template <typename KT>
struct KvTraits;
template <>
struct KvTraits<uint16_t> {
    static constexpr int EPL = 8; // elements per 16-byte load
    RFP4_DEV static void widen(const uint4 r, float *o)
    {
        const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            o[2 * i] = f16_bits_to_f32((uint16_t)(w[i] & 0xFFFFu));
            o[2 * i + 1] = f16_bits_to_f32((uint16_t)(w[i] >> 16));
        }
    }
};
template <>
struct KvTraits<float> {
    static constexpr int EPL = 4;
    RFP4_DEV static void widen(const uint4 r, float *o)
    {
        o[0] = __uint_as_float(r.x);
        o[1] = __uint_as_float(r.y);
        o[2] = __uint_as_float(r.z);
        o[3] = __uint_as_float(r.w);
    }
};

// Sum over aligned groups of N lanes (N = 4, 8, 16, 32, 64); every lane of
// the group receives the group sum.
template <int N>
RFP4_DEV float group_sum(float v)
{
    v += dpp_mov<DPP_QUAD_1032>(v);
    v += dpp_mov<DPP_QUAD_2301>(v);
    if (N >= 8) v += dpp_mov<DPP_ROW_HALF_MIRROR>(v);
    if (N >= 16) v += dpp_mov<DPP_ROW_MIRROR>(v);
    if (N >= 32) v += __shfl_xor(v, 16, 64);
    if (N >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

// Merge the nsplit partial states of the G heads of one KV head:
//   M = max m_i, L = sum l_i e^(m_i - M), out = (sum acc_i e^(m_i - M)) / L.
// scratch: >= 4*8*HD floats of LDS (the P.V reduction buffer, free by now).
// (m, l) pairs are staged in LDS with one round of loads; the accumulators
// are read as float4 in batches of independent loads.
template <int HD>
RFP4_DEV void attn_merge(const AttnArgs &a, uint32_t kvh, uint32_t G, uint32_t nsplit, float *scratch, int tid,
                         int lane, int wave)
{
    constexpr uint32_t STRIDE = HD + 4;
    constexpr uint32_t CAP = 4 * ATTN_MAX_GROUP * HD / 2; // (m, l) pairs that fit the scratch
    __shared__ float s_M[ATTN_MAX_GROUP], s_L[ATTN_MAX_GROUP];
    float *ms = scratch, *ls = scratch + CAP;
    const bool staged = G * nsplit <= CAP;
    if (staged) {
        for (uint32_t i = tid; i < G * nsplit; i += blockDim.x) {
            uint32_t g = i / nsplit, sp = i % nsplit;
            const float *pp = a.part + ((size_t)(kvh * G + g) * a.max_splits + sp) * STRIDE;
            ms[i] = pp[0];
            ls[i] = pp[1];
        }
        __syncthreads();
    }
    // per head: M, then e_i = exp(m_i - M) in place of m_i, and L
    for (uint32_t g = wave; g < G; g += 4) {
        const float *hp = a.part + (size_t)(kvh * G + g) * a.max_splits * STRIDE;
        float M = -3.402823466e38f;
        for (uint32_t sp = lane; sp < nsplit; sp += 64) M = fmaxf(M, staged ? ms[g * nsplit + sp] : hp[sp * STRIDE]);
        M = wave_max(M);
        float L = 0.0f;
        for (uint32_t sp = lane; sp < nsplit; sp += 64) {
            float m = staged ? ms[g * nsplit + sp] : hp[sp * STRIDE];
            float l = staged ? ls[g * nsplit + sp] : hp[sp * STRIDE + 1];
            float e = expf(m - M);
            if (staged) ms[g * nsplit + sp] = e;
            L = fmaf(l, e, L);
        }
        L = wave_sum(L);
        if (lane == 0) {
            s_M[g] = M;
            s_L[g] = L;
        }
    }
    __syncthreads();
    // outputs: one float4 of one head per thread, all splits
    const uint32_t quads = G * HD / 4;
    for (uint32_t qd = tid; qd < quads; qd += blockDim.x) {
        const uint32_t g = qd / (HD / 4), d4 = qd % (HD / 4);
        const float *hp = a.part + (size_t)(kvh * G + g) * a.max_splits * STRIDE + 4 + d4 * 4;
        const float M = s_M[g];
        float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        uint32_t sp = 0;
        for (; sp + 8 <= nsplit; sp += 8) {
            float4 v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = *(const float4 *)(hp + (size_t)(sp + j) * STRIDE);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                float e = staged ? ms[g * nsplit + sp + j] : expf(hp[(size_t)(sp + j) * STRIDE - 4 - d4 * 4] - M);
                o.x = fmaf(v[j].x, e, o.x);
                o.y = fmaf(v[j].y, e, o.y);
                o.z = fmaf(v[j].z, e, o.z);
                o.w = fmaf(v[j].w, e, o.w);
            }
        }
        for (; sp < nsplit; sp++) {
            float4 v = *(const float4 *)(hp + (size_t)sp * STRIDE);
            float e = staged ? ms[g * nsplit + sp] : expf(hp[(size_t)sp * STRIDE - 4 - d4 * 4] - M);
            o.x = fmaf(v.x, e, o.x);
            o.y = fmaf(v.y, e, o.y);
            o.z = fmaf(v.z, e, o.z);
            o.w = fmaf(v.w, e, o.w);
        }
        const float L = s_L[g];
        float *dst = a.out + (size_t)(kvh * G + g) * HD + d4 * 4;
        dst[0] = __fdiv_rn(o.x, L);
        dst[1] = __fdiv_rn(o.y, L);
        dst[2] = __fdiv_rn(o.z, L);
        dst[3] = __fdiv_rn(o.w, L);
    }
}

template <int HD, typename KT>
RFP4_DEV void attn_body(const AttnArgs &a)
{
    constexpr int EPL = KvTraits<KT>::EPL;
    constexpr int LPT = HD / EPL;          // lanes per token row
    constexpr int TPS = 256 / LPT;         // tokens per workgroup step
    static_assert(LPT >= 4 && LPT <= 32, "row split");
    __shared__ float qs[ATTN_MAX_GROUP][HD];
    __shared__ float ps[ATTN_MAX_GROUP][TPS * ATTN_MAX_STEPS];
    __shared__ float vred[4][ATTN_MAX_GROUP][HD];
    __shared__ float s_m[ATTN_MAX_GROUP], s_l[ATTN_MAX_GROUP];
    __shared__ uint16_t knew[HD], vnew[HD];
    __shared__ int s_last;

    const uint32_t kvh = blockIdx.x, split = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = tid % LPT, slot = tid / LPT;
    const uint32_t chunk = a.chunk;
    uint32_t seq = a.pos_ptr ? (uint32_t)(*a.pos_ptr + 1) : a.seq;
    seq = min(seq, chunk * a.max_splits); // never read past the planned splits
    const uint32_t nsplit = (seq + chunk - 1) / chunk;
    if (split >= nsplit) return;
    const uint32_t G = a.n_heads / a.n_kv_heads;
    const uint32_t t0 = split * chunk;
    const uint32_t nt = min(seq, t0 + chunk) - t0;
    const uint32_t nstep = (chunk + TPS - 1) / TPS;
    const uint32_t pos = seq - 1;
    const bool fused = a.cosv != nullptr;
    const bool owner = fused && (pos >= t0) && (pos < t0 + nt);
    const KT *kc = (const KT *)a.kc + (size_t)kvh * a.hs;
    const KT *vc = (const KT *)a.vc + (size_t)kvh * a.hs;

    // ---- issue every K and V load of this split first
    uint4 kr[ATTN_MAX_STEPS], vr[ATTN_MAX_STEPS];
#pragma unroll
    for (int s = 0; s < ATTN_MAX_STEPS; s++) {
        uint32_t t = (uint32_t)s * TPS + (uint32_t)slot;
        kr[s] = make_uint4(0, 0, 0, 0);
        vr[s] = make_uint4(0, 0, 0, 0);
        if ((uint32_t)s < nstep && t < nt) {
            size_t off = (size_t)(t0 + t) * a.ts + (size_t)li * EPL;
            kr[s] = *(const uint4 *)(kc + off);
            vr[s] = *(const uint4 *)(vc + off);
        }
    }

    // ---- q (rotated if fused) into LDS; the owner split appends k, v
    const float *qg = a.q + (size_t)(kvh * G) * HD;
    if (fused) {
        const uint32_t half = HD / 2;
        const float *cp = a.cosv + (size_t)pos * half, *sp = a.sinv + (size_t)pos * half;
        for (uint32_t i = tid; i < G * half; i += blockDim.x) {
            uint32_t g = i / half, j = i % half;
            float x0 = qg[g * HD + j], x1 = qg[g * HD + j + half];
            qs[g][j] = __fsub_rn(__fmul_rn(x0, cp[j]), __fmul_rn(x1, sp[j]));
            qs[g][j + half] = __fadd_rn(__fmul_rn(x1, cp[j]), __fmul_rn(x0, sp[j]));
        }
        if (owner) {
            const float *kn = a.k_new + (size_t)kvh * HD, *vn = a.v_new + (size_t)kvh * HD;
            uint16_t *kdst = (uint16_t *)a.kc + (size_t)kvh * a.hs + (size_t)pos * a.ts;
            uint16_t *vdst = (uint16_t *)a.vc + (size_t)kvh * a.hs + (size_t)pos * a.ts;
            for (uint32_t j = tid; j < half; j += blockDim.x) {
                float x0 = kn[j], x1 = kn[j + half];
                uint16_t r0 = f32_to_f16_bits(__fsub_rn(__fmul_rn(x0, cp[j]), __fmul_rn(x1, sp[j])));
                uint16_t r1 = f32_to_f16_bits(__fadd_rn(__fmul_rn(x1, cp[j]), __fmul_rn(x0, sp[j])));
                knew[j] = r0;
                knew[j + half] = r1;
                kdst[j] = r0;
                kdst[j + half] = r1;
            }
            for (uint32_t j = tid; j < HD; j += blockDim.x) {
                uint16_t r = f32_to_f16_bits(vn[j]);
                vnew[j] = r;
                vdst[j] = r;
            }
        }
    } else {
        for (uint32_t i = tid; i < G * HD; i += blockDim.x) qs[i / HD][i % HD] = qg[i];
    }
    __syncthreads();
    if (owner) {
        // the thread holding position `pos` takes the freshly rotated row
        uint32_t tl = pos - t0;
        if ((uint32_t)slot == tl % TPS) {
            uint32_t s = tl / TPS;
            uint4 kk, vv;
            const uint16_t *kp = knew + li * EPL, *vp = vnew + li * EPL;
            kk.x = kp[0] | ((uint32_t)kp[1] << 16); kk.y = kp[2] | ((uint32_t)kp[3] << 16);
            kk.z = kp[4] | ((uint32_t)kp[5] << 16); kk.w = kp[6] | ((uint32_t)kp[7] << 16);
            vv.x = vp[0] | ((uint32_t)vp[1] << 16); vv.y = vp[2] | ((uint32_t)vp[3] << 16);
            vv.z = vp[4] | ((uint32_t)vp[5] << 16); vv.w = vp[6] | ((uint32_t)vp[7] << 16);
#pragma unroll
            for (int st = 0; st < ATTN_MAX_STEPS; st++)
                if ((uint32_t)st == s) {
                    kr[st] = kk;
                    vr[st] = vv;
                }
        }
    }

    // ---- scores
    float qv[ATTN_MAX_GROUP][EPL];
#pragma unroll
    for (int g = 0; g < ATTN_MAX_GROUP; g++)
#pragma unroll
        for (int e = 0; e < EPL; e++) qv[g][e] = (uint32_t)g < G ? qs[g][li * EPL + e] : 0.0f;
    const float scale = __fdiv_rn(1.0f, __fsqrt_rn((float)HD));
#pragma unroll
    for (int s = 0; s < ATTN_MAX_STEPS; s++) {
        if ((uint32_t)s >= nstep) break;
        float kf[EPL];
        KvTraits<KT>::widen(kr[s], kf);
        uint32_t t = (uint32_t)s * TPS + (uint32_t)slot;
#pragma unroll
        for (int g = 0; g < ATTN_MAX_GROUP; g++) {
            if ((uint32_t)g >= G) break;
            float d = 0.0f;
#pragma unroll
            for (int e = 0; e < EPL; e++) d = fmaf(qv[g][e], kf[e], d);
            d = group_sum<LPT>(d);
            if (li == 0 && t < nt) ps[g][t] = d * scale;
        }
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

    // ---- P.V over this thread's tokens, then reduce over token slots
    float acc[ATTN_MAX_GROUP][EPL];
#pragma unroll
    for (int g = 0; g < ATTN_MAX_GROUP; g++)
#pragma unroll
        for (int e = 0; e < EPL; e++) acc[g][e] = 0.0f;
#pragma unroll
    for (int s = 0; s < ATTN_MAX_STEPS; s++) {
        if ((uint32_t)s >= nstep) break;
        uint32_t t = (uint32_t)s * TPS + (uint32_t)slot;
        if (t >= nt) continue;
        float vf[EPL];
        KvTraits<KT>::widen(vr[s], vf);
#pragma unroll
        for (int g = 0; g < ATTN_MAX_GROUP; g++) {
            if ((uint32_t)g >= G) break;
            float p = ps[g][t];
#pragma unroll
            for (int e = 0; e < EPL; e++) acc[g][e] = fmaf(p, vf[e], acc[g][e]);
        }
    }
    // lanes li, li+LPT, ... of a wave hold the same dims: fold them
#pragma unroll
    for (int g = 0; g < ATTN_MAX_GROUP; g++) {
        if ((uint32_t)g >= G) break;
#pragma unroll
        for (int e = 0; e < EPL; e++) {
            float v = acc[g][e];
            for (int off = LPT; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
            acc[g][e] = v;
        }
    }
    if (lane < LPT) {
#pragma unroll
        for (int g = 0; g < ATTN_MAX_GROUP; g++) {
            if ((uint32_t)g >= G) break;
#pragma unroll
            for (int e = 0; e < EPL; e++) vred[wave][g][li * EPL + e] = acc[g][e];
        }
    }
    __syncthreads();

    // ---- write this split's partial state: [m, l, -, -, acc[HD]] per (head, split)
    const uint32_t stride = HD + 4;
    for (uint32_t i = tid; i < G * HD; i += blockDim.x) {
        uint32_t g = i / HD, d = i % HD;
        float v = vred[0][g][d] + vred[1][g][d] + vred[2][g][d] + vred[3][g][d];
        size_t base = ((size_t)(kvh * G + g) * a.max_splits + split) * stride;
        a.part[base + 4 + d] = v;
        if (d == 0) {
            a.part[base] = s_m[g];
            a.part[base + 1] = s_l[g];
        }
    }

    // ---- last workgroup of this KV head merges all splits.  Every wave waits
    // for its own partial stores, then one agent-scope release by thread 0
    // publishes the workgroup's stores before the counter increment (an
    // agent-scope fence writes back the L2, so it is issued once per
    // workgroup, not once per wave); the merging workgroup acquires once.
    __builtin_amdgcn_s_waitcnt(0x0f70); // vmcnt(0)
    __syncthreads();
    if (tid == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        uint32_t prev = atomicAdd(&a.counters[kvh], 1u);
        s_last = (prev == nsplit - 1) ? 1 : 0;
        if (s_last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    __syncthreads();
    if (!s_last) return;
    attn_merge<HD>(a, kvh, G, nsplit, &vred[0][0][0], tid, lane, wave);
    if (tid == 0) a.counters[kvh] = 0u;
}

// Largest chunk (tokens per split) the register plan of attn_body holds.
constexpr uint32_t attn_max_chunk(uint32_t hd, uint32_t elem_bytes)
{
    return (256u / (hd * elem_bytes / 16u)) * ATTN_MAX_STEPS;
}
