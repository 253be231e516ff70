// Split-K flash-decode GQA attention for one query token (gfx950).
//
// Semantics: llama_run/src/main.rs:148-242 / llama_attn_decode/src/main.rs:150-179:
//   out[h] = softmax((q_h . k_t) * 1/sqrt(HD)) . v_t  over t < seq, kvh = h / (NH/NKV).
//
// Grid (n_kv_heads, splits).  A workgroup owns one KV head and `chunk` tokens
// and serves every query head of its GQA group, so each K/V byte is read from
// HBM once.  A token row is split over LPT lanes, 16 bytes each.  The split is
// walked in sub-chunks of as many rows as the registers hold (attn_sub_chunk):
// every K and V load of a sub-chunk is issued before its arithmetic, the next
// sub-chunk's K loads go out right after the scores and its V loads right
// after P.V, and an online softmax (m, l, acc[HD]) carries over.  A split that
// covers the whole sequence writes the output itself; otherwise each split
// writes its state and a second kernel (attn_merge_body, same stream) merges
// them: M = max m_i, L = sum l_i e^(m_i-M), out = sum acc_i e^(m_i-M) / L.
// (A last-workgroup merge inside this kernel would need an agent-scope
// release per workgroup, an L2 writeback on gfx950, which costs more than the
// kernel boundary.)
//
// Optional fusion (engine): with rope tables given, q and the current token's
// k are rotated here (llama_run/src/main.rs:517-518) and the split owning
// position seq-1 appends fp16 k, v to the caches (:519-521); that split uses
// the new row directly instead of its own load of the not-yet-written row.
#pragma once
#include "common.h"
#include "norm_rope.h"

#define ATTN_MAX_GROUP 8
#define ATTN_MAX_STEPS 9

// 16-byte row pieces each thread holds per sub-chunk: 9 for fp16 rows of 128
// (144 tokens, so a 4096-token context needs 29 splits per KV head and 8 KV
// heads fit one workgroup per CU), 8 otherwise.
template <int HD, typename KT>
constexpr int attn_steps()
{
    return (HD == 128 && sizeof(KT) == 2) ? 9 : 8;
}

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
    if (N >= 32) v = xor16_sum(v);
    if (N >= 64) v = xor32_sum(v);
    return v;
}

// ---- in-kernel merge of the split states (no fence).  Every word another
// workgroup reads is written and read with agent-scope atomic accesses
// (global_store / global_load sc1: coherent on their own on gfx950, as the
// compiler's own release/acquire sequences assume), so publishing them
// needs only their completion (s_waitcnt vmcnt(0)) before the arrival
// counter is bumped; no L2 writeback or invalidate.  No workgroup waits for
// another: the one that arrives last merges, the others exit.
RFP4_DEV void attn_store_agent(float *p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
RFP4_DEV float attn_load_agent(const float *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

#define ATTN_INMERGE_MAX_SPLITS 8
// The last split's merge (at most ATTN_INMERGE_MAX_SPLITS splits): every
// thread first issues the loads of its outputs' split values (two outputs of
// the G x HD per thread), one wave per query head turns (m_i, l_i) into the
// weights e^(m_i - M) and L, then each output is sum_i w_i acc_i / L with the
// splits in order.  One round trip of loads.
template <int HD>
RFP4_DEV void attn_merge_last(const AttnArgs &a, const float *prow, uint32_t kvh, uint32_t G, uint32_t nsplit)
{
    constexpr int S = ATTN_INMERGE_MAX_SPLITS, OPT = ATTN_MAX_GROUP * HD / 256; // outputs per thread (max)
    __shared__ uint32_t s_last;
    __shared__ float s_w[ATTN_MAX_GROUP][S], s_L[ATTN_MAX_GROUP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t stride = HD + 4;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); // this thread's states have landed
    __syncthreads();
    if (tid == 0) {
        const uint32_t old = __hip_atomic_fetch_add(a.counters + kvh, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = old + 1u == nsplit ? 1u : 0u;
    }
    __syncthreads();
    if (!s_last) return;
    if (tid == 0) __hip_atomic_store(a.counters + kvh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); // for the next launch
    // split values of this thread's outputs i = tid + 256 j
    float v[OPT][S];
#pragma unroll
    for (int j = 0; j < OPT; j++) {
        const uint32_t i = (uint32_t)tid + 256u * (uint32_t)j;
        const uint32_t g = i / HD, d = i % HD;
        const float *hp = prow + (size_t)(kvh * G + min(g, G - 1u)) * a.max_splits * stride + 4 + d;
#pragma unroll
        for (int sp = 0; sp < S; sp++) v[j][sp] = (g < G && (uint32_t)sp < nsplit) ? attn_load_agent(hp + (size_t)sp * stride) : 0.0f;
    }
    // weights per head (one wave per head; lane = split)
    for (uint32_t g = (uint32_t)wave; g < G; g += 4) {
        const float *hp = prow + (size_t)(kvh * G + g) * a.max_splits * stride;
        const bool in = (uint32_t)lane < nsplit;
        const float m = in ? attn_load_agent(hp + (size_t)lane * stride) : -3.402823466e38f;
        const float l = in ? attn_load_agent(hp + (size_t)lane * stride + 1) : 0.0f;
        const float M = wave_max(m);
        const float w = in ? expf(m - M) : 0.0f;
        if (in) s_w[g][lane] = w;
        const float L = wave_sum(l * w);
        if (lane == 0) s_L[g] = L;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < OPT; j++) {
        const uint32_t i = (uint32_t)tid + 256u * (uint32_t)j;
        const uint32_t g = i / HD, d = i % HD;
        if (g >= G) break;
        float acc = 0.0f;
#pragma unroll
        for (int sp = 0; sp < S; sp++)
            if ((uint32_t)sp < nsplit) acc = fmaf(s_w[g][sp], v[j][sp], acc);
        a.out[(size_t)(kvh * G + g) * HD + d] = __fdiv_rn(acc, s_L[g]);
    }
}

template <int HD, typename KT>
RFP4_DEV void attn_body(const AttnArgs &a)
{
    constexpr int EPL = KvTraits<KT>::EPL;
    constexpr int LPT = HD / EPL;          // lanes per token row
    constexpr int TPS = 256 / LPT;         // tokens per workgroup step
    constexpr int NSTEP = attn_steps<HD, KT>();
    constexpr uint32_t CAPT = TPS * NSTEP;  // tokens of one sub-chunk (held in registers)
    static_assert(LPT >= 4 && LPT <= 32, "row split");
    __shared__ float qs[ATTN_MAX_GROUP][HD];
    __shared__ float ps[ATTN_MAX_GROUP][CAPT];
    __shared__ float vred[4][ATTN_MAX_GROUP][HD];
    __shared__ float s_m[ATTN_MAX_GROUP], s_l[ATTN_MAX_GROUP], s_alpha[ATTN_MAX_GROUP];
    __shared__ uint16_t knew[HD], vnew[HD];

    const uint32_t kvh = blockIdx.x, split = blockIdx.y, row = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = tid % LPT, slot = tid / LPT;
    const uint32_t chunk = a.chunk;
    uint32_t seq = (a.pos_ptr ? (uint32_t)(*a.pos_ptr + 1) : a.seq) + row;
    const float *qrow = a.q + (size_t)row * a.q_rs;
    float *orow = a.out + (size_t)row * a.out_rs;
    float *prow = a.part + (size_t)row * a.n_heads * a.max_splits * (HD + 4);
    seq = min(seq, chunk * a.max_splits); // never read past the planned splits
    const uint32_t nsplit = (seq + chunk - 1) / chunk;
    if (split >= nsplit) return;
    const uint32_t G = a.n_heads / a.n_kv_heads;
    const uint32_t t0 = split * chunk;
    const uint32_t nt = min(seq, t0 + chunk) - t0;
    const uint32_t nsub = (nt + CAPT - 1) / CAPT;
    const uint32_t pos = seq - 1;
    const bool fused = a.cosv != nullptr;
    const bool owner = fused && (pos >= t0) && (pos < t0 + nt);
    const KT *kc = (const KT *)a.kc + (size_t)kvh * a.hs;
    const KT *vc = (const KT *)a.vc + (size_t)kvh * a.hs;

    // ---- K and V rows of sub-chunk C: token t0 + C*CAPT + s*TPS + slot, lanes split the row
    uint4 kr[NSTEP], vr[NSTEP];
#define RFP4_ATTN_LOAD(R, BASE, C)                                                              \
    do {                                                                                        \
        _Pragma("unroll") for (int s_ = 0; s_ < NSTEP; s_++) {                         \
            const uint32_t t_ = (C) * CAPT + (uint32_t)s_ * TPS + (uint32_t)slot;               \
            R[s_] = make_uint4(0, 0, 0, 0);                                                     \
            if (t_ < nt) R[s_] = *(const uint4 *)((BASE) + (size_t)(t0 + t_) * a.ts + (size_t)li * EPL); \
        }                                                                                       \
    } while (0)
    RFP4_ATTN_LOAD(kr, kc, 0u);
    RFP4_ATTN_LOAD(vr, vc, 0u);

    // ---- q (rotated if fused) into LDS; the owner split appends k, v
    const float *qg = qrow + (size_t)(kvh * G) * HD;
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
    if (tid < (int)G) {
        s_m[tid] = -3.402823466e38f;
        s_l[tid] = 0.0f;
    }
    __syncthreads();

    float qv[ATTN_MAX_GROUP][EPL];
#pragma unroll
    for (int g = 0; g < ATTN_MAX_GROUP; g++)
#pragma unroll
        for (int e = 0; e < EPL; e++) qv[g][e] = (uint32_t)g < G ? qs[g][li * EPL + e] : 0.0f;
    const float scale = __fdiv_rn(1.0f, __fsqrt_rn((float)HD));
    float acc[ATTN_MAX_GROUP][EPL];
#pragma unroll
    for (int g = 0; g < ATTN_MAX_GROUP; g++)
#pragma unroll
        for (int e = 0; e < EPL; e++) acc[g][e] = 0.0f;

    for (uint32_t c = 0; c < nsub; c++) {
        const uint32_t tb = c * CAPT, ntc = min(CAPT, nt - tb);
        if (owner && pos - t0 >= tb && pos - t0 < tb + ntc) {
            // the thread holding position `pos` takes the freshly rotated row
            const uint32_t tl = pos - t0 - tb;
            if ((uint32_t)slot == tl % TPS) {
                const uint32_t s = tl / TPS;
                uint4 kk, vv;
                const uint16_t *kp = knew + li * EPL, *vp = vnew + li * EPL;
                kk.x = kp[0] | ((uint32_t)kp[1] << 16); kk.y = kp[2] | ((uint32_t)kp[3] << 16);
                kk.z = kp[4] | ((uint32_t)kp[5] << 16); kk.w = kp[6] | ((uint32_t)kp[7] << 16);
                vv.x = vp[0] | ((uint32_t)vp[1] << 16); vv.y = vp[2] | ((uint32_t)vp[3] << 16);
                vv.z = vp[4] | ((uint32_t)vp[5] << 16); vv.w = vp[6] | ((uint32_t)vp[7] << 16);
#pragma unroll
                for (int st = 0; st < NSTEP; st++)
                    if ((uint32_t)st == s) {
                        kr[st] = kk;
                        vr[st] = vv;
                    }
            }
        }

        // ---- scores of this sub-chunk, then the next sub-chunk's K loads
#pragma unroll
        for (int s = 0; s < NSTEP; s++) {
            const uint32_t t = (uint32_t)s * TPS + (uint32_t)slot;
            if ((uint32_t)s * TPS >= ntc) break;
            float kf[EPL];
            KvTraits<KT>::widen(kr[s], kf);
#pragma unroll
            for (int g = 0; g < ATTN_MAX_GROUP; g++) {
                if ((uint32_t)g >= G) break;
                float d = 0.0f;
#pragma unroll
                for (int e = 0; e < EPL; e++) d = fmaf(qv[g][e], kf[e], d);
                d = group_sum<LPT>(d);
                if (li == 0 && t < ntc) ps[g][t] = d * scale;
            }
        }
        if (c + 1 < nsub) RFP4_ATTN_LOAD(kr, kc, c + 1);
        __syncthreads();

        // ---- online softmax per head (wave w handles heads w, w+4):
        //      m' = max(m, max_t s_t), p_t = e^(s_t - m'), l' = l e^(m - m') + sum_t p_t
        for (uint32_t g = wave; g < G; g += 4) {
            float mc = -3.402823466e38f;
            for (uint32_t t = lane; t < ntc; t += 64) mc = fmaxf(mc, ps[g][t]);
            mc = wave_max(mc);
            const float m_old = s_m[g], m_new = fmaxf(m_old, mc);
            float l = 0.0f;
            for (uint32_t t = lane; t < ntc; t += 64) {
                float p = expf(ps[g][t] - m_new);
                ps[g][t] = p;
                l += p;
            }
            l = wave_sum(l);
            if (lane == 0) {
                const float alpha = expf(m_old - m_new);
                s_alpha[g] = alpha;
                s_l[g] = fmaf(s_l[g], alpha, l);
                s_m[g] = m_new;
            }
        }
        __syncthreads();

        // ---- rescale the running P.V, add this sub-chunk's, then the next sub-chunk's V loads
#pragma unroll
        for (int g = 0; g < ATTN_MAX_GROUP; g++) {
            if ((uint32_t)g >= G) break;
            const float alpha = s_alpha[g];
#pragma unroll
            for (int e = 0; e < EPL; e++) acc[g][e] *= alpha;
        }
#pragma unroll
        for (int s = 0; s < NSTEP; s++) {
            const uint32_t t = (uint32_t)s * TPS + (uint32_t)slot;
            if ((uint32_t)s * TPS >= ntc) break;
            if (t >= ntc) continue;
            float vf[EPL];
            KvTraits<KT>::widen(vr[s], vf);
#pragma unroll
            for (int g = 0; g < ATTN_MAX_GROUP; g++) {
                if ((uint32_t)g >= G) break;
                const float p = ps[g][t];
#pragma unroll
                for (int e = 0; e < EPL; e++) acc[g][e] = fmaf(p, vf[e], acc[g][e]);
            }
        }
        if (c + 1 < nsub) RFP4_ATTN_LOAD(vr, vc, c + 1);
        __syncthreads(); // ps is rewritten by the next sub-chunk
    }
#undef RFP4_ATTN_LOAD

    // lanes li, li+LPT, ... of a wave hold the same dims: fold them (xor 8 by
    // DPP, 16 and 32 by the row-swap instructions; same sums as shuffles)
#pragma unroll
    for (int g = 0; g < ATTN_MAX_GROUP; g++) {
        if ((uint32_t)g >= G) break;
#pragma unroll
        for (int e = 0; e < EPL; e++) {
            float v = acc[g][e];
            if (LPT <= 4) v += __shfl_xor(v, 4, 64);
            if (LPT <= 8) v += dpp_mov<DPP_ROW_ROR8>(v);
            if (LPT <= 16) v = xor16_sum(v);
            acc[g][e] = xor32_sum(v);
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

    if (nsplit == 1) {
        // one split holds the whole sequence: normalise and write the heads' outputs
        for (uint32_t i = tid; i < G * HD; i += blockDim.x) {
            const uint32_t g = i / HD, d = i % HD;
            const float v = vred[0][g][d] + vred[1][g][d] + vred[2][g][d] + vred[3][g][d];
            orow[(size_t)(kvh * G + g) * HD + d] = __fdiv_rn(v, s_l[g]);
        }
        return;
    }

    // ---- write this split's partial state: [m, l, -, -, acc[HD]] per (head, split);
    // the merge kernel launched next on the same stream combines them, or
    // (counters given) the last split of this KV head to arrive does
    const uint32_t stride = HD + 4;
    const bool inmerge = a.counters != nullptr;
    for (uint32_t i = tid; i < G * HD; i += blockDim.x) {
        uint32_t g = i / HD, d = i % HD;
        float v = vred[0][g][d] + vred[1][g][d] + vred[2][g][d] + vred[3][g][d];
        size_t base = ((size_t)(kvh * G + g) * a.max_splits + split) * stride;
        if (inmerge) {
            attn_store_agent(prow + base + 4 + d, v);
            if (d == 0) {
                attn_store_agent(prow + base, s_m[g]);
                attn_store_agent(prow + base + 1, s_l[g]);
            }
        } else {
            prow[base + 4 + d] = v;
            if (d == 0) {
                prow[base] = s_m[g];
                prow[base + 1] = s_l[g];
            }
        }
    }
    if (!inmerge) return;
    attn_merge_last<HD>(a, prow, kvh, G, nsplit);
}

// Merge kernel body: grid (n_heads), launched after attn_body on the same
// stream (the kernel boundary orders the partial states before these reads).
// Computes the split count exactly as attn_body did; one split means
// attn_body already wrote the output.  For query head h:
//   M = max m_i, L = sum l_i e^(m_i - M), out = (sum acc_i e^(m_i - M)) / L,
// computed online (running max).  Thread tid owns float4 q = tid % (HD/4) of
// the head and the splits p, p + P, p + 2P, ... (p = tid / (HD/4), P = 256 /
// (HD/4)), every load of a batch in flight at once; the P partial states of a
// float4 are then combined through LDS.
#define ATTN_MERGE_BATCH 8
template <int HD>
RFP4_DEV void attn_merge_body(const AttnArgs &a)
{
    constexpr uint32_t Q = HD / 4, P = 256 / Q, STRIDE = HD + 4;
    __shared__ float sh[P][Q][6];
    const uint32_t row = blockIdx.z;
    const uint32_t h = blockIdx.x; // the partial state of head h sits at (h * max_splits + split) * STRIDE
    const uint32_t q = threadIdx.x % Q, p = threadIdx.x / Q;
    const float *hp = a.part + (size_t)row * a.n_heads * a.max_splits * STRIDE + (size_t)h * a.max_splits * STRIDE;
    // the first batch is loaded before the split count is known (indices
    // clamped inside the workspace; states past the count are discarded), so
    // the position read and these loads are one round trip
    float2 ml[ATTN_MERGE_BATCH];
    float4 v[ATTN_MERGE_BATCH];
#pragma unroll
    for (int j = 0; j < ATTN_MERGE_BATCH; j++) {
        const uint32_t sp = min(p + P * j, a.max_splits - 1u);
        ml[j] = *(const float2 *)(hp + (size_t)sp * STRIDE);
        v[j] = *(const float4 *)(hp + (size_t)sp * STRIDE + 4 + q * 4);
    }
    uint32_t seq = (a.pos_ptr ? (uint32_t)(*a.pos_ptr + 1) : a.seq) + row;
    seq = min(seq, a.chunk * a.max_splits);
    const uint32_t nsplit = (seq + a.chunk - 1) / a.chunk;
    if (nsplit <= 1) return;
    float M = -3.402823466e38f, L = 0.0f;
    float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (uint32_t sp0 = p; sp0 < nsplit; sp0 += P * ATTN_MERGE_BATCH) {
        if (sp0 != p) {
#pragma unroll
            for (int j = 0; j < ATTN_MERGE_BATCH; j++) {
                const uint32_t sp = min(sp0 + P * j, nsplit - 1u);
                ml[j] = *(const float2 *)(hp + (size_t)sp * STRIDE);
                v[j] = *(const float4 *)(hp + (size_t)sp * STRIDE + 4 + q * 4);
            }
        }
#pragma unroll
        for (int j = 0; j < ATTN_MERGE_BATCH; j++) {
            if (sp0 + P * j >= nsplit) break;
            const float Mn = fmaxf(M, ml[j].x);
            const float ea = expf(M - Mn), eb = expf(ml[j].x - Mn);
            L = fmaf(L, ea, ml[j].y * eb);
            o.x = fmaf(o.x, ea, v[j].x * eb);
            o.y = fmaf(o.y, ea, v[j].y * eb);
            o.z = fmaf(o.z, ea, v[j].z * eb);
            o.w = fmaf(o.w, ea, v[j].w * eb);
            M = Mn;
        }
    }
    float *me = sh[p][q];
    me[0] = M; me[1] = L; me[2] = o.x; me[3] = o.y; me[4] = o.z; me[5] = o.w;
    __syncthreads();
    if (p != 0) return;
    for (uint32_t r = 1; r < P; r++) {
        const float *o2 = sh[r][q];
        const float Mn = fmaxf(M, o2[0]), ea = expf(M - Mn), eb = expf(o2[0] - Mn);
        L = fmaf(L, ea, o2[1] * eb);
        o.x = fmaf(o.x, ea, o2[2] * eb);
        o.y = fmaf(o.y, ea, o2[3] * eb);
        o.z = fmaf(o.z, ea, o2[4] * eb);
        o.w = fmaf(o.w, ea, o2[5] * eb);
        M = Mn;
    }
    float *dst = a.out + (size_t)row * a.out_rs + (size_t)h * HD + q * 4;
    dst[0] = __fdiv_rn(o.x, L);
    dst[1] = __fdiv_rn(o.y, L);
    dst[2] = __fdiv_rn(o.z, L);
    dst[3] = __fdiv_rn(o.w, L);
}

// Tokens of one sub-chunk (the K/V rows attn_body holds in registers at once).
constexpr uint32_t attn_sub_chunk(uint32_t hd, uint32_t elem_bytes)
{
    return (256u / (hd * elem_bytes / 16u)) * ((hd == 128u && elem_bytes == 2u) ? 9u : 8u);
}
