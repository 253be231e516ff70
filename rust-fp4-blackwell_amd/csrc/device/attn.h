// Split-K flash-decode GQA attention for one query token (gfx950).
//
// Semantics: llama_run/src/main.rs:148-242 / llama_attn_decode/src/main.rs:150-179:
//   out[h] = softmax((q_h . k_t) * 1/sqrt(HD)) . v_t  over t < seq, kvh = h / (NH/NKV).
//
// Grid (n_kv_heads, splits).  A workgroup owns one KV head and `chunk` tokens
// and serves every query head of its GQA group (GT heads at compile time, the
// real group G <= GT; heads past G carry zero q and write nothing), so each
// K/V byte is read from HBM once.  A token row is split over LPT lanes, 16
// bytes each.  The split is walked in sub-chunks of as many rows as the
// registers hold (attn_steps_for): every K and V load of a sub-chunk is issued
// before its arithmetic, the next sub-chunk's K loads go out right after the
// scores and its V loads right after P.V.  Loads that need no position (q, the
// current token's k and v) go out first, then the rope tables of the position,
// then K and V, so the rotation of q overlaps the K/V stream.  Scores stay in
// registers: one cross-wave max per head and sub-chunk, then p = 2^(s - m),
// l and P.V in registers, an online rescale carrying (m, l, acc[HD]) from one
// sub-chunk to the next.  A split that covers the whole sequence writes the
// output itself; otherwise each split writes its state and the states are
// merged, M = max m_i, L = sum l_i 2^(m_i-M), out = sum acc_i 2^(m_i-M) / L,
// by the last split to finish (attn_merge_last, few splits) or by a second
// kernel on the same stream (attn_merge_body).
//
// Optional fusion (engine): with rope tables given, q and the current token's
// k are rotated here (llama_run/src/main.rs:517-518) and the split owning
// position seq-1 appends k, v to the caches (:519-521), rounded to the cache's
// element type (fp16 RNE, or f32 as the reference's copy_into); that split uses
// the new row directly instead of its own load of the not-yet-written row.
#pragma once
#include "common.h"
#include "norm_rope.h"

#define ATTN_MAX_GROUP 8

// Scores are kept in base-2 units, s = (q . k) * (log2(e) / sqrt(HD)), so
// every exponential is one v_exp_f32 (2^x) of a difference; the split states'
// m is in the same units (softmax weights are unchanged: 2^(s2 - m2) =
// e^(s - m)).  Relative error of a weight: the hardware 2^x (about 1 ulp)
// plus the rounding of the scaled score (|s| * 2^-24).
RFP4_DEV float attn_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

template <typename KT>
struct KvTraits;
// Per KV element type: elements per 16-byte load, widening to f32, the
// cache's rounding of a new f32 value (fp16: RNE; f32: as is), and the
// 16-byte load of EPL stored elements.
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
    RFP4_DEV static uint16_t from_f32(float v) { return f32_to_f16_bits(v); }
    RFP4_DEV static uint4 pack(const uint16_t *p)
    {
        return make_uint4(p[0] | ((uint32_t)p[1] << 16), p[2] | ((uint32_t)p[3] << 16), p[4] | ((uint32_t)p[5] << 16),
                          p[6] | ((uint32_t)p[7] << 16));
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
    RFP4_DEV static float from_f32(float v) { return v; }
    RFP4_DEV static uint4 pack(const float *p)
    {
        return make_uint4(__float_as_uint(p[0]), __float_as_uint(p[1]), __float_as_uint(p[2]), __float_as_uint(p[3]));
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

// Sum / max over the token slots of a wave: lanes that hold the same part of
// a row (the same lane index within groups of LPT) are combined (xor 4 by a
// swizzle, xor 8 by DPP row_ror:8, 16 and 32 by the row-swap instructions).
template <int LPT>
RFP4_DEV float slots_sum(float v)
{
    if (LPT <= 4) v += __shfl_xor(v, 4, 64);
    if (LPT <= 8) v += dpp_mov<DPP_ROW_ROR8>(v);
    if (LPT <= 16) v = xor16_sum(v);
    return xor32_sum(v);
}

template <int LPT>
RFP4_DEV float slots_max(float v)
{
    if (LPT <= 4) v = fmaxf(v, __shfl_xor(v, 4, 64));
    if (LPT <= 8) v = fmaxf(v, dpp_mov<DPP_ROW_ROR8>(v));
    if (LPT <= 16) v = xor16_max(v);
    return xor32_max(v);
}

// ---- in-kernel merge of the split states (no fence).  No workgroup waits
// for another: the one that arrives last merges, the others exit.
//
// HARD REQUIREMENT (gfx950 memory system): this protocol publishes one
// workgroup's split state to another without a release/acquire pair.  It
// holds because on gfx950 (a) a relaxed agent-scope atomic store compiles to
// global_store ... sc1, which writes through the XCD's L2 to the device-
// coherent level, (b) a relaxed agent-scope atomic load compiles to
// global_load ... sc1, which misses the non-coherent L2 and reads that level,
// and (c) s_waitcnt vmcnt(0) returns only after this thread's stores are
// acknowledged there.  So every state word is stored with agent-scope stores,
// every thread waits for its own stores (vmcnt(0)), the workgroup
// synchronises, and only then does one thread bump the KV head's arrival
// counter (a device-coherent atomic); the workgroup whose increment completes
// the count has every other split's stores acknowledged before their
// increments, and its agent-scope loads read them.  These are the cache-bypass
// semantics the compiler's own agent-scope release/acquire sequences assume
// on this target, minus the L2 writeback and invalidate (buffer_wbl2 /
// buffer_inv sc1) that a fence adds: measured at 5.8 us per launch on 264
// workgroups.  Another target, or a compiler that stops mapping these atomics
// to sc1 accesses, needs the fence back.  The merge-mode tests compare with
// the second-kernel merge and repeat the in-kernel merge 20 times (a stale
// state would change a result).  The in-kernel merge is used up to 8 splits:
// measured at 29 splits (the 8B context), its atomic and state round trips
// cost 5.5 us inside the kernel against 4.2 us for the merge kernel.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "the in-kernel attention merge's publication protocol is written for gfx950's sc1 accesses"
#endif
RFP4_DEV void attn_store_agent(float *p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
RFP4_DEV float attn_load_agent(const float *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

#define ATTN_INMERGE_MAX_SPLITS 8
// Splits the persistent decode kernel merges in place (one round of loads).
#define ATTN_PERSIST_MAX_SPLITS 32
// Splits per batch of the merge kernel's loads.
#define ATTN_MERGE_BATCH 64
// Splits of the tagged in-kernel merge (at most ATTN_MERGE_BATCH: the merge
// kernel's summation order is one batch).
#define ATTN_TAG_MAX_SPLITS 32
// The last split's merge (at most ATTN_INMERGE_MAX_SPLITS splits): every
// thread first issues the loads of its outputs' split values (the G x HD
// outputs, 256 per pass), one wave per query head turns (m_i, l_i) into the
// weights 2^(m_i - M) and L, then each output is sum_i w_i acc_i / L with the
// splits in order.  One round trip of loads.
template <int HD, int GT>
RFP4_DEV void attn_merge_last(const AttnArgs &a, const float *prow, uint32_t cidx, uint32_t hbase, uint32_t G, uint32_t nsplit)
{
    constexpr int S = ATTN_INMERGE_MAX_SPLITS, OPT = (GT * HD + 255) / 256; // outputs per thread (max)
    __shared__ uint32_t s_last;
    __shared__ __align__(16) float s_w[GT][S];
    __shared__ float s_L[GT];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t stride = HD + 4;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); // this thread's states have landed
    __syncthreads();
    if (tid == 0) {
        const uint32_t old = __hip_atomic_fetch_add(a.counters + cidx, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = old + 1u == nsplit ? 1u : 0u;
    }
    __syncthreads();
    if (!s_last) return;
    if (tid == 0) __hip_atomic_store(a.counters + cidx, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); // for the next launch
    // split values of this thread's outputs i = tid + 256 j
    float v[OPT][S];
#pragma unroll
    for (int j = 0; j < OPT; j++) {
        const uint32_t i = (uint32_t)tid + 256u * (uint32_t)j;
        const uint32_t g = i / HD, d = i % HD;
        const float *hp = prow + (size_t)(hbase + min(g, G - 1u)) * a.max_splits * stride + 4 + d;
#pragma unroll
        for (int sp = 0; sp < S; sp++) v[j][sp] = (g < G && (uint32_t)sp < nsplit) ? attn_load_agent(hp + (size_t)sp * stride) : 0.0f;
    }
    // weights per head (one wave per head; lane = split)
    for (uint32_t g = (uint32_t)wave; g < G; g += 4) {
        const float *hp = prow + (size_t)(hbase + g) * a.max_splits * stride;
        const bool in = (uint32_t)lane < nsplit;
        const float m = in ? attn_load_agent(hp + (size_t)lane * stride) : -3.402823466e38f;
        const float l = in ? attn_load_agent(hp + (size_t)lane * stride + 1) : 0.0f;
        const float M = wave_max(m);
        const float w = in ? attn_exp2(m - M) : 0.0f;
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
        float w[S];
#pragma unroll
        for (int sp = 0; sp < S; sp += 4) {
            const float4 w4 = *(const float4 *)&s_w[g][sp];
            w[sp] = w4.x;
            w[sp + 1] = w4.y;
            w[sp + 2] = w4.z;
            w[sp + 3] = w4.w;
        }
        float acc = 0.0f;
#pragma unroll
        for (int sp = 0; sp < S; sp++) {
            const float t = fmaf(w[sp], v[j][sp], acc);
            acc = (uint32_t)sp < nsplit ? t : acc;
        }
        a.out[(size_t)(hbase + g) * HD + d] = __fdiv_rn(acc, s_L[g]);
    }
}

// ---- tagged in-kernel merge (engine decode, one query row, at most
// ATTN_TAG_MAX_SPLITS splits): no arrival counter and no wait for store
// acknowledgements.  Every word of a split state is one 64-bit relaxed
// atomic holding the float's bits and a tag, the launch's sequence length,
// which differs between the steps of a generation (the engine clears the
// per-layer workspace before a generation starts, so no word of an earlier
// one carries a current tag).  A load that returns the tag returns the value
// stored with it (a single atomic object), so the merging workgroup polls
// every word it needs until it carries the tag, with no ordering between
// words and no fence.  In the language memory model this rests only on the
// coherence of each atomic object and on relaxed stores becoming visible in
// finite time.  Split g of a workgroup column merges its query head g (and
// g + nsplit, ... below G) after finishing its own split; at most n_heads
// workgroups wait, each only for workgroups that never wait, so the launch
// completes whenever the device holds n_heads + 1 of them at once.  A poll
// that reaches the spin limit writes NaN outputs and sets *err.  The sums
// follow the merge kernel's order (attn_merge_body), so the outputs are
// bit-identical to the two-launch step.
#define ATTN_TAG_SPIN_LIMIT (1u << 20)
RFP4_DEV void attn_store_tagged(unsigned long long *p, float v, uint32_t tag)
{
    __hip_atomic_store(p, ((unsigned long long)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
RFP4_DEV unsigned long long attn_load_tagged(const unsigned long long *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
RFP4_DEV bool attn_tag_ok(unsigned long long w, uint32_t tag) { return (uint32_t)(w >> 32) == tag; }
RFP4_DEV float attn_tag_val(unsigned long long w) { return __uint_as_float((uint32_t)w); }

// Merge of one query head: hp = its first state word, out = its HD outputs.
// Wave 0 first polls (m, l) of split `lane` until every split has published
// them (small polls, no traffic against the splits still streaming K/V), then
// thread (d = tid % HD, p = tid / HD) loads the acc words of splits p, p + P,
// ... (P = 256 / HD) and reloads any that do not carry the tag yet.
// Measured against polling every word from the start (Llama-3-8B, 29 splits):
// 10.4 against 10.8 us per launch.
template <int HD>
RFP4_DEV void attn_merge_tagged(const AttnArgs &a, const unsigned long long *hp, float *out, uint32_t nsplit, uint32_t tag)
{
    constexpr uint32_t P = 256 / HD, STRIDE = HD + 4, NB = ATTN_TAG_MAX_SPLITS / P;
    static_assert(ATTN_TAG_MAX_SPLITS <= ATTN_MERGE_BATCH && ATTN_TAG_MAX_SPLITS <= 64, "one batch, one split per lane");
    __shared__ __align__(16) float t_w[ATTN_TAG_MAX_SPLITS]; // split i at (i % P) * NB + i / P
    __shared__ float t_part[P][HD];
    __shared__ float t_L;
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid)); // no per-lane address of the merge is hoisted above the split's loop
    const int lane = tid & 63, wave = tid >> 6;
    const uint32_t d = (uint32_t)tid % HD, p = (uint32_t)tid / HD;
    __syncthreads(); // a previous head's merge in this workgroup has read t_w and t_part
    // (m, l) of every split first (wave 0, one split per lane), then the acc words
    const bool ml = wave == 0 && (uint32_t)lane < nsplit;
    unsigned long long mw = 0ull, lw = 0ull;
    bool timeout = false;
    if (wave == 0) {
        if (ml) {
            mw = attn_load_tagged(hp + (size_t)lane * STRIDE);
            lw = attn_load_tagged(hp + (size_t)lane * STRIDE + 1);
        }
        for (uint32_t spin = 0;; spin++) {
            const bool stale = ml && !(attn_tag_ok(mw, tag) && attn_tag_ok(lw, tag));
            if (!__any(stale)) break;
            if (spin >= ATTN_TAG_SPIN_LIMIT) {
                timeout = true;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
            if (ml && !attn_tag_ok(mw, tag)) mw = attn_load_tagged(hp + (size_t)lane * STRIDE);
            if (ml && !attn_tag_ok(lw, tag)) lw = attn_load_tagged(hp + (size_t)lane * STRIDE + 1);
        }
    }
    __syncthreads();
    unsigned long long v[NB];
#pragma unroll
    for (int j = 0; j < (int)NB; j++) {
        const uint32_t sp = p + P * (uint32_t)j;
        v[j] = sp < nsplit ? attn_load_tagged(hp + (size_t)sp * STRIDE + 4 + d) : 0ull;
    }
    for (uint32_t spin = 0;; spin++) {
        bool stale = false;
#pragma unroll
        for (int j = 0; j < (int)NB; j++) stale = stale || (p + P * (uint32_t)j < nsplit && !attn_tag_ok(v[j], tag));
        if (!stale) break;
        if (spin >= ATTN_TAG_SPIN_LIMIT) {
            timeout = true;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int j = 0; j < (int)NB; j++) {
            const uint32_t sp = p + P * (uint32_t)j;
            if (sp < nsplit && !attn_tag_ok(v[j], tag)) v[j] = attn_load_tagged(hp + (size_t)sp * STRIDE + 4 + d);
        }
    }
    if (wave == 0) {
        const float m = ml ? attn_tag_val(mw) : -3.402823466e38f;
        const float M = wave_max(m);
        const float w = ml ? attn_exp2(m - M) : 0.0f;
        if (ml) t_w[((uint32_t)lane % P) * NB + (uint32_t)lane / P] = w;
        const float L = wave_sum(ml ? fmaf(attn_tag_val(lw), w, 0.0f) : 0.0f);
        if (lane == 0) t_L = L;
    }
    const bool bad = __syncthreads_or(timeout);
    float w[NB];
#pragma unroll
    for (int j = 0; j < (int)NB; j += 4) {
        const float4 w4 = *(const float4 *)&t_w[p * NB + (uint32_t)j];
        w[j] = w4.x;
        w[j + 1] = w4.y;
        w[j + 2] = w4.z;
        w[j + 3] = w4.w;
    }
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < (int)NB; j++) {
        const float t = fmaf(w[j], attn_tag_val(v[j]), acc);
        acc = p + P * (uint32_t)j < nsplit ? t : acc;
    }
    if (p > 0) t_part[p][d] = acc;
    __syncthreads();
    if (p == 0) {
#pragma unroll
        for (uint32_t r = 1; r < P; r++) acc += t_part[r][d];
        out[d] = bad ? __builtin_nanf("") : __fdiv_rn(acc, t_L);
    }
    if (bad && tid == 0 && a.err) __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Reads and writes of values that the persistent decode kernel produces and
// consumes inside one launch (q, the new k and v, split states, outputs) go
// through agent scope (AG); the stand-alone kernels use plain accesses.
template <bool AG>
RFP4_DEV float attn_in(const float *p)
{
    return AG ? attn_load_agent(p) : *p;
}
template <bool AG>
RFP4_DEV void attn_out(float *p, float v)
{
    if (AG)
        attn_store_agent(p, v);
    else
        *p = v;
}

// The last split's merge in the merge kernel's summation order
// (attn_merge_body), for up to S splits in one round of loads: the
// persistent decode kernel merges in place and stays bit-identical to the
// two-launch step.  Output (g, d) sums splits p, p + P, p + 2P, ... (P =
// 256 / HD) per partial p with one FMA chain each, then the partials in p
// order, divided by L.
template <int HD, int GT, int S>
RFP4_DEV void attn_merge_last_ordered(const AttnArgs &a, const float *prow, uint32_t cidx, uint32_t hbase, uint32_t G,
                                      uint32_t nsplit)
{
    constexpr int P = 256 / HD, OPT = (GT * HD + 255) / 256, NJ = (S + P - 1) / P;
    static_assert(S <= 64, "one split per lane");
    __shared__ uint32_t s_last;
    __shared__ __align__(16) float s_w[GT][S];
    __shared__ float s_L[GT];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t stride = HD + 4;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); // this thread's states have landed
    __syncthreads();
    if (tid == 0) {
        const uint32_t old = __hip_atomic_fetch_add(a.counters + cidx, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = old + 1u == nsplit ? 1u : 0u;
    }
    __syncthreads();
    if (!s_last) return;
    if (tid == 0) __hip_atomic_store(a.counters + cidx, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); // for the next launch
    float v[OPT][S];
#pragma unroll
    for (int j = 0; j < OPT; j++) {
        const uint32_t i = (uint32_t)tid + 256u * (uint32_t)j;
        const uint32_t g = i / HD, d = i % HD;
        const float *hp = prow + (size_t)(hbase + min(g, G - 1u)) * a.max_splits * stride + 4 + d;
#pragma unroll
        for (int sp = 0; sp < S; sp++) v[j][sp] = (g < G && (uint32_t)sp < nsplit) ? attn_load_agent(hp + (size_t)sp * stride) : 0.0f;
    }
    for (uint32_t g = (uint32_t)wave; g < G; g += 4) {
        const float *hp = prow + (size_t)(hbase + g) * a.max_splits * stride;
        const bool in = (uint32_t)lane < nsplit;
        const float m = in ? attn_load_agent(hp + (size_t)lane * stride) : -3.402823466e38f;
        const float l = in ? attn_load_agent(hp + (size_t)lane * stride + 1) : 0.0f;
        const float M = wave_max(m);
        const float w = in ? attn_exp2(m - M) : 0.0f;
        if ((uint32_t)lane < (uint32_t)S) s_w[g][lane] = w;
        const float L = wave_sum(fmaf(l, w, 0.0f));
        if (lane == 0) s_L[g] = L;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < OPT; j++) {
        const uint32_t i = (uint32_t)tid + 256u * (uint32_t)j;
        const uint32_t g = i / HD, d = i % HD;
        if (g >= G) break;
        float out = 0.0f;
#pragma unroll
        for (int p = 0; p < P; p++) {
            float acc = 0.0f;
#pragma unroll
            for (int jj = 0; jj < NJ; jj++) {
                const int sp = p + P * jj;
                if (sp < S) {
                    const float t = fmaf(s_w[g][sp], v[j][sp], acc);
                    acc = (uint32_t)sp < nsplit ? t : acc;
                }
            }
            out = p == 0 ? acc : out + acc;
        }
        attn_store_agent(a.out + (size_t)(hbase + g) * HD + d, __fdiv_rn(out, s_L[g]));
    }
}

// One split of one KV head: the phases of the attention workgroup.  The
// stand-alone kernel runs load_q, issue and finish back to back; the
// persistent decode kernel issues the K/V stream (issue) before the grid
// barrier that publishes q, then loads q and finishes.  TAG: the split
// states go to the tagged workspace and are merged by the first splits of
// each workgroup column (kernels of their own: the merge's registers stay out
// of the other kernels' allocation).  QT: q and the current token's k and v
// come as tagged words from the q|k|v GEMV of the same launch (fused kernel,
// device/qkva.h): load_q_tagged after issue, in place of load_q.
template <int HD, typename KT, int GT, bool AG, bool TAG = false, bool QT = false>
struct AttnSplit {
    static constexpr int EPL = KvTraits<KT>::EPL;
    static constexpr int LPT = HD / EPL;          // lanes per token row
    static constexpr int TPS = 256 / LPT;         // tokens per workgroup step
    static constexpr int NSTEP = attn_steps_for(HD, (int)sizeof(KT), GT);
    static constexpr uint32_t CAPT = TPS * NSTEP;  // tokens of one sub-chunk (held in registers)
    static constexpr uint32_t HALF = HD / 2;
    static constexpr int QPT = (GT * (int)HALF + 255) / 256; // q rotation pairs per thread
    static_assert(LPT >= 4 && LPT <= 32, "row split");
    static_assert(256 % HALF == 0, "a thread's rotation pairs share one table column");
    static_assert(GT == 1 || GT == 2 || GT == 4 || GT == 8, "group");

    float qa[QPT], qb[QPT];
    uint4 kr[NSTEP], vr[NSTEP];
    float cs, sn;
    uint32_t kvh, split, row, G, seq, nsplit, t0, nt, nsub, pos;
    uint32_t hbase, cidx; // first query head of this workgroup, its merge-counter index
    bool fused, owner, writer;
    bool q_timeout = false; // QT: a poll of q|k|v hit its spin limit (NaN q, no K/V append)

    // Workgroup x index -> KV head and query-head slice: with head_split HS,
    // x = hg * n_kv_heads + kvh takes query heads hg*G .. hg*G + G - 1 of the
    // KV head's group (G = group / HS); the HS workgroups of one KV head have
    // indices n_kv_heads apart (the same XCD under round-robin dispatch), and
    // slice 0 writes the appended K/V row.
    RFP4_DEV void heads(const AttnArgs &a, uint32_t x)
    {
        const uint32_t hs = a.head_split > 1u ? a.head_split : 1u;
        const uint32_t gfull = a.n_heads / a.n_kv_heads;
        kvh = x % a.n_kv_heads;
        const uint32_t hg = x / a.n_kv_heads;
        G = gfull / hs;
        hbase = kvh * gfull + hg * G;
        cidx = x;
        writer = hg == 0u;
    }
    const KT *kc, *vc;
    float tkv[4]; // QT, owner split, tid < HD/2: k[tid], k[tid + HD/2], v[tid], v[tid + HD/2] of the current token

    // QT: this thread's q pairs (as load_q) and, in the split owning the
    // current position, the current token's k and v, from words tagged with
    // `tag` (the launch's sequence length).  After issue (owner known).
    // Every word is polled until it carries the tag; each word read with the
    // tag is the value stored with it (one 64-bit atomic object), so no fence
    // or counter is needed.  A poll past ATTN_TAG_SPIN_LIMIT spins sets *err
    // (the engine reports it), makes q and the current token's k, v NaN (so
    // the outputs are NaN) and keeps the split from appending to the cache.
    RFP4_DEV void load_q_tagged(const AttnArgs &a, uint32_t tag)
    {
        const int tid = threadIdx.x;
        const unsigned long long *qg = a.qkv_t + (size_t)hbase * HD;
        const unsigned long long *kn = a.qkv_t + (size_t)(a.n_heads + kvh) * HD;
        const unsigned long long *vn = a.qkv_t + (size_t)(a.n_heads + a.n_kv_heads + kvh) * HD;
        const bool kv = owner && (uint32_t)tid < HALF;
        unsigned long long wa[QPT], wb[QPT], wk[4];
#pragma unroll
        for (int m = 0; m < QPT; m++) {
            const uint32_t i = (uint32_t)tid + 256u * (uint32_t)m;
            const uint32_t g = i / HALF, j = i % HALF;
            const bool in = g < G;
            wa[m] = in ? attn_load_tagged(qg + g * HD + j) : 0ull;
            wb[m] = in ? attn_load_tagged(qg + g * HD + j + HALF) : 0ull;
        }
        if (kv) {
            wk[0] = attn_load_tagged(kn + tid);
            wk[1] = attn_load_tagged(kn + tid + HALF);
            wk[2] = attn_load_tagged(vn + tid);
            wk[3] = attn_load_tagged(vn + tid + HALF);
        }
        bool timeout = false;
        for (uint32_t spin = 0;; spin++) {
            bool stale = false;
#pragma unroll
            for (int m = 0; m < QPT; m++) {
                const bool in = (uint32_t)tid + 256u * (uint32_t)m < G * HALF;
                stale = stale || (in && !(attn_tag_ok(wa[m], tag) && attn_tag_ok(wb[m], tag)));
            }
            if (kv)
#pragma unroll
                for (int r = 0; r < 4; r++) stale = stale || !attn_tag_ok(wk[r], tag);
            if (!__syncthreads_or(stale)) break;
            if (spin >= ATTN_TAG_SPIN_LIMIT) {
                timeout = true;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (int m = 0; m < QPT; m++) {
                const uint32_t i = (uint32_t)tid + 256u * (uint32_t)m;
                const uint32_t g = i / HALF, j = i % HALF;
                if (g < G && !attn_tag_ok(wa[m], tag)) wa[m] = attn_load_tagged(qg + g * HD + j);
                if (g < G && !attn_tag_ok(wb[m], tag)) wb[m] = attn_load_tagged(qg + g * HD + j + HALF);
            }
            if (kv) {
                if (!attn_tag_ok(wk[0], tag)) wk[0] = attn_load_tagged(kn + tid);
                if (!attn_tag_ok(wk[1], tag)) wk[1] = attn_load_tagged(kn + tid + HALF);
                if (!attn_tag_ok(wk[2], tag)) wk[2] = attn_load_tagged(vn + tid);
                if (!attn_tag_ok(wk[3], tag)) wk[3] = attn_load_tagged(vn + tid + HALF);
            }
        }
        const float nan = __uint_as_float(0x7FC00000u);
#pragma unroll
        for (int m = 0; m < QPT; m++) {
            qa[m] = timeout ? nan : attn_tag_val(wa[m]);
            qb[m] = timeout ? nan : attn_tag_val(wb[m]);
        }
#pragma unroll
        for (int r = 0; r < 4; r++) tkv[r] = timeout ? nan : (kv ? attn_tag_val(wk[r]) : 0.0f);
        q_timeout = timeout;
        if (timeout && tid == 0 && a.err) __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // This thread's q pairs (j, j + HD/2) of pair index i = tid + 256 m.
    RFP4_DEV void load_q(const AttnArgs &a, uint32_t x, uint32_t row_)
    {
        const int tid = threadIdx.x;
        heads(a, x);
        row = row_;
        const float *qg = a.q + (size_t)row * a.q_rs + (size_t)hbase * HD;
#pragma unroll
        for (int m = 0; m < QPT; m++) {
            const uint32_t i = (uint32_t)tid + 256u * (uint32_t)m;
            const uint32_t g = i / HALF, j = i % HALF;
            const bool in = g < G;
            qa[m] = in ? attn_in<AG>(qg + g * HD + j) : 0.0f;
            qb[m] = in ? attn_in<AG>(qg + g * HD + j + HALF) : 0.0f;
        }
    }

    // Split geometry at sequence length seq_, the rope table column of the
    // position, and every K/V load of sub-chunk 0.  False: this split is
    // past the sequence (nothing to do).
    RFP4_DEV bool issue(const AttnArgs &a, uint32_t x, uint32_t split_, uint32_t row_, uint32_t seq_)
    {
        int tid = threadIdx.x;
        if (AG) asm volatile("" : "+v"(tid)); // the persistent kernel's layer loop: no hoisted addresses
        const int li = tid % LPT, slot = tid / LPT;
        heads(a, x);
        split = split_;
        row = row_;
        fused = a.cosv != nullptr;
        seq = min(seq_, a.chunk * a.max_splits); // never read past the planned splits
        nsplit = (seq + a.chunk - 1) / a.chunk;
        if (split >= nsplit) return false;
        t0 = split * a.chunk;
        nt = min(seq, t0 + a.chunk) - t0;
        nsub = (nt + CAPT - 1) / CAPT;
        pos = seq - 1;
        owner = fused && (pos >= t0) && (pos < t0 + nt);
        kc = (const KT *)a.kc + (size_t)kvh * a.hs;
        vc = (const KT *)a.vc + (size_t)kvh * a.hs;
        cs = 1.0f;
        sn = 0.0f;
        if (fused) {
            const uint32_t j = (uint32_t)tid % HALF;
            cs = a.cosv[(size_t)pos * HALF + j];
            sn = a.sinv[(size_t)pos * HALF + j];
        }
        // K and V rows of sub-chunk 0: token t0 + s*TPS + slot, lanes split
        // the row.  Slots past the split re-read its last row (in bounds,
        // finite; their scores are masked and their p is 0): no branch around
        // the loads, so the wait for the rope tables does not wait for them.
#pragma unroll
        for (int s_ = 0; s_ < NSTEP; s_++) {
            const uint32_t t_ = min((uint32_t)s_ * TPS + (uint32_t)slot, nt - 1u);
            kr[s_] = load_nt16(kc + (size_t)(t0 + t_) * a.ts + (size_t)li * EPL);
        }
#pragma unroll
        for (int s_ = 0; s_ < NSTEP; s_++) {
            const uint32_t t_ = min((uint32_t)s_ * TPS + (uint32_t)slot, nt - 1u);
            vr[s_] = load_nt16(vc + (size_t)(t0 + t_) * a.ts + (size_t)li * EPL);
        }
        return true;
    }

    RFP4_DEV void finish(const AttnArgs &a)
    {
        __shared__ __align__(16) float qs[GT][HD];
        __shared__ __align__(16) float vred[4][GT][HD];
        __shared__ float s_mx[2][4][GT], s_lred[4][GT], s_mfin[GT];
        __shared__ KT knew[HD], vnew[HD];
        const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
        const int li = tid % LPT, slot = tid / LPT;
        float *orow = a.out + (size_t)row * a.out_rs;
        float *prow = a.part + (size_t)row * a.n_heads * a.max_splits * (HD + 4);

        // ---- q (rotated if fused) into LDS; the owner split appends k, v
#pragma unroll
        for (int m = 0; m < QPT; m++) {
            const uint32_t i = (uint32_t)tid + 256u * (uint32_t)m;
            if (i >= GT * HALF) break;
            const uint32_t g = i / HALF, j = i % HALF;
            float r0 = qa[m], r1 = qb[m];
            if (fused) {
                r0 = __fsub_rn(__fmul_rn(qa[m], cs), __fmul_rn(qb[m], sn));
                r1 = __fadd_rn(__fmul_rn(qb[m], cs), __fmul_rn(qa[m], sn));
            }
            qs[g][j] = r0;
            qs[g][j + HALF] = r1;
        }
        if (owner && (uint32_t)tid < HALF) {
            // the current token's k and v, loaded by the owner split only (after
            // its K/V stream, so no other split waits on them)
            float kna, knb, vna, vnb;
            if (QT) {
                kna = tkv[0];
                knb = tkv[1];
                vna = tkv[2];
                vnb = tkv[3];
            } else {
                const float *kn = a.k_new + (size_t)kvh * HD, *vn = a.v_new + (size_t)kvh * HD;
                kna = attn_in<AG>(kn + tid);
                knb = attn_in<AG>(kn + tid + HALF);
                vna = attn_in<AG>(vn + tid);
                vnb = attn_in<AG>(vn + tid + HALF);
            }
            KT *kdst = (KT *)a.kc + (size_t)kvh * a.hs + (size_t)pos * a.ts;
            KT *vdst = (KT *)a.vc + (size_t)kvh * a.hs + (size_t)pos * a.ts;
            const KT r0 = KvTraits<KT>::from_f32(__fsub_rn(__fmul_rn(kna, cs), __fmul_rn(knb, sn)));
            const KT r1 = KvTraits<KT>::from_f32(__fadd_rn(__fmul_rn(knb, cs), __fmul_rn(kna, sn)));
            const KT w0 = KvTraits<KT>::from_f32(vna), w1 = KvTraits<KT>::from_f32(vnb);
            knew[tid] = r0;
            knew[tid + HALF] = r1;
            vnew[tid] = w0;
            vnew[tid + HALF] = w1;
            if (writer && !q_timeout) {
                kdst[tid] = r0;
                kdst[tid + HALF] = r1;
                vdst[tid] = w0;
                vdst[tid + HALF] = w1;
            }
        }
        __syncthreads();

        float qv[GT][EPL];
#pragma unroll
        for (int g = 0; g < GT; g++)
#pragma unroll
            for (int e = 0; e < EPL; e += 4) {
                const float4 v4 = *(const float4 *)&qs[g][li * EPL + e];
                qv[g][e] = v4.x;
                qv[g][e + 1] = v4.y;
                qv[g][e + 2] = v4.z;
                qv[g][e + 3] = v4.w;
            }
        const float scale = __fmul_rn(1.4426950408889634f, __fdiv_rn(1.0f, __fsqrt_rn((float)HD))); // log2(e) / sqrt(HD)
        float acc[GT][EPL], lsum[GT], mrun[GT];
#pragma unroll
        for (int g = 0; g < GT; g++) {
            lsum[g] = 0.0f;
            mrun[g] = -3.402823466e38f;
#pragma unroll
            for (int e = 0; e < EPL; e++) acc[g][e] = 0.0f;
        }

#define RFP4_ATTN_LOAD(R, BASE, C)                                                              \
    do {                                                                                        \
        _Pragma("unroll") for (int s_ = 0; s_ < NSTEP; s_++) {                         \
            const uint32_t t_ = min((C) * CAPT + (uint32_t)s_ * TPS + (uint32_t)slot, nt - 1u); \
            R[s_] = load_nt16((BASE) + (size_t)(t0 + t_) * a.ts + (size_t)li * EPL);           \
        }                                                                                       \
    } while (0)
        for (uint32_t c = 0; c < nsub; c++) {
            const uint32_t tb = c * CAPT, ntc = min(CAPT, nt - tb);
            if (owner && pos - t0 >= tb && pos - t0 < tb + ntc) {
                // the thread holding position `pos` takes the freshly rotated row
                const uint32_t tl = pos - t0 - tb;
                if ((uint32_t)slot == tl % TPS) {
                    const uint32_t s = tl / TPS;
                    const uint4 kk = KvTraits<KT>::pack(knew + li * EPL), vv = KvTraits<KT>::pack(vnew + li * EPL);
#pragma unroll
                    for (int st = 0; st < NSTEP; st++)
                        if ((uint32_t)st == s) {
                            kr[st] = kk;
                            vr[st] = vv;
                        }
                }
            }

            // ---- scores of this sub-chunk (every lane of a row gets its row's
            //      score), this wave's max per head, then the next sub-chunk's K loads
            float sc[NSTEP][GT], mloc[GT];
#pragma unroll
            for (int g = 0; g < GT; g++) mloc[g] = -3.402823466e38f;
#pragma unroll
            for (int s = 0; s < NSTEP; s++) {
                const bool valid = (uint32_t)s * TPS + (uint32_t)slot < ntc;
                float kf[EPL];
                KvTraits<KT>::widen(kr[s], kf);
#pragma unroll
                for (int g = 0; g < GT; g++) {
                    float d = 0.0f;
#pragma unroll
                    for (int e = 0; e < EPL; e++) d = fmaf(qv[g][e], kf[e], d);
                    d = group_sum<LPT>(d) * scale;
                    sc[s][g] = valid ? d : -3.402823466e38f;
                    mloc[g] = fmaxf(mloc[g], sc[s][g]);
                }
            }
            if (c + 1 < nsub) RFP4_ATTN_LOAD(kr, kc, c + 1);
#pragma unroll
            for (int g = 0; g < GT; g++) mloc[g] = slots_max<LPT>(mloc[g]);
            if (lane == 0) {
#pragma unroll
                for (int g = 0; g < GT; g++) s_mx[c & 1u][wave][g] = mloc[g];
            }
            __syncthreads(); // s_mx is double-buffered: the next sub-chunk's writes wait for this barrier's successor

            // ---- online softmax: m' = max(m, max_t s_t), acc and l scaled by
            //      2^(m - m'), then p_t = 2^(s_t - m'), l += p_t, acc += p_t v_t (base 2)
#pragma unroll
            for (int g = 0; g < GT; g++) {
                const float mx = fmaxf(fmaxf(s_mx[c & 1u][0][g], s_mx[c & 1u][1][g]),
                                       fmaxf(s_mx[c & 1u][2][g], s_mx[c & 1u][3][g]));
                const float mnew = fmaxf(mrun[g], mx);
                const float alpha = attn_exp2(mrun[g] - mnew);
                mrun[g] = mnew;
                lsum[g] *= alpha;
#pragma unroll
                for (int e = 0; e < EPL; e++) acc[g][e] *= alpha;
            }
#pragma unroll
            for (int s = 0; s < NSTEP; s++) {
                const bool valid = (uint32_t)s * TPS + (uint32_t)slot < ntc;
                float vf[EPL];
                KvTraits<KT>::widen(vr[s], vf);
#pragma unroll
                for (int g = 0; g < GT; g++) {
                    const float p = valid ? attn_exp2(sc[s][g] - mrun[g]) : 0.0f;
                    lsum[g] += p;
#pragma unroll
                    for (int e = 0; e < EPL; e++) acc[g][e] = fmaf(p, vf[e], acc[g][e]);
                }
            }
            if (c + 1 < nsub) RFP4_ATTN_LOAD(vr, vc, c + 1);
        }
#undef RFP4_ATTN_LOAD

        // ---- fold the token slots of each wave, then the four waves through LDS
#pragma unroll
        for (int g = 0; g < GT; g++) {
            lsum[g] = slots_sum<LPT>(lsum[g]);
#pragma unroll
            for (int e = 0; e < EPL; e++) acc[g][e] = slots_sum<LPT>(acc[g][e]);
        }
        if (lane < LPT) {
#pragma unroll
            for (int g = 0; g < GT; g++)
#pragma unroll
                for (int e = 0; e < EPL; e += 4)
                    *(float4 *)&vred[wave][g][li * EPL + e] = make_float4(acc[g][e], acc[g][e + 1], acc[g][e + 2], acc[g][e + 3]);
        }
        if (lane == 0) {
#pragma unroll
            for (int g = 0; g < GT; g++) s_lred[wave][g] = lsum[g];
        }
        if (tid == 0) {
#pragma unroll
            for (int g = 0; g < GT; g++) s_mfin[g] = mrun[g];
        }
        __syncthreads();

        if (nsplit == 1) {
            // one split holds the whole sequence: normalise and write the heads' outputs
            for (uint32_t i = tid; i < G * HD; i += blockDim.x) {
                const uint32_t g = i / HD, d = i % HD;
                const float v = vred[0][g][d] + vred[1][g][d] + vred[2][g][d] + vred[3][g][d];
                const float l = (s_lred[0][g] + s_lred[1][g]) + (s_lred[2][g] + s_lred[3][g]);
                attn_out<AG>(orow + (size_t)(hbase + g) * HD + d, __fdiv_rn(v, l));
            }
            return;
        }

        // ---- write this split's partial state: [m, l, -, -, acc[HD]] per (head, split);
        // the merge kernel launched next on the same stream combines them, or
        // (counters given) the last split of this KV head to arrive does, or
        // (tagged workspace given) the first splits of the column do
        const uint32_t stride = HD + 4;
        if (TAG) {
            const uint32_t tag = seq;
            for (uint32_t i = tid; i < G * HD; i += blockDim.x) {
                const uint32_t g = i / HD, d = i % HD;
                const float v = vred[0][g][d] + vred[1][g][d] + vred[2][g][d] + vred[3][g][d];
                const float l = (s_lred[0][g] + s_lred[1][g]) + (s_lred[2][g] + s_lred[3][g]);
                unsigned long long *tp = a.tagged + ((size_t)(hbase + g) * a.tag_splits + split) * stride;
                attn_store_tagged(tp + 4 + d, v, tag);
                if (d == 0) {
                    attn_store_tagged(tp, s_mfin[g], tag);
                    attn_store_tagged(tp + 1, l, tag);
                }
            }
            for (uint32_t g = split; g < G; g += nsplit)
                attn_merge_tagged<HD>(a, a.tagged + (size_t)(hbase + g) * a.tag_splits * stride, orow + (size_t)(hbase + g) * HD,
                                      nsplit, tag);
            return;
        }
        const bool inmerge = a.counters != nullptr;
        for (uint32_t i = tid; i < G * HD; i += blockDim.x) {
            uint32_t g = i / HD, d = i % HD;
            float v = vred[0][g][d] + vred[1][g][d] + vred[2][g][d] + vred[3][g][d];
            size_t base = ((size_t)(hbase + g) * a.max_splits + split) * stride;
            const float l = (s_lred[0][g] + s_lred[1][g]) + (s_lred[2][g] + s_lred[3][g]);
            if (inmerge || AG) {
                attn_store_agent(prow + base + 4 + d, v);
                if (d == 0) {
                    attn_store_agent(prow + base, s_mfin[g]);
                    attn_store_agent(prow + base + 1, l);
                }
            } else {
                prow[base + 4 + d] = v;
                if (d == 0) {
                    prow[base] = s_mfin[g];
                    prow[base + 1] = l;
                }
            }
        }
        if (!inmerge) return;
        if (AG)
            attn_merge_last_ordered<HD, GT, ATTN_PERSIST_MAX_SPLITS>(a, prow, cidx, hbase, G, nsplit);
        else
            attn_merge_last<HD, GT>(a, prow, cidx, hbase, G, nsplit);
    }
};

template <int HD, typename KT, int GT, bool TAG = false>
RFP4_DEV void attn_body(const AttnArgs &a)
{
    AttnSplit<HD, KT, GT, false, TAG> u;
    const uint32_t x = blockIdx.x, split = blockIdx.y, row = blockIdx.z; // x: KV head and query-head slice
    // loads that need no position first (q), then the position, the rope
    // tables and the K/V stream, so the rotation of q overlaps the stream
    u.load_q(a, x, row);
    const uint32_t seq = (a.pos_ptr ? (uint32_t)(*a.pos_ptr + 1) : a.seq) + row;
    if (!u.issue(a, x, split, row, seq)) return;
    u.finish(a);
}

// Merge kernel body: grid (n_heads), launched after attn_body on the same
// stream (the kernel boundary orders the partial states before these reads).
// Computes the split count exactly as attn_body did; one split means
// attn_body already wrote the output.  For query head h:
//   M = max m_i, w_i = 2^(m_i - M), L = sum l_i w_i, out = sum w_i acc_i / L
// (m in the base-2 units of attn_body's scores).
// Thread tid owns output d = tid % HD and the splits p, p + P, p + 2P, ...
// (p = tid / HD, P = 256 / HD) of each batch of ATTN_MERGE_BATCH splits.
// Every thread issues the value loads of the first batch at once, before the
// split count is known (indices clamped inside the workspace; values past the
// count are discarded by select), while wave 0 loads (m_i, l_i), one split
// per lane, and turns them into M, L and the batch's weights, stored in LDS
// partition-major (split p + P j at p * NB + j) so that a thread reads its NB
// weights as float4s; the rest is FMAs and one LDS combine of the P partial
// sums.  Up to ATTN_MERGE_BATCH splits this is one round trip of loads.
template <int HD>
RFP4_DEV void attn_merge_body(const AttnArgs &a)
{
    constexpr uint32_t P = 256 / HD, STRIDE = HD + 4, NB = ATTN_MERGE_BATCH / P;
    __shared__ __align__(16) float s_w[ATTN_MERGE_BATCH]; // batch split i at (i % P) * NB + i / P
    __shared__ float s_part[P][HD];
    __shared__ float s_L, s_M;
    const uint32_t row = blockIdx.z;
    const uint32_t h = blockIdx.x; // the partial state of head h sits at (h * max_splits + split) * STRIDE
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t d = (uint32_t)tid % HD, p = (uint32_t)tid / HD;
    const float *hp = a.part + (size_t)row * a.n_heads * a.max_splits * STRIDE + (size_t)h * a.max_splits * STRIDE;
    const uint32_t last = a.max_splits - 1u;
    float v[NB];
#pragma unroll
    for (int j = 0; j < (int)NB; j++) v[j] = hp[(size_t)min(p + P * (uint32_t)j, last) * STRIDE + 4 + d];
    float m0 = 0.0f, l0 = 0.0f;
    if (wave == 0) {
        const uint32_t sp = min((uint32_t)lane, last);
        m0 = hp[(size_t)sp * STRIDE];
        l0 = hp[(size_t)sp * STRIDE + 1];
    }
    uint32_t seq = (a.pos_ptr ? (uint32_t)(*a.pos_ptr + 1) : a.seq) + row;
    seq = min(seq, a.chunk * a.max_splits);
    const uint32_t nsplit = (seq + a.chunk - 1) / a.chunk;
    if (nsplit <= 1) return;
    if (wave == 0) {
        float M = (uint32_t)lane < nsplit ? m0 : -3.402823466e38f;
        for (uint32_t i = (uint32_t)lane + 64u; i < nsplit; i += 64u) M = fmaxf(M, hp[(size_t)i * STRIDE]);
        M = wave_max(M);
        float L = 0.0f;
        for (uint32_t i = (uint32_t)lane; i < nsplit; i += 64u) {
            const float mi = i == (uint32_t)lane ? m0 : hp[(size_t)i * STRIDE];
            const float li = i == (uint32_t)lane ? l0 : hp[(size_t)i * STRIDE + 1];
            const float w = attn_exp2(mi - M);
            if (i < ATTN_MERGE_BATCH) s_w[(i % P) * NB + i / P] = w;
            L = fmaf(li, w, L);
        }
        L = wave_sum(L);
        if (lane == 0) {
            s_L = L;
            s_M = M;
        }
    }
    __syncthreads();
    float acc = 0.0f;
    for (uint32_t b = 0; b < nsplit; b += ATTN_MERGE_BATCH) {
        if (b > 0) {
#pragma unroll
            for (int j = 0; j < (int)NB; j++) v[j] = hp[(size_t)min(b + p + P * (uint32_t)j, last) * STRIDE + 4 + d];
            __syncthreads(); // the previous batch's weights are read
            if (wave == 0 && b + (uint32_t)lane < nsplit)
                s_w[((uint32_t)lane % P) * NB + (uint32_t)lane / P] = attn_exp2(hp[(size_t)(b + lane) * STRIDE] - s_M);
            __syncthreads();
        }
        float w[NB];
#pragma unroll
        for (int j = 0; j < (int)NB; j += 4) {
            const float4 w4 = *(const float4 *)&s_w[p * NB + (uint32_t)j];
            w[j] = w4.x;
            w[j + 1] = w4.y;
            w[j + 2] = w4.z;
            w[j + 3] = w4.w;
        }
#pragma unroll
        for (int j = 0; j < (int)NB; j++) {
            const float t = fmaf(w[j], v[j], acc); // stale workspace values are never kept
            acc = b + p + P * (uint32_t)j < nsplit ? t : acc;
        }
    }
    if (p > 0) s_part[p][d] = acc;
    __syncthreads();
    if (p != 0) return;
#pragma unroll
    for (uint32_t r = 1; r < P; r++) acc += s_part[r][d];
    a.out[(size_t)row * a.out_rs + (size_t)h * HD + d] = __fdiv_rn(acc, s_L);
}
