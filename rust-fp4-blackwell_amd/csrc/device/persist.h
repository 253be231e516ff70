// Persistent decode: every layer of one step in one launch (gfx950).
//
// The step's layers are five dependent stages each (q|k|v GEMV with the
// attention RMSNorm, attention with RoPE + KV append and its split merge, o
// GEMV + residual, gate|up GEMV with the FFN RMSNorm and SwiGLU, down GEMV +
// residual; llama_run/src/main.rs:492-530).  Launched as five kernels per
// layer, each stage pays a kernel boundary and then the first-load latency of
// its weights.  Here one cooperative launch keeps one workgroup per CU for
// the whole step; a grid barrier separates the stages, and before entering a
// barrier every workgroup issues the first weight loads of its share of the
// next stage (or, before attention, its whole K/V stream), which depend on
// nothing the barrier publishes.  So the barrier's latency overlaps the next
// stage's ramp.
//
// Data produced and consumed inside the launch (q|k|v, split states,
// attention rows, the residual stream, SwiGLU rows) moves through agent
// scope: stores are write-through past the XCD's L2 and loads miss it (the
// protocol of the attention merge, device/attn.h).  Every wave waits for its
// own stores (vmcnt(0)) before the barrier; wave 0 of each workgroup then
// publishes the workgroup's generation and polls all of them.  Weights, norms,
// rope tables and K/V rows below the position were written before the launch.
//
// Arithmetic is the stand-alone kernels' own: each GEMV row is gemv_body's
// (same slices, chunk order, scale application and DPP reduction, and the
// RMSNorm of stage_x_regs over 256 threads), attention is AttnSplit, and the
// split merge follows the merge kernel's summation order, so a step is
// bit-identical to the two-launch-per-stage step at contexts of more than 8
// splits (fewer splits merge in the attention kernel in another order there).
#pragma once
#include "common.h"
#include "gemv.h"
#include "attn.h"

RFP4_DEV void ag_store(float *p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
RFP4_DEV float ag_load(const float *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
RFP4_DEV float4 ag_load4(const float *p)
{
    const uint64_t a = __hip_atomic_load((const uint64_t *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t b = __hip_atomic_load((const uint64_t *)p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_float4(__uint_as_float((uint32_t)a), __uint_as_float((uint32_t)(a >> 32)), __uint_as_float((uint32_t)b),
                       __uint_as_float((uint32_t)(b >> 32)));
}
// An opaque copy: per-layer address arithmetic is recomputed from it instead
// of being hoisted out of the layer loop (where it would hold registers for
// the whole launch).
RFP4_DEV uint32_t opaque(uint32_t v)
{
    asm volatile("" : "+v"(v));
    return v;
}
RFP4_DEV void vm_drain() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Grid barrier of generation gen.  The caller's waves have drained their
// stores (vm_drain) and may have loads in flight: __syncthreads waits for LDS
// only, and only wave 0 (which polls) waits for its own loads.  False: a
// spin limit was hit somewhere (the error flag is set; the caller leaves).
RFP4_DEV bool grid_sync(const PersistArgs &a, uint32_t gen)
{
    __shared__ uint32_t s_ok;
    __syncthreads();
    if (threadIdx.x < 64) {
        const uint32_t lane = threadIdx.x;
        if (lane == 0) __hip_atomic_store(a.flags + blockIdx.x, gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        bool ok = true;
        for (uint32_t it = 0;; it++) {
            bool mine = true;
            for (uint32_t i = lane; i < gridDim.x; i += 64u)
                mine = mine && (int32_t)(__hip_atomic_load(a.flags + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - gen) >= 0;
            if (__all(mine)) break;
            const uint32_t e = __hip_atomic_load(a.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (__any(e != 0u) || it >= a.spin_limit) {
                ok = false;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        if (lane == 0) {
            if (!ok) __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_ok = ok ? 1u : 0u;
        }
    }
    __syncthreads();
    return s_ok != 0u;
}

// ---- GEMV stages.  A wave owns RW consecutive logical rows, walked in parts
// of RP rows (NP physical: SwiGLU pairs gate row r with up row r + pair_off),
// two parts in flight.  Weights E8M0.
template <int NS, int NP>
struct WParts {
    uint4 q[NS][NP];
    uint32_t sb[NS][NP];
};

// Weight pointers come from the layer table in device memory, so the
// compiler cannot infer their address space: cast to global so the loads are
// global_load (a flat load would also count against lgkmcnt, which every
// __syncthreads waits for).
typedef __attribute__((address_space(1))) u32x4 g_u32x4;
typedef __attribute__((address_space(1))) uint8_t g_u8;
RFP4_DEV uint4 ldg_nt16(const uint8_t *p)
{
    const u32x4 v = __builtin_nontemporal_load((const g_u32x4 *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
RFP4_DEV uint32_t ldg_nt_u8(const uint8_t *p) { return __builtin_nontemporal_load((const g_u8 *)p); }

template <int NS, int RP, bool PAIR>
RFP4_DEV void w_issue(WParts<NS, PAIR ? 2 * RP : RP> &w, const uint8_t *codes, const uint8_t *scales, uint32_t n,
                      uint32_t k, uint32_t r0, uint32_t rend, uint32_t pair_off)
{
    const uint32_t lane = opaque(threadIdx.x & 63u);
    r0 = opaque(r0);
    const uint32_t nchunk = k >> 5, clast = nchunk - 1u;
    const size_t rowbytes = (size_t)(k >> 1);
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const uint32_t cl = min(lane + 64u * (uint32_t)s, clast);
#pragma unroll
        for (int i = 0; i < RP; i++) {
            const uint32_t lr = min(min(r0 + (uint32_t)i, rend - 1u), n - 1u); // clamp: loads stay in bounds
            w.q[s][i] = ldg_nt16(codes + (size_t)lr * rowbytes + (size_t)cl * 16u);
            w.sb[s][i] = ldg_nt_u8(scales + (size_t)lr * nchunk + cl);
            if (PAIR) {
                w.q[s][RP + i] = ldg_nt16(codes + (size_t)(lr + pair_off) * rowbytes + (size_t)cl * 16u);
                w.sb[s][RP + i] = ldg_nt_u8(scales + (size_t)(lr + pair_off) * nchunk + cl);
            }
        }
    }
}

// acc[p] = row p of the part against x in LDS, reduced over the wave
// (gemv_body's order: slices in order, one fmaf per 32-value chunk).
template <int NS, int NP>
RFP4_DEV void w_dot(const WParts<NS, NP> &w, const float *xs, uint32_t k, float *acc)
{
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t nchunk = k >> 5, clast = nchunk - 1u;
#pragma unroll
    for (int p = 0; p < NP; p++) acc[p] = 0.0f;
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const uint32_t c = lane + 64u * (uint32_t)s;
        const float live = c < nchunk ? 1.0f : 0.0f;
        float4 xv[8];
        const float4 *xp = (const float4 *)(xs + (size_t)min(c, clast) * GEMV_XS_CHUNK);
#pragma unroll
        for (int j = 0; j < 8; j++) xv[j] = xp[j];
#pragma unroll
        for (int p = 0; p < NP; p++) acc[p] = fmaf(live * e8m0_to_f32(w.sb[s][p]), dot_chunk32(w.q[s][p], xv), acc[p]);
    }
#pragma unroll
    for (int p = 0; p < NP; p++) acc[p] = wave_sum(acc[p]);
}

// x (K floats produced in this launch) into LDS in the GEMV layout, with the
// fused RMSNorm when norm_w is given: stage_x_regs over 256 threads.
template <int NS>
RFP4_DEV void stage_x_agent(float *xs, const float *x, uint32_t k, const uint16_t *norm_w, float eps)
{
    constexpr int XV = (512 * NS + 255) / 256;
    float4 xr[XV];
    uint2 wr[XV];
    const uint32_t tid = opaque(threadIdx.x), k4 = k >> 2;
#pragma unroll
    for (int v = 0; v < XV; v++) {
        const uint32_t i4 = tid + 256u * (uint32_t)v;
        const bool in = i4 < k4;
        xr[v] = in ? ag_load4(x + 4u * i4) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        wr[v] = (in && norm_w) ? ((const uint2 *)norm_w)[i4] : make_uint2(0, 0);
    }
    stage_x_regs<XV, 4>(xs, xr, wr, k, norm_w != nullptr, eps);
}

// Part PART of a GEMV stage: its weights are in `cur` (part PART + 1's in
// `nxt`, in flight); part PART + 2 is issued into `cur` once it is consumed.
template <int EPI, int NS, int RW, int RP, int PART>
RFP4_DEV void gemv_parts(WParts<NS, EPI == RFP4_EPI_SWIGLU ? 2 * RP : RP> &cur,
                         WParts<NS, EPI == RFP4_EPI_SWIGLU ? 2 * RP : RP> &nxt, const uint8_t *codes,
                         const uint8_t *scales, uint32_t n, uint32_t k, uint32_t pair_off, const float *yres, float *y,
                         const float *xs, uint32_t r0, uint32_t rend)
{
    constexpr bool PAIR = EPI == RFP4_EPI_SWIGLU;
    constexpr int NP = PAIR ? 2 * RP : RP, NPART = (RW + RP - 1) / RP;
    if constexpr (PART < NPART) {
        float acc[NP];
        w_dot<NS, NP>(cur, xs, k, acc);
        if (PART + 2 < NPART) w_issue<NS, RP, PAIR>(cur, codes, scales, n, k, r0 + (uint32_t)(PART + 2) * RP, rend, pair_off);
        if ((threadIdx.x & 63u) == 0) {
#pragma unroll
            for (int i = 0; i < RP; i++) {
                const uint32_t lr = r0 + (uint32_t)(PART * RP + i);
                if (PART * RP + i >= RW || lr >= rend) continue;
                if (EPI == RFP4_EPI_STORE)
                    ag_store(y + lr, acc[i]);
                else if (EPI == RFP4_EPI_RESIDUAL)
                    ag_store(y + lr, __fadd_rn(yres[PART * RP + i], acc[i]));
                else
                    ag_store(y + lr, __fmul_rn(silu_ref(acc[i]), acc[RP + i]));
            }
        }
        gemv_parts<EPI, NS, RW, RP, PART + 1>(nxt, cur, codes, scales, n, k, pair_off, yres, y, xs, r0, rend);
    }
}

// One GEMV stage for this wave: rows [r0, r0 + RW) of n (parts of RP), part
// 0 already issued into w0 by the caller (before the barrier).  EPI:
// STORE y[r] = acc; RESIDUAL y[r] = y[r] + acc (y read at agent scope first);
// SWIGLU y[r] = silu(gate) * up.  Stores at agent scope.
template <int EPI, int NS, int RW, int RP>
RFP4_DEV void gemv_stage(WParts<NS, EPI == RFP4_EPI_SWIGLU ? 2 * RP : RP> &w0, const uint8_t *codes, const uint8_t *scales,
                         uint32_t n, uint32_t k, uint32_t pair_off, const float *x, const uint16_t *norm_w, float eps,
                         float *y, float *xs)
{
    constexpr bool PAIR = EPI == RFP4_EPI_SWIGLU;
    constexpr int NP = PAIR ? 2 * RP : RP, NPART = (RW + RP - 1) / RP;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t r0 = opaque((blockIdx.x * 4u + wave) * (uint32_t)RW), rend = min(r0 + (uint32_t)RW, n);
    // residual rows first (agent loads, before anything waits)
    float yres[EPI == RFP4_EPI_RESIDUAL ? RW : 1];
    if (EPI == RFP4_EPI_RESIDUAL) {
#pragma unroll
        for (int i = 0; i < RW; i++) yres[i] = r0 + (uint32_t)i < rend ? ag_load(y + r0 + i) : 0.0f;
    } else {
        yres[0] = 0.0f;
    }
    WParts<NS, NP> w1;
    if (NPART > 1) w_issue<NS, RP, PAIR>(w1, codes, scales, n, k, r0 + RP, rend, pair_off);
    stage_x_agent<NS>(xs, x, k, norm_w, eps);
    gemv_parts<EPI, NS, RW, RP, 0>(w0, w1, codes, scales, n, k, pair_off, yres, y, xs, r0, rend);
}

// The model shape the persistent kernel is compiled for: head dim, query-head
// group, K slices of the dim / q / ffn contractions, and per stage the rows
// of one wave (RW) and of one part (RP) with one workgroup per CU.
struct PersistShape8B {
    static constexpr int HD = 128, GT = 4, NS_DIM = 2, NS_Q = 2, NS_FFN = 7;
    static constexpr int RW_QKV = 6, RP_QKV = 3, RW_O = 4, RP_O = 2, RW_GU = 14, RP_GU = 2, RW_D = 4, RP_D = 2;
};

template <class C>
RFP4_DEV void decode_layers_body(const PersistArgs &a)
{
    extern __shared__ float xs[]; // GEMV x staging (the widest K)
    const uint32_t qd = a.n_heads * a.head_dim, kvd = a.n_kv_heads * a.head_dim, nqkv = qd + 2 * kvd;
    const uint32_t seq = (uint32_t)(a.state->pos + 1); // written by the previous launch
    const uint32_t nsplit = min((seq + a.chunk - 1u) / a.chunk, a.max_splits);
    const uint32_t units = a.n_kv_heads * nsplit, unit = blockIdx.x;
    const bool has_attn = unit < units;
    uint32_t gen = a.gen0;

    AttnArgs aa{};
    aa.q = a.qkv;
    aa.out = a.att;
    aa.part = a.part;
    aa.pos_ptr = nullptr;
    aa.cosv = a.cosv;
    aa.sinv = a.sinv;
    aa.k_new = a.qkv + qd;
    aa.v_new = a.qkv + qd + kvd;
    aa.ts = a.head_dim;
    aa.hs = (uint64_t)a.max_seq_alloc * a.head_dim;
    aa.n_heads = a.n_heads;
    aa.n_kv_heads = a.n_kv_heads;
    aa.head_dim = a.head_dim;
    aa.seq = seq;
    aa.chunk = a.chunk;
    aa.max_splits = a.max_splits;
    aa.counters = nsplit > 1 ? a.counters : nullptr;

    WParts<C::NS_DIM, C::RP_QKV> wq;
    {
        const PersistLayer &L0 = a.layers[0];
        w_issue<C::NS_DIM, C::RP_QKV, false>(wq, L0.qkv_c, L0.qkv_s, nqkv, a.dim, (blockIdx.x * 4u + (threadIdx.x >> 6)) * C::RW_QKV,
                                             min((blockIdx.x * 4u + (threadIdx.x >> 6)) * C::RW_QKV + C::RW_QKV, nqkv), 0);
    }
    for (uint32_t l = 0; l < a.n_layers; l++) {
        const PersistLayer &L = a.layers[l];
        const uint32_t wave = threadIdx.x >> 6;
        // ---- q|k|v = W_qkv . rmsnorm(x)
        gemv_stage<RFP4_EPI_STORE, C::NS_DIM, C::RW_QKV, C::RP_QKV>(wq, L.qkv_c, L.qkv_s, nqkv, a.dim, 0, a.x,
                                                                     a.norm_attn + (size_t)l * a.dim, a.eps, a.qkv, xs);
        vm_drain();
        AttnSplit<C::HD, uint16_t, C::GT, true> at;
        aa.kc = (const uint16_t *)a.kcache + (size_t)l * a.kv_layer_elems;
        aa.vc = (const uint16_t *)a.vcache + (size_t)l * a.kv_layer_elems;
        if (has_attn) at.issue(aa, unit / nsplit, unit % nsplit, 0, seq); // the K/V stream, before the barrier
        if (!grid_sync(a, ++gen)) return;
        // ---- attention (RoPE, KV append, splits merged by the last to finish)
        if (has_attn) {
            at.load_q(aa, unit / nsplit, 0);
            at.finish(aa);
        }
        vm_drain();
        WParts<C::NS_Q, C::RP_O> wo;
        {
            const uint32_t r0 = (blockIdx.x * 4u + wave) * C::RW_O;
            w_issue<C::NS_Q, C::RP_O, false>(wo, L.o_c, L.o_s, a.dim, qd, r0, min(r0 + C::RW_O, a.dim), 0);
        }
        if (!grid_sync(a, ++gen)) return;
        // ---- x += W_o . attention
        gemv_stage<RFP4_EPI_RESIDUAL, C::NS_Q, C::RW_O, C::RP_O>(wo, L.o_c, L.o_s, a.dim, qd, 0, a.att, nullptr, 0.0f,
                                                                  a.x, xs);
        vm_drain();
        WParts<C::NS_DIM, 2 * C::RP_GU> wg;
        {
            const uint32_t r0 = (blockIdx.x * 4u + wave) * C::RW_GU;
            w_issue<C::NS_DIM, C::RP_GU, true>(wg, L.gu_c, L.gu_s, a.ffn, a.dim, r0, min(r0 + C::RW_GU, a.ffn), a.ffn);
        }
        if (!grid_sync(a, ++gen)) return;
        // ---- sw = silu(W_gate . rmsnorm(x)) * (W_up . rmsnorm(x))
        gemv_stage<RFP4_EPI_SWIGLU, C::NS_DIM, C::RW_GU, C::RP_GU>(wg, L.gu_c, L.gu_s, a.ffn, a.dim, a.ffn, a.x,
                                                                    a.norm_ffn + (size_t)l * a.dim, a.eps, a.sw, xs);
        vm_drain();
        WParts<C::NS_FFN, C::RP_D> wd;
        {
            const uint32_t r0 = (blockIdx.x * 4u + wave) * C::RW_D;
            w_issue<C::NS_FFN, C::RP_D, false>(wd, L.d_c, L.d_s, a.dim, a.ffn, r0, min(r0 + C::RW_D, a.dim), 0);
        }
        if (!grid_sync(a, ++gen)) return;
        // ---- x += W_down . sw
        gemv_stage<RFP4_EPI_RESIDUAL, C::NS_FFN, C::RW_D, C::RP_D>(wd, L.d_c, L.d_s, a.dim, a.ffn, 0, a.sw, nullptr, 0.0f,
                                                                    a.x, xs);
        vm_drain();
        if (l + 1 < a.n_layers) {
            const PersistLayer &N = a.layers[l + 1];
            const uint32_t r0 = (blockIdx.x * 4u + wave) * C::RW_QKV;
            w_issue<C::NS_DIM, C::RP_QKV, false>(wq, N.qkv_c, N.qkv_s, nqkv, a.dim, r0, min(r0 + C::RW_QKV, nqkv), 0);
            if (!grid_sync(a, ++gen)) return;
        }
    }
}
