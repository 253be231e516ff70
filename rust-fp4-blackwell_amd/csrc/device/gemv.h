// MXFP4 decode GEMV for gfx950.
//
// y[n] = sum_blocks scale[n,b] * sum_{k in b} e2m1(W[n,k]) * x[k]
// (reference: llama_run/src/main.rs:34-77, fp4_gemv/src/main.rs:32-92).
//
// Layout: the reference's row-major packing, K/2 code bytes per row (two E2M1
// codes per byte, low nibble = lower k) and K/32 scales per row.
//
// Mapping (wave64): lane l owns 16-byte chunk c = l + 64*s of every row it
// touches (32 codes = exactly one scale block), so one global_load_dwordx4
// per row covers 1 KiB of a row contiguously across the wave.  A workgroup
// (4 waves, 4R logical rows) stages x in LDS once (36 floats per 32-value
// chunk, which keeps the per-lane reads free of bank conflicts) -- optionally RMS-normalized
// on the way (the rmsnorm launch of llama_run/src/main.rs:513,525 folded in)
// -- and each lane reads its 32 activations per slice from LDS and reuses them
// for all R rows of its wave.  Weight loads are double-buffered across
// slices; the first slice is issued before x is staged.  Partial sums are
// reduced across the wave with DPP at the end.
#pragma once
#include "common.h"

template <int SCALE_F32>
RFP4_DEV float load_scale(const void *scales, size_t idx)
{
    if (SCALE_F32) return ((const float *)scales)[idx];
    return e8m0_to_f32(((const uint8_t *)scales)[idx]);
}

RFP4_DEV float silu_ref(float g)
{
    // llama_run/src/main.rs:248-249: g / (1 + exp(-g))
    return __fdiv_rn(g, __fadd_rn(1.0f, expf(-g)));
}

// x in LDS: each 32-value chunk (one scale block) takes 36 floats, so chunk
// c starts at 16-byte slot 9c.  The dot loops read the same float4 of 64
// consecutive chunks at once (one chunk per lane); at 9 slots per chunk any
// 16 consecutive lanes fall on 16 distinct 16-byte bank groups (no conflict
// with 64 four-byte banks, nor with 32), where packed 128-byte chunks would
// put a whole wave on one or two bank groups.
#define GEMV_XS_CHUNK 36u
RFP4_DEV uint32_t xs_slot(uint32_t i4) { return (i4 >> 3) * 9u + (i4 & 7u); } // LDS float4 of x float4 i4

// Stage x (K floats) into LDS; with norm_w, store x * rms * w instead
// (rms = 1/sqrt(sum(x^2)/K + eps), llama_rmsnorm/src/main.rs:75-77).
RFP4_DEV void stage_x(float *xs, const float *x, uint32_t k, const uint16_t *norm_w, float eps)
{
    __shared__ float red[4];
    const int tid = threadIdx.x;
    const uint32_t k4 = k >> 2;
    float4 *xs4 = (float4 *)xs;
    if (norm_w == nullptr) {
        for (uint32_t i = tid; i < k4; i += 256) xs4[xs_slot(i)] = ((const float4 *)x)[i];
        __syncthreads();
        return;
    }
    float ss = 0.0f;
    for (uint32_t i = tid; i < k4; i += 256) {
        float4 v = ((const float4 *)x)[i];
        xs4[xs_slot(i)] = v;
        ss = __fadd_rn(ss, __fmul_rn(v.x, v.x));
        ss = __fadd_rn(ss, __fmul_rn(v.y, v.y));
        ss = __fadd_rn(ss, __fmul_rn(v.z, v.z));
        ss = __fadd_rn(ss, __fmul_rn(v.w, v.w));
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    float total = (red[0] + red[1]) + (red[2] + red[3]);
    float rms = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(total, (float)k), eps)));
    for (uint32_t i = tid; i < k4; i += 256) {
        float4 v = xs4[xs_slot(i)];
        const uint16_t *w = norm_w + 4u * i;
        v.x = __fmul_rn(__fmul_rn(v.x, rms), f16_bits_to_f32(w[0]));
        v.y = __fmul_rn(__fmul_rn(v.y, rms), f16_bits_to_f32(w[1]));
        v.z = __fmul_rn(__fmul_rn(v.z, rms), f16_bits_to_f32(w[2]));
        v.w = __fmul_rn(__fmul_rn(v.w, rms), f16_bits_to_f32(w[3]));
        xs4[xs_slot(i)] = v;
    }
    __syncthreads();
}

// stage_x from registers (XV float4 of x and uint2 of fp16 norm weights per
// thread, element 4*(tid + T*v) + j for T = 64*W threads, zero past K).
template <int XV, int W = 4>
RFP4_DEV void stage_x_regs(float *xs, const float4 *xr, const uint2 *wr, uint32_t k, bool norm, float eps)
{
    constexpr uint32_t T = 64u * W;
    __shared__ float red[W];
    const int tid = threadIdx.x;
    const uint32_t k4 = k >> 2;
    float rms = 1.0f;
    if (norm) {
        float ss = 0.0f;
#pragma unroll
        for (int v = 0; v < XV; v++) {
            ss = __fadd_rn(ss, __fmul_rn(xr[v].x, xr[v].x));
            ss = __fadd_rn(ss, __fmul_rn(xr[v].y, xr[v].y));
            ss = __fadd_rn(ss, __fmul_rn(xr[v].z, xr[v].z));
            ss = __fadd_rn(ss, __fmul_rn(xr[v].w, xr[v].w));
        }
        ss = wave_sum(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        float total = (red[0] + red[1]) + (red[2] + red[3]);
#pragma unroll
        for (int w = 4; w < W; w += 4) total += (red[w] + red[w + 1]) + (red[w + 2] + red[w + 3]);
        rms = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(total, (float)k), eps)));
    }
#pragma unroll
    for (int v = 0; v < XV; v++) {
        const uint32_t i4 = (uint32_t)tid + T * (uint32_t)v;
        if (i4 >= k4) break;
        float4 o = xr[v];
        if (norm) {
            o.x = __fmul_rn(__fmul_rn(o.x, rms), f16_bits_to_f32((uint16_t)(wr[v].x & 0xFFFFu)));
            o.y = __fmul_rn(__fmul_rn(o.y, rms), f16_bits_to_f32((uint16_t)(wr[v].x >> 16)));
            o.z = __fmul_rn(__fmul_rn(o.z, rms), f16_bits_to_f32((uint16_t)(wr[v].y & 0xFFFFu)));
            o.w = __fmul_rn(__fmul_rn(o.w, rms), f16_bits_to_f32((uint16_t)(wr[v].y >> 16)));
        }
        ((float4 *)xs)[xs_slot(i4)] = o;
    }
    __syncthreads();
}

// x (and the fp16 norm weights) for stage_x_regs, XV float4 per thread of T
// (element 4*(tid + T*v) + j).  issue() sends the loads with no per-element
// branch (the index clamped into range; the norm weights behind one uniform
// branch), so nothing separates them from the caller's weight loads that
// follow; settle(), after those are issued, zeroes what lies past K through a
// mask the compiler cannot see through (else it turns the selects back into
// branches around the loads).  Measured on the 8B gate|up GEMV with its fused
// norm: 13.7-13.9 -> 13.3-13.4 us per launch, values unchanged.
template <int XV, uint32_t T>
struct XRegs {
    float4 xr[XV];
    uint2 wr[XV];

    RFP4_DEV void issue(const float *x, const uint16_t *norm_w, uint32_t k)
    {
        const uint32_t k4 = k >> 2;
#pragma unroll
        for (int v = 0; v < XV; v++) xr[v] = ((const float4 *)x)[min(threadIdx.x + T * (uint32_t)v, k4 - 1u)];
        if (norm_w) {
#pragma unroll
            for (int v = 0; v < XV; v++) wr[v] = ((const uint2 *)norm_w)[min(threadIdx.x + T * (uint32_t)v, k4 - 1u)];
        } else {
#pragma unroll
            for (int v = 0; v < XV; v++) wr[v] = make_uint2(0, 0);
        }
    }

    RFP4_DEV void settle(uint32_t k)
    {
        const uint32_t k4 = k >> 2;
#pragma unroll
        for (int v = 0; v < XV; v++) {
            uint32_t m = threadIdx.x + T * (uint32_t)v < k4 ? 0xFFFFFFFFu : 0u;
            asm volatile("" : "+v"(m));
            xr[v] = make_float4(__uint_as_float(__float_as_uint(xr[v].x) & m), __uint_as_float(__float_as_uint(xr[v].y) & m),
                                __uint_as_float(__float_as_uint(xr[v].z) & m), __uint_as_float(__float_as_uint(xr[v].w) & m));
            wr[v] = make_uint2(wr[v].x & m, wr[v].y & m);
        }
    }
};

// Raw scale bits now, value at use: keeps the loads free of dependent ALU
// work so they can all be in flight together.
template <int SCALE_F32>
RFP4_DEV uint32_t load_scale_bits(const void *scales, size_t idx)
{
    if (SCALE_F32) return load_nt_u32((const uint32_t *)scales + idx);
    return load_nt_u8((const uint8_t *)scales + idx);
}

template <int SCALE_F32>
RFP4_DEV float scale_from_bits(uint32_t b)
{
    return SCALE_F32 ? __uint_as_float(b) : e8m0_to_f32(b);
}

// NS: K-slices of 64 chunks (2048 values) per row, fixed at compile time so
// all loads are issued up front; NS = 0 handles any K with a slice loop.
// W: waves per workgroup (4, or 8 / 16 with NS > 0: more, shorter waves
// share one staging of x).
template <int SCALE_F32, int EPI, int R, int NS, int W = 4>
RFP4_DEV void gemv_body(const GemvArgs &a)
{
    static_assert(W == 4 || NS > 0, "the slice loop stages x with 4 waves");
    static_assert(W % 4 == 0 && W <= 16, "waves per workgroup");
    constexpr int NP = (EPI == RFP4_EPI_SWIGLU) ? 2 * R : R;
    constexpr uint32_t T = 64u * W;
    extern __shared__ float xs[]; // K/32 chunks of GEMV_XS_CHUNK floats (dynamic LDS)
    __shared__ unsigned long long s_best[W];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const uint32_t lrow0 = (blockIdx.x * (uint32_t)W + (uint32_t)wave) * (uint32_t)R;
    const uint32_t nchunk = a.k >> 5;
    const size_t rowbytes = (size_t)(a.k >> 1);

    const uint8_t *rowp[NP];
    size_t srow[NP];
#pragma unroll
    for (int i = 0; i < R; i++) {
        uint32_t lr = lrow0 + (uint32_t)i;
        uint32_t r = lr < a.n ? lr : a.n - 1; // clamp: loads stay in bounds
        rowp[i] = (const uint8_t *)a.w + (size_t)r * rowbytes;
        srow[i] = (size_t)r * nchunk;
        if (EPI == RFP4_EPI_SWIGLU) {
            rowp[R + i] = (const uint8_t *)a.w + (size_t)(r + a.pair_off) * rowbytes;
            srow[R + i] = (size_t)(r + a.pair_off) * nchunk;
        }
    }

    const uint32_t clast = nchunk - 1u;
    float acc[NP];
#pragma unroll
    for (int p = 0; p < NP; p++) acc[p] = 0.0f;
    // residual epilogue: the rows' current values are fetched before any
    // weight load, so the epilogue does not wait on a memory round trip
    float yres[EPI == RFP4_EPI_RESIDUAL ? R : 1];
    if (EPI == RFP4_EPI_RESIDUAL) {
#pragma unroll
        for (int i = 0; i < R; i++) {
            const uint32_t lr = lrow0 + (uint32_t)i;
            yres[i] = lr < a.n ? a.y[lr] : 0.0f;
        }
    }

    if (NS > 0) {
        // x (and norm weights) go into registers first, then every weight load
        // of this wave (NS slices x NP rows): waiting for x then never waits
        // for the weights (vmcnt retires in issue order).  A lane past the
        // last chunk re-reads the last chunk (in bounds) and gets scale 0.
        constexpr int XV = NS > 0 ? (512 * NS + (int)T - 1) / (int)T : 1; // float4 of x per thread: K <= 2048 * NS
        XRegs<XV, T> xg;
        xg.issue(a.x, a.norm_w, a.k);
        __builtin_amdgcn_sched_barrier(0); // x before the weight stream
        uint4 q[NS > 0 ? NS : 1][NP];
        uint32_t sb[NS > 0 ? NS : 1][NP];
#pragma unroll
        for (int s = 0; s < NS; s++) {
            const uint32_t cl = min((uint32_t)lane + 64u * (uint32_t)s, clast);
#pragma unroll
            for (int p = 0; p < NP; p++) {
                q[s][p] = load_nt16(rowp[p] + (size_t)cl * 16u);
                sb[s][p] = load_scale_bits<SCALE_F32>(a.scales, srow[p] + cl);
            }
        }
        xg.settle(a.k);
        stage_x_regs<XV, W>(xs, xg.xr, xg.wr, a.k, a.norm_w != nullptr, a.eps);
#pragma unroll
        for (int s = 0; s < NS; s++) {
            const uint32_t c = (uint32_t)lane + 64u * (uint32_t)s;
            const float live = c < nchunk ? 1.0f : 0.0f;
            float4 xv[8];
            const float4 *xp = (const float4 *)(xs + (size_t)min(c, clast) * GEMV_XS_CHUNK);
#pragma unroll
            for (int j = 0; j < 8; j++) xv[j] = xp[j];
#pragma unroll
            for (int p = 0; p < NP; p++)
                acc[p] = fmaf(live * scale_from_bits<SCALE_F32>(sb[s][p]), dot_chunk32(q[s][p], xv), acc[p]);
        }
    } else {
        // any K: one slice at a time
        stage_x(xs, a.x, a.k, a.norm_w, a.eps);
        for (uint32_t c = (uint32_t)lane; c < nchunk; c += 64u) {
            uint4 q[NP];
            float sc[NP];
#pragma unroll
            for (int p = 0; p < NP; p++) {
                q[p] = load_nt16(rowp[p] + (size_t)c * 16u);
                sc[p] = scale_from_bits<SCALE_F32>(load_scale_bits<SCALE_F32>(a.scales, srow[p] + c));
            }
            float4 xv[8];
            const float4 *xp = (const float4 *)(xs + (size_t)c * GEMV_XS_CHUNK);
#pragma unroll
            for (int j = 0; j < 8; j++) xv[j] = xp[j];
#pragma unroll
            for (int p = 0; p < NP; p++) acc[p] = fmaf(sc[p], dot_chunk32(q[p], xv), acc[p]);
        }
    }

#pragma unroll
    for (int p = 0; p < NP; p++) acc[p] = wave_sum(acc[p]);

    if (EPI == RFP4_EPI_ARGMAX) {
        if (lane == 0) {
            float bv = -1e30f;
            uint32_t bi = 0;
            bool any = false;
#pragma unroll
            for (int i = 0; i < R; i++) {
                uint32_t lr = lrow0 + (uint32_t)i;
                if (lr < a.n) {
                    a.y[lr] = acc[i];
                    if (acc[i] > bv) {
                        bv = acc[i];
                        bi = lr;
                        any = true;
                    }
                }
            }
            s_best[wave] = any ? pack_argmax(bv, bi) : pack_argmax(-1e30f, 0u);
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned long long b = s_best[0];
            for (int w = 1; w < W; w++) b = s_best[w] > b ? s_best[w] : b;
            a.best[blockIdx.x] = b;
        }
        return;
    }

    if (lane == 0) {
#pragma unroll
        for (int i = 0; i < R; i++) {
            uint32_t lr = lrow0 + (uint32_t)i;
            if (lr >= a.n) continue;
            if (EPI == RFP4_EPI_STORE) {
                a.y[lr] = acc[i];
            } else if (EPI == RFP4_EPI_RESIDUAL) {
                a.y[lr] = __fadd_rn(yres[EPI == RFP4_EPI_RESIDUAL ? i : 0], acc[i]);
            } else { // SWIGLU: silu(gate) * up  (llama_run/src/main.rs:244-252)
                a.y[lr] = __fmul_rn(silu_ref(acc[i]), acc[R + i]);
            }
        }
    }
}
