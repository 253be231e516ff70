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
// per row covers 1 KiB of a row contiguously across the wave.  The lane loads
// its 32 activations once per slice and reuses them for all R rows of the
// wave; partial sums are reduced across the wave with DPP at the end.
// A workgroup is 4 waves = 4R logical rows.
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

template <int SCALE_F32, int EPI, int R>
RFP4_DEV void gemv_body(const GemvArgs &a)
{
    constexpr int NP = (EPI == RFP4_EPI_SWIGLU) ? 2 * R : R;
    __shared__ unsigned long long s_best[4];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const uint32_t lrow0 = (blockIdx.x * 4u + (uint32_t)wave) * (uint32_t)R;
    const uint32_t nchunk = a.k >> 5;
    const size_t rowbytes = (size_t)(a.k >> 1);

    uint32_t prow[NP];
#pragma unroll
    for (int i = 0; i < R; i++) {
        uint32_t lr = lrow0 + (uint32_t)i;
        uint32_t r = lr < a.n ? lr : a.n - 1; // clamp: loads stay in bounds
        prow[i] = r;
        if (EPI == RFP4_EPI_SWIGLU) prow[R + i] = r + a.pair_off;
    }

    float acc[NP];
#pragma unroll
    for (int p = 0; p < NP; p++) acc[p] = 0.0f;

    const uint8_t *wb = (const uint8_t *)a.w;
    for (uint32_t c = (uint32_t)lane; c < nchunk; c += 64u) {
        uint4 q[NP];
        float sc[NP];
#pragma unroll
        for (int p = 0; p < NP; p++) {
            q[p] = *(const uint4 *)(wb + (size_t)prow[p] * rowbytes + (size_t)c * 16u);
            sc[p] = load_scale<SCALE_F32>(a.scales, (size_t)prow[p] * nchunk + c);
        }
        float4 xv[8];
        const float4 *xp = (const float4 *)(a.x) + (size_t)c * 8u;
#pragma unroll
        for (int j = 0; j < 8; j++) xv[j] = xp[j];
#pragma unroll
        for (int p = 0; p < NP; p++) acc[p] = fmaf(sc[p], dot_chunk32(q[p], xv), acc[p]);
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
            for (int w = 1; w < 4; w++) b = s_best[w] > b ? s_best[w] : b;
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
                a.y[lr] = __fadd_rn(a.y[lr], acc[i]);
            } else { // SWIGLU: silu(gate) * up  (llama_run/src/main.rs:244-252)
                a.y[lr] = __fmul_rn(silu_ref(acc[i]), acc[R + i]);
            }
        }
    }
}
