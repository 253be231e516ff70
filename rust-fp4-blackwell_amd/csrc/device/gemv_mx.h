// MXFP4 decode GEMV on the gfx950 block-scaled matrix cores, weights fed to
// v_mfma_scale_f32_16x16x128_f8f6f4 as stored (E2M1 codes + E8M0 scales, no
// conversion instruction per weight).
//
// Same contract as gemv.h (y = W.x over the reference packing,
// fp4_gemv/src/main.rs:113-120; epilogues store / residual / SwiGLU /
// argmax).  The activation x is split into GEMV_MX_PLANES planes of OCP FP8
// (E4M3) values, each with its own E8M0 scale per 32 values:
//     r_0 = x,  p_c = e4m3(r_c / s_c),  r_{c+1} = r_c - s_c * p_c,
// s_c = 2^(floor(log2 max|r_c|) - 7) over the block, so |r_c / s_c| < 256
// (inside E4M3's range, rounding to nearest even: a plane takes the next 4
// significant bits of the block's largest residual).  Six planes leave a
// residual below 2^-24 of the block's largest |x|: the f32 level of the
// reference's own sums.  The planes are the columns of the MFMA's second
// operand: D[row][c] = sum_k W[row][k] * p_c[k] (E2M1 x E4M3 products are
// exact, each scaled by 2^(sW + s_c)), and y[row] = sum_c D[row][c].
//
// Layout: a workgroup owns one tile of 16 weight rows (SwiGLU: the gate tile
// and the matching up tile) and splits K over its 4 waves in segments of 512
// values (PER segments per wave).  Lane l holds weight row
// l%16 and the 64 bytes 64*(l/16) .. +63 of the segment's 256 bytes; MFMA t
// (0..3) of the segment takes bytes 16t .. 16t+15 of those, i.e. the values
// 512 s + 128 q + 32 t + (0..31) for q = l/16.  The planes are stored in LDS
// per 32-value block in that order, and each lane of the E4M3 operand reads
// the two 16-value halves its MFMA-K slots pair with (the K permutation is
// applied to both operands, so the dot product is unchanged).  Every weight load of a wave is issued before
// the planes are built, so building them overlaps the HBM latency.
#pragma once
#include "common.h"
#include "gemv.h"
#include "mma.h"
#include "norm_rope.h"

#define GEMV_MX_PLANES 6
#define MX_FMT_FP8 0

typedef short mx_v2i16 __attribute__((ext_vector_type(2)));

// Bytes of LDS the planes of a K-vector take (codes, then per-(segment,
// quarter, plane) dwords of 4 block scales).
constexpr uint32_t gemv_mx_lds_bytes(uint32_t k) { return k * GEMV_MX_PLANES + (k / 32u) * GEMV_MX_PLANES; }

// One 32-value block r[] (consumed) -> GEMV_MX_PLANES planes of E4M3 codes
// and E8M0 scale bytes, written at their MFMA-order place in LDS.
RFP4_DEV void gemv_mx_planes_block(float *r, uint32_t b, uint8_t *codes, uint8_t *scales)
{
    const uint32_t seg = b >> 4, q = (b >> 2) & 3u, t = b & 3u;
#pragma unroll
    for (int c = 0; c < GEMV_MX_PLANES; c++) {
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(r[i]));
        const uint32_t e = (__float_as_uint(amax) >> 23) & 0xFFu; // biased exponent of the block max
        const bool live = e > 7u;                                   // else the residual is below 2^-120: drop it
        const uint32_t sbyte = live ? e - 7u : 0u;
        const float scale = __uint_as_float((live ? sbyte : 1u) << 23);
        uint32_t w[8];
#pragma unroll
        for (int d = 0; d < 8; d++) {
            mx_v2i16 p = {0, 0};
            p = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(p, r[4 * d], r[4 * d + 1], scale, false);
            p = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(p, r[4 * d + 2], r[4 * d + 3], scale, true);
            w[d] = live ? __builtin_bit_cast(uint32_t, p) : 0u;
        }
        if (c + 1 < GEMV_MX_PLANES) {
#pragma unroll
            for (int d = 0; d < 8; d++) {
                const f32x2 lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w[d], scale, false);
                const f32x2 hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w[d], scale, true);
                r[4 * d] = __fsub_rn(r[4 * d], lo.x);
                r[4 * d + 1] = __fsub_rn(r[4 * d + 1], lo.y);
                r[4 * d + 2] = __fsub_rn(r[4 * d + 2], hi.x);
                r[4 * d + 3] = __fsub_rn(r[4 * d + 3], hi.y);
            }
        }
        uint4 *dst = (uint4 *)(codes + ((((size_t)seg * 4u + t) * 4u + q) * GEMV_MX_PLANES + (uint32_t)c) * 32u);
        dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
        dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
        scales[(((size_t)seg * 4u + q) * GEMV_MX_PLANES + (uint32_t)c) * 4u + t] = (uint8_t)sbyte;
    }
}

// EPI: epilogue; NORM: x is RMS-normalised with a.norm_w first; PER:
// 512-value segments per wave (K <= 2048 * PER, all loads issued up front).
// One 16-row output tile per workgroup (SwiGLU: its gate tile and the
// matching up tile); each thread builds the planes of XB 32-value blocks.
template <int EPI, int NORM, int PER>
RFP4_DEV void gemv_mx_body(const GemvArgs &a)
{
    constexpr int P = GEMV_MX_PLANES;
    constexpr int NT = (EPI == RFP4_EPI_SWIGLU) ? 2 : 1; // weight tiles
    constexpr int NO = 1;                                 // output tiles
    constexpr int XB = PER > 4 ? 2 : 1;                   // K <= 8192 * XB
    extern __shared__ __align__(16) uint8_t mx_lds[];
    __shared__ float red[4][NT * 16];
    __shared__ float sred[16];

    const uint32_t k = a.k, nseg = k >> 9, nblk = k >> 5, rowbytes = k >> 1;
    uint8_t *pcodes = mx_lds;
    uint8_t *pscales = mx_lds + (size_t)k * P;
    const int tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane((uint32_t)tid >> 6);
    const uint32_t r16 = (uint32_t)lane & 15u, q = (uint32_t)lane >> 4;
    const uint32_t row0 = blockIdx.x * (uint32_t)NO * 16u; // first output row

    // ---- 1) x (and norm weights) of this thread's blocks into registers
    constexpr bool norm = NORM != 0;
    float4 xr[XB][8];
    uint4 wr[XB][4];
#pragma unroll
    for (int j = 0; j < XB; j++) {
        const uint32_t b = (uint32_t)tid + 256u * (uint32_t)j;
        const bool in = b < nblk;
#pragma unroll
        for (int v = 0; v < 8; v++)
            xr[j][v] = in ? ((const float4 *)a.x)[b * 8u + (uint32_t)v] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int v = 0; v < 4; v++)
            wr[j][v] = (in && norm) ? ((const uint4 *)a.norm_w)[b * 4u + (uint32_t)v] : make_uint4(0, 0, 0, 0);
    }

    // ---- 2) every weight load of this wave: tile tt, segment s, 64 bytes + 4 scale bytes
    const uint8_t *rowp[NT];
    const uint8_t *srow[NT];
#pragma unroll
    for (int tt = 0; tt < NT; tt++) {
        uint32_t lr = row0 + (uint32_t)(tt % NO) * 16u + r16;
        uint32_t r = lr < a.n ? lr : a.n - 1u; // clamp: loads stay in bounds
        if (EPI == RFP4_EPI_SWIGLU && tt >= NO) r += a.pair_off;
        rowp[tt] = (const uint8_t *)a.w + (size_t)r * rowbytes + q * 64u;
        srow[tt] = (const uint8_t *)a.scales + (size_t)r * nblk + q * 4u;
    }
    uint4 wq[NT][PER][4];
    uint32_t ws[NT][PER];
#pragma unroll
    for (int s = 0; s < PER; s++) {
        const uint32_t seg = min(wave * (uint32_t)PER + (uint32_t)s, nseg - 1u);
#pragma unroll
        for (int tt = 0; tt < NT; tt++) {
#pragma unroll
            for (int t = 0; t < 4; t++) wq[tt][s][t] = *(const uint4 *)(rowp[tt] + (size_t)seg * 256u + t * 16u);
            ws[tt][s] = *(const uint32_t *)(srow[tt] + (size_t)seg * 16u);
        }
    }
    // residual epilogue: the rows' current values, fetched early
    float yres = 0.0f;
    if (EPI == RFP4_EPI_RESIDUAL && wave == 0 && lane < NO * 16) {
        const uint32_t lr = row0 + (uint32_t)lane;
        yres = lr < a.n ? a.y[lr] : 0.0f;
    }

    // ---- 3) planes of x (RMS-normalised first when norm_w is given)
    float rms = 1.0f;
    if (norm) {
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < XB; j++)
#pragma unroll
            for (int v = 0; v < 8; v++) {
                const float4 u = xr[j][v];
                ss = __fadd_rn(ss, __fmul_rn(u.x, u.x));
                ss = __fadd_rn(ss, __fmul_rn(u.y, u.y));
                ss = __fadd_rn(ss, __fmul_rn(u.z, u.z));
                ss = __fadd_rn(ss, __fmul_rn(u.w, u.w));
            }
        const float total = block_sum(ss, sred);
        rms = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(total, (float)k), a.eps)));
    }
#pragma unroll
    for (int j = 0; j < XB; j++) {
        const uint32_t b = (uint32_t)tid + 256u * (uint32_t)j;
        if (b >= nblk) break;
        float r[32];
#pragma unroll
        for (int v = 0; v < 8; v++) {
            r[4 * v] = xr[j][v].x;
            r[4 * v + 1] = xr[j][v].y;
            r[4 * v + 2] = xr[j][v].z;
            r[4 * v + 3] = xr[j][v].w;
        }
        if (norm) {
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const uint32_t h[4] = {wr[j][v].x, wr[j][v].y, wr[j][v].z, wr[j][v].w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int e = 8 * v + 2 * i;
                    r[e] = __fmul_rn(__fmul_rn(r[e], rms), f16_bits_to_f32((uint16_t)(h[i] & 0xFFFFu)));
                    r[e + 1] = __fmul_rn(__fmul_rn(r[e + 1], rms), f16_bits_to_f32((uint16_t)(h[i] >> 16)));
                }
            }
        }
        gemv_mx_planes_block(r, b, pcodes, pscales);
    }
    __syncthreads();

    // ---- 4) MFMAs: lane (c = l%16, q) reads plane c of its K slots (zero for c >= P)
    v4f32 acc[NT];
#pragma unroll
    for (int tt = 0; tt < NT; tt++) acc[tt] = (v4f32){0.0f, 0.0f, 0.0f, 0.0f};
    const bool pl = r16 < (uint32_t)P;
#pragma unroll
    for (int s = 0; s < PER; s++) {
        const uint32_t seg = wave * (uint32_t)PER + (uint32_t)s;
        if (seg >= nseg) break; // wave-uniform
        const uint32_t sbw = pl ? *(const uint32_t *)(pscales + (((size_t)seg * 4u + q) * P + r16) * 4u) : 0u;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            v8i32 b8 = {0, 0, 0, 0, 0, 0, 0, 0};
            if (pl) {
                // E4M3 operand layout (pinned on the device): lane (c, g) holds
                // MFMA-K 16g .. 16g+15 in bytes 0..15 and 64+16g .. 64+16g+15 in
                // bytes 16..31, i.e. half g&1 of the blocks of quarters g>>1 and
                // 2 + (g>>1) (the E2M1 operand holds MFMA-K 32g .. 32g+31).
                const size_t base = ((size_t)seg * 4u + (uint32_t)t) * 4u;
                const uint32_t half = (q & 1u) * 16u;
                const uint4 lo = *(const uint4 *)(pcodes + ((base + (q >> 1)) * P + r16) * 32u + half);
                const uint4 hi = *(const uint4 *)(pcodes + ((base + 2u + (q >> 1)) * P + r16) * 32u + half);
                b8 = (v8i32){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
            }
            const int sb = (int)((sbw >> (8 * t)) & 0xFFu);
#pragma unroll
            for (int tt = 0; tt < NT; tt++) {
                const uint4 w = wq[tt][s][t];
                const v8i32 a8 = {(int)w.x, (int)w.y, (int)w.z, (int)w.w, 0, 0, 0, 0};
                const int sa = (int)((ws[tt][s] >> (8 * t)) & 0xFFu);
                acc[tt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a8, b8, acc[tt], MX_FMT_FP4, MX_FMT_FP8, 0,
                                                                           sa, 0, sb);
            }
        }
    }

    // ---- 5) y = sum over planes (lanes of a 16-lane row group; columns >= P
    // are zero), rows 4*(l/16) + r in register r; K quarters summed in wave order
#pragma unroll
    for (int tt = 0; tt < NT; tt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float v = acc[tt][r];
            v += dpp_mov<DPP_QUAD_1032>(v);
            v += dpp_mov<DPP_QUAD_2301>(v);
            v += dpp_mov<DPP_ROW_HALF_MIRROR>(v);
            v += dpp_mov<DPP_ROW_MIRROR>(v);
            if (r16 == 0) red[wave][tt * 16 + q * 4 + (uint32_t)r] = v;
        }
    __syncthreads();
    if (wave != 0) return;

    const uint32_t i = (uint32_t)lane;
    const uint32_t lr = row0 + i;
    const bool ok = i < (uint32_t)NO * 16u && lr < a.n;
    float yv = 0.0f, uv = 0.0f;
    if (i < (uint32_t)NO * 16u) {
        yv = ((red[0][i] + red[1][i]) + red[2][i]) + red[3][i];
        if (EPI == RFP4_EPI_SWIGLU)
            uv = ((red[0][NO * 16 + i] + red[1][NO * 16 + i]) + red[2][NO * 16 + i]) + red[3][NO * 16 + i];
    }
    if (EPI == RFP4_EPI_ARGMAX) {
        unsigned long long key = ok ? pack_argmax(yv, lr) : pack_argmax(-1e30f, 0u);
        if (ok) a.y[lr] = yv;
        for (int off = 32; off >= 1; off >>= 1) {
            const unsigned long long o = __shfl_xor(key, off, 64);
            key = o > key ? o : key;
        }
        if (lane == 0) a.best[blockIdx.x] = key;
        return;
    }
    if (!ok) return;
    if (EPI == RFP4_EPI_STORE) a.y[lr] = yv;
    else if (EPI == RFP4_EPI_RESIDUAL) a.y[lr] = __fadd_rn(yres, yv);
    else a.y[lr] = __fmul_rn(silu_ref(yv), uv);
}
