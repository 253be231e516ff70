// MXFP4 decode GEMV on the gfx950 matrix cores.
//
// Same contract as gemv.h (y = W.x, E2M1 codes + E8M0 block scales,
// row-major reference packing); the arithmetic moves from VALU FMAs to
// v_mfma_f32_16x16x32_bf16:
//  - A (weights): each lane converts its 32 codes of one scale block to
//    bf16 with v_cvt_scalef32_pk_bf16_fp4, the E8M0 scale folded in (the
//    conversion uses the scale's exponent, and code * 2^e is exact in bf16);
//  - B (activation): x = hi + mid + lo, three bf16 planes (exact to 2^-27
//    relative), staged in LDS once per workgroup -- RMS-normalized on the way
//    when norm_w is given -- and occupying B columns 0..2 (columns 3..15 zero);
//  - y[row] = D[row][0] + D[row][1] + D[row][2] (bf16 x bf16 products are
//    exact, accumulation is f32 in the matrix core).
// VALU work per 16 code bytes drops from ~50 instructions (decode + FMA) to
// the 4 conversions per MFMA, so the loads of a wave are the only latency.
//
// Mapping: a wave covers 16-row tiles; lane l holds row l%16 and, within each
// 128-value super-chunk, the 32 values of block 4*sc + l/16 (one 16-byte
// load, one scale byte).  MFMA t of a super-chunk takes 8 of those values per
// lane (K-permuted consistently in A and B, which leaves the dot product
// unchanged).  The 4 waves of a workgroup split K; their partial rows are
// combined through LDS in a fixed order.
#pragma once
#include "common.h"

typedef __bf16 mfma_bf16x8 __attribute__((ext_vector_type(8)));
typedef float mfma_f32x4 __attribute__((ext_vector_type(4)));

RFP4_DEV uint32_t f32_to_bf16_rne_bits(float f)
{
    uint32_t u = __float_as_uint(f);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16; // finite inputs
}

// Stage x (optionally x*rms*w) as three bf16 planes [3][k] in LDS.
RFP4_DEV void stage_planes(uint16_t *planes, const float *x, uint32_t k, const uint16_t *norm_w, float eps)
{
    __shared__ float red[4];
    const int tid = threadIdx.x;
    float rms = 1.0f;
    if (norm_w != nullptr) {
        float ss = 0.0f;
        for (uint32_t i = tid; i < (k >> 2); i += 256) {
            float4 v = ((const float4 *)x)[i];
            ss = __fadd_rn(ss, __fmul_rn(v.x, v.x));
            ss = __fadd_rn(ss, __fmul_rn(v.y, v.y));
            ss = __fadd_rn(ss, __fmul_rn(v.z, v.z));
            ss = __fadd_rn(ss, __fmul_rn(v.w, v.w));
        }
        ss = wave_sum(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        float total = (red[0] + red[1]) + (red[2] + red[3]);
        rms = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(total, (float)k), eps)));
    }
    for (uint32_t i = tid; i < k; i += 256) {
        float v = x[i];
        if (norm_w != nullptr) v = __fmul_rn(__fmul_rn(v, rms), f16_bits_to_f32(norm_w[i]));
        uint32_t hi = f32_to_bf16_rne_bits(v);
        float r1 = __fsub_rn(v, bf16_bits_to_f32(hi));
        uint32_t mid = f32_to_bf16_rne_bits(r1);
        float r2 = __fsub_rn(r1, bf16_bits_to_f32(mid));
        uint32_t lo = f32_to_bf16_rne_bits(r2);
        planes[i] = (uint16_t)hi;
        planes[k + i] = (uint16_t)mid;
        planes[2 * k + i] = (uint16_t)lo;
    }
    __syncthreads();
}

// Same, from x (and norm weights) already in registers: XV float4 per
// thread, element 4*(tid + 256*v) + j.  Loading x before the weight loads
// keeps the staging from waiting on them (vmcnt retires in issue order).
template <int XV>
RFP4_DEV void stage_planes_regs(uint16_t *planes, const float4 *xr, const uint2 *wr, uint32_t k, bool norm,
                                float eps)
{
    __shared__ float red[4];
    const int tid = threadIdx.x;
    const uint32_t k4 = k >> 2;
    float rms = 1.0f;
    if (norm) {
        float ss = 0.0f;
#pragma unroll
        for (int v = 0; v < XV; v++) {
            float4 q = xr[v]; // zero beyond k
            ss = __fadd_rn(ss, __fmul_rn(q.x, q.x));
            ss = __fadd_rn(ss, __fmul_rn(q.y, q.y));
            ss = __fadd_rn(ss, __fmul_rn(q.z, q.z));
            ss = __fadd_rn(ss, __fmul_rn(q.w, q.w));
        }
        ss = wave_sum(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        float total = (red[0] + red[1]) + (red[2] + red[3]);
        rms = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(total, (float)k), eps)));
    }
#pragma unroll
    for (int v = 0; v < XV; v++) {
        const uint32_t i4 = (uint32_t)tid + 256u * (uint32_t)v;
        if (i4 >= k4) break;
        const float e[4] = {xr[v].x, xr[v].y, xr[v].z, xr[v].w};
        const uint32_t wv[4] = {wr[v].x & 0xFFFFu, wr[v].x >> 16, wr[v].y & 0xFFFFu, wr[v].y >> 16};
        uint32_t hp[2] = {0, 0}, mp[2] = {0, 0}, lp[2] = {0, 0};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float val = e[j];
            if (norm) val = __fmul_rn(__fmul_rn(val, rms), f16_bits_to_f32((uint16_t)wv[j]));
            uint32_t hi = f32_to_bf16_rne_bits(val);
            float r1 = __fsub_rn(val, bf16_bits_to_f32(hi));
            uint32_t mid = f32_to_bf16_rne_bits(r1);
            float r2 = __fsub_rn(r1, bf16_bits_to_f32(mid));
            uint32_t lo = f32_to_bf16_rne_bits(r2);
            hp[j >> 1] |= hi << (16 * (j & 1));
            mp[j >> 1] |= mid << (16 * (j & 1));
            lp[j >> 1] |= lo << (16 * (j & 1));
        }
        *(uint2 *)(planes + 4 * i4) = make_uint2(hp[0], hp[1]);
        *(uint2 *)(planes + k + 4 * i4) = make_uint2(mp[0], mp[1]);
        *(uint2 *)(planes + 2 * k + 4 * i4) = make_uint2(lp[0], lp[1]);
    }
    __syncthreads();
}

// 8 bf16 of one MFMA's A fragment: the 8 codes of dword w, times 2^(sb-127).
RFP4_DEV mfma_bf16x8 a_frag(uint32_t w, float scale)
{
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    b2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0);
    b2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1);
    b2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2);
    b2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3);
    mfma_bf16x8 r;
    r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
    r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
    return r;
}

// RT: 16-row tiles per wave (logical); NSC: super-chunks (128 values of K)
// per wave, fixed so that all A loads are issued up front (0 = loop).
template <int EPI, int RT, int NSC>
RFP4_DEV void gemv_mfma_body(const GemvArgs &a)
{
    constexpr int NT = (EPI == RFP4_EPI_SWIGLU) ? 2 * RT : RT;
    extern __shared__ uint16_t planes[]; // [3][k] bf16
    __shared__ float red[4][NT * 16];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); // uniform: scalar branches
    const uint32_t rit = lane & 15, grp = lane >> 4;
    const uint32_t k = a.k, nsc = k >> 7, rowbytes = k >> 1, nblk = k >> 5;
    const uint32_t per_wave = (nsc + 3) / 4;
    const uint32_t sc0 = (uint32_t)wave * per_wave;

    const uint8_t *rowp[NT];
    const uint8_t *srow[NT];
#pragma unroll
    for (int tt = 0; tt < NT; tt++) {
        uint32_t lr = (blockIdx.x * RT + (uint32_t)(tt % RT)) * 16u + rit;
        uint32_t r = lr < a.n ? lr : a.n - 1;
        if (EPI == RFP4_EPI_SWIGLU && tt >= RT) r += a.pair_off;
        rowp[tt] = (const uint8_t *)a.w + (size_t)r * rowbytes + grp * 16u;
        srow[tt] = (const uint8_t *)a.scales + (size_t)r * nblk + grp;
    }

    // four independent accumulator chains per tile (one per MFMA of a
    // super-chunk), summed at the end
    mfma_f32x4 acc[NT][4];
#pragma unroll
    for (int tt = 0; tt < NT; tt++)
#pragma unroll
        for (int t = 0; t < 4; t++) acc[tt][t] = (mfma_f32x4){0.0f, 0.0f, 0.0f, 0.0f};

    // B fragment of MFMA t in super-chunk sc: plane `rit` (lanes 0..2 of each
    // row group), values 128*sc + 32*grp + 8*t .. +8; zero in other lanes.
    auto b_frag = [&](uint32_t sc, int t) -> mfma_bf16x8 {
        uint4 v = make_uint4(0, 0, 0, 0);
        if (rit < 3) v = *(const uint4 *)(planes + (size_t)rit * k + sc * 128u + grp * 32u + (uint32_t)t * 8u);
        return __builtin_bit_cast(mfma_bf16x8, v);
    };

    if (NSC > 0) {
        // 1) x (and norm weights) into registers, 2) every weight load of the
        // wave, 3) planes from registers: the staging never waits on weights.
        constexpr int XV = NSC > 0 ? (NSC + 1) / 2 : 1; // float4 of x per thread: K <= 512 * NSC
        const int tid = threadIdx.x;
        const bool norm = a.norm_w != nullptr;
        float4 xr[XV];
        uint2 wr[XV];
#pragma unroll
        for (int v = 0; v < XV; v++) {
            const uint32_t i4 = (uint32_t)tid + 256u * (uint32_t)v;
            const bool in = i4 < (k >> 2);
            xr[v] = in ? ((const float4 *)a.x)[i4] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            wr[v] = (in && norm) ? ((const uint2 *)a.norm_w)[i4] : make_uint2(0, 0);
        }
        uint4 q[NT][NSC > 0 ? NSC : 1];
        uint32_t sb[NT][NSC > 0 ? NSC : 1];
#pragma unroll
        for (int s = 0; s < NSC; s++) {
            const uint32_t sc = min(sc0 + (uint32_t)s, nsc - 1u);
#pragma unroll
            for (int tt = 0; tt < NT; tt++) {
                q[tt][s] = *(const uint4 *)(rowp[tt] + (size_t)sc * 64u);
                sb[tt][s] = srow[tt][(size_t)sc * 4u];
            }
        }
        stage_planes_regs<XV>(planes, xr, wr, k, norm, a.eps);
#pragma unroll
        for (int s = 0; s < NSC; s++) {
            const uint32_t sc = sc0 + (uint32_t)s;
            if ((uint32_t)s < per_wave && sc < nsc) { // wave-uniform
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    mfma_bf16x8 bf = b_frag(sc, t);
#pragma unroll
                    for (int tt = 0; tt < NT; tt++) {
                        const uint32_t w = t == 0 ? q[tt][s].x : t == 1 ? q[tt][s].y : t == 2 ? q[tt][s].z : q[tt][s].w;
                        acc[tt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            a_frag(w, __uint_as_float(sb[tt][s] << 23)), bf, acc[tt][t], 0, 0, 0);
                    }
                }
            }
        }
    } else {
        stage_planes(planes, a.x, k, a.norm_w, a.eps);
        for (uint32_t sc = sc0; sc < min(sc0 + per_wave, nsc); sc++) {
            uint4 q[NT];
            uint32_t sb[NT];
#pragma unroll
            for (int tt = 0; tt < NT; tt++) {
                q[tt] = *(const uint4 *)(rowp[tt] + (size_t)sc * 64u);
                sb[tt] = srow[tt][(size_t)sc * 4u];
            }
#pragma unroll
            for (int t = 0; t < 4; t++) {
                mfma_bf16x8 bf = b_frag(sc, t);
#pragma unroll
                for (int tt = 0; tt < NT; tt++) {
                    const uint32_t w = t == 0 ? q[tt].x : t == 1 ? q[tt].y : t == 2 ? q[tt].z : q[tt].w;
                    acc[tt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_frag(w, __uint_as_float(sb[tt] << 23)),
                                                                         bf, acc[tt][t], 0, 0, 0);
                }
            }
        }
    }

    // D[row][c] lives in lane 16*(row/4) + c, register row%4; sum columns
    // 0..3 (3 is zero) with two DPP steps, then lane 16g holds rows 4g..4g+3.
#pragma unroll
    for (int tt = 0; tt < NT; tt++) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float v = (acc[tt][0][r] + acc[tt][1][r]) + (acc[tt][2][r] + acc[tt][3][r]);
            v += dpp_mov<DPP_QUAD_1032>(v);
            v += dpp_mov<DPP_QUAD_2301>(v);
            if (rit == 0) red[wave][tt * 16 + grp * 4 + r] = v;
        }
    }
    __syncthreads();
    if (wave != 0) return;

    // lane i < 16*RT: logical row blockIdx.x*16*RT + i, waves summed in order
    const int i = lane;
    float yv = 0.0f, uv = 0.0f;
    uint32_t lr = blockIdx.x * RT * 16u + (uint32_t)i;
    bool ok = i < RT * 16 && lr < a.n;
    if (i < RT * 16) {
        yv = ((red[0][i] + red[1][i]) + red[2][i]) + red[3][i];
        if (EPI == RFP4_EPI_SWIGLU)
            uv = ((red[0][RT * 16 + i] + red[1][RT * 16 + i]) + red[2][RT * 16 + i]) + red[3][RT * 16 + i];
    }
    if (EPI == RFP4_EPI_ARGMAX) {
        unsigned long long key = ok && yv > -1e30f ? pack_argmax(yv, lr) : pack_argmax(-1e30f, 0u);
        if (ok) a.y[lr] = yv;
        for (int off = 32; off >= 1; off >>= 1) {
            unsigned long long o = __shfl_xor(key, off, 64);
            key = o > key ? o : key;
        }
        if (lane == 0) a.best[blockIdx.x] = key;
        return;
    }
    if (!ok) return;
    if (EPI == RFP4_EPI_STORE) {
        a.y[lr] = yv;
    } else if (EPI == RFP4_EPI_RESIDUAL) {
        a.y[lr] = __fadd_rn(a.y[lr], yv);
    } else {
        float g = yv;
        a.y[lr] = __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, expf(-g))), uv);
    }
}
