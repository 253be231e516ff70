// Device helpers shared by every gfx950 kernel of the engine.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../shared/kernel_args.h"

#define RFP4_DEV __device__ __forceinline__

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Non-temporal loads for data read once per launch (weights, KV rows): on
// MI355X a one-launch stream of 58.7 MB measured 10.4 us with them against
// 11.1 us with ordinary loads.
RFP4_DEV uint4 load_nt16(const void *p)
{
    const u32x4 v = __builtin_nontemporal_load((const u32x4 *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
RFP4_DEV uint32_t load_nt_u8(const uint8_t *p) { return __builtin_nontemporal_load(p); }
RFP4_DEV uint32_t load_nt_u32(const uint32_t *p) { return __builtin_nontemporal_load(p); }

// ---------------------------------------------------------------- wave64 reductions
// DPP controls (GCN/CDNA encoding).
#define DPP_QUAD_1032 0xB1   // quad_perm [1,0,3,2]
#define DPP_QUAD_2301 0x4E   // quad_perm [2,3,0,1]
#define DPP_ROW_MIRROR 0x140
#define DPP_ROW_HALF_MIRROR 0x141
#define DPP_ROW_ROR8 0x128   // row_ror:8 = lane ^ 8 within a row of 16


template <int CTRL>
RFP4_DEV float dpp_mov(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over the 16 lanes of each DPP row; every lane of the row gets the sum.
RFP4_DEV float row16_sum(float v)
{
    v += dpp_mov<DPP_QUAD_1032>(v);
    v += dpp_mov<DPP_QUAD_2301>(v);
    v += dpp_mov<DPP_ROW_HALF_MIRROR>(v);
    v += dpp_mov<DPP_ROW_MIRROR>(v);
    return v;
}

// v + v(lane ^ 16) and v + v(lane ^ 32) on the gfx950 row-swap
// instructions (no LDS round trip).  permlane16_swap(v, v) returns v with odd
// rows replaced by the even row below and v with even rows replaced by the
// odd row above; the sum of the pair is v + v^16 in every lane (pinned on the
// device), likewise permlane32_swap for the two halves of the wave.
RFP4_DEV float xor16_sum(float v)
{
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

RFP4_DEV float xor32_sum(float v)
{
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

RFP4_DEV float xor16_max(float v)
{
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}

RFP4_DEV float xor32_max(float v)
{
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}

// Max over the 16 lanes of each DPP row; every lane of the row gets it.
RFP4_DEV float row16_max(float v)
{
    v = fmaxf(v, dpp_mov<DPP_QUAD_1032>(v));
    v = fmaxf(v, dpp_mov<DPP_QUAD_2301>(v));
    v = fmaxf(v, dpp_mov<DPP_ROW_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_mov<DPP_ROW_MIRROR>(v));
    return v;
}

// Sum over all 64 lanes; every lane gets the total.
RFP4_DEV float wave_sum(float v)
{
    return xor32_sum(xor16_sum(row16_sum(v)));
}


RFP4_DEV float wave_max(float v)
{
    v = fmaxf(v, dpp_mov<DPP_QUAD_1032>(v));
    v = fmaxf(v, dpp_mov<DPP_QUAD_2301>(v));
    v = fmaxf(v, dpp_mov<DPP_ROW_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_mov<DPP_ROW_MIRROR>(v));
    return xor32_max(xor16_max(v));
}

// ---------------------------------------------------------------- fp16 matrix-core operands
// v_mfma_f32_16x16x32_f16 operands: lane l holds A row / B column l % 16 and
// K = 8 (l / 16) .. +7; accumulator r of lane l is D[4 (l / 16) + r][l % 16]
// (pinned by the fp16 layout test).
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// x -> hi + lo, both fp16 (hi = fp16(x), lo = fp16(x - hi); x - hi is exact):
// about 2^-22 relative with two matrix-core products per operand
RFP4_DEV void split_hi_lo8(const float *v, f16x8 &hi, f16x8 &lo)
{
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const _Float16 h = (_Float16)v[i];
        hi[i] = h;
        lo[i] = (_Float16)(v[i] - (float)h);
    }
}

// The same split in three instructions per pair of values: hi by the packed
// conversion, lo = fp16(v - hi) by v_fma_mix{lo,hi}_f16 (v * 1.0 + -hi with
// hi taken as an fp16 half, one rounding of the exact difference: the same
// bits as split_hi_lo8).
RFP4_DEV void split_hi_lo8_mix(const float *v, f16x8 &hi, f16x8 &lo)
{
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
    u32x4v hw, lw;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){v[2 * j], v[2 * j + 1]}, f16x2));
        uint32_t l;
        asm("v_fma_mixlo_f16 %0, %1, 1.0, -%2 op_sel_hi:[0,0,1]" : "=v"(l) : "v"(v[2 * j]), "v"(h));
        asm("v_fma_mixhi_f16 %0, %1, 1.0, -%2 op_sel:[0,0,1] op_sel_hi:[0,0,1]" : "+v"(l) : "v"(v[2 * j + 1]), "v"(h));
        hw[j] = h;
        lw[j] = l;
    }
    hi = __builtin_bit_cast(f16x8, hw);
    lo = __builtin_bit_cast(f16x8, lw);
}

// ---------------------------------------------------------------- E2M1 / E8M0
// Two E2M1 codes of byte SEL of w -> (low nibble, high nibble) as f32, via the
// gfx950 hardware conversion (scale 1.0, so the value is the plain code value).
template <int SEL>
RFP4_DEV f32x2 fp4x2_to_f32(uint32_t w)
{
    return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, SEL);
}

// E8M0 byte -> f32 2^(b-127), exact including b = 0 (2^-127, subnormal) and
// b = 0xFF (NaN).
RFP4_DEV float e8m0_to_f32(uint32_t b)
{
    uint32_t bits = b == 0u ? 0x00400000u : (b == 0xFFu ? 0x7FC00000u : (b << 23));
    return __uint_as_float(bits);
}

// sum_{i<32} fp4(q_i) * x_i for one 16-byte chunk (32 codes, low nibble first)
// against 32 consecutive activations.  Two partial chains for ILP.
RFP4_DEV float dot_chunk32(const uint4 q, const float4 *xv)
{
    float s0 = 0.0f, s1 = 0.0f;
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const float4 xa = xv[2 * d], xb = xv[2 * d + 1];
        f32x2 v0 = fp4x2_to_f32<0>(w[d]);
        f32x2 v1 = fp4x2_to_f32<1>(w[d]);
        f32x2 v2 = fp4x2_to_f32<2>(w[d]);
        f32x2 v3 = fp4x2_to_f32<3>(w[d]);
        s0 = fmaf(v0.x, xa.x, s0);
        s1 = fmaf(v0.y, xa.y, s1);
        s0 = fmaf(v1.x, xa.z, s0);
        s1 = fmaf(v1.y, xa.w, s1);
        s0 = fmaf(v2.x, xb.x, s0);
        s1 = fmaf(v2.y, xb.y, s1);
        s0 = fmaf(v3.x, xb.z, s0);
        s1 = fmaf(v3.y, xb.w, s1);
    }
    return s0 + s1;
}

// ---------------------------------------------------------------- synthetic init RNG
// Counter-based SplitMix64 finalizer over (seed, stream, index); pure u64
// arithmetic so host generators produce identical values.
RFP4_DEV uint64_t mix64(uint64_t seed, uint64_t stream, uint64_t index)
{
    uint64_t z = seed + 0x9E3779B97F4A7C15ull * (index + 1ull) + 0xD1342543DE82EF95ull * stream;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Irwin-Hall(4) normal: centred sum of the four 16-bit fields, times coef
// (coef = sigma / sqrt((65536^2-1)/3), computed on the host).
RFP4_DEV float ih4_normal(uint64_t r, float coef)
{
    int32_t s = (int32_t)(r & 0xFFFFu) + (int32_t)((r >> 16) & 0xFFFFu) + (int32_t)((r >> 32) & 0xFFFFu) +
                (int32_t)((r >> 48) & 0xFFFFu) - 2 * 65535;
    return __fmul_rn((float)s, coef);
}

// IEEE f32 -> f16 bits, round to nearest even (hardware conversion).
RFP4_DEV uint16_t f32_to_f16_bits(float f)
{
    _Float16 h = (_Float16)f;
    return __builtin_bit_cast(uint16_t, h);
}

RFP4_DEV float f16_bits_to_f32(uint16_t b)
{
    return (float)__builtin_bit_cast(_Float16, b);
}

// bf16 bits -> f32 (exact: the upper half of the f32 pattern)
RFP4_DEV float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// A 16-bit norm weight or embedding element, stored as bf16 or fp16: exact.
RFP4_DEV float half_bits_to_f32(uint32_t b, bool bf16)
{
    return bf16 ? bf16_bits_to_f32(b & 0xFFFFu) : f16_bits_to_f32((uint16_t)b);
}

// Orderable key of a float for unsigned max-reduction (NaN excluded by callers).
RFP4_DEV uint32_t float_order_key(float f)
{
    uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

RFP4_DEV float float_from_order_key(uint32_t k)
{
    uint32_t u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
    return __uint_as_float(u);
}

// (value, index) packed so that u64 max picks the larger value and, on ties,
// the smaller index.
RFP4_DEV uint64_t pack_argmax(float v, uint32_t idx)
{
    return ((uint64_t)float_order_key(v) << 32) | (uint64_t)(0xFFFFFFFFu - idx);
}
