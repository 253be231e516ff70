// gfx950 block-scaled MFMA tiles (v_mfma_scale_f32_*_f8f6f4, E2M1 operands,
// E8M0 scales): the CDNA4 counterpart of the reference's m16n8k64
// mma.sync ... kind::mxf4.block_scale tile (fp4_mma/src/main.rs:18-54,
// trackb/FP4_M16N8K64_LAYOUT.md).
#pragma once
#include "common.h"

typedef int v8i32 __attribute__((ext_vector_type(8)));
typedef float v4f32 __attribute__((ext_vector_type(4)));
typedef float v16f32 __attribute__((ext_vector_type(16)));

#define MX_FMT_FP4 4

// One 16x16x128 MXFP4 MFMA from raw per-lane registers (layout pinning):
// a, b: 8 dwords per lane (E2M1 uses the first 4); sa, sb: one dword per lane
// (byte 0 is used); out: 4 floats per lane, the raw accumulator registers.
RFP4_DEV void mma16_tile_body(const MmaTileArgs &a)
{
    const int lane = threadIdx.x & 63;
    v8i32 av, bv;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        av[j] = (int)a.a[lane * 8 + j];
        bv[j] = (int)a.b[lane * 8 + j];
    }
    v4f32 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, acc, MX_FMT_FP4, MX_FMT_FP4, 0, (int)a.sa[lane], 0,
                                                           (int)a.sb[lane]);
#pragma unroll
    for (int r = 0; r < 4; r++) a.out[lane * 4 + r] = acc[r];
}

// Same for the 32x32x64 shape: 16 accumulator floats per lane.
RFP4_DEV void mma32_tile_body(const MmaTileArgs &a)
{
    const int lane = threadIdx.x & 63;
    v8i32 av, bv;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        av[j] = (int)a.a[lane * 8 + j];
        bv[j] = (int)a.b[lane * 8 + j];
    }
    v16f32 acc;
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0.0f;
    acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, acc, MX_FMT_FP4, MX_FMT_FP4, 0, (int)a.sa[lane], 0,
                                                          (int)a.sb[lane]);
#pragma unroll
    for (int r = 0; r < 16; r++) a.out[lane * 16 + r] = acc[r];
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

// One v_mfma_f32_16x16x32_bf16 (mode 0) or v_mfma_f32_16x16x32_f16 (mode 1)
// from raw per-lane registers: a, b hold 4 dwords (8 bf16 / fp16) per lane;
// out receives the 4 accumulator floats per lane.
RFP4_DEV void mma_bf16_tile_body(const MmaTileArgs &a)
{
    const int lane = threadIdx.x & 63;
    uint4 ar = ((const uint4 *)a.a)[lane], br = ((const uint4 *)a.b)[lane];
    v4f32 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    if (a.mode == 1) { // fp16 operands: v_mfma_f32_16x16x32_f16
        const f16x8_t av = __builtin_bit_cast(f16x8_t, ar), bv = __builtin_bit_cast(f16x8_t, br);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc, 0, 0, 0);
    } else {
        const bf16x8_t av = __builtin_bit_cast(bf16x8_t, ar), bv = __builtin_bit_cast(bf16x8_t, br);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 4; r++) a.out[lane * 4 + r] = acc[r];
}

// All-ones known answer (fp4_mma/src/main.rs:24-31): A = B = 1.0 (E2M1 0x2)
// over K = 128 with the A scale 2^-1 (E8M0 0x7E) and B scale 1.0 (0x7F), so
// every element is 128 * 0.5 = 64.0, the reference's expected value.  Writes
// the 16x8 corner D[i][j], i < 16, j < 8, row-major (128 floats).
RFP4_DEV void mma_allones_body(float *out)
{
    const int lane = threadIdx.x & 63;
    v8i32 av, bv;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        av[j] = j < 4 ? 0x22222222 : 0;
        bv[j] = j < 4 ? 0x22222222 : 0;
    }
    v4f32 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, acc, MX_FMT_FP4, MX_FMT_FP4, 0, 0x7E7E7E7E, 0,
                                                           0x7F7F7F7F);
    // The MFMA reads the operand registers of all 64 lanes whatever EXEC is;
    // consuming its result here keeps the compiler from sinking it (and the
    // operand set-up) into the divergent store below.
    asm volatile("" ::"v"(acc[0]), "v"(acc[1]), "v"(acc[2]), "v"(acc[3]));
    const int col = lane & 15, rb = (lane >> 4) * 4;
    if (col < 8)
#pragma unroll
        for (int r = 0; r < 4; r++) out[(rb + r) * 8 + col] = acc[r];
}
