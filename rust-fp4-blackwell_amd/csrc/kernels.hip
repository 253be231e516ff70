// All gfx950 kernels of the engine, compiled into one code object
// (hipcc --genco --offload-arch=gfx950) that the host runtime embeds and
// loads with hipModuleLoadData.  Every kernel takes one argument block by
// value (shared/kernel_args.h).
#include "device/common.h"
#include "device/gemv.h"
#include "device/norm_rope.h"
#include "device/attn.h"
#include "device/misc.h"
#include "device/mma.h"
#include "device/gemm.h"
#include "device/gemm_rows.h"
#include "device/prefill.h"
#include "device/attn_prefill.h"
#include "device/persist.h"
#include "device/qkva.h"

#define K256 extern "C" __global__ __launch_bounds__(256)
#define K512 extern "C" __global__ __launch_bounds__(512)
#define K1024 extern "C" __global__ __launch_bounds__(1024)

// ---- GEMV: rfp4_gemv_<scale>_<epilogue>_r<R>_s<NS>
// (R rows per wave, NS = K/2048 slices issued up front, 0 = any K).  The host
// selects among these (runtime.cpp gemv_variant); keep the two lists in sync.
#define GEMV_KERNEL(SNAME, SF32, ENAME, EPI, R, NS) \
    K256 void rfp4_gemv_##SNAME##_##ENAME##_r##R##_s##NS(GemvArgs a) { gemv_body<SF32, EPI, R, NS>(a); }
#define GEMV_NS_FULL(SNAME, SF32, ENAME, EPI, R) \
    GEMV_KERNEL(SNAME, SF32, ENAME, EPI, R, 0) \
    GEMV_KERNEL(SNAME, SF32, ENAME, EPI, R, 1) \
    GEMV_KERNEL(SNAME, SF32, ENAME, EPI, R, 2) \
    GEMV_KERNEL(SNAME, SF32, ENAME, EPI, R, 3) \
    GEMV_KERNEL(SNAME, SF32, ENAME, EPI, R, 4) \
    GEMV_KERNEL(SNAME, SF32, ENAME, EPI, R, 7)
#define GEMV_NS_SHORT(SNAME, SF32, ENAME, EPI, R) \
    GEMV_KERNEL(SNAME, SF32, ENAME, EPI, R, 0) \
    GEMV_KERNEL(SNAME, SF32, ENAME, EPI, R, 1) \
    GEMV_KERNEL(SNAME, SF32, ENAME, EPI, R, 2)

GEMV_NS_FULL(e8m0, 0, store, RFP4_EPI_STORE, 1)
GEMV_NS_FULL(e8m0, 0, store, RFP4_EPI_STORE, 2)
GEMV_NS_FULL(e8m0, 0, store, RFP4_EPI_STORE, 4)
GEMV_NS_SHORT(e8m0, 0, store, RFP4_EPI_STORE, 8)
GEMV_NS_FULL(e8m0, 0, resid, RFP4_EPI_RESIDUAL, 1)
GEMV_NS_FULL(e8m0, 0, resid, RFP4_EPI_RESIDUAL, 2)
GEMV_NS_FULL(e8m0, 0, resid, RFP4_EPI_RESIDUAL, 4)
GEMV_NS_SHORT(e8m0, 0, resid, RFP4_EPI_RESIDUAL, 8)
GEMV_NS_FULL(e8m0, 0, argmax, RFP4_EPI_ARGMAX, 2)
GEMV_NS_FULL(e8m0, 0, argmax, RFP4_EPI_ARGMAX, 4)
GEMV_NS_SHORT(e8m0, 0, argmax, RFP4_EPI_ARGMAX, 8)
GEMV_NS_FULL(e8m0, 0, swiglu, RFP4_EPI_SWIGLU, 1)
GEMV_NS_FULL(e8m0, 0, swiglu, RFP4_EPI_SWIGLU, 2)
// gate/up at R=4: capped at 128 VGPRs (4 waves per SIMD) so that every
// workgroup of the 8B shape (896) is resident at once
#define GEMV_KERNEL_OCC4(SNAME, SF32, ENAME, EPI, R, NS) \
    extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void \
        rfp4_gemv_##SNAME##_##ENAME##_r##R##_s##NS(GemvArgs a) { gemv_body<SF32, EPI, R, NS>(a); }
GEMV_KERNEL_OCC4(e8m0, 0, swiglu, RFP4_EPI_SWIGLU, 4, 0)
GEMV_KERNEL_OCC4(e8m0, 0, swiglu, RFP4_EPI_SWIGLU, 4, 1)
GEMV_KERNEL_OCC4(e8m0, 0, swiglu, RFP4_EPI_SWIGLU, 4, 2)
GEMV_KERNEL(e8m0, 0, swiglu, RFP4_EPI_SWIGLU, 4, 3) // 128 VGPRs would spill
// f32 per-32 scales (the reference's format, fp4_gemv/src/main.rs:32-92):
// the variants the planner picks (runtime.cpp gemv_variant)
GEMV_NS_FULL(f32, 1, store, RFP4_EPI_STORE, 2)
GEMV_NS_SHORT(f32, 1, store, RFP4_EPI_STORE, 8)
GEMV_NS_FULL(f32, 1, resid, RFP4_EPI_RESIDUAL, 2)
GEMV_NS_SHORT(f32, 1, resid, RFP4_EPI_RESIDUAL, 8)
GEMV_NS_FULL(f32, 1, argmax, RFP4_EPI_ARGMAX, 2)
GEMV_NS_SHORT(f32, 1, argmax, RFP4_EPI_ARGMAX, 8)
GEMV_NS_FULL(f32, 1, swiglu, RFP4_EPI_SWIGLU, 1)
// 8 waves per workgroup for one-slice shapes (K <= 2048) and the 1-row
// residual GEMVs of one and three slices, the default there (runtime.cpp
// gemv_variant): TinyLlama decode 1811 -> 1836 tok/s, then 2307 -> 2338 with
// the residual ones; at K = 4096 and 14336 slower (8B down at 1 row per wave
// on 8 waves: 686 -> 661 tok/s).  rfp4_gemv_<scale>_<epilogue>_r<R>_s<NS>_w<W>
#define GEMV_KERNEL_W(SNAME, SF32, ENAME, EPI, R, NS, W)                                                         \
    extern "C" __global__ __launch_bounds__(64 * W) void rfp4_gemv_##SNAME##_##ENAME##_r##R##_s##NS##_w##W(GemvArgs a) \
    {                                                                                                           \
        gemv_body<SF32, EPI, R, NS, W>(a);                                                                      \
    }
GEMV_KERNEL_W(e8m0, 0, swiglu, RFP4_EPI_SWIGLU, 1, 1, 8)
GEMV_KERNEL_W(e8m0, 0, store, RFP4_EPI_STORE, 2, 1, 8)
GEMV_KERNEL_W(f32, 1, swiglu, RFP4_EPI_SWIGLU, 1, 1, 8)
GEMV_KERNEL_W(f32, 1, store, RFP4_EPI_STORE, 2, 1, 8)
GEMV_KERNEL_W(e8m0, 0, resid, RFP4_EPI_RESIDUAL, 1, 1, 8)
GEMV_KERNEL_W(e8m0, 0, resid, RFP4_EPI_RESIDUAL, 1, 3, 8)

// ---- norm / rope / embed
K1024 void rfp4_rmsnorm_f32w(RmsnormArgs a) { rmsnorm_body<0>(a); }
K1024 void rfp4_rmsnorm_f16w(RmsnormArgs a) { rmsnorm_body<1>(a); }
K256 void rfp4_rope(RopeArgs a) { rope_body(a); }
K256 void rfp4_embed(EmbedArgs a) { embed_body(a); }

// ---- attention: rfp4_attn_hd<HD>_<KV type>_g<query heads per KV head, padded to 1/2/4/8>[_t: tagged merge]
#define ATTN_KERNELS(HD, KNAME, KT) \
    K256 void rfp4_attn_hd##HD##_##KNAME##_g1(AttnArgs a) { attn_body<HD, KT, 1>(a); } \
    K256 void rfp4_attn_hd##HD##_##KNAME##_g2(AttnArgs a) { attn_body<HD, KT, 2>(a); } \
    K256 void rfp4_attn_hd##HD##_##KNAME##_g4(AttnArgs a) { attn_body<HD, KT, 4>(a); } \
    K256 void rfp4_attn_hd##HD##_##KNAME##_g8(AttnArgs a) { attn_body<HD, KT, 8>(a); } \
    K256 void rfp4_attn_hd##HD##_##KNAME##_g1_t(AttnArgs a) { attn_body<HD, KT, 1, true>(a); } \
    K256 void rfp4_attn_hd##HD##_##KNAME##_g2_t(AttnArgs a) { attn_body<HD, KT, 2, true>(a); } \
    K256 void rfp4_attn_hd##HD##_##KNAME##_g4_t(AttnArgs a) { attn_body<HD, KT, 4, true>(a); } \
    K256 void rfp4_attn_hd##HD##_##KNAME##_g8_t(AttnArgs a) { attn_body<HD, KT, 8, true>(a); }
ATTN_KERNELS(64, f32, float)
ATTN_KERNELS(64, f16, uint16_t)
ATTN_KERNELS(128, f32, float)
ATTN_KERNELS(128, f16, uint16_t)
// rfp4_attn_prefill_hd<HD>_g<group>_w<waves per workgroup>[_q: the output
// rows quantized to MXFP4 as well, AttnPrefillArgs::q_codes]
#define K512Q extern "C" __global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
#define ATTN_PREFILL_KERNELS(HD) \
    K256 void rfp4_attn_prefill_hd##HD##_g1_w4(AttnPrefillArgs a) { attn_prefill_body<HD, 1, 4>(a); } \
    K256 void rfp4_attn_prefill_hd##HD##_g2_w4(AttnPrefillArgs a) { attn_prefill_body<HD, 2, 4>(a); } \
    K256 void rfp4_attn_prefill_hd##HD##_g4_w4(AttnPrefillArgs a) { attn_prefill_body<HD, 4, 4>(a); } \
    K256 void rfp4_attn_prefill_hd##HD##_g8_w4(AttnPrefillArgs a) { attn_prefill_body<HD, 8, 4>(a); } \
    K512 void rfp4_attn_prefill_hd##HD##_g1_w8(AttnPrefillArgs a) { attn_prefill_body<HD, 1, 8>(a); } \
    K512 void rfp4_attn_prefill_hd##HD##_g2_w8(AttnPrefillArgs a) { attn_prefill_body<HD, 2, 8>(a); } \
    K512 void rfp4_attn_prefill_hd##HD##_g4_w8(AttnPrefillArgs a) { attn_prefill_body<HD, 4, 8>(a); } \
    K512 void rfp4_attn_prefill_hd##HD##_g8_w8(AttnPrefillArgs a) { attn_prefill_body<HD, 8, 8>(a); } \
    K256 void rfp4_attn_prefill_hd##HD##_g1_w4_q(AttnPrefillArgs a) { attn_prefill_body<HD, 1, 4, true>(a); } \
    K256 void rfp4_attn_prefill_hd##HD##_g2_w4_q(AttnPrefillArgs a) { attn_prefill_body<HD, 2, 4, true>(a); } \
    K256 void rfp4_attn_prefill_hd##HD##_g4_w4_q(AttnPrefillArgs a) { attn_prefill_body<HD, 4, 4, true>(a); } \
    K256 void rfp4_attn_prefill_hd##HD##_g8_w4_q(AttnPrefillArgs a) { attn_prefill_body<HD, 8, 4, true>(a); } \
    K512Q void rfp4_attn_prefill_hd##HD##_g1_w8_q(AttnPrefillArgs a) { attn_prefill_body<HD, 1, 8, true>(a); } \
    K512Q void rfp4_attn_prefill_hd##HD##_g2_w8_q(AttnPrefillArgs a) { attn_prefill_body<HD, 2, 8, true>(a); } \
    K512Q void rfp4_attn_prefill_hd##HD##_g4_w8_q(AttnPrefillArgs a) { attn_prefill_body<HD, 4, 8, true>(a); } \
    K512Q void rfp4_attn_prefill_hd##HD##_g8_w8_q(AttnPrefillArgs a) { attn_prefill_body<HD, 8, 8, true>(a); }
ATTN_PREFILL_KERNELS(64)
ATTN_PREFILL_KERNELS(128)
// key-split variants (two key groups of 4 waves each, _s2; groups of up to 4
// query heads: runtime.cpp attn_prefill_launch)
#define ATTN_PREFILL_SPLIT_KERNELS(HD) \
    K512 void rfp4_attn_prefill_hd##HD##_g1_w4_s2(AttnPrefillArgs a) { attn_prefill_body<HD, 1, 4, false, 2>(a); } \
    K512 void rfp4_attn_prefill_hd##HD##_g2_w4_s2(AttnPrefillArgs a) { attn_prefill_body<HD, 2, 4, false, 2>(a); } \
    K512 void rfp4_attn_prefill_hd##HD##_g4_w4_s2(AttnPrefillArgs a) { attn_prefill_body<HD, 4, 4, false, 2>(a); } \
    K512Q void rfp4_attn_prefill_hd##HD##_g1_w4_q_s2(AttnPrefillArgs a) { attn_prefill_body<HD, 1, 4, true, 2>(a); } \
    K512Q void rfp4_attn_prefill_hd##HD##_g2_w4_q_s2(AttnPrefillArgs a) { attn_prefill_body<HD, 2, 4, true, 2>(a); } \
    K512Q void rfp4_attn_prefill_hd##HD##_g4_w4_q_s2(AttnPrefillArgs a) { attn_prefill_body<HD, 4, 4, true, 2>(a); }
ATTN_PREFILL_SPLIT_KERNELS(64)
ATTN_PREFILL_SPLIT_KERNELS(128)
#undef ATTN_PREFILL_SPLIT_KERNELS
// ---- fused q|k|v GEMV + attention: rfp4_qkva_hd<HD>_g<group>[_t: tagged merge]
// (device/qkva.h).  HD 64 with K = 2048 (one slice, R = 2 or 1 (_r1), the
// 8-wave GEMV's RMS order); HD 128 with K = 4096 (two slices, R = 4, the
// 4-wave order).
// The host checks the engine's shape against these (engine.cpp qkva_plan).
#define QKVA_KERNELS(HD, NS, R, WREF, SFX) \
    K256 void rfp4_qkva_hd##HD##_g1##SFX(QkvaArgs a) { qkva_body<HD, 1, false, NS, R, WREF>(a); } \
    K256 void rfp4_qkva_hd##HD##_g2##SFX(QkvaArgs a) { qkva_body<HD, 2, false, NS, R, WREF>(a); } \
    K256 void rfp4_qkva_hd##HD##_g4##SFX(QkvaArgs a) { qkva_body<HD, 4, false, NS, R, WREF>(a); } \
    K256 void rfp4_qkva_hd##HD##_g8##SFX(QkvaArgs a) { qkva_body<HD, 8, false, NS, R, WREF>(a); } \
    K256 void rfp4_qkva_hd##HD##_g1_t##SFX(QkvaArgs a) { qkva_body<HD, 1, true, NS, R, WREF>(a); } \
    K256 void rfp4_qkva_hd##HD##_g2_t##SFX(QkvaArgs a) { qkva_body<HD, 2, true, NS, R, WREF>(a); } \
    K256 void rfp4_qkva_hd##HD##_g4_t##SFX(QkvaArgs a) { qkva_body<HD, 4, true, NS, R, WREF>(a); } \
    K256 void rfp4_qkva_hd##HD##_g8_t##SFX(QkvaArgs a) { qkva_body<HD, 8, true, NS, R, WREF>(a); }
QKVA_KERNELS(64, 1, 2, 8, )
QKVA_KERNELS(128, 2, 4, 4, )
// HD 64 with 1 row per wave (twice the GEMV tiles), used where its grid
// still fits the device at once: TinyLlama decode 2306 -> 2334 tok/s
QKVA_KERNELS(64, 1, 1, 8, _r1)
K256 void rfp4_attn_merge_hd64(AttnArgs a) { attn_merge_body<64>(a); }
K256 void rfp4_attn_merge_hd128(AttnArgs a) { attn_merge_body<128>(a); }

// ---- misc
K256 void rfp4_fill(FillArgs a) { fill_body(a); }
K256 void rfp4_copy_into_f32(CopyArgs a) { copy_into_body<0>(a); }
K256 void rfp4_copy_into_f16(CopyArgs a) { copy_into_body<1>(a); }
K256 void rfp4_swiglu(EltwiseArgs a) { swiglu_body(a); }
K256 void rfp4_residual(EltwiseArgs a) { residual_body(a); }
K1024 void rfp4_argmax(ArgmaxArgs a) { argmax_body(a); }
K1024 void rfp4_step(StepArgs a) { step_body(a); }
K256 void rfp4_synth_weight(SynthWeightArgs a) { synth_weight_body(a); }
K256 void rfp4_synth_f16(SynthF16Args a) { synth_f16_body(a); }
K256 void rfp4_synth_kv(SynthKvArgs a) { synth_kv_body(a); }
// fp4_pack2 (the hardware conversion every quantizer uses) against
// e2m1_rne_code(ldexpf(v, -se)) on every f32 bit pattern (the values a block
// of shared exponent se holds, |v| < 2^(se + 3), and all others: saturation,
// infinities, NaNs), se = se0 + blockIdx.y: v in the low nibble and -v in the
// high one.  tested counts the patterns below 2^(se + 3).  One atomic pair
// per thread.
K256 void rfp4_fp4_encode_check(Fp4CheckArgs a)
{
    const int se = a.se0 + (int)blockIdx.y;
    const float sc = ldexpf(1.0f, se), lim = ldexpf(1.0f, se + 3);
    unsigned long long mis = 0, nt = 0;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t u = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; u < (1ull << 32); u += stride) {
        const float v = __uint_as_float((uint32_t)u), w = __uint_as_float((uint32_t)u ^ 0x80000000u);
        nt += fabsf(v) < lim ? 1ull : 0ull;
        const uint32_t sw = e2m1_rne_code(ldexpf(v, -se)) | e2m1_rne_code(ldexpf(w, -se)) << 4;
        mis += fp4_pack2<0>(0u, v, w, sc) != sw ? 1ull : 0ull;
    }
    if (mis) atomicAdd(&a.mismatches[blockIdx.y], mis);
    if (nt) atomicAdd(&a.tested[blockIdx.y], nt);
}
K256 void rfp4_quant_mx_f32(QuantMxArgs a) { quant_mx_body<0>(a); }
K256 void rfp4_quant_mx_bf16(QuantMxArgs a) { quant_mx_body<1>(a); }
K256 void rfp4_selftest_cvt(SelftestArgs a) { selftest_cvt_body(a); }

// ---- MFMA tiles
K256 void rfp4_mma16_tile(MmaTileArgs a) { mma16_tile_body(a); }
K256 void rfp4_mma32_tile(MmaTileArgs a) { mma32_tile_body(a); }
K256 void rfp4_mma_allones(MmaTileArgs a) { mma_allones_body(a.out); }
K256 void rfp4_mma_bf16_tile(MmaTileArgs a) { mma_bf16_tile_body(a); }

// ---- batched MXFP4 GEMM: rfp4_gemm_<BM>x<BN> (4 waves in WM x WN, wave tile 32FA x 32FB).
// The host picks among these (runtime.cpp gemm_plan); keep the lists in sync.
// Tiles whose two register sets of operands fit beside the accumulators run
// the pipelined K loop (the next step's LDS reads under this step's MFMAs);
// the 256x256 tile (8 fragments per wave) keeps the serial one.
#define GEMM_PIPE(FA, FB) ((FA) + (FB) <= 6)
#define GEMM_KERNEL(BM, BN, WM, WN, FA, FB) \
    K256 void rfp4_gemm_##BM##x##BN(GemmArgs a) { gemm_body<WM, WN, FA, FB, 2, GEMM_PIPE(FA, FB)>(a); }
GEMM_KERNEL(32, 128, 1, 4, 1, 1)
GEMM_KERNEL(64, 128, 2, 2, 1, 2)
GEMM_KERNEL(128, 128, 2, 2, 2, 2)
GEMM_KERNEL(256, 128, 2, 2, 4, 2)
GEMM_KERNEL(256, 256, 2, 2, 4, 4)
// deeper DMA pipelines (NST stages, NST - 1 steps of lookahead) for the
// small tiles: rfp4_gemm_<BM>x<BN>_p<NST>
#define GEMM_KERNEL_P(BM, BN, WM, WN, FA, FB, NST) \
    K256 void rfp4_gemm_##BM##x##BN##_p##NST(GemmArgs a) { gemm_body<WM, WN, FA, FB, NST, GEMM_PIPE(FA, FB)>(a); }
GEMM_KERNEL_P(32, 128, 1, 4, 1, 1, 4)
GEMM_KERNEL_P(64, 128, 2, 2, 1, 2, 4)
GEMM_KERNEL_P(64, 128, 2, 2, 1, 2, 3)
GEMM_KERNEL_P(128, 128, 2, 2, 2, 2, 3)
GEMM_KERNEL_P(256, 128, 2, 2, 4, 2, 3)
// 8-wave ping-pong tiles (two waves per SIMD, one computing while the other
// copies and reads): rfp4_gemm_<BM>x<BN>_pp, wave tile 32FA x 32FB
#define GEMM_KERNEL_PP(BM, BN, FA, FB) \
    K512 void rfp4_gemm_##BM##x##BN##_pp(GemmArgs a) { gemm_pp_body<FA, FB>(a); }
GEMM_KERNEL_PP(256, 256, 4, 2)
GEMM_KERNEL_PP(256, 128, 4, 1)
// the prefill's gate|up projection with SwiGLU and the MXFP4 rows of its
// output in the epilogue (GemmArgs::q_codes)
K512 void rfp4_gemm_256x256_ppsw(GemmArgs a) { gemm_pp_body<4, 2, 1>(a); }
// the same epilogue on the 4-wave 128x128 tile (64 output columns per tile)
K256 void rfp4_gemm_128x128_sw(GemmArgs a) { gemm_body<2, 2, 2, 2, 2, GEMM_PIPE(2, 2), false, true>(a); }
K256 void rfp4_gemm_128x128_p3_sw(GemmArgs a) { gemm_body<2, 2, 2, 2, 3, GEMM_PIPE(2, 2), false, true>(a); }
// the prefill's q|k|v projection with RoPE and the fp16 K/V cache rows in
// the epilogue (GemmArgs::rope_cos): the 4-wave tiles up to 128 rows and the
// ping-pong 256x256 (a 256x128 variant measured slower than the GEMM + the
// row kernel: TinyLlama 2048 rows 28.5 against 16.8 + 9.6 us)
#define GEMM_KERNEL_ROPE(BM, BN, WM, WN, FA, FB) \
    K256 void rfp4_gemm_##BM##x##BN##_rope(GemmArgs a) { gemm_body<WM, WN, FA, FB, 2, GEMM_PIPE(FA, FB), true>(a); }
#define GEMM_KERNEL_P_ROPE(BM, BN, WM, WN, FA, FB, NST) \
    K256 void rfp4_gemm_##BM##x##BN##_p##NST##_rope(GemmArgs a) { gemm_body<WM, WN, FA, FB, NST, GEMM_PIPE(FA, FB), true>(a); }
GEMM_KERNEL_ROPE(32, 128, 1, 4, 1, 1)
GEMM_KERNEL_ROPE(64, 128, 2, 2, 1, 2)
GEMM_KERNEL_ROPE(128, 128, 2, 2, 2, 2)
GEMM_KERNEL_P_ROPE(32, 128, 1, 4, 1, 1, 4)
GEMM_KERNEL_P_ROPE(64, 128, 2, 2, 1, 2, 4)
GEMM_KERNEL_P_ROPE(64, 128, 2, 2, 1, 2, 3)
GEMM_KERNEL_P_ROPE(128, 128, 2, 2, 2, 2, 3)
K512 void rfp4_gemm_256x256_pp_rope(GemmArgs a) { gemm_pp_body<4, 2, 2>(a); }
K256 void rfp4_gemm_reduce(GemmArgs a) { gemm_reduce_body(a); }
// row-major E8M0 scales -> the step-blocked copy the tiled kernels read
K256 void rfp4_scales_tile(ScaleTileArgs a) { scales_tile_body(a); }
// few activation rows (M <= 16 MB) x 16 NF W rows per workgroup, up to 8
// waves of up to SEG K segments of 512 each (device/gemm_rows.h):
// rfp4_gemm_rows_m<16 MB>_s<SEG>_f<NF>, the combinations whose loads fit the
// registers (runtime.cpp gemm_rows_has); keep the two lists in sync.
#define GEMM_ROWS_KERNEL(M, MB, SEG, NF) \
    K512 void rfp4_gemm_rows_m##M##_s##SEG##_f##NF(GemmArgs a) { gemm_rows_body<MB, SEG, NF>(a); }
#define GEMM_ROWS_SMALL_M(M, MB) \
    GEMM_ROWS_KERNEL(M, MB, 1, 1) \
    GEMM_ROWS_KERNEL(M, MB, 1, 2) \
    GEMM_ROWS_KERNEL(M, MB, 1, 4) \
    GEMM_ROWS_KERNEL(M, MB, 2, 1) \
    GEMM_ROWS_KERNEL(M, MB, 2, 2) \
    GEMM_ROWS_KERNEL(M, MB, 4, 1)
GEMM_ROWS_SMALL_M(16, 1)
GEMM_ROWS_SMALL_M(32, 2)
GEMM_ROWS_KERNEL(64, 4, 1, 1)
GEMM_ROWS_KERNEL(64, 4, 1, 2)
GEMM_ROWS_KERNEL(64, 4, 2, 1)

// ---- persistent decode of every layer of a step, one workgroup per CU
// (device/persist.h): rfp4_decode_layers_<shape>
K256 void rfp4_decode_layers_8b(PersistArgs a) { decode_layers_body<PersistShape8B>(a); }

// ---- batched prefill row kernels (device/prefill.h)
K256 void rfp4_embed_rows(RowsArgs a) { embed_rows_body(a); }
K256 void rfp4_rmsnorm_quant_rows(RowsArgs a) { rmsnorm_quant_rows_body(a); }
K256 void rfp4_swiglu_quant_rows(RowsArgs a) { swiglu_quant_rows_body(a); }
K256 void rfp4_rope_kv_rows(RopeRowsArgs a) { rope_kv_rows_body(a); }
