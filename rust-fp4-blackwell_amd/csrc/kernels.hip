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

#define K256 extern "C" __global__ __launch_bounds__(256)
#define K1024 extern "C" __global__ __launch_bounds__(1024)

// ---- GEMV: rfp4_gemv_<scale>_<epilogue>_r<R>
#define GEMV_KERNEL(SNAME, SF32, ENAME, EPI, R) \
    K256 void rfp4_gemv_##SNAME##_##ENAME##_r##R(GemvArgs a) { gemv_body<SF32, EPI, R>(a); }
#define GEMV_ALL_R(SNAME, SF32, ENAME, EPI) \
    GEMV_KERNEL(SNAME, SF32, ENAME, EPI, 2) \
    GEMV_KERNEL(SNAME, SF32, ENAME, EPI, 4) \
    GEMV_KERNEL(SNAME, SF32, ENAME, EPI, 8)

GEMV_ALL_R(e8m0, 0, store, RFP4_EPI_STORE)
GEMV_ALL_R(e8m0, 0, resid, RFP4_EPI_RESIDUAL)
GEMV_ALL_R(e8m0, 0, swiglu, RFP4_EPI_SWIGLU)
GEMV_ALL_R(e8m0, 0, argmax, RFP4_EPI_ARGMAX)
GEMV_ALL_R(f32, 1, store, RFP4_EPI_STORE)

// ---- norm / rope / embed
K1024 void rfp4_rmsnorm_f32w(RmsnormArgs a) { rmsnorm_body<0>(a); }
K1024 void rfp4_rmsnorm_f16w(RmsnormArgs a) { rmsnorm_body<1>(a); }
K256 void rfp4_rope(RopeArgs a) { rope_body(a); }
K256 void rfp4_rope_append(RopeAppendArgs a) { rope_append_body(a); }
K256 void rfp4_embed(EmbedArgs a) { embed_body(a); }

// ---- attention
K256 void rfp4_attn_hd64_f32(AttnArgs a) { attn_body<64, float>(a); }
K256 void rfp4_attn_hd64_f16(AttnArgs a) { attn_body<64, uint16_t>(a); }
K256 void rfp4_attn_hd128_f32(AttnArgs a) { attn_body<128, float>(a); }
K256 void rfp4_attn_hd128_f16(AttnArgs a) { attn_body<128, uint16_t>(a); }

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
K256 void rfp4_quant_mx_f32(QuantMxArgs a) { quant_mx_body<0>(a); }
K256 void rfp4_quant_mx_bf16(QuantMxArgs a) { quant_mx_body<1>(a); }
K256 void rfp4_selftest_cvt(SelftestArgs a) { selftest_cvt_body(a); }

// ---- MFMA tiles
K256 void rfp4_mma16_tile(MmaTileArgs a) { mma16_tile_body(a); }
K256 void rfp4_mma32_tile(MmaTileArgs a) { mma32_tile_body(a); }
K256 void rfp4_mma_allones(MmaTileArgs a) { mma_allones_body(a.out); }
