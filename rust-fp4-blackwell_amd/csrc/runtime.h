// Internal host-side declarations shared by runtime.cpp and engine.cpp.
#pragma once
#include <hip/hip_runtime_api.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/rfp4.h"
#include "shared/kernel_args.h"

namespace rfp4 {

constexpr uint32_t kAttnMaxHeads = 128;
constexpr uint32_t kAttnMaxSplits = 512;

constexpr size_t kGemmPartFloats = (size_t)8 << 20; // 32 MiB
// A split-K workspace is kGemmPartFloats floats of partial planes followed by
// kGemmCounters arrival counters (zero between launches) for the two-way
// splits that sum inside the launch.
constexpr uint32_t kGemmCounters = 16384;
constexpr size_t kGemmWorkspaceWords = kGemmPartFloats + kGemmCounters;
// Step-blocked scale copies the drop-in fp4_gemm makes for the tiled kernels
// when the caller passes only row-major scales (A's, then W's).
constexpr size_t kGemmStBytes = (size_t)64 << 20;

struct Runtime {
    int device = 0;
    int num_cus = 256;
    hipModule_t module = nullptr;
    std::unordered_map<std::string, hipFunction_t> fns;
    float *attn_part = nullptr;       // default split-K workspace of attn_decode
    size_t attn_part_floats = 0;
    float *gemm_part = nullptr;       // split-K workspace of fp4_gemm (kGemmWorkspaceWords)
    uint8_t *gemm_st = nullptr;       // step-blocked scales of fp4_gemm's operands (kGemmStBytes)
    uint32_t *attn_counters = nullptr; // in-kernel attention merge (kAttnMaxHeads words, zero between calls)
    size_t max_lds = 65536;           // LDS bytes per workgroup
};

Runtime *runtime();
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_check(hipError_t e, const char *what);
int launch(const char *name, dim3 grid, dim3 block, hipStream_t s, void *args, unsigned shmem = 0);
// Cooperative launch (every workgroup resident at once, or an error): for
// kernels with grid barriers.  Timed like launch() while a record list is
// installed (events recorded around the launch on the stream).
int launch_coop(const char *name, dim3 grid, dim3 block, hipStream_t s, void *args, unsigned shmem);
// Workgroups of `name` with `block` threads and `shmem` dynamic LDS bytes
// that fit on one CU at once.
int kernel_occupancy(const char *name, int block, unsigned shmem, int *per_cu);

// Per-launch timing: while a record list is installed on this thread, every
// launch() goes through hipExtModuleLaunchKernel with its own start and stop
// events, which take the kernel's dispatch timestamps (the interval rocprof
// reports as its duration).  Eager launches only (not under stream capture).
struct KernelTiming {
    const char *name; // a kernel-table key: lives as long as the runtime
    hipEvent_t start, stop;
};
void timing_install(std::vector<KernelTiming> *records); // nullptr = off

int fill_words(uint32_t *p, uint64_t n_words, uint32_t value, hipStream_t s);
int gemv_check(uint32_t n, uint32_t k, const void *w, const void *sc, const float *x, const float *y);
struct GemvVariant {
    int R, NS, W; // rows per wave, up-front K slices (0 = loop), waves per workgroup
};
// The variant a launch of this shape gets now (honours this thread's
// rfp4_debug_gemv_* overrides); an engine fixes its variants at creation.
GemvVariant gemv_variant(uint32_t n, uint32_t k, int epi, bool f32scale);
// Dynamic LDS of a GEMV's x staging for reduction length k (36 floats per
// 32-value chunk, device/gemv.h).
uint32_t gemv_lds_bytes(uint32_t k);
inline uint32_t gemv_grid(uint32_t n, const GemvVariant &v) { return (n + (uint32_t)(v.W * v.R) - 1) / (uint32_t)(v.W * v.R); }
int gemv_launch_v(const char *scale_name, int epi, const GemvArgs &args, hipStream_t s, const GemvVariant &v);
int gemv_launch(const char *scale_name, int epi, const GemvArgs &args, hipStream_t s);
int attn_launch(const AttnArgs &args, int kv_f16, hipStream_t s, uint32_t max_seq_for_grid, uint32_t rows);
// Query-head slices per KV head for an attention grid of `splits` splits
// (args.head_split = 0 asks attn_launch for this).
uint32_t attn_head_split_for(uint32_t n_heads, uint32_t n_kv_heads, uint32_t splits, uint32_t num_cus);
// One-row attention over caller K/V with split states in `part` (at least
// n_heads * splits * (head_dim + 4) floats, checked); allow_inmerge = false
// always merges with the second kernel (no counters, nothing that must start
// at zero).
int attn_decode_ws(hipStream_t s, uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t seq, const float *q, const void *kc,
                   const void *vc, uint64_t ts, uint64_t hs, float *out, int f16, float *part, size_t part_floats,
                   bool allow_inmerge);
// Destroys every engine still alive (rfp4_shutdown); returns how many.
size_t engines_destroy_all();
// Looks up, once per device and with that device current, the address of
// the allocation-free entry points' static scratch (csrc/noalloc.hip).
int noalloc_setup(int device);
// fp4_gemm with the caller's split-K workspace (kGemmWorkspaceWords words, the
// counters zeroed; the engine owns one, so engines on different streams do
// not share partials).  a_st / w_st: the step-blocked copies of the scales
// (device/gemm.h); where either is null and the plan is a tiled kernel, both
// are made first in the runtime's workspace (one more launch).  accumulate:
// c += the product (each element one f32 addition of c and the sum, as a
// residual add after the GEMM would make it); tiled plans only
// (gemm_accumulate_ok).
int gemm_launch(hipStream_t stream, uint32_t m, uint32_t n, uint32_t k, const uint8_t *a_codes, const uint8_t *a_scales,
                const uint8_t *a_st, const uint8_t *w_codes, const uint8_t *w_scales, const uint8_t *w_st, float *c,
                float *part, bool accumulate = false);
bool gemm_accumulate_ok(uint32_t m, uint32_t n, uint32_t k);
// The gate|up projection of the prefill with SwiGLU and the MXFP4 rows of its
// output in the GEMM's epilogue (rfp4_gemm_256x256_ppsw): m rows of K = k,
// W = [gate; up] of 2 ffn rows; y = silu(gate) * up quantized per 32 into
// q_codes [m][ffn/2], q_scales [m][ffn/32] and q_scales_t (step-blocked).
// gemm_swiglu_ok: whether the plan of the plain GEMM (m, 2 ffn, k) is that
// kernel's tile (256x256 ping-pong, no K split) and ffn a multiple of 256.
bool gemm_swiglu_ok(uint32_t m, uint32_t ffn, uint32_t k);
int gemm_swiglu_launch(hipStream_t stream, uint32_t m, uint32_t ffn, uint32_t k, const uint8_t *a_codes,
                       const uint8_t *a_scales, const uint8_t *a_st, const uint8_t *w_codes, const uint8_t *w_scales,
                       const uint8_t *w_st, uint8_t *q_codes, uint8_t *q_scales, uint8_t *q_scales_t);
// The prefill's q|k|v projection with RoPE and the fp16 K/V cache rows in
// the GEMM's epilogue (the _rope kernels; GemmArgs::rope_cos): m rows of
// K = k into n = q + 2 kv columns of c, heads hd wide, row r at position
// pos0 + r, cache element (pos, kv head, d) at pos * ts + head * hs + d.
// gemm_rope_ok: whether the plan of the plain GEMM (m, n, k) is a tile with
// that epilogue compiled (128x128 with 2 or 3 stages, 256x256 ping-pong; no
// K split) and hd 64 or 128; its output is then bit-identical to the GEMM
// followed by the RoPE + K/V row kernel.
struct GemmRope {
    const float *cosv, *sinv;
    uint16_t *kc, *vc;
    uint64_t ts, hs;
    uint32_t pos0, q, kv, hd;
};
bool gemm_rope_ok(uint32_t m, uint32_t n, uint32_t k, uint32_t hd);
int gemm_rope_launch(hipStream_t stream, uint32_t m, uint32_t n, uint32_t k, const uint8_t *a_codes,
                     const uint8_t *a_scales, const uint8_t *a_st, const uint8_t *w_codes, const uint8_t *w_scales,
                     const uint8_t *w_st, float *c, const GemmRope &r);
// Bytes of the step-blocked copy of [rows][k/32] E8M0 scales.
inline size_t scales_tiled_bytes(uint32_t rows, uint32_t k) { return (size_t)((rows + 31u) / 32u) * 32u * (k / 32u); }
// Row-major scales of one or two matrices (rows1 = 0: one) into step-blocked copies, k % 256 == 0.
int scales_tile_launch(hipStream_t s, uint32_t k, const uint8_t *src0, uint8_t *dst0, uint32_t rows0,
                       const uint8_t *src1, uint8_t *dst1, uint32_t rows1);
// mx4_quantize that also writes the step-blocked copy of the scales (null: none; k % 256 == 0 otherwise).
int mx4_quantize_st(hipStream_t stream, uint64_t rows, uint64_t k, const void *src, int src_is_bf16, uint8_t *codes,
                    uint8_t *scales, uint8_t *scales_t);
uint32_t attn_group_pad(uint32_t group);
// Causal prefill attention (device/attn_prefill.h), fp16 caches.
int attn_prefill_launch(const AttnPrefillArgs &a, uint32_t head_dim, hipStream_t s);
// tokens per register sub-chunk of the decode attention with a compiled
// query-head group (1, 2, 4, 8) serving `group` heads
uint32_t attn_sub_chunk(uint32_t head_dim, uint32_t elem_bytes, uint32_t group);
// Whether one-row attention with `max_splits` splits merges inside the split
// kernel (arrival counters) instead of in a second launch.
bool attn_inmerge(uint32_t max_splits);
int attn_merge_mode();                           // this thread's rfp4_debug_attn_merge setting
int prefill_attn_mode();                         // this thread's rfp4_debug_prefill_attn setting
int attn_head_split_mode();                      // this thread's rfp4_debug_attn_head_split setting
int qkva_mode();                                 // this thread's rfp4_debug_qkv_attn setting
int prefill_stop();                              // this thread's rfp4_debug_prefill_stop setting
int prefill_swiglu_mode();                       // this thread's rfp4_debug_prefill_swiglu setting
int prefill_rope_mode();                         // this thread's rfp4_debug_prefill_rope setting
int prefill_attn_quant_mode();                   // this thread's rfp4_debug_prefill_attn_quant setting
bool attn_inmerge_mode(int mode, uint32_t splits); // attn_inmerge under an explicit setting
constexpr uint32_t kAttnInmergeMaxSplits = 8;
// Whether an engine's one-row attention with `splits` splits uses the tagged
// in-kernel merge (a per-layer tagged workspace of at most kAttnTagMaxSplits
// splits per head, cleared before each generation).
bool attn_tagged_mode(int mode, uint32_t splits);
constexpr uint32_t kAttnTagMaxSplits = 32; // ATTN_TAG_MAX_SPLITS (device/attn.h)
uint32_t attn_chunk_for(uint32_t n_kv_heads, uint32_t seq, uint32_t num_cus, uint32_t head_dim, uint32_t elem_bytes,
                        uint32_t group);

// sigma / sqrt((65536^2 - 1)/3): the Irwin-Hall(4) normal coefficient shared
// with every host generator of the synthetic init.
inline float ih4_coef(float sigma) { return (float)((double)sigma / 37837.22723720648); }

} // namespace rfp4
