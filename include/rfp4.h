/*
 * rfp4.h -- C ABI of the MI355X (gfx950) MXFP4 Llama decode engine.
 *
 * Drop-in boundary for the reference's kernel API (botBehavior/rust-fp4-blackwell).
 * The reference launches each kernel through a cuda-oxide typed launcher,
 *     module.<kernel>(&stream, LaunchConfig, args...) -> Result
 * (llama_run/src/main.rs:513-534).  Every kernel entry point below keeps the
 * reference's name and argument order and adds the stream in front; launch
 * geometry is chosen by the library.  Buffers are device pointers owned by the
 * caller (the reference's DeviceBuffer<T>); the engine API owns its own.
 *
 * Conventions
 *  - Return 0 on success, a negative RFP4_E_* code otherwise; the message of
 *    the last failure on this thread is rfp4_last_error().  The reference
 *    panics on any launch error (`.unwrap()`); a binding maps a non-zero
 *    return to that panic.
 *  - Calls are asynchronous on `stream` except rfp4_d2h, rfp4_*_synchronize,
 *    llama_decode_step and llama_generate, which block.
 *  - One host thread per engine; the library is not reentrant per stream.
 *  - rfp4_init(device) must precede every other call (CudaContext::new +
 *    kernels::load, llama_run/src/main.rs:432,488).
 */
#ifndef RFP4_H
#define RFP4_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *rfp4_stream_t; /* a hipStream_t; NULL = the null stream */
typedef void *rfp4_event_t;  /* a hipEvent_t */

enum {
    RFP4_OK = 0,
    RFP4_E_INVALID = -1,     /* null pointer, zero size, bad enum */
    RFP4_E_SHAPE = -2,       /* K not a multiple of 32, unsupported head_dim, ... */
    RFP4_E_CAPACITY = -3,    /* exceeds a workspace or LDS plan */
    RFP4_E_KV_OVERFLOW = -4, /* position >= max_seq */
    RFP4_E_NOT_INIT = -5,    /* rfp4_init not called */
    RFP4_E_ALIGN = -6,       /* pointer not 16-byte aligned where required */
    RFP4_E_HIP = -7,         /* HIP runtime error, see rfp4_last_error() */
    RFP4_E_NO_DEVICE = -8,
    RFP4_E_WAIT = -9,        /* a device-side wait of a decode step hit its spin limit
                                (workgroups not co-resident): that generation's tokens
                                are invalid; the next llama_engine_begin* clears it */
};

const char *rfp4_last_error(void);
int rfp4_version(void);

/* Kernels of the embedded gfx950 code object, read from its symbol table (no
 * device needed): how many, and the name of kernel i.  Test hook: the CPU
 * tests check that every kernel the host launches is present.  No reference
 * counterpart. */
int rfp4_kernel_count(uint32_t *count);
int rfp4_kernel_name(uint32_t i, char *buf, size_t cap);

/* ------------------------------------------------------------------ runtime
 * Replaces cuda-oxide's context / stream / DeviceBuffer / event API used by
 * the reference (fp4_gemv/src/main.rs:144-150,177-191). */
/* CudaContext::new(device) + kernels::load(&ctx): llama_run/src/main.rs:432,488 */
int rfp4_init(int device);
/* Releases every HIP object the library holds: waits for the device,
 * destroys every engine still alive (its step graphs, stream and memory),
 * frees the runtime's workspaces and unloads the code object.  Call it before
 * the host program exits (the Python binding registers it with atexit);
 * rfp4_init may be called again afterwards.  Caller-owned buffers, streams
 * and events stay the caller's to free.  No reference counterpart (the
 * reference's RAII drops free its objects at the end of main). */
int rfp4_shutdown(void);
int rfp4_device_count(int *count);
/* Compute units, LDS bytes per workgroup and peak clock of the initialised device. */
int rfp4_device_info(int *num_cus, size_t *lds_per_block, int *clock_khz);
/* ctx.default_stream(): llama_run/src/main.rs:433 (here: a new HIP stream) */
int rfp4_stream_create(rfp4_stream_t *stream);
int rfp4_stream_destroy(rfp4_stream_t stream);
int rfp4_stream_synchronize(rfp4_stream_t stream); /* stream.synchronize(): fp4_gemv/src/main.rs:177 */
/* DeviceBuffer allocation (from_host / zeroed): llama_run/src/main.rs:436,454 */
int rfp4_malloc(void **dptr, size_t bytes);
int rfp4_free(void *dptr);
/* DeviceBuffer::zeroed (a fill kernel, so it may be captured in a graph); bytes % 4 == 0 */
int rfp4_memset_zero(void *dptr, size_t bytes, rfp4_stream_t stream);
/* DeviceBuffer::from_host: llama_run/src/main.rs:436 */
int rfp4_h2d(void *dst, const void *src, size_t bytes, rfp4_stream_t stream);
/* DeviceBuffer::to_host_vec (blocking): llama_run/src/main.rs:535 */
int rfp4_d2h(void *dst, const void *src, size_t bytes, rfp4_stream_t stream);
/* stream.record_event / elapsed_ms: fp4_gemv/src/main.rs:179-191 */
int rfp4_event_create(rfp4_event_t *ev);
int rfp4_event_destroy(rfp4_event_t ev);
int rfp4_event_record(rfp4_event_t ev, rfp4_stream_t stream);
int rfp4_event_synchronize(rfp4_event_t ev);
int rfp4_event_elapsed_ms(float *ms, rfp4_event_t start, rfp4_event_t end);

/* ------------------------------------------------------------------ kernels */
/* fp4_gemv(n, k, w, scales, x, y): llama_run/src/main.rs:34-77 (also
 * fp4_gemv/src/main.rs:32-92).  W: E2M1 packed 8 per u32, low nibble first,
 * row-major K/8 words per row; scales: f32 per (row, 32-block); x: K floats.
 * K % 32 == 0; w and x 16-byte aligned.  All N rows are computed (the
 * reference's grid N/8 truncates when N % 8 != 0). */
int fp4_gemv(rfp4_stream_t stream, uint32_t n, uint32_t k, const uint32_t *w, const float *scales,
             const float *x, float *y);
/* fp4_gemv with OCP E8M0 scales (one byte 2^(b-127) per row and 32-block):
 * the BASELINE MXFP4 numerics (trackb/fp4_scale_test.cu:12). */
int mx4_gemv(rfp4_stream_t stream, uint32_t n, uint32_t k, const uint8_t *codes, const uint8_t *scales,
             const float *x, float *y);
/* Fused epilogues of the same kernel (llama_run/src/main.rs:523-530 folded):
 *  mx4_gemv_residual: x_res[r] += W.x      (fp4_gemv + residual, :523-524,:529-530)
 *  mx4_gemv_swiglu:   out[r] = silu(G.x)[r] * (U.x)[r], where G is rows
 *                     [0,n) and U rows [pair_off, pair_off+n) of `codes`
 *                     (fp4_gemv gate/up + swiglu, :526-528)
 *  mx4_gemv_argmax:   y = W.x and *best_token = argmax(y) with the
 *                     reference's tie rule (fp4_gemv lm_head + argmax, :533-534);
 *                     workspace: at least mx4_gemv_argmax_workspace(n) =
 *                     round_up(n, 8) + 64 bytes, 8-byte aligned (one 8-byte key
 *                     per workgroup, then a 16-byte cursor).  The library cannot
 *                     see the caller's allocation: a smaller buffer is written
 *                     out of bounds, so size it with that function. */
/* rmsnorm + fp4_gemv (llama_run/src/main.rs:513-514 fused): y = W.(x*rms*w_norm),
 * rms = 1/sqrt(sum(x^2)/k + eps), fp16 norm weights. */
int mx4_gemv_rmsnorm(rfp4_stream_t stream, uint32_t n, uint32_t k, const uint8_t *codes, const uint8_t *scales,
                     const float *x, const uint16_t *norm_w, float eps, float *y);
int mx4_gemv_residual(rfp4_stream_t stream, uint32_t n, uint32_t k, const uint8_t *codes,
                      const uint8_t *scales, const float *x, float *x_res);
int mx4_gemv_swiglu(rfp4_stream_t stream, uint32_t n, uint32_t k, uint32_t pair_off, const uint8_t *codes,
                    const uint8_t *scales, const float *x, float *out);
size_t mx4_gemv_argmax_workspace(uint32_t n);
int mx4_gemv_argmax(rfp4_stream_t stream, uint32_t n, uint32_t k, const uint8_t *codes, const uint8_t *scales,
                    const float *x, float *y, void *workspace, uint32_t *best_token);
/* rmsnorm(dim, eps, x, weight, y): llama_run/src/main.rs:79-116 */
int rmsnorm(rfp4_stream_t stream, uint32_t dim, float eps, const float *x, const float *weight, float *y);
/* rmsnorm with fp16 weights (the configs keep norms in fp16) */
int rmsnorm_f16w(rfp4_stream_t stream, uint32_t dim, float eps, const float *x, const uint16_t *weight,
                 float *y);
/* rope(num_heads, head_dim, cos_base, cos, sin, q): llama_run/src/main.rs:118-138 */
int rope(rfp4_stream_t stream, uint32_t num_heads, uint32_t head_dim, uint32_t cos_base, const float *cos_tab,
         const float *sin_tab, float *q);
/* copy_into(n, off, src, dst): llama_run/src/main.rs:140-146 (f32 KV append) */
int copy_into(rfp4_stream_t stream, uint32_t n, uint32_t off, const float *src, float *dst);
/* copy_into with an fp16 destination (RNE), the configs' KV-cache format */
int kv_append_f16(rfp4_stream_t stream, uint32_t n, uint32_t off, const float *src, uint16_t *dst);
/* attn_decode(n_heads, n_kv_heads, seq, q, kc, vc, out): llama_run/src/main.rs:148-242.
 * Reference layout: f32 K/V [t][kv_head][64], head_dim 64.  No MAXSEQ cap:
 * split-K over the sequence (the reference caps seq at MAXSEQ=2048, :18). */
int attn_decode(rfp4_stream_t stream, uint32_t n_heads, uint32_t n_kv_heads, uint32_t seq, const float *q,
                const float *kc, const float *vc, float *out);
/* attn_decode over fp16 K/V with head_dim 64 or 128 and any token / head
 * strides (elements): element (t, kvh, d) at t*token_stride + kvh*head_stride + d.
 * attn_decode and attn_decode_f16 keep their split states (and the in-kernel
 * merge's arrival counters) in one library workspace per device: calls that
 * overlap on one device (two streams, two threads) race; serialise them on
 * one stream.  Engines have workspaces of their own. */
int attn_decode_f16(rfp4_stream_t stream, uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                    uint32_t seq, const float *q, const uint16_t *kc, const uint16_t *vc, uint64_t token_stride,
                    uint64_t head_stride, float *out);
/* attn_decode_f16 that allocates nothing.  No counterpart in the reference:
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The split
 * states live in a static device array of 4 MiB per device (set up by
 * rfp4_init) instead of the library workspace; shapes whose states exceed it
 * (n_heads * splits * (head_dim + 4) floats > 2^20) fail with
 * RFP4_E_CAPACITY.  Splits are always merged by a second kernel.  Every call
 * on a device shares that array: calls that overlap on one device race. */
int attn_decode_f16_noalloc(rfp4_stream_t stream, uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                            uint32_t seq, const float *q, const uint16_t *kc, const uint16_t *vc,
                            uint64_t token_stride, uint64_t head_stride, float *out);
/* Causal attention of `rows` query rows at positions pos0 .. pos0+rows-1 over
 * fp16 K/V (the rows' own k, v already in the caches): row r is attn_decode_f16
 * with seq = pos0 + r + 1 (llama_run/src/main.rs:148-242 applied row by row;
 * the reference feeds a prompt one token at a time, :550-556).  q row r at
 * q + r*q_row_stride, out row r at out + r*out_row_stride (floats); q, out and
 * the K/V rows 16-byte aligned (row strides multiples of 4 floats / 8 halves),
 * else RFP4_E_ALIGN.  fp16 matrix-core operands, f32 accumulation.  No
 * reference counterpart as one call. */
int attn_prefill_f16(rfp4_stream_t stream, uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim, uint32_t pos0,
                     uint32_t rows, const float *q, uint32_t q_row_stride, const uint16_t *kc, const uint16_t *vc,
                     uint64_t token_stride, uint64_t head_stride, float *out, uint32_t out_row_stride);
/* swiglu(n, gate, up, out): llama_run/src/main.rs:244-252 */
int swiglu(rfp4_stream_t stream, uint32_t n, const float *gate, const float *up, float *out);
/* residual(n, y, x): x += y, llama_run/src/main.rs:254-261 */
int residual(rfp4_stream_t stream, uint32_t n, const float *y, float *x);
/* argmax(n, logits, out): llama_run/src/main.rs:263-315 (ties -> lowest index) */
int argmax(rfp4_stream_t stream, uint32_t n, const float *logits, uint32_t *out);
/* fp4_mma_allones(out): fp4_mma/src/main.rs:18-54.  One gfx950 scaled MFMA
 * tile; writes 128 floats (D[16][8], row-major), all 64.0. */
int fp4_mma_allones(rfp4_stream_t stream, float *out);
/* The reference's host packer (llama_run/src/main.rs:334-376, quant_fp4):
 * per block of 32, scale = absmax/6 (1.0 for an all-zero block), codes to the
 * nearest E2M1 magnitude (ties to the smaller), 8 codes per word low nibble
 * first; rows x k f32 in, rows*k/8 words and rows*k/32 f32 scales out (the
 * operands of fp4_gemv).  Host only, no device needed. */
int fp4_quantize_absmax(const float *w, uint32_t rows, uint32_t k, uint32_t *packed, float *scales);
/* OCP MX quantization of rows x k values (f32, or bf16 if src_is_bf16) into
 * E2M1 codes (k/2 bytes per row) and E8M0 scales (k/32 per row).  Same bits
 * as the engine's weight quantizer; src 16-byte aligned (8 for bf16), codes
 * 16-byte aligned.  No reference counterpart on the engine
 * path (the reference quantizes with f32 absmax/6 scales on the host,
 * llama_run/src/main.rs:334-376); needed for MXFP4 activations. */
int mx4_quantize(rfp4_stream_t stream, uint64_t rows, uint64_t k, const void *src, int src_is_bf16,
                 uint8_t *codes, uint8_t *scales);
/* Batched MXFP4 GEMM c[m][n] = a[m][k] . w[n][k]^T (f32 out) on scaled MFMA.
 * a_codes/w_codes: E2M1 rows of k/2 bytes (low nibble first); a_scales/
 * w_scales: E8M0 rows of k/32 bytes.  k % 256 == 0, n % 4 == 0; codes and c
 * 16-byte aligned, scales 8-byte aligned.  The reference has only the
 * single m16n8k64 block-scaled tile (fp4_mma/src/main.rs:18-54) and its CPU
 * closed form D = sum_k A SFA B SFB (trackb/fp4_scale_test.cu:37); this is
 * that contraction at M x N x K.  Split-K shapes use a library workspace:
 * calls that overlap on one device race.  The tiled kernels (more than 32
 * activation rows) read the scales in a step-blocked layout (below), which
 * this entry point makes first in a library workspace of 64 MiB (one more
 * launch; shapes whose copies exceed it fail with RFP4_E_CAPACITY: use
 * fp4_gemm_tiled). */
int fp4_gemm(rfp4_stream_t stream, uint32_t m, uint32_t n, uint32_t k, const uint8_t *a_codes,
             const uint8_t *a_scales, const uint8_t *w_codes, const uint8_t *w_scales, float *c);
/* Step-blocked copy of [rows][k/32] E8M0 scales (k % 256 == 0): for each
 * 32-row block and each K step of 256 values, 256 contiguous bytes holding,
 * for h = 0, 1 and rows r = 0..31, the step's scale bytes 4h .. 4h + 3 of the
 * block's row r; ceil(rows/32) blocks, rows past `rows` zero.  It is the
 * tiled GEMM's LDS layout, so each K step of a 32-row block is one 256-byte
 * copy instead of 32 row-strided 8-byte pieces.  No reference counterpart
 * (the reference has no GEMM, main.tex:228).  mx4_scales_tiled_bytes: its
 * size; mx4_scales_tile: makes it on the device (both pointers 4-byte
 * aligned). */
size_t mx4_scales_tiled_bytes(uint32_t rows, uint32_t k);
int mx4_scales_tile(rfp4_stream_t stream, uint32_t rows, uint32_t k, const uint8_t *scales, uint8_t *scales_tiled);
/* mx4_quantize that also writes the step-blocked copy of the scales
 * (k % 256 == 0; the bytes of its rows only: the padding rows of a last
 * partial block are left as they are, which the GEMM never reads into an
 * output it stores).  No reference counterpart. */
int mx4_quantize_tiled(rfp4_stream_t stream, uint64_t rows, uint64_t k, const void *src, int src_is_bf16,
                       uint8_t *codes, uint8_t *scales, uint8_t *scales_tiled);
/* fp4_gemm with the operands' step-blocked scales supplied as well (made by
 * mx4_scales_tile or mx4_quantize_tiled, or an engine's, see
 * llama_engine_weight_scales_tiled): no copy is made, so the call adds no
 * launch and has no workspace limit beyond fp4_gemm's split-K one.  The
 * few-row kernel (m <= 32) reads the row-major scales, the tiled kernels the
 * step-blocked ones; both must describe the same scales.  Same results as
 * fp4_gemm, bit for bit.  No reference counterpart (see fp4_gemm). */
int fp4_gemm_tiled(rfp4_stream_t stream, uint32_t m, uint32_t n, uint32_t k, const uint8_t *a_codes,
                   const uint8_t *a_scales, const uint8_t *a_scales_tiled, const uint8_t *w_codes,
                   const uint8_t *w_scales, const uint8_t *w_scales_tiled, float *c);
/* Test hook: force the GEMM tile (index into the compiled list, largest
 * first: 256x256, 256x128, 128x128, 64x128, 32x128, then 5 = the few-row
 * kernel for k a multiple of 512, up to 16384 for m <= 32 and up to 8192
 * for m <= 64; -1 = automatic)
 * and K split (0 = automatic; for the few-row kernel: W fragments of 16 rows
 * per workgroup, 1, 2 or 4) of later fp4_gemm calls on this thread.  No
 * reference counterpart. */
int rfp4_debug_gemm_plan(int tile, int kz);
/* Test hook (this thread): DMA stages of the tiled MXFP4 GEMM's K pipeline
 * (0 = the planner's choice, 2 = double buffer, 3 or 4 = that many stages
 * where a kernel is compiled for the tile; others fail at launch).  No
 * reference counterpart. */
int rfp4_debug_gemm_stages(int nst);
/* Test hook (this thread): the 8-wave ping-pong kernels of the 256x256 and
 * 256x128 tiles (two waves per SIMD, one running MFMAs while the other issues
 * the next copies and LDS reads; bit-identical to the 4-wave kernels): 0 =
 * the planner's choice, 1 = 4-wave kernels only, 2 = ping-pong wherever the
 * plan picks one of those tiles and the matrices' codes stay under 4 GiB.  No
 * reference counterpart. */
int rfp4_debug_gemm_pp(int mode);
/* Test hook (this thread): 1 = every split-K sum of later fp4_gemm calls in
 * the reduce kernel launched after the GEMM; 0 = two-way splits summed inside
 * the GEMM launch by the last split of each tile (the default; the same
 * sums).  No reference counterpart. */
int rfp4_debug_gemm_reduce_kernel(int on);
/* Test hook: tokens per split of later attn_decode / attn_decode_f16 calls
 * on this thread (0 = automatic).  No reference counterpart. */
int rfp4_debug_attn_chunk(uint32_t chunk);
/* Test hook: how later one-row attention launches on this thread (and
 * engines created by it) merge their splits: 0 = automatic (in-kernel by the
 * last split up to 8 splits; engines: from tagged states up to 32; else a
 * second kernel), 1 = always a second kernel, 2 = the last split of each KV
 * head inside the attention kernel wherever it can (at most 8 splits), 3 =
 * engines only: the first splits of each workgroup column inside the
 * attention kernel, polling tagged split states (2 to 32 splits; other
 * launches as 0).  No reference counterpart. */
int rfp4_debug_attn_merge(int mode);
/* Test hook (this thread): the q|k|v GEMV and the decode attention of
 * engines created afterwards: 0 = one fused launch per layer for steps whose
 * attention is one split, where the engine's shape has a fused kernel and
 * its grid fits the device (the default: faster there, measured), 1 = two
 * launches, 2 = fused at every split count where the grid fits.  Outputs are
 * bit-identical in every mode.  No reference counterpart (the reference
 * launches them apart, llama_run/src/main.rs:513-529). */
int rfp4_debug_qkv_attn(int mode);
/* Test hook (this thread): query-head slices per KV head of the decode
 * attention of engines created afterwards (0 = automatic, 1, 2, 4, 8; a
 * value that does not divide the group means 1). */
int rfp4_debug_attn_head_split(int hs);
/* Test hook (this thread): the gate|up projection of the batched prefill:
 * 0 = SwiGLU and the MXFP4 rows of its output in the GEMM's epilogue where the
 * GEMM's plan is the 256x256 ping-pong tile (no f32 gate|up output is
 * written; the sums within f32 rounding of the plain GEMM's), 1 = the GEMM,
 * then the SwiGLU + MXFP4 row kernel.  No reference counterpart (the
 * reference has no batched prefill). */
int rfp4_debug_prefill_swiglu(int mode);
/* Test hook (this thread): the q|k|v projection of the batched prefill:
 * 0 = RoPE and the fp16 K/V cache rows in the GEMM's epilogue where the
 * GEMM's plan has that kernel (128x128 tile, or 256x256 ping-pong; heads of
 * 64 or 128; bit-identical to mode 1), 1 = the GEMM, then the RoPE + K/V row
 * kernel.  No reference counterpart (the reference has no batched prefill). */
int rfp4_debug_prefill_rope(int mode);
/* Test hook (this thread): the batched prefill's attention rows: 0 =
 * quantized to MXFP4 in the attention kernel's epilogue (the row quantizer's
 * bytes; no f32 rows written), 1 = f32 rows, then the row quantizer.  No
 * reference counterpart. */
int rfp4_debug_prefill_attn_quant(int mode);
/* Test hook: the batched prefill's attention on this thread: 0 = the
 * matrix-core prefill kernel, 1 = the decode kernel, one grid row per prompt
 * row.  No reference counterpart. */
int rfp4_debug_prefill_attn(int mode);
/* Test hook (this thread): llama_engine_prefill stops after one stage and
 * returns *next_token = UINT32_MAX with that stage's output in its workspace
 * (llama_engine_prefill_buffers).  after = -1: the embedding rows; 10 * layer
 * + s: stage s of that layer, s = 0 residual add + RMSNorm + MXFP4 rows, 1 the
 * q|k|v GEMM, 2 RoPE + fp16 K/V append, 3 causal attention, 4 MXFP4 of the
 * attention rows, 5 the o GEMM, 6 residual add + RMSNorm + MXFP4 rows, 7 the
 * gate|up GEMM, 8 SwiGLU + MXFP4 rows, 9 the down GEMM.  -2 = no stop. */
int rfp4_debug_prefill_stop(int after);
/* Test hook: waves per workgroup of the matrix-core prefill attention on
 * this thread (0 = automatic, 4 or 8).  No reference counterpart. */
int rfp4_debug_prefill_waves(int waves);
/* Test hook (this thread): key groups per workgroup of the batched
 * prefill's attention: 0 = automatic (two where the plan is 4 waves and
 * groups of up to 4 query heads), 1 = one, 2 = two where compiled (two
 * groups of waves take alternate key blocks of the same query tiles and
 * merge their softmax states).  No reference counterpart. */
int rfp4_debug_prefill_ksplit(int groups);
/* Test hook: query-tile pairing of the matrix-core prefill attention on this
 * thread (0 = automatic, 1 = one tile per workgroup, 2 = tiles t and
 * ntiles-1-t per workgroup).  No reference counterpart. */
int rfp4_debug_prefill_pairing(int mode);
/* The tile and K split fp4_gemm would use for this shape (honours the test
 * hook).  No reference counterpart. */
int rfp4_gemm_plan(uint32_t m, uint32_t n, uint32_t k, int *tile_m, int *tile_n, int *kz);
/* The kernel fp4_gemm would launch for this shape, with its K split
 * ("<kernel>/kz<splits>"; the few-row kernel's name carries its plan). */
int rfp4_gemm_plan_kernel(uint32_t m, uint32_t n, uint32_t k, char *buf, size_t cap);

/* ------------------------------------------------------------------ test hooks
 * Raw single-tile MFMA (layout pinning, the role of trackb/fp4_mapping_test.cu
 * and trackb/fp4_scale_test.cu): a, b hold 8 dwords per lane (64 lanes),
 * sa, sb one dword per lane; out receives the raw accumulator registers
 * (4 floats per lane for 16x16x128, 16 for 32x32x64). */
int rfp4_mma_tile16(rfp4_stream_t stream, const uint32_t *a, const uint32_t *b, const uint32_t *sa,
                    const uint32_t *sb, float *out);
int rfp4_mma_tile32(rfp4_stream_t stream, const uint32_t *a, const uint32_t *b, const uint32_t *sa,
                    const uint32_t *sb, float *out);
/* Test hook: force the GEMV variant of later launches on this thread
 * (rows per wave 2/4/8, up-front K-slices or 0 for the slice loop;
 * 0, -1 = automatic).  No reference counterpart. */
int rfp4_debug_gemv_variant(int rows_per_wave, int slices);
/* Test hook: waves per workgroup of later VALU GEMV launches on this thread
 * (0 = automatic, 4 or 8; 8 exists for one-slice SwiGLU at 1 row per wave,
 * store at 2, and the residual epilogue at 1 row per wave with one or three
 * slices).  No reference counterpart. */
int rfp4_debug_gemv_waves(int waves);
/* Test hook: the hardware FP4 encoder every quantizing kernel uses
 * (v_cvt_scalef32_pk_fp4_f32 with scale 2^se) against the software encoder
 * of the OCP MX rules (e2m1, round to nearest even, saturating at 6, the sign
 * kept for zero) on every f32 bit pattern (infinities and NaNs included),
 * for se = se0 .. se0 + n_se - 1 within -127 .. 125.  mismatches[i] (all
 * patterns) and tested[i] (the patterns a block of shared exponent se holds,
 * |v| < 2^(se + 3)) (device, n_se counters each, zeroed by the caller) are
 * incremented for se0 + i.  No reference counterpart. */
int rfp4_debug_fp4_encode_check(rfp4_stream_t stream, int32_t se0, uint32_t n_se, unsigned long long *mismatches,
                                unsigned long long *tested);
/* Test hook: one GEMV launch with any epilogue (0 store, 1 residual,
 * 2 SwiGLU with gate rows [0, n) and up rows [pair_off, pair_off + n),
 * 3 argmax), scales of either format (RFP4_SCALE_*: E8M0 bytes or f32) and,
 * when norm_w is not null, the RMSNorm of x fused in front: the engine's
 * fused launches, reachable alone.  Argmax needs
 * mx4_gemv_argmax_workspace(n) bytes of workspace.  No reference
 * counterpart. */
int rfp4_debug_gemv_fused(rfp4_stream_t stream, int epi, int scale_format, uint32_t n, uint32_t k, uint32_t pair_off,
                          const uint8_t *codes, const void *scales, const float *x, const uint16_t *norm_w,
                          float eps, float *y, void *workspace, uint32_t *best_token);
/* Hardware E2M1 conversion of n words (8 codes each) to 8n floats. */
int rfp4_selftest_cvt_fp4(rfp4_stream_t stream, uint32_t n, const uint32_t *words, float *out);
/* One v_mfma_f32_16x16x32_bf16 from raw per-lane registers (4 dwords per
 * lane for a and b); out receives 4 accumulator floats per lane. */
int rfp4_mma_bf16_tile(rfp4_stream_t stream, const uint32_t *a, const uint32_t *b, float *out);
/* The same with fp16 operands (v_mfma_f32_16x16x32_f16, the prefill
 * attention's instruction).  Test hook; no reference counterpart. */
int rfp4_mma_f16_tile(rfp4_stream_t stream, const uint32_t *a, const uint32_t *b, float *out);
/* Synthetic weight generator used by the engine (rows [r0, r0+nrows)). */
int rfp4_synth_mx_weight(rfp4_stream_t stream, uint64_t seed, uint64_t stream_id, float sigma, uint64_t k,
                         uint64_t r0, uint64_t nrows, uint8_t *codes, uint8_t *scales);
int rfp4_synth_f16(rfp4_stream_t stream, uint64_t seed, uint64_t stream_id, float sigma, float offset, uint64_t n,
                   uint16_t *out);

/* ------------------------------------------------------------------ engine
 * The step loop of llama_run / llama_decode (llama_run/src/main.rs:492-570,
 * llama_decode/src/main.rs:428-492) with the model constants of
 * llama_run/src/main.rs:318-332 made a runtime config. */
/* Per-32 block scales of every projection: OCP E8M0 bytes (the BASELINE
 * MXFP4 numerics), or the reference engine's f32 scales
 * (llama_run/src/main.rs:334-376, llama_decode/src/main.rs:307-325). */
enum { RFP4_SCALE_E8M0 = 0, RFP4_SCALE_F32 = 1 };
/* KV-cache elements: fp16 (the configs), or f32 as the reference
 * (llama_run/src/main.rs:388-389). */
enum { RFP4_KV_F16 = 0, RFP4_KV_F32 = 1 };

typedef struct rfp4_model_config {
    uint32_t dim, n_layers, n_heads, n_kv_heads, head_dim, ffn, vocab, max_seq;
    double theta;
    float eps;
    uint16_t scale_format; /* RFP4_SCALE_* (0 = E8M0) */
    uint16_t kv_format;    /* RFP4_KV_* (0 = fp16) */
} rfp4_model_config;

typedef struct llama_engine llama_engine;

/* Allocates weights, KV caches and workspaces.  Synthetic init from `seed`:
 *  - E8M0 scales: weights N(0, 0.02^2) quantized by the OCP MX rules,
 *    embeddings N(0, 0.02^2) fp16, norms 1 + 0.02 N, generated on the device;
 *  - f32 scales: the reference harness's weights (llama_decode/src/main.rs:
 *    300-325,369-393: xorshift32 from the low 32 bits of `seed`, per layer
 *    q, k, v, o, gate, up, down, then the LM head, each its packed words then
 *    its scales 0.25 + (r % 8) / 32) and its activation vector
 *    (r % 2001) / 1000 - 1 (:421), norms 1.0; embeddings as for E8M0. */
int llama_engine_create(const rfp4_model_config *cfg, uint64_t seed, llama_engine **out);
/* Real weights (the reference's loader, llama_run/src/main.rs:413-460): a
 * safetensors checkpoint with the Llama tensor names (model.layers.N.
 * self_attn.{q,k,v,o}_proj.weight, mlp.{gate,up,down}_proj.weight,
 * input_layernorm / post_attention_layernorm.weight, model.norm.weight,
 * model.embed_tokens.weight, lm_head.weight or tied embeddings) in BF16, F16
 * or F32, shapes as cfg.  Projections are quantized on the device to MXFP4
 * (OCP rules, E8M0 per 32; mx4_quantize); norm weights are held as fp16
 * (exact for bf16 gains of magnitude 2^-17 .. 65504, as the reference's f32
 * copies), embeddings as stored when BF16 or F16 (F32 rounded to bf16). */
int llama_engine_create_from_safetensors(const rfp4_model_config *cfg, const char *path, llama_engine **out);
/* With cfg.scale_format = RFP4_SCALE_F32 the projections are quantized on the
 * host by the reference's own packer instead (absmax/6 f32 scales,
 * fp4_quantize_absmax, llama_run/src/main.rs:334-376). */
/* Packed-weight cache (no reference counterpart; the reference re-quantizes
 * at every start): the engine's MXFP4 weights, norms and embeddings with its
 * config, written as one file, and an engine rebuilt from such a file with
 * the given max_seq (no quantization on load). */
int llama_engine_save(llama_engine *e, const char *path);
int llama_engine_load(const char *path, uint32_t max_seq, llama_engine **out);
/* The engine's config and embedding format (1 = bf16, 0 = fp16). */
int llama_engine_info(const llama_engine *e, rfp4_model_config *cfg, int *embed_bf16);
int llama_engine_destroy(llama_engine *e);
/* Fill K/V positions [0, upto) of every layer with f16(0.1 * N(0,1))
 * (the pre-filled context of llama_decode/src/main.rs:357,375-376). */
int llama_engine_prefill_kv(llama_engine *e, uint64_t seed, uint32_t upto);
/* forward(tok, pos) -> argmax, blocking: llama_run/src/main.rs:492-536 */
int llama_decode_step(llama_engine *e, uint32_t tok, uint32_t pos, uint32_t *next);
/* Batched prefill (no reference counterpart; the reference feeds the prompt
 * token by token, llama_run/src/main.rs:550-556), for E8M0 engines with fp16
 * caches: prompt[0..n) at positions
 * pos0.. through the MXFP4 GEMM, every projection input quantised to MXFP4
 * per 32 along K (OCP rules).  Writes those positions' K/V and returns in
 * *next_token the greedy token after the last one; decoding continues with
 * llama_decode_step / llama_generate from position pos0 + n.  Blocking.
 * Needs dim, n_heads*head_dim and ffn to be multiples of 256. */
int llama_engine_prefill(llama_engine *e, const uint32_t *prompt, uint32_t n_prompt, uint32_t pos0,
                         uint32_t *next_token);
/* Prompt-then-greedy loop without the EOS stop (llama_run/src/main.rs:544-570):
 * feeds prompt[0..n_prompt) from position pos0, generates n_new tokens into
 * out.  The whole loop runs on the device (one graph replay per token, token
 * feedback through device memory); one host sync at the end. */
int llama_generate(llama_engine *e, const uint32_t *prompt, uint32_t n_prompt, uint32_t pos0, uint32_t n_new,
                   uint32_t *out);
/* Asynchronous building blocks of llama_generate for timing: arm the cursor,
 * replay n steps, read back the produced tokens. */
int llama_engine_begin(llama_engine *e, const uint32_t *prompt, uint32_t n_prompt, uint32_t pos0,
                       uint32_t ids_cap);
/* The reference's random-weight decode harness (llama_decode/src/main.rs:
 * 356-492) on an f32-scale engine made by llama_engine_create: every K/V
 * position [0, ctx) set to 0.01 (:375-376,388-389), the activation x set to
 * the harness vector, and the cursor armed at position ctx.  Each following
 * llama_engine_run_steps step is that harness's decode_step: no embedding
 * lookup, x carries over from the previous step, and the step's argmax is
 * written to ids[1 + i] (llama_engine_read_ids).  Graph replays as usual. */
int llama_engine_begin_harness(llama_engine *e, uint32_t ctx, uint32_t ids_cap);
int llama_engine_run_steps(llama_engine *e, uint32_t n_steps);
/* Timing of the step's kernels in place: n_steps more steps (advancing the
 * cursor exactly like llama_engine_run_steps), launched one by one, each
 * kernel bracketed by start/stop events taken from its own dispatch
 * (hipExtModuleLaunchKernel), so a record is the kernel's duration inside the
 * decode step.  Blocking; up to `cap` records in launch order, `*count` set
 * to the number of launches.  No reference counterpart (the reference times
 * whole steps, llama_decode/src/main.rs:486-492). */
typedef struct rfp4_kernel_time {
    char name[64];
    float us;
} rfp4_kernel_time;
int llama_engine_time_steps(llama_engine *e, uint32_t n_steps, rfp4_kernel_time *out, uint32_t cap, uint32_t *count);
int llama_engine_read_ids(llama_engine *e, uint32_t *ids, uint32_t count);
/* Logits of the last step (vocab floats, blocking). */
int llama_engine_logits(llama_engine *e, float *host_logits);
rfp4_stream_t llama_engine_stream(llama_engine *e);
/* 1 = replay the captured step graph (default), 0 = launch kernels eagerly */
int llama_engine_use_graph(llama_engine *e, int enable);
/* Persistent decode: every layer of a step in one cooperative launch (one
 * workgroup per CU, grid barriers between the stages of a layer), then the
 * LM head; tokens bit-identical to the graph step past 8 attention splits.
 * Available where the model has the Llama-3-8B widths (dim 4096, 32/8 heads
 * of 128, FFN 14336; any layer count and vocabulary) with E8M0 weights and
 * fp16 caches on a 256-CU device; off by default (the graph step is faster on
 * MI355X: a grid barrier costs more than the kernel boundary it replaces).
 * enable = 1 fails with RFP4_E_SHAPE where the shape does not allow it;
 * llama_engine_persistent tells which step is in use.  No reference
 * counterpart (the reference launches every kernel, llama_run/src/main.rs:
 * 492-530). */
int llama_engine_use_persistent(llama_engine *e, int enable);
int llama_engine_persistent(const llama_engine *e);
/* Device views for parity tests.  proj: 0..6 = q,k,v,o,gate,up,down; layer -1 = LM head. */
int llama_engine_weight(llama_engine *e, int layer, int proj, const uint8_t **codes, const uint8_t **scales,
                        size_t *code_bytes, size_t *scale_bytes);
/* The step-blocked copy of the same weight's scales (mx4_scales_tile's
 * layout), which engines that can prefill hold for the tiled GEMM
 * (fp4_gemm_tiled); RFP4_E_SHAPE for other engines.  No reference
 * counterpart. */
int llama_engine_weight_scales_tiled(llama_engine *e, int layer, int proj, const uint8_t **scales_tiled,
                                     size_t *bytes);
/* K/V caches of a layer, [kv_head][cache positions][head_dim] elements of the
 * engine's kv_format (fp16 bits or f32); count = elements per cache. */
int llama_engine_kv(llama_engine *e, int layer, const void **k, const void **v, size_t *count);
/* Test hook: the batched prefill's workspace, device pointers valid until a
 * longer prompt regrows it: x [rows][dim] f32 (the residual stream), MXFP4
 * activation rows (codes [rows][kmax/2], E8M0 [rows][kmax/32], rows packed
 * at the stage's K), the GEMM output c [rows][widest projection] f32 and the
 * attention output a [rows][n_heads*head_dim] f32. */
int llama_engine_prefill_buffers(llama_engine *e, float **x, uint8_t **codes, uint8_t **scales, float **c, float **a,
                                 uint32_t *rows_cap);
/* Test hook of the decode step's device-side waits (no reference
 * counterpart): for a step with `nsplit` attention splits, *err_wired = 1 if
 * every layer's attention (plain, tagged merge or fused q|k|v poll) reports
 * a spin-limit hit to the engine's error word, *fused = 1 if that step runs
 * the fused q|k|v + attention launch, *checked = 1 if llama_engine_read_ids
 * and llama_engine_time_steps read the word for this engine.  set_err = 1
 * then sets the word as a timed-out wait would (no kernel is launched), so
 * that the next read returns RFP4_E_WAIT until llama_engine_begin* clears
 * it. */
int rfp4_debug_engine_wait(llama_engine *e, int set_err, uint32_t nsplit, int *err_wired, int *checked, int *fused);
/* Per-token weight and KV bytes the step streams at a given position. */
uint64_t llama_engine_weight_bytes(const llama_engine *e);

/* ------------------------------------------------------------------ safetensors
 * Read-only view of a safetensors file (memory-mapped; the format the
 * reference reads, llama_run/src/main.rs:413-430).  rfp4_st_read_f32 widens
 * BF16, F16 or F32 to f32 exactly as the reference's `get` closure
 * (:419-430).  No device needed. */
typedef struct rfp4_st rfp4_st;
int rfp4_st_open(const char *path, rfp4_st **out);
int rfp4_st_close(rfp4_st *st);
int rfp4_st_count(const rfp4_st *st, uint32_t *count);
int rfp4_st_name(const rfp4_st *st, uint32_t i, const char **name);
int rfp4_st_info(const rfp4_st *st, const char *name, char dtype[8], uint32_t *ndim, uint64_t shape[8], uint64_t *nbytes);
int rfp4_st_read_f32(const rfp4_st *st, const char *name, float *out, uint64_t count);
/* The tensor as fp16 bits (no reference counterpart: how the engine stores
 * norm weights): F16 as stored, BF16 and F32 rounded to nearest even, exact
 * for bf16 values of magnitude 2^-17 .. 65504. */
int rfp4_st_read_f16(const rfp4_st *st, const char *name, uint16_t *out, uint64_t count);

#ifdef __cplusplus
}
#endif
#endif
