// Kernel argument blocks, passed by value as the single kernel parameter.
// Shared verbatim by the host launcher (g++) and the device code (hipcc), so
// only plain C types appear here.
#pragma once
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// GEMV epilogues.
enum {
    RFP4_EPI_STORE = 0,   // y[r] = acc
    RFP4_EPI_RESIDUAL = 1, // y[r] += acc  (residual stream update)
    RFP4_EPI_SWIGLU = 2,  // y[r] = silu(acc(gate row r)) * acc(up row r + pair_off)
    RFP4_EPI_ARGMAX = 3,  // y[r] = acc, plus one packed (max, argmin-index) per workgroup
};

typedef struct GemvArgs {
    const void *w;        // codes, row-major, K/2 bytes per row (== reference u32 words)
    const void *scales;   // E8M0 bytes or f32, row-major, K/32 per row
    const float *x;       // activation, K floats
    float *y;             // output (see epilogue)
    unsigned long long *best; // ARGMAX: one packed key per workgroup
    const uint16_t *norm_w;   // optional fp16 RMSNorm weights: x -> x*rms*w first
    uint32_t n;           // logical output rows
    uint32_t k;           // reduction length, multiple of 32
    uint32_t pair_off;    // SWIGLU: physical row offset of the up rows
    float eps;            // RMSNorm epsilon (with norm_w)
} GemvArgs;

typedef struct RmsnormArgs {
    const float *x;
    const void *w;        // f32 or f16 weights
    float *y;
    uint32_t dim;
    float eps;
} RmsnormArgs;

typedef struct RopeArgs {
    float *q;             // [num_heads][head_dim], rotated in place
    const float *cosv;    // table [pos][head_dim/2]
    const float *sinv;
    uint32_t num_heads, head_dim, cos_base;
    uint32_t pad;
} RopeArgs;

typedef struct CopyArgs {
    const float *src;
    void *dst;
    uint32_t n, off;
} CopyArgs;

typedef struct EltwiseArgs {
    const float *a, *b;
    float *out;
    uint32_t n, pad;
} EltwiseArgs;

typedef struct ArgmaxArgs {
    const float *logits;
    uint32_t *out;
    uint32_t n, pad;
} ArgmaxArgs;

// Split-K flash-decode attention.
typedef struct AttnArgs {
    const float *q;       // [n_heads][head_dim]
    const void *kc, *vc;  // element (t, kvh, d) at t*ts + kvh*hs + d
    float *out;           // [n_heads][head_dim]
    float *part;          // workspace: [n_heads][max_splits][head_dim + 4] = (m, l, -, -, acc)
    const int32_t *pos_ptr; // if non-null, seq = *pos_ptr + 1
    // Fused RoPE + KV append (null cosv = off): q is un-rotated, the
    // current token (position seq-1) has un-rotated k_new and v_new
    // ([n_kv_heads][head_dim]); tables are [pos][head_dim/2].
    const float *cosv, *sinv;
    const float *k_new, *v_new;
    uint64_t ts, hs;      // token and head strides (elements)
    uint32_t n_heads, n_kv_heads, head_dim, seq;
    uint32_t chunk, max_splits;
    // Several query rows (grid z = row, batched prefill): row r reads q + r*q_rs,
    // writes out + r*out_rs, sees seq + r positions (causal), and owns its own
    // workspace slice of n_heads*max_splits*(head_dim+4) floats.  One row: 0, 0.
    uint32_t q_rs, out_rs;
    // In-kernel merge (one query row): arrival counters per workgroup column
    // (KV head x query-head slice), zero between launches; the last split of
    // a column merges.  Null = the merge kernel runs after this one.
    uint32_t *counters;
    // Query-head slices per KV head (grid x = head_split * n_kv_heads; 0 or 1:
    // every workgroup serves the KV head's whole group).
    uint32_t head_split, pad2;
    // Tagged in-kernel merge (engine decode, one query row, splits <=
    // tag_splits <= 64; null = off): split states as 64-bit words (float bits
    // | tag << 32, tag = the launch's sequence length), word (h, split, i) at
    // (h * tag_splits + split) * (head_dim + 4) + i, i = 0 m, 1 l, 4 + d acc.
    // The workspace must hold no word tagged with a sequence length this
    // launch could use before its first launch of a generation (the engine
    // clears it).  err: set to 1 if a merge hit its spin limit.
    unsigned long long *tagged;
    uint32_t *err;
    uint32_t tag_splits, pad3;
    // Fused q|k|v GEMV (one row; null = off): q, the current token's k and
    // v as 64-bit words (float bits | tag << 32, tag = the launch's sequence
    // length), [n_heads + 2 n_kv_heads][head_dim], stored by the GEMV
    // workgroups of the same launch and polled by the attention workgroups.
    // No other launch of the same sequence length may have written these
    // words (the engine keeps one region per layer and clears them before
    // each generation).
    const unsigned long long *qkv_t;
} AttnArgs;

// Fused q|k|v GEMV + decode attention (device/qkva.h): workgroup b takes GEMV
// tile b (b < n_tiles; 4R consecutive rows, RMSNorm fused) and attention
// workgroup b (b < n_attn; KV head x query-head slice = b % (n_kv_heads *
// head_split), split = b / (n_kv_heads * head_split)).
typedef struct QkvaArgs {
    GemvArgs g;               // the q|k|v GEMV (g.y unused: outputs go to yt)
    AttnArgs a;               // the attention; a.qkv_t = yt
    unsigned long long *yt;   // tagged q|k|v outputs, [n_heads + 2 n_kv_heads][head_dim]
    uint32_t n_tiles, n_attn;
} QkvaArgs;

// Causal attention of the batched prefill (device/attn_prefill.h): prompt
// row r sits at position pos0 + r and its k, v are already in the caches.
typedef struct AttnPrefillArgs {
    const float *q;          // row r: q + r*q_rs, [n_heads][head_dim]
    const uint16_t *kc, *vc; // fp16 caches: element (t, kvh, d) at t*ts + kvh*hs + d
    float *out;              // row r: out + r*out_rs, [n_heads][head_dim]
    uint64_t ts, hs;
    uint32_t q_rs, out_rs, n_heads, n_kv_heads, pos0, rows;
    uint32_t paired;         // nonzero: workgroup x takes query tiles ntiles-1-x and x (grid ceil(ntiles/2))
    // Optional (null = off): the output rows quantized to MXFP4 per 32 as the
    // row quantizer does it, codes [rows][n_heads*head_dim/2], scales
    // [rows][n_heads*head_dim/32] and, if not null, their step-blocked copy
    // (GemmArgs::a_st; n_heads*head_dim a multiple of 256).  out may then be
    // null (no f32 rows).
    uint8_t *q_codes, *q_scales, *q_scales_t;
} AttnPrefillArgs;

// Batched prefill row kernels (device/prefill.h).
typedef struct RowsArgs {
    const float *x;          // rmsnorm: rows [rows][k]; swiglu: gate|up rows [rows][2k]
    const uint16_t *w;       // rmsnorm: fp16 weights [k]
    uint8_t *codes, *scales; // quantised rows [rows][k/2], [rows][k/32]
    const uint32_t *ids;     // embed: token ids [rows]
    const uint16_t *embed;   // embed: fp16 table [vocab][k]
    float *y;                // embed: output rows [rows][k]
    uint32_t rows, k, vocab;
    float eps;
    uint32_t bf16;           // embed holds bf16 (1) or fp16 (0) bit patterns
    const float *add;        // rmsnorm: rows added into x first (the layer's residual add), or null
    float *x_out;            // rmsnorm with add: where x + add is stored (x itself)
    uint8_t *scales_t;       // rmsnorm, swiglu: the scales step-blocked as well (GemmArgs), or null
} RowsArgs;

typedef struct RopeRowsArgs {
    float *qkv;               // [rows][row_stride]: n_heads q, n_kv_heads k, n_kv_heads v (head_dim each)
    const float *cosv, *sinv; // [pos][head_dim/2]
    uint16_t *kc, *vc;        // fp16 caches: element (t, kvh, d) at t*ts + kvh*hs + d
    uint64_t ts, hs;
    uint32_t rows, row_stride, n_heads, n_kv_heads, head_dim, pos0;
} RopeRowsArgs;

typedef struct FillArgs {
    uint32_t *p;
    uint64_t n_words;
    uint32_t value, pad;
} FillArgs;

// Synthetic MXFP4 weight rows [r0, r0+nrows) of a K-wide matrix.
typedef struct SynthWeightArgs {
    uint8_t *packed;      // nrows * K/2
    uint8_t *scales;      // nrows * K/32
    uint64_t seed, stream;
    uint64_t r0, nrows, k;
    float coef;
    uint32_t pad;
} SynthWeightArgs;

// Synthetic fp16 tensor: f16(offset + N*coef) over index i in [0, n).
typedef struct SynthF16Args {
    uint16_t *out;
    uint64_t seed, stream, n;
    float coef, offset;
} SynthF16Args;

// Synthetic KV prefill: positions [0, upto) of [kvh][max_seq][hd] fp16 (or
// f32) caches.
typedef struct SynthKvArgs {
    void *cache;
    uint64_t seed, stream;
    uint32_t upto, n_kv_heads, head_dim, max_seq;
    float coef;
    uint32_t kv_f32;      // nonzero: f32 elements, else fp16 bits
} SynthKvArgs;

// OCP MX quantization of f32 (or bf16) rows into codes + E8M0.
typedef struct QuantMxArgs {
    const void *src;      // f32 or bf16, rows x K
    uint8_t *packed, *scales;
    uint64_t rows, k;
    uint8_t *scales_t;    // the scales step-blocked as well (GemmArgs; k % 256 == 0), or null
} QuantMxArgs;

// rfp4_debug_fp4_encode_check: per shared exponent se0 + blockIdx.y, the
// count of values whose hardware and software FP4 codes differ, and of values
// compared
typedef struct Fp4CheckArgs {
    unsigned long long *mismatches, *tested;
    int32_t se0;
    uint32_t pad;
} Fp4CheckArgs;

// Device-resident decode cursor: lets one captured step graph replay for
// every token.  pos = absolute position, step = index into ids[].
typedef struct StepState {
    int32_t pos;
    int32_t step;
    uint32_t n_prompt;    // ids[0, n_prompt) are prompt tokens
    uint32_t ids_cap;     // capacity of ids[]
} StepState;

// Embedding gather: x[i] = f16(embed[ids[state->step]][i]).
typedef struct EmbedArgs {
    const uint16_t *embed;
    const uint32_t *ids;
    const StepState *state;
    float *x;
    uint32_t dim, vocab;
    uint32_t bf16;        // embed holds bf16 (1) or fp16 (0) bit patterns
} EmbedArgs;

// End-of-step bookkeeping for on-device greedy decode: reduce the LM head's
// per-workgroup keys, record the token, advance the cursor.
typedef struct StepArgs {
    const unsigned long long *best;
    StepState *state;
    uint32_t *ids;
    uint32_t *last_tok;
    uint32_t n_best, pad;
    // optional (embed non-null): the next step's embedding row into x, as
    // rfp4_embed would gather it at the start of that step
    const uint16_t *embed;
    float *x;
    uint32_t dim, vocab, bf16, pad2;
} StepArgs;

// Scaled-MFMA MXFP4 GEMM: C[M][N] = A[M][K] * W[N][K]^T, both MXFP4 (E2M1 +
// E8M0 per 32 along K), f32 output.
typedef struct GemmArgs {
    const uint8_t *a_codes, *a_scales;   // [m][k/2], [m][k/32]
    const uint8_t *w_codes, *w_scales;   // [n][k/2], [n][k/32]
    float *c;                            // [m][n]
    float *part;                         // [kz][m][n] split-K partials (kz > 1)
    uint32_t m, n, k, kz;
    // kz > 1: arrival counter per output tile (zero between launches); the
    // last split of a tile to arrive sums the planes.  Null: the reduce
    // kernel launched next sums them.
    uint32_t *counters;
    // the same scales step-blocked (the tiled kernels read only these, the
    // few-row kernels only the row-major ones): per 32-row block and K step
    // of 256 values, 256 contiguous bytes, for h = 0, 1 and rows r = 0..31
    // the step's scale bytes 4h .. 4h + 3 of the block's row r
    const uint8_t *a_st, *w_st;
    // SwiGLU + MXFP4 epilogue (the 256x256 ping-pong kernel _ppsw only, kz =
    // 1, n = 2 pair_off): the W rows of column tile nt are gate rows 128 nt ..
    // +127 and up rows pair_off + 128 nt .. +127; the tile writes y = silu(gate)
    // * up for its 128 columns of the pair_off wide output, quantized per 32
    // along it by the row quantizer's rules: q_codes [m][pair_off/2], q_scales
    // [m][pair_off/32] and, if not null, q_scales_t (step-blocked over K =
    // pair_off).  c is not written.
    uint8_t *q_codes, *q_scales, *q_scales_t;
    uint32_t pair_off;
    // nonzero: c += A . W^T (each element c + the sum, one rounding, as a
    // residual add after the plain GEMM; the plain epilogues, the split-K sums
    // and the reduce kernel), not with the SwiGLU or RoPE epilogues
    uint32_t c_add;
    // RoPE + K/V cache epilogue (the _rope kernels only, kz = 1): the output
    // columns are rope_q / rope_hd q heads, then rope_kv / rope_hd k heads,
    // then as many v heads, rope_hd (64 or 128) wide; row r is position
    // rope_pos0 + r.  The tile rotates the q and k columns by rope_cos /
    // rope_sin ([pos][rope_hd / 2]), writes rotated q, k and plain v to c,
    // and k (rotated) and v as fp16 into kc / vc: element (pos, kv head, d)
    // at pos * kv_ts + head * kv_hs + d.
    const float *rope_cos, *rope_sin;
    uint16_t *kc, *vc;
    uint64_t kv_ts, kv_hs;
    uint32_t rope_pos0, rope_q, rope_kv, rope_hd;
} GemmArgs;

// Row-major E8M0 scales [rows][k/32] -> the step-blocked layout of GemmArgs
// (ceil(rows/32) blocks; rows past `rows` hold zero bytes), for up to two
// matrices of the same k in one launch (rows[1] = 0: one).
typedef struct ScaleTileArgs {
    const uint8_t *src[2];
    uint8_t *dst[2];
    uint32_t rows[2], k;
} ScaleTileArgs;

// Persistent decode of every layer of one step (device/persist.h): one
// workgroup per CU, grid barriers between the stages of a layer.
typedef struct PersistLayer {
    const uint8_t *qkv_c, *qkv_s, *o_c, *o_s, *gu_c, *gu_s, *d_c, *d_s; // E8M0 MXFP4, as the engine stacks them
} PersistLayer;

typedef struct PersistArgs {
    const PersistLayer *layers;           // [n_layers], device memory
    const uint16_t *norm_attn, *norm_ffn; // fp16 [n_layers][dim]
    void *kcache, *vcache;                // fp16; layer l starts kv_layer_elems * l elements in
    uint64_t kv_layer_elems;
    const float *cosv, *sinv;             // rope tables [pos][head_dim/2]
    const StepState *state;               // the step's position
    float *x;                             // residual stream [dim], in and out
    float *qkv, *att, *sw;                // stage outputs [nq + 2 nkv][hd], [nq][hd], [ffn]
    float *part;                          // split states [n_heads][max_splits][head_dim + 4]
    uint32_t *counters;                   // [n_kv_heads] merge arrivals, zero between launches
    uint32_t *flags;                      // [gridDim.x] barrier generations (monotonic)
    uint32_t *err;                        // nonzero: a barrier hit its spin limit
    uint32_t n_layers, dim, n_heads, n_kv_heads, head_dim, ffn;
    uint32_t max_seq_alloc, chunk, max_splits;
    uint32_t gen0, spin_limit;            // generation before this launch's first barrier
    float eps;
} PersistArgs;

typedef struct MmaTileArgs {
    const uint32_t *a;    // per-lane A registers
    const uint32_t *b;
    const uint32_t *sa, *sb;
    float *out;
    uint32_t mode, pad;
} MmaTileArgs;

typedef struct SelftestArgs {
    const uint32_t *in;
    float *out;
    const float *scale;   // per-word scale (bf16 conversion test)
    uint32_t n, pad;
} SelftestArgs;

#ifdef __cplusplus
}

// Attention: 16-byte row pieces of K (and of V) each thread holds per
// sub-chunk, for head_dim, KV element bytes and the compile-time query-head
// group (1, 2, 4, 8).  9 for fp16 rows of 128 with groups up to 4 (144
// tokens: a 4096-token context takes 29 splits per KV head, and 8 KV heads
// fit one workgroup per CU); 4 with 8 heads per group (their scores and
// accumulators take the registers); else 8.  Tokens per sub-chunk: this
// times 256 / (head_dim * elem_bytes / 16).
constexpr int attn_steps_for(int head_dim, int elem_bytes, int group)
{
    return group == 8 ? 4 : (head_dim == 128 && elem_bytes == 2) ? 9 : 8;
}
// Prompt rows per workgroup of the prefill attention with `waves` waves and
// a query-head group padded to `group`: one 16-row tile per wave when the
// group allows, at least 16 rows.
constexpr int attn_prefill_rows(int group, int waves)
{
    return 16 * waves / group > 16 ? 16 * waves / group : 16;
}
#endif
