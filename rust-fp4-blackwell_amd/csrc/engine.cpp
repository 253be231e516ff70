// Llama MXFP4 decode engine: the step loop of llama_run / llama_decode
// (llama_run/src/main.rs:492-570, llama_decode/src/main.rs:428-492),
// rebuilt around one HIP graph per token.
//
// Device memory per engine:
//  - weights (MXFP4, row-major codes + per-32 scales: E8M0 bytes or the
//    reference's f32, per the config's scale_format), per layer
//      qkv  [(NH+2*NKV)*HD][DIM]   q, k, v stacked: one GEMV launch
//      o    [DIM][NH*HD]
//      gu   [2*FFN][DIM]           gate rows then up rows: one GEMV + SwiGLU
//      down [DIM][FFN]
//    plus the LM head [VOCAB][DIM]; embeddings and norms fp16.
//  - KV caches fp16 or f32 [layer][kvh][max_seq_alloc][HD] (head-major, so a split-K
//    attention workgroup streams one contiguous token range).
//  - a device cursor (position, step) and the token array ids[]; the LM-head
//    GEMV reduces its argmax per workgroup and the step kernel writes the next
//    token into ids[], so consecutive steps need no host round trip.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <thread>
#include <unordered_set>
#include <vector>

#include "runtime.h"
#include "safetensors.h"

using namespace rfp4;

// Stream ids of the synthetic init; the CPU oracle uses the same ids.
static inline uint64_t stream_w(uint32_t l, uint32_t p) { return ((uint64_t)l << 8) | p; }
static const uint64_t kStreamLm = 0xFFFF00ull;
static const uint64_t kStreamEmbed = 0xE0000ull;
static inline uint64_t stream_norm(uint32_t l, uint32_t w) { return 0xA0000ull + ((uint64_t)l << 1) + w; }
static const uint64_t kStreamNormFinal = 0xAFFFFull;
static inline uint64_t stream_kv(uint32_t l, uint32_t isv) { return 0x4B560000ull + ((uint64_t)l << 1) + isv; }

struct LayerW {
    uint8_t *qkv_c, *qkv_s, *o_c, *o_s, *gu_c, *gu_s, *d_c, *d_s; // scales: sb bytes per 32-block
    // the E8M0 scales again, step-blocked for the prefill's tiled GEMM
    // (GemmArgs::w_st; engines that can prefill, else null)
    uint8_t *qkv_st = nullptr, *o_st = nullptr, *gu_st = nullptr, *d_st = nullptr;
};

// The engine's GEMV launches, their variants fixed at creation.
enum { GV_QKV = 0, GV_O, GV_GU, GV_D, GV_LM, GV_N };

struct llama_engine {
    rfp4_model_config c{};
    hipStream_t stream = nullptr;
    std::vector<void *> allocs;
    std::vector<LayerW> L;
    uint16_t *norm_attn = nullptr, *norm_ffn = nullptr, *norm_final = nullptr, *embed = nullptr;
    uint8_t *lm_c = nullptr, *lm_s = nullptr, *lm_st = nullptr;
    void *kcache = nullptr, *vcache = nullptr;
    uint32_t sb = 1, kvb = 2;  // bytes per scale (E8M0 1, f32 4) and per KV element (fp16 2, f32 4)
    const char *sname = "e8m0"; // kernel-name token of the scale format
    GemvVariant gv[GV_N]{};     // GEMV variants, fixed at creation (the LM head's sizes `best`)
    float *gemm_part = nullptr; // split-K workspace of the prefill GEMMs (kGemmWorkspaceWords, counters zeroed)
    std::vector<float> harness_x; // llama_decode's activation vector (f32-scale synthetic init)
    bool no_embed = false;        // harness steps: x carries over, no embedding lookup
    uint32_t max_seq_alloc = 0;
    float *cos_tab = nullptr, *sin_tab = nullptr;
    float *x = nullptr, *h = nullptr, *qkv = nullptr, *attn_out = nullptr, *sw = nullptr, *logits = nullptr;
    unsigned long long *best = nullptr;
    uint32_t n_best = 0;
    float *attn_part = nullptr;
    uint32_t attn_chunk = 64, attn_max_splits = 1;
    uint32_t *attn_counters = nullptr; // arrival counters of the in-kernel attention merge (zero between steps)
    int attn_merge_mode = 0;           // merge policy fixed at creation (rfp4_debug_attn_merge)
    // tagged attention merge: per layer [n_heads][attn_tag_splits][head_dim + 4] 64-bit words,
    // cleared before each generation (tags are sequence lengths)
    unsigned long long *attn_tagged = nullptr;
    uint32_t attn_tag_splits = 0;
    size_t attn_tag_layer = 0; // words per layer
    uint32_t attn_head_split = 0;      // query-head slices per KV head (0: per grid, attn_head_split_for)
    // fused q|k|v GEMV + attention launch (device/qkva.h): rows per wave of its
    // GEMV tiles (0 = no fused kernel for this shape), its tagged q|k|v words
    // (one region per layer: the tag is the step's sequence length, so a
    // layer must not see another layer's words of the same step; cleared with
    // the tagged merge workspace), the policy fixed at creation
    uint32_t qkva_R = 0;
    unsigned long long *qkv_t = nullptr;
    int qkva_mode = 0; // 0 = fused for one-split steps, 1 = two launches, 2 = fused wherever the grid fits
    StepState *state = nullptr;
    uint32_t *ids = nullptr, *last_tok = nullptr;
    uint32_t ids_alloc = 0;
    uint32_t embed_bf16 = 0; // embeddings hold bf16 (1) or fp16 (0) bits; norms are fp16
    // one step graph per attention split count (index = splits launched), captured on demand
    std::vector<hipGraph_t> graphs;
    std::vector<hipGraphExec_t> graph_execs;
    bool use_graph = true;
    // host mirror of the cursor, for bounds checks
    int64_t h_pos = 0, h_step = 0, h_ids_cap = 0;
    bool armed = false;
    // batched prefill workspace (rows of the prompt), grown on demand
    uint32_t pf_cap = 0;
    float *pf_x = nullptr, *pf_c = nullptr, *pf_a = nullptr, *pf_part = nullptr; // pf_part: decode-kernel test path only
    uint8_t *pf_codes = nullptr, *pf_scales = nullptr;
    uint8_t *pf_scales_t = nullptr; // the activation scales step-blocked, written beside pf_scales
    // the SwiGLU rows' MXFP4 (the down projection's input) where the gate|up
    // GEMM's epilogue writes them: not pf_codes, which that GEMM is reading;
    // pf_q_alt: the last MXFP4 rows written are these (prefill buffer hook)
    uint8_t *pf_codes2 = nullptr, *pf_scales2 = nullptr, *pf_scales_t2 = nullptr;
    bool pf_q_alt = false;
    uint32_t *pf_ids = nullptr;
    // persistent decode (one cooperative launch for all layers of a step)
    bool persist_ok = false, persist = false; // shape and device allow it / chosen
    PersistLayer *p_layers = nullptr;       // device copy of the layer table
    uint32_t *p_flags = nullptr;
    uint32_t *p_err = nullptr; // set by a device-side wait that hit its spin limit (grid barrier, tagged merge)
    uint32_t p_gen = 0, p_grid = 0, p_lds = 0;
};

static int dalloc(llama_engine *e, void **p, size_t bytes)
{
    int rc = hip_check(hipMalloc(p, bytes), "hipMalloc(engine)");
    if (!rc) e->allocs.push_back(*p);
    return rc;
}

template <typename T>
static int dalloc_t(llama_engine *e, T **p, size_t count)
{
    return dalloc(e, (void **)p, count * sizeof(T));
}

static uint32_t qdim(const rfp4_model_config &c) { return c.n_heads * c.head_dim; }
static uint32_t kvdim(const rfp4_model_config &c) { return c.n_kv_heads * c.head_dim; }
static uint32_t scale_bytes(const rfp4_model_config &c) { return c.scale_format == RFP4_SCALE_F32 ? 4u : 1u; }
static uint32_t kv_bytes(const rfp4_model_config &c) { return c.kv_format == RFP4_KV_F32 ? 4u : 2u; }
// Layer l's K (isv 0) or V (1) cache: [kvh][max_seq_alloc][hd] elements.
static void *kv_layer(const llama_engine *e, uint32_t l, int isv)
{
    const size_t per = (size_t)e->c.n_kv_heads * e->max_seq_alloc * e->c.head_dim * e->kvb;
    return (char *)(isv ? e->vcache : e->kcache) + (size_t)l * per;
}

// Whether the engine can prefill (llama_engine_prefill's shape and format
// conditions): only then does it hold step-blocked weight scales.
static bool prefill_shape_ok(const rfp4_model_config &c)
{
    return c.dim % 256u == 0 && qdim(c) % 256u == 0 && c.ffn % 256u == 0 && c.scale_format == RFP4_SCALE_E8M0 &&
           c.kv_format == RFP4_KV_F16;
}

static int validate(const rfp4_model_config &c)
{
    if (!c.dim || !c.n_layers || !c.n_heads || !c.n_kv_heads || !c.head_dim || !c.ffn || !c.vocab || !c.max_seq)
        return set_error(RFP4_E_SHAPE, "model config has a zero dimension");
    if (c.head_dim != 64 && c.head_dim != 128) return set_error(RFP4_E_SHAPE, "head_dim %u unsupported (64, 128)", c.head_dim);
    if (c.n_heads % c.n_kv_heads || c.n_heads / c.n_kv_heads > 8)
        return set_error(RFP4_E_SHAPE, "n_heads %u / n_kv_heads %u: group must divide and be <= 8", c.n_heads, c.n_kv_heads);
    if (c.dim % 32 || c.ffn % 32 || qdim(c) % 32) return set_error(RFP4_E_SHAPE, "dim, ffn and n_heads*head_dim must be multiples of 32");
    if (c.n_heads > kAttnMaxHeads) return set_error(RFP4_E_SHAPE, "n_heads %u > %u", c.n_heads, kAttnMaxHeads);
    if (c.scale_format > RFP4_SCALE_F32) return set_error(RFP4_E_INVALID, "scale_format %u unknown", c.scale_format);
    if (c.kv_format > RFP4_KV_F32) return set_error(RFP4_E_INVALID, "kv_format %u unknown", c.kv_format);
    return RFP4_OK;
}

// ---------------------------------------------------------------- step enqueue
// The fused q|k|v GEMV + attention launch (device/qkva.h) of a step with
// `nsplit` attention splits: kernel name, query-head slices, GEMV tiles,
// attention workgroups and grid.  False where the engine has no fused kernel
// for its shape, the policy says two launches, or the grid does not fit the
// device at once (the attention workgroups wait for the GEMV tiles' words,
// so every workgroup must be resident).  The default policy fuses one-split
// steps only.  Measured (graph replays, tok/s, separate -> fused): TinyLlama
// at context 16-270 2235 -> 2304, at 300 2083 -> 2121, at 1000 (16 splits)
// 1909 -> 1891; Llama-3-8B at context 16 779 -> 791, at 1000 (16 splits)
// 730 -> 735, at 4096 (29 splits) 668 -> 656: with many splits the GEMV
// tiles and the K/V stream share the launch's bandwidth and the attention
// starts only after the last tile, which costs more than the kernel
// boundary saves.
struct QkvaPlan {
    char name[48];
    uint32_t hs, n_tiles, n_attn, grid;
};

static bool qkva_plan(const llama_engine *e, uint32_t nsplit, bool tagged, QkvaPlan *pl)
{
    const rfp4_model_config &c = e->c;
    if (!e->qkva_R || e->qkva_mode == 1 || (e->qkva_mode == 0 && nsplit > 1)) return false;
    Runtime *rt = runtime();
    const uint32_t G = c.n_heads / c.n_kv_heads;
    const uint32_t hs = e->attn_head_split ? e->attn_head_split
                                           : attn_head_split_for(c.n_heads, c.n_kv_heads, nsplit, (uint32_t)rt->num_cus);
    if (hs == 0 || G % hs) return false;
    const uint32_t rows = qdim(c) + 2u * kvdim(c);
    pl->hs = hs;
    pl->n_attn = c.n_kv_heads * hs * nsplit;
    // 1 row per wave first where compiled (HD 64), then the engine's rows per
    // wave: the first whose whole grid fits the device at once
    for (uint32_t R : {1u, e->qkva_R}) {
        if (R == 1u && c.head_dim != 64) continue;
        snprintf(pl->name, sizeof pl->name, "rfp4_qkva_hd%u_g%u%s%s", c.head_dim, attn_group_pad(G / hs), tagged ? "_t" : "",
                 R == 1u && e->qkva_R != 1u ? "_r1" : "");
        pl->n_tiles = (rows + 4u * R - 1u) / (4u * R);
        pl->grid = std::max(pl->n_tiles, pl->n_attn);
        int per_cu = 0;
        if (kernel_occupancy(pl->name, 256, gemv_lds_bytes(c.dim), &per_cu) || per_cu < 1) continue;
        if ((uint64_t)per_cu * (uint64_t)rt->num_cus >= pl->grid) return true;
    }
    return false;
}

// Layer l's attention arguments in a decode step with `nsplit` splits: the
// merge by arrival counters (up to 8 splits), by tagged states (9-32) or by
// the merge kernel; every device-side wait of the step reports to p_err.
static AttnArgs step_attn_args(const llama_engine *e, uint32_t l, uint32_t nsplit)
{
    const rfp4_model_config &c = e->c;
    const uint32_t qd = qdim(c), kvd = kvdim(c), hd = c.head_dim;
    AttnArgs aa{};
    aa.q = e->qkv; aa.kc = kv_layer(e, l, 0); aa.vc = kv_layer(e, l, 1); aa.out = e->attn_out;
    aa.part = e->attn_part; aa.pos_ptr = &e->state->pos;
    aa.cosv = e->cos_tab; aa.sinv = e->sin_tab; aa.k_new = e->qkv + qd; aa.v_new = e->qkv + qd + kvd;
    aa.ts = hd; aa.hs = (uint64_t)e->max_seq_alloc * hd;
    aa.n_heads = c.n_heads; aa.n_kv_heads = c.n_kv_heads; aa.head_dim = hd; aa.seq = 0;
    aa.chunk = e->attn_chunk; aa.max_splits = e->attn_max_splits;
    aa.err = e->p_err; // every device-side wait (tagged merge, fused q|k|v poll) reports here
    if (e->attn_tagged && attn_tagged_mode(e->attn_merge_mode, nsplit)) {
        aa.tagged = e->attn_tagged + (size_t)l * e->attn_tag_layer;
        aa.tag_splits = e->attn_tag_splits;
    } else {
        aa.counters = attn_inmerge_mode(e->attn_merge_mode, nsplit) ? e->attn_counters : nullptr;
    }
    aa.head_split = e->attn_head_split;
    return aa;
}

// The decode step at a position whose context needs `nsplit` attention
// splits: the attention grid launches exactly those, and up to 8 splits are
// merged inside the attention kernel (attn_inmerge_mode).  Where the fused
// kernel applies, the q|k|v GEMV and the attention are one launch.
static int enqueue_step(llama_engine *e, uint32_t nsplit)
{
    const rfp4_model_config &c = e->c;
    hipStream_t s = e->stream;
    const uint32_t qd = qdim(c), kvd = kvdim(c), hd = c.head_dim;
    int rc;
    const char *sn = e->sname;
    for (uint32_t l = 0; l < c.n_layers; l++) {
        const LayerW &w = e->L[l];
        GemvArgs qa{w.qkv_c, w.qkv_s, e->x, e->qkv, nullptr, e->norm_attn + (size_t)l * c.dim, qd + 2 * kvd, c.dim, 0, c.eps};
        AttnArgs aa = step_attn_args(e, l, nsplit);
        QkvaPlan pl;
        if (qkva_plan(e, nsplit, aa.tagged != nullptr, &pl)) {
            unsigned long long *yt = e->qkv_t + (size_t)l * (qd + 2 * kvd);
            QkvaArgs fa{qa, aa, yt, pl.n_tiles, pl.n_attn};
            fa.a.head_split = pl.hs;
            fa.a.qkv_t = yt;
            if ((rc = launch(pl.name, dim3(pl.grid), dim3(256), s, &fa, gemv_lds_bytes(c.dim)))) return rc;
            // more splits than either in-kernel merge takes: the merge kernel
            if (nsplit > 1 && !aa.counters && !aa.tagged &&
                (rc = launch(hd == 64 ? "rfp4_attn_merge_hd64" : "rfp4_attn_merge_hd128", dim3(c.n_heads), dim3(256), s, &aa)))
                return rc;
        } else {
            if ((rc = gemv_launch_v(sn, RFP4_EPI_STORE, qa, s, e->gv[GV_QKV]))) return rc;
            if ((rc = attn_launch(aa, e->kvb == 2 ? 1 : 0, s, e->attn_chunk * nsplit, 1))) return rc;
        }
        GemvArgs oa{w.o_c, w.o_s, e->attn_out, e->x, nullptr, nullptr, c.dim, qd, 0, 0.0f};
        if ((rc = gemv_launch_v(sn, RFP4_EPI_RESIDUAL, oa, s, e->gv[GV_O]))) return rc;
        GemvArgs ga{w.gu_c, w.gu_s, e->x, e->sw, nullptr, e->norm_ffn + (size_t)l * c.dim, c.ffn, c.dim, c.ffn, c.eps};
        if ((rc = gemv_launch_v(sn, RFP4_EPI_SWIGLU, ga, s, e->gv[GV_GU]))) return rc;
        GemvArgs da{w.d_c, w.d_s, e->sw, e->x, nullptr, nullptr, c.dim, c.ffn, 0, 0.0f};
        if ((rc = gemv_launch_v(sn, RFP4_EPI_RESIDUAL, da, s, e->gv[GV_D]))) return rc;
    }
    GemvArgs la{e->lm_c, e->lm_s, e->x, e->logits, e->best, e->norm_final, c.vocab, c.dim, 0, c.eps};
    if ((rc = gemv_launch_v(sn, RFP4_EPI_ARGMAX, la, s, e->gv[GV_LM]))) return rc;
    StepArgs sa{e->best, e->state, e->ids, e->last_tok, e->n_best, 0,
                e->no_embed ? nullptr : e->embed, e->x, c.dim, c.vocab, e->embed_bf16, 0};
    return launch("rfp4_step", dim3(1), dim3(1024), s, &sa);
}

// ---------------------------------------------------------------- persistent decode
// The shape rfp4_decode_layers_8b is compiled for (device/persist.h
// PersistShape8B): Llama-3-8B widths at one workgroup of 256 threads per CU on
// a 256-CU device; any layer count, vocabulary and context whose attention
// splits fit the grid and the in-place merge.
static const char *kPersistKernel = "rfp4_decode_layers_8b";
static const uint32_t kPersistGrid = 256, kPersistMaxSplits = 32;

static uint32_t persist_barriers(const llama_engine *e) { return 5u * e->c.n_layers - 1u; }

static int persist_setup(llama_engine *e)
{
    const rfp4_model_config &c = e->c;
    Runtime *rt = runtime();
    if (c.dim != 4096 || c.n_heads != 32 || c.n_kv_heads != 8 || c.head_dim != 128 || c.ffn != 14336) return RFP4_OK;
    if (c.scale_format != RFP4_SCALE_E8M0 || c.kv_format != RFP4_KV_F16) return RFP4_OK;
    if ((uint32_t)rt->num_cus != kPersistGrid) return RFP4_OK;
    if (e->attn_max_splits > kPersistMaxSplits || c.n_kv_heads * e->attn_max_splits > kPersistGrid) return RFP4_OK;
    const uint32_t kmax = std::max(std::max(c.dim, qdim(c)), c.ffn);
    e->p_lds = gemv_lds_bytes(kmax);
    int per_cu = 0;
    int rc = kernel_occupancy(kPersistKernel, 256, e->p_lds, &per_cu);
    if (rc || per_cu < 1) return rc;
    std::vector<PersistLayer> tab(c.n_layers);
    for (uint32_t l = 0; l < c.n_layers; l++) {
        const LayerW &w = e->L[l];
        tab[l] = PersistLayer{w.qkv_c, w.qkv_s, w.o_c, w.o_s, w.gu_c, w.gu_s, w.d_c, w.d_s};
    }
    rc = dalloc_t(e, &e->p_layers, c.n_layers);
    if (!rc) rc = hip_check(hipMemcpy(e->p_layers, tab.data(), tab.size() * sizeof(PersistLayer), hipMemcpyHostToDevice),
                            "H2D layer table");
    if (!rc) rc = dalloc_t(e, &e->p_flags, kPersistGrid);
    if (!rc) rc = fill_words(e->p_flags, kPersistGrid, 0u, e->stream);
    if (rc) return rc;
    e->p_grid = kPersistGrid;
    e->persist_ok = true; // available; the graph step stays the default (faster, measured)
    return RFP4_OK;
}

// One decode step with every layer in the persistent kernel: embedding,
// rfp4_decode_layers, LM head + argmax, cursor.
static int enqueue_step_persist(llama_engine *e)
{
    const rfp4_model_config &c = e->c;
    hipStream_t s = e->stream;
    int rc;
    if (e->p_gen > 0x40000000u) { // barrier generations restart from zero (stream order: no launch still polls)
        if ((rc = fill_words(e->p_flags, e->p_grid, 0u, s))) return rc;
        e->p_gen = 0;
    }
    PersistArgs pa{};
    pa.layers = e->p_layers;
    pa.norm_attn = e->norm_attn;
    pa.norm_ffn = e->norm_ffn;
    pa.kcache = e->kcache;
    pa.vcache = e->vcache;
    pa.kv_layer_elems = (uint64_t)c.n_kv_heads * e->max_seq_alloc * c.head_dim;
    pa.cosv = e->cos_tab;
    pa.sinv = e->sin_tab;
    pa.state = e->state;
    pa.x = e->x;
    pa.qkv = e->qkv;
    pa.att = e->attn_out;
    pa.sw = e->sw;
    pa.part = e->attn_part;
    pa.counters = e->attn_counters;
    pa.flags = e->p_flags;
    pa.err = e->p_err;
    pa.n_layers = c.n_layers;
    pa.dim = c.dim;
    pa.n_heads = c.n_heads;
    pa.n_kv_heads = c.n_kv_heads;
    pa.head_dim = c.head_dim;
    pa.ffn = c.ffn;
    pa.max_seq_alloc = e->max_seq_alloc;
    pa.chunk = e->attn_chunk;
    pa.max_splits = e->attn_max_splits;
    pa.gen0 = e->p_gen;
    pa.spin_limit = 1u << 20;
    pa.eps = c.eps;
    if ((rc = launch_coop(kPersistKernel, dim3(e->p_grid), dim3(256), s, &pa, e->p_lds))) return rc;
    e->p_gen += persist_barriers(e);
    GemvArgs la{e->lm_c, e->lm_s, e->x, e->logits, e->best, e->norm_final, c.vocab, c.dim, 0, c.eps};
    if ((rc = gemv_launch_v(e->sname, RFP4_EPI_ARGMAX, la, s, e->gv[GV_LM]))) return rc;
    StepArgs sa{e->best, e->state, e->ids, e->last_tok, e->n_best, 0,
                e->no_embed ? nullptr : e->embed, e->x, c.dim, c.vocab, e->embed_bf16, 0};
    return launch("rfp4_step", dim3(1), dim3(1024), s, &sa);
}

// A grid barrier of the persistent kernel, a tagged attention merge or the
// fused q|k|v + attention launch's poll that hit its spin limit leaves the
// error word set: the generation's results are not valid.  The word is
// cleared when the next generation begins (llama_engine_begin*).
static int wait_check(llama_engine *e)
{
    if (!e->persist_ok && !e->attn_tagged && !e->qkva_R) return RFP4_OK;
    uint32_t err = 0;
    int rc = hip_check(hipMemcpyAsync(&err, e->p_err, 4, hipMemcpyDeviceToHost, e->stream), "D2H wait error");
    if (!rc) rc = hip_check(hipStreamSynchronize(e->stream), "hipStreamSynchronize(wait error)");
    if (rc) return rc;
    if (err)
        return set_error(RFP4_E_WAIT, "decode: a device-side wait hit its spin limit (persistent grid barrier, tagged "
                                      "attention merge or fused q|k|v poll: workgroups not co-resident); the "
                                      "generation's tokens are invalid");
    return RFP4_OK;
}

// Before a generation: no word of the tagged merge workspace may carry a tag
// (sequence length) that this generation's steps will use.
static int tag_clear(llama_engine *e)
{
    int rc = RFP4_OK;
    if (e->qkv_t)
        rc = fill_words((uint32_t *)e->qkv_t, (size_t)e->c.n_layers * (qdim(e->c) + 2u * kvdim(e->c)) * 2u, 0u, e->stream);
    if (rc || !e->attn_tagged) return rc;
    return fill_words((uint32_t *)e->attn_tagged, e->attn_tag_layer * e->c.n_layers * 2, 0u, e->stream);
}

// ---------------------------------------------------------------- batched prefill
static void dfree(llama_engine *e, void *p)
{
    if (!p) return;
    hipFree(p);
    for (size_t i = 0; i < e->allocs.size(); i++)
        if (e->allocs[i] == p) {
            e->allocs.erase(e->allocs.begin() + (long)i);
            break;
        }
}

static int prefill_reserve(llama_engine *e, uint32_t n)
{
    if (n <= e->pf_cap) return RFP4_OK;
    const rfp4_model_config &c = e->c;
    const uint32_t qd = qdim(c), kvd = kvdim(c);
    const uint32_t cap = (n + 255u) / 256u * 256u;
    hipStreamSynchronize(e->stream);
    dfree(e, e->pf_x); dfree(e, e->pf_c); dfree(e, e->pf_a); dfree(e, e->pf_part);
    dfree(e, e->pf_codes); dfree(e, e->pf_scales); dfree(e, e->pf_scales_t); dfree(e, e->pf_ids);
    dfree(e, e->pf_codes2); dfree(e, e->pf_scales2); dfree(e, e->pf_scales_t2);
    e->pf_x = e->pf_c = e->pf_a = e->pf_part = nullptr;
    e->pf_codes = e->pf_scales = e->pf_scales_t = nullptr;
    e->pf_codes2 = e->pf_scales2 = e->pf_scales_t2 = nullptr;
    e->pf_ids = nullptr;
    e->pf_cap = 0;
    const size_t kmax = std::max(std::max(c.dim, qd), c.ffn);
    const size_t ncols = std::max(std::max(qd + 2 * kvd, 2 * c.ffn), c.dim);
    int rc = RFP4_OK;
    if (!e->gemm_part) {
        rc = dalloc_t(e, &e->gemm_part, kGemmWorkspaceWords);
        if (!rc) rc = fill_words((uint32_t *)(e->gemm_part + kGemmPartFloats), kGemmCounters, 0u, e->stream);
    }
    if (!rc) rc = dalloc_t(e, &e->pf_x, (size_t)cap * c.dim);
    if (!rc) rc = dalloc_t(e, &e->pf_c, (size_t)cap * ncols);
    if (!rc) rc = dalloc_t(e, &e->pf_a, (size_t)cap * qd);
    if (!rc) rc = dalloc_t(e, &e->pf_codes, (size_t)cap * kmax / 2);
    if (!rc) rc = dalloc_t(e, &e->pf_scales, (size_t)cap * kmax / 32);
    if (!rc) rc = dalloc_t(e, &e->pf_scales_t, scales_tiled_bytes(cap, (uint32_t)kmax));
    if (!rc) rc = dalloc_t(e, &e->pf_codes2, (size_t)cap * c.ffn / 2);
    if (!rc) rc = dalloc_t(e, &e->pf_scales2, (size_t)cap * c.ffn / 32);
    if (!rc) rc = dalloc_t(e, &e->pf_scales_t2, scales_tiled_bytes(cap, c.ffn));
    if (!rc) rc = dalloc_t(e, &e->pf_ids, cap);
    if (!rc) e->pf_cap = cap;
    return rc;
}

// The prompt through the MXFP4 GEMM: llama_run/src/main.rs:550-556 feed it
// token by token; here all n positions of a layer run at once, every
// projection input quantised to MXFP4 per 32 along K (the GEMM is FP4 x FP4).
// enqueue_prefill's return when the rfp4_debug_prefill_stop hook ended it early
constexpr int kPrefillStopped = 1;

static int enqueue_prefill(llama_engine *e, uint32_t n, uint32_t pos0)
{
    const rfp4_model_config &c = e->c;
    hipStream_t s = e->stream;
    const uint32_t qd = qdim(c), kvd = kvdim(c), hd = c.head_dim, nqkv = qd + 2 * kvd;
    int rc;
    e->pf_q_alt = false;
    RowsArgs ea{};
    ea.ids = e->pf_ids; ea.embed = e->embed; ea.y = e->pf_x; ea.rows = n; ea.k = c.dim; ea.vocab = c.vocab;
    ea.bf16 = e->embed_bf16;
    if ((rc = launch("rfp4_embed_rows", dim3(n), dim3(256), s, &ea))) return rc;
    // test hook: stop after stage `stop` (-1: the embedding; 10 * layer + s: stage s of that layer)
    const int stop = prefill_stop();
    if (stop == -1) return kPrefillStopped;
#define RFP4_PF_STAGE(S) \
    if (stop == (int)(10u * l + (S))) return kPrefillStopped
    // the down projection added into x by its GEMM (else left in pf_c for the next norm to add)
    bool down_in_x = false;
    for (uint32_t l = 0; l < c.n_layers; l++) {
        const LayerW &w = e->L[l];
        uint16_t *kc = (uint16_t *)kv_layer(e, l, 0), *vc = (uint16_t *)kv_layer(e, l, 1); // fp16 (checked by the caller)
        RowsArgs na{};
        na.x = e->pf_x; na.w = e->norm_attn + (size_t)l * c.dim; na.codes = e->pf_codes; na.scales = e->pf_scales;
        na.scales_t = e->pf_scales_t; na.rows = n; na.k = c.dim; na.eps = c.eps;
        // layer l > 0: the previous layer's down projection (pf_c) is added into the residual stream here
        // (unless its GEMM added it into x)
        na.add = l > 0 && !down_in_x ? e->pf_c : nullptr;
        na.x_out = e->pf_x;
        if ((rc = launch("rfp4_rmsnorm_quant_rows", dim3(n), dim3(256), s, &na))) return rc;
        e->pf_q_alt = false;
        RFP4_PF_STAGE(0);
        // q|k|v: RoPE and the fp16 K/V cache rows in the GEMM's epilogue
        // where the plan has that kernel (bit-identical to the row kernel
        // after the GEMM; not when the stage test hook wants the GEMM's output)
        const uint64_t kv_hs = (uint64_t)e->max_seq_alloc * hd;
        if (stop != (int)(10u * l + 1u) && prefill_rope_mode() == 0 && gemm_rope_ok(n, nqkv, c.dim, hd)) {
            const GemmRope gr{e->cos_tab, e->sin_tab, kc, vc, hd, kv_hs, pos0, qd, kvd, hd};
            if ((rc = gemm_rope_launch(s, n, nqkv, c.dim, e->pf_codes, e->pf_scales, e->pf_scales_t, w.qkv_c, w.qkv_s,
                                       w.qkv_st, e->pf_c, gr))) return rc;
        } else {
            if ((rc = gemm_launch(s, n, nqkv, c.dim, e->pf_codes, e->pf_scales, e->pf_scales_t, w.qkv_c, w.qkv_s,
                                  w.qkv_st, e->pf_c, e->gemm_part))) return rc;
            RFP4_PF_STAGE(1);
            RopeRowsArgs ra{};
            ra.qkv = e->pf_c; ra.cosv = e->cos_tab; ra.sinv = e->sin_tab; ra.kc = kc; ra.vc = vc;
            ra.ts = hd; ra.hs = kv_hs;
            ra.rows = n; ra.row_stride = nqkv; ra.n_heads = c.n_heads; ra.n_kv_heads = c.n_kv_heads;
            ra.head_dim = hd; ra.pos0 = pos0;
            if ((rc = launch("rfp4_rope_kv_rows", dim3(n), dim3(256), s, &ra))) return rc;
        }
        RFP4_PF_STAGE(2);
        // causal attention of the prompt rows (row r sees positions 0 .. pos0 + r)
        bool attn_q = false; // quantized by the attention kernel itself
        if (prefill_attn_mode() == 1) {
            // test path: the decode kernel, one query row per grid z (split states per row)
            if (!e->pf_part &&
                (rc = dalloc_t(e, &e->pf_part, (size_t)e->pf_cap * c.n_heads * e->attn_max_splits * (hd + 4))))
                return rc;
            AttnArgs aa{};
            aa.q = e->pf_c; aa.q_rs = nqkv; aa.kc = kc; aa.vc = vc; aa.out = e->pf_a; aa.out_rs = qd;
            aa.part = e->pf_part; aa.pos_ptr = nullptr; aa.seq = pos0 + 1;
            aa.ts = hd; aa.hs = (uint64_t)e->max_seq_alloc * hd;
            aa.n_heads = c.n_heads; aa.n_kv_heads = c.n_kv_heads; aa.head_dim = hd;
            aa.chunk = e->attn_chunk; aa.max_splits = e->attn_max_splits;
            if ((rc = attn_launch(aa, 1, s, pos0 + n, n))) return rc;
        } else {
            // the attention rows quantized to MXFP4 in the kernel's epilogue
            // (the row quantizer's bytes; no f32 rows), unless the stage test
            // hook wants the f32 rows
            attn_q = stop != (int)(10u * l + 3u) && prefill_attn_quant_mode() == 0;
            AttnPrefillArgs pa{e->pf_c, kc, vc, attn_q ? nullptr : e->pf_a, hd, (uint64_t)e->max_seq_alloc * hd, nqkv, qd,
                               c.n_heads, c.n_kv_heads, pos0, n, 0u}; // pairing: chosen by the launcher
            if (attn_q) {
                pa.q_codes = e->pf_codes;
                pa.q_scales = e->pf_scales;
                pa.q_scales_t = e->pf_scales_t;
            }
            if ((rc = attn_prefill_launch(pa, hd, s))) return rc;
        }
        RFP4_PF_STAGE(3);
        if (!attn_q && (rc = mx4_quantize_st(s, n, qd, e->pf_a, 0, e->pf_codes, e->pf_scales, e->pf_scales_t))) return rc;
        e->pf_q_alt = false;
        RFP4_PF_STAGE(4);
        // o: x += O projection in the GEMM's epilogue (the residual add's
        // arithmetic; not when the stage test hook wants the GEMM's output)
        const bool o_in_x = stop != (int)(10u * l + 5u) && gemm_accumulate_ok(n, c.dim, qd);
        if ((rc = gemm_launch(s, n, c.dim, qd, e->pf_codes, e->pf_scales, e->pf_scales_t, w.o_c, w.o_s, w.o_st,
                              o_in_x ? e->pf_x : e->pf_c, e->gemm_part, o_in_x))) return rc;
        RFP4_PF_STAGE(5);
        na.w = e->norm_ffn + (size_t)l * c.dim;
        na.add = o_in_x ? nullptr : e->pf_c; // x += O projection (unless added already), then the FFN norm
        if ((rc = launch("rfp4_rmsnorm_quant_rows", dim3(n), dim3(256), s, &na))) return rc;
        e->pf_q_alt = false;
        RFP4_PF_STAGE(6);
        // gate|up: SwiGLU and the MXFP4 rows of its output in the GEMM's
        // epilogue where the plan is the 256x256 ping-pong tile (no f32
        // gate|up output; not when the stage test hook wants that output)
        if (stop != (int)(10u * l + 7u) && prefill_swiglu_mode() == 0 && gemm_swiglu_ok(n, c.ffn, c.dim)) {
            if ((rc = gemm_swiglu_launch(s, n, c.ffn, c.dim, e->pf_codes, e->pf_scales, e->pf_scales_t, w.gu_c, w.gu_s,
                                         w.gu_st, e->pf_codes2, e->pf_scales2, e->pf_scales_t2))) return rc;
            e->pf_q_alt = true;
        } else {
            if ((rc = gemm_launch(s, n, 2 * c.ffn, c.dim, e->pf_codes, e->pf_scales, e->pf_scales_t, w.gu_c, w.gu_s,
                                  w.gu_st, e->pf_c, e->gemm_part))) return rc;
            RFP4_PF_STAGE(7);
            RowsArgs sa{};
            sa.x = e->pf_c; sa.codes = e->pf_codes; sa.scales = e->pf_scales; sa.scales_t = e->pf_scales_t;
            sa.rows = n; sa.k = c.ffn;
            // parts of about 1024 float4 per row (measured: 8B 512 rows x 14336)
            if ((rc = launch("rfp4_swiglu_quant_rows", dim3(n, std::max(1u, (c.ffn / 4u + 1023u) / 1024u)), dim3(256), s,
                             &sa)))
                return rc;
        }
        RFP4_PF_STAGE(8);
        uint8_t *dc = e->pf_q_alt ? e->pf_codes2 : e->pf_codes, *ds = e->pf_q_alt ? e->pf_scales2 : e->pf_scales;
        uint8_t *dst_ = e->pf_q_alt ? e->pf_scales_t2 : e->pf_scales_t;
        down_in_x = stop != (int)(10u * l + 9u) && gemm_accumulate_ok(n, c.dim, c.ffn);
        if ((rc = gemm_launch(s, n, c.dim, c.ffn, dc, ds, dst_, w.d_c, w.d_s, w.d_st, down_in_x ? e->pf_x : e->pf_c,
                              e->gemm_part, down_in_x))) return rc;
        RFP4_PF_STAGE(9);
        // x += down projection: in its GEMM, else by the next layer's first norm, after the last layer here
        if (l + 1 == c.n_layers && !down_in_x && (rc = residual(s, n * c.dim, e->pf_c, e->pf_x))) return rc;
    }
#undef RFP4_PF_STAGE
    // last row: the decode step's final norm + LM head, then argmax
    rc = hip_check(hipMemcpyAsync(e->x, e->pf_x + (size_t)(n - 1) * c.dim, c.dim * sizeof(float),
                                  hipMemcpyDeviceToDevice, s), "hipMemcpyAsync(prefill row)");
    GemvArgs la{e->lm_c, e->lm_s, e->x, e->logits, nullptr, e->norm_final, c.vocab, c.dim, 0, c.eps};
    if (!rc) rc = gemv_launch(e->sname, RFP4_EPI_STORE, la, s);
    if (!rc) rc = argmax(s, c.vocab, e->logits, e->last_tok);
    return rc;
}

static uint32_t splits_at(const llama_engine *e, int64_t pos)
{
    const uint64_t ns = ((uint64_t)pos + e->attn_chunk) / e->attn_chunk; // ceil((pos + 1) / chunk)
    return (uint32_t)(ns < e->attn_max_splits ? ns : e->attn_max_splits);
}

// The step graph for `nsplit` attention splits (captured once).
static int step_graph(llama_engine *e, uint32_t nsplit, hipGraphExec_t *out)
{
    if (e->graph_execs.size() <= nsplit) {
        e->graph_execs.resize(nsplit + 1, nullptr);
        e->graphs.resize(nsplit + 1, nullptr);
    }
    if (!e->graph_execs[nsplit]) {
        int rc = hip_check(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
        if (rc) return rc;
        int rc_enq = enqueue_step(e, nsplit);
        hipGraph_t g = nullptr;
        rc = hip_check(hipStreamEndCapture(e->stream, &g), "hipStreamEndCapture");
        if (rc_enq) {
            if (g) hipGraphDestroy(g);
            return rc_enq;
        }
        if (rc) return rc;
        e->graphs[nsplit] = g;
        rc = hip_check(hipGraphInstantiate(&e->graph_execs[nsplit], g, nullptr, nullptr, 0), "hipGraphInstantiate");
        if (rc) return rc;
    }
    *out = e->graph_execs[nsplit];
    return RFP4_OK;
}

// Step graphs for every position in [pos_first, pos_last].
static int step_graphs_for(llama_engine *e, int64_t pos_first, int64_t pos_last)
{
    if (!e->use_graph || e->persist) return RFP4_OK;
    hipGraphExec_t g;
    for (uint32_t ns = splits_at(e, pos_first); ns <= splits_at(e, pos_last); ns++) {
        int rc = step_graph(e, ns, &g);
        if (rc) return rc;
    }
    return RFP4_OK;
}

// Drop the captured step graphs (the step's launch list changes with the
// embedding mode); they are captured again on demand.
static void drop_graphs(llama_engine *e)
{
    for (hipGraphExec_t &g : e->graph_execs)
        if (g) hipGraphExecDestroy(g), g = nullptr;
    for (hipGraph_t &g : e->graphs)
        if (g) hipGraphDestroy(g), g = nullptr;
}

// Embedding lookup per step (llama_run) or a carried activation (the
// llama_decode harness): switching drops the graphs of the other mode.
// The first step's embedding row (later steps' rows are gathered by the
// previous step's cursor kernel).
static int embed_first(llama_engine *e)
{
    const rfp4_model_config &c = e->c;
    EmbedArgs ea{e->embed, e->ids, e->state, e->x, c.dim, c.vocab, e->embed_bf16};
    return launch("rfp4_embed", dim3((c.dim + 255) / 256), dim3(256), e->stream, &ea);
}

static int set_embed_mode(llama_engine *e, bool no_embed)
{
    if (e->no_embed == no_embed) return RFP4_OK;
    int rc = hip_check(hipStreamSynchronize(e->stream), "hipStreamSynchronize(mode)");
    if (rc) return rc;
    drop_graphs(e);
    e->no_embed = no_embed;
    return RFP4_OK;
}

// Engines handed out by the creation calls and not yet destroyed: a stale or
// foreign handle given to llama_engine_destroy is refused, and
// rfp4_shutdown destroys whatever is left.
static std::mutex g_engines_mu;
static std::unordered_set<llama_engine *> g_engines;

static void engine_register(llama_engine *e)
{
    std::lock_guard<std::mutex> lk(g_engines_mu);
    g_engines.insert(e);
}

static bool engine_unregister(llama_engine *e)
{
    std::lock_guard<std::mutex> lk(g_engines_mu);
    return g_engines.erase(e) != 0;
}

static void engine_free(llama_engine *e)
{
    if (!e) return;
    engine_unregister(e);
    if (e->stream) hipStreamSynchronize(e->stream);
    drop_graphs(e);
    for (void *p : e->allocs) hipFree(p);
    if (e->stream) hipStreamDestroy(e->stream);
    delete e;
}

size_t rfp4::engines_destroy_all()
{
    std::vector<llama_engine *> live;
    {
        std::lock_guard<std::mutex> lk(g_engines_mu);
        live.assign(g_engines.begin(), g_engines.end());
    }
    for (llama_engine *e : live) engine_free(e);
    return live.size();
}

// ---------------------------------------------------------------- creation
// Device memory of an engine for `cfg` (weights unfilled), KV caches zeroed,
// RoPE tables, activations and workspaces.
static int engine_alloc(const rfp4_model_config *cfg, llama_engine **out)
{
    if (!cfg || !out) return set_error(RFP4_E_INVALID, "llama_engine: null argument");
    *out = nullptr;
    Runtime *rt = runtime();
    if (!rt) return set_error(RFP4_E_NOT_INIT, "rfp4_init has not been called");
    int rc = validate(*cfg);
    if (rc) return rc;
    llama_engine *e = new llama_engine();
    e->c = *cfg;
    const rfp4_model_config &c = e->c;
    const uint32_t qd = qdim(c), kvd = kvdim(c), hd = c.head_dim;
    e->sb = scale_bytes(c);
    e->kvb = kv_bytes(c);
    e->sname = c.scale_format == RFP4_SCALE_F32 ? "f32" : "e8m0";
    const size_t sb = e->sb;
    rc = hip_check(hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking), "hipStreamCreate");
    // attention split plan over the full cache capacity
    e->attn_chunk = attn_chunk_for(c.n_kv_heads, c.max_seq, rt->num_cus, hd, e->kvb, c.n_heads / c.n_kv_heads);
    e->attn_max_splits = (c.max_seq + e->attn_chunk - 1) / e->attn_chunk;
    e->max_seq_alloc = (e->attn_chunk * e->attn_max_splits + 255u) / 256u * 256u;
    hipStream_t s = e->stream;
    e->L.resize(c.n_layers);
    for (uint32_t l = 0; l < c.n_layers && !rc; l++) {
        LayerW &w = e->L[l];
        uint32_t nqkv = qd + 2 * kvd;
        rc = dalloc_t(e, &w.qkv_c, (size_t)nqkv * c.dim / 2);
        if (!rc) rc = dalloc_t(e, &w.qkv_s, (size_t)nqkv * c.dim / 32 * sb);
        if (!rc) rc = dalloc_t(e, &w.o_c, (size_t)c.dim * qd / 2);
        if (!rc) rc = dalloc_t(e, &w.o_s, (size_t)c.dim * qd / 32 * sb);
        if (!rc) rc = dalloc_t(e, &w.gu_c, (size_t)2 * c.ffn * c.dim / 2);
        if (!rc) rc = dalloc_t(e, &w.gu_s, (size_t)2 * c.ffn * c.dim / 32 * sb);
        if (!rc) rc = dalloc_t(e, &w.d_c, (size_t)c.dim * c.ffn / 2);
        if (!rc) rc = dalloc_t(e, &w.d_s, (size_t)c.dim * c.ffn / 32 * sb);
    }
    if (!rc) rc = dalloc_t(e, &e->norm_attn, (size_t)c.n_layers * c.dim);
    if (!rc) rc = dalloc_t(e, &e->norm_ffn, (size_t)c.n_layers * c.dim);
    if (!rc) rc = dalloc_t(e, &e->norm_final, c.dim);
    if (!rc) rc = dalloc_t(e, &e->embed, (size_t)c.vocab * c.dim);
    if (!rc) rc = dalloc_t(e, &e->lm_c, (size_t)c.vocab * c.dim / 2);
    if (!rc) rc = dalloc_t(e, &e->lm_s, (size_t)c.vocab * c.dim / 32 * sb);
    // step-blocked E8M0 scales for the prefill's tiled GEMM (made by engine_finish)
    if (prefill_shape_ok(c)) {
        for (uint32_t l = 0; l < c.n_layers && !rc; l++) {
            LayerW &w = e->L[l];
            rc = dalloc_t(e, &w.qkv_st, scales_tiled_bytes(qd + 2 * kvd, c.dim));
            if (!rc) rc = dalloc_t(e, &w.o_st, scales_tiled_bytes(c.dim, qd));
            if (!rc) rc = dalloc_t(e, &w.gu_st, scales_tiled_bytes(2 * c.ffn, c.dim));
            if (!rc) rc = dalloc_t(e, &w.d_st, scales_tiled_bytes(c.dim, c.ffn));
        }
        if (!rc) rc = dalloc_t(e, &e->lm_st, scales_tiled_bytes(c.vocab, c.dim));
    }
    const size_t kv_bytes_all = (size_t)c.n_layers * c.n_kv_heads * e->max_seq_alloc * hd * e->kvb;
    if (!rc) rc = dalloc(e, &e->kcache, kv_bytes_all);
    if (!rc) rc = dalloc(e, &e->vcache, kv_bytes_all);
    if (!rc) rc = fill_words((uint32_t *)e->kcache, kv_bytes_all / 4, 0u, s);
    if (!rc) rc = fill_words((uint32_t *)e->vcache, kv_bytes_all / 4, 0u, s);
    // rotary table in f64 -> f32 (llama_run/src/main.rs:462-471)
    const uint32_t half = hd / 2;
    std::vector<float> cosv((size_t)e->max_seq_alloc * half), sinv((size_t)e->max_seq_alloc * half);
    for (uint32_t pos = 0; pos < e->max_seq_alloc; pos++)
        for (uint32_t j = 0; j < half; j++) {
            double freq = 1.0 / std::pow(c.theta, 2.0 * (double)j / (double)hd);
            double a = (double)pos * freq;
            cosv[(size_t)pos * half + j] = (float)std::cos(a);
            sinv[(size_t)pos * half + j] = (float)std::sin(a);
        }
    if (!rc) rc = dalloc_t(e, &e->cos_tab, cosv.size());
    if (!rc) rc = dalloc_t(e, &e->sin_tab, sinv.size());
    if (!rc) rc = hip_check(hipMemcpyAsync(e->cos_tab, cosv.data(), cosv.size() * 4, hipMemcpyHostToDevice, s), "H2D cos");
    if (!rc) rc = hip_check(hipMemcpyAsync(e->sin_tab, sinv.data(), sinv.size() * 4, hipMemcpyHostToDevice, s), "H2D sin");
    // the host tables are freed on return: wait for the copies
    if (!rc) rc = hip_check(hipStreamSynchronize(s), "hipStreamSynchronize(tables)");
    // activations and workspaces
    uint32_t big = c.dim > qd ? c.dim : qd;
    if (!rc) rc = dalloc_t(e, &e->x, c.dim);
    if (!rc) rc = dalloc_t(e, &e->h, big);
    if (!rc) rc = dalloc_t(e, &e->qkv, qd + 2 * kvd);
    if (!rc) rc = dalloc_t(e, &e->attn_out, qd);
    if (!rc) rc = dalloc_t(e, &e->sw, c.ffn);
    if (!rc) rc = dalloc_t(e, &e->logits, c.vocab);
    // GEMV variants fixed now: later thread-local overrides cannot change the
    // LM head's grid, whose per-workgroup keys `best` holds
    const bool f32s = c.scale_format == RFP4_SCALE_F32;
    e->gv[GV_QKV] = gemv_variant(qd + 2 * kvd, c.dim, RFP4_EPI_STORE, f32s);
    e->gv[GV_O] = gemv_variant(c.dim, qd, RFP4_EPI_RESIDUAL, f32s);
    e->gv[GV_GU] = gemv_variant(c.ffn, c.dim, RFP4_EPI_SWIGLU, f32s);
    e->gv[GV_D] = gemv_variant(c.dim, c.ffn, RFP4_EPI_RESIDUAL, f32s);
    e->gv[GV_LM] = gemv_variant(c.vocab, c.dim, RFP4_EPI_ARGMAX, f32s);
    e->n_best = gemv_grid(c.vocab, e->gv[GV_LM]);
    // the fused q|k|v GEMV + attention kernels (kernels.hip QKVA_KERNELS):
    // E8M0 weights and fp16 caches, with the q|k|v GEMV variant whose RMS
    // order the fused tile reproduces (bit-identical outputs)
    e->qkva_mode = qkva_mode();
    if (!f32s && c.kv_format == RFP4_KV_F16) {
        const GemvVariant &v = e->gv[GV_QKV];
        if (c.head_dim == 64 && c.dim == 2048 && v.R == 2 && v.NS == 1 && v.W == 8) e->qkva_R = 2;
        if (c.head_dim == 128 && c.dim == 4096 && v.R == 2 && v.NS == 2 && v.W == 4) e->qkva_R = 4;
    }
    if (!rc && e->qkva_R) rc = dalloc_t(e, &e->qkv_t, (size_t)c.n_layers * (qd + 2 * kvd));
    if (!rc) rc = dalloc_t(e, &e->best, e->n_best);
    if (!rc) rc = dalloc_t(e, &e->attn_part, (size_t)c.n_heads * e->attn_max_splits * (hd + 4));
    e->attn_merge_mode = attn_merge_mode();
    {
        const uint32_t g = c.n_heads / c.n_kv_heads, hs = (uint32_t)attn_head_split_mode();
        e->attn_head_split = hs == 0u ? 0u : (g % hs == 0u ? hs : 1u);
    }
    // one arrival counter per attention workgroup column (KV head x query-head slice)
    if (!rc) rc = dalloc_t(e, &e->attn_counters, c.n_heads);
    if (!rc) rc = fill_words(e->attn_counters, c.n_heads, 0u, s);
    if (e->attn_max_splits > 1) {
        e->attn_tag_splits = std::min(e->attn_max_splits, kAttnTagMaxSplits);
        e->attn_tag_layer = (size_t)c.n_heads * e->attn_tag_splits * (hd + 4);
        if (!rc) rc = dalloc_t(e, &e->attn_tagged, e->attn_tag_layer * c.n_layers);
        if (!rc) rc = tag_clear(e);
    }
    if (!rc) rc = tag_clear(e);
    if (!rc) rc = dalloc_t(e, &e->p_err, 1);
    if (!rc) rc = fill_words(e->p_err, 1, 0u, s);
    if (!rc) rc = dalloc(e, (void **)&e->state, sizeof(StepState));
    e->ids_alloc = c.max_seq + 2;
    if (!rc) rc = dalloc_t(e, &e->ids, e->ids_alloc);
    if (!rc) rc = dalloc_t(e, &e->last_tok, 1);
    if (!rc) rc = fill_words((uint32_t *)e->state, sizeof(StepState) / 4, 0u, s);
    if (!rc) rc = fill_words(e->ids, e->ids_alloc, 0u, s);
    if (!rc) rc = persist_setup(e);
    if (rc) {
        engine_free(e);
        return rc;
    }
    *out = e;
    return RFP4_OK;
}

// Synthetic MXFP4 init from `seed` (generated on the device; the CPU oracle
// uses the same counters).
static int engine_synth(llama_engine *e, uint64_t seed)
{
    const rfp4_model_config &c = e->c;
    const uint32_t qd = qdim(c), kvd = kvdim(c);
    hipStream_t s = e->stream;
    const float sigma = 0.02f;
    int rc = RFP4_OK;
    for (uint32_t l = 0; l < c.n_layers && !rc; l++) {
        LayerW &w = e->L[l];
        // q, k, v stacked; each keeps its own stream and local row index
        rc = rfp4_synth_mx_weight(s, seed, stream_w(l, 0), sigma, c.dim, 0, qd, w.qkv_c, w.qkv_s);
        if (!rc) rc = rfp4_synth_mx_weight(s, seed, stream_w(l, 1), sigma, c.dim, 0, kvd, w.qkv_c + (size_t)qd * c.dim / 2,
                                           w.qkv_s + (size_t)qd * c.dim / 32);
        if (!rc) rc = rfp4_synth_mx_weight(s, seed, stream_w(l, 2), sigma, c.dim, 0, kvd,
                                           w.qkv_c + (size_t)(qd + kvd) * c.dim / 2, w.qkv_s + (size_t)(qd + kvd) * c.dim / 32);
        if (!rc) rc = rfp4_synth_mx_weight(s, seed, stream_w(l, 3), sigma, qd, 0, c.dim, w.o_c, w.o_s);
        if (!rc) rc = rfp4_synth_mx_weight(s, seed, stream_w(l, 4), sigma, c.dim, 0, c.ffn, w.gu_c, w.gu_s);
        if (!rc) rc = rfp4_synth_mx_weight(s, seed, stream_w(l, 5), sigma, c.dim, 0, c.ffn,
                                           w.gu_c + (size_t)c.ffn * c.dim / 2, w.gu_s + (size_t)c.ffn * c.dim / 32);
        if (!rc) rc = rfp4_synth_mx_weight(s, seed, stream_w(l, 6), sigma, c.ffn, 0, c.dim, w.d_c, w.d_s);
    }
    for (uint32_t l = 0; l < c.n_layers && !rc; l++) {
        rc = rfp4_synth_f16(s, seed, stream_norm(l, 0), sigma, 1.0f, c.dim, e->norm_attn + (size_t)l * c.dim);
        if (!rc) rc = rfp4_synth_f16(s, seed, stream_norm(l, 1), sigma, 1.0f, c.dim, e->norm_ffn + (size_t)l * c.dim);
    }
    if (!rc) rc = rfp4_synth_f16(s, seed, kStreamNormFinal, sigma, 1.0f, c.dim, e->norm_final);
    if (!rc) rc = rfp4_synth_f16(s, seed, kStreamEmbed, sigma, 0.0f, (size_t)c.vocab * c.dim, e->embed);
    if (!rc) rc = rfp4_synth_mx_weight(s, seed, kStreamLm, sigma, c.dim, 0, c.vocab, e->lm_c, e->lm_s);
    e->embed_bf16 = 0;
    return rc;
}

static int engine_finish(llama_engine *e)
{
    // the weights are final: their step-blocked scale copies (engines that can prefill)
    const rfp4_model_config &c = e->c;
    const uint32_t qd = qdim(c), kvd = kvdim(c);
    int rc = RFP4_OK;
    if (e->lm_st) {
        for (uint32_t l = 0; l < c.n_layers && !rc; l++) {
            const LayerW &w = e->L[l];
            rc = scales_tile_launch(e->stream, c.dim, w.qkv_s, w.qkv_st, qd + 2 * kvd, w.gu_s, w.gu_st, 2 * c.ffn);
            if (!rc) rc = scales_tile_launch(e->stream, qd, w.o_s, w.o_st, c.dim, nullptr, nullptr, 0u);
            if (!rc) rc = scales_tile_launch(e->stream, c.ffn, w.d_s, w.d_st, c.dim, nullptr, nullptr, 0u);
        }
        if (!rc) rc = scales_tile_launch(e->stream, c.dim, e->lm_s, e->lm_st, c.vocab, nullptr, nullptr, 0u);
    }
    // step graphs are captured by llama_engine_begin for the positions it can reach
    if (!rc) rc = hip_check(hipStreamSynchronize(e->stream), "hipStreamSynchronize(create)");
    return rc;
}

// ---------------------------------------------------------------- real weights
// Checkpoint names of the reference's loader (llama_run/src/main.rs:444-460).
static const char *kProjNames[7] = {"self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
                                    "self_attn.o_proj.weight", "mlp.gate_proj.weight",    "mlp.up_proj.weight",
                                    "mlp.down_proj.weight"};

struct ProjDst {
    uint8_t *codes, *scales;
    uint32_t rows, k;
};

// Where projection p of layer l lives in the engine (q, k, v stacked; gate, up stacked).
static ProjDst proj_dst(llama_engine *e, uint32_t l, int p)
{
    const rfp4_model_config &c = e->c;
    const uint32_t qd = qdim(c), kvd = kvdim(c);
    LayerW &w = e->L[l];
    switch (p) {
    case 0: return {w.qkv_c, w.qkv_s, qd, c.dim};
    case 1: return {w.qkv_c + (size_t)qd * c.dim / 2, w.qkv_s + (size_t)qd * c.dim / 32 * e->sb, kvd, c.dim};
    case 2: return {w.qkv_c + (size_t)(qd + kvd) * c.dim / 2, w.qkv_s + (size_t)(qd + kvd) * c.dim / 32 * e->sb, kvd, c.dim};
    case 3: return {w.o_c, w.o_s, c.dim, qd};
    case 4: return {w.gu_c, w.gu_s, c.ffn, c.dim};
    case 5: return {w.gu_c + (size_t)c.ffn * c.dim / 2, w.gu_s + (size_t)c.ffn * c.dim / 32 * e->sb, c.ffn, c.dim};
    default: return {w.d_c, w.d_s, c.dim, c.ffn};
    }
}

// ---------------------------------------------------------------- the reference harness's init
// xorshift32 13/17/5 (llama_decode/src/main.rs:300-305).
static inline uint32_t xorshift32(uint32_t *s)
{
    uint32_t x = *s;
    x ^= x << 13;
    x ^= x >> 17;
    x ^= x << 5;
    *s = x;
    return x;
}

// mk_fp4 (llama_decode/src/main.rs:307-325): rows*k/8 packed words, one
// xorshift output each (uniform codes), then rows*k/32 f32 scales
// 0.25 + (r % 8) * 0.03125, uploaded to the projection's place.
static int mk_fp4_upload(uint32_t *st, const ProjDst &d)
{
    std::vector<uint32_t> w((size_t)d.rows * d.k / 8);
    for (auto &v : w) v = xorshift32(st);
    std::vector<float> sc((size_t)d.rows * (d.k / 32));
    for (auto &v : sc) v = 0.25f + (float)(xorshift32(st) % 8u) * 0.03125f;
    int rc = hip_check(hipMemcpy(d.codes, w.data(), w.size() * 4, hipMemcpyHostToDevice), "H2D weights");
    if (!rc) rc = hip_check(hipMemcpy(d.scales, sc.data(), sc.size() * 4, hipMemcpyHostToDevice), "H2D scales");
    return rc;
}

// f32-scale synthetic init: the reference harness's weights in its order
// (llama_decode/src/main.rs:369-393: per layer q, k, v, o, gate, up, down,
// then the LM head), norms 1.0 (:381-383,392) and the activation vector
// (r % 2001) / 1000 - 1 drawn after them (:421); embeddings as the E8M0
// init's (the harness has none).
static int engine_synth_mk_fp4(llama_engine *e, uint64_t seed)
{
    const rfp4_model_config &c = e->c;
    hipStream_t s = e->stream;
    uint32_t st = (uint32_t)seed;
    int rc = RFP4_OK;
    for (uint32_t l = 0; l < c.n_layers && !rc; l++)
        for (int p = 0; p < 7 && !rc; p++) rc = mk_fp4_upload(&st, proj_dst(e, l, p));
    if (!rc) rc = mk_fp4_upload(&st, ProjDst{e->lm_c, e->lm_s, c.vocab, c.dim});
    e->harness_x.resize(c.dim);
    for (auto &v : e->harness_x) v = (float)(xorshift32(&st) % 2001u) / 1000.0f - 1.0f;
    const uint32_t one2 = 0x3C003C00u; // two fp16 1.0
    if (!rc) rc = fill_words((uint32_t *)e->norm_attn, (size_t)c.n_layers * c.dim / 2, one2, s);
    if (!rc) rc = fill_words((uint32_t *)e->norm_ffn, (size_t)c.n_layers * c.dim / 2, one2, s);
    if (!rc) rc = fill_words((uint32_t *)e->norm_final, c.dim / 2, one2, s);
    if (!rc) rc = rfp4_synth_f16(s, seed, kStreamEmbed, 0.02f, 0.0f, (size_t)c.vocab * c.dim, e->embed);
    e->embed_bf16 = 0;
    return rc;
}

static int st_tensor(const StFile &f, const std::string &name, uint64_t d0, uint64_t d1, const StTensor **out)
{
    const StTensor *t = f.find(name);
    if (!t) return set_error(RFP4_E_SHAPE, "checkpoint has no tensor %s", name.c_str());
    const bool ok = d1 ? (t->shape.size() == 2 && t->shape[0] == d0 && t->shape[1] == d1)
                       : (t->shape.size() == 1 && t->shape[0] == d0);
    if (!ok) {
        std::string sh;
        for (uint64_t d : t->shape) sh += (sh.empty() ? "" : "x") + std::to_string(d);
        return set_error(RFP4_E_SHAPE, "%s has shape [%s], the config needs [%llu%s%s]", name.c_str(), sh.c_str(),
                         (unsigned long long)d0, d1 ? "x" : "", d1 ? std::to_string(d1).c_str() : "");
    }
    if (t->dtype != "BF16" && t->dtype != "F16" && t->dtype != "F32")
        return set_error(RFP4_E_SHAPE, "%s has dtype %s (BF16, F16 or F32 expected)", name.c_str(), t->dtype.c_str());
    *out = t;
    return RFP4_OK;
}

// One [rows][k] checkpoint matrix -> MXFP4 (OCP rules, E8M0 per 32) with the
// device quantizer; bf16 and f32 rows go up as stored, f16 rows widened first.
static int load_proj(llama_engine *e, const StFile &f, const StTensor &t, uint8_t *codes, uint8_t *scales, void *stage)
{
    hipStream_t s = e->stream;
    const uint64_t rows = t.shape[0], k = t.shape[1], n = rows * k;
    int rc;
    if (e->sb == 4) {
        // the reference's packer (llama_run/src/main.rs:334-376) on the host,
        // rows split over threads (each row's result is independent of them)
        std::vector<float> w(n);
        rc = f.read_f32(t, w.data(), n);
        if (rc) return rc;
        std::vector<uint32_t> packed(n / 8);
        std::vector<float> sc(n / 32);
        const uint64_t nt = std::max<uint64_t>(1, std::min<uint64_t>(std::min<uint64_t>(16, rows),
                                                                     std::thread::hardware_concurrency()));
        std::vector<std::thread> th;
        std::vector<int> rcs(nt, 0);
        for (uint64_t i = 0; i < nt; i++) {
            const uint64_t r0 = rows * i / nt, r1 = rows * (i + 1) / nt;
            th.emplace_back([&, i, r0, r1] {
                if (r1 > r0)
                    rcs[i] = fp4_quantize_absmax(w.data() + r0 * k, (uint32_t)(r1 - r0), (uint32_t)k,
                                                 packed.data() + r0 * k / 8, sc.data() + r0 * k / 32);
            });
        }
        for (auto &x : th) x.join();
        for (int r : rcs)
            if (r) return set_error(RFP4_E_SHAPE, "absmax quantization of %s failed", t.name.c_str());
        rc = hip_check(hipMemcpy(codes, packed.data(), n / 2, hipMemcpyHostToDevice), "H2D checkpoint codes");
        if (!rc) rc = hip_check(hipMemcpy(scales, sc.data(), n / 32 * 4, hipMemcpyHostToDevice), "H2D checkpoint scales");
        return rc;
    }
    if (t.dtype == "F16") {
        std::vector<float> tmp(n);
        rc = f.read_f32(t, tmp.data(), n);
        if (!rc) rc = hip_check(hipMemcpy(stage, tmp.data(), n * 4, hipMemcpyHostToDevice), "H2D checkpoint");
        if (!rc) rc = mx4_quantize(s, rows, k, stage, 0, codes, scales);
    } else {
        const bool bf16 = t.dtype == "BF16";
        rc = hip_check(hipMemcpy(stage, f.data(t), n * (bf16 ? 2 : 4), hipMemcpyHostToDevice), "H2D checkpoint");
        if (!rc) rc = mx4_quantize(s, rows, k, stage, bf16 ? 1 : 0, codes, scales);
    }
    // the next tensor reuses the staging buffer
    if (!rc) rc = hip_check(hipStreamSynchronize(s), "hipStreamSynchronize(load)");
    return rc;
}

// Norm weights as fp16 (RNE from BF16 / F32; exact for bf16 values of
// magnitude 2^-17 .. 65504, i.e. any RMSNorm gain), embeddings as stored when
// BF16 or F16 (F32 rounded to bf16).
static int load_norm(const StFile &f, const StTensor &t, uint16_t *dst)
{
    std::vector<uint16_t> h(t.numel());
    int rc = f.read_f16(t, h.data(), h.size());
    if (!rc) rc = hip_check(hipMemcpy(dst, h.data(), h.size() * 2, hipMemcpyHostToDevice), "H2D checkpoint");
    return rc;
}

static int load_embed(llama_engine *e, const StFile &f, const StTensor &t, uint16_t *dst)
{
    const uint64_t n = t.numel();
    if (t.dtype == "BF16" || t.dtype == "F16")
        return hip_check(hipMemcpy(dst, f.data(t), n * 2, hipMemcpyHostToDevice), "H2D checkpoint");
    std::vector<float> tmp(n);
    int rc = f.read_f32(t, tmp.data(), n);
    if (rc) return rc;
    std::vector<uint16_t> h(n);
    for (uint64_t i = 0; i < n; i++) h[i] = f32_to_bf16_rne_host(tmp[i]);
    (void)e;
    return hip_check(hipMemcpy(dst, h.data(), n * 2, hipMemcpyHostToDevice), "H2D checkpoint");
}

static int engine_load_safetensors(llama_engine *e, const char *path)
{
    const rfp4_model_config &c = e->c;
    const uint32_t qd = qdim(c), kvd = kvdim(c);
    StFile f;
    int rc = f.open(path);
    if (rc) return rc;
    // every tensor present with the configured shape before any upload
    const uint64_t pshape[7][2] = {{qd, c.dim}, {kvd, c.dim}, {kvd, c.dim}, {c.dim, qd},
                                   {c.ffn, c.dim}, {c.ffn, c.dim}, {c.dim, c.ffn}};
    std::vector<const StTensor *> proj((size_t)c.n_layers * 7), na(c.n_layers), nf(c.n_layers);
    for (uint32_t l = 0; l < c.n_layers && !rc; l++) {
        const std::string pre = "model.layers." + std::to_string(l) + ".";
        for (int p = 0; p < 7 && !rc; p++) rc = st_tensor(f, pre + kProjNames[p], pshape[p][0], pshape[p][1], &proj[l * 7 + p]);
        if (!rc) rc = st_tensor(f, pre + "input_layernorm.weight", c.dim, 0, &na[l]);
        if (!rc) rc = st_tensor(f, pre + "post_attention_layernorm.weight", c.dim, 0, &nf[l]);
    }
    const StTensor *fin = nullptr, *emb = nullptr, *lm = nullptr;
    if (!rc) rc = st_tensor(f, "model.norm.weight", c.dim, 0, &fin);
    if (!rc) rc = st_tensor(f, "model.embed_tokens.weight", c.vocab, c.dim, &emb);
    // a checkpoint with tied embeddings has no lm_head.weight
    if (!rc) rc = f.find("lm_head.weight") ? st_tensor(f, "lm_head.weight", c.vocab, c.dim, &lm) : RFP4_OK;
    if (rc) return rc;
    if (!lm) lm = emb;

    e->embed_bf16 = emb->dtype == "F16" ? 0u : 1u;

    size_t stage_bytes = 0;
    for (const StTensor *t : proj) stage_bytes = std::max<size_t>(stage_bytes, t->numel() * 4);
    stage_bytes = std::max<size_t>(stage_bytes, lm->numel() * 4);
    void *stage = nullptr;
    rc = hip_check(hipMalloc(&stage, stage_bytes), "hipMalloc(checkpoint staging)");
    for (uint32_t l = 0; l < c.n_layers && !rc; l++)
        for (int p = 0; p < 7 && !rc; p++) {
            ProjDst d = proj_dst(e, l, p);
            rc = load_proj(e, f, *proj[l * 7 + p], d.codes, d.scales, stage);
        }
    if (!rc) rc = load_proj(e, f, *lm, e->lm_c, e->lm_s, stage);
    if (stage) hipFree(stage);
    for (uint32_t l = 0; l < c.n_layers && !rc; l++) {
        rc = load_norm(f, *na[l], e->norm_attn + (size_t)l * c.dim);
        if (!rc) rc = load_norm(f, *nf[l], e->norm_ffn + (size_t)l * c.dim);
    }
    if (!rc) rc = load_norm(f, *fin, e->norm_final);
    if (!rc) rc = load_embed(e, f, *emb, e->embed);
    return rc;
}

// ---------------------------------------------------------------- packed cache
// File: "RFP4PACK", u32 version, u32 embed_bf16, rfp4_model_config, u32 count,
// then `count` blobs (u64 bytes + bytes) in engine_blobs order.  Version 2
// carries the scale and KV formats in the config (version 1 files, written
// before the formats existed, hold zeros there: E8M0 and fp16).
static const char kPackMagic[8] = {'R', 'F', 'P', '4', 'P', 'A', 'C', 'K'};
static const uint32_t kPackVersion = 2;

static std::vector<std::pair<void *, size_t>> engine_blobs(llama_engine *e)
{
    const rfp4_model_config &c = e->c;
    const uint32_t qd = qdim(c), kvd = kvdim(c), nqkv = qd + 2 * kvd;
    std::vector<std::pair<void *, size_t>> b;
    for (uint32_t l = 0; l < c.n_layers; l++) {
        LayerW &w = e->L[l];
        b.push_back({w.qkv_c, (size_t)nqkv * c.dim / 2});
        b.push_back({w.qkv_s, (size_t)nqkv * c.dim / 32 * e->sb});
        b.push_back({w.o_c, (size_t)c.dim * qd / 2});
        b.push_back({w.o_s, (size_t)c.dim * qd / 32 * e->sb});
        b.push_back({w.gu_c, (size_t)2 * c.ffn * c.dim / 2});
        b.push_back({w.gu_s, (size_t)2 * c.ffn * c.dim / 32 * e->sb});
        b.push_back({w.d_c, (size_t)c.dim * c.ffn / 2});
        b.push_back({w.d_s, (size_t)c.dim * c.ffn / 32 * e->sb});
    }
    b.push_back({e->norm_attn, (size_t)c.n_layers * c.dim * 2});
    b.push_back({e->norm_ffn, (size_t)c.n_layers * c.dim * 2});
    b.push_back({e->norm_final, (size_t)c.dim * 2});
    b.push_back({e->embed, (size_t)c.vocab * c.dim * 2});
    b.push_back({e->lm_c, (size_t)c.vocab * c.dim / 2});
    b.push_back({e->lm_s, (size_t)c.vocab * c.dim / 32 * e->sb});
    return b;
}

extern "C" {

int llama_engine_create(const rfp4_model_config *cfg, uint64_t seed, llama_engine **out)
{
    llama_engine *e = nullptr;
    int rc = engine_alloc(cfg, &e);
    if (rc) return rc;
    rc = e->sb == 4 ? engine_synth_mk_fp4(e, seed) : engine_synth(e, seed);
    if (!rc) rc = engine_finish(e);
    if (rc) {
        engine_free(e);
        return rc;
    }
    engine_register(e);
    *out = e;
    return RFP4_OK;
}

int llama_engine_destroy(llama_engine *e)
{
    if (!e) return RFP4_OK;
    if (!engine_unregister(e)) return set_error(RFP4_E_INVALID, "llama_engine_destroy: not a live engine");
    engine_free(e);
    return RFP4_OK;
}

int llama_engine_prefill_kv(llama_engine *e, uint64_t seed, uint32_t upto)
{
    if (!e) return set_error(RFP4_E_INVALID, "null engine");
    const rfp4_model_config &c = e->c;
    if (upto > c.max_seq) return set_error(RFP4_E_KV_OVERFLOW, "prefill %u > max_seq %u", upto, c.max_seq);
    const float coef = ih4_coef(0.1f);
    for (uint32_t l = 0; l < c.n_layers; l++)
        for (uint32_t isv = 0; isv < 2; isv++) {
            SynthKvArgs a{kv_layer(e, l, (int)isv), seed, stream_kv(l, isv), upto, c.n_kv_heads, c.head_dim,
                          e->max_seq_alloc, coef, e->kvb == 4 ? 1u : 0u};
            uint64_t total = (uint64_t)upto * c.n_kv_heads * c.head_dim;
            uint64_t blocks = (total + 255) / 256;
            if (blocks > 65536) blocks = 65536;
            if (blocks == 0) continue;
            int rc = launch("rfp4_synth_kv", dim3((unsigned)blocks), dim3(256), e->stream, &a);
            if (rc) return rc;
        }
    return hip_check(hipStreamSynchronize(e->stream), "hipStreamSynchronize(prefill)");
}

int llama_engine_begin(llama_engine *e, const uint32_t *prompt, uint32_t n_prompt, uint32_t pos0, uint32_t ids_cap)
{
    if (!e || !prompt) return set_error(RFP4_E_INVALID, "llama_engine_begin: null argument");
    if (n_prompt == 0) return set_error(RFP4_E_INVALID, "llama_engine_begin: empty prompt");
    if (ids_cap < n_prompt || ids_cap > e->ids_alloc) return set_error(RFP4_E_CAPACITY, "ids capacity %u out of range", ids_cap);
    if (pos0 >= e->c.max_seq) return set_error(RFP4_E_KV_OVERFLOW, "start position %u >= max_seq %u", pos0, e->c.max_seq);
    for (uint32_t i = 0; i < n_prompt; i++)
        if (prompt[i] >= e->c.vocab) return set_error(RFP4_E_INVALID, "prompt token %u >= vocab %u", prompt[i], e->c.vocab);
    int rc = hip_check(hipStreamSynchronize(e->stream), "hipStreamSynchronize(begin)");
    if (!rc) rc = set_embed_mode(e, false);
    if (rc) return rc;
    rc = hip_check(hipMemcpy(e->ids, prompt, (size_t)n_prompt * 4, hipMemcpyHostToDevice), "H2D prompt");
    StepState st{(int32_t)pos0, 0, n_prompt, ids_cap};
    if (!rc) rc = hip_check(hipMemcpy(e->state, &st, sizeof st, hipMemcpyHostToDevice), "H2D cursor");
    if (!rc) rc = tag_clear(e);
    if (!rc) rc = fill_words(e->p_err, 1, 0u, e->stream); // a new generation: no wait has failed yet
    if (!rc) rc = embed_first(e);
    if (rc) return rc;
    e->h_pos = pos0;
    e->h_step = 0;
    e->h_ids_cap = ids_cap;
    // the step graphs for every position this generation can reach
    const int64_t last = std::min<int64_t>((int64_t)pos0 + ids_cap - 2, (int64_t)e->c.max_seq - 1);
    rc = step_graphs_for(e, pos0, std::max<int64_t>(last, pos0));
    if (rc) return rc;
    e->armed = true;
    return RFP4_OK;
}

int llama_engine_begin_harness(llama_engine *e, uint32_t ctx, uint32_t ids_cap)
{
    if (!e) return set_error(RFP4_E_INVALID, "llama_engine_begin_harness: null engine");
    const rfp4_model_config &c = e->c;
    if (e->harness_x.size() != c.dim)
        return set_error(RFP4_E_INVALID, "the harness needs an f32-scale engine from llama_engine_create");
    if (ctx >= c.max_seq) return set_error(RFP4_E_KV_OVERFLOW, "context %u >= max_seq %u", ctx, c.max_seq);
    if (ids_cap < 2 || ids_cap > e->ids_alloc) return set_error(RFP4_E_CAPACITY, "ids capacity %u out of range", ids_cap);
    int rc = hip_check(hipStreamSynchronize(e->stream), "hipStreamSynchronize(harness)");
    if (!rc) rc = set_embed_mode(e, true);
    if (rc) return rc;
    // every K/V position [0, ctx) := 0.01 (llama_decode/src/main.rs:375-376,388-389)
    const float v = 0.01f;
    uint32_t word;
    if (e->kvb == 4) {
        std::memcpy(&word, &v, 4);
    } else {
        const uint32_t h = f32_to_f16_rne_host(v);
        word = h | (h << 16);
    }
    const size_t head_bytes = (size_t)e->max_seq_alloc * c.head_dim * e->kvb;
    for (uint32_t l = 0; l < c.n_layers && !rc; l++)
        for (int isv = 0; isv < 2 && !rc; isv++)
            for (uint32_t h = 0; h < c.n_kv_heads && !rc; h++)
                rc = fill_words((uint32_t *)((char *)kv_layer(e, l, isv) + h * head_bytes),
                                (size_t)ctx * c.head_dim * e->kvb / 4, word, e->stream);
    if (!rc) rc = hip_check(hipStreamSynchronize(e->stream), "hipStreamSynchronize(harness kv)");
    // x := the harness vector; the cursor at ctx, ids[1 + i] <- step i's argmax
    if (!rc) rc = hip_check(hipMemcpy(e->x, e->harness_x.data(), (size_t)c.dim * 4, hipMemcpyHostToDevice), "H2D x");
    const uint32_t zero = 0;
    if (!rc) rc = hip_check(hipMemcpy(e->ids, &zero, 4, hipMemcpyHostToDevice), "H2D ids");
    StepState st{(int32_t)ctx, 0, 1u, ids_cap};
    if (!rc) rc = hip_check(hipMemcpy(e->state, &st, sizeof st, hipMemcpyHostToDevice), "H2D cursor");
    if (!rc) rc = tag_clear(e);
    if (!rc) rc = fill_words(e->p_err, 1, 0u, e->stream); // a new generation: no wait has failed yet
    if (rc) return rc;
    e->h_pos = ctx;
    e->h_step = 0;
    e->h_ids_cap = ids_cap;
    const int64_t last = std::min<int64_t>((int64_t)ctx + ids_cap - 2, (int64_t)c.max_seq - 1);
    rc = step_graphs_for(e, ctx, std::max<int64_t>(last, ctx));
    if (rc) return rc;
    e->armed = true;
    return RFP4_OK;
}

int llama_engine_run_steps(llama_engine *e, uint32_t n_steps)
{
    if (!e) return set_error(RFP4_E_INVALID, "null engine");
    if (!e->armed) return set_error(RFP4_E_INVALID, "llama_engine_begin has not been called");
    if (e->h_pos + n_steps > (int64_t)e->c.max_seq)
        return set_error(RFP4_E_KV_OVERFLOW, "steps would reach position %lld >= max_seq %u", (long long)(e->h_pos + n_steps),
                         e->c.max_seq);
    if (e->h_step + n_steps > e->h_ids_cap - 1)
        return set_error(RFP4_E_CAPACITY, "steps exceed the token array (%lld + %u > %lld)", (long long)e->h_step, n_steps,
                         (long long)(e->h_ids_cap - 1));
    for (uint32_t i = 0; i < n_steps; i++) {
        const uint32_t ns = splits_at(e, e->h_pos + i);
        int rc;
        if (e->persist) {
            rc = enqueue_step_persist(e);
        } else if (e->use_graph) {
            hipGraphExec_t g;
            rc = step_graph(e, ns, &g);
            if (!rc) rc = hip_check(hipGraphLaunch(g, e->stream), "hipGraphLaunch");
        } else {
            rc = enqueue_step(e, ns);
        }
        if (rc) return rc;
    }
    e->h_pos += n_steps;
    e->h_step += n_steps;
    return RFP4_OK;
}

int llama_engine_time_steps(llama_engine *e, uint32_t n_steps, rfp4_kernel_time *out, uint32_t cap, uint32_t *count)
{
    if (!e || !count || (cap && !out)) return set_error(RFP4_E_INVALID, "llama_engine_time_steps: null argument");
    if (!e->armed) return set_error(RFP4_E_INVALID, "llama_engine_begin has not been called");
    if (e->h_pos + n_steps > (int64_t)e->c.max_seq)
        return set_error(RFP4_E_KV_OVERFLOW, "steps would reach position %lld >= max_seq %u", (long long)(e->h_pos + n_steps),
                         e->c.max_seq);
    if (e->h_step + n_steps > e->h_ids_cap - 1)
        return set_error(RFP4_E_CAPACITY, "steps exceed the token array");
    std::vector<KernelTiming> rec;
    int rc = RFP4_OK;
    timing_install(&rec);
    for (uint32_t i = 0; i < n_steps && !rc; i++)
        rc = e->persist ? enqueue_step_persist(e) : enqueue_step(e, splits_at(e, e->h_pos + i));
    timing_install(nullptr);
    if (!rc) rc = hip_check(hipStreamSynchronize(e->stream), "hipStreamSynchronize(timing)");
    *count = (uint32_t)rec.size();
    for (size_t i = 0; i < rec.size(); i++) {
        float ms = 0.0f;
        if (!rc) rc = hip_check(hipEventElapsedTime(&ms, rec[i].start, rec[i].stop), "hipEventElapsedTime");
        if (!rc && i < cap) {
            snprintf(out[i].name, sizeof out[i].name, "%s", rec[i].name);
            out[i].us = ms * 1000.0f;
        }
        hipEventDestroy(rec[i].start);
        hipEventDestroy(rec[i].stop);
    }
    if (rc) return rc;
    e->h_pos += n_steps;
    e->h_step += n_steps;
    return wait_check(e);
}

int llama_engine_read_ids(llama_engine *e, uint32_t *ids, uint32_t count)
{
    if (!e || !ids) return set_error(RFP4_E_INVALID, "null argument");
    if (count > e->ids_alloc) return set_error(RFP4_E_CAPACITY, "count %u > %u", count, e->ids_alloc);
    int rc = hip_check(hipMemcpyAsync(ids, e->ids, (size_t)count * 4, hipMemcpyDeviceToHost, e->stream), "D2H ids");
    if (rc) return rc;
    rc = hip_check(hipStreamSynchronize(e->stream), "hipStreamSynchronize(ids)");
    return rc ? rc : wait_check(e);
}

int llama_generate(llama_engine *e, const uint32_t *prompt, uint32_t n_prompt, uint32_t pos0, uint32_t n_new,
                   uint32_t *out)
{
    if (!out) return set_error(RFP4_E_INVALID, "null output");
    if (n_new == 0) return RFP4_OK;
    uint32_t cap = n_prompt + n_new;
    int rc = llama_engine_begin(e, prompt, n_prompt, pos0, cap);
    if (!rc) rc = llama_engine_run_steps(e, n_prompt + n_new - 1);
    if (rc) return rc;
    std::vector<uint32_t> ids(cap);
    rc = llama_engine_read_ids(e, ids.data(), cap);
    if (rc) return rc;
    std::memcpy(out, ids.data() + n_prompt, (size_t)n_new * 4);
    return RFP4_OK;
}

int llama_decode_step(llama_engine *e, uint32_t tok, uint32_t pos, uint32_t *next)
{
    if (!next) return set_error(RFP4_E_INVALID, "null output");
    return llama_generate(e, &tok, 1, pos, 1, next);
}

int llama_engine_logits(llama_engine *e, float *host_logits)
{
    if (!e || !host_logits) return set_error(RFP4_E_INVALID, "null argument");
    int rc = hip_check(hipMemcpyAsync(host_logits, e->logits, (size_t)e->c.vocab * 4, hipMemcpyDeviceToHost, e->stream),
                       "D2H logits");
    if (rc) return rc;
    return hip_check(hipStreamSynchronize(e->stream), "hipStreamSynchronize(logits)");
}

rfp4_stream_t llama_engine_stream(llama_engine *e) { return e ? (rfp4_stream_t)e->stream : nullptr; }

int rfp4_debug_engine_wait(llama_engine *e, int set_err, uint32_t nsplit, int *err_wired, int *checked, int *fused)
{
    if (!e || !err_wired || !checked || !fused) return set_error(RFP4_E_INVALID, "rfp4_debug_engine_wait: null argument");
    if (nsplit == 0 || nsplit > e->attn_max_splits)
        return set_error(RFP4_E_INVALID, "rfp4_debug_engine_wait: %u splits (1..%u)", nsplit, e->attn_max_splits);
    int wired = 1;
    for (uint32_t l = 0; l < e->c.n_layers; l++) wired &= step_attn_args(e, l, nsplit).err == e->p_err ? 1 : 0;
    *err_wired = wired;
    QkvaPlan pl;
    const AttnArgs a0 = step_attn_args(e, 0, nsplit);
    *fused = qkva_plan(e, nsplit, a0.tagged != nullptr, &pl) ? 1 : 0;
    *checked = (e->persist_ok || e->attn_tagged || e->qkva_R) ? 1 : 0;
    if (set_err) {
        int rc = fill_words(e->p_err, 1, 1u, e->stream);
        if (!rc) rc = hip_check(hipStreamSynchronize(e->stream), "hipStreamSynchronize(debug wait)");
        return rc;
    }
    return RFP4_OK;
}

int llama_engine_use_graph(llama_engine *e, int enable)
{
    if (!e) return set_error(RFP4_E_INVALID, "null engine");
    e->use_graph = enable != 0;
    return RFP4_OK;
}

int llama_engine_use_persistent(llama_engine *e, int enable)
{
    if (!e) return set_error(RFP4_E_INVALID, "null engine");
    if (enable && !e->persist_ok)
        return set_error(RFP4_E_SHAPE, "persistent decode needs the Llama-3-8B widths, E8M0 weights, fp16 caches, "
                                       "a 256-CU device and at most %u attention splits", kPersistMaxSplits);
    int rc = hip_check(hipStreamSynchronize(e->stream), "hipStreamSynchronize(mode)");
    if (!rc) e->persist = enable != 0;
    return rc;
}

int llama_engine_persistent(const llama_engine *e) { return e && e->persist ? 1 : 0; }

int llama_engine_weight(llama_engine *e, int layer, int proj, const uint8_t **codes, const uint8_t **scales,
                        size_t *code_bytes, size_t *scale_bytes)
{
    if (!e || !codes || !scales || !code_bytes || !scale_bytes) return set_error(RFP4_E_INVALID, "null argument");
    const rfp4_model_config &c = e->c;
    const uint32_t qd = qdim(c), kvd = kvdim(c);
    if (layer < 0) {
        *codes = e->lm_c;
        *scales = e->lm_s;
        *code_bytes = (size_t)c.vocab * c.dim / 2;
        *scale_bytes = (size_t)c.vocab * c.dim / 32 * e->sb;
        return RFP4_OK;
    }
    if ((uint32_t)layer >= c.n_layers || proj < 0 || proj > 6) return set_error(RFP4_E_INVALID, "bad layer/proj");
    const LayerW &w = e->L[layer];
    size_t rows_before = 0, rows = 0, K = c.dim;
    const uint8_t *bc = nullptr, *bs = nullptr;
    switch (proj) {
    case 0: bc = w.qkv_c; bs = w.qkv_s; rows_before = 0; rows = qd; break;
    case 1: bc = w.qkv_c; bs = w.qkv_s; rows_before = qd; rows = kvd; break;
    case 2: bc = w.qkv_c; bs = w.qkv_s; rows_before = qd + kvd; rows = kvd; break;
    case 3: bc = w.o_c; bs = w.o_s; rows = c.dim; K = qd; break;
    case 4: bc = w.gu_c; bs = w.gu_s; rows = c.ffn; break;
    case 5: bc = w.gu_c; bs = w.gu_s; rows_before = c.ffn; rows = c.ffn; break;
    default: bc = w.d_c; bs = w.d_s; rows = c.dim; K = c.ffn; break;
    }
    *codes = bc + rows_before * K / 2;
    *scales = bs + rows_before * K / 32 * e->sb;
    *code_bytes = rows * K / 2;
    *scale_bytes = rows * K / 32 * e->sb;
    return RFP4_OK;
}

int llama_engine_weight_scales_tiled(llama_engine *e, int layer, int proj, const uint8_t **scales_tiled,
                                     size_t *bytes)
{
    if (!e || !scales_tiled || !bytes) return set_error(RFP4_E_INVALID, "null argument");
    if (!e->lm_st) return set_error(RFP4_E_SHAPE, "llama_engine_weight_scales_tiled: the engine cannot prefill, so holds none");
    const rfp4_model_config &c = e->c;
    const uint32_t qd = qdim(c), kvd = kvdim(c);
    if (layer < 0) {
        *scales_tiled = e->lm_st;
        *bytes = scales_tiled_bytes(c.vocab, c.dim);
        return RFP4_OK;
    }
    if ((uint32_t)layer >= c.n_layers || proj < 0 || proj > 6) return set_error(RFP4_E_INVALID, "bad layer/proj");
    const LayerW &w = e->L[layer];
    // stacked matrices: every part starts on a 32-row block (qd, kvd, ffn are multiples of 256)
    size_t rows_before = 0, rows = 0, K = c.dim;
    const uint8_t *bs = nullptr;
    switch (proj) {
    case 0: bs = w.qkv_st; rows = qd; break;
    case 1: bs = w.qkv_st; rows_before = qd; rows = kvd; break;
    case 2: bs = w.qkv_st; rows_before = qd + kvd; rows = kvd; break;
    case 3: bs = w.o_st; rows = c.dim; K = qd; break;
    case 4: bs = w.gu_st; rows = c.ffn; break;
    case 5: bs = w.gu_st; rows_before = c.ffn; rows = c.ffn; break;
    default: bs = w.d_st; rows = c.dim; K = c.ffn; break;
    }
    *scales_tiled = bs + rows_before * K / 32;
    *bytes = scales_tiled_bytes((uint32_t)rows, (uint32_t)K);
    return RFP4_OK;
}

int llama_engine_kv(llama_engine *e, int layer, const void **k, const void **v, size_t *count)
{
    if (!e || !k || !v || !count) return set_error(RFP4_E_INVALID, "null argument");
    if (layer < 0 || (uint32_t)layer >= e->c.n_layers) return set_error(RFP4_E_INVALID, "bad layer");
    *k = kv_layer(e, (uint32_t)layer, 0);
    *v = kv_layer(e, (uint32_t)layer, 1);
    *count = (size_t)e->c.n_kv_heads * e->max_seq_alloc * e->c.head_dim;
    return RFP4_OK;
}

int llama_engine_prefill(llama_engine *e, const uint32_t *prompt, uint32_t n_prompt, uint32_t pos0,
                         uint32_t *next_token)
{
    if (!e || !prompt || !next_token || n_prompt == 0)
        return set_error(RFP4_E_INVALID, "llama_engine_prefill: null argument or empty prompt");
    const rfp4_model_config &c = e->c;
    if ((uint64_t)pos0 + n_prompt > c.max_seq)
        return set_error(RFP4_E_KV_OVERFLOW, "prefill of %u tokens at position %u runs past max_seq %u", n_prompt, pos0,
                         c.max_seq);
    if (c.dim % 256u || qdim(c) % 256u || c.ffn % 256u)
        return set_error(RFP4_E_SHAPE, "prefill runs on the MXFP4 GEMM: dim, n_heads*head_dim and ffn must be multiples of 256");
    if (c.scale_format != RFP4_SCALE_E8M0 || c.kv_format != RFP4_KV_F16)
        return set_error(RFP4_E_SHAPE, "prefill runs on the MXFP4 GEMM: it needs E8M0 weights and fp16 caches");
    for (uint32_t i = 0; i < n_prompt; i++)
        if (prompt[i] >= c.vocab) return set_error(RFP4_E_INVALID, "prompt token %u out of range", prompt[i]);
    int rc = prefill_reserve(e, n_prompt);
    if (!rc)
        rc = hip_check(hipMemcpyAsync(e->pf_ids, prompt, n_prompt * sizeof(uint32_t), hipMemcpyHostToDevice, e->stream),
                       "hipMemcpyAsync(prompt)");
    if (!rc) rc = enqueue_prefill(e, n_prompt, pos0);
    if (rc == kPrefillStopped) {
        // stopped by the test hook: the workspace holds that stage's output, no token
        rc = hip_check(hipStreamSynchronize(e->stream), "hipStreamSynchronize");
        if (!rc) *next_token = UINT32_MAX;
        return rc;
    }
    uint32_t tok = 0;
    if (!rc)
        rc = hip_check(hipMemcpyAsync(&tok, e->last_tok, sizeof(uint32_t), hipMemcpyDeviceToHost, e->stream),
                       "hipMemcpyAsync(token)");
    if (!rc) rc = hip_check(hipStreamSynchronize(e->stream), "hipStreamSynchronize");
    if (!rc) *next_token = tok;
    return rc;
}

int llama_engine_prefill_buffers(llama_engine *e, float **x, uint8_t **codes, uint8_t **scales, float **c, float **a,
                                 uint32_t *rows_cap)
{
    if (!e || !x || !codes || !scales || !c || !a || !rows_cap)
        return set_error(RFP4_E_INVALID, "llama_engine_prefill_buffers: null argument");
    *x = e->pf_x;
    *codes = e->pf_q_alt ? e->pf_codes2 : e->pf_codes; // the MXFP4 rows written last
    *scales = e->pf_q_alt ? e->pf_scales2 : e->pf_scales;
    *c = e->pf_c;
    *a = e->pf_a;
    *rows_cap = e->pf_cap;
    return RFP4_OK;
}

int llama_engine_create_from_safetensors(const rfp4_model_config *cfg, const char *path, llama_engine **out)
{
    if (!path) return set_error(RFP4_E_INVALID, "llama_engine_create_from_safetensors: null path");
    llama_engine *e = nullptr;
    int rc = engine_alloc(cfg, &e);
    if (rc) return rc;
    rc = engine_load_safetensors(e, path);
    if (!rc) rc = engine_finish(e);
    if (rc) {
        engine_free(e);
        return rc;
    }
    engine_register(e);
    *out = e;
    return RFP4_OK;
}

int llama_engine_save(llama_engine *e, const char *path)
{
    if (!e || !path) return set_error(RFP4_E_INVALID, "llama_engine_save: null argument");
    FILE *fp = fopen(path, "wb");
    if (!fp) return set_error(RFP4_E_INVALID, "llama_engine_save: cannot create %s", path);
    auto blobs = engine_blobs(e);
    const uint32_t count = (uint32_t)blobs.size();
    bool ok = fwrite(kPackMagic, 1, 8, fp) == 8 && fwrite(&kPackVersion, 4, 1, fp) == 1 &&
              fwrite(&e->embed_bf16, 4, 1, fp) == 1 && fwrite(&e->c, sizeof(rfp4_model_config), 1, fp) == 1 &&
              fwrite(&count, 4, 1, fp) == 1;
    int rc = hip_check(hipStreamSynchronize(e->stream), "hipStreamSynchronize(save)");
    std::vector<uint8_t> host;
    for (size_t i = 0; i < blobs.size() && ok && !rc; i++) {
        const uint64_t n = blobs[i].second;
        host.resize(n);
        rc = hip_check(hipMemcpy(host.data(), blobs[i].first, n, hipMemcpyDeviceToHost), "D2H save");
        ok = !rc && fwrite(&n, 8, 1, fp) == 1 && fwrite(host.data(), 1, n, fp) == n;
    }
    if (fclose(fp) != 0) ok = false;
    if (rc) return rc;
    if (!ok) return set_error(RFP4_E_INVALID, "llama_engine_save: write to %s failed", path);
    return RFP4_OK;
}

int llama_engine_load(const char *path, uint32_t max_seq, llama_engine **out)
{
    if (!path || !out) return set_error(RFP4_E_INVALID, "llama_engine_load: null argument");
    *out = nullptr;
    FILE *fp = fopen(path, "rb");
    if (!fp) return set_error(RFP4_E_INVALID, "llama_engine_load: cannot open %s", path);
    char magic[8];
    uint32_t version = 0, half = 0, count = 0;
    rfp4_model_config cfg{};
    bool ok = fread(magic, 1, 8, fp) == 8 && memcmp(magic, kPackMagic, 8) == 0 && fread(&version, 4, 1, fp) == 1 &&
              (version == 1 || version == kPackVersion) && fread(&half, 4, 1, fp) == 1 && half <= 1 &&
              fread(&cfg, sizeof cfg, 1, fp) == 1 && fread(&count, 4, 1, fp) == 1;
    if (!ok) {
        fclose(fp);
        return set_error(RFP4_E_SHAPE, "llama_engine_load: %s is not a packed engine (version %u)", path, kPackVersion);
    }
    cfg.max_seq = max_seq;
    if (version == 1) cfg.scale_format = cfg.kv_format = 0;
    llama_engine *e = nullptr;
    int rc = engine_alloc(&cfg, &e);
    if (rc) {
        fclose(fp);
        return rc;
    }
    e->embed_bf16 = half;
    auto blobs = engine_blobs(e);
    if (count != blobs.size()) rc = set_error(RFP4_E_SHAPE, "llama_engine_load: %u blobs, the config needs %zu", count, blobs.size());
    std::vector<uint8_t> host;
    for (size_t i = 0; i < blobs.size() && !rc; i++) {
        uint64_t n = 0;
        if (fread(&n, 8, 1, fp) != 1 || n != blobs[i].second) {
            rc = set_error(RFP4_E_SHAPE, "llama_engine_load: blob %zu has the wrong size", i);
            break;
        }
        host.resize(n);
        if (fread(host.data(), 1, n, fp) != n) {
            rc = set_error(RFP4_E_SHAPE, "llama_engine_load: %s is truncated", path);
            break;
        }
        rc = hip_check(hipMemcpy(blobs[i].first, host.data(), n, hipMemcpyHostToDevice), "H2D load");
    }
    fclose(fp);
    if (!rc) rc = engine_finish(e);
    if (rc) {
        engine_free(e);
        return rc;
    }
    engine_register(e);
    *out = e;
    return RFP4_OK;
}

int llama_engine_info(const llama_engine *e, rfp4_model_config *cfg, int *embed_bf16)
{
    if (!e) return set_error(RFP4_E_INVALID, "llama_engine_info: null engine");
    if (cfg) *cfg = e->c;
    if (embed_bf16) *embed_bf16 = (int)e->embed_bf16;
    return RFP4_OK;
}

uint64_t llama_engine_weight_bytes(const llama_engine *e)
{
    if (!e) return 0;
    const rfp4_model_config &c = e->c;
    uint64_t per_layer = (uint64_t)(qdim(c) + 2 * kvdim(c)) * c.dim + (uint64_t)c.dim * qdim(c) +
                         3ull * c.ffn * c.dim;
    uint64_t elems = per_layer * c.n_layers + (uint64_t)c.vocab * c.dim;
    return elems / 2 + elems / 32 * e->sb;
}

} // extern "C"
