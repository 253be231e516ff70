// Causal GQA attention for the batched prefill (gfx950 matrix cores).
//
// Semantics as attn.h for every prompt row r (absolute position pos0 + r):
//   out[r][h] = softmax over t <= pos0 + r of (q_h . k_t) / sqrt(HD), times v_t
// (llama_run/src/main.rs:148-242 applied row by row), with the prompt's own
// rows already appended to the fp16 caches.
//
// Grid (query tiles, n_kv_heads).  A workgroup of NW waves takes BQ =
// max(16, 16 NW / GT) prompt rows and every query head of one KV head (GT
// heads, G <= GT real), i.e. NT = (BQ/16) * GT tiles of 16 (row, head) pairs,
// MT = NT / NW per wave, and walks the keys 0 .. last
// row's position in blocks of 32: K rows staged in LDS as loaded, V rows
// staged transposed (dimension-major), both as v_mfma_f32_16x16x32_f16
// operands read with one 16-byte LDS read per lane:
//   S (16 x 32) = Q (16 x HD) . K^T        -- A = q as two fp16 terms
//   online softmax per row (base 2, f32)   -- rows live in 16-lane groups
//   O (16 x HD) += P (16 x 32) . V         -- A = p as two fp16 terms, through LDS
// q and p enter as hi + lo (hi = fp16(x), lo = fp16(x - hi): about 2^-22
// relative, two MFMAs per product; K and V are fp16 already), products exact
// and f32 accumulation, so the output matches the f32 decode kernel's to
// about 1e-6: one fp16 rounding of q and p (2^-11) moves enough of the O
// projection's MXFP4 input codes across rounding boundaries to shift the
// logits by percent.  Operand
// layout (pinned by the fp16 layout test): lane l holds A row / B column
// l % 16 and K = 8 (l / 16) .. +7; accumulator r of lane l is D[4 (l/16) + r][l % 16].
// The next two blocks' K/V loads are in flight while the current block computes.
#pragma once
#include "common.h"

#define PF_BK 32   // keys per block
#define PF_KPAD 8  // fp16 padding of a staged K row (16 consecutive rows -> 16 distinct bank groups)
#define PF_TPAD 8  // fp16 padding of a transposed V row / a P row

// One query tile: prompt rows r0 .. r0 + BQ of KV head blockIdx.y.
template <int HD, int GT, int NW>
RFP4_DEV void attn_prefill_tile(const AttnPrefillArgs &a, uint32_t r0)
{
    const uint32_t pos0 = a.pos0, nrows = a.rows;
    constexpr int BQ = attn_prefill_rows(GT, NW);    // prompt rows per workgroup
    constexpr int NT = (BQ / 16) * GT;               // 16-row tiles per workgroup
    constexpr int MT = NT / NW;                      // tiles per wave
    constexpr int KS = HD / 32;                      // K steps of S = Q K^T
    constexpr int NN = HD / 16;                      // 16-wide column tiles of O
    constexpr int KROW = HD + PF_KPAD, TROW = PF_BK + PF_TPAD;
    constexpr int LPK = HD / 8;                      // 16-byte pieces per K/V row
    constexpr int T = 64 * NW;                       // threads
    constexpr int LD = (PF_BK * LPK + T - 1) / T;    // K (and V) pieces per thread per block
    constexpr bool LFULL = PF_BK * LPK % T == 0;     // every thread loads LD pieces
    static_assert(NT % NW == 0 && MT >= 1, "tiles per wave");
    static_assert(LFULL || LD == 1, "block load split");
    __shared__ __align__(16) _Float16 ks[PF_BK][KROW];
    __shared__ __align__(16) _Float16 vt[HD][TROW];
    __shared__ __align__(16) _Float16 ps[NW][MT][2][16][TROW]; // P hi, lo

    const uint32_t kvh = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t l16 = (uint32_t)lane & 15u, q4 = (uint32_t)lane >> 4;
    const uint32_t G = a.n_heads / a.n_kv_heads;
    const uint16_t *kc = a.kc + (size_t)kvh * a.hs;
    const uint16_t *vc = a.vc + (size_t)kvh * a.hs;
    // keys of this workgroup: 0 .. position of its last row
    const uint32_t last_row = min(r0 + (uint32_t)BQ, nrows) - 1u;
    const uint32_t nk = pos0 + last_row + 1u;
    const uint32_t nblk = (nk + PF_BK - 1) / PF_BK;
    const float scale = __fmul_rn(1.4426950408889634f, __fdiv_rn(1.0f, __fsqrt_rn((float)HD))); // log2(e) / sqrt(HD)

    // ---- Q tiles of this wave as fp16 A operands (rows past the prompt or heads past G: zero)
    f16x8 qa[MT][KS], ql[MT][KS];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const uint32_t t = (uint32_t)(wave * MT + mt), g = t % GT, row = r0 + 16u * (t / GT) + l16;
        const bool in = row < nrows && g < G;
        const float *qp = a.q + (size_t)min(row, nrows - 1u) * a.q_rs + (size_t)(kvh * G + min(g, G - 1u)) * HD + 8u * q4;
#pragma unroll
        for (int k = 0; k < KS; k++) {
            float v[8];
            const float4 x0 = *(const float4 *)(qp + 32 * k), x1 = *(const float4 *)(qp + 32 * k + 4);
            v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w;
            v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = in ? v[i] : 0.0f;
            split_hi_lo8(v, qa[mt][k], ql[mt][k]);
        }
    }

    f32x4 o[MT][NN];
    float mrun[MT][4], lrun[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            mrun[mt][r] = -3.402823466e38f;
            lrun[mt][r] = 0.0f;
        }
#pragma unroll
        for (int n = 0; n < NN; n++) o[mt][n] = {0.0f, 0.0f, 0.0f, 0.0f};
    }

    // ---- K / V block loads: K piece (key tid / LPK, dims 8 (tid % LPK)), V
    // piece (key tid % 32, dims 8 (tid / 32)) -- consecutive lanes take
    // consecutive keys, so the transposed V writes fall on consecutive halves.
    // Cached loads (each key row is read by every query tile of its KV head),
    // two register sets: block b + 2's loads are issued when block b's data
    // has gone to LDS, so each load has two blocks' compute to land.
    // (each set one 8-word vector value per operand, piece j in words 4j ..
    // 4j + 3: vectors stay in registers where the two sets' code is merged)
    static_assert(LD <= 2, "at most two 16-byte pieces per thread and block");
    typedef uint32_t pf_u32x8 __attribute__((ext_vector_type(8)));
    pf_u32x8 kr0, vr0, kr1, vr1;
#define RFP4_PF_LOAD(B, KR, VR)                                                                           \
    do {                                                                                                  \
        _Pragma("unroll") for (int j = 0; j < LD; j++) {                                                  \
            /* threads past the block's pieces load the last one again (unused) */                        \
            const uint32_t p = min((uint32_t)tid + (uint32_t)T * (uint32_t)j, (uint32_t)(PF_BK * LPK) - 1u); \
            const uint32_t kk = min((B) * PF_BK + p / LPK, nk - 1u), kd = 8u * (p % LPK);                 \
            const uint32_t vk = min((B) * PF_BK + p % PF_BK, nk - 1u), vd = 8u * (p / PF_BK);              \
            const u32x4 kx = *(const u32x4 *)(kc + (size_t)kk * a.ts + kd);                               \
            const u32x4 vx = *(const u32x4 *)(vc + (size_t)vk * a.ts + vd);                               \
            if (j == 0) { KR.lo = kx; VR.lo = vx; } else { KR.hi = kx; VR.hi = vx; }                      \
        }                                                                                                 \
    } while (0)
    // block b's K rows and transposed V rows into LDS, then block b + 2's loads into the same registers
#define RFP4_PF_STAGE(b, KR, VR)                                                                          \
    do {                                                                                                  \
        __syncthreads(); /* the previous block's LDS reads are done */                                    \
        _Pragma("unroll") for (int j = 0; j < LD; j++) {                                                  \
            const uint32_t p = (uint32_t)tid + (uint32_t)T * (uint32_t)j;                                 \
            if (!LFULL && p >= (uint32_t)(PF_BK * LPK)) break;                                            \
            const u32x4 kx = j == 0 ? KR.lo : KR.hi, vx = j == 0 ? VR.lo : VR.hi;                          \
            *(u32x4 *)&ks[p / LPK][8u * (p % LPK)] = kx;                                                  \
            const uint32_t vk = p % PF_BK, vd = 8u * (p / PF_BK);                                          \
            _Pragma("unroll") for (int i = 0; i < 4; i++) {                                               \
                vt[vd + 2u * i][vk] = __builtin_bit_cast(_Float16, (uint16_t)(vx[i] & 0xFFFFu));          \
                vt[vd + 2u * i + 1u][vk] = __builtin_bit_cast(_Float16, (uint16_t)(vx[i] >> 16));         \
            }                                                                                             \
        }                                                                                                 \
        __syncthreads();                                                                                  \
        RFP4_PF_LOAD((b) + 2u, KR, VR);                                                                   \
    } while (0)
    // Every load is issued on every path (keys clamped to the last one, so a
    // block past the end re-reads it): the compiler's wait for a set then
    // counts exactly the other set's loads behind it, where paths with and
    // without a load would make it wait for both sets.
    RFP4_PF_LOAD(0u, kr0, vr0);
    RFP4_PF_LOAD(1u, kr1, vr1);

    // the block's scores, softmax and P V from the staged K / V
    auto block = [&](uint32_t b) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const uint32_t t = (uint32_t)(wave * MT + mt);
            // ---- S = Q K^T for the block's two 16-key halves
            f32x4 s[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                s[h] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int k = 0; k < KS; k++) {
                    const f16x8 kb = *(const f16x8 *)&ks[16u * h + l16][32 * k + 8u * q4];
                    s[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[mt][k], kb, s[h], 0, 0, 0);
                    s[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ql[mt][k], kb, s[h], 0, 0, 0);
                }
            }
            // ---- causal mask, online softmax (base 2) per row 4 q4 + r
            float p[2][4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t qrow = r0 + 16u * (t / GT) + 4u * q4 + (uint32_t)r;
                const uint32_t qpos = pos0 + min(qrow, nrows - 1u);
                float mx = -3.402823466e38f;
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const uint32_t key = b * PF_BK + 16u * h + l16;
                    const float v = s[h][r] * scale;
                    p[h][r] = key <= qpos ? v : -3.402823466e38f;
                    mx = fmaxf(mx, p[h][r]);
                }
                mx = row16_max(mx);
                const float mnew = fmaxf(mrun[mt][r], mx);
                const float alpha = __builtin_amdgcn_exp2f(mrun[mt][r] - mnew);
                mrun[mt][r] = mnew;
                float ls = 0.0f;
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    p[h][r] = __builtin_amdgcn_exp2f(p[h][r] - mnew);
                    ls += p[h][r];
                }
                lrun[mt][r] = fmaf(lrun[mt][r], alpha, row16_sum(ls));
#pragma unroll
                for (int n = 0; n < NN; n++) o[mt][n][r] *= alpha;
            }
            // ---- P (hi, lo) to the A layout through LDS (this wave's rows only)
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const _Float16 ph = (_Float16)p[h][r];
                    ps[wave][mt][0][4u * q4 + (uint32_t)r][16u * h + l16] = ph;
                    ps[wave][mt][1][4u * q4 + (uint32_t)r][16u * h + l16] = (_Float16)(p[h][r] - (float)ph);
                }
            __builtin_amdgcn_wave_barrier();
            const f16x8 pa = *(const f16x8 *)&ps[wave][mt][0][l16][8u * q4];
            const f16x8 pl = *(const f16x8 *)&ps[wave][mt][1][l16][8u * q4];
            // ---- O += P V
#pragma unroll
            for (int n = 0; n < NN; n++) {
                const f16x8 vb = *(const f16x8 *)&vt[16u * n + l16][8u * q4];
                o[mt][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, vb, o[mt][n], 0, 0, 0);
                o[mt][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl, vb, o[mt][n], 0, 0, 0);
            }
        }
    };
    uint32_t b = 0;
    for (; b + 1u < nblk; b += 2u) {
        RFP4_PF_STAGE(b, kr0, vr0);
        block(b);
        RFP4_PF_STAGE(b + 1u, kr1, vr1);
        block(b + 1u);
    }
    if (b < nblk) {
        RFP4_PF_STAGE(b, kr0, vr0);
        block(b);
    }
#undef RFP4_PF_STAGE
#undef RFP4_PF_LOAD

    // ---- out[row][head][dim] = O / l for rows in the prompt and heads < G
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const uint32_t t = (uint32_t)(wave * MT + mt), g = t % GT;
        if (g >= G) continue;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t row = r0 + 16u * (t / GT) + 4u * q4 + (uint32_t)r;
            if (row >= nrows) continue;
            float *op = a.out + (size_t)row * a.out_rs + (size_t)(kvh * G + g) * HD + l16;
#pragma unroll
            for (int n = 0; n < NN; n++) op[16 * n] = __fdiv_rn(o[mt][n][r], lrun[mt][r]);
        }
    }
}

// Workgroup x of KV head blockIdx.y: query tile x, or, paired, tiles
// ntiles - 1 - x (the longer causal range, first) and x, so that every
// workgroup walks ntiles + 1 key ranges' worth of blocks.
template <int HD, int GT, int NW = 4>
RFP4_DEV void attn_prefill_body(const AttnPrefillArgs &a)
{
    constexpr uint32_t BQ = (uint32_t)attn_prefill_rows(GT, NW);
    const uint32_t ntiles = (a.rows + BQ - 1u) / BQ, x = blockIdx.x;
    const uint32_t t0 = a.paired ? ntiles - 1u - x : x;
    const uint32_t npass = a.paired && x < t0 ? 2u : 1u;
#pragma nounroll
    for (uint32_t pass = 0; pass < npass; pass++) attn_prefill_tile<HD, GT, NW>(a, (pass == 0 ? t0 : x) * BQ);
}
