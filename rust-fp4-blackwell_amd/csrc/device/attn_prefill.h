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
// row's position in blocks of 64 keys (head dim 64) or 32 (128): K rows staged in LDS as loaded, V rows
// staged transposed (dimension-major), as v_mfma_f32_16x16x32_f16 operands,
// every product transposed so that the scores' accumulator is the next
// product's operand as it lies in the registers:
//   S^T (32 x 16) = K (32 x HD) . Q^T         -- B = q as two fp16 terms
//   online softmax per row (base 2, f32)      -- a row lives in the 4 lanes
//                                                l % 16 = row of the wave
//   O^T (HD x 16) += V^T (HD x 32) . P^T      -- B = p as two fp16 terms
// Lane (q4 = l / 16, row l % 16) holds the scores of keys 4 q4 .. +3 and
// 16 + 4 q4 .. +3 of each 32-key half of a block, which are the 8 K values
// of its P^T operand for that half; the V^T operand takes the same 8 keys of
// each dimension (two 8-byte reads of the transposed V rows), so P never
// leaves the registers.
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
#include "misc.h"

#define PF_KPAD 8  // fp16 padding of a staged K row (16 consecutive rows -> 16 distinct bank groups)
#define PF_TPAD 8  // fp16 padding of a transposed V row

// One query tile: prompt rows r0 .. r0 + BQ of KV head blockIdx.y.  QO: the
// kernel variant that can quantize its output rows (AttnPrefillArgs::q_codes;
// a separate instantiation: the epilogue's code changes how the compiler
// schedules the main loop's LDS reads in the same function).
// KSP: key groups.  KSP groups of NW waves take the same query tiles and
// alternate key blocks (group g blocks g, g + KSP, ...; each staging step
// brings KSP blocks into LDS), then merge their softmax states through LDS
// (m the maximum, l and O rescaled by 2^(m_g - m) and summed): the serial
// chain of blocks of a tile is KSP times shorter.
template <int HD, int GT, int NW, bool QO, int KSP = 1>
RFP4_DEV void attn_prefill_tile(const AttnPrefillArgs &a, uint32_t r0)
{
    const uint32_t pos0 = a.pos0, nrows = a.rows;
    constexpr int BQ = attn_prefill_rows(GT, NW);    // prompt rows per workgroup
    constexpr int NT = (BQ / 16) * GT;               // 16-row tiles per workgroup
    constexpr int MT = NT / NW;                      // tiles per wave
    constexpr int KS = HD / 32;                      // K steps of S = Q K^T
    constexpr int NN = HD / 16;                      // 16-wide column tiles of O
    // keys per block: 64 for head dim 64, 32 for 128 (measured: 8B 2048-row
    // kernel 96.4 us with 32, 103.2 with 64; TinyLlama 41.2 -> 37.8 us)
    constexpr int PF_BK = HD == 64 ? 64 : 32;
    constexpr int KROW = HD + PF_KPAD, TROW = PF_BK + PF_TPAD;
    constexpr int LPK = HD / 8;                      // 16-byte pieces per K/V row
    constexpr int T = 64 * NW * KSP;                 // threads
    constexpr int NP = KSP * PF_BK * LPK;            // 16-byte K (and V) pieces per staging step
    constexpr int LD = (NP + T - 1) / T;             // K (and V) pieces per thread per step
    constexpr bool LFULL = NP % T == 0;              // every thread loads LD pieces
    static_assert(NT % NW == 0 && MT >= 1, "tiles per wave");
    static_assert(LFULL || LD == 1, "block load split");
    __shared__ __align__(16) _Float16 ks[KSP][PF_BK][KROW];
    __shared__ __align__(16) _Float16 vt[KSP][HD][TROW];

    const uint32_t kvh = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63;
    // key group; wave within it (KSP = 1: the plain kernel's code, group 0)
    const int kgrp = KSP > 1 ? (tid >> 6) / NW : 0, wave = KSP > 1 ? (tid >> 6) % NW : tid >> 6;
    const uint32_t l16 = (uint32_t)lane & 15u, q4 = (uint32_t)lane >> 4;
    const uint32_t G = a.n_heads / a.n_kv_heads;
    const uint16_t *kc = a.kc + (size_t)kvh * a.hs;
    const uint16_t *vc = a.vc + (size_t)kvh * a.hs;
    // keys of this workgroup: 0 .. position of its last row
    const uint32_t last_row = min(r0 + (uint32_t)BQ, nrows) - 1u;
    const uint32_t nk = pos0 + last_row + 1u;
    const uint32_t nblk = (nk + PF_BK - 1) / PF_BK;
    const uint32_t niter = KSP > 1 ? (nblk + KSP - 1) / KSP : nblk; // staging steps
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

    // O^T tile n: accumulator r of lane l is dimension 16 n + 4 q4 + r of row l16;
    // the running max and sum are the lane's row's
    f32x4 o[MT][NN];
    float mrun[MT], lrun[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        mrun[mt] = -3.402823466e38f;
        lrun[mt] = 0.0f;
#pragma unroll
        for (int n = 0; n < NN; n++) o[mt][n] = {0.0f, 0.0f, 0.0f, 0.0f};
    }

    // ---- K / V block loads: K piece (key tid / LPK, dims 8 (tid % LPK)), V
    // piece (key tid % PF_BK, dims 8 (tid / PF_BK)) -- consecutive lanes take
    // consecutive keys, so the transposed V writes fall on consecutive halves.
    // Cached loads (each key row is read by every query tile of its KV head),
    // two register sets: block b + 2's loads are issued when block b's data
    // has gone to LDS, so each load has two blocks' compute to land.
    // (each set one 8-word vector value per operand, piece j in words 4j ..
    // 4j + 3: vectors stay in registers where the two sets' code is merged)
    static_assert(LD == 1 || LD == 2 || LD == 4, "16-byte pieces per thread and block");
    typedef uint32_t pf_vec __attribute__((ext_vector_type(4 * LD)));
    pf_vec kr0, vr0, kr1, vr1;
    // staging step I holds blocks I KSP .. I KSP + KSP - 1: piece p is piece
    // p % (PF_BK LPK) of block slot p / (PF_BK LPK)
#define RFP4_PF_LOAD(I, KR, VR)                                                                           \
    do {                                                                                                  \
        _Pragma("unroll") for (int j = 0; j < LD; j++) {                                                  \
            /* threads past the step's pieces load the last one again (unused) */                         \
            const uint32_t pa = min((uint32_t)tid + (uint32_t)T * (uint32_t)j, (uint32_t)NP - 1u);        \
            const uint32_t kb0 = ((I) * KSP + pa / (PF_BK * LPK)) * PF_BK, p = pa % (PF_BK * LPK);       \
            const uint32_t kk = min(kb0 + p / LPK, nk - 1u), kd = 8u * (p % LPK);                         \
            const uint32_t vk = min(kb0 + p % PF_BK, nk - 1u), vd = 8u * (p / PF_BK);                      \
            const u32x4 kx = *(const u32x4 *)(kc + (size_t)kk * a.ts + kd);                               \
            const u32x4 vx = *(const u32x4 *)(vc + (size_t)vk * a.ts + vd);                               \
            _Pragma("unroll") for (int i = 0; i < 4; i++) {                                               \
                KR[4 * j + i] = kx[i];                                                                    \
                VR[4 * j + i] = vx[i];                                                                    \
            }                                                                                             \
        }                                                                                                 \
    } while (0)
    // block b's K rows and transposed V rows into LDS, then block b + 2's loads into the same registers
#define RFP4_PF_STAGE(I, KR, VR)                                                                          \
    do {                                                                                                  \
        __syncthreads(); /* the previous step's LDS reads are done */                                     \
        _Pragma("unroll") for (int j = 0; j < LD; j++) {                                                  \
            const uint32_t pa = (uint32_t)tid + (uint32_t)T * (uint32_t)j;                                \
            if (!LFULL && pa >= (uint32_t)NP) break;                                                      \
            const uint32_t sl = pa / (PF_BK * LPK), p = pa % (PF_BK * LPK);                              \
            const u32x4 kx = {KR[4 * j], KR[4 * j + 1], KR[4 * j + 2], KR[4 * j + 3]};                    \
            const u32x4 vx = {VR[4 * j], VR[4 * j + 1], VR[4 * j + 2], VR[4 * j + 3]};                    \
            *(u32x4 *)&ks[sl][p / LPK][8u * (p % LPK)] = kx;                                              \
            const uint32_t vk = p % PF_BK, vd = 8u * (p / PF_BK);                                          \
            _Pragma("unroll") for (int i = 0; i < 4; i++) {                                               \
                vt[sl][vd + 2u * i][vk] = __builtin_bit_cast(_Float16, (uint16_t)(vx[i] & 0xFFFFu));      \
                vt[sl][vd + 2u * i + 1u][vk] = __builtin_bit_cast(_Float16, (uint16_t)(vx[i] >> 16));     \
            }                                                                                             \
        }                                                                                                 \
        __syncthreads();                                                                                  \
        RFP4_PF_LOAD((I) + 2u, KR, VR);                                                                   \
    } while (0)
    // Every load is issued on every path (keys clamped to the last one, so a
    // block past the end re-reads it): the compiler's wait for a set then
    // counts exactly the other set's loads behind it, where paths with and
    // without a load would make it wait for both sets.
    RFP4_PF_LOAD(0u, kr0, vr0);
    RFP4_PF_LOAD(1u, kr1, vr1);

    // the block's scores, softmax and P V from the staged K / V (this key
    // group's block b of the step in slot kgrp; none past the last block)
    auto block = [&](uint32_t b) {
        if (KSP > 1 && b >= nblk) return; // the same for the whole key group
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const uint32_t t = (uint32_t)(wave * MT + mt);
            // ---- S^T = K Q^T for the block's 16-key quarters h: accumulator r
            // of lane l is key 16 h + 4 q4 + r of row l16
            constexpr int NQ = PF_BK / 16;
            f32x4 s[NQ];
#pragma unroll
            for (int h = 0; h < NQ; h++) {
                s[h] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int k = 0; k < KS; k++) {
                    const f16x8 ka = *(const f16x8 *)&ks[kgrp][16u * h + l16][32 * k + 8u * q4];
                    s[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qa[mt][k], s[h], 0, 0, 0);
                    s[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, ql[mt][k], s[h], 0, 0, 0);
                }
            }
            // ---- causal mask (only in blocks that reach past the tile's first
            // row), online softmax (base 2) of the lane's row
            const uint32_t row0 = r0 + 16u * (t / GT);
            const uint32_t qpos = pos0 + min(row0 + l16, nrows - 1u);
            const bool masked = (b + 1u) * PF_BK > pos0 + min(row0, nrows - 1u) + 1u; // the same for the whole wave
            float p[4 * NQ];
            if (masked) {
#pragma unroll
                for (int h = 0; h < NQ; h++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const uint32_t key = b * PF_BK + 16u * h + 4u * q4 + (uint32_t)r;
                        p[4 * h + r] = key <= qpos ? s[h][r] : -3.402823466e38f;
                    }
            } else {
#pragma unroll
                for (int h = 0; h < NQ; h++)
#pragma unroll
                    for (int r = 0; r < 4; r++) p[4 * h + r] = s[h][r];
            }
            // the maximum of the raw scores, then scaled: rounding is monotonic,
            // so this is the maximum of the scaled scores
            float mx = p[0];
#pragma unroll
            for (int i = 1; i < 4 * NQ; i++) mx = fmaxf(mx, p[i]);
            mx = xor32_max(xor16_max(mx)) * scale;
            const float mnew = fmaxf(mrun[mt], mx);
            const float alpha = __builtin_amdgcn_exp2f(mrun[mt] - mnew);
            mrun[mt] = mnew;
            float ls = 0.0f;
#pragma unroll
            for (int i = 0; i < 4 * NQ; i++) {
                p[i] = __builtin_amdgcn_exp2f(p[i] * scale - mnew);
                ls += p[i];
            }
            lrun[mt] = fmaf(lrun[mt], alpha, xor32_sum(xor16_sum(ls)));
#pragma unroll
            for (int n = 0; n < NN; n++) o[mt][n] *= alpha;
            // ---- O^T += V^T P^T per 32-key chunk c (quarters 2c, 2c + 1): P^T as
            // hi + lo operands straight from the registers; V^T dimension row
            // 16 n + l16 at the lane's 8 keys of the chunk
#pragma unroll
            for (int c = 0; c < NQ / 2; c++) {
                f16x8 pb, pl;
                split_hi_lo8_mix(p + 8 * c, pb, pl);
#pragma unroll
                for (int n = 0; n < NN; n++) {
                    const _Float16 *vrow = &vt[kgrp][16u * n + l16][32u * c + 4u * q4];
                    typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
                    const f16x4 v0 = *(const f16x4 *)vrow, v1 = *(const f16x4 *)(vrow + 16);
                    const f16x8 va = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                    o[mt][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb, o[mt][n], 0, 0, 0);
                    o[mt][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pl, o[mt][n], 0, 0, 0);
                }
            }
        }
    };
    uint32_t it = 0;
    for (; it + 1u < niter; it += 2u) {
        RFP4_PF_STAGE(it, kr0, vr0);
        block(it * KSP + (uint32_t)kgrp);
        RFP4_PF_STAGE(it + 1u, kr1, vr1);
        block((it + 1u) * KSP + (uint32_t)kgrp);
    }
    if (it < niter) {
        RFP4_PF_STAGE(it, kr0, vr0);
        block(it * KSP + (uint32_t)kgrp);
    }
#undef RFP4_PF_STAGE
#undef RFP4_PF_LOAD

    if constexpr (KSP > 1) {
        // ---- the key groups' states merged into group 0's: groups 1.. put
        // (O, m, l) in LDS (lane-contiguous words), group 0 combines
        __shared__ float mg[KSP - 1][NW][MT][NN * 4 + 2][64];
        if (kgrp > 0) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                float(*w)[64] = mg[kgrp - 1][wave][mt];
#pragma unroll
                for (int n = 0; n < NN; n++)
#pragma unroll
                    for (int r = 0; r < 4; r++) w[4 * n + r][lane] = o[mt][n][r];
                w[NN * 4][lane] = mrun[mt];
                w[NN * 4 + 1][lane] = lrun[mt];
            }
        }
        __syncthreads();
        if (kgrp > 0) return; // group 0 writes the output
#pragma unroll
        for (int g2 = 0; g2 < KSP - 1; g2++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const float(*w)[64] = mg[g2][wave][mt];
                const float m2 = w[NN * 4][lane], l2 = w[NN * 4 + 1][lane];
                const float m = fmaxf(mrun[mt], m2);
                const float a0 = __builtin_amdgcn_exp2f(mrun[mt] - m), a1 = __builtin_amdgcn_exp2f(m2 - m);
                mrun[mt] = m;
                lrun[mt] = fmaf(lrun[mt], a0, l2 * a1);
#pragma unroll
                for (int n = 0; n < NN; n++)
#pragma unroll
                    for (int r = 0; r < 4; r++) o[mt][n][r] = fmaf(o[mt][n][r], a0, w[4 * n + r][lane] * a1);
            }
    }

    // ---- out[row][head][dim] = O / l for rows in the prompt and heads < G
    // (lane: row l16, dimensions 16 n + 4 q4 .. +3 of each tile n)
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const uint32_t t = (uint32_t)(wave * MT + mt), g = t % GT;
        if (g >= G) continue; // the same for the whole wave
        const uint32_t row = r0 + 16u * (t / GT) + l16, head = kvh * G + g;
        if (a.out && row < nrows) {
            float *op = a.out + (size_t)row * a.out_rs + (size_t)head * HD + 4u * q4;
#pragma unroll
            for (int n = 0; n < NN; n++)
                *(float4 *)(op + 16 * n) = make_float4(__fdiv_rn(o[mt][n][0], lrun[mt]), __fdiv_rn(o[mt][n][1], lrun[mt]),
                                                       __fdiv_rn(o[mt][n][2], lrun[mt]), __fdiv_rn(o[mt][n][3], lrun[mt]));
        }
        if (QO && a.q_codes) {
            // MXFP4 per 32 dimensions (quant_block32's arithmetic): block b of
            // the head is tiles 2b, 2b + 1, i.e. this lane's 8 values and those
            // of lanes ^16, ^32, ^48 (the same row); the maximum first over all
            // four, then each lane codes its two runs of 4 dimensions.  One
            // block at a time, each value formed as the f32 rows would hold it.
            const uint32_t qd = a.n_heads * HD, qd32 = qd / 32u;
#pragma unroll
            for (int b = 0; b < HD / 32; b++) {
                float y[8];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    y[r] = __fdiv_rn(o[mt][2 * b][r], lrun[mt]);
                    y[4 + r] = __fdiv_rn(o[mt][2 * b + 1][r], lrun[mt]);
                }
                float amax = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(y[i]));
                amax = xor32_max(xor16_max(amax));
                int se = 0;
                uint32_t sbyte = 0;
                if (amax != 0.0f) {
                    se = floor_log2_pos(amax) - 2;
                    se = se < -127 ? -127 : (se > 127 ? 127 : se);
                    sbyte = (uint32_t)(se + 127);
                }
                const float sc = ldexpf(1.0f, se); // 1 where amax is 0 (se = 0)
                const uint32_t lo = fp4_pack2<1>(fp4_pack2<0>(0u, y[0], y[1], sc), y[2], y[3], sc);
                const uint32_t hi = fp4_pack2<1>(fp4_pack2<0>(0u, y[4], y[5], sc), y[6], y[7], sc);
                if (row < nrows) {
                    uint8_t *cp = a.q_codes + (size_t)row * (qd / 2u) + (size_t)head * (HD / 2) + 16u * b + 2u * q4;
                    *(uint16_t *)cp = (uint16_t)lo;
                    *(uint16_t *)(cp + 8) = (uint16_t)hi;
                    if (q4 == 0u) {
                        const uint32_t blk = head * (HD / 32) + (uint32_t)b;
                        a.q_scales[(size_t)row * qd32 + blk] = (uint8_t)sbyte;
                        if (a.q_scales_t) a.q_scales_t[mx_st_offset(row, blk, qd / 256u)] = (uint8_t)sbyte;
                    }
                }
            }
        }
    }
}

// Workgroup x of KV head blockIdx.y: query tile x, or, paired, tiles
// ntiles - 1 - x (the longer causal range, first) and x, so that every
// workgroup walks ntiles + 1 key ranges' worth of blocks.
template <int HD, int GT, int NW = 4, bool QO = false, int KSP = 1>
RFP4_DEV void attn_prefill_body(const AttnPrefillArgs &a)
{
    constexpr uint32_t BQ = (uint32_t)attn_prefill_rows(GT, NW);
    const uint32_t ntiles = (a.rows + BQ - 1u) / BQ, x = blockIdx.x;
    const uint32_t t0 = a.paired ? ntiles - 1u - x : x;
    const uint32_t npass = a.paired && x < t0 ? 2u : 1u;
#pragma nounroll
    for (uint32_t pass = 0; pass < npass; pass++) attn_prefill_tile<HD, GT, NW, QO, KSP>(a, (pass == 0 ? t0 : x) * BQ);
}
