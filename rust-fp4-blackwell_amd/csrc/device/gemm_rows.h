// MXFP4 GEMM for few activation rows (M <= 16 MB, the batched-decode case),
// streamed like the decode GEMV: C[M][N] = A[M][K] . W[N][K]^T, A and W
// MXFP4 (E2M1 codes two per byte, low nibble first; E8M0 per 32 along K),
// C f32.  Semantics as gemm.h (trackb/fp4_scale_test.cu:37 taken to M x N x K).
//
// MFMA: v_mfma_scale_f32_16x16x128_f8f6f4 with the W rows as the A operand
// and the activation rows as the B operand, so D[i][j] = sum_k W[n0 + i][k]
// A[16 mb + j][k]: lane l holds operand row l % 16 and the K values
// 32 (l / 16) .. +31 of the 128-wide tile with that block's scale byte, and
// D register r of lane l is D[4 (l / 16) + r][l % 16] (pinned by the 16x16
// layout test).  K advances in segments of 512 values (256 bytes per row):
// MFMA t (0..3) of a segment takes bytes 64 t + 16 q .. +15 of it (values
// 128 t + 32 q .. +31, E8M0 block 4 t + q) in lane (r, q = l / 16), in W and
// A alike, so each W load instruction reads 64 contiguous bytes of 16 rows
// and one 16-byte load per lane brings a row's 16 scale bytes of the segment.
//
// Workgroup: one block of 16 NF W rows (NF fragments, which share every
// activation load) and all of K; its NW <= 8 waves (blockDim / 64) take the K
// segments w, w + NW, ... (at most SEG each), with every load of a wave (W,
// the activation rows, their scales) issued before its first MFMA, like the
// GEMV's slices.  The NW partial 16 NF x 16 MB tiles are summed through LDS
// in wave order.  Each weight byte is read once; the activations (M x K/2
// bytes) are re-read by every workgroup from the L2.
//
// The activation rows go through LDS: each wave copies its segments' rows
// with the LDS DMA (global_load_lds, 4 rows x 256 contiguous bytes per
// instruction, the 16-byte chunks XOR-swizzled by row so the fragment reads
// hit distinct banks) and reads them back in the MFMA layout, in passes of at
// most 4 / SEG fragments (16 KB per wave, 128 KB per workgroup) when all MB
// do not fit.  Loading the same bytes straight into registers as 64-byte
// pieces of 16 rows (the W pattern) cost far more from L2, measured at M = 32
// (us): 4096x4096 6.97 -> 6.01, 28672x4096 at NF = 4 20.70 -> 17.77,
// 4096x14336 (two passes) 14.52 -> 11.66; both forms put the same bytes in
// the same MFMA lanes (bit-identical).
#pragma once
#include "common.h"
#include "mma.h"

typedef __attribute__((address_space(3))) uint8_t rows_lds_u8;
typedef __attribute__((address_space(1))) void rows_glb_void;

// activation rows through LDS (see the header), AH fragments of 16 rows per
// pass: with MB > AH the wave takes the MB / AH passes one after another,
// each a DMA of its rows into the same LDS block, the wait, and its MFMAs
// (the W registers and the accumulators of every fragment stay live)
template <int MB, int SEG, int NF, int AH>
RFP4_DEV void gemm_rows_lds_body(const GemmArgs &g)
{
    static_assert(MB % AH == 0, "whole passes");
    constexpr uint32_t ABLK = 4u * AH * 1024u; // one segment's activation rows of one pass, one wave
    static_assert(NF * MB * 4 * 64 * 4 <= (int)(SEG * ABLK), "the partial tiles fit the wave's block");
    __shared__ __attribute__((aligned(1024))) uint8_t lds_raw[8 * SEG * ABLK];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nw = blockDim.x >> 6;
    const uint32_t r16 = lane & 15u, q = lane >> 4;
    const uint32_t n0 = blockIdx.x * 16u * NF;
    const uint32_t kbytes = g.k >> 1, nblk = g.k >> 5, nseg = g.k >> 9;
    rows_lds_u8 *ablk = (rows_lds_u8 *)lds_raw + wave * SEG * ABLK;

    // the DMA of pass P's activation rows (instruction i: pass rows 4 i ..
    // 4 i + 3, lane l: pass row 4 i + l / 16, the row's chunk (l % 16) ^
    // (row % 16) into position l % 16)
    auto dma_pass = [&](uint32_t P) {
#pragma unroll
        for (int s = 0; s < SEG; s++) {
            const uint32_t seg = wave + nw * (uint32_t)s;
            if (seg >= nseg) break;
#pragma unroll
            for (int i = 0; i < 4 * AH; i++) {
                const uint32_t row = 4u * (uint32_t)i + (lane >> 4), arow = min(16u * AH * P + row, g.m - 1u);
                const uint32_t chunk = (lane & 15u) ^ (row & 15u);
                __builtin_amdgcn_global_load_lds(
                    (rows_glb_void *)(g.a_codes + (size_t)arow * kbytes + (size_t)seg * 256u + chunk * 16u),
                    ablk + (uint32_t)s * ABLK + (uint32_t)i * 1024u, 16, 0, 0);
            }
        }
    };

    // every load of this wave's segments first: the first pass's activation
    // rows, all activation scales, the W rows and scales
    dma_pass(0u);
    uint4 wv[SEG][NF][4], wsv[SEG][NF], asv[SEG][MB];
#pragma unroll
    for (int s = 0; s < SEG; s++) {
        const uint32_t seg = wave + nw * (uint32_t)s;
        if (seg >= nseg) break;
#pragma unroll
        for (int mb = 0; mb < MB; mb++)
            asv[s][mb] = *(const uint4 *)(g.a_scales + (size_t)min(16u * mb + r16, g.m - 1u) * nblk + (size_t)seg * 16u);
#pragma unroll
        for (int f = 0; f < NF; f++) {
            const uint32_t wrow = min(n0 + 16u * f + r16, g.n - 1u); // clamp: loads stay in bounds
            const uint8_t *wc = g.w_codes + (size_t)wrow * kbytes + q * 16u;
#pragma unroll
            for (int t = 0; t < 4; t++) wv[s][f][t] = *(const uint4 *)(wc + (size_t)seg * 256u + t * 64u);
            wsv[s][f] = *(const uint4 *)(g.w_scales + (size_t)wrow * nblk + (size_t)seg * 16u);
        }
    }

    v4f32 acc[NF][MB];
#pragma unroll
    for (int f = 0; f < NF; f++)
#pragma unroll
        for (int mb = 0; mb < MB; mb++) acc[f][mb] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int P = 0; P < MB / AH; P++) {
        if (P > 0) {
            // the previous pass's LDS reads have returned before the DMA overwrites the block
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            dma_pass((uint32_t)P);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); // this pass's DMA has landed (each wave reads only its own block)
#pragma unroll
        for (int s = 0; s < SEG; s++) {
            const uint32_t seg = wave + nw * (uint32_t)s;
            if (seg >= nseg) break;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                uint4 av[AH];
#pragma unroll
                for (int h = 0; h < AH; h++) {
                    // pass row R = 16 h + r16, chunk 4 t + q: position (4 t + q) ^ r16 of instruction R / 4, slot R % 4
                    const uint32_t R = 16u * h + r16, pos = (4u * t + q) ^ r16;
                    av[h] = *(const uint4 *)(ablk + (uint32_t)s * ABLK + (R >> 2) * 1024u + (16u * (R & 3u) + pos) * 16u);
                }
#pragma unroll
                for (int f = 0; f < NF; f++) {
                    const uint4 w = wv[s][f][t];
                    const v8i32 w8 = {(int)w.x, (int)w.y, (int)w.z, (int)w.w, 0, 0, 0, 0};
                    const uint32_t sws[4] = {wsv[s][f].x, wsv[s][f].y, wsv[s][f].z, wsv[s][f].w};
                    const int sw = (int)((sws[t] >> (8u * q)) & 0xFFu); // block 4 t + q
#pragma unroll
                    for (int h = 0; h < AH; h++) {
                        const int mb = P * AH + h;
                        const uint4 a = av[h];
                        const v8i32 a8 = {(int)a.x, (int)a.y, (int)a.z, (int)a.w, 0, 0, 0, 0};
                        const uint32_t sas[4] = {asv[s][mb].x, asv[s][mb].y, asv[s][mb].z, asv[s][mb].w};
                        const int sa = (int)((sas[t] >> (8u * q)) & 0xFFu);
                        acc[f][mb] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(w8, a8, acc[f][mb], MX_FMT_FP4,
                                                                                      MX_FMT_FP4, 0, sw, 0, sa);
                    }
                }
            }
        }
    }

    // ---- the partial tiles into the wave's own block (its LDS reads above
    // complete first), then summed in wave order; lane (r16, q) of tile
    // (f, mb) stores C[16 mb + r16][n0 + 16 f + 4 q .. +3]
    float *red = (float *)(lds_raw + wave * SEG * ABLK);
#pragma unroll
    for (int f = 0; f < NF; f++)
#pragma unroll
        for (int mb = 0; mb < MB; mb++)
#pragma unroll
            for (int r = 0; r < 4; r++) red[((f * MB + mb) * 4 + r) * 64 + lane] = acc[f][mb][r];
    __syncthreads();
    for (uint32_t fm = wave; fm < (uint32_t)(NF * MB); fm += nw) {
        const uint32_t f = fm / MB, mb = fm % MB;
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float sum = ((const float *)lds_raw)[(fm * 4 + r) * 64 + lane];
            for (uint32_t w = 1; w < nw; w++)
                sum = __fadd_rn(sum, ((const float *)(lds_raw + w * SEG * ABLK))[(fm * 4 + r) * 64 + lane]);
            v[r] = sum;
        }
        const uint32_t row = 16u * mb + r16, col = n0 + 16u * f + 4u * q;
        if (row >= g.m) continue;
        float *cp = g.c + (size_t)row * g.n + col;
        if (col + 3u < g.n && (g.n & 3u) == 0u) {
            *(float4 *)cp = make_float4(v[0], v[1], v[2], v[3]);
        } else {
#pragma unroll
            for (int r = 0; r < 4; r++)
                if (col + (uint32_t)r < g.n) cp[r] = v[r];
        }
    }
}

// the activation rows through LDS in passes of at most 4 / SEG fragments
template <int MB, int SEG, int NF>
RFP4_DEV void gemm_rows_body(const GemmArgs &g)
{
    static_assert(SEG <= 4 && (SEG * MB <= 4 || MB % (4 / SEG) == 0), "whole passes of at most 16 KB per wave");
    gemm_rows_lds_body<MB, SEG, NF, (SEG * MB <= 4 ? MB : 4 / SEG)>(g);
}
