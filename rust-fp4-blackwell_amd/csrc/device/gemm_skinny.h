// MXFP4 GEMM for few activation rows (M <= 64): the batched-decode case,
// streamed like a GEMV.  C[M][N] = A[M][K] . W[N][K]^T, A and W MXFP4 (E2M1
// codes two per byte, low nibble first; E8M0 per 32 along K), C f32.
// Semantics as gemm.h (trackb/fp4_scale_test.cu:37 taken to M x N x K).
//
// MFMA: v_mfma_scale_f32_16x16x128_f8f6f4, A = activation rows, B = W rows.
// Lane l holds row l%16 of its fragment and the K values 32*(l/16) .. +31 of
// the 128-wide tile with that block's scale byte; D register r of lane l is
// D[4*(l/16) + r][l%16] (pinned by the 16x16 layout test).  K advances in
// segments of 512 values (256 bytes per row): lane (r, q = l/16) loads the
// 64 bytes 64q .. 64q+63 of the segment and one dword of its 4 scale bytes;
// MFMA t (0..3) of the segment takes bytes 64q + 16t .. +15 (values 128q +
// 32t .. +31) and scale byte t of the dword, in A and W alike, so the K
// permutation cancels.
//
// Workgroup: 16 * NB rows of W (NB B fragments), all M rows of A (MA
// fragments of 16), 4 waves splitting K in quarters.  Each wave keeps the
// loads of the next segment in flight while it runs the MFMAs of the current
// one; the four partial tiles are summed through LDS in wave order.
#pragma once
#include "common.h"
#include "mma.h"

template <int MA, int NB>
RFP4_DEV void gemm_skinny_body(const GemmArgs &g)
{
    constexpr uint32_t NF = (uint32_t)(MA + NB);
    __shared__ float red[3][MA * NB * 4][64];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t r16 = lane & 15u, q = lane >> 4;
    const uint32_t n0 = blockIdx.x * (16u * NB);
    const uint32_t kbytes = g.k >> 1, nblk = g.k >> 5;
    const uint32_t nseg = g.k >> 9, per = nseg / 4u; // host: k % 2048 == 0
    const uint32_t seg0 = wave * per;

    // row pointers of the MA + NB fragments (clamped: loads stay in bounds)
    const uint8_t *cp[NF], *sp[NF];
#pragma unroll
    for (int f = 0; f < MA; f++) {
        const uint32_t row = min(16u * f + r16, g.m - 1u);
        cp[f] = g.a_codes + (size_t)row * kbytes + q * 64u;
        sp[f] = g.a_scales + (size_t)row * nblk + q * 4u;
    }
#pragma unroll
    for (int f = 0; f < NB; f++) {
        const uint32_t row = min(n0 + 16u * f + r16, g.n - 1u);
        cp[MA + f] = g.w_codes + (size_t)row * kbytes + q * 64u;
        sp[MA + f] = g.w_scales + (size_t)row * nblk + q * 4u;
    }

    v4f32 acc[MA][NB];
#pragma unroll
    for (int a = 0; a < MA; a++)
#pragma unroll
        for (int b = 0; b < NB; b++) acc[a][b] = {0.0f, 0.0f, 0.0f, 0.0f};

    uint4 cur[NF][4], nxt[NF][4];
    uint32_t scur[NF], snxt[NF];
#define RFP4_SKINNY_LOAD(DST, SDST, SEG)                                                        \
    do {                                                                                        \
        _Pragma("unroll") for (uint32_t f = 0; f < NF; f++) {                                   \
            _Pragma("unroll") for (int t = 0; t < 4; t++) DST[f][t] =                           \
                *(const uint4 *)(cp[f] + (size_t)(SEG) * 256u + t * 16u);                       \
            SDST[f] = *(const uint32_t *)(sp[f] + (size_t)(SEG) * 16u);                        \
        }                                                                                       \
    } while (0)
    RFP4_SKINNY_LOAD(cur, scur, seg0);
    for (uint32_t s = 0; s < per; s++) {
        if (s + 1u < per) RFP4_SKINNY_LOAD(nxt, snxt, seg0 + s + 1u);
#pragma unroll
        for (int t = 0; t < 4; t++) {
#pragma unroll
            for (int a = 0; a < MA; a++) {
                const v8i32 a8 = {(int)cur[a][t].x, (int)cur[a][t].y, (int)cur[a][t].z, (int)cur[a][t].w, 0, 0, 0, 0};
                const int sa = (int)((scur[a] >> (8 * t)) & 0xFFu);
#pragma unroll
                for (int b = 0; b < NB; b++) {
                    const uint4 w = cur[MA + b][t];
                    const v8i32 b8 = {(int)w.x, (int)w.y, (int)w.z, (int)w.w, 0, 0, 0, 0};
                    const int sb = (int)((scur[MA + b] >> (8 * t)) & 0xFFu);
                    acc[a][b] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a8, b8, acc[a][b], MX_FMT_FP4,
                                                                                 MX_FMT_FP4, 0, sa, 0, sb);
                }
            }
        }
        if (s + 1u < per) {
#pragma unroll
            for (uint32_t f = 0; f < NF; f++) {
#pragma unroll
                for (int t = 0; t < 4; t++) cur[f][t] = nxt[f][t];
                scur[f] = snxt[f];
            }
        }
    }
#undef RFP4_SKINNY_LOAD

    // ---- sum the four K quarters in wave order, then store rows < M, cols < N
    if (wave > 0) {
#pragma unroll
        for (int a = 0; a < MA; a++)
#pragma unroll
            for (int b = 0; b < NB; b++)
#pragma unroll
                for (int r = 0; r < 4; r++) red[wave - 1][(a * NB + b) * 4 + r][lane] = acc[a][b][r];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int a = 0; a < MA; a++)
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float v = acc[a][b][r];
#pragma unroll
                for (int w = 0; w < 3; w++) v = __fadd_rn(v, red[w][(a * NB + b) * 4 + r][lane]);
                const uint32_t row = 16u * a + 4u * q + (uint32_t)r, col = n0 + 16u * b + r16;
                if (row < g.m && col < g.n) g.c[(size_t)row * g.n + col] = v;
            }
}
