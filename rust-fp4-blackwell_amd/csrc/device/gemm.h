// Batched MXFP4 GEMM on gfx950 scaled MFMA:
//   C[M][N] = A[M][K] . W[N][K]^T, A and W MXFP4 (E2M1 codes two per byte,
//   low nibble first; one E8M0 scale per 32 values along K; row-major, the
//   layout the engine stores weights in), C f32 row-major.
// The reference validates one m16n8k64 block-scaled tile (fp4_mma,
// trackb/*) and has no GEMM (main.tex:228); the CPU closed form is
// trackb/fp4_scale_test.cu:37 extended to M x N x K.
//
// MFMA: v_mfma_scale_f32_32x32x64_f8f6f4, both operands E2M1.  Lane l holds
// row l%32 of its fragment and the 32 K values 32*(l/32) .. +31 of the
// 64-wide tile, with that block's scale byte (pinned by the 32x32 layout
// test).  K advances in steps of 256 values = 128 bytes per row: lane
// (r, h = l/32) takes bytes 64h .. 64h+63 of the step, and MFMA t (0..3) of
// the step consumes bytes 64h + 16t .. +15 (values 128h + 32t .. +31) with
// scale byte 4h + t of the step.  A and W are permuted along K the same way,
// so C is unchanged.
//
// Workgroup: 4 waves in a WM x WN grid, wave tile (32 FA) x (32 FB), block
// tile BM x BN.  Each K step (BM + BN rows of 128 code bytes and 8 scale
// bytes) is copied global -> LDS by the DMA path (global_load_lds, no
// staging registers) into a ring of NST stage buffers.  The scales come from
// the step-blocked copies (GemmArgs::a_st, w_st): a 32-row block's 8 bytes
// per row of one step are 256 contiguous bytes, copied as they are into the
// stage's two 32-word planes.  From the row-major [rows][k/32] scales each
// step would touch one cache line per row for 8 bytes, as many L2 requests as
// the code bytes need (measured on the DMA stream alone, M = 512: 64x128
// tiles 7.8 us without scales, 12.3 us with row-major scales, 8.4 us with
// step-blocked ones).  A wave reads all its
// operands of step s from LDS, issues the DMA of step s + NST - 1 into the
// buffer step s - 1 used, then runs the step's MFMAs while the copies are in
// flight; one barrier per step.  NST = 2 (double buffering) waits for all of
// the wave's copies (vmcnt(0)) before the barrier; deeper rings wait only for
// step s + 1's copies (every wave issues the same number per step, so the
// count is a constant) and use a bare s_barrier, since __syncthreads' release
// fence would make the compiler wait for every copy in flight.  Code rows are
// 128 bytes with the 16-byte chunks XOR-swizzled by row (gemm_swz).
//
// Grid: one dimension, tiles ordered m fastest, then n, then the K split z;
// the linear id is first remapped so that each XCD (id % 8 at dispatch) gets
// a contiguous range of tiles and the m-tiles sharing a W tile share its L2.
// With kz > 1 each split writes its partial tile to part[z]; the reduce
// kernel launched next sums the kz planes in z order, so the result does not
// depend on the order the workgroups ran in.
#pragma once
#include <type_traits>
#include "common.h"
#include "mma.h"
#include "misc.h"
#include "gemv.h"

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) uint8_t rfp4_lds_u8;
typedef __attribute__((address_space(1))) void rfp4_glb_void;

// Physical 16-byte chunk of logical chunk q in LDS row r: an XOR swizzle that
// keeps the fragment reads of 8 (and of 16) consecutive rows on distinct banks.
RFP4_DEV uint32_t gemm_swz(uint32_t r) { return (r ^ (r >> 3)) & 7u; }

// Wait until at most n steps' DMAs of this wave are in flight (C DMA
// instructions per step; n < 4): they complete in issue order.
template <uint32_t C>
RFP4_DEV void gemm_wait_steps(uint32_t n)
{
    static_assert(3u * C < 64u, "vmcnt field");
#define RFP4_VMCNT(V) (((V) & 0xFu) | (((V) >> 4) << 14) | (0x7u << 4) | (0xFu << 8))
    if (n == 0u) __builtin_amdgcn_s_waitcnt(RFP4_VMCNT(0u));
    else if (n == 1u) __builtin_amdgcn_s_waitcnt(RFP4_VMCNT(C));
    else if (n == 2u) __builtin_amdgcn_s_waitcnt(RFP4_VMCNT(2u * C));
    else __builtin_amdgcn_s_waitcnt(RFP4_VMCNT(3u * C));
#undef RFP4_VMCNT
}

// Two-way split-K sum inside the launch (kz = 2): each split stores its
// partial tile to part[z] with agent-scope stores, waits for them, and bumps
// the tile's arrival counter; the split whose increment completes the count
// reads the other plane with agent-scope loads and writes c = part[0] +
// part[1] (its own plane from registers), the reduce kernel's sums bit for
// bit, then resets the counter for the next launch.  No split waits for
// another.  Publication without a fence: on gfx950 a relaxed agent-scope
// store is a write-through global_store ... sc1, s_waitcnt vmcnt(0) returns
// once it is acknowledged at the device-coherent level, and a relaxed
// agent-scope load (global_load ... sc1) reads that level; the attention
// merge (device/attn.h) relies on the same three facts.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "the in-launch split-K sum's publication protocol is written for gfx950's sc1 accesses"
#endif
template <int FA, int FB>
RFP4_DEV void gemm_splitk_last(const GemmArgs &g, const v16f32 (&acc)[FA][FB], uint32_t m0, uint32_t n0, uint32_t r32,
                               uint32_t h, uint32_t z, uint32_t tile)
{
    __shared__ uint32_t s_last;
    const size_t plane = (size_t)g.m * g.n;
    float *mine = g.part + (size_t)z * plane;
#pragma unroll
    for (int fa = 0; fa < FA; fa++)
#pragma unroll
        for (int fb = 0; fb < FB; fb++) {
            const uint32_t col = n0 + 32u * fb + r32;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const uint32_t row = m0 + 32u * fa + 8u * (uint32_t)(r / 4) + 4u * h + (uint32_t)(r % 4);
                if (row < g.m && col < g.n)
                    __hip_atomic_store(mine + (size_t)row * g.n + col, acc[fa][fb][r], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); // this thread's partial is acknowledged
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t old = __hip_atomic_fetch_add(g.counters + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = old + 1u == g.kz ? 1u : 0u;
    }
    __syncthreads();
    if (!s_last) return;
    if (threadIdx.x == 0) __hip_atomic_store(g.counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // every load of the other plane (and, with c_add, of c) first (one round
    // trip), then the sums
    const float *other = g.part + (size_t)(1u - z) * plane;
    float o[FA][FB][16], cv[FA][FB][16];
#pragma unroll
    for (int fa = 0; fa < FA; fa++)
#pragma unroll
        for (int fb = 0; fb < FB; fb++) {
            const uint32_t col = min(n0 + 32u * fb + r32, g.n - 1u);
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const uint32_t row = min(m0 + 32u * fa + 8u * (uint32_t)(r / 4) + 4u * h + (uint32_t)(r % 4), g.m - 1u);
                o[fa][fb][r] = __hip_atomic_load(other + (size_t)row * g.n + col, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (g.c_add) cv[fa][fb][r] = g.c[(size_t)row * g.n + col];
            }
        }
#pragma unroll
    for (int fa = 0; fa < FA; fa++)
#pragma unroll
        for (int fb = 0; fb < FB; fb++) {
            const uint32_t col = n0 + 32u * fb + r32;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const uint32_t row = m0 + 32u * fa + 8u * (uint32_t)(r / 4) + 4u * h + (uint32_t)(r % 4);
                float v = z == 0u ? __fadd_rn(acc[fa][fb][r], o[fa][fb][r]) : __fadd_rn(o[fa][fb][r], acc[fa][fb][r]);
                if (g.c_add) v = __fadd_rn(cv[fa][fb][r], v);
                if (row < g.m && col < g.n) g.c[(size_t)row * g.n + col] = v;
            }
        }
}

// The plain epilogue: the wave's accumulators (tile rows m0 .., columns n0
// ..) into dst, or, with c_add (kz = 1), added to dst: for FAB row
// fragments at a time every element of dst is loaded first, then one wait,
// then the sums and stores (a load issued behind a store would also wait
// for that store: one batch where the registers hold the whole tile).
// FAB = 0: no accumulating path compiled (the host does not ask it of that
// kernel).
template <int FA, int FB, int FAB>
RFP4_DEV void gemm_store_c(const GemmArgs &g, const v16f32 (&acc)[FA][FB], float *dst, uint32_t m0, uint32_t n0,
                           uint32_t r32, uint32_t h)
{
    static_assert(FAB == 0 || FA % FAB == 0, "whole batches");
    if constexpr (FAB > 0) if (g.c_add && g.kz == 1u) {
#pragma unroll
        for (int f0 = 0; f0 < FA; f0 += FAB) {
            float cv[FAB][FB][16];
#pragma unroll
            for (int i = 0; i < FAB; i++)
#pragma unroll
                for (int fb = 0; fb < FB; fb++) {
                    const uint32_t col = min(n0 + 32u * fb + r32, g.n - 1u);
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const uint32_t row =
                            min(m0 + 32u * (f0 + i) + 8u * (uint32_t)(r / 4) + 4u * h + (uint32_t)(r % 4), g.m - 1u);
                        cv[i][fb][r] = dst[(size_t)row * g.n + col];
                    }
                }
            __builtin_amdgcn_s_waitcnt(0x0F70); // vmcnt(0): the batch's c
#pragma unroll
            for (int i = 0; i < FAB; i++)
#pragma unroll
                for (int fb = 0; fb < FB; fb++) {
                    const uint32_t col = n0 + 32u * fb + r32;
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const uint32_t row = m0 + 32u * (f0 + i) + 8u * (uint32_t)(r / 4) + 4u * h + (uint32_t)(r % 4);
                        if (row < g.m && col < g.n)
                            __builtin_nontemporal_store(__fadd_rn(cv[i][fb][r], acc[f0 + i][fb][r]),
                                                        dst + (size_t)row * g.n + col);
                    }
                }
        }
        return;
    }
#pragma unroll
    for (int fa = 0; fa < FA; fa++)
#pragma unroll
        for (int fb = 0; fb < FB; fb++) {
            const uint32_t col = n0 + 32u * fb + r32;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const uint32_t row = m0 + 32u * fa + 8u * (uint32_t)(r / 4) + 4u * h + (uint32_t)(r % 4);
                // non-temporal: C is written once and read by the next launch
                if (row < g.m && col < g.n) __builtin_nontemporal_store(acc[fa][fb][r], dst + (size_t)row * g.n + col);
            }
        }
}

// RoPE + K/V cache epilogue of the prefill's q|k|v projection
// (GemmArgs::rope_cos; rope_kv_rows_body's result in the GEMM's launch).
// Heads are rope_hd = 64 or 128 columns, a divisor of the tile width, so a
// head lies in one tile and a 32-column fragment in one head: whether a
// fragment is q, k or v, and which half of its head, is the same for every
// lane.  The partner of head column j < half is j + half and the other way
// round: tile column c ^ half, which is the same lane and accumulator
// register of the wave that covers that column (half >= 32).  The waves of
// a workgroup put FS row fragments (fa0 .. fa0 + FS - 1) of their
// accumulators in LDS, slot xw, fragment-native (gemm_rope_put: consecutive
// lanes, consecutive words), and each then reads its own values and its
// partners' from there (gemm_rope_store).  The rotation is rope_pair's,
// each product and sum rounded in the same order, and C's sums are those of
// the same GEMM without the epilogue: the result is bit-identical to the
// GEMM followed by rope_kv_rows_body.
template <int FA, int FB, int FS>
RFP4_DEV void gemm_rope_put(float *xl, uint32_t xw, const v16f32 (&acc)[FA][FB], int fa0, uint32_t lane)
{
#pragma unroll
    for (int fs = 0; fs < FS; fs++)
#pragma unroll
        for (int fb = 0; fb < FB; fb++)
#pragma unroll
            for (int r = 0; r < 16; r++)
                xl[(((xw * FS + fs) * FB + fb) * 16u + (uint32_t)r) * 64u + lane] = acc[fa0 + fs][fb][r];
}

// The FS x FB fragments put from row fragment fa0 on: xw0 is the slot of
// the wave's first column wave (its set holds the same rows), wn its column
// index in the set (columns from tile column 32 FB wn; slot xw0 + wn), m0
// its first row (of row fragment 0), nt0 the tile's first column.  UB
// fragments per batch: the batch's cos and sin loads are issued, then one
// wait, then its LDS reads (own and partner values), rotations and stores,
// with no global load behind a store (gfx9 counts stores in vmcnt: a wait
// for a load issued after a store waits for the store's write too).
template <int FS, int FB, int UB>
RFP4_DEV void gemm_rope_store(const GemmArgs &g, const float *xl, uint32_t xw0, uint32_t wn, uint32_t m0, int fa0,
                              uint32_t nt0, uint32_t lane)
{
    constexpr int NU = FS * FB;
    static_assert(NU % UB == 0, "whole batches");
    const uint32_t r32 = lane & 31u, h = lane >> 5;
    const uint32_t hd = g.rope_hd, half = hd >> 1, qk = g.rope_q + g.rope_kv;
    const float *__restrict__ cosv = g.rope_cos;
    const float *__restrict__ sinv = g.rope_sin;
    // fragment u = fs * FB + fb: its tile column and first row
    auto frag = [&](uint32_t u, uint32_t &col0, uint32_t &rbase) {
        col0 = nt0 + wn * (32u * FB) + 32u * (u % FB);
        rbase = m0 + 32u * ((uint32_t)fa0 + u / FB) + 4u * h;
    };
#pragma unroll 1
    for (uint32_t u0 = 0; u0 < (uint32_t)NU; u0 += UB) {
        float cv[UB][16], sv[UB][16];
#pragma unroll
        for (int i = 0; i < UB; i++) {
            uint32_t col0, rbase;
            frag(u0 + i, col0, rbase);
            const uint32_t j = (col0 + r32) & (half - 1u);
            if (col0 < qk) {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const uint32_t row = min(rbase + 8u * (uint32_t)(r / 4) + (uint32_t)(r % 4), g.m - 1u);
                    const size_t t = (size_t)(g.rope_pos0 + row) * half + j;
                    cv[i][r] = cosv[t];
                    sv[i][r] = sinv[t];
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0x0F70); // vmcnt(0): the batch's cos and sin
#pragma unroll
        for (int i = 0; i < UB; i++) {
            const uint32_t u = u0 + i, fs = u / FB, fb = u % FB;
            uint32_t col0, rbase;
            frag(u, col0, rbase);
            const uint32_t col = col0 + r32, tc = col0 - nt0, pc = tc ^ half;
            const uint32_t pw = pc / (32u * FB), pfb = (pc >> 5) % (uint32_t)FB;
            const float *op = xl + ((((xw0 + wn) * FS + fs) * FB + fb) * 16u) * 64u + lane;
            const float *pp = xl + ((((xw0 + pw) * FS + fs) * FB + pfb) * 16u) * 64u + lane;
            float v[16];
#pragma unroll
            for (int r = 0; r < 16; r++) v[r] = op[(uint32_t)r * 64u];
            if (col0 < qk) {
                if ((col0 & (hd - 1u)) < half) {
#pragma unroll
                    for (int r = 0; r < 16; r++)
                        v[r] = __fsub_rn(__fmul_rn(v[r], cv[i][r]), __fmul_rn(pp[(uint32_t)r * 64u], sv[i][r]));
                } else {
#pragma unroll
                    for (int r = 0; r < 16; r++)
                        v[r] = __fadd_rn(__fmul_rn(v[r], cv[i][r]), __fmul_rn(pp[(uint32_t)r * 64u], sv[i][r]));
                }
            }
            const bool kv = col0 >= g.rope_q, is_v = col0 >= qk;
            const uint32_t kcol = col - g.rope_q - (is_v ? g.rope_kv : 0u); // k or v columns only
            uint16_t *cache = (is_v ? g.vc : g.kc) + (size_t)(kcol / hd) * g.kv_hs + (kcol & (hd - 1u));
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const uint32_t row = rbase + 8u * (uint32_t)(r / 4) + (uint32_t)(r % 4);
                if (row >= g.m || col >= g.n) continue;
                __builtin_nontemporal_store(v[r], g.c + (size_t)row * g.n + col);
                if (kv) cache[(size_t)(g.rope_pos0 + row) * g.kv_ts] = f32_to_f16_bits(v[r]);
            }
        }
    }
}

// The same epilogue where a wave's 32 FB columns hold whole heads (32 FB >=
// rope_hd): the partner of fragment fb is fragment fb ^ (rope_hd / 64) of
// the same lane and register, no exchange.  n0: the wave's first column.
// RB rows of fragments per batch: the batch's cos and sin loads, one wait,
// then its rotations and stores with no load in flight (the stores sit in
// branches on the column's role, where the compiler would otherwise wait
// for every store before each later load's use).
template <int FA, int FB, int RB>
RFP4_DEV void gemm_rope_store_regs(const GemmArgs &g, const v16f32 (&acc)[FA][FB], uint32_t m0, uint32_t n0,
                                   uint32_t lane)
{
    static_assert(FA % RB == 0, "whole batches");
    const uint32_t r32 = lane & 31u, h = lane >> 5;
    const uint32_t hd = g.rope_hd, half = hd >> 1, qk = g.rope_q + g.rope_kv;
    const float *__restrict__ cosv = g.rope_cos;
    const float *__restrict__ sinv = g.rope_sin;
#pragma unroll
    for (int f0 = 0; f0 < FA; f0 += RB) {
        float cv[RB][FB][16], sv[RB][FB][16];
#pragma unroll
        for (int i = 0; i < RB; i++)
#pragma unroll
            for (int fb = 0; fb < FB; fb++) {
                const uint32_t col0 = n0 + 32u * fb, j = (col0 + r32) & (half - 1u);
                if (col0 < qk) {
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const uint32_t row =
                            min(m0 + 32u * (f0 + i) + 8u * (uint32_t)(r / 4) + 4u * h + (uint32_t)(r % 4), g.m - 1u);
                        const size_t t = (size_t)(g.rope_pos0 + row) * half + j;
                        cv[i][fb][r] = cosv[t];
                        sv[i][fb][r] = sinv[t];
                    }
                }
            }
        __builtin_amdgcn_s_waitcnt(0x0F70); // vmcnt(0): the batch's cos and sin
#pragma unroll
        for (int i = 0; i < RB; i++)
#pragma unroll
            for (int fb = 0; fb < FB; fb++) {
                const int fa = f0 + i;
                const uint32_t col0 = n0 + 32u * fb, col = col0 + r32;
                const bool lo = (col0 & (hd - 1u)) < half, kv = col0 >= g.rope_q, is_v = col0 >= qk;
                const uint32_t kcol = col - g.rope_q - (is_v ? g.rope_kv : 0u); // k or v columns only
                uint16_t *cache = (is_v ? g.vc : g.kc) + (size_t)(kcol / hd) * g.kv_hs + (kcol & (hd - 1u));
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const uint32_t row = m0 + 32u * fa + 8u * (uint32_t)(r / 4) + 4u * h + (uint32_t)(r % 4);
                    float v = acc[fa][fb][r];
                    if (col0 < qk) {
                        // the partner fragment: fb ^ 1 for heads of 64, fb ^ 2 for 128 (FB = 4)
                        const float o = FB >= 4 && hd == 128u ? acc[fa][(fb ^ 2) % FB][r] : acc[fa][(fb ^ 1) % FB][r];
                        v = lo ? __fsub_rn(__fmul_rn(v, cv[i][fb][r]), __fmul_rn(o, sv[i][fb][r]))
                               : __fadd_rn(__fmul_rn(v, cv[i][fb][r]), __fmul_rn(o, sv[i][fb][r]));
                    }
                    if (row >= g.m || col >= g.n) continue;
                    __builtin_nontemporal_store(v, g.c + (size_t)row * g.n + col);
                    if (kv) cache[(size_t)(g.rope_pos0 + row) * g.kv_ts] = f32_to_f16_bits(v);
                }
            }
    }
}

// LDS reads in inline asm (see gemm_body's step) and the wait for them.
RFP4_DEV void gemm_lds_rd16(u32x4 &dst, uint32_t addr) { asm volatile("ds_read_b128 %0, %1" : "=v"(dst) : "v"(addr)); }
RFP4_DEV void gemm_lds_rd4(uint32_t &dst, uint32_t addr) { asm volatile("ds_read_b32 %0, %1" : "=v"(dst) : "v"(addr)); }
// Wait until MFMA group t's fragments (and the scales, read first) have
// returned: at most the 4 (FA + FB) reads per group of groups t + 1 .. 3 may
// be outstanding (a count above 15 waits for 15).  The values are tied to the
// wait, so every use is ordered after it.
template <int FA, int FB>
RFP4_DEV void gemm_lds_wait_group(uint32_t t, u32x4 (&a)[FA], u32x4 (&b)[FB], uint32_t (&sa)[FA], uint32_t (&sb)[FB])
{
    constexpr int G = FA + FB;
    if (t == 0u) asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(3 * G < 15 ? 3 * G : 15));
    else if (t == 1u) asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(2 * G < 15 ? 2 * G : 15));
    else if (t == 2u) asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(G < 15 ? G : 15));
    else asm volatile("s_waitcnt lgkmcnt(0)");
#pragma unroll
    for (int i = 0; i < FA; i++) asm volatile("" : "+v"(a[i]), "+v"(sa[i]));
#pragma unroll
    for (int i = 0; i < FB; i++) asm volatile("" : "+v"(b[i]), "+v"(sb[i]));
}

// The operands of one K step in registers (PIPE), and the wait for their
// reads with every register tied to it.
template <int FA, int FB>
struct GemmOps {
    u32x4 av[4][FA], bv[4][FB];
    uint32_t sa[FA], sb[FB];
};
template <int FA, int FB>
RFP4_DEV void gemm_lds_wait_all(GemmOps<FA, FB> &o)
{
    asm volatile("s_waitcnt lgkmcnt(0)");
#pragma unroll
    for (int t = 0; t < 4; t++) {
#pragma unroll
        for (int i = 0; i < FA; i++) asm volatile("" : "+v"(o.av[t][i]));
#pragma unroll
        for (int i = 0; i < FB; i++) asm volatile("" : "+v"(o.bv[t][i]));
    }
#pragma unroll
    for (int i = 0; i < FA; i++) asm volatile("" : "+v"(o.sa[i]));
#pragma unroll
    for (int i = 0; i < FB; i++) asm volatile("" : "+v"(o.sb[i]));
}

// PIPE: next step's LDS reads overlap this step's MFMAs (two register sets
// of operands); without it the reads and MFMAs of a step run back to back.
// SWQ: the SwiGLU + MXFP4 epilogue of the prefill's gate|up projection, as
// gemm_pp_body's (GemmArgs::q_codes): column tile nt's W rows are gate rows
// (BN/2) nt .. +BN/2 - 1 and the matching up rows pair_off + (BN/2) nt ..;
// the tile writes BN/2 output columns as MXFP4, no C.
template <int WM, int WN, int FA, int FB, int NST = 2, bool PIPE = false, bool ROPE = false, bool SWQ = false>
RFP4_DEV void gemm_body(const GemmArgs &g)
{
    static_assert(WM * WN == 4, "4 waves");
    static_assert(NST >= 2 && NST <= 4, "stages");
    constexpr uint32_t BM = 32u * FA * WM, BN = 32u * FB * WN, R = BM + BN;
    constexpr uint32_t NJ = R / 32u;                 // 8-row code blocks per wave per step (1 KB each)
    constexpr uint32_t NSB = (R / 32u + 3u) / 4u;    // 32-row scale blocks per wave per step (256 B each)
    constexpr uint32_t SC0 = R * 128u, STAGE = R * 128u + R * 8u;
    __shared__ __attribute__((aligned(1024))) uint8_t lds_raw[NST * STAGE];
    rfp4_lds_u8 *lds = (rfp4_lds_u8 *)lds_raw;

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave / WN, wn = wave % WN;
    const uint32_t r32 = lane & 31u, h = lane >> 5;

    // ---- tile of this workgroup
    const uint32_t total = gridDim.x, L = blockIdx.x, q = total >> 3;
    const uint32_t lg = (L < q * 8u) ? (L & 7u) * q + (L >> 3) : L;
    const uint32_t mt_n = (g.m + BM - 1u) / BM, nt_n = (g.n + BN - 1u) / BN;
    const uint32_t mt = lg % mt_n, rest = lg / mt_n, nt = rest % nt_n, z = rest / nt_n;
    const uint32_t kbytes = g.k >> 1, nsuper = g.k >> 8;
    const uint32_t per = (nsuper + g.kz - 1u) / g.kz;
    const uint32_t s0 = min(nsuper, z * per), s1 = min(nsuper, s0 + per);
    // K steps in a rotated order: the workgroup's i-th step copies and
    // multiplies step s0 + (i + rot) % (s1 - s0), rot spread over the W
    // tiles, so that the workgroups of a launch do not all stream the same K
    // offset of their rows at once (DMA stream alone at M = 512: 256x128
    // tiles 15.9 -> 14.8 us, 256x256 25.2 -> 21.6 us).  The sum over K runs
    // in that order, which depends on the column tile only: an output row
    // gets the same sums in whichever row tile it sits (batch invariance).
    const uint32_t nsteps = s1 - s0, rot = nsteps ? (nt * 5u) % nsteps : 0u;
    auto kstep = [&](uint32_t i) {
        const uint32_t t = i - s0 + rot;
        return s0 + (t >= nsteps ? t - nsteps : t);
    };

    // ---- DMA sources.  Code block j of this wave covers tile rows 8 (wave + 4 j) .. +7; lane l
    // fetches logical chunk (l & 7) ^ swz(row) of row 8 (wave + 4 j) + l / 8, which the DMA writes
    // to physical chunk l & 7.  A stage holds each 32-row scale block as two planes of 32 words (the
    // step's scale bytes 0-3, then 4-7, of each row; the step-blocked layout as it is): the 32 lanes
    // of one half-wave read 32 consecutive words, free of bank conflicts (row-major 8-byte rows
    // would put rows r and r + 16 on one bank).
    const uint8_t *src[NJ];
#pragma unroll
    for (uint32_t j = 0; j < NJ; j++) {
        const uint32_t row = 8u * (wave + 4u * j) + (lane >> 3);
        const uint32_t qq = (lane & 7u) ^ gemm_swz(row);
        if (row < BM) src[j] = g.a_codes + (size_t)min(mt * BM + row, g.m - 1u) * kbytes + qq * 16u;
        else if (SWQ) {
            const uint32_t wr = row - BM; // gate rows, then the matching up rows
            src[j] = g.w_codes + (size_t)((wr < BN / 2u ? 0u : g.pair_off - BN / 2u) + nt * (BN / 2u) + wr) * kbytes + qq * 16u;
        } else src[j] = g.w_codes + (size_t)min(nt * BN + (row - BM), g.n - 1u) * kbytes + qq * 16u;
    }
    // Scale block b of this wave covers tile rows 32 (wave + 4 b) .. +31: the
    // step-blocked block of those rows (clamped to the last block, so that
    // every copy stays in bounds), lane l's word at byte 4 l of the step
    const uint8_t *ssrc[NSB];
#pragma unroll
    for (uint32_t b = 0; b < NSB; b++) {
        const uint32_t tb = min(wave + 4u * b, R / 32u - 1u);
        const uint32_t wb = tb - BM / 32u; // W block of the tile (tb >= BM / 32)
        const uint32_t wblk = SWQ ? (wb < BN / 64u ? 0u : (g.pair_off - BN / 2u) >> 5) + nt * (BN / 64u) + wb
                                  : min(nt * (BN / 32u) + wb, (g.n - 1u) >> 5);
        const uint8_t *base = tb < BM / 32u
                                  ? g.a_st + (size_t)min(mt * (BM / 32u) + tb, (g.m - 1u) >> 5) * nsuper * 256u
                                  : g.w_st + (size_t)wblk * nsuper * 256u;
        ssrc[b] = base + lane * 4u;
    }
#define RFP4_GEMM_DMA(S, BUF)                                                                              \
    do {                                                                                                   \
        rfp4_lds_u8 *st_ = lds + (BUF) * STAGE;                                                            \
        _Pragma("unroll") for (uint32_t j = 0; j < NJ; j++) __builtin_amdgcn_global_load_lds(              \
            (rfp4_glb_void *)(src[j] + (size_t)kstep(S) * 128u), st_ + 1024u * (wave + 4u * j), 16, 0, 0); \
        _Pragma("unroll") for (uint32_t b = 0; b < NSB; b++) {                                             \
            const uint32_t bb = ((NST > 2 || PIPE) && wave + 4u * b >= R / 32u) ? 0u : b; /* uniform count: again block 0 */ \
            if (NST > 2 || PIPE || wave + 4u * b < R / 32u)                                                \
                __builtin_amdgcn_global_load_lds((rfp4_glb_void *)(ssrc[bb] + (size_t)kstep(S) * 256u),    \
                                                 st_ + SC0 + 256u * (wave + 4u * bb), 4, 0, 0);            \
        }                                                                                                  \
    } while (0)

    v16f32 acc[FA][FB];
#pragma unroll
    for (int fa = 0; fa < FA; fa++)
#pragma unroll
        for (int fb = 0; fb < FB; fb++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[fa][fb][r] = 0.0f;

    // fragment rows of this lane, their swizzles and scale words (plane h of the row's block)
    uint32_t aoff[FA], boff[FB], asw[FA], bsw[FB], asc[FA], bsc[FB];
#pragma unroll
    for (int fa = 0; fa < FA; fa++) {
        const uint32_t r = wm * (32u * FA) + 32u * fa + r32;
        aoff[fa] = r * 128u;
        asw[fa] = gemm_swz(r);
        asc[fa] = SC0 + 256u * (r >> 5) + 128u * h + 4u * (r & 31u);
    }
#pragma unroll
    for (int fb = 0; fb < FB; fb++) {
        const uint32_t r = BM + wn * (32u * FB) + 32u * fb + r32;
        boff[fb] = r * 128u;
        bsw[fb] = gemm_swz(r);
        bsc[fb] = SC0 + 256u * (r >> 5) + 128u * h + 4u * (r & 31u);
    }

    constexpr uint32_t C = NJ + NSB; // DMA instructions per step and wave (NST > 2: uniform)
    uint32_t s = s0;
    if constexpr (!PIPE) {
    // the first NST - 1 steps in flight, then wait for the first
    uint32_t issued = 0;
#pragma unroll
    for (uint32_t k = 0; k + 1u < (uint32_t)NST; k++)
        if (s0 + k < s1) {
            RFP4_GEMM_DMA(s0 + k, k);
            issued++;
        }
    if (NST == 2) {
        __builtin_amdgcn_s_waitcnt(0x0f70); // vmcnt(0): this wave's DMA has landed in LDS
        __syncthreads();
    } else {
        // a bare barrier: __syncthreads' release fence would wait for every
        // DMA in flight (vmcnt(0)); each wave has waited for its own copies
        // of the first step, and LDS is coherent inside the CU
        gemm_wait_steps<C>(issued > 0u ? issued - 1u : 0u);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    }
    // one K step; FULL: a step with NST - 1 steps of DMA still to issue
    auto step = [&](uint32_t s, auto full_c) {
        constexpr bool FULL = decltype(full_c)::value;
        const uint32_t cur = (s - s0) % (uint32_t)NST;
        const rfp4_lds_u8 *st = lds + cur * STAGE;
        // all operands of the step into registers first (scales, then MFMA t's
        // fragments for t = 0..3), then the next step's DMA, then the MFMAs.
        // The reads are inline asm: the compiler treats every LDS read after an
        // LDS DMA as a possible alias of it and would wait for every DMA in
        // flight (vmcnt(0)) before the first read, so the steps of lookahead
        // of the deeper rings would be waited for one step later anyway.  The
        // stage read here is complete (the wait and barrier before this
        // step); each MFMA group waits for its own reads (LDS reads return in
        // order) with the fragments tied to the wait.
        const uint32_t stb = (uint32_t)(uintptr_t)st;
        u32x4 av[4][FA], bv[4][FB];
        uint32_t sa[FA], sb[FB];
#pragma unroll
        for (int fa = 0; fa < FA; fa++) gemm_lds_rd4(sa[fa], stb + asc[fa]);
#pragma unroll
        for (int fb = 0; fb < FB; fb++) gemm_lds_rd4(sb[fb], stb + bsc[fb]);
#pragma unroll
        for (uint32_t t = 0; t < 4; t++) {
#pragma unroll
            for (int fa = 0; fa < FA; fa++) gemm_lds_rd16(av[t][fa], stb + aoff[fa] + (((4u * h + t) ^ asw[fa]) << 4));
#pragma unroll
            for (int fb = 0; fb < FB; fb++) gemm_lds_rd16(bv[t][fb], stb + boff[fb] + (((4u * h + t) ^ bsw[fb]) << 4));
        }
        if (FULL || s + (uint32_t)NST - 1u < s1) RFP4_GEMM_DMA(s + (uint32_t)NST - 1u, (cur + (uint32_t)NST - 1u) % (uint32_t)NST);
#pragma unroll
        for (uint32_t t = 0; t < 4; t++) {
            // at most the reads of MFMA groups t + 1 .. 3 outstanding (lgkmcnt saturates at 15)
            gemm_lds_wait_group<FA, FB>(t, av[t], bv[t], sa, sb);
#pragma unroll
            for (int fa = 0; fa < FA; fa++) {
                const v8i32 a8 = {(int)av[t][fa].x, (int)av[t][fa].y, (int)av[t][fa].z, (int)av[t][fa].w, 0, 0, 0, 0};
                const int sca = (int)((sa[fa] >> (8u * t)) & 0xFFu);
#pragma unroll
                for (int fb = 0; fb < FB; fb++) {
                    const v8i32 b8 = {(int)bv[t][fb].x, (int)bv[t][fb].y, (int)bv[t][fb].z, (int)bv[t][fb].w,
                                      0, 0, 0, 0};
                    const int scb = (int)((sb[fb] >> (8u * t)) & 0xFFu);
                    acc[fa][fb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, b8, acc[fa][fb], MX_FMT_FP4,
                                                                                  MX_FMT_FP4, 0, sca, 0, scb);
                }
            }
        }
        // the wait for the next step's DMA goes after every MFMA of this step
        __builtin_amdgcn_sched_barrier(0);
        if (NST == 2) {
            __builtin_amdgcn_s_waitcnt(0x0f70); // vmcnt(0)
            __syncthreads();
        } else {
            if (FULL) {
                gemm_wait_steps<C>((uint32_t)NST - 2u);
            } else if (s + 1u < s1) {
                const uint32_t last = min(s + (uint32_t)NST - 1u, s1 - 1u); // the last step whose DMA is out
                gemm_wait_steps<C>(last - (s + 1u));
            }
            // this wave's operand reads of step s returned before its MFMAs:
            // the buffer the next DMA overwrites is free after the barrier
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
        }
    };
    // Deeper rings run the steps with a full lookahead in a loop of their
    // own: its wait count is a constant, so the step is one basic block and
    // the MFMAs stay ahead of the wait (with the wait's branches in the
    // loop the compiler sank them below it, serialising MFMA and copies).
    if constexpr (NST > 2)
        for (; s + (uint32_t)NST - 1u < s1; s++) step(s, std::integral_constant<bool, true>());
    for (; s < s1; s++) step(s, std::integral_constant<bool, false>());
    } else {
    // ---- PIPE: the operands of step s + 1 are read from LDS into a second
    // register set while step s's MFMAs run.  Step s: wait for step s + 1's
    // DMA and the barrier (after it every wave's copies of s + 1 are in LDS
    // and every wave's reads of stage s, waited for at the end of step
    // s - 1, are done), the DMA of step s + NST into stage s's buffer, the
    // reads of step s + 1, the MFMAs of step s (registers complete), then
    // the wait for the reads, with the registers tied to it so that no use or
    // copy of them moves above it.  NST stages give NST - 1 steps of DMA
    // lookahead.  The MFMA sequence is the same as above (bit-identical).
    GemmOps<FA, FB> o0, o1;
    auto reads = [&](uint32_t rs, GemmOps<FA, FB> &o) {
        const uint32_t stb = (uint32_t)(uintptr_t)(lds + ((rs - s0) % (uint32_t)NST) * STAGE);
#pragma unroll
        for (int fa = 0; fa < FA; fa++) gemm_lds_rd4(o.sa[fa], stb + asc[fa]);
#pragma unroll
        for (int fb = 0; fb < FB; fb++) gemm_lds_rd4(o.sb[fb], stb + bsc[fb]);
#pragma unroll
        for (uint32_t t = 0; t < 4; t++) {
#pragma unroll
            for (int fa = 0; fa < FA; fa++) gemm_lds_rd16(o.av[t][fa], stb + aoff[fa] + (((4u * h + t) ^ asw[fa]) << 4));
#pragma unroll
            for (int fb = 0; fb < FB; fb++) gemm_lds_rd16(o.bv[t][fb], stb + boff[fb] + (((4u * h + t) ^ bsw[fb]) << 4));
        }
    };
    auto mfmas = [&](const GemmOps<FA, FB> &o) {
#pragma unroll
        for (uint32_t t = 0; t < 4; t++)
#pragma unroll
            for (int fa = 0; fa < FA; fa++) {
                const v8i32 a8 = {(int)o.av[t][fa].x, (int)o.av[t][fa].y, (int)o.av[t][fa].z, (int)o.av[t][fa].w, 0, 0, 0, 0};
                const int sca = (int)((o.sa[fa] >> (8u * t)) & 0xFFu);
#pragma unroll
                for (int fb = 0; fb < FB; fb++) {
                    const v8i32 b8 = {(int)o.bv[t][fb].x, (int)o.bv[t][fb].y, (int)o.bv[t][fb].z, (int)o.bv[t][fb].w,
                                      0, 0, 0, 0};
                    const int scb = (int)((o.sb[fb] >> (8u * t)) & 0xFFu);
                    acc[fa][fb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, b8, acc[fa][fb], MX_FMT_FP4,
                                                                                  MX_FMT_FP4, 0, sca, 0, scb);
                }
            }
    };
    auto bar = [&]() {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };
    // prologue: the first NST steps in flight (one per stage), step s0 landed, its reads
    uint32_t issued = 0;
#pragma unroll
    for (uint32_t k = 0; k < (uint32_t)NST; k++)
        if (s0 + k < s1) {
            RFP4_GEMM_DMA(s0 + k, k);
            issued++;
        }
    gemm_wait_steps<C>(issued > 0u ? min(issued - 1u, 3u) : 0u);
    bar();
    if (s0 < s1) {
        reads(s0, o0);
        gemm_lds_wait_all<FA, FB>(o0);
    }
    // a step whose successor exists and whose DMA (step s + NST) is issued:
    // the wait counts are constants
    // One wave issues its DMA, LDS reads and MFMAs in program order, and a
    // DMA instruction waits at issue while the CU's memory path is busy (about
    // 60 cycles each, measured), an LDS read while the LDS is: issued back to
    // back the three phases of a 256x128 step took 0.38 + 0.27 + 0.47 us.
    // So the step's DMA and reads go between its MFMAs (MFMA i, then memory
    // instructions i NMEM / NM .. (i + 1) NMEM / NM - 1, alternating DMA and
    // reads), each group pinned by a scheduling barrier; an MFMA runs in its
    // pipe while the next instructions wait to issue.  Each accumulator's
    // MFMAs keep their order (t = 0..3), so the sums are unchanged.
    constexpr int NM = 4 * FA * FB, ND = (int)C, NR = 5 * (FA + FB), NMEM = ND + NR;
    auto mem_op = [&](int j, uint32_t dstep, uint32_t dbuf, uint32_t rstb, GemmOps<FA, FB> &o) {
        // merged order: DMA 0, read 0, DMA 1, read 1, ..., then the rest of the longer list
        const int pairs = ND < NR ? ND : NR;
        int d = -1, r = -1;
        if (j < 2 * pairs) (j & 1) ? (r = j >> 1) : (d = j >> 1);
        else if (ND > NR) d = j - pairs;
        else r = j - pairs;
        if (d >= 0) {
            rfp4_lds_u8 *st_ = lds + dbuf * STAGE;
            if (d < (int)NJ) {
                __builtin_amdgcn_global_load_lds((rfp4_glb_void *)(src[d] + (size_t)kstep(dstep) * 128u),
                                                 st_ + 1024u * (wave + 4u * (uint32_t)d), 16, 0, 0);
            } else {
                const uint32_t b = (uint32_t)d - NJ;
                const uint32_t bb = wave + 4u * b >= R / 32u ? 0u : b; // uniform count: again block 0
                __builtin_amdgcn_global_load_lds((rfp4_glb_void *)(ssrc[bb] + (size_t)kstep(dstep) * 256u),
                                                 st_ + SC0 + 256u * (wave + 4u * bb), 4, 0, 0);
            }
        }
        if (r >= 0) {
            if (r < FA) gemm_lds_rd4(o.sa[r], rstb + asc[r]);
            else if (r < FA + FB) gemm_lds_rd4(o.sb[r - FA], rstb + bsc[r - FA]);
            else {
                const int q = r - FA - FB, t = q / (FA + FB), f = q % (FA + FB);
                if (f < FA) gemm_lds_rd16(o.av[t][f], rstb + aoff[f] + (((4u * h + (uint32_t)t) ^ asw[f]) << 4));
                else gemm_lds_rd16(o.bv[t][f - FA], rstb + boff[f - FA] + (((4u * h + (uint32_t)t) ^ bsw[f - FA]) << 4));
            }
        }
    };
    auto step_full = [&](uint32_t fs, GemmOps<FA, FB> &cur, GemmOps<FA, FB> &nxt) {
        gemm_wait_steps<C>((uint32_t)NST - 2u);
        bar();
        const uint32_t dbuf = (fs - s0) % (uint32_t)NST;
        const uint32_t rstb = (uint32_t)(uintptr_t)(lds + ((fs + 1u - s0) % (uint32_t)NST) * STAGE);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < NM; i++) {
            const int t = i / (FA * FB), fa = (i / FB) % FA, fb = i % FB;
            const v8i32 a8 = {(int)cur.av[t][fa].x, (int)cur.av[t][fa].y, (int)cur.av[t][fa].z, (int)cur.av[t][fa].w,
                              0, 0, 0, 0};
            const v8i32 b8 = {(int)cur.bv[t][fb].x, (int)cur.bv[t][fb].y, (int)cur.bv[t][fb].z, (int)cur.bv[t][fb].w,
                              0, 0, 0, 0};
            const int sca = (int)((cur.sa[fa] >> (8u * (uint32_t)t)) & 0xFFu);
            const int scb = (int)((cur.sb[fb] >> (8u * (uint32_t)t)) & 0xFFu);
            acc[fa][fb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, b8, acc[fa][fb], MX_FMT_FP4, MX_FMT_FP4,
                                                                          0, sca, 0, scb);
#pragma unroll
            for (int j = i * NMEM / NM; j < (i + 1) * NMEM / NM; j++) mem_op(j, fs + (uint32_t)NST, dbuf, rstb, nxt);
            __builtin_amdgcn_sched_barrier(0);
        }
        gemm_lds_wait_all<FA, FB>(nxt);
    };
    auto step_tail = [&](uint32_t ts, GemmOps<FA, FB> &cur, GemmOps<FA, FB> &nxt) {
        if (ts + 1u < s1) {
            const uint32_t last = min(ts + (uint32_t)NST - 1u, s1 - 1u); // the last step whose DMA is out
            gemm_wait_steps<C>(last - (ts + 1u));
            bar();
            if (ts + (uint32_t)NST < s1) RFP4_GEMM_DMA(ts + (uint32_t)NST, (ts - s0) % (uint32_t)NST);
            reads(ts + 1u, nxt);
        }
        mfmas(cur);
        __builtin_amdgcn_sched_barrier(0);
        if (ts + 1u < s1) gemm_lds_wait_all<FA, FB>(nxt);
    };
    for (; s + (uint32_t)NST + 1u < s1; s += 2u) {
        step_full(s, o0, o1);
        step_full(s + 1u, o1, o0);
    }
    for (; s < s1; s += 2u) { // s - s0 is even here: o0 holds step s
        step_tail(s, o0, o1);
        if (s + 1u < s1) step_tail(s + 1u, o1, o0);
    }
    }
#undef RFP4_GEMM_DMA

    // ---- epilogue: accumulator r of lane l is C[8 (r/4) + 4 (l/32) + r%4][l%32] of its fragment
    const uint32_t m0 = mt * BM + wm * (32u * FA), n0 = nt * BN + wn * (32u * FB);
    if constexpr (SWQ) {
        // the 4 waves' accumulators in the stages as a [BM][gate BN/2 | up
        // BN/2] tile (constant register indices), then each thread takes
        // blocks of 32 output columns of one row (consecutive threads on
        // consecutive rows, distinct banks with the padded row) and quantizes
        // them whole, with the row kernel's arithmetic (quant_block32)
        constexpr uint32_t GLD = BN + 4u, NBLK = BN / 64u; // floats per LDS row (padded); output blocks per row
        static_assert(BM * GLD * 4u <= NST * STAGE, "the tile in the stages");
        float *tl = (float *)lds_raw;
        __syncthreads(); // the loop's last LDS reads are done
#pragma unroll
        for (int fa = 0; fa < FA; fa++)
#pragma unroll
            for (int fb = 0; fb < FB; fb++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const uint32_t rl = wm * (32u * FA) + 32u * fa + 8u * (uint32_t)(r / 4) + 4u * h + (uint32_t)(r % 4);
                    tl[rl * GLD + wn * (32u * FB) + 32u * fb + r32] = acc[fa][fb][r];
                }
        __syncthreads();
        const uint32_t nblk = g.pair_off >> 5, nsup = g.pair_off >> 8;
        for (uint32_t e = tid; e < BM * NBLK; e += 256u) {
            const uint32_t rl = e % BM, bl = e / BM;
            const uint32_t row = mt * BM + rl, blk = nt * NBLK + bl;
            const float4 *gp = (const float4 *)(tl + rl * GLD + 32u * bl), *up = (const float4 *)(tl + rl * GLD + BN / 2u + 32u * bl);
            float y[32];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float4 gv = gp[i], uv = up[i];
                y[4 * i] = __fmul_rn(silu_ref(gv.x), uv.x);
                y[4 * i + 1] = __fmul_rn(silu_ref(gv.y), uv.y);
                y[4 * i + 2] = __fmul_rn(silu_ref(gv.z), uv.z);
                y[4 * i + 3] = __fmul_rn(silu_ref(gv.w), uv.w);
            }
            uint4 q16;
            const uint32_t sbyte = quant_block32(y, (uint8_t *)&q16);
            if (row < g.m) {
                *(uint4 *)(g.q_codes + (size_t)row * (g.pair_off >> 1) + (size_t)blk * 16u) = q16;
                g.q_scales[(size_t)row * nblk + blk] = (uint8_t)sbyte;
                if (g.q_scales_t) g.q_scales_t[mx_st_offset(row, blk, nsup)] = (uint8_t)sbyte;
            }
        }
        return;
    }
    if constexpr (ROPE) {
        // Heads that lie whole in the wave's columns (32 FB >= rope_hd):
        // partners in its own registers.  Else the 4 waves' accumulators go
        // to the stages (free after the loop's last LDS reads), slot = wave;
        // a wave's partners sit in its row of waves (the same wm).  Batches
        // of cos / sin loads: the whole wave tile (at most 4 fragments here).
        if constexpr (FB >= 2) {
            if (32u * FB >= g.rope_hd) {
                gemm_rope_store_regs<FA, FB, FA >= 2 ? 2 : 1>(g, acc, m0, n0, lane);
                return;
            }
        }
        static_assert(4u * FA * FB * 16u * 64u * 4u <= NST * STAGE && FA * FB <= 4,
                      "the RoPE epilogue's tiles: the 4 waves' accumulators in the stages");
        float *xl = (float *)lds_raw;
        __syncthreads();
        gemm_rope_put<FA, FB, FA>(xl, wave, acc, 0, lane);
        __syncthreads();
        gemm_rope_store<FA, FB, FA * FB>(g, xl, wm * WN, wn, m0, 0, nt * BN, lane);
        return;
    }
    // (up to 256x128: the other plane's values fit the registers beside the
    // accumulators; the host passes no counters for larger tiles)
    if constexpr (FA * FB <= 8) {
        if (g.kz == 2u && g.counters) {
            gemm_splitk_last<FA, FB>(g, acc, m0, n0, r32, h, z, mt + mt_n * nt);
            return;
        }
    }
    // (c_add: the tiles up to 256x128, one batch; the 4-wave 256x256 tile
    // has no registers for it)
    gemm_store_c<FA, FB, FA * FB <= 8 ? FA : 0>(g, acc, g.kz > 1u ? g.part + (size_t)z * g.m * g.n : g.c, m0, n0, r32, h);
}

// Ping-pong tiled GEMM: 8 waves, two per SIMD, in two groups.  Group g of
// the workgroup (g = wave >> 2; waves w and w + 4 share SIMD w % 4) computes
// tile rows 32 FA g .. +32 FA - 1, wave w % 4 of it the columns 32 FB (w % 4)
// .. +32 FB - 1; block tile BM = 64 FA by BN = 128 FB, the same stage layout
// and DMA sources as gemm_body.  A K step runs as two halves (MFMA groups
// t = 0, 1 and t = 2, 3), each a memory phase (group 0 only: this half's
// share of the next step's DMA; both: the half's operand reads from LDS,
// waited for) and a compute phase (MFMAs only), one workgroup barrier after
// each phase.  Group 1 starts one barrier late, so on every SIMD one wave
// computes while the other issues its copies and reads: the DMA instructions
// that wait at issue no longer hold back the MFMAs.  Barrier events E_0,
// E_1, ...: group 0's memory phase of half-step q (q = 2 (s - s0) + half)
// runs between E_2q and E_2q+1, its compute phase until E_2q+2; group 1's
// phases one event later.  Stage s is complete at E_4(s - s0) (group 0 waits
// for its DMA at the end of the compute phase of half-step 2 (s - s0) - 1);
// group 1 finishes reading stage s - 1 before E_4(s - s0), after which group
// 0 copies step s + 1 into that buffer (the weight rows in half 0, the
// activation rows in half 1).
// Both groups pass the same number of barriers (group 1 one extra at the
// start, group 0 one at the end).  Every accumulator receives its MFMAs in
// gemm_body's order (steps in the rotated order, t = 0..3), so C is
// bit-identical to gemm_body's.  No split-K sum in the launch (kz > 1 writes
// the partial planes for the reduce kernel).
//
// SWQ (the prefill's gate|up projection, GemmArgs::q_codes): the tile's W
// rows are the gate rows and the up rows of 128 output columns (column tile
// nt: gate 128 nt .. +127 in tile columns 0-127, up pair_off + 128 nt .. in
// 128-255), so waves 0, 1 of each group hold gate columns and waves 2, 3 the
// matching up columns.  After the loop the accumulators go through LDS (free
// by then), one wave group at a time, and every thread forms y = silu(g) * u
// for one 32-column block of one row with the row kernel's arithmetic and
// quantizes it (quant_block32: the row quantizer's bytes for the same
// values).  The K steps run in the order rotated for this tile's nt, so the
// sums are those of a GEMM whose column tiles are these pairs: within f32
// rounding of the plain GEMM's (whose gate and up columns sit in different
// tiles), not bit-identical to them.
// EPI: 0 C only, 1 the SwiGLU + MXFP4 epilogue (SWQ), 2 the RoPE + K/V
// cache epilogue (gemm_rope_store; two passes, one per wave group)
template <int FA, int FB, int EPI = 0>
RFP4_DEV void gemm_pp_body(const GemmArgs &g)
{
    constexpr bool SWQ = EPI == 1;
    constexpr uint32_t BM = 64u * FA, BN = 128u * FB, R = BM + BN;
    constexpr uint32_t NJ = R / 32u;                 // 8-row code blocks per group-0 wave per step
    constexpr uint32_t NSB = (R / 32u + 3u) / 4u;    // 32-row scale blocks per group-0 wave per step
    static_assert(R % 128u == 0u, "every group-0 wave copies the same number of blocks");
    constexpr uint32_t SC0 = R * 128u, STAGE = R * 128u + R * 8u;
    __shared__ __attribute__((aligned(1024))) uint8_t lds_raw[2 * STAGE];
    rfp4_lds_u8 *lds = (rfp4_lds_u8 *)lds_raw;

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t grp = wave >> 2, wv = wave & 3u;
    const uint32_t r32 = lane & 31u, h = lane >> 5;

    const uint32_t total = gridDim.x, L = blockIdx.x, q = total >> 3;
    const uint32_t lg = (L < q * 8u) ? (L & 7u) * q + (L >> 3) : L;
    const uint32_t mt_n = (g.m + BM - 1u) / BM, nt_n = (g.n + BN - 1u) / BN;
    const uint32_t mt = lg % mt_n, rest = lg / mt_n, nt = rest % nt_n, z = rest / nt_n;
    const uint32_t kbytes = g.k >> 1, nsuper = g.k >> 8;
    const uint32_t per = (nsuper + g.kz - 1u) / g.kz;
    const uint32_t s0 = min(nsuper, z * per), s1 = min(nsuper, s0 + per);
    const uint32_t nsteps = s1 - s0, rot = nsteps ? (nt * 5u) % nsteps : 0u;
    auto kstep = [&](uint32_t i) {
        const uint32_t t = i - s0 + rot;
        return s0 + (t >= nsteps ? t - nsteps : t);
    };

    // DMA of a group-0 wave: half 0 the weight rows of step S, half 1 the
    // activation rows.  Sources are 32-bit offsets from the matrix bases (the
    // host keeps each matrix's codes and step-blocked scales under 4 GiB),
    // formed at each copy from the lane index, made opaque per call: kept
    // across the loop they would not fit beside the accumulators.
    auto dma = [&](uint32_t S, uint32_t buf, int half) {
        rfp4_lds_u8 *st = lds + buf * STAGE;
        const size_t ko = (size_t)kstep(S) * 128u, so = (size_t)kstep(S) * 256u;
        uint32_t ln = lane;
        asm volatile("" : "+v"(ln));
#pragma unroll
        for (uint32_t j = 0; j < NJ; j++) {
            const bool is_a = 8u * (4u * j) < BM; // rows 8 (wv + 4 j) .. +7 < BM for every wv
            if (is_a != (half == 1)) continue;
            const uint32_t row = 8u * (wv + 4u * j) + (ln >> 3);
            const uint32_t qq = (ln & 7u) ^ gemm_swz(row);
            uint32_t wrow = nt * BN + (row - BM);
            if (SWQ) wrow = (row - BM < BN / 2u ? 0u : g.pair_off - BN / 2u) + nt * (BN / 2u) + (row - BM);
            const uint32_t off = is_a ? min(mt * BM + row, g.m - 1u) * kbytes + qq * 16u
                                      : min(wrow, g.n - 1u) * kbytes + qq * 16u;
            __builtin_amdgcn_global_load_lds((rfp4_glb_void *)((is_a ? g.a_codes : g.w_codes) + ko + off),
                                             st + 1024u * (wv + 4u * j), 16, 0, 0);
        }
#pragma unroll
        for (uint32_t b = 0; b < NSB; b++) {
            const bool is_a = 4u * b < BM / 32u; // block wv + 4 b < BM / 32 for every wv
            if (is_a != (half == 1)) continue;
            const uint32_t tb = wv + 4u * b;
            uint32_t wblk = nt * (BN / 32u) + (tb - BM / 32u);
            if (SWQ)
                wblk = (tb - BM / 32u < BN / 64u ? 0u : (g.pair_off - BN / 2u) >> 5) + nt * (BN / 64u) + (tb - BM / 32u);
            const uint32_t blk = is_a ? min(mt * (BM / 32u) + tb, (g.m - 1u) >> 5) : min(wblk, (g.n - 1u) >> 5);
            __builtin_amdgcn_global_load_lds((rfp4_glb_void *)((is_a ? g.a_st : g.w_st) + so + blk * nsuper * 256u + ln * 4u),
                                             st + SC0 + 256u * tb, 4, 0, 0);
        }
    };

    v16f32 acc[FA][FB];
#pragma unroll
    for (int fa = 0; fa < FA; fa++)
#pragma unroll
        for (int fb = 0; fb < FB; fb++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[fa][fb][r] = 0.0f;

    // fragment rows of this lane: the row's offset with its swizzled chunk
    // of t = 0, and its scale word (plane h of the row's block)
    uint32_t aoff[FA], boff[FB], asc[FA], bsc[FB];
#pragma unroll
    for (int fa = 0; fa < FA; fa++) {
        const uint32_t r = grp * (32u * FA) + 32u * fa + r32;
        aoff[fa] = r * 128u + (((4u * h) ^ gemm_swz(r)) << 4);
        asc[fa] = SC0 + 256u * (r >> 5) + 128u * h + 4u * (r & 31u);
    }
#pragma unroll
    for (int fb = 0; fb < FB; fb++) {
        const uint32_t r = BM + wv * (32u * FB) + 32u * fb + r32;
        boff[fb] = r * 128u + (((4u * h) ^ gemm_swz(r)) << 4);
        bsc[fb] = SC0 + 256u * (r >> 5) + 128u * h + 4u * (r & 31u);
    }

    u32x4 av[2][FA], bv[2][FB];
    uint32_t sa[FA], sb[FB];
    auto bar = [&]() {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };
    // memory phase of (step S, half): this half's operand reads of stage S
    // (the scale words in half 0), then the wait for them with every register
    // tied to it
    auto reads = [&](uint32_t S, int half) {
        uint32_t stb = (uint32_t)(uintptr_t)(lds + ((S - s0) & 1u) * STAGE);
        // opaque to the compiler, so that the 4 (FA + FB) read addresses are
        // formed here (one XOR each) rather than kept in registers across the loop
        asm volatile("" : "+v"(stb));
        if (half == 0) {
#pragma unroll
            for (int fa = 0; fa < FA; fa++) gemm_lds_rd4(sa[fa], stb + asc[fa]);
#pragma unroll
            for (int fb = 0; fb < FB; fb++) gemm_lds_rd4(sb[fb], stb + bsc[fb]);
        }
        // stage bases are 1 KB aligned and rows 128 bytes, so the chunk
        // offset ((4 h + t) ^ swz) << 4 = (4 h ^ swz) << 4 ^ t << 4 is ORed in
#pragma unroll
        for (uint32_t u = 0; u < 2; u++) {
            const uint32_t t = 2u * (uint32_t)half + u;
#pragma unroll
            for (int fa = 0; fa < FA; fa++) gemm_lds_rd16(av[u][fa], (stb + aoff[fa]) ^ (t << 4));
#pragma unroll
            for (int fb = 0; fb < FB; fb++) gemm_lds_rd16(bv[u][fb], (stb + boff[fb]) ^ (t << 4));
        }
        asm volatile("s_waitcnt lgkmcnt(0)");
#pragma unroll
        for (uint32_t u = 0; u < 2; u++) {
#pragma unroll
            for (int fa = 0; fa < FA; fa++) asm volatile("" : "+v"(av[u][fa]));
#pragma unroll
            for (int fb = 0; fb < FB; fb++) asm volatile("" : "+v"(bv[u][fb]));
        }
#pragma unroll
        for (int fa = 0; fa < FA; fa++) asm volatile("" : "+v"(sa[fa]));
#pragma unroll
        for (int fb = 0; fb < FB; fb++) asm volatile("" : "+v"(sb[fb]));
    };
    // MFMA group t takes byte t of each scale word (the instruction's
    // scale byte select), so no byte is extracted into a register of its own
    auto mfma_t = [&](uint32_t u, auto t_c) {
        constexpr int T = decltype(t_c)::value;
#pragma unroll
        for (int fa = 0; fa < FA; fa++) {
            const v8i32 a8 = {(int)av[u][fa].x, (int)av[u][fa].y, (int)av[u][fa].z, (int)av[u][fa].w, 0, 0, 0, 0};
#pragma unroll
            for (int fb = 0; fb < FB; fb++) {
                const v8i32 b8 = {(int)bv[u][fb].x, (int)bv[u][fb].y, (int)bv[u][fb].z, (int)bv[u][fb].w, 0, 0, 0, 0};
                acc[fa][fb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, b8, acc[fa][fb], MX_FMT_FP4, MX_FMT_FP4,
                                                                              T, (int)sa[fa], T, (int)sb[fb]);
            }
        }
    };
    // a half's MFMAs, then every accumulator tied to an empty volatile asm:
    // MFMAs have no side effects, and without the tie the compiler sinks
    // them below the barrier that ends the compute phase
    auto mfmas = [&](int half) {
        if (half == 0) {
            mfma_t(0u, std::integral_constant<int, 0>());
            mfma_t(1u, std::integral_constant<int, 1>());
        } else {
            mfma_t(0u, std::integral_constant<int, 2>());
            mfma_t(1u, std::integral_constant<int, 3>());
        }
#pragma unroll
        for (int fa = 0; fa < FA; fa++)
#pragma unroll
            for (int fb = 0; fb < FB; fb++) asm volatile("" : "+v"(acc[fa][fb]));
    };

    // prologue: group 0 copies step s0 and waits for it (E_0 makes it visible)
    if (grp == 0u && s0 < s1) {
        dma(s0, 0u, 0);
        dma(s0, 0u, 1);
        __builtin_amdgcn_s_waitcnt(0x0f70); // vmcnt(0)
    }
    bar();
    if (grp == 1u) bar(); // group 1 one phase behind
    for (uint32_t s = s0; s < s1; s++) {
        const uint32_t nbuf = ((s - s0) & 1u) ^ 1u;
        const bool more = s + 1u < s1;
#pragma unroll
        for (int half = 0; half < 2; half++) {
            __builtin_amdgcn_sched_barrier(0);
            if (grp == 0u && more) dma(s + 1u, nbuf, half);
            reads(s, half);
            __builtin_amdgcn_sched_barrier(0);
            bar();
            __builtin_amdgcn_sched_barrier(0);
            mfmas(half);
            __builtin_amdgcn_sched_barrier(0);
            if (half == 1 && grp == 0u && more) __builtin_amdgcn_s_waitcnt(0x0f70); // step s + 1 landed
            bar();
        }
    }
    if (grp == 0u) bar(); // the barrier count of group 1

    if constexpr (SWQ) {
        // Every wave is past its last LDS read: the stages are free.  Two
        // passes, one per group: the group's waves put their accumulators in
        // LDS as a [128 rows][gate 128 | up 128] tile (constant register
        // indices), then each of the 512 threads takes one block of 32 output
        // columns of one row (row t % 128, block t / 128: consecutive lanes on
        // consecutive rows, distinct banks with the padded row) and quantizes
        // it whole (quant_block32: no cross-lane step, no register array
        // indexed at run time, which would put the accumulators in scratch).
        constexpr uint32_t GR = 32u * FA, GLD = BN + 4u; // rows per group; floats per LDS row (padded)
        static_assert(GR * GLD * 4u <= 2u * STAGE && BN == 256u && GR * 4u == 512u, "a group's tile in the stages");
        float *tl = (float *)lds_raw;
        const uint32_t nblk = g.pair_off >> 5, nsup = g.pair_off >> 8;
        for (uint32_t pass = 0; pass < 2u; pass++) {
            __syncthreads(); // the previous pass's readers (or the loop's last LDS reads) are done
            if (grp == pass) {
#pragma unroll
                for (int fa = 0; fa < FA; fa++)
#pragma unroll
                    for (int fb = 0; fb < FB; fb++)
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            const uint32_t rl = 32u * fa + 8u * (uint32_t)(r / 4) + 4u * h + (uint32_t)(r % 4);
                            tl[rl * GLD + wv * (32u * FB) + 32u * fb + r32] = acc[fa][fb][r];
                        }
            }
            __syncthreads();
            const uint32_t rl = tid & (GR - 1u), bl = tid / GR;
            const uint32_t row = mt * BM + pass * GR + rl, blk = nt * (BN / 64u) + bl;
            const float4 *gp = (const float4 *)(tl + rl * GLD + 32u * bl), *up = (const float4 *)(tl + rl * GLD + BN / 2u + 32u * bl);
            float y[32];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float4 gv = gp[i], uv = up[i];
                y[4 * i] = __fmul_rn(silu_ref(gv.x), uv.x);
                y[4 * i + 1] = __fmul_rn(silu_ref(gv.y), uv.y);
                y[4 * i + 2] = __fmul_rn(silu_ref(gv.z), uv.z);
                y[4 * i + 3] = __fmul_rn(silu_ref(gv.w), uv.w);
            }
            uint4 q16;
            const uint32_t sbyte = quant_block32(y, (uint8_t *)&q16);
            if (row < g.m) {
                *(uint4 *)(g.q_codes + (size_t)row * (g.pair_off >> 1) + (size_t)blk * 16u) = q16;
                g.q_scales[(size_t)row * nblk + blk] = (uint8_t)sbyte;
                if (g.q_scales_t) g.q_scales_t[mx_st_offset(row, blk, nsup)] = (uint8_t)sbyte;
            }
        }
        return;
    }

    const uint32_t m0 = mt * BM + grp * (32u * FA), n0 = nt * BN + wv * (32u * FB);
    if constexpr (EPI == 2) {
        // two passes over halves of the row fragments, all 8 waves in each
        // (slot = wave; a group's 4 waves hold the same rows)
        constexpr int FS = FA / 2;
        static_assert(FA % 2 == 0 && 8u * FS * FB * 16u * 64u * 4u <= 2u * STAGE, "half the accumulators in the stages");
        float *xl = (float *)lds_raw;
#pragma unroll
        for (int pass = 0; pass < 2; pass++) {
            __syncthreads(); // the previous pass's readers (or the loop's last LDS reads) are done
            gemm_rope_put<FA, FB, FS>(xl, wave, acc, FS * pass, lane);
            __syncthreads();
            gemm_rope_store<FS, FB, 2>(g, xl, 4u * grp, wv, m0, FS * pass, nt * BN, lane);
        }
        return;
    }
    gemm_store_c<FA, FB, 1>(g, acc, g.kz > 1u ? g.part + (size_t)z * g.m * g.n : g.c, m0, n0, r32, h);
}

// Split-K sum: c = part[0] + part[1] + ... + part[kz-1] in that order (the
// launch after the GEMM on the same stream, so no cross-workgroup ordering is
// needed).  Four floats per thread.
RFP4_DEV void gemm_reduce_body(const GemmArgs &g)
{
    const size_t plane = (size_t)g.m * g.n, n4 = plane / 4u;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < n4; e += (size_t)gridDim.x * blockDim.x) {
        float4 sum = ((const float4 *)g.part)[e];
        for (uint32_t z = 1; z < g.kz; z++) {
            const float4 p = ((const float4 *)(g.part + z * plane))[e];
            sum.x = __fadd_rn(sum.x, p.x);
            sum.y = __fadd_rn(sum.y, p.y);
            sum.z = __fadd_rn(sum.z, p.z);
            sum.w = __fadd_rn(sum.w, p.w);
        }
        if (g.c_add) {
            const float4 c = ((const float4 *)g.c)[e];
            sum = make_float4(__fadd_rn(c.x, sum.x), __fadd_rn(c.y, sum.y), __fadd_rn(c.z, sum.z), __fadd_rn(c.w, sum.w));
        }
        ((float4 *)g.c)[e] = sum;
    }
}

// Row-major E8M0 scales -> the step-blocked layout (GemmArgs::a_st): one
// thread per output word, matrix 0's words first; word l of (row block rb,
// step s) is bytes 8 s + 4 (l / 32) .. +3 of row 32 rb + l % 32 (zero past
// the last row).
RFP4_DEV void scales_tile_body(const ScaleTileArgs &a)
{
    const uint32_t nsuper = a.k >> 8, nblk = a.k >> 5;
    const uint64_t w0 = (uint64_t)((a.rows[0] + 31u) >> 5) * nsuper * 64u;
    const uint64_t words = w0 + (uint64_t)((a.rows[1] + 31u) >> 5) * nsuper * 64u;
    for (uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; t < words; t += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t mtx = t < w0 ? 0u : 1u;
        const uint64_t w = t - (mtx ? w0 : 0u);
        const uint32_t l = (uint32_t)(w & 63u);
        const uint64_t bs = w >> 6;
        const uint32_t st = (uint32_t)(bs % nsuper), rb = (uint32_t)(bs / nsuper);
        const uint32_t row = 32u * rb + (l & 31u);
        uint32_t v = 0u;
        if (row < a.rows[mtx]) v = *(const uint32_t *)(a.src[mtx] + (size_t)row * nblk + 8u * st + 4u * (l >> 5));
        ((uint32_t *)a.dst[mtx])[w] = v;
    }
}
