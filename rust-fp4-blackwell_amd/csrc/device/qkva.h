// Fused q|k|v GEMV and decode attention: one launch per layer in place of
// the q|k|v GEMV launch and the attention launch (engine decode step, E8M0
// weights, fp16 caches).  Semantics as the two launches it replaces:
// q|k|v = W_qkv . rmsnorm(x) (llama_run/src/main.rs:513-516), then attention
// with fused RoPE and K/V append (:517-529).
//
// Workgroup b takes GEMV tile b (b < n_tiles: rows 4R b .. 4R b + 4R - 1,
// wave w rows 4R b + R w + i) and attention workgroup b (b < n_attn: KV head
// x query-head slice b % (n_kv_heads * head_split), split b / (...)).  Its
// order of work: the position (a scalar load), the tile's x, norm-weight and
// weight loads, the split's rope-table and K/V loads, the tile's staging and
// dot products, its outputs stored as tagged words (float bits | tag << 32,
// tag = the sequence length pos + 1), then the split's q (and, in the split
// owning the current position, the new k and v) polled from those words, and
// the split's arithmetic and merge.  So the K/V stream and the position read
// overlap the GEMV, and one kernel boundary per layer goes away.
//
// Every row is computed with the stand-alone GEMV's arithmetic: the same
// chunk per lane, slice order and wave reduction, and x staged with the RMS
// sum in the order of the WREF-wave GEMV variant the engine would launch
// (WREF = 8: the 512-thread variant's per-thread and per-wave sums, formed by
// 256 threads that each hold two of its threads' values).  The outputs are
// therefore bit-identical to the two-launch step.
//
// Progress: a workgroup waits only in its attention part, only for words
// that GEMV tiles (which never wait) and other splits (tagged merge) store.
// The host launches this kernel only where the whole grid fits on the
// device at once (occupancy x CUs), so every awaited workgroup is resident.
// A poll past its spin limit sets *err, which the engine reports.
#pragma once
#include "attn.h"
#include "gemv.h"

// stage_x_regs<XV / 2, 8> (512 threads, thread t holding x float4 t + 512 v)
// formed by 256 threads that hold float4 tid + 256 j, j < XV: j even belongs
// to virtual thread tid (wave w), j odd to virtual thread tid + 256 (wave w + 4).
template <int XV>
RFP4_DEV void stage_x_regs_w8(float *xs, const float4 *xr, const uint2 *wr, uint32_t k, bool norm, float eps)
{
    __shared__ float red[8];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t k4 = k >> 2;
    float rms = 1.0f;
    if (norm) {
        float se = 0.0f, so = 0.0f;
#pragma unroll
        for (int j = 0; j < XV; j++) {
            float &s = (j & 1) ? so : se;
            s = __fadd_rn(s, __fmul_rn(xr[j].x, xr[j].x));
            s = __fadd_rn(s, __fmul_rn(xr[j].y, xr[j].y));
            s = __fadd_rn(s, __fmul_rn(xr[j].z, xr[j].z));
            s = __fadd_rn(s, __fmul_rn(xr[j].w, xr[j].w));
        }
        se = wave_sum(se);
        so = wave_sum(so);
        if (lane == 0) {
            red[wave] = se;
            red[wave + 4] = so;
        }
        __syncthreads();
        float total = (red[0] + red[1]) + (red[2] + red[3]);
        total += (red[4] + red[5]) + (red[6] + red[7]);
        rms = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(total, (float)k), eps)));
    }
#pragma unroll
    for (int j = 0; j < XV; j++) {
        const uint32_t i4 = (uint32_t)tid + 256u * (uint32_t)j;
        if (i4 >= k4) break;
        float4 o = xr[j];
        if (norm) {
            o.x = __fmul_rn(__fmul_rn(o.x, rms), f16_bits_to_f32((uint16_t)(wr[j].x & 0xFFFFu)));
            o.y = __fmul_rn(__fmul_rn(o.y, rms), f16_bits_to_f32((uint16_t)(wr[j].x >> 16)));
            o.z = __fmul_rn(__fmul_rn(o.z, rms), f16_bits_to_f32((uint16_t)(wr[j].y & 0xFFFFu)));
            o.w = __fmul_rn(__fmul_rn(o.w, rms), f16_bits_to_f32((uint16_t)(wr[j].y >> 16)));
        }
        ((float4 *)xs)[xs_slot(i4)] = o;
    }
    __syncthreads();
}

// One GEMV tile of the fused kernel (E8M0 scales, K <= 2048 NS): the
// stand-alone GEMV's NS > 0 path (device/gemv.h gemv_body) split into the
// load issue and the arithmetic, with tagged stores.
template <int NS, int R, int WREF>
struct QkvTile {
    static constexpr int XV = 2 * NS; // float4 of x per thread (256 threads)
    XRegs<XV, 256u> xg;
    uint4 q[NS][R];
    uint32_t sb[NS][R];
    uint32_t lrow0;

    RFP4_DEV void issue(const GemvArgs &a, uint32_t tile)
    {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        lrow0 = (tile * 4u + (uint32_t)wave) * (uint32_t)R;
        const uint32_t nchunk = a.k >> 5, clast = nchunk - 1u;
        const size_t rowbytes = (size_t)(a.k >> 1);
        xg.issue(a.x, a.norm_w, a.k);
        __builtin_amdgcn_sched_barrier(0); // x before the weight stream
#pragma unroll
        for (int s = 0; s < NS; s++) {
            const uint32_t cl = min((uint32_t)lane + 64u * (uint32_t)s, clast);
#pragma unroll
            for (int p = 0; p < R; p++) {
                const uint32_t lr = lrow0 + (uint32_t)p;
                const uint32_t r = lr < a.n ? lr : a.n - 1u; // clamp: loads stay in bounds
                q[s][p] = load_nt16((const uint8_t *)a.w + (size_t)r * rowbytes + (size_t)cl * 16u);
                sb[s][p] = load_scale_bits<0>(a.scales, (size_t)r * nchunk + cl);
            }
        }
    }

    RFP4_DEV void finish(const GemvArgs &a, unsigned long long *yt, uint32_t tag)
    {
        extern __shared__ float xs[];
        const int lane = threadIdx.x & 63;
        const uint32_t nchunk = a.k >> 5, clast = nchunk - 1u;
        xg.settle(a.k);
        if (WREF == 8)
            stage_x_regs_w8<XV>(xs, xg.xr, xg.wr, a.k, a.norm_w != nullptr, a.eps);
        else
            stage_x_regs<XV, 4>(xs, xg.xr, xg.wr, a.k, a.norm_w != nullptr, a.eps);
        float acc[R];
#pragma unroll
        for (int p = 0; p < R; p++) acc[p] = 0.0f;
#pragma unroll
        for (int s = 0; s < NS; s++) {
            const uint32_t c = (uint32_t)lane + 64u * (uint32_t)s;
            const float live = c < nchunk ? 1.0f : 0.0f;
            float4 xv[8];
            const float4 *xp = (const float4 *)(xs + (size_t)min(c, clast) * GEMV_XS_CHUNK);
#pragma unroll
            for (int j = 0; j < 8; j++) xv[j] = xp[j];
#pragma unroll
            for (int p = 0; p < R; p++) acc[p] = fmaf(live * scale_from_bits<0>(sb[s][p]), dot_chunk32(q[s][p], xv), acc[p]);
        }
#pragma unroll
        for (int p = 0; p < R; p++) acc[p] = wave_sum(acc[p]);
        if (lane == 0) {
#pragma unroll
            for (int p = 0; p < R; p++) {
                const uint32_t lr = lrow0 + (uint32_t)p;
                if (lr < a.n) attn_store_tagged(yt + lr, acc[p], tag);
            }
        }
    }
};

template <int HD, int GT, bool TAG, int NS, int R, int WREF>
RFP4_DEV void qkva_body(const QkvaArgs &p)
{
    const uint32_t b = blockIdx.x;
    const bool tile = b < p.n_tiles;
    QkvTile<NS, R, WREF> t;
    if (tile) t.issue(p.g, b);
    // the position only now: its scalar load would otherwise be waited for
    // (with the kernel arguments) before the tile's first vector load
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t tag = (uint32_t)(*p.a.pos_ptr + 1); // the step's sequence length
    AttnSplit<HD, uint16_t, GT, false, TAG, true> u;
    const uint32_t ncol = p.a.n_kv_heads * p.a.head_split;
    const bool attn = b < p.n_attn && u.issue(p.a, b % ncol, b / ncol, 0u, tag);
    if (tile) t.finish(p.g, p.yt, tag);
    if (!attn) return;
    u.load_q_tagged(p.a, tag);
    u.finish(p.a);
}
