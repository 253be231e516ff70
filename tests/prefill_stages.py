"""Stage-by-stage check of the engine's batched prefill on identical inputs.

The engine's prefill (llama_engine_prefill) is stopped after every stage of
every layer (rfp4_debug_prefill_stop); each stage's output is compared with
the oracle's restatement of that stage applied to the GPU's own inputs of
the stage, so a boundary decision in an earlier stage cannot hide or excuse
a later one, and every position of every layer is held to a bar:

- residual adds: bit-exact f32 (x + y);
- RMSNorm + MXFP4 rows and SwiGLU + MXFP4 rows: every E8M0 scale and E2M1
  code is the OCP round-to-nearest-even of the exact (float64) value of the
  stage on the GPU's inputs; where that exact value lies within REL_QUANT of a
  rounding boundary (a scale's power of two, or the midpoint of two codes)
  either neighbour is accepted, since f32 arithmetic in another order may
  land on either side;
- the MXFP4 GEMMs (q|k|v, o, gate|up, down): every element within
  1e-5 * sum_k |a_k w_k| of the exact float64 contraction of the GPU's
  MXFP4 activation rows with the weights;
- RoPE of q and k, the fp16 K/V append: bit-exact against the oracle's rope
  (llama_run/src/main.rs:75-84) and fp16 RNE;
- causal attention: row r against the oracle's attn_decode at
  seq = pos0 + r + 1 over the GPU's caches, the reference harness's 1e-4
  (llama_attn_decode/src/main.rs:203-204);
- MXFP4 of the attention rows: bit-exact against the oracle's quantizer;
- after the last layer: x + down bit-exact, and the logits of the last row
  (final RMSNorm fused into the LM-head GEMV) within 1e-5 * sum |w x| of the
  exact float64 GEMV of the GPU's final x.
"""
import numpy as np

E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0])
# |t| decision boundaries between adjacent E2M1 magnitudes 0, 0.5, 1, 1.5, 2, 3, 4, 6
_MAGS = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])
_BOUNDS = (_MAGS[1:] + _MAGS[:-1]) / 2
REL_QUANT = 1e-5
GEMM_REL = 1e-5


def unpack_codes(packed, rows, k):
    p = np.asarray(packed, np.uint8).reshape(rows, k // 2)
    out = np.empty((rows, k), np.uint8)
    out[:, 0::2] = p & 15
    out[:, 1::2] = p >> 4
    return out


# byte -> (value of the low nibble, value of the high nibble)
_PAIR = np.stack([E2M1[np.arange(256) & 15], E2M1[np.arange(256) >> 4]], axis=1)


def dequant(packed, scales, rows, k):
    """MXFP4 rows (codes low nibble first, E8M0 per 32) -> float64."""
    v = _PAIR[np.asarray(packed, np.uint8).reshape(rows, k // 2)].reshape(rows, k // 32, 32)
    e = np.asarray(scales, np.uint8).reshape(rows, k // 32, 1).astype(np.float64)
    v *= np.where(e == 255, np.nan, np.exp2(e - 127.0))
    return v.reshape(rows, k)


def rne_mag(t):
    """Round-to-nearest-even E2M1 magnitude of |t| (saturating at 6)."""
    a = np.abs(t)
    idx = np.searchsorted(_BOUNDS, a, side="left")       # a < bound[i] -> index i
    ties = np.isin(a, _BOUNDS)
    # at a tie, take the even code: codes 0..7 have mantissa bit = code & 1
    up = np.searchsorted(_BOUNDS, a, side="right")
    idx = np.where(ties & (idx % 2 == 1), up, idx)
    return _MAGS[np.minimum(idx, 7)]


def check_quant(codes, scales, exact, rows, k, what):
    """GPU MXFP4 rows against the exact values they quantize (OCP rules)."""
    exact = np.asarray(exact, np.float64).reshape(rows, k)
    blocks = exact.reshape(rows, k // 32, 32)
    amax = np.abs(blocks).max(axis=2)
    e = np.asarray(scales, np.uint8).reshape(rows, k // 32).astype(np.int64)
    with np.errstate(divide="ignore"):
        lg = np.log2(np.where(amax > 0, amax, 1.0))
    want = np.where(amax > 0, np.floor(lg).astype(np.int64) - 2 + 127, 0)
    near_pow2 = np.abs(amax / np.exp2(np.round(lg)) - 1.0) <= REL_QUANT
    ok_scale = (e == want) | (near_pow2 & (np.abs(e - want) == 1))
    bad = np.argwhere(~ok_scale)
    assert len(bad) == 0, (f"{what}: {len(bad)} block scales off, first (row, block) {bad[0].tolist()} "
                           f"gpu {e[tuple(bad[0])]} want {want[tuple(bad[0])]} amax {amax[tuple(bad[0])]:.9g}")
    t = blocks / np.exp2(e[:, :, None] - 127.0)
    g = E2M1[unpack_codes(codes, rows, k)].reshape(rows, k // 32, 32)
    r = np.copysign(rne_mag(t), t)
    diff = (np.abs(g) != np.abs(r)) | ((g != 0) & (np.sign(g) != np.sign(t)))
    if diff.any():
        # accepted only next to a decision boundary between the two magnitudes
        lo = np.minimum(np.abs(g), np.abs(r))
        hi = np.maximum(np.abs(g), np.abs(r))
        adjacent = np.searchsorted(_MAGS, hi) - np.searchsorted(_MAGS, lo) == 1
        b = (lo + hi) / 2
        near = np.abs(np.abs(t) - b) <= REL_QUANT * b
        signs = (g == 0) | (np.sign(g) == np.sign(t))
        bad = diff & ~(adjacent & near & signs)
        idx = np.argwhere(bad)
        assert len(idx) == 0, (f"{what}: {len(idx)} codes off, first (row, block, i) {idx[0].tolist()} "
                               f"gpu {g[tuple(idx[0])]} t {t[tuple(idx[0])]:.9g}")


def check_gemm(c, a_codes, a_scales, w_parts, m, n, k, what, chunk=4096):
    """c [m][n] against the exact contraction of MXFP4 rows a with the weight
    rows stacked from w_parts [(codes, scales, rows)], dequantized chunk by
    chunk; every element within GEMM_REL * sum_k |a_k w_k|."""
    a = dequant(a_codes, a_scales, m, k)
    aa = np.abs(a)
    c = np.asarray(c, np.float64).reshape(m, n)
    col = 0
    for codes, scales, rows in w_parts:
        codes = np.asarray(codes, np.uint8).reshape(rows, k // 2)
        scales = np.asarray(scales, np.uint8).reshape(rows, k // 32)
        for r0 in range(0, rows, chunk):
            r1 = min(rows, r0 + chunk)
            w = dequant(codes[r0:r1], scales[r0:r1], r1 - r0, k)
            ref = a @ w.T
            bound = GEMM_REL * (aa @ np.abs(w).T) + 1e-30
            err = np.abs(c[:, col + r0:col + r1] - ref)
            bad = np.argwhere(err > bound)
            assert len(bad) == 0, (f"{what}: {len(bad)} elements off in columns {col + r0}..{col + r1}, first "
                                   f"{bad[0].tolist()} err/sum|aw| {(err / bound * GEMM_REL)[tuple(bad[0])]:.3e}")
        col += rows
    assert col == n, f"{what}: weight rows {col} != {n}"


def assert_attn_close(got, ref, what):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    bound = 1e-4 * np.maximum(np.abs(ref), 1e-3) + 1e-6 * np.abs(ref).max()
    bad = np.argwhere(err > bound)
    assert len(bad) == 0, f"{what}: {len(bad)} outputs off, first {bad[0].tolist()}"


def _norm_exact(x, w16, eps):
    """Exact (float64) x * rms * w of f32 rows x and fp16 weights, rms =
    1 / sqrt(mean(x^2) + eps) (llama_rmsnorm/src/main.rs:75-77)."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w16, np.uint16).view(np.float16).astype(np.float64)
    rms = 1.0 / np.sqrt((x * x).mean(axis=-1, keepdims=True) + float(np.float32(eps)))
    return x * rms * w


def _silu_exact(g):
    g = np.asarray(g, np.float64)
    return g / (1.0 + np.exp(-g))


class _Weights:
    """The oracle's MXFP4 weights of one layer, as (codes, scales, rows) parts
    stacked in the order the engine launches them (q|k|v, gate|up)."""

    def __init__(self, ref, cfg, layer):
        dim, ffn = cfg["dim"], cfg["ffn"]
        qd, kvd = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
        f = lambda p, n: (ref.codes(layer, p), ref.scales(layer, p), n)
        self.qkv = [f(0, qd), f(1, kvd), f(2, kvd)]
        self.o = [f(3, dim)]
        self.gu = [f(4, ffn), f(5, ffn)]
        self.d = [f(6, dim)]


def check_prefill_stages(rf, orc, eng, ref, cfg, prompt, pos0, log=print):
    """Run the staged comparison of one llama_engine_prefill call (prompt at
    pos0; the caches below pos0 as the caller left them).  ref is the oracle
    Model built from the same seed (its weights and norms)."""
    n = len(prompt)
    L, dim, ffn = cfg["n_layers"], cfg["dim"], cfg["ffn"]
    nh, nkv, hd = cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"]
    qd, kvd = nh * hd, nkv * hd
    nqkv = qd + 2 * kvd
    eps = cfg["eps"]
    half = hd // 2
    cos_t, sin_t = orc.rope_table(pos0 + n, hd, cfg["theta"])

    def stop(after):
        eng.prefill_stop(prompt, pos0, after)

    def buf(name, cols, dtype=np.float32):
        return eng.prefill_buffer(name, (n, cols), dtype)

    def qrows(cols):
        return buf("codes", cols // 2, np.uint8), buf("scales", cols // 32, np.uint8)

    stop(-1)
    x = buf("x", dim)
    down = None
    for l in range(L):
        W = _Weights(ref, cfg, l)
        # 0: x (+ previous down) -> RMSNorm -> MXFP4
        stop(10 * l + 0)
        x_new = buf("x", dim)
        want_x = x if down is None else (x + down).astype(np.float32)
        np.testing.assert_array_equal(x_new, want_x, err_msg=f"layer {l} residual before the attention norm")
        x = x_new
        c0, s0 = qrows(dim)
        check_quant(c0, s0, _norm_exact(x, ref.norm(l, 0), eps), n, dim, f"layer {l} attention norm rows")
        # 1: q|k|v GEMM
        stop(10 * l + 1)
        qkv = buf("c", nqkv)
        check_gemm(qkv, c0, s0, W.qkv, n, nqkv, dim, f"layer {l} q|k|v GEMM")
        # 2: RoPE of q and k, fp16 K/V at pos0 + r
        stop(10 * l + 2)
        qkv_r = buf("c", nqkv)
        kg, vg = eng.kv_host(l)
        alloc = kg.size // (nkv * hd)
        kg3, vg3 = kg.reshape(nkv, alloc, hd), vg.reshape(nkv, alloc, hd)
        q_want = np.empty((n, qd), np.float32)
        k_rot = np.empty((n, kvd), np.float32)
        for r in range(n):
            pos = pos0 + r
            cp, sp = cos_t[pos * half:(pos + 1) * half], sin_t[pos * half:(pos + 1) * half]
            q_want[r] = orc.rope(qkv[r, :qd], nh, hd, cp, sp)
            k_rot[r] = orc.rope(qkv[r, qd:qd + kvd], nkv, hd, cp, sp)
        np.testing.assert_array_equal(qkv_r[:, :qd], q_want, err_msg=f"layer {l} rotated q")
        k_want = orc.f32_to_f16(k_rot).reshape(n, nkv, hd).transpose(1, 0, 2)
        v_want = orc.f32_to_f16(qkv[:, qd + kvd:]).reshape(n, nkv, hd).transpose(1, 0, 2)
        np.testing.assert_array_equal(kg3[:, pos0:pos0 + n], k_want, err_msg=f"layer {l} fp16 k rows")
        np.testing.assert_array_equal(vg3[:, pos0:pos0 + n], v_want, err_msg=f"layer {l} fp16 v rows")
        # 3: causal attention over the GPU's caches
        stop(10 * l + 3)
        att = buf("a", qd)
        oref = np.stack([orc.attn_decode(nh, nkv, hd, pos0 + r + 1, np.ascontiguousarray(qkv_r[r, :qd]), kg, vg,
                                         hd, alloc * hd) for r in range(n)])
        assert_attn_close(att, oref, f"layer {l} attention")
        # 4: MXFP4 of the attention rows (deterministic given the f32 rows)
        stop(10 * l + 4)
        c4, s4 = qrows(qd)
        oc, os_ = orc.quant_mx(att)
        np.testing.assert_array_equal(c4.reshape(-1), oc, err_msg=f"layer {l} attention rows codes")
        np.testing.assert_array_equal(s4.reshape(-1), os_, err_msg=f"layer {l} attention rows scales")
        # 5: o GEMM
        stop(10 * l + 5)
        o = buf("c", dim)
        check_gemm(o, c4, s4, W.o, n, dim, qd, f"layer {l} o GEMM")
        # 6: x + o -> RMSNorm -> MXFP4
        stop(10 * l + 6)
        x_new = buf("x", dim)
        np.testing.assert_array_equal(x_new, (x + o).astype(np.float32), err_msg=f"layer {l} residual after o")
        x = x_new
        c6, s6 = qrows(dim)
        check_quant(c6, s6, _norm_exact(x, ref.norm(l, 1), eps), n, dim, f"layer {l} FFN norm rows")
        # 7: gate|up GEMM
        stop(10 * l + 7)
        gu = buf("c", 2 * ffn)
        check_gemm(gu, c6, s6, W.gu, n, 2 * ffn, dim, f"layer {l} gate|up GEMM")
        # 8: SwiGLU -> MXFP4
        stop(10 * l + 8)
        c8, s8 = qrows(ffn)
        h = _silu_exact(gu[:, :ffn]) * np.asarray(gu[:, ffn:], np.float64)
        check_quant(c8, s8, h, n, ffn, f"layer {l} SwiGLU rows")
        # 9: down GEMM
        stop(10 * l + 9)
        down = buf("c", dim)
        check_gemm(down, c8, s8, W.d, n, dim, ffn, f"layer {l} down GEMM")
        log(f"  layer {l}: every stage on identical inputs within its bar", flush=True)
    # full run: x + down of the last layer, LM head of the last row
    tok = eng.prefill(prompt, pos0)
    x_fin = buf("x", dim)
    np.testing.assert_array_equal(x_fin, (x + down).astype(np.float32), err_msg="residual after the last layer")
    hn = _norm_exact(x_fin[-1], ref.norm(-1, 0), eps)
    lg = eng.logits()
    V = cfg["vocab"]
    lc = np.asarray(ref.codes(-1, 0), np.uint8).reshape(V, dim // 2)
    ls = np.asarray(ref.scales(-1, 0), np.uint8).reshape(V, dim // 32)
    for r0 in range(0, V, 8192):
        r1 = min(V, r0 + 8192)
        wl = dequant(lc[r0:r1], ls[r0:r1], r1 - r0, dim)
        y64 = wl @ hn
        bound = GEMM_REL * (np.abs(wl) @ np.abs(hn)) + 1e-30
        bad = np.nonzero(np.abs(lg[r0:r1] - y64) > bound)[0]
        assert len(bad) == 0, f"logits: {len(bad)} off, first {r0 + bad[0]}"
    assert tok == int(np.argmax(lg)), "next token is not the argmax of the logits"
    return tok
