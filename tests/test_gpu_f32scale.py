"""The reference engine's own numerics on the GPU: E2M1 weights with f32
per-32 scales (llama_run/src/main.rs:334-376, llama_decode/src/main.rs:
307-325), f32 K/V caches, and the llama_decode random-weight harness
(llama_decode/src/main.rs:356-492) replayed token for token against the
oracle's restatement of it."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

FP4 = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6], np.float64)

SMALL = dict(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=1024,
             theta=10000.0, eps=1e-5, max_seq=64)
# llama_decode/src/main.rs:289-298 (the "Llama-1B" harness), SEQ_MAX = P + WARM + GEN + 8 (:357-360)
HARNESS = dict(dim=2048, n_layers=16, n_heads=32, n_kv_heads=8, head_dim=64, ffn=8192, vocab=128256,
               theta=500000.0, eps=1e-5, max_seq=512 + 4 + 32 + 8)


def _engine(rf, cfg, seed, scale_format, kv_format):
    c = {k: v for k, v in cfg.items() if k != "max_seq"}
    return rf.Engine(rf.model_config(max_seq=cfg["max_seq"], scale_format=scale_format, kv_format=kv_format, **c),
                     seed)


def _oracle(orc, cfg, seed, scale_format, kv_format):
    return orc.Model(dict(cfg, scale_format=scale_format, kv_format=kv_format), seed)


def _dev(rf, a, s):
    return rf.DeviceBuffer.from_host(np.ascontiguousarray(a), s)


def _f32_matrix(orc, n, k, seed):
    """mk_fp4-style operands: uniform packed words, scales 0.25 + (r % 8) / 32."""
    words, st = orc.xorshift32(seed, n * k // 8)
    r, st = orc.xorshift32(st, n * k // 32)
    scales = np.float32(0.25) + (r % 8).astype(np.float32) * np.float32(0.03125)
    return words, scales


def _deq64(orc, words, scales, n, k):
    c = orc.unpack(words.view(np.uint8)).reshape(n, k)
    v = np.where(c & 8, -1.0, 1.0) * FP4[c & 7]
    return v * np.repeat(scales.astype(np.float64).reshape(n, k // 32), 32, axis=1)


@pytest.mark.parametrize("epi", ["store", "resid", "argmax", "swiglu"])
@pytest.mark.parametrize("n,k", [(67, 96), (300, 2048), (130, 4096), (64, 14336), (70000, 64)])
@pytest.mark.parametrize("norm", [False, True])
def test_gemv_f32scale_epilogues(rf, orc, stream, epi, n, k, norm):
    """Every f32-scale GEMV variant the planner picks (store with 8-wave and
    8-row workgroups, residual, argmax, SwiGLU; slice loop and up-front
    slices), with and without the fused RMSNorm, against the float64
    product: |y - y64| <= 1e-5 sum|w x| per row."""
    if epi == "swiglu" and n == 70000:
        pytest.skip("SwiGLU has no wide-matrix variant")
    rows = 2 * n if epi == "swiglu" else n
    words, scales = _f32_matrix(orc, rows, k, seed=n * 7 + k)
    rng = np.random.default_rng(n + k)
    x = rng.standard_normal(k).astype(np.float32)
    w16 = (1 + 0.02 * rng.standard_normal(k)).astype(np.float16) if norm else None
    h = orc.rmsnorm(x, w16.astype(np.float32), 1e-5) if norm else x
    W = _deq64(orc, words, scales, rows, k)
    y64 = W @ h.astype(np.float64)
    absy = np.abs(W) @ np.abs(h.astype(np.float64))
    base = np.linspace(-1, 1, n).astype(np.float32)
    dy = _dev(rf, base if epi == "resid" else np.zeros(n, np.float32), stream)
    ws = rf.DeviceBuffer(rf.mx4_gemv_argmax_workspace(n)) if epi == "argmax" else None
    best = rf.DeviceBuffer.zeroed(1, np.uint32, stream) if epi == "argmax" else None
    e = {"store": 0, "resid": 1, "swiglu": 2, "argmax": 3}[epi]
    # the device buffers stay referenced until the result is read back
    dw, ds, dx = _dev(rf, words, stream), _dev(rf, scales, stream), _dev(rf, x, stream)
    dn = _dev(rf, w16.view(np.uint16), stream) if norm else None
    rf.check(rf.load().rfp4_debug_gemv_fused(
        stream.h, e, rf.SCALE_F32, n, k, n if epi == "swiglu" else 0, dw.ptr, ds.ptr, dx.ptr, dn.ptr if norm else None,
        1e-5, dy.ptr, ws.ptr if ws else None, best.ptr if best else None))
    got = dy.to_host(n, np.float32, stream).astype(np.float64)
    # the fused norm's rms can differ from the oracle's in the last place: normwise bound
    tol = 1e-5 * absy + 1e-30
    if epi in ("store", "argmax"):
        assert np.all(np.abs(got - y64[:n]) <= tol[:n])
    elif epi == "resid":
        assert np.all(np.abs(got - (y64 + base)) <= tol + 1e-7 * np.abs(base))
    else:
        g, u = y64[:n], y64[n:]
        silu = g / (1 + np.exp(-np.clip(g, -80, 80)))
        bound = 1.1 * tol[:n] * np.abs(u) + np.abs(silu) * tol[n:] + 1e-6 * np.abs(silu * u) + 1e-30
        assert np.all(np.abs(got - silu * u) <= bound)
    if best is not None:
        assert int(best.to_host(1, np.uint32, stream)[0]) == orc.argmax(got.astype(np.float32))


def test_fp4_gemv_dropin_matches_reference_loop(rf, orc, stream):
    """The drop-in fp4_gemv on the reference harness's own data
    (fp4_gemv/src/main.rs:101-128: seed 0x12345678, scales 0.5 + (r % 8)
    * 0.25, x = ((r % 17) - 8) * 0.1, 4096 x 4096) against the oracle's
    restatement of its CPU loop (:130-143), by the reference's own gate
    |d| / max(|ref|, 1e-3) <= 1e-2 on every row."""
    n = k = 4096
    st = 0x12345678
    codes_r, st = orc.xorshift32(st, n * k)
    codes = (codes_r & 0xF).astype(np.uint8)
    words = orc.pack(codes).view(np.uint32)
    r, st = orc.xorshift32(st, n * k // 32)
    scales = np.float32(0.5) + (r % 8).astype(np.float32) * np.float32(0.25)
    r, st = orc.xorshift32(st, k)
    x = ((r % 17).astype(np.float32) - np.float32(8.0)) * np.float32(0.1)
    dy = rf.DeviceBuffer.zeroed(n, np.float32, stream)
    dw, ds, dx = _dev(rf, words, stream), _dev(rf, scales, stream), _dev(rf, x, stream)
    rf.fp4_gemv(stream, n, k, dw, ds, dx, dy)
    got = dy.to_host(n, np.float32, stream)
    ref = orc.gemv_f32scale(n, k, words, scales, x)
    rel = np.abs(got.astype(np.float64) - ref) / np.maximum(np.abs(ref), 1e-3)
    assert (rel > 1e-2).sum() == 0, rel.max()


def test_f32_engine_weights_are_mk_fp4(rf, orc):
    """llama_engine_create with f32 scales holds the harness's weights byte
    for byte (the oracle restates mk_fp4's order; pinned on the CPU)."""
    seed = 0xDEADBEEF
    eng = _engine(rf, SMALL, seed, 1, 1)
    ref = _oracle(orc, SMALL, seed, 1, 1)
    for layer in range(SMALL["n_layers"]):
        for p in range(7):
            c, s = eng.weight_host(layer, p)
            np.testing.assert_array_equal(c, ref.codes(layer, p))
            np.testing.assert_array_equal(s, ref.scales(layer, p))
    c, s = eng.weight_host(-1, 0)
    np.testing.assert_array_equal(c, ref.codes(-1, 0))
    np.testing.assert_array_equal(s, ref.scales(-1, 0))
    eng.close()
    ref.close()


@pytest.mark.parametrize("scale_format,kv_format", [(1, 0), (1, 1), (0, 1)])
def test_format_engines_tokens_match_oracle(rf, orc, scale_format, kv_format):
    """Token-driven greedy decode (llama_run/src/main.rs:544-570) with f32
    scales and/or f32 caches: tokens identical to the oracle; the written
    K/V positions within one rounding of the oracle's."""
    seed = 0x5EED0
    eng = _engine(rf, SMALL, seed, scale_format, kv_format)
    ref = _oracle(orc, SMALL, seed, scale_format, kv_format)
    prompt = [1, 7, 42, 99, 5]
    gpu = eng.generate(prompt, 0, 24)
    cpu, margins = ref.generate(prompt, 0, 24)
    assert list(gpu) == list(cpu), f"gpu {list(gpu)}\ncpu {list(cpu)}\nmargins {margins}"
    hd, nkv, npos = SMALL["head_dim"], SMALL["n_kv_heads"], len(prompt) + 24 - 1
    for layer in range(SMALL["n_layers"]):
        k, _ = eng.kv_host(layer)
        stride = k.size // (nkv * hd)
        kg = k.reshape(nkv, stride, hd)[:, :npos]
        kr = ref.kcache(layer).reshape(nkv, SMALL["max_seq"], hd)[:, :npos]
        if kv_format == 0:
            kg, kr = kg.view(np.float16).astype(np.float32), kr.view(np.float16).astype(np.float32)
        assert kg.dtype == np.float32
        assert np.max(np.abs(kg - kr)) <= 2e-3 * max(1.0, np.abs(kr).max())
    eng.close()
    ref.close()


def _harness_replay(rf, orc, cfg, seed, ctx, steps):
    eng = _engine(rf, cfg, seed, 1, 1)
    eng.begin_harness(ctx, steps + 1)
    eng.run_steps(steps)
    gpu = eng.read_ids(steps + 1)[1:]
    ref = _oracle(orc, cfg, seed, 1, 1)
    ref.harness_begin(ctx)
    cpu, margins = [], []
    for i in range(steps):
        t, lg = ref.step_noembed(ctx + i, want_logits=True)
        srt = np.sort(lg)
        cpu.append(t)
        margins.append(float(srt[-1] - srt[-2]))
    return eng, ref, list(gpu), cpu, margins


def test_harness_small_and_mode_switch(rf, orc):
    """The harness steps on a small model (context 20, 12 steps) equal the
    oracle's; then the same engine decodes tokens normally (the embedding
    step graphs are captured again) and matches the oracle's generate."""
    eng, ref, gpu, cpu, margins = _harness_replay(rf, orc, SMALL, 0xDEADBEEF, 20, 12)
    assert gpu == cpu, f"gpu {gpu}\ncpu {cpu}\nmargins {margins}"
    ref.close()
    ref = _oracle(orc, SMALL, 0xDEADBEEF, 1, 1)
    out = eng.generate([3, 4, 5], 0, 8)
    exp, _ = ref.generate([3, 4, 5], 0, 8)
    assert list(out) == list(exp)
    eng.close()
    ref.close()


def test_llama_decode_harness_replay(rf, orc):
    """The reference's llama_decode run itself: Llama-3.2-1B shape, mk_fp4
    weights from seed 0xdeadbeef with f32 scales, f32 K/V pre-filled with
    0.01 to P = 512, WARM + GEN = 4 + 32 decode steps at positions 512..547
    with x carried over (llama_decode/src/main.rs:356-492).  Every step's
    argmax identical to the oracle's restatement."""
    eng, ref, gpu, cpu, margins = _harness_replay(rf, orc, HARNESS, 0xDEADBEEF, 512, 36)
    print(f"harness tokens {gpu}; min top-2 margin {min(margins):.3e}")
    assert gpu == cpu, f"gpu {gpu}\ncpu {cpu}\nmargins {margins}"
    logits = eng.logits()
    assert np.all(np.isfinite(logits))  # the reference's own pass condition (:493-505)
    eng.close()
    ref.close()


def test_engine_variants_fixed_at_creation(rf, orc):
    """GEMV overrides set after creation do not change the engine's launches:
    an engine created with every GEMV forced to 4 rows per wave (the LM
    head's grid of argmax keys half the automatic one) decodes with that plan
    after the override is lifted, and one created without overrides ignores
    a later override.  Tokens identical to the oracle in both cases."""
    seed = 0x0F1
    ref = orc.Model(SMALL, seed)
    exp, _ = ref.generate([8, 9, 10], 0, 10)
    lib = rf.load()
    rf.check(lib.rfp4_debug_gemv_variant(4, 0))
    try:
        a = _engine(rf, SMALL, seed, 0, 0)
    finally:
        rf.check(lib.rfp4_debug_gemv_variant(0, -1))
    assert list(a.generate([8, 9, 10], 0, 10)) == list(exp)
    a.close()
    b = _engine(rf, SMALL, seed, 0, 0)
    rf.check(lib.rfp4_debug_gemv_variant(4, 0))
    try:
        assert list(b.generate([8, 9, 10], 0, 10)) == list(exp)
    finally:
        rf.check(lib.rfp4_debug_gemv_variant(0, -1))
    b.close()
    ref.close()
