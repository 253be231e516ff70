"""Pins the CPU oracle (oracle/oracle.c) against facts that do not come from
its own formulas: the reference's literal tables and known answers, published
test vectors, closed forms, invariants, and independent brute-force
restatements in numpy (different code, float64).  CPU only."""
import math

import numpy as np
import pytest

FP4_TABLE = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]  # fp4_gemv/src/main.rs:130


# ---------------------------------------------------------------- RNG
def test_xorshift32_marsaglia_known_answer(orc):
    """Marsaglia (2003), 'Xorshift RNGs': seed 2463534242 -> 723471715."""
    out, _ = orc.xorshift32(2463534242, 1)
    assert int(out[0]) == 723471715


def test_mix64_splitmix64_test_vector(orc):
    """SplitMix64 (Steele, Lea, Flood 2014) from state 1234567 (published
    reference sequence); stream 0 of the counter form is that sequence."""
    expect = [6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431,
              16408922859458223821]
    assert [orc.mix64(1234567, 0, i) for i in range(5)] == expect


def test_ih4_normal_moments(orc):
    coef = orc.lib().orc_ih4_coef(1.0)
    z = np.array([orc.lib().orc_ih4_normal(orc.mix64(7, 1, i), coef) for i in range(200000)])
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01
    assert np.abs(z).max() <= 2 * 65535 / 37837.22723720648 + 1e-6  # Irwin-Hall(4) support


# ---------------------------------------------------------------- codecs
def test_e2m1_both_reference_forms(orc):
    """The table form (fp4_gemv/src/main.rs:130-134) and the arithmetic form
    (llama_run/src/main.rs:21-32) agree with the literal table on all codes."""
    for c in range(16):
        expect = -FP4_TABLE[c & 7] if c & 8 else FP4_TABLE[c & 7]
        assert orc.lib().orc_e2m1_decode(c) == expect
        assert orc.lib().orc_e2m1_decode_arith(c) == expect
    assert math.copysign(1.0, orc.lib().orc_e2m1_decode(8)) == -1.0  # code 8 is -0


def test_e8m0_decode_all_bytes(orc):
    for b in range(255):
        assert orc.lib().orc_e8m0_decode(b) == math.ldexp(1.0, b - 127)
    assert math.isnan(orc.lib().orc_e8m0_decode(255))


def test_e8m0_encode_trackb(orc):
    """ue8m0 = 127 + log2(s) for powers of two (trackb/fp4_scale_test.cu:12)."""
    for e in range(-127, 128):
        assert orc.lib().orc_e8m0_encode_pow2(math.ldexp(1.0, e)) == 127 + e
    assert [orc.lib().orc_e8m0_encode_pow2(s) for s in (0.5, 1, 2, 4)] == [126, 127, 128, 129]


def test_packing_low_nibble_first(orc):
    """8 codes per u32, low nibble = lowest k (fp4_gemv/src/main.rs:113-120):
    codes 0..7 pack to the little-endian word 0x76543210."""
    packed = orc.pack(np.arange(8, dtype=np.uint8))
    assert packed.view(np.uint32)[0] == 0x76543210
    rng = np.random.default_rng(0)
    c = rng.integers(0, 16, 4096).astype(np.uint8)
    np.testing.assert_array_equal(orc.unpack(orc.pack(c)), c)


def test_f16_conversions_exhaustive(orc):
    """half_to_f32 (llama_run/src/main.rs:591-614) on all 65536 patterns and
    f32 -> f16 RNE against numpy's IEEE conversion."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([orc.lib().orc_f16_to_f32(int(v)) for v in h], np.float32)
    finite = np.isfinite(ref)
    np.testing.assert_array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(ref)]))
    rng = np.random.default_rng(1)
    f = np.concatenate([rng.standard_normal(20000) * 10.0 ** rng.integers(-9, 6, 20000),
                        [65504, 65519.99, 65520, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, 0.0, -0.0, 1e-10]]).astype(np.float32)
    got = np.array([orc.lib().orc_f32_to_f16(float(v)) for v in f], np.uint16)
    np.testing.assert_array_equal(got, f.astype(np.float16).view(np.uint16))


def test_bf16_conversions(orc):
    rng = np.random.default_rng(2)
    f = (rng.standard_normal(5000) * 10.0 ** rng.integers(-30, 30, 5000)).astype(np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    rne = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    got = np.array([orc.lib().orc_f32_to_bf16(float(v)) for v in f], np.uint16)
    np.testing.assert_array_equal(got, rne)
    for b in (0x3F80, 0xC000, 0x0001, 0x7F7F):
        assert orc.lib().orc_bf16_to_f32(b) == np.array([b << 16], np.uint32).view(np.float32)[0]


# ---------------------------------------------------------------- quantizers
def _brute_rne(v):
    """Nearest E2M1 value, ties to the even code, saturating: brute force."""
    a = min(abs(v), 6.0)
    d = [abs(a - m) for m in FP4_TABLE]
    best = min(d)
    cands = [i for i, x in enumerate(d) if x == best]
    c = cands[0] if len(cands) == 1 else [i for i in cands if i % 2 == 0][0]
    return c | (8 if math.copysign(1.0, v) < 0 else 0)


def test_e2m1_rne_against_brute_force(orc):
    grid = np.concatenate([np.arange(-8, 8, 1 / 64.0), [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, -0.25, 7.0, 100.0, -0.0]])
    for v in grid.astype(np.float32):
        assert orc.lib().orc_e2m1_rne(float(v)) == _brute_rne(float(v)), v


def test_quant_mx_ocp_rules(orc):
    """OCP MX: shared exponent floor(log2(amax)) - 2, elements RNE on the
    scaled grid, all-zero block -> byte 0; decoding is within half an ulp."""
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((40, 64)) * 10.0 ** rng.uniform(-6, 6, (40, 1))).astype(np.float32)
    w[0, :32] = 0.0
    w[1, :32] = 0.0
    w[1, 5] = 6.0  # exactly representable at scale 1
    packed, scales = orc.quant_mx(w)
    codes = orc.unpack(packed).reshape(40, 64)
    sc = scales.reshape(40, 2)
    assert sc[0, 0] == 0 and not codes[0, :32].any()
    assert sc[1, 0] == 127 and codes[1, 5] == 7
    for r in range(40):
        for b in range(2):
            blk = w[r, 32 * b:32 * b + 32].astype(np.float64)
            amax = np.abs(blk).max()
            if amax == 0:
                continue
            e = math.floor(math.log2(amax)) - 2
            assert sc[r, b] == 127 + e
            for i in range(32):
                assert codes[r, 32 * b + i] == _brute_rne(blk[i] / 2.0 ** e)


def test_quant_fp4_absmax_reference_rules(orc):
    """quant_fp4 (llama_run/src/main.rs:334-376): scale absmax/6 (1.0 for a zero
    block), nearest level by strict '<' linear search -- ties to the LOWER
    code, i.e. numpy argmin's first minimum -- and sign iff v < 0."""
    rng = np.random.default_rng(4)
    w = rng.standard_normal((8, 64)).astype(np.float32)
    w[2, :32] = 0.0
    w[3, 32:] = np.float32(-0.0)
    w[4, :32] = np.array([6.0] + [0.25 * 1.0, 0.75, 1.25] * 10 + [0.0], np.float32)  # ties at scale 1
    packed, scales = orc.quant_fp4_absmax(w)
    codes = orc.unpack(packed).reshape(8, 64)
    sc = scales.reshape(8, 2)
    assert sc[2, 0] == 1.0 and not codes[2, :32].any()
    assert not codes[3, 32:].any()  # -0.0 is not < 0
    for r in range(8):
        for b in range(2):
            blk = w[r, 32 * b:32 * b + 32]
            amax = np.float32(np.abs(blk).max())
            s = np.float32(amax / np.float32(6.0)) if amax > 0 else np.float32(1.0)
            assert sc[r, b] == s
            v = (blk / s).astype(np.float32)
            d = np.abs(np.abs(v)[:, None] - np.array(FP4_TABLE, np.float32)[None, :])
            c = np.argmin(d, axis=1) | np.where(v < 0, 8, 0)
            np.testing.assert_array_equal(codes[r, 32 * b:32 * b + 32], c)
    assert list(codes[4, 1:4]) == [0, 1, 2]  # 0.25 -> 0, 0.75 -> 0.5, 1.25 -> 1.0 (lower)


def test_synth_weight_is_quantized_normal(orc):
    """The synthetic init: ih4 normals quantized with quant_mx, byte for byte."""
    k, rows = 256, 5
    packed, scales = orc.synth_mx_weight(99, 3, 0.02, k, 7, rows)
    coef = orc.lib().orc_ih4_coef(0.02)
    w = np.array([[orc.lib().orc_ih4_normal(orc.mix64(99, 3, (7 + r) * k + i), coef) for i in range(k)]
                  for r in range(rows)], np.float32)
    p2, s2 = orc.quant_mx(w)
    np.testing.assert_array_equal(packed, p2)
    np.testing.assert_array_equal(scales, s2)


# ---------------------------------------------------------------- GEMV / GEMM / MMA tile
def _deq(orc, codes_packed, scales_e8m0, n, k):
    c = orc.unpack(codes_packed).reshape(n, k)
    sign = np.where(c & 8, -1.0, 1.0)
    mag = np.array(FP4_TABLE)[c & 7]
    s = np.ldexp(1.0, scales_e8m0.astype(np.int64) - 127).reshape(n, k // 32)
    return sign * mag * np.repeat(s, 32, axis=1)


def test_gemv_against_numpy_f64(orc):
    n, k = 96, 2048
    rng = np.random.default_rng(5)
    packed = rng.integers(0, 256, n * k // 2).astype(np.uint8)
    scales = rng.integers(121, 130, n * k // 32).astype(np.uint8)
    x = rng.standard_normal(k).astype(np.float32)
    W = _deq(orc, packed, scales, n, k)
    ref = W @ x.astype(np.float64)
    absr = np.abs(W) @ np.abs(x.astype(np.float64))
    y = orc.gemv_e8m0(n, k, packed, scales, x)
    assert np.max(np.abs(y - ref) / absr) < 1e-6
    y64, a64 = orc.gemv_e8m0_f64(n, k, packed, scales, x)
    np.testing.assert_allclose(y64, ref, rtol=1e-12, atol=1e-12 * absr.max())
    np.testing.assert_allclose(a64, absr, rtol=1e-12)


def test_gemv_closed_forms(orc):
    n, k = 4, 64
    ones = orc.pack(np.full(n * k, 2, np.uint8))  # E2M1 1.0
    sc = np.full(n * k // 32, 127 + 3, np.uint8)  # scale 8
    y = orc.gemv_e8m0(n, k, ones, sc, np.ones(k, np.float32))
    assert np.all(y == 8.0 * k)
    x = np.zeros(k, np.float32)
    x[37] = 1.0  # one-hot selects column 37 of W
    codes = np.tile(np.arange(16, dtype=np.uint8), n * k // 16)
    y = orc.gemv_e8m0(n, k, orc.pack(codes), sc, x)
    expect = 8.0 * (-FP4_TABLE[37 % 16 & 7] if (37 % 16) & 8 else FP4_TABLE[37 % 16 & 7])
    assert np.all(y == expect)


def test_gemv_reference_harness_replay(orc):
    """fp4_gemv/src/main.rs:95-175 at a reduced 512x4096 (same seed stream,
    f32 scales): the reference's 'bad' count (rel > 1e-2 against the CPU loop)
    is zero for an independent f64 evaluation."""
    N, K = 512, 4096
    st = 0x12345678
    r, st = orc.xorshift32(st, N * K)
    codes = (r & 0xF).astype(np.uint8)
    w = orc.pack(codes).view(np.uint32)
    r, st = orc.xorshift32(st, N * K // 32)
    scales = (0.5 + (r % 8).astype(np.float32) * 0.25).astype(np.float32)
    r, st = orc.xorshift32(st, K)
    x = (((r % 17).astype(np.float32) - 8.0) * 0.1).astype(np.float32)
    y = orc.gemv_f32scale(N, K, w, scales, x)
    sign = np.where(codes & 8, -1.0, 1.0)
    deq = sign * np.array(FP4_TABLE)[codes & 7] * np.repeat(scales.astype(np.float64), 32)
    ref = deq.reshape(N, K) @ x.astype(np.float64)
    rel = np.abs(y - ref) / np.maximum(np.abs(ref), 1e-3)
    assert (rel > 1e-2).sum() == 0


def _trackb_data():
    SV = [0.5, 1.0, 2.0, 4.0]
    A = np.array([[FP4_TABLE[(i * 7 + k * 3) % 8] for k in range(64)] for i in range(16)], np.float32)
    B = np.array([[FP4_TABLE[(k * 5 + j * 2) % 8] for j in range(8)] for k in range(64)], np.float32)
    SFA = np.array([[SV[(i + b) % 4] for b in range(2)] for i in range(16)], np.float32)
    SFB = np.array([[SV[(j + b * 2) % 4] for j in range(8)] for b in range(2)], np.float32)
    return A, B, SFA, SFB


def test_mma_tile_known_answers(orc):
    """trackb: all-ones -> 64.0 (fp4_mma/src/main.rs:75); the mapping and scale
    data (trackb/fp4_mapping_test.cu:38-40, fp4_scale_test.cu:34-37) against a
    float64 numpy matmul -- exact, the products are short dyadics."""
    one = np.ones((16, 64), np.float32)
    D = orc.mma_m16n8k64_ref(one, np.ones((64, 8), np.float32), np.ones((16, 2), np.float32), np.ones((2, 8), np.float32))
    assert np.all(D == 64.0)
    A, B, SFA, SFB = _trackb_data()
    D = orc.mma_m16n8k64_ref(A, B, np.ones((16, 2), np.float32), np.ones((2, 8), np.float32))
    np.testing.assert_array_equal(D, A.astype(np.float64) @ B.astype(np.float64))
    D = orc.mma_m16n8k64_ref(A, B, SFA, SFB)
    As = A.astype(np.float64) * np.repeat(SFA, 32, axis=1)
    Bs = B.astype(np.float64) * np.repeat(SFB, 32, axis=0)
    np.testing.assert_array_equal(D, As @ Bs)


def test_gemm_against_numpy(orc):
    M, N, K = 8, 24, 256
    rng = np.random.default_rng(6)
    ac = rng.integers(0, 256, M * K // 2).astype(np.uint8)
    asc = rng.integers(120, 134, M * K // 32).astype(np.uint8)
    wc = rng.integers(0, 256, N * K // 2).astype(np.uint8)
    wsc = rng.integers(120, 134, N * K // 32).astype(np.uint8)
    c, absc = orc.gemm_mx_f64(M, N, K, ac, asc, wc, wsc)
    A = _deq(orc, ac, asc, M, K)
    W = _deq(orc, wc, wsc, N, K)
    np.testing.assert_allclose(c, A @ W.T, rtol=1e-12, atol=1e-9)
    np.testing.assert_allclose(absc, np.abs(A) @ np.abs(W).T, rtol=1e-12)


# ---------------------------------------------------------------- layers
def test_rmsnorm_closed_form_and_harness(orc):
    c, d, eps = np.float32(3.0), 2048, np.float32(1e-5)
    w = np.linspace(0.5, 1.5, d).astype(np.float32)
    y = orc.rmsnorm(np.full(d, c, np.float32), w, eps)
    expect = c / np.sqrt(np.float64(c) ** 2 + eps) * w
    np.testing.assert_allclose(y, expect, rtol=2e-7)
    # llama_rmsnorm/src/main.rs:63-73 inputs, against numpy f64
    r, st = orc.xorshift32(0x9E3779B9, d)
    x = (((r % 2001).astype(np.float32) - 1000.0) / 500.0).astype(np.float32)
    r, st = orc.xorshift32(st, d)
    w = (0.5 + (r % 1000).astype(np.float32) / 1000.0).astype(np.float32)
    y = orc.rmsnorm(x, w, 1e-5)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt(np.mean(x64 * x64) + 1e-5) * w
    assert np.max(np.abs(y - ref) / np.maximum(np.abs(ref), 1e-3)) < 1e-5  # reference gate 1e-4


def test_rope_identities(orc):
    hd, theta = 64, 10000.0
    cos_t, sin_t = orc.rope_table(300, hd, theta)
    half = hd // 2
    # table against numpy's float64 formulas (1 ulp of f32 slack for libm)
    j = np.arange(half)
    ang = np.arange(300)[:, None] * (1.0 / np.power(theta, 2.0 * j / hd))[None, :]
    np.testing.assert_allclose(cos_t.reshape(300, half), np.cos(ang).astype(np.float32), rtol=0, atol=1.2e-7)
    np.testing.assert_allclose(sin_t.reshape(300, half), np.sin(ang).astype(np.float32), rtol=0, atol=1.2e-7)
    rng = np.random.default_rng(7)
    q = rng.standard_normal(4 * hd).astype(np.float32)
    # position 0 is the identity
    np.testing.assert_array_equal(orc.rope(q, 4, hd, cos_t[:half], sin_t[:half]), q)
    # each (j, j+half) pair keeps its norm
    pos = 123
    r = orc.rope(q, 4, hd, cos_t[pos * half:(pos + 1) * half], sin_t[pos * half:(pos + 1) * half]).reshape(4, hd)
    q2 = q.reshape(4, hd)
    n0 = q2[:, :half] ** 2 + q2[:, half:] ** 2
    n1 = r[:, :half].astype(np.float64) ** 2 + r[:, half:].astype(np.float64) ** 2
    np.testing.assert_allclose(n1, n0, rtol=1e-5)
    # rotate-half pairing: out[j] = x0 c - x1 s
    c0, s0 = cos_t[pos * half], sin_t[pos * half]
    assert abs(r[0, 0] - (q2[0, 0] * c0 - q2[0, half] * s0)) < 1e-6


def test_attention_closed_forms(orc):
    nh, nkv, hd, seq = 8, 2, 64, 37
    rng = np.random.default_rng(8)
    kc = rng.standard_normal(seq * nkv * hd).astype(np.float32)
    vc = rng.standard_normal(seq * nkv * hd).astype(np.float32)
    # q = 0: uniform weights -> mean of V of the head's KV group
    out = orc.attn_decode(nh, nkv, hd, seq, np.zeros(nh * hd, np.float32), kc, vc, nkv * hd, hd).reshape(nh, hd)
    V = vc.reshape(seq, nkv, hd).astype(np.float64)
    for h in range(nh):
        np.testing.assert_allclose(out[h], V[:, h // (nh // nkv)].mean(axis=0), rtol=1e-5, atol=1e-6)
    # general q against a float64 numpy softmax (llama_attn_decode/src/main.rs:150-179)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    out = orc.attn_decode(nh, nkv, hd, seq, q, kc, vc, nkv * hd, hd).reshape(nh, hd)
    K = kc.reshape(seq, nkv, hd).astype(np.float64)
    for h in range(nh):
        kvh = h // (nh // nkv)
        s = K[:, kvh] @ q.reshape(nh, hd)[h].astype(np.float64) / math.sqrt(hd)
        p = np.exp(s - s.max())
        np.testing.assert_allclose(out[h], (p / p.sum()) @ V[:, kvh], rtol=2e-5, atol=2e-6)


def test_swiglu_residual_argmax(orc):
    g = np.array([-30.0, -1.0, 0.0, 0.5, 2.0, 30.0], np.float32)
    u = np.array([1.0, 2.0, 3.0, -1.0, 0.5, 1.0], np.float32)
    np.testing.assert_allclose(orc.swiglu(g, u), g / (1 + np.exp(-g.astype(np.float64))) * u, rtol=1e-6, atol=1e-30)
    x = np.array([1.0, -2.0], np.float32)
    np.testing.assert_array_equal(orc.residual(np.array([0.5, 0.25], np.float32), x), [1.5, -1.75])
    v = np.array([1.0, 3.0, 3.0, 2.0], np.float32)
    assert orc.argmax(v) == 1  # ties -> lowest index
    assert orc.argmax(np.array([np.nan, 1.0, np.nan], np.float32)) == 1
    assert orc.argmax(np.full(5, -np.inf, np.float32)) == 0  # nothing > -1e30


def test_small_golden_fixtures_reproduce(orc):
    """The committed config-1 and config-2 fixtures are what the oracle
    computes now (a change to the oracle that moves them fails here)."""
    import importlib.util
    import os

    from conftest import GOLDEN
    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(GOLDEN, "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    fx = np.load(os.path.join(GOLDEN, "config1_gemv.npz"))
    codes, scales, x = mg.config1_inputs()
    assert mg.sha(codes) == str(fx["sha_codes"]) and mg.sha(x) == str(fx["sha_x"])
    np.testing.assert_array_equal(orc.gemv_e8m0(2048, 2048, codes, scales, x), fx["y"])
    y64, absy = orc.gemv_e8m0_f64(2048, 2048, codes, scales, x)
    np.testing.assert_array_equal(y64, fx["y64"])
    fx2 = np.load(os.path.join(GOLDEN, "config2_kernels.npz"))
    r, _ = orc.xorshift32(0x13579BDF, 32 * 64)
    q = (((r % 2001).astype(np.float32) - 1000.0) / 500.0).astype(np.float32)
    c, s = orc.rope_table(2048, 64, 10000.0)
    np.testing.assert_array_equal(orc.rope(q, 32, 64, c[2047 * 32:], s[2047 * 32:]), fx2["rope_pos2047"])
