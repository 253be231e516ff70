"""The staged prefill checker's own pins (CPU): its MXFP4 dequantizer and
rounding rule against the oracle's OCP quantizer, and planted mistakes that
it must reject (a code one step off away from a boundary, a wrong block
scale, a GEMM element off by more than the bar)."""
import numpy as np
import pytest

from prefill_stages import check_gemm, check_quant, dequant, rne_mag


def _rows(seed, rows, k):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, k)) * np.exp2(rng.integers(-6, 6, (rows, 1)))
    return x.astype(np.float32)


def test_rne_mag_ties_and_saturation():
    t = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 7.9, 100.0, 0.2, 0.3, 4.9, 5.1])
    want = np.array([0.0, 1.0, 1.0, 2.0, 2.0, 4.0, 4.0, 6.0, 6.0, 0.0, 0.5, 4.0, 6.0])
    np.testing.assert_array_equal(rne_mag(t), want)


def test_checker_accepts_the_oracle_quantizer(orc):
    x = _rows(1, 16, 512)
    codes, scales = orc.quant_mx(x)
    check_quant(codes, scales, x, 16, 512, "oracle")
    d = dequant(codes, scales, 16, 512)
    # every dequantized value is the block scale times an E2M1 value
    assert np.all(np.isfinite(d))
    assert np.max(np.abs(d - x)) <= np.max(np.abs(x)) / 4


def test_checker_rejects_a_wrong_code(orc):
    x = _rows(2, 4, 256)
    codes, scales = orc.quant_mx(x)
    blocks = x.reshape(4, 8, 32).astype(np.float64) / np.exp2(scales.reshape(4, 8, 1).astype(np.float64) - 127)
    # pick an element far from any boundary and move its code by one
    frac = np.abs(np.abs(blocks) - np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0])[:, None, None, None]).min(axis=0)
    i = int(np.argmax(frac.reshape(-1)))
    un = np.empty(codes.size * 2, np.uint8)
    un[0::2], un[1::2] = codes & 15, codes >> 4
    un[i] = (un[i] & 8) | (((un[i] & 7) + 1) % 8 if (un[i] & 7) < 7 else 6)
    bad = (un[0::2] | (un[1::2] << 4)).astype(np.uint8)
    with pytest.raises(AssertionError, match="codes off"):
        check_quant(bad, scales, x, 4, 256, "planted")


def test_checker_rejects_a_wrong_scale(orc):
    x = _rows(3, 4, 256)
    codes, scales = orc.quant_mx(x)
    s2 = scales.copy()
    s2[5] += 1
    with pytest.raises(AssertionError, match="scales off"):
        check_quant(codes, s2, x, 4, 256, "planted")


def test_checker_gemm_bar(orc):
    a = _rows(4, 8, 256)
    w = _rows(5, 24, 256)
    ac, as_ = orc.quant_mx(a)
    wc, ws = orc.quant_mx(w)
    c64, _ = orc.gemm_mx_f64(8, 24, 256, ac, as_, wc, ws)
    check_gemm(c64.astype(np.float32), ac, as_, [(wc, ws, 24)], 8, 24, 256, "f32 of the exact sum")
    check_gemm(c64, ac, as_, [(wc[:16 * 128], ws[:16 * 8], 16), (wc[16 * 128:], ws[16 * 8:], 8)], 8, 24, 256,
               "two parts, chunked", chunk=5)
    bad = c64.copy()
    bad[3, 7] *= 1 + 1e-3
    with pytest.raises(AssertionError, match="elements off"):
        check_gemm(bad, ac, as_, [(wc, ws, 24)], 8, 24, 256, "planted")
