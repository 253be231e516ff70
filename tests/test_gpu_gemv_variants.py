"""Every compiled GEMV variant (rows per wave x up-front K-slices) and the
fused RMSNorm prologue, against the oracle."""
import numpy as np
import pytest

from conftest import reference_rel_err
from test_gpu_kernels import _assert_gemv_close, _config1, _dev

pytestmark = pytest.mark.gpu

_VARIANTS = {  # epilogue -> {R: compiled NS}; mirrors kernels.hip and runtime.cpp gemv_has_ns
    "store": {1: (0, 1, 2, 3, 4, 7), 2: (0, 1, 2, 3, 4, 7), 4: (0, 1, 2, 3, 4, 7), 8: (0, 1, 2)},
    "resid": {1: (0, 1, 2, 3, 4, 7), 2: (0, 1, 2, 3, 4, 7), 4: (0, 1, 2, 3, 4, 7), 8: (0, 1, 2)},
    "argmax": {2: (0, 1, 2, 3, 4, 7), 4: (0, 1, 2, 3, 4, 7), 8: (0, 1, 2)},
    "swiglu": {1: (0, 1, 2, 3, 4, 7), 2: (0, 1, 2, 3, 4, 7), 4: (0, 1, 2, 3)},
}


def _force(rf, r, ns):
    rf.check(rf.load().rfp4_debug_gemv_variant(r, ns))


def _run_epi(rf, stream, epi, n, k, dc, ds, dx, base):
    dy = _dev(rf, base, stream)
    best = None
    if epi == "store":
        rf.mx4_gemv(stream, n, k, dc, ds, dx, dy)
    elif epi == "resid":
        rf.mx4_gemv_residual(stream, n, k, dc, ds, dx, dy)
    elif epi == "argmax":
        ws = rf.DeviceBuffer(rf.mx4_gemv_argmax_workspace(n))
        best = rf.DeviceBuffer.zeroed(1, np.uint32, stream)
        rf.mx4_gemv_argmax(stream, n, k, dc, ds, dx, dy, ws, best)
    else:
        rf.mx4_gemv_swiglu(stream, n, k, n, dc, ds, dx, dy)
    got = dy.to_host(n, np.float32, stream)
    return got, (int(best.to_host(1, np.uint32, stream)[0]) if best is not None else None)


def _activation_like(orc, n, k, codes, scales, x, epi):
    """x scaled by a power of two (W.x scales exactly) so that the SwiGLU
    gates have the magnitudes of a real activation (RMS about 3, most |g| < 10)
    instead of config 1's hundreds, where silu saturates."""
    if epi != "swiglu":
        return x
    g = orc.gemv_e8m0(n, k, codes, scales, x)[:n // 2]
    e = int(np.round(np.log2(3.0 / max(float(np.sqrt(np.mean(g.astype(np.float64) ** 2))), 1e-30))))
    return (x * np.float32(2.0 ** e)).astype(np.float32)


def _assert_gates_unsaturated(f64, n):
    g = f64[:n]
    assert np.mean(np.abs(g) < 10.0) >= 0.5, "gates mostly saturated"
    assert np.mean(np.abs(g) < 1.0) >= 0.1, "no gates in silu's curved range"


def _check_epi(orc, epi, got, best, n, full, f64, absf, base, tag):
    if epi in ("store", "argmax"):
        _assert_gemv_close(got, full[:n], f64[:n], absf[:n])
    elif epi == "resid":
        # x + W.x: the GEMV's normwise bound carries through the add
        err = np.abs(got.astype(np.float64) - (f64[:n] + base))
        assert np.all(err <= 1e-5 * (absf[:n] + np.abs(base)) + 1e-30), tag
    else:
        # silu(g)*u: |d| <= |silu'(g)| |dg| |u| + |silu(g)| |du|, |silu'| < 1.1
        g, u = f64[:n], f64[n:]
        silu = g / (1 + np.exp(-g))
        bound = 1e-5 * (1.1 * absf[:n] * np.abs(u) + np.abs(silu) * absf[n:]) + 1e-30
        assert np.all(np.abs(got - silu * u) <= bound), tag
    if best is not None:
        assert best == orc.argmax(got), tag


@pytest.mark.parametrize("epi", ["store", "resid", "argmax", "swiglu"])
@pytest.mark.parametrize("k", [96, 2048, 4096, 5632, 14336])
def test_gemv_all_variants(rf, orc, stream, epi, k):
    n = 67  # not a multiple of any workgroup row count
    codes, scales, x = _config1(orc, 2 * n, k, seed=k + len(epi))
    x = _activation_like(orc, 2 * n, k, codes, scales, x, epi)
    dc, ds, dx = _dev(rf, codes, stream), _dev(rf, scales, stream), _dev(rf, x, stream)
    full = orc.gemv_e8m0(2 * n, k, codes, scales, x)
    f64, absf = orc.gemv_e8m0_f64(2 * n, k, codes, scales, x)
    if epi == "swiglu":
        _assert_gates_unsaturated(f64, n)
    need = (k + 2047) // 2048
    base = np.linspace(-1, 1, n).astype(np.float32)
    ran = 0
    try:
        for r, nss in _VARIANTS[epi].items():
            for ns in nss:
                if ns not in (0, need):
                    continue
                _force(rf, r, ns)
                got, best = _run_epi(rf, stream, epi, n, k, dc, ds, dx, base)
                _check_epi(orc, epi, got, best, n, full, f64, absf, base, f"valu {epi} R={r} NS={ns} k={k}")
                ran += 1
    finally:
        _force(rf, 0, -1)
    assert ran >= 2


@pytest.mark.parametrize("n,k", [(6144, 4096), (2560, 2048), (100, 14336)])
def test_gemv_fused_rmsnorm(rf, orc, stream, n, k):
    """rmsnorm + fp4_gemv in one launch (llama_run/src/main.rs:513-514)."""
    codes, scales, _ = _config1(orc, n, k, seed=n)
    rng = np.random.default_rng(k)
    x = (0.02 * rng.standard_normal(k)).astype(np.float32)
    w16 = (1 + 0.02 * rng.standard_normal(k)).astype(np.float16)
    h = orc.rmsnorm(x, w16.astype(np.float32), 1e-5)
    f64, absf = orc.gemv_e8m0_f64(n, k, codes, scales, h)
    dy = rf.DeviceBuffer.zeroed(n, np.float32, stream)
    rf.mx4_gemv_rmsnorm(stream, n, k, _dev(rf, codes, stream), _dev(rf, scales, stream), _dev(rf, x, stream),
                        _dev(rf, w16.view(np.uint16), stream), 1e-5, dy)
    got = dy.to_host(n, np.float32, stream)
    # the fused norm sums x^2 in another order than the oracle: its rms may
    # differ in the last place, which the normwise bound absorbs
    cond = np.abs(got.astype(np.float64) - f64) / np.maximum(absf, 1e-300)
    assert cond.max() < 1e-5, cond.max()
    assert (reference_rel_err(got, f64) > 1e-2).sum() == 0


@pytest.mark.parametrize("epi,r,ns", [("swiglu", 1, 1), ("store", 2, 1), ("resid", 1, 1), ("resid", 1, 3)])
@pytest.mark.parametrize("n,k", [(67, 512), (300, 2048), (5632, 2048), (2048, 5632)])
def test_gemv_eight_wave_variants(rf, orc, stream, epi, r, ns, n, k):
    """8 waves per workgroup (one K slice; three for the residual at 1 row
    per wave), forced; and the automatic choice on the same shape."""
    if (k + 2047) // 2048 > ns:
        pytest.skip("k needs more slices than the variant issues")
    codes, scales, x = _config1(orc, 2 * n, k, seed=n + k + r)
    x = _activation_like(orc, 2 * n, k, codes, scales, x, epi)
    dc, ds, dx = _dev(rf, codes, stream), _dev(rf, scales, stream), _dev(rf, x, stream)
    full = orc.gemv_e8m0(2 * n, k, codes, scales, x)
    f64, absf = orc.gemv_e8m0_f64(2 * n, k, codes, scales, x)
    if epi == "swiglu":
        _assert_gates_unsaturated(f64, n)
    base = np.linspace(-1, 1, n).astype(np.float32)
    try:
        for forced in (True, False):
            if forced:
                _force(rf, r, ns)
                rf.check(rf.load().rfp4_debug_gemv_waves(8))
            got, best = _run_epi(rf, stream, epi, n, k, dc, ds, dx, base)
            _check_epi(orc, epi, got, best, n, full, f64, absf, base, f"{epi} R={r} W=8 k={k} forced={forced}")
            _force(rf, 0, -1)
            rf.check(rf.load().rfp4_debug_gemv_waves(0))
    finally:
        _force(rf, 0, -1)
        rf.check(rf.load().rfp4_debug_gemv_waves(0))
