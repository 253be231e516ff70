"""GPU results against the committed golden fixtures of tests/golden/ (written
by make_golden.py from the CPU oracle on the BASELINE configs' seeded
inputs): config 1 GEMV, config 2 kernels, config 3 TinyLlama-1.1B tokens,
config 4 Llama-3-8B tokens.  The fixtures stand in for the oracle where
running it takes minutes (config 4: ~8 min on 8 cores)."""
import hashlib
import importlib.util
import json
import os

import numpy as np
import pytest

from conftest import GOLDEN, reference_rel_err
from test_gpu_kernels import _assert_gemv_close

pytestmark = pytest.mark.gpu


def _make_golden():
    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(GOLDEN, "make_golden.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _dev(rf, arr, s):
    return rf.DeviceBuffer.from_host(np.ascontiguousarray(arr), s)


def test_config1_gemv_fixture(rf, stream):
    """2048x2048 MXFP4 GEMV (uniform codes, E8M0 exponents in [-6, 2],
    x ~ N(0,1)) against the stored f32 oracle output and exact f64 sum."""
    fx = np.load(os.path.join(GOLDEN, "config1_gemv.npz"))
    codes, scales, x = _make_golden().config1_inputs()
    assert (_sha(codes), _sha(scales), _sha(x)) == (str(fx["sha_codes"]), str(fx["sha_scales"]), str(fx["sha_x"]))
    dy = rf.DeviceBuffer.zeroed(2048, np.float32, stream)
    rf.mx4_gemv(stream, 2048, 2048, _dev(rf, codes, stream), _dev(rf, scales, stream), _dev(rf, x, stream), dy)
    _assert_gemv_close(dy.to_host(2048, np.float32, stream), fx["y"], fx["y64"], fx["absy"])


def test_config2_kernel_fixtures(rf, orc, stream):
    """RMSNorm (harness inputs, rel 1e-5), RoPE at position 2047 (bit-exact)
    and the 32q/8kv attention harness (rel 1e-4) against stored outputs."""
    fx = np.load(os.path.join(GOLDEN, "config2_kernels.npz"))
    r, st = orc.xorshift32(0x9E3779B9, 2048)
    xn = (((r % 2001).astype(np.float32) - 1000.0) / 500.0).astype(np.float32)
    r, st = orc.xorshift32(st, 2048)
    wn = (0.5 + (r % 1000).astype(np.float32) / 1000.0).astype(np.float32)
    dy = rf.DeviceBuffer.zeroed(2048, np.float32, stream)
    rf.rmsnorm(stream, 2048, 1e-5, _dev(rf, xn, stream), _dev(rf, wn, stream), dy)
    assert reference_rel_err(dy.to_host(2048, np.float32, stream), fx["rmsnorm_y"]).max() < 1e-5

    r, _ = orc.xorshift32(0x13579BDF, 32 * 64)
    q = (((r % 2001).astype(np.float32) - 1000.0) / 500.0).astype(np.float32)
    c, s = orc.rope_table(2048, 64, 10000.0)
    dq = _dev(rf, q, stream)
    rf.rope(stream, 32, 64, 2047 * 32, _dev(rf, c, stream), _dev(rf, s, stream), dq)
    np.testing.assert_array_equal(dq.to_host(32 * 64, np.float32, stream), fx["rope_pos2047"])

    r, _ = orc.xorshift32(0xABCD1234, 32 * 64 + 2 * 512 * 8 * 64)
    vals = (((r % 2001).astype(np.float32) - 1000.0) / 700.0).astype(np.float32)
    dout = rf.DeviceBuffer.zeroed(32 * 64, np.float32, stream)
    rf.attn_decode(stream, 32, 8, 512, _dev(rf, vals[:2048], stream), _dev(rf, vals[2048:2048 + 262144], stream),
                   _dev(rf, vals[2048 + 262144:], stream), dout)
    rel = reference_rel_err(dout.to_host(32 * 64, np.float32, stream), fx["attn_harness_out"])
    assert (rel > 1e-4).sum() == 0, rel.max()


def _engine_tokens(rf, fx, persistent=None):
    cfg = dict(fx["config"])
    eng = rf.Engine(rf.model_config(**cfg), fx["seed"])
    try:
        if persistent is not None:
            eng.use_persistent(persistent)
        assert _sha(eng.weight_host(-1, 0)[0]) == fx["hashes"]["lm_codes"]
        assert _sha(eng.weight_host(0, 0)[0]) == fx["hashes"]["l0_wq_codes"]
        assert _sha(eng.weight_host(0, 6)[1]) == fx["hashes"]["l0_wd_scales"]
        if fx["prefill"]:
            eng.prefill_kv(*fx["prefill"])
        return eng.generate(np.array(fx["prompt"], np.uint32), fx["pos0"], fx["n_new"])
    finally:
        eng.close()


def _check_tokens(gpu, fx):
    want = np.array(fx["tokens"], np.uint32)
    mism = np.nonzero(gpu != want)[0]
    assert mism.size == 0, (f"first mismatch at step {mism[0]}: gpu {gpu[mism[0]]} oracle {want[mism[0]]}, "
                            f"oracle top-1 margin {fx['margins'][mism[0]]:.3e}")


def test_config3_tinyllama_tokens(rf):
    """TinyLlama-1.1B architecture, random MXFP4 weights, 16-token random
    prompt, 256 greedy steps: every token identical to the oracle's."""
    with open(os.path.join(GOLDEN, "tinyllama_tokens.json")) as f:
        fx = json.load(f)
    _check_tokens(_engine_tokens(rf, fx), fx)


@pytest.mark.parametrize("persistent", [True, False])
def test_config4_llama3_8b_tokens(rf, persistent):
    """Llama-3-8B architecture, random MXFP4 weights, fp16 KV pre-filled to
    4096 positions, 128 greedy steps from token 1: identical to the oracle,
    with the persistent step (one launch for all layers) and the graph step."""
    with open(os.path.join(GOLDEN, "llama3_8b_tokens.json")) as f:
        fx = json.load(f)
    _check_tokens(_engine_tokens(rf, fx, persistent), fx)
