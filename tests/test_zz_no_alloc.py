"""attn_decode_f16_noalloc: the allocation-free variant of attn_decode_f16
(split states in a static device array, set up by rfp4_init).  Two calls in a
row, the second with a smaller input, each against attn_decode_f16 on the
same plan (splits merged by the second kernel: bit-identical) and against the
oracle; a shape whose split states exceed the array is rejected before any
launch."""
import numpy as np
import pytest

from test_gpu_kernels import _assert_attn_close, _dev

pytestmark = pytest.mark.gpu


def _case(orc, nh, nkv, hd, seq, seed):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    cap = seq + 3
    kc = rng.standard_normal(nkv * cap * hd).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal(nkv * cap * hd).astype(np.float16).view(np.uint16)
    return q, kc, vc, cap


def test_noalloc_matches_allocating_entry_point(rf, orc, stream):
    lib = rf.load()
    # 32 x 244 x 132 floats of split state (the array holds 2^20) at context
    # 35000, then a smaller context (3000 tokens) on the same array
    for nh, nkv, hd, seq in [(32, 8, 128, 35000), (32, 4, 64, 3000)]:
        q, kc, vc, cap = _case(orc, nh, nkv, hd, seq, seq)
        dq, dk, dv = _dev(rf, q, stream), _dev(rf, kc, stream), _dev(rf, vc, stream)
        got = rf.DeviceBuffer.zeroed(nh * hd, np.float32, stream)
        exp = rf.DeviceBuffer.zeroed(nh * hd, np.float32, stream)
        rf.check(lib.attn_decode_f16_noalloc(stream.h, nh, nkv, hd, seq, dq.ptr, dk.ptr, dv.ptr, hd, cap * hd, got.ptr))
        rf.check(lib.rfp4_debug_attn_merge(1))  # the allocating call on the same merge path
        try:
            rf.attn_decode_f16(stream, nh, nkv, hd, seq, dq, dk, dv, hd, cap * hd, exp)
        finally:
            rf.check(lib.rfp4_debug_attn_merge(0))
        g = got.to_host(nh * hd, np.float32, stream)
        e = exp.to_host(nh * hd, np.float32, stream)
        np.testing.assert_array_equal(g, e)
        _assert_attn_close(g, orc.attn_decode(nh, nkv, hd, seq, q, kc, vc, hd, cap * hd))


def test_noalloc_rejects_states_beyond_the_array(rf, stream):
    """Context 40000 at 32 heads / head_dim 128 needs 278 splits: 1,174,272
    floats of state > 2^20.  Rejected on the host (the buffers are full size
    all the same)."""
    nh, nkv, hd, seq = 32, 8, 128, 40000
    n = nkv * (seq + 3) * hd
    dq = rf.DeviceBuffer.zeroed(nh * hd, np.float32, stream)
    dk = rf.DeviceBuffer.zeroed(n, np.uint16, stream)
    dv = rf.DeviceBuffer.zeroed(n, np.uint16, stream)
    out = rf.DeviceBuffer.zeroed(nh * hd, np.float32, stream)
    rc = rf.load().attn_decode_f16_noalloc(stream.h, nh, nkv, hd, seq, dq.ptr, dk.ptr, dv.ptr, hd, (seq + 3) * hd, out.ptr)
    assert rc == -3, rc
    assert b"exceed" in rf.load().rfp4_last_error()
