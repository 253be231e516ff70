"""Pins the operand / accumulator lane layout of the 16x16x32 bf16 and fp16
MFMAs against the host (the fp16 form is the prefill attention's
instruction)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

FP4V = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6], dtype=np.float32)


def _e2m1(c):
    return (-1.0 if c & 8 else 1.0) * FP4V[c & 7]


def _bf16_bits(v):
    """RNE f32 -> bf16 bits (host reference)."""
    u = np.asarray(v, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32)
    return r.astype(np.uint16)


def test_mfma_bf16_16x16x32_layout(rf, stream):
    """lane l: A row l%16 / B col l%16, K = 8*(l//16) + e (bf16 e in dword
    e//2, low half first); accumulator r of lane l = D[4*(l//16)+r][l%16]."""
    rng = np.random.default_rng(11)
    A = rng.integers(-4, 5, (16, 32)).astype(np.float32)
    B = rng.integers(-4, 5, (32, 16)).astype(np.float32)
    D = A @ B
    ra = np.zeros((64, 8), np.uint16)
    rb = np.zeros((64, 8), np.uint16)
    for lane in range(64):
        for e in range(8):
            k = 8 * (lane // 16) + e
            ra[lane, e] = _bf16_bits(A[lane % 16, k])
            rb[lane, e] = _bf16_bits(B[k, lane % 16])
    out = rf.DeviceBuffer.zeroed(256, np.float32, stream)
    da = rf.DeviceBuffer.from_host(ra.view(np.uint32), stream)
    db = rf.DeviceBuffer.from_host(rb.view(np.uint32), stream)
    rf.check(rf.load().rfp4_mma_bf16_tile(stream.h, da.ptr, db.ptr, out.ptr))
    regs = out.to_host(256, np.float32, stream).reshape(64, 4)
    got = np.zeros((16, 16), np.float32)
    for lane in range(64):
        for r in range(4):
            got[4 * (lane // 16) + r, lane % 16] = regs[lane, r]
    np.testing.assert_array_equal(got, D)


def test_mfma_f16_16x16x32_layout(rf, stream):
    """The fp16 form used by the prefill attention: the same lane layout as
    the bf16 one (A row / B col l%16, K = 8*(l//16) + e; D[4*(l//16)+r][l%16]),
    fp16 products exact in the f32 accumulator."""
    rng = np.random.default_rng(12)
    A = (rng.integers(-64, 65, (16, 32)) / 16.0).astype(np.float32)
    B = (rng.integers(-64, 65, (32, 16)) / 8.0).astype(np.float32)
    D = A.astype(np.float64) @ B.astype(np.float64)
    ra = np.zeros((64, 8), np.float16)
    rb = np.zeros((64, 8), np.float16)
    for lane in range(64):
        for e in range(8):
            k = 8 * (lane // 16) + e
            ra[lane, e] = A[lane % 16, k]
            rb[lane, e] = B[k, lane % 16]
    out = rf.DeviceBuffer.zeroed(256, np.float32, stream)
    da = rf.DeviceBuffer.from_host(ra.view(np.uint32), stream)
    db = rf.DeviceBuffer.from_host(rb.view(np.uint32), stream)
    rf.check(rf.load().rfp4_mma_f16_tile(stream.h, da.ptr, db.ptr, out.ptr))
    regs = out.to_host(256, np.float32, stream).reshape(64, 4)
    got = np.zeros((16, 16), np.float32)
    for lane in range(64):
        for r in range(4):
            got[4 * (lane // 16) + r, lane % 16] = regs[lane, r]
    np.testing.assert_array_equal(got, D.astype(np.float32))
