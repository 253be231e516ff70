"""Real-weight loading on the CPU: the safetensors reader (the format the
reference reads, llama_run/src/main.rs:413-430, widened to f32 as its `get`
closure does) and the reference's absmax/6 host packer
(llama_run/src/main.rs:334-376) against the oracle.  No device needed."""
import json
import os
import struct

import numpy as np
import pytest

import rfp4
import st_writer as stw


def _rng(seed=0):
    return np.random.default_rng(seed)


def test_reader_dtypes_shapes_and_widening(tmp_path):
    r = _rng(1)
    vals = {n: r.standard_normal(s).astype(np.float32) * 0.1 for n, s in
            [("a.bf16", (3, 64)), ("b.f16", (5,)), ("c.f32", (2, 3, 4)), ("d.scalar", ())]}
    tensors = {"a.bf16": ("BF16", stw.as_stored("BF16", vals["a.bf16"])),
               "b.f16": ("F16", stw.as_stored("F16", vals["b.f16"])),
               "c.f32": ("F32", vals["c.f32"]),
               "d.scalar": ("F32", vals["d.scalar"])}
    p = str(tmp_path / "m.safetensors")
    stw.write(p, tensors, metadata={"format": "pt", "note": "x\"y\\u00e9"}, pad_header=7)
    with rfp4.SafeTensors(p) as st:
        assert st.names() == list(tensors)
        for name, (dt, raw) in tensors.items():
            dtype, shape, nbytes = st.info(name)
            assert (dtype, shape, nbytes) == (dt, raw.shape, raw.nbytes)
            got = st.read_f32(name)
            np.testing.assert_array_equal(got.view(np.uint32), stw.widen(dt, raw).view(np.uint32).reshape(got.shape))


def test_reader_matches_the_safetensors_package(tmp_path):
    """Files written by the safetensors package itself (F16, F32, I32)."""
    from safetensors.numpy import save_file

    r = _rng(2)
    t = {"model.layers.0.mlp.up_proj.weight": r.standard_normal((8, 32)).astype(np.float16),
         "model.norm.weight": r.standard_normal(32).astype(np.float32),
         "ids": np.arange(6, dtype=np.int32)}
    p = str(tmp_path / "pkg.safetensors")
    save_file(t, p, metadata={"k": "v"})
    with rfp4.SafeTensors(p) as st:
        assert sorted(st.names()) == sorted(t)
        assert st.info("ids")[:2] == ("I32", (6,))
        np.testing.assert_array_equal(st.read_f32("model.layers.0.mlp.up_proj.weight"),
                                      t["model.layers.0.mlp.up_proj.weight"].astype(np.float32))
        np.testing.assert_array_equal(st.read_f32("model.norm.weight"), t["model.norm.weight"])
        with pytest.raises(rfp4.Rfp4Error) as e:
            st.read_f32("ids")  # integers are listed but not widened
        assert e.value.code == -2


def test_bf16_widening_is_exact_on_every_pattern(tmp_path):
    """All 65536 bf16 bit patterns (NaNs included) widen to the f32 whose
    upper half they are (the reference's `(bits as u32) << 16`)."""
    raw = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    p = str(tmp_path / "all.safetensors")
    stw.write(p, {"all": ("BF16", raw)})
    with rfp4.SafeTensors(p) as st:
        got = st.read_f32("all").view(np.uint32)
    np.testing.assert_array_equal(got, raw.astype(np.uint32) << 16)


def test_f16_widening_is_exact_on_every_pattern(tmp_path):
    raw = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    p = str(tmp_path / "allh.safetensors")
    stw.write(p, {"all": ("F16", raw)})
    with rfp4.SafeTensors(p) as st:
        got = st.read_f32("all")
    ref = raw.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    np.testing.assert_array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(ref)]))
    assert np.array_equal(got[np.isinf(ref)], ref[np.isinf(ref)])


def test_f16_rounding_matches_numpy(tmp_path):
    """rfp4_st_read_f16 (how the engine stores norm weights): every bf16 bit
    pattern, and f32 values across the f16 normal, subnormal and overflow
    ranges, round to nearest even exactly as numpy's float16 conversion."""
    raw = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    r = _rng(7)
    f = np.concatenate([
        r.standard_normal(20000) * 10.0 ** r.uniform(-9, 5, 20000),
        np.array([65504, 65519.99, 65520, 65536, 2 ** -24, 2 ** -25, 2 ** -25 * 1.0000001, 3 * 2 ** -26,
                  6.1e-5, 6.0e-5, 1.0009765625, 1.00048828125, 1.000732421875, -0.0, 0.0], np.float64),
    ]).astype(np.float32)
    p = str(tmp_path / "h.safetensors")
    stw.write(p, {"b": ("BF16", raw), "f": ("F32", f)})
    with rfp4.SafeTensors(p) as st:
        got_b, got_f = st.read_f16("b"), st.read_f16("f")
    for got, vals in ((got_b, stw.bf16_to_f32(raw)), (got_f, f)):
        ref = vals.astype(np.float16).view(np.uint16)
        nan = np.isnan(vals)
        np.testing.assert_array_equal(got[~nan], ref[~nan])
        assert np.all(np.isnan(got[nan].view(np.float16)))
    # bf16 gains between 2^-17 and 65504 survive exactly
    b = stw.bf16_to_f32(raw)
    ok = np.isfinite(b) & (np.abs(b) >= 2.0 ** -17) & (np.abs(b) <= 65504)
    np.testing.assert_array_equal(got_b[ok].view(np.float16).astype(np.float32), b[ok])


def _raw_file(path, header_obj, data=b"", hlen=None):
    h = header_obj if isinstance(header_obj, bytes) else json.dumps(header_obj).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h) if hlen is None else hlen))
        f.write(h)
        f.write(data)


@pytest.mark.parametrize("case", ["short", "hlen", "notobj", "json", "range", "size", "dtype", "missing_key"])
def test_reader_rejects_malformed_files(tmp_path, case):
    p = str(tmp_path / f"{case}.safetensors")
    good = {"w": {"dtype": "F32", "shape": [2, 2], "data_offsets": [0, 16]}}
    if case == "short":
        open(p, "wb").write(b"\x01\x02")
    elif case == "hlen":
        _raw_file(p, good, b"\0" * 16, hlen=1 << 40)
    elif case == "notobj":
        _raw_file(p, b"[1, 2]")
    elif case == "json":
        _raw_file(p, b'{"w": {"dtype": "F32", "shape": [2, 2], "data_offsets": [0, 16]', b"\0" * 16)
    elif case == "range":
        _raw_file(p, {"w": {"dtype": "F32", "shape": [2, 2], "data_offsets": [0, 16]}}, b"\0" * 8)
    elif case == "size":
        _raw_file(p, {"w": {"dtype": "F32", "shape": [2, 3], "data_offsets": [0, 16]}}, b"\0" * 16)
    elif case == "dtype":
        _raw_file(p, {"w": {"dtype": "Q4", "shape": [2, 2], "data_offsets": [0, 16]}}, b"\0" * 16)
    else:
        _raw_file(p, {"w": {"dtype": "F32", "shape": [2, 2]}}, b"\0" * 16)
    with pytest.raises(rfp4.Rfp4Error) as e:
        rfp4.SafeTensors(p)
    assert e.value.code in (-1, -2)
    assert b"safetensors" in rfp4.load().rfp4_last_error()


def test_reader_missing_file_and_tensor(tmp_path):
    with pytest.raises(rfp4.Rfp4Error):
        rfp4.SafeTensors(str(tmp_path / "nope.safetensors"))
    p = str(tmp_path / "one.safetensors")
    stw.write(p, {"w": ("F32", np.zeros(4, np.float32))})
    with rfp4.SafeTensors(p) as st:
        with pytest.raises(rfp4.Rfp4Error):
            st.info("v")


def test_absmax_packer_matches_the_oracle(orc):
    """fp4_quantize_absmax (product, host) == orc_quant_fp4_absmax (the
    restated reference loop) word for word, including the tie rule: values
    placed exactly on the midpoints between E2M1 magnitudes round down."""
    r = _rng(3)
    rows, k = 40, 256
    w = (r.standard_normal((rows, k)) * 10.0 ** r.uniform(-3, 1, (rows, 1))).astype(np.float32)
    w[0, :32] = 0.0                                   # all-zero block: scale 1
    w[1, :32] = -0.0
    mids = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], np.float32)
    w[2, :32] = np.resize(np.concatenate([mids, -mids, [6.0]]), 32).astype(np.float32)  # scale 1: exact ties
    w[3, :32] = np.resize(np.concatenate([mids * 4, [24.0]]), 32).astype(np.float32)     # scale 4: exact ties
    w[4, :32] = np.nextafter(w[2, :32], np.float32(np.inf))
    packed, scales = rfp4.fp4_quantize_absmax(w)
    opacked, oscales = orc.quant_fp4_absmax(w)
    np.testing.assert_array_equal(scales.view(np.uint32), oscales.view(np.uint32))
    np.testing.assert_array_equal(packed.view(np.uint8), opacked)
    # the ties went down: code of 0.25 is 0 (zero), of 0.75 is 1 (0.5)
    codes = np.stack([(packed[(2 * k) // 8 + i // 8] >> (4 * (i % 8))) & 15 for i in range(7)])
    assert list(codes) == [0, 1, 2, 3, 4, 5, 6]


def test_absmax_packer_rejects_bad_shapes():
    with pytest.raises(rfp4.Rfp4Error):
        rfp4.fp4_quantize_absmax(np.zeros((2, 33), np.float32))
