"""Batched MXFP4 GEMM (fp4_gemm, scaled MFMA) against the oracle's exact
float64 contraction C = sum_k A SFA W SFW (trackb/fp4_scale_test.cu:37 taken
to M x N x K; the reference has only the m16n8k64 tile, fp4_mma/src/main.rs).

Bar (fp32 accumulate): |c - c64| <= 1e-5 * sum_k |a_k w_k| on every element;
the reference's 1e-2 gate on every element whose exact value is not
cancellation-dominated (|c64| >= 1e-3 * sum_k |a_k w_k|: below that, the
normwise bound itself allows more than 1e-2 relative for any fp32 order);
and >= 99.9% of elements within 1e-3 relative of the exact sum.  Config-5 shapes too large for the CPU oracle are
checked on sampled rows and columns: C[i][j] depends only on row i of A and
row j of W, so a sub-GEMM of the sampled rows is an exact restatement."""
import numpy as np
import pytest

from conftest import reference_rel_err

pytestmark = pytest.mark.gpu

TILES = [(256, 256), (256, 128), (128, 128), (64, 128), (32, 128)]
CONFIG5_NK = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336), (128256, 4096)]


def _dev(rf, arr, s):
    return rf.DeviceBuffer.from_host(np.ascontiguousarray(arr), s)


def _uniform_mx(orc, rows, k, seed):
    """Codes uniform over the 16 E2M1 codes, E8M0 exponents uniform in [-6, 2]
    (the weight distribution of BASELINE config 1)."""
    words, st = orc.xorshift32(seed, rows * k // 8)
    codes = words.view(np.uint8).copy()
    r, _ = orc.xorshift32(st, rows * k // 32)
    return codes, (127 - 6 + (r % 9)).astype(np.uint8)


def _bf16_normal(rows, k, seed):
    """bf16 bits of N(0,1) samples (round to nearest even from f32)."""
    u = np.random.default_rng(seed).standard_normal((rows, k), dtype=np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _assert_gemm_close(c, c64, absc):
    c = np.asarray(c, np.float64)
    cond = np.abs(c - c64) / np.maximum(absc, 1e-300)
    assert cond.max() < 1e-5, f"max |c-c64|/sum|aw| = {cond.max():.3e}"
    rel = reference_rel_err(c, c64)
    well = np.abs(c64) >= 1e-3 * absc
    assert (rel[well] > 1e-2).sum() == 0, f"{(rel[well] > 1e-2).sum()} elements past 1e-2, max {rel[well].max():.3e}"
    assert np.mean(rel <= 1e-3) >= 0.999, f"{(rel > 1e-3).sum()} elements over 1e-3 (max {rel.max():.3e})"


def _gemm(rf, stream, m, n, k, ac, asc, wc, wsc):
    d = [_dev(rf, t, stream) if isinstance(t, np.ndarray) else t for t in (ac, asc, wc, wsc)]
    dc = rf.DeviceBuffer(m * n * 4)
    rf.fp4_gemm(stream, m, n, k, *d, dc)
    return dc.to_host(m * n, np.float32, stream).reshape(m, n)


@pytest.fixture
def forced_plan(rf):
    yield rf.debug_gemm_plan
    rf.debug_gemm_plan(-1, 0)


@pytest.mark.parametrize("tile", range(len(TILES)))
@pytest.mark.parametrize("kz", [1, 3])
def test_gemm_every_tile_and_split(rf, orc, stream, forced_plan, tile, kz):
    """Ragged m and n (neither a multiple of any tile), k of 4 K-steps; kz=3
    leaves the last split empty (ceil(4/3) = 2 steps per split)."""
    m, n, k = 80, 292, 1024
    ac, asc = _uniform_mx(orc, m, k, 11)
    wc, wsc = _uniform_mx(orc, n, k, 12)
    forced_plan(tile, kz)
    assert rf.gemm_plan(m, n, k) == (*TILES[tile], kz)
    c = _gemm(rf, stream, m, n, k, ac, asc, wc, wsc)
    c64, absc = orc.gemm_mx_f64(m, n, k, ac, asc, wc, wsc)
    _assert_gemm_close(c, c64, absc)
    c2 = _gemm(rf, stream, m, n, k, ac, asc, wc, wsc)
    np.testing.assert_array_equal(c.view(np.uint32), c2.view(np.uint32))  # deterministic


@pytest.mark.parametrize("m", [1, 7, 16, 17, 32, 33, 64])
@pytest.mark.parametrize("n,k", [(4, 2048), (292, 2048), (1040, 6144), (36, 512), (100, 5632), (60, 14336), (20, 16384)])
def test_gemm_few_rows_kernel(rf, orc, stream, forced_plan, m, n, k):
    """The few-row kernel (m <= 64, k a multiple of 512 up to 16384: 16/32/64
    activation rows per fragment, K segments of 512 over up to 8 waves, 1, 2
    or 4 per wave (64 rows: up to 2): k = 512 one wave, 5632 eleven segments
    over six waves of two, 14336 and 16384 over seven and eight waves of
    four) on ragged m and n, forced and automatic (m <= 32), against the
    oracle."""
    if m > 32 and k > 8192:
        pytest.skip("64-row fragments take k <= 8192")
    ac, asc = _uniform_mx(orc, m, k, 61 + m)
    wc, wsc = _uniform_mx(orc, n, k, 71 + n)
    c64, absc = orc.gemm_mx_f64(m, n, k, ac, asc, wc, wsc)
    plans = ((5, 0), (-1, 0)) if m <= 32 else ((5, 0),)
    for plan in plans:
        forced_plan(*plan)
        tm, tn, kz = rf.gemm_plan(m, n, k)
        assert tm == (16 if m <= 16 else 32 if m <= 32 else 64) and tn == 16 * kz and kz == 1
        c = _gemm(rf, stream, m, n, k, ac, asc, wc, wsc)
        _assert_gemm_close(c, c64, absc)
        c2 = _gemm(rf, stream, m, n, k, ac, asc, wc, wsc)
        np.testing.assert_array_equal(c.view(np.uint32), c2.view(np.uint32))  # deterministic


# every compiled few-row variant: (activation fragments, K segments per wave, W fragments)
ROWS_VARIANTS = [(mb, seg, nf) for mb in (1, 2) for seg, nf in ((1, 1), (1, 2), (1, 4), (2, 1), (2, 2), (4, 1))] + \
    [(4, 1, 1), (4, 1, 2), (4, 2, 1)]


@pytest.mark.parametrize("mb,seg,nf", ROWS_VARIANTS)
def test_gemm_few_rows_every_variant(rf, orc, stream, forced_plan, mb, seg, nf):
    """Each few-row variant, forced through its W-fragment count, on ragged m
    (16 mb - 3 rows), n (a ragged last workgroup) and a K whose segment count
    needs its segments per wave."""
    m = 16 * mb - 3
    k = 512 * (8 * seg - 3 if seg > 1 else 5)
    n = 16 * nf * 3 + 4
    ac, asc = _uniform_mx(orc, m, k, 91 + mb)
    wc, wsc = _uniform_mx(orc, n, k, 95 + nf)
    forced_plan(5, nf)
    assert rf.gemm_plan(m, n, k) == (16 * mb, 16 * nf, nf)
    c = _gemm(rf, stream, m, n, k, ac, asc, wc, wsc)
    c64, absc = orc.gemm_mx_f64(m, n, k, ac, asc, wc, wsc)
    _assert_gemm_close(c, c64, absc)


def test_gemm_few_rows_wide_n(rf, orc, stream, forced_plan):
    """Wide N takes 2 or 4 W fragments per workgroup (here 4: 257 workgroups
    of 64 rows) with a ragged last workgroup."""
    m, n, k = 32, 16396, 2048
    ac, asc = _uniform_mx(orc, m, k, 81)
    wc, wsc = _uniform_mx(orc, n, k, 82)
    forced_plan(5, 0)
    assert rf.gemm_plan(m, n, k) == (32, 64, 4)
    c = _gemm(rf, stream, m, n, k, ac, asc, wc, wsc)
    cols = np.unique(np.concatenate([np.arange(48), n - 48 + np.arange(48),
                                     np.random.default_rng(1).choice(n, 400, replace=False)]))
    c64, absc = orc.gemm_mx_f64(m, len(cols), k, ac, asc, wc.reshape(n, -1)[cols], wsc.reshape(n, -1)[cols])
    _assert_gemm_close(c[:, cols], c64, absc)


def test_gemm_row_permutation_is_exact(rf, orc, stream, forced_plan):
    """Each C[i][j] is computed by the same MFMA sequence wherever row i sits
    in its tile: permuting A's rows permutes C's rows bit for bit."""
    m, n, k = 96, 256, 2048
    ac, asc = _uniform_mx(orc, m, k, 21)
    wc, wsc = _uniform_mx(orc, n, k, 22)
    perm = np.random.default_rng(3).permutation(m)
    forced_plan(3, 2)
    c = _gemm(rf, stream, m, n, k, ac, asc, wc, wsc)
    cp = _gemm(rf, stream, m, n, k, ac.reshape(m, -1)[perm], asc.reshape(m, -1)[perm], wc, wsc)
    np.testing.assert_array_equal(c[perm].view(np.uint32), cp.view(np.uint32))


def test_gemm_small_edges(rf, orc, stream):
    """m = 1, n = 4 (smaller than every tile), k = 256 (a single K step),
    an all-zero block and scale extremes 2^-127 / 2^+20."""
    for m, n, k in [(1, 4, 256), (33, 36, 512), (7, 132, 256)]:
        ac, asc = _uniform_mx(orc, m, k, 31 + m)
        wc, wsc = _uniform_mx(orc, n, k, 41 + n)
        ac.reshape(m, -1)[0, :16] = 0            # zero block in row 0
        asc.reshape(m, -1)[-1, 0] = 0            # 2^-127
        wsc.reshape(n, -1)[0, -1] = 127 + 20
        c = _gemm(rf, stream, m, n, k, ac, asc, wc, wsc)
        c64, absc = orc.gemm_mx_f64(m, n, k, ac, asc, wc, wsc)
        _assert_gemm_close(c, c64, absc)


def test_gemm_one_hot_selects_weight_value(rf, orc, stream):
    """A row i = 1.0 at one K position p (code 0x2, scale 2^0): C[i][j] is
    exactly the dequantised W[j][p]."""
    n, k = 128, 512
    wc, wsc = _uniform_mx(orc, n, k, 51)
    ps = [0, 1, 31, 32, 63, 64, 127, 128, 255, 256, 300, 511]
    m = len(ps)
    codes = np.zeros((m, k), np.uint8)
    for i, p in enumerate(ps):
        codes[i, p] = 0x2
    ac = orc.pack(codes.reshape(-1)).reshape(-1)
    asc = np.full(m * k // 32, 127, np.uint8)
    c = _gemm(rf, stream, m, n, k, ac, asc, wc, wsc)
    e2m1 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0.0, -.5, -1, -1.5, -2, -3, -4, -6])
    wv = e2m1[orc.unpack(wc)].reshape(n, k) * np.exp2(
        np.repeat(wsc.reshape(n, -1).astype(np.float64) - 127, 32, axis=1))
    for i, p in enumerate(ps):
        np.testing.assert_array_equal(c[i], wv[:, p].astype(np.float32))


def _config5_case(rf, orc, stream, m, n, k, sample_rows=None, sample_cols=None):
    """bf16 activations ~N(0,1) quantised on the device (bit-exact against the
    oracle quantiser), uniform MXFP4 weights, then the GEMM."""
    a16 = _bf16_normal(m, k, m * 7 + k)
    da = _dev(rf, a16, stream)
    dac, das = rf.DeviceBuffer(m * k // 2), rf.DeviceBuffer(m * k // 32)
    rf.mx4_quantize(stream, m, k, da, True, dac, das)
    ac = dac.to_host(m * k // 2, np.uint8, stream)
    asc = das.to_host(m * k // 32, np.uint8, stream)
    a32 = (a16.astype(np.uint32) << 16).view(np.float32)
    c_ref, s_ref = orc.quant_mx(a32)
    np.testing.assert_array_equal(ac, c_ref)
    np.testing.assert_array_equal(asc, s_ref)
    wc, wsc = _uniform_mx(orc, n, k, (n * 31 + k) | 1)
    c = _gemm(rf, stream, m, n, k, dac, das, wc, wsc)
    rows = np.arange(m) if sample_rows is None else sample_rows
    cols = np.arange(n) if sample_cols is None else sample_cols
    ac2, as2 = ac.reshape(m, -1)[rows], asc.reshape(m, -1)[rows]
    wc2, ws2 = wc.reshape(n, -1)[cols], wsc.reshape(n, -1)[cols]
    c64, absc = orc.gemm_mx_f64(len(rows), len(cols), k, ac2, as2, wc2, ws2)
    _assert_gemm_close(c[np.ix_(rows, cols)], c64, absc)
    assert np.isfinite(c).all()


@pytest.mark.parametrize("n,k", CONFIG5_NK)
def test_gemm_config5_decode_batch32(rf, orc, stream, n, k):
    """BASELINE config 5, decode at batch 32: the whole C against the oracle
    (LM-head shape: 4096 sampled columns incl. both ends)."""
    cols = None
    if n > 16384:
        cols = np.unique(np.concatenate([np.arange(64), n - 64 + np.arange(64),
                                         np.random.default_rng(n).choice(n, 3968, replace=False)]))
    _config5_case(rf, orc, stream, 32, n, k, sample_cols=cols)


@pytest.mark.parametrize("n,k", CONFIG5_NK)
def test_gemm_config5_prefill512(rf, orc, stream, n, k):
    """BASELINE config 5, prefill of 512 tokens: 24 sampled rows (first and
    last of the tile rows included) x up to 1024 sampled columns."""
    rng = np.random.default_rng(n + k)
    rows = np.unique(np.concatenate([[0, 1, 31, 32, 63, 64, 127, 128, 255, 256, 510, 511],
                                     rng.choice(512, 12, replace=False)]))
    cols = np.unique(np.concatenate([np.arange(32), n - 32 + np.arange(32),
                                     rng.choice(n, min(n, 960), replace=False)]))
    _config5_case(rf, orc, stream, 512, n, k, sample_rows=rows, sample_cols=cols)


# tiles with deeper K pipelines compiled (kernels.hip GEMM_KERNEL_P): tile index -> stages
DEEP = {1: (3,), 2: (3,), 3: (3, 4), 4: (4,)}


@pytest.mark.parametrize("tile", sorted(DEEP))
@pytest.mark.parametrize("kz", [1, 3])
def test_gemm_deep_pipelines_bit_identical(rf, orc, stream, forced_plan, tile, kz):
    """Every deeper DMA pipeline of a tile gives the double-buffered result
    bit for bit (same MFMA sequence), on ragged m and n, K splits included,
    with K step counts below and above the pipeline depth (k = 512: 2 steps;
    k = 2816: 11), and stays within the bar against the oracle."""
    m, n = 200, 900
    lib = rf.load()
    for k in (512, 2816):
        ac, asc = _uniform_mx(orc, m, k, 41 + k)
        wc, wsc = _uniform_mx(orc, n, k, 43 + k)
        forced_plan(tile, kz)
        try:
            rf.check(lib.rfp4_debug_gemm_stages(2))
            c2 = _gemm(rf, stream, m, n, k, ac, asc, wc, wsc)
            for nst in DEEP[tile]:
                rf.check(lib.rfp4_debug_gemm_stages(nst))
                cd = _gemm(rf, stream, m, n, k, ac, asc, wc, wsc)
                np.testing.assert_array_equal(c2.view(np.uint32), cd.view(np.uint32), err_msg=f"k {k} stages {nst}")
        finally:
            rf.check(lib.rfp4_debug_gemm_stages(0))
        c64, absc = orc.gemm_mx_f64(m, n, k, ac, asc, wc, wsc)
        _assert_gemm_close(c2, c64, absc)


@pytest.mark.parametrize("tile", range(len(TILES)))
def test_gemm_two_way_split_summed_in_launch(rf, orc, stream, forced_plan, tile):
    """Two-way K splits summed inside the launch (the last split of each tile
    adds the other's plane) give the reduce kernel's result bit for bit, on
    ragged m and n, with one and with several K steps per split, over
    repeated calls with a smaller shape in between (a counter left non-zero
    or a stale plane would change a result), and within the bar against the
    oracle."""
    lib = rf.load()
    cases = [(200, 900, 512), (200, 900, 2816), (33, 132, 1024)]
    data = {}
    for m, n, k in cases:
        ac, asc = _uniform_mx(orc, m, k, 81 + k + m)
        wc, wsc = _uniform_mx(orc, n, k, 83 + k + n)
        data[(m, n, k)] = (ac, asc, wc, wsc)
    forced_plan(tile, 2)
    try:
        ref = {}
        rf.check(lib.rfp4_debug_gemm_reduce_kernel(1))
        for key, d in data.items():
            ref[key] = _gemm(rf, stream, *key, *d)
        rf.check(lib.rfp4_debug_gemm_reduce_kernel(0))
        for rep in range(4):
            for key, d in data.items():
                got = _gemm(rf, stream, *key, *d)
                np.testing.assert_array_equal(ref[key].view(np.uint32), got.view(np.uint32), err_msg=f"{key} rep {rep}")
    finally:
        rf.check(lib.rfp4_debug_gemm_reduce_kernel(0))
    for key, (ac, asc, wc, wsc) in data.items():
        c64, absc = orc.gemm_mx_f64(*key, ac, asc, wc, wsc)
        _assert_gemm_close(ref[key], c64, absc)


@pytest.mark.parametrize("tile", [0, 1])
@pytest.mark.parametrize("kz", [1, 3])
def test_gemm_ping_pong_bit_identical(rf, orc, stream, forced_plan, tile, kz):
    """The 8-wave ping-pong kernels of the 256x256 and 256x128 tiles give the
    4-wave kernels' results bit for bit (each accumulator gets the same MFMA
    sequence; the scale byte comes from the instruction's byte select), on
    ragged m and n (the second wave group's rows partly or wholly past m), with
    1, 2 and 11 K steps and K splits (the reduce kernel sums them), and stay
    within the bar against the oracle."""
    lib = rf.load()
    for m, n, k in ((200, 900, 256), (200, 900, 512), (100, 900, 2816), (512, 1024, 4096)):
        ac, asc = _uniform_mx(orc, m, k, 61 + k + m)
        wc, wsc = _uniform_mx(orc, n, k, 63 + k + n)
        forced_plan(tile, kz)
        try:
            rf.check(lib.rfp4_debug_gemm_pp(1))
            c4 = _gemm(rf, stream, m, n, k, ac, asc, wc, wsc)
            rf.check(lib.rfp4_debug_gemm_pp(2))
            cp = _gemm(rf, stream, m, n, k, ac, asc, wc, wsc)
            cp2 = _gemm(rf, stream, m, n, k, ac, asc, wc, wsc)
        finally:
            rf.check(lib.rfp4_debug_gemm_pp(0))
        np.testing.assert_array_equal(c4.view(np.uint32), cp.view(np.uint32), err_msg=f"{m}x{n}x{k}")
        np.testing.assert_array_equal(cp.view(np.uint32), cp2.view(np.uint32), err_msg=f"{m}x{n}x{k} repeat")
        if m * n * k <= 200 * 900 * 2816:
            c64, absc = orc.gemm_mx_f64(m, n, k, ac, asc, wc, wsc)
            _assert_gemm_close(cp, c64, absc)


def test_gemm_pp_hook_rejects_bad_values(rf):
    lib = rf.load()
    assert lib.rfp4_debug_gemm_pp(3) == -1
    assert lib.rfp4_debug_gemm_pp(-1) == -1
    rf.check(lib.rfp4_debug_gemm_pp(0))


def test_gemm_reduce_hook_rejects_bad_values(rf):
    lib = rf.load()
    assert lib.rfp4_debug_gemm_reduce_kernel(2) == -1
    assert lib.rfp4_debug_gemm_reduce_kernel(-1) == -1
    rf.check(lib.rfp4_debug_gemm_reduce_kernel(0))


def test_gemm_stage_hook_rejects_bad_values(rf):
    lib = rf.load()
    assert lib.rfp4_debug_gemm_stages(1) == -1
    assert lib.rfp4_debug_gemm_stages(5) == -1
    rf.check(lib.rfp4_debug_gemm_stages(0))


# ---------------------------------------------------------------- step-blocked scales
def tile_scales_np(sc, rows, k):
    """The step-blocked layout (include/rfp4.h, mx4_scales_tile): for row block
    rb, K step s, half h, row r and byte j, scale block 8 s + 4 h + j of row
    32 rb + r; rows past `rows` zero."""
    nb = (rows + 31) // 32
    pad = np.zeros((nb * 32, k // 32), np.uint8)
    pad[:rows] = np.asarray(sc, np.uint8).reshape(rows, k // 32)
    t = pad.reshape(nb, 32, k // 256, 2, 4)           # rb, r, s, h, j
    return np.ascontiguousarray(t.transpose(0, 2, 3, 1, 4)).reshape(-1)  # rb, s, h, r, j


def test_tile_scales_np_layout():
    """The restatement against hand-placed bytes: row 33's scale block 13 of a
    k = 512 matrix (step 1, half 1, byte 1) sits in block 1 at
    (1 * 2 + 1) * 256 + 128 + 4 * 1 + 1."""
    sc = np.zeros((40, 16), np.uint8)
    sc[33, 13] = 7
    t = tile_scales_np(sc, 40, 512)
    assert t.size == 64 * 16
    assert np.flatnonzero(t).tolist() == [(1 * 2 + 1) * 256 + 128 + 4 + 1] and t.max() == 7


@pytest.mark.parametrize("rows,k", [(1, 256), (33, 256), (80, 1024), (292, 768), (4096, 4096)])
def test_scales_tile_layout(rf, stream, rows, k):
    sc = np.random.default_rng(rows + k).integers(0, 256, rows * k // 32, dtype=np.uint8)
    nbytes = rf.mx4_scales_tiled_bytes(rows, k)
    assert nbytes == (rows + 31) // 32 * 32 * k // 32
    dt = rf.DeviceBuffer(nbytes)
    rf.mx4_scales_tile(stream, rows, k, _dev(rf, sc, stream), dt)
    np.testing.assert_array_equal(dt.to_host(nbytes, np.uint8, stream), tile_scales_np(sc, rows, k))


@pytest.mark.parametrize("bf16", [True, False])
def test_quantize_tiled_writes_both_layouts(rf, stream, bf16):
    """mx4_quantize_tiled: the codes and row-major scales of mx4_quantize, bit
    for bit, plus their step-blocked copy."""
    rows, k = 37, 1280
    if bf16:
        src = _bf16_normal(rows, k, 3)
    else:
        src = np.random.default_rng(3).standard_normal((rows, k), dtype=np.float32)
    ds = _dev(rf, src, stream)
    c0, s0 = rf.DeviceBuffer(rows * k // 2), rf.DeviceBuffer(rows * k // 32)
    c1, s1 = rf.DeviceBuffer(rows * k // 2), rf.DeviceBuffer(rows * k // 32)
    st = rf.DeviceBuffer(rf.mx4_scales_tiled_bytes(rows, k))
    rf.mx4_quantize(stream, rows, k, ds, bf16, c0, s0)
    rf.mx4_quantize_tiled(stream, rows, k, ds, bf16, c1, s1, st)
    sc = s0.to_host(rows * k // 32, np.uint8, stream)
    np.testing.assert_array_equal(c1.to_host(rows * k // 2, np.uint8, stream), c0.to_host(rows * k // 2, np.uint8, stream))
    np.testing.assert_array_equal(s1.to_host(rows * k // 32, np.uint8, stream), sc)
    # the quantizer writes the blocks of its rows only (rows 37-63 of the last block are left as they were)
    valid = tile_scales_np(np.ones(rows * k // 32, np.uint8), rows, k) == 1
    got = st.to_host(st.nbytes, np.uint8, stream)
    np.testing.assert_array_equal(got[valid], tile_scales_np(sc, rows, k)[valid])
    with pytest.raises(rf.Rfp4Error):
        rf.mx4_quantize_tiled(stream, rows, 1056, ds, bf16, c1, s1, st)  # k not a multiple of 256


@pytest.mark.parametrize("tile", list(range(len(TILES))) + [5])
def test_gemm_tiled_entry_bit_identical(rf, orc, stream, forced_plan, tile):
    """fp4_gemm_tiled with the caller's step-blocked scales equals fp4_gemm
    (which makes them itself) bit for bit, on every tiled kernel and the
    few-row kernel (which reads the row-major scales), and the oracle."""
    m, n, k = (80, 292, 1024) if tile < 5 else (16, 292, 1024)
    ac, asc = _uniform_mx(orc, m, k, 21)
    wc, wsc = _uniform_mx(orc, n, k, 22)
    d = [_dev(rf, t, stream) for t in (ac, asc, wc, wsc)]
    ast = _dev(rf, tile_scales_np(asc, m, k), stream)
    wst = _dev(rf, tile_scales_np(wsc, n, k), stream)
    forced_plan(tile, 1 if tile < 5 else 2)
    c0 = _gemm(rf, stream, m, n, k, *d)
    dc = rf.DeviceBuffer(m * n * 4)
    rf.fp4_gemm_tiled(stream, m, n, k, d[0], d[1], ast, d[2], d[3], wst, dc)
    c1 = dc.to_host(m * n, np.float32, stream).reshape(m, n)
    np.testing.assert_array_equal(c1.view(np.uint32), c0.view(np.uint32))
    c64, absc = orc.gemm_mx_f64(m, n, k, ac, asc, wc, wsc)
    _assert_gemm_close(c1, c64, absc)
