"""Batched prefill (the prompt through the MXFP4 GEMM, activations quantised
to MXFP4 per 32 along K) against the CPU oracle.  The reference feeds a
prompt token by token (llama_run/src/main.rs:550-556); the oracle's prefill
(orc_model_prefill) restates that loop with every projection input quantised
by the OCP rules.  Every case is checked stage by stage on identical inputs
(prefill_stages.check_prefill_stages: each stage of each layer against the
oracle's restatement of that stage applied to the GPU's own inputs, every
position, the logits of the last row included), and end to end: the next
token equals the oracle's own prefill's."""
import numpy as np
import pytest

from prefill_stages import check_prefill_stages

pytestmark = pytest.mark.gpu

TINY = dict(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=1024,
            theta=10000.0, eps=1e-5, max_seq=64)
TINY128 = dict(dim=512, n_layers=2, n_heads=8, n_kv_heads=2, head_dim=128, ffn=1024, vocab=2048,
               theta=500000.0, eps=1e-5, max_seq=300)

G8 = dict(dim=256, n_layers=2, n_heads=8, n_kv_heads=1, head_dim=64, ffn=512, vocab=1024,
          theta=10000.0, eps=1e-5, max_seq=200)    # 8 query heads per KV head
G1 = dict(dim=256, n_layers=2, n_heads=2, n_kv_heads=2, head_dim=128, ffn=512, vocab=1024,
          theta=500000.0, eps=1e-5, max_seq=200)   # no grouping
# Llama-3-8B widths (dim 4096, 32/8 heads, head dim 128, FFN 14336), two layers
W8B = dict(dim=4096, n_layers=2, n_heads=32, n_kv_heads=8, head_dim=128, ffn=14336, vocab=2048,
           theta=500000.0, eps=1e-5, max_seq=640)


def _engine(rf, cfg, seed):
    c = {k: v for k, v in cfg.items() if k != "max_seq"}
    return rf.Engine(rf.model_config(max_seq=cfg["max_seq"], **c), seed)


def _kv(eng, ref, cfg, layer, lo, hi):
    hd, nkv = cfg["head_dim"], cfg["n_kv_heads"]
    k, v = eng.kv_host(layer)
    stride = k.size // (nkv * hd)
    f = lambda a, s: a.reshape(nkv, s, hd)[:, lo:hi].view(np.float16).astype(np.float32)
    return (f(k, stride), f(v, stride),
            f(ref.kcache(layer), cfg["max_seq"]), f(ref.vcache(layer), cfg["max_seq"]))


def _rel(a, b):
    return float(np.max(np.abs(a - b)) / max(np.abs(b).max(), 1e-30))


@pytest.mark.parametrize("cfg,n", [(TINY, 1), (TINY, 5), (TINY, 37), (TINY128, 3), (TINY128, 200), (TINY128, 250), (G8, 70),
                                   (G1, 130)])
def test_prefill_matches_oracle(rf, orc, cfg, n):
    seed = 0x5EED + n
    rng = np.random.default_rng(n)
    prompt = rng.integers(0, cfg["vocab"], n, dtype=np.uint32)
    print(f"prefill cfg dim={cfg['dim']} n={n}", flush=True)
    eng = _engine(rf, cfg, seed)
    ref = orc.Model(cfg, seed)
    tok = check_prefill_stages(rf, orc, eng, ref, cfg, prompt, 0)
    rtok, rlog = ref.prefill(prompt, 0, want_logits=True)
    top2 = np.sort(rlog)[-2:]
    assert tok == rtok, f"gpu {tok} cpu {rtok} margin {top2[1] - top2[0]:.4g}"
    eng.close()


def test_prefill_stages_8b_widths(rf, orc):
    """Llama-3-8B widths, 512 prompt rows, two layers: every stage of both
    layers on identical inputs (no end-to-end oracle run at this size)."""
    cfg, seed = W8B, 0x8B8B
    prompt = np.random.default_rng(512).integers(0, cfg["vocab"], 512, dtype=np.uint32)
    print("prefill stages at 8B widths, 512 rows", flush=True)
    eng = _engine(rf, cfg, seed)
    ref = orc.Model(cfg, seed)
    check_prefill_stages(rf, orc, eng, ref, cfg, prompt, 0)
    eng.close()


@pytest.mark.parametrize("cfg", [TINY, TINY128])
def test_prefill_then_decode(rf, orc, cfg):
    """Prefill, then the on-device decode loop from position n: greedy tokens
    identical to the oracle's prefill + decode."""
    seed = 0xD0C
    prompt = [1, 7, 42, 99, 5, 3, 8, 250, 17, 64, 11]
    n_new = 16
    eng = _engine(rf, cfg, seed)
    ref = orc.Model(cfg, seed)
    t0 = eng.prefill(prompt, 0)
    r0 = ref.prefill(prompt, 0)
    assert t0 == r0
    gpu = eng.generate([t0], len(prompt), n_new)
    cpu, margins = ref.generate([r0], len(prompt), n_new)
    assert list(gpu) == list(cpu), f"gpu {list(gpu)}\ncpu {list(cpu)}\nmargins {margins}"
    eng.close()


@pytest.mark.parametrize("cfg", [TINY, TINY128, G8, G1])
def test_prefill_in_chunks(rf, orc, cfg):
    """A chunk prefilled at pos0 > 0 attends to the K/V of an earlier chunk
    (causal offset: row r sees pos0 + r + 1 positions)."""
    seed = 0xCAFE
    head = [4, 8, 15, 16, 23]
    chunk = list(range(100, 140))
    eng = _engine(rf, cfg, seed)
    ref = orc.Model(cfg, seed)
    assert eng.prefill(head, 0) == ref.prefill(head, 0)
    tok = check_prefill_stages(rf, orc, eng, ref, cfg, chunk, len(head))
    rtok = ref.prefill(chunk, len(head))
    assert tok == rtok
    eng.close()


def test_prefill_after_decode(rf, orc):
    """A chunk prefilled after the decode loop wrote the first positions.  The
    decode path keeps f32 activations, so its K/V differ from the oracle's by
    fp16 rounding (checked below); through the MXFP4 activation quantiser such
    a difference can move a block's absmax across a power of two and re-scale
    all 32 values of that block, so only the greedy token is held exact."""
    cfg, seed = TINY128, 0xCAFE
    head = [4, 8, 15, 16, 23]
    chunk = list(range(100, 140))
    eng = _engine(rf, cfg, seed)
    ref = orc.Model(cfg, seed)
    g = eng.generate(head, 0, 1)
    c, _ = ref.generate(head, 0, 1)
    assert list(g) == list(c)
    for layer in range(cfg["n_layers"]):
        kg, vg, kr, vr = _kv(eng, ref, cfg, layer, 0, len(head))
        assert _rel(kg, kr) <= 2e-3 and _rel(vg, vr) <= 2e-3
    tok = eng.prefill(chunk, len(head))
    rtok, rlog = ref.prefill(chunk, len(head), want_logits=True)
    top2 = np.sort(rlog)[-2:]
    assert tok == rtok, f"gpu {tok} cpu {rtok} margin {top2[1] - top2[0]:.4g}"
    eng.close()


def test_prefill_repeatable_and_regrows(rf):
    """Same prompt twice gives bit-identical logits; a longer prompt after a
    short one regrows the workspace and still matches a fresh engine."""
    cfg, seed = TINY, 0x1234
    eng = _engine(rf, cfg, seed)
    p = list(range(3, 40))
    t1 = eng.prefill(p[:4], 0)
    l1 = eng.logits()
    t2 = eng.prefill(p[:4], 0)
    np.testing.assert_array_equal(eng.logits(), l1)
    assert t1 == t2
    t3 = eng.prefill(p, 0)
    l3 = eng.logits()
    fresh = _engine(rf, cfg, seed)
    assert fresh.prefill(p, 0) == t3
    np.testing.assert_array_equal(fresh.logits(), l3)
    fresh.close()
    eng.close()


def test_prefill_errors(rf):
    eng = _engine(rf, TINY, 1)
    with pytest.raises(rf.Rfp4Error) as e:
        eng.prefill([1, 2, 3], TINY["max_seq"] - 2)  # runs past max_seq
    assert e.value.code == -4
    with pytest.raises(rf.Rfp4Error) as e:
        eng.prefill([TINY["vocab"]], 0)              # token out of range
    assert e.value.code == -1
    with pytest.raises(rf.Rfp4Error) as e:
        eng.prefill([], 0)
    assert e.value.code == -1
    eng.close()
    odd = dict(TINY, ffn=288)                        # ffn not a multiple of 256
    eng = _engine(rf, odd, 1)
    with pytest.raises(rf.Rfp4Error) as e:
        eng.prefill([1, 2], 0)
    assert e.value.code == -2
    eng.close()


def test_engine_step_blocked_weight_scales(rf):
    """An engine that can prefill holds each projection's E8M0 scales again in
    the step-blocked layout the tiled GEMM reads: equal to mx4_scales_tile of
    its row-major scales (stacked parts included); engines that cannot
    prefill hold none."""
    from test_gpu_gemm import tile_scales_np

    eng = _engine(rf, TINY128, 77)
    cfg = TINY128
    qd, kvd = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
    shapes = {0: (qd, cfg["dim"]), 1: (kvd, cfg["dim"]), 2: (kvd, cfg["dim"]), 3: (cfg["dim"], qd),
              4: (cfg["ffn"], cfg["dim"]), 5: (cfg["ffn"], cfg["dim"]), 6: (cfg["dim"], cfg["ffn"])}
    views = [(l, p) for l in range(cfg["n_layers"]) for p in range(7)] + [(-1, 0)]
    for layer, proj in views:
        rows, k = (cfg["vocab"], cfg["dim"]) if layer < 0 else shapes[proj]
        _, sc = eng.weight_host(layer, proj)
        ptr, nbytes = eng.weight_scales_tiled(layer, proj)
        assert nbytes == rows * k // 32
        got = np.empty(nbytes, np.uint8)
        rf.check(rf.load().rfp4_d2h(got.ctypes.data, ptr, nbytes, eng.stream.h))
        eng.stream.synchronize()
        np.testing.assert_array_equal(got, tile_scales_np(sc, rows, k), err_msg=f"layer {layer} proj {proj}")
    eng.close()
    c = {k: v for k, v in TINY.items() if k != "max_seq"}
    eng = rf.Engine(rf.model_config(max_seq=TINY["max_seq"], kv_format=1, **c), 1)  # f32 caches: no prefill
    with pytest.raises(rf.Rfp4Error):
        eng.weight_scales_tiled(0, 0)
    eng.close()


def test_prefill_swiglu_in_gemm_epilogue(rf, orc):
    """Llama-3-8B widths, 450 prompt rows (the second 256-row tile ragged):
    the gate|up GEMM's plan is the 256x256 ping-pong tile, so SwiGLU and the
    MXFP4 rows of its output come from the GEMM's epilogue.  Every stage on
    identical inputs within its bar (the SwiGLU rows against the exact values
    of the plain GEMM's output, which the stage hook stopped after the GEMM
    still writes), and against the GEMM + row kernel path (rfp4_debug_prefill_
    swiglu(1)): the same scale bytes and codes but where the two f32 sums lie
    at a rounding boundary (their K orders differ), and the same next token."""
    cfg, seed, n = W8B, 0x5A1F, 450
    assert rf.gemm_plan_kernel(n, 2 * cfg["ffn"], cfg["dim"]).startswith("rfp4_gemm_256x256_pp/kz1")
    prompt = np.random.default_rng(450).integers(0, cfg["vocab"], n, dtype=np.uint32)
    print("prefill at 8B widths, 450 rows, SwiGLU in the gate|up epilogue", flush=True)
    eng = _engine(rf, cfg, seed)
    ref = orc.Model(cfg, seed)
    tok = check_prefill_stages(rf, orc, eng, ref, cfg, prompt, 0)
    ffn = cfg["ffn"]
    rows = {}
    lib = rf.load()
    try:
        for mode in (0, 1):
            rf.check(lib.rfp4_debug_prefill_swiglu(mode))
            eng.prefill_stop(prompt, 0, 18)  # layer 1's SwiGLU rows
            rows[mode] = (eng.prefill_buffer("codes", (n, ffn // 2), np.uint8),
                          eng.prefill_buffer("scales", (n, ffn // 32), np.uint8))
            rows[mode] += (eng.prefill(prompt, 0),)
    finally:
        rf.check(lib.rfp4_debug_prefill_swiglu(0))
    (cf, sf, tf), (cu, su, tu) = rows[0], rows[1]
    assert tf == tu == tok
    off_s = np.count_nonzero(sf != su)
    off_c = np.count_nonzero(cf != cu)
    assert off_s <= n * ffn // 32 // 10000 and off_c <= n * ffn // 2 // 10000, (off_s, off_c)
    eng.close()
    ref.close()


@pytest.mark.parametrize("cfg,n,pos0,tile,nst,plan", [
    (TINY, 37, 0, 2, 2, "rfp4_gemm_128x128/kz1"),             # heads of 64
    (TINY128, 250, 0, 2, 3, "rfp4_gemm_128x128_p3/kz1"),      # heads of 128, ragged rows
    (TINY128, 200, 0, 0, 0, "rfp4_gemm_256x256_pp/kz1"),
    (G8, 70, 5, 0, 0, "rfp4_gemm_256x256_pp/kz1"),            # 640 columns: a ragged column tile; pos0 > 0
    (TINY, 37, 0, 4, 2, "rfp4_gemm_32x128/kz1"),
    (TINY128, 120, 3, 4, 4, "rfp4_gemm_32x128_p4/kz1"),
    (TINY128, 250, 0, 3, 3, "rfp4_gemm_64x128_p3/kz1"),
    (G8, 70, 0, 3, 4, "rfp4_gemm_64x128_p4/kz1"),
    (G8, 130, 0, 2, 3, "rfp4_gemm_128x128_p3/kz1"),            # heads of 64: partners in the wave's registers
])
def test_prefill_rope_in_gemm_epilogue(rf, orc, cfg, n, pos0, tile, nst, plan):
    """RoPE and the fp16 K/V cache rows in the q|k|v GEMM's epilogue (the
    _rope kernels of every tile and stage count compiled), each reached by a
    forced plan, heads of 64 and 128: the staged check (stage 2 compares
    the rotated q and the fp16 K/V rows bit for bit with the oracle's RoPE of
    the GEMM's own output, which the stop after stage 1 takes from the plain
    GEMM), and against the GEMM + row kernel path (rfp4_debug_prefill_rope(1)):
    identical q|k|v rows and caches after stage 2 of every layer, and the same
    next token."""
    seed = 0x20BE + n
    hd, dim = cfg["head_dim"], cfg["dim"]
    nqkv = (cfg["n_heads"] + 2 * cfg["n_kv_heads"]) * hd
    rng = np.random.default_rng(n + 1000 * tile)
    head = [int(t) for t in rng.integers(0, cfg["vocab"], pos0)]
    prompt = rng.integers(0, cfg["vocab"], n, dtype=np.uint32)
    print(f"prefill RoPE epilogue: dim={dim} head_dim={hd} n={n} pos0={pos0} plan {plan}", flush=True)
    lib = rf.load()
    eng = _engine(rf, cfg, seed)
    ref = orc.Model(cfg, seed)
    got = {}
    try:
        rf.debug_gemm_plan(tile, 1)
        rf.check(lib.rfp4_debug_gemm_stages(nst))
        assert rf.gemm_plan_kernel(n, nqkv, dim) == plan
        if pos0:
            assert eng.prefill(head, 0) == ref.prefill(head, 0)
        tok = check_prefill_stages(rf, orc, eng, ref, cfg, prompt, pos0)
        for mode in (0, 1):
            rf.check(lib.rfp4_debug_prefill_rope(mode))
            outs = []
            for l in range(cfg["n_layers"]):
                eng.prefill_stop(prompt, pos0, 10 * l + 2)
                outs.append(eng.prefill_buffer("c", (n, nqkv)))
                outs.extend(eng.kv_host(l))
            got[mode] = (outs, eng.prefill(prompt, pos0))
    finally:
        rf.check(lib.rfp4_debug_prefill_rope(0))
        rf.check(lib.rfp4_debug_gemm_stages(0))
        rf.debug_gemm_plan(-1, 0)
    for i, (a, b) in enumerate(zip(got[0][0], got[1][0])):
        np.testing.assert_array_equal(a, b, err_msg=f"output {i} (layer {i // 3}: q|k|v rows, k cache, v cache)")
    assert got[0][1] == got[1][1] == tok
    eng.close()
    ref.close()


def test_prefill_rope_hook_rejects_bad_values(rf):
    lib = rf.load()
    assert lib.rfp4_debug_prefill_rope(2) == -1
    assert lib.rfp4_debug_prefill_rope(-1) == -1
    rf.check(lib.rfp4_debug_prefill_rope(0))


@pytest.mark.parametrize("tile,kz,reduce_kernel", [(2, 2, 0), (2, 2, 1), (1, 3, 0), (3, 1, 0), (0, 1, 0)])
def test_prefill_residual_in_gemm_epilogue(rf, orc, tile, kz, reduce_kernel):
    """x += o and x += down in the o and down GEMMs' epilogues (GemmArgs::
    c_add) under forced plans: two K splits summed inside the launch, the
    same summed by the reduce kernel, three splits, one split, the ping-pong
    256x256 tile.  The staged check compares x after each residual add (stage
    6, and stage 0 of the next layer) bit for bit with x + the plain GEMM's
    output (the stop after stage 5 or 9 takes the plain GEMM), and the next
    token with the oracle's prefill."""
    cfg, n, seed = TINY128, 200, 0xADD0 + 10 * tile + kz
    prompt = np.random.default_rng(seed).integers(0, cfg["vocab"], n, dtype=np.uint32)
    print(f"prefill residual epilogue: tile {tile} kz {kz} reduce kernel {reduce_kernel}", flush=True)
    lib = rf.load()
    eng = _engine(rf, cfg, seed)
    ref = orc.Model(cfg, seed)
    try:
        rf.debug_gemm_plan(tile, kz)
        rf.check(lib.rfp4_debug_gemm_reduce_kernel(reduce_kernel))
        tok = check_prefill_stages(rf, orc, eng, ref, cfg, prompt, 0)
    finally:
        rf.check(lib.rfp4_debug_gemm_reduce_kernel(0))
        rf.debug_gemm_plan(-1, 0)
    rtok, rlog = ref.prefill(prompt, 0, want_logits=True)
    top2 = np.sort(rlog)[-2:]
    assert tok == rtok, f"gpu {tok} cpu {rtok} margin {top2[1] - top2[0]:.4g}"
    eng.close()
    ref.close()


def test_prefill_attn_quant_hook_rejects_bad_values(rf):
    lib = rf.load()
    assert lib.rfp4_debug_prefill_attn_quant(2) == -1
    assert lib.rfp4_debug_prefill_attn_quant(-1) == -1
    rf.check(lib.rfp4_debug_prefill_attn_quant(0))


@pytest.mark.parametrize("cfg,n", [(TINY, 37), (TINY128, 200), (G1, 130), (W8B, 300)])
def test_prefill_attention_key_groups(rf, orc, cfg, n):
    """Two key groups per attention workgroup (alternate key blocks, softmax
    states merged through LDS; the default where the plan is 4 waves) against
    one (rfp4_debug_prefill_ksplit(1)): with the f32 rows (stop after stage 3)
    and the quantizing epilogue, every stage within its bar, both head dims,
    query-head groups 1, 2 and 4; the next token equal to the one-group
    kernel's."""
    seed = 0x5B11 + n
    prompt = np.random.default_rng(seed).integers(0, cfg["vocab"], n, dtype=np.uint32)
    print(f"prefill, two key groups: dim={cfg['dim']} n={n}", flush=True)
    lib = rf.load()
    eng = _engine(rf, cfg, seed)
    ref = orc.Model(cfg, seed)
    try:
        rf.check(lib.rfp4_debug_prefill_ksplit(1))
        plain = eng.prefill(prompt, 0)
        rf.check(lib.rfp4_debug_prefill_ksplit(2))
        rf.check(lib.rfp4_debug_prefill_waves(4))
        tok = check_prefill_stages(rf, orc, eng, ref, cfg, prompt, 0)
    finally:
        rf.check(lib.rfp4_debug_prefill_ksplit(0))
        rf.check(lib.rfp4_debug_prefill_waves(0))
    assert tok == plain
    eng.close()
    ref.close()


def test_prefill_ksplit_hook_rejects_bad_values(rf):
    lib = rf.load()
    assert lib.rfp4_debug_prefill_ksplit(3) == -1
    assert lib.rfp4_debug_prefill_ksplit(-1) == -1
    rf.check(lib.rfp4_debug_prefill_ksplit(0))


@pytest.mark.parametrize("cfg,n,nst,kernel", [(TINY128, 200, 2, "rfp4_gemm_128x128/kz1"),
                                              (TINY128, 130, 3, "rfp4_gemm_128x128_p3/kz1"),
                                              (W8B, 300, 3, "rfp4_gemm_128x128_p3/kz1")])
def test_prefill_swiglu_epilogue_128x128(rf, orc, cfg, n, nst, kernel):
    """SwiGLU and the MXFP4 rows of its output in the 4-wave 128x128 GEMM's
    epilogue (rfp4_gemm_128x128[_p3]_sw: 64 gate rows paired with the
    matching 64 up rows per tile), reached by a forced plan: every stage
    within its bar (the SwiGLU rows against the exact values of the plain
    GEMM's output), and against the GEMM + row kernel path: the same scale
    bytes and codes but at rounding boundaries (the paired tile's K order),
    the same next token."""
    seed = 0x5E11 + n
    prompt = np.random.default_rng(seed).integers(0, cfg["vocab"], n, dtype=np.uint32)
    print(f"prefill SwiGLU epilogue on 128x128: dim={cfg['dim']} n={n} stages {nst}", flush=True)
    ffn = cfg["ffn"]
    lib = rf.load()
    eng = _engine(rf, cfg, seed)
    ref = orc.Model(cfg, seed)
    rows = {}
    try:
        rf.debug_gemm_plan(2, 1)
        rf.check(lib.rfp4_debug_gemm_stages(nst))
        assert rf.gemm_plan_kernel(n, 2 * ffn, cfg["dim"]) == kernel
        tok = check_prefill_stages(rf, orc, eng, ref, cfg, prompt, 0)
        for mode in (0, 1):
            rf.check(lib.rfp4_debug_prefill_swiglu(mode))
            eng.prefill_stop(prompt, 0, 18)  # layer 1's SwiGLU rows
            rows[mode] = (eng.prefill_buffer("codes", (n, ffn // 2), np.uint8),
                          eng.prefill_buffer("scales", (n, ffn // 32), np.uint8), eng.prefill(prompt, 0))
    finally:
        rf.check(lib.rfp4_debug_prefill_swiglu(0))
        rf.check(lib.rfp4_debug_gemm_stages(0))
        rf.debug_gemm_plan(-1, 0)
    (cf, sf, tf), (cu, su, tu) = rows[0], rows[1]
    assert tf == tu == tok
    assert np.count_nonzero(sf != su) <= max(2, n * ffn // 32 // 10000)
    assert np.count_nonzero(cf != cu) <= max(4, n * ffn // 2 // 10000)
    eng.close()
    ref.close()
