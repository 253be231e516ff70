"""End-to-end parity of the decode engine against the CPU oracle decode loop
on the same packed weights and seeds (greedy tokens identical over the test
horizon; llama_run/src/main.rs:492-570 is the loop both restate)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TINY = dict(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=1024,
            theta=10000.0, eps=1e-5, max_seq=64)
TINY128 = dict(dim=512, n_layers=2, n_heads=8, n_kv_heads=2, head_dim=128, ffn=1024, vocab=2048,
               theta=500000.0, eps=1e-5, max_seq=300)


def _engine(rf, cfg, seed):
    c = {k: v for k, v in cfg.items() if k != "max_seq"}
    return rf.Engine(rf.model_config(max_seq=cfg["max_seq"], **c), seed)


def _proj_rows(cfg, p):
    qd, kvd = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
    return [(qd, cfg["dim"]), (kvd, cfg["dim"]), (kvd, cfg["dim"]), (cfg["dim"], qd),
            (cfg["ffn"], cfg["dim"]), (cfg["ffn"], cfg["dim"]), (cfg["dim"], cfg["ffn"])][p]


@pytest.mark.parametrize("cfg", [TINY, TINY128])
def test_engine_weights_bit_exact(rf, orc, cfg):
    seed = 0x5EED
    eng = _engine(rf, cfg, seed)
    ref = orc.Model(cfg, seed)
    for layer in range(cfg["n_layers"]):
        for p in range(7):
            c, s = eng.weight_host(layer, p)
            np.testing.assert_array_equal(c, ref.codes(layer, p), err_msg=f"codes l{layer} p{p}")
            np.testing.assert_array_equal(s, ref.scales(layer, p), err_msg=f"scales l{layer} p{p}")
    c, s = eng.weight_host(-1, 0)
    np.testing.assert_array_equal(c, ref.codes(-1, 0))
    np.testing.assert_array_equal(s, ref.scales(-1, 0))
    eng.close()


@pytest.mark.parametrize("cfg", [TINY, TINY128])
def test_engine_tokens_match_oracle(rf, orc, cfg):
    seed = 0x5EED
    eng = _engine(rf, cfg, seed)
    ref = orc.Model(cfg, seed)
    prompt = [1, 7, 42, 99, 5]
    n_new = 24
    gpu = eng.generate(prompt, 0, n_new)
    cpu, margins = ref.generate(prompt, 0, n_new)
    assert list(gpu) == list(cpu), f"gpu {list(gpu)}\ncpu {list(cpu)}\nmargins {margins}"
    # KV cache after the run: fp16 K/V equal to the oracle's for written positions
    hd, nkv = cfg["head_dim"], cfg["n_kv_heads"]
    npos = len(prompt) + n_new - 1
    for layer in range(cfg["n_layers"]):
        k, v = eng.kv_host(layer)
        stride = k.size // (nkv * hd)
        kg = k.reshape(nkv, stride, hd)[:, :npos].astype(np.uint16).view(np.float16).astype(np.float32)
        kr = ref.kcache(layer).reshape(nkv, cfg["max_seq"], hd)[:, :npos].view(np.float16).astype(np.float32)
        assert np.max(np.abs(kg - kr)) <= 2e-3 * max(1.0, np.abs(kr).max())
    eng.close()


def test_engine_graph_equals_eager(rf, orc):
    seed = 0xABC
    eng = _engine(rf, TINY, seed)
    prompt = [3, 1, 4, 1, 5, 9]
    g = eng.generate(prompt, 0, 12)
    lg = eng.logits()
    eng.use_graph(False)
    e = eng.generate(prompt, 0, 12)
    le = eng.logits()
    assert list(g) == list(e)
    np.testing.assert_array_equal(lg, le)
    eng.close()


def test_decode_step_matches_generate(rf, orc):
    """llama_decode_step (one blocking forward) equals the on-device loop."""
    seed = 0x77
    eng = _engine(rf, TINY, seed)
    ref = orc.Model(TINY, seed)
    toks = [11, 22, 33]
    for pos, t in enumerate(toks):
        nxt = eng.decode_step(t, pos)
        assert nxt == ref.step(t, pos)
    eng.close()


def test_engine_errors(rf):
    eng = _engine(rf, TINY, 1)
    with pytest.raises(rf.Rfp4Error) as e:
        eng.generate([1, 2], TINY["max_seq"] - 1, 4)  # would run past max_seq
    assert e.value.code == -4
    with pytest.raises(rf.Rfp4Error):
        eng.generate([TINY["vocab"]], 0, 1)             # token out of range
    eng.close()


@pytest.mark.parametrize("cfg", [TINY, TINY128])
@pytest.mark.parametrize("mode", [1, 2, 3])
def test_engine_attn_merge_modes_tokens(rf, orc, cfg, mode):
    """The decode step with the attention splits merged by a second kernel
    (mode 1), inside the attention kernel by the last split (mode 2) or by
    the first splits polling tagged states (mode 3): the same greedy tokens as
    the oracle over a context that needs several splits."""
    seed = 0x1A2B
    rf.check(rf.load().rfp4_debug_attn_merge(mode))
    rf.debug_attn_chunk(cfg["max_seq"] // 6 + 1)  # 6 splits over the context
    try:
        eng = _engine(rf, cfg, seed)
    finally:
        rf.debug_attn_chunk(0)
        rf.check(rf.load().rfp4_debug_attn_merge(0))
    ref = orc.Model(cfg, seed)
    prompt = [2, 9, 77, 401, 5, 6, 7]
    gpu = eng.generate(prompt, 0, 30)
    cpu, margins = ref.generate(prompt, 0, 30)
    assert list(gpu) == list(cpu), f"gpu {list(gpu)}\ncpu {list(cpu)}\nmargins {margins}"
    eng.close()


G8E = dict(dim=256, n_layers=2, n_heads=8, n_kv_heads=1, head_dim=64, ffn=512, vocab=1024,
           theta=10000.0, eps=1e-5, max_seq=200)  # 8 query heads per KV head


@pytest.mark.parametrize("cfg,slices", [(TINY128, (1, 2, 4)), (G8E, (1, 2, 4, 8))])
@pytest.mark.parametrize("merge", [1, 2, 3])
def test_engine_attn_head_slices_bit_identical(rf, orc, cfg, slices, merge):
    """Query-head slices per KV head (rfp4_debug_attn_head_split): each
    attention workgroup serves group/slices query heads of its KV head; the
    per-head arithmetic is unchanged, so tokens and logits are bit-identical
    for every slice count, with the splits merged by the second kernel (1), in
    the attention kernel by the last split (2) or from tagged states (3), and
    the tokens are the oracle's."""
    seed = 0x51CE
    prompt = [2, 9, 77, 401, 5, 6, 7]
    outs = []
    for hs in slices:
        rf.check(rf.load().rfp4_debug_attn_head_split(hs))
        rf.check(rf.load().rfp4_debug_attn_merge(merge))
        rf.debug_attn_chunk(cfg["max_seq"] // 6 + 1)  # 6 splits over the context
        try:
            eng = _engine(rf, cfg, seed)
        finally:
            rf.debug_attn_chunk(0)
            rf.check(rf.load().rfp4_debug_attn_merge(0))
            rf.check(rf.load().rfp4_debug_attn_head_split(0))
        toks = eng.generate(prompt, 0, 40)
        outs.append((np.array(toks), eng.logits()))
        eng.close()
    for t, l in outs[1:]:
        np.testing.assert_array_equal(t, outs[0][0])
        np.testing.assert_array_equal(l, outs[0][1])
    ref = orc.Model(cfg, seed)
    cpu, margins = ref.generate(prompt, 0, 40)
    assert list(outs[0][0]) == list(cpu), f"gpu {list(outs[0][0])}\ncpu {list(cpu)}\nmargins {margins}"


def _merge_engine(rf, cfg, seed, mode, chunk):
    rf.check(rf.load().rfp4_debug_attn_merge(mode))
    rf.debug_attn_chunk(chunk)
    try:
        return _engine(rf, cfg, seed)
    finally:
        rf.debug_attn_chunk(0)
        rf.check(rf.load().rfp4_debug_attn_merge(0))


@pytest.mark.parametrize("cfg", [dict(TINY128, max_seq=400), dict(G8E, max_seq=400)])
def test_engine_tagged_merge_bit_identical(rf, orc, cfg):
    """The tagged in-kernel merge (mode 3) sums in the merge kernel's order:
    tokens and logits bit-identical to mode 1 over contexts of 1 to 30 splits
    (10-token splits), and past the tagged merge's 32 splits (up to 34: the
    merge kernel takes over).  A second generation on the same engine at the same
    positions (the workspace then holds the first one's states under the
    same tags until the engine clears it) gives the oracle's tokens for its
    own prompt, and repeating the first prompt repeats its logits."""
    seed = 0x7A66
    chunk = 10
    ref = orc.Model(cfg, seed)
    p1, p2 = [2, 9, 77, 401, 5, 6, 7], [13, 600, 3, 3, 250]
    n1 = min(cfg["max_seq"] - len(p1) - 1, 330)
    a = _merge_engine(rf, cfg, seed, 1, chunk)
    b = _merge_engine(rf, cfg, seed, 3, chunk)
    ta, tb = a.generate(p1, 0, n1), b.generate(p1, 0, n1)
    la, lb = a.logits(), b.logits()
    np.testing.assert_array_equal(np.array(ta), np.array(tb))
    np.testing.assert_array_equal(la, lb)
    # second generation at the same positions, another prompt
    t2 = b.generate(p2, 0, 40)
    cpu2, margins = ref.generate(p2, 0, 40)
    assert list(t2) == list(cpu2), f"gpu {list(t2)}\ncpu {list(cpu2)}\nmargins {margins}"
    np.testing.assert_array_equal(np.array(b.generate(p1, 0, n1)), np.array(ta))
    np.testing.assert_array_equal(b.logits(), lb)
    cpu1, margins = ref.generate(p1, 0, 40)
    assert list(ta[:40]) == list(cpu1), f"gpu {list(ta[:40])}\ncpu {list(cpu1)}\nmargins {margins}"
    a.close()
    b.close()
