"""The fused q|k|v GEMV + decode attention launch (device/qkva.h): one launch
per layer in place of the GEMV launch and the attention launch of
llama_run/src/main.rs:513-529.  Its outputs are computed with the two
launches' arithmetic, so tokens and logits must be bit-identical to an
engine made with the fusion off (rfp4_debug_qkv_attn(1)), in every merge
regime of the attention splits (one split, the last-arriver merge up to 8,
tagged states up to 32, the merge kernel beyond; mode 2 fuses at every split
count, the default only one-split steps) and every query-head slice count,
and the tokens must be the oracle's."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# the two shapes the fused kernels are compiled for: K = 2048 with head_dim 64
# (TinyLlama, Llama-3.2-1B widths) and K = 4096 with head_dim 128 (Llama-3-8B)
W64 = dict(dim=2048, n_layers=2, n_heads=32, n_kv_heads=4, head_dim=64, ffn=512, vocab=1024,
           theta=10000.0, eps=1e-5, max_seq=400)
W128 = dict(dim=4096, n_layers=2, n_heads=32, n_kv_heads=8, head_dim=128, ffn=512, vocab=1024,
            theta=500000.0, eps=1e-5, max_seq=400)


def _engine(rf, cfg, seed, fused, chunk=0, slices=0):
    c = {k: v for k, v in cfg.items() if k != "max_seq"}
    rf.check(rf.load().rfp4_debug_qkv_attn(2 if fused else 1))
    rf.check(rf.load().rfp4_debug_attn_head_split(slices))
    rf.debug_attn_chunk(chunk)
    try:
        return rf.Engine(rf.model_config(max_seq=cfg["max_seq"], **c), seed)
    finally:
        rf.debug_attn_chunk(0)
        rf.check(rf.load().rfp4_debug_attn_head_split(0))
        rf.check(rf.load().rfp4_debug_qkv_attn(0))


def _kernels(eng, prompt):
    eng.begin(prompt, 0, len(prompt) + 4)
    names = {n for n, _ in eng.time_steps(1)}
    return names


@pytest.mark.parametrize("cfg", [W64, W128], ids=["hd64", "hd128"])
@pytest.mark.parametrize("chunk", [0, 60, 12, 8], ids=["auto", "le8", "tagged", "kernel"])
def test_fused_bit_identical_to_two_launches(rf, orc, cfg, chunk):
    """Greedy tokens and the last step's logits of the fused launch equal the
    two-launch step bit for bit; the fused kernel is the one that ran; the
    tokens are the oracle's.  Chunks: automatic (one split at these
    contexts), 60 tokens (up to 6 splits, merged by the last split), 12 (up
    to 30: tagged states), 8 (up to 45: the merge kernel past 32)."""
    seed = 0x9A11
    prompt = [3, 17, 200, 999, 5, 64, 7, 81]
    n_new = 60 if chunk != 8 else 300  # the merge-kernel regime needs more than 32 splits
    a = _engine(rf, cfg, seed, fused=False, chunk=chunk)
    b = _engine(rf, cfg, seed, fused=True, chunk=chunk)
    ka, kb = _kernels(a, prompt), _kernels(b, prompt)
    assert not any(n.startswith("rfp4_qkva") for n in ka), ka
    assert any(n.startswith("rfp4_qkva") for n in kb), kb
    ta, tb = a.generate(prompt, 0, n_new), b.generate(prompt, 0, n_new)
    np.testing.assert_array_equal(ta, tb)
    np.testing.assert_array_equal(a.logits(), b.logits())
    ref = orc.Model(cfg, seed)
    cpu, margins = ref.generate(prompt, 0, 40)
    assert list(tb[:40]) == list(cpu), f"gpu {list(tb[:40])}\ncpu {list(cpu)}\nmargins {margins}"
    a.close()
    b.close()
    ref.close()


@pytest.mark.parametrize("cfg,slices", [(W64, (1, 2, 4, 8)), (W128, (1, 2, 4))], ids=["hd64", "hd128"])
def test_fused_slices_bit_identical(rf, cfg, slices):
    """Every query-head slice count gives the two-launch tokens and logits
    (30-token splits: 2 to 3 splits at these contexts).  The engine fuses
    wherever the grid fits the device at once (a slice count whose kernel
    needs more than 256 VGPRs fits one workgroup per CU and may not); most
    slice counts here must take the fused launch."""
    seed = 0x51CF
    prompt = [2, 9, 77, 401, 5, 6, 7]
    base = _engine(rf, cfg, seed, fused=False, chunk=30)
    t0 = base.generate(prompt, 0, 50)
    l0 = base.logits()
    base.close()
    fused = []
    for hs in slices:
        e = _engine(rf, cfg, seed, fused=True, chunk=30, slices=hs)
        if any(n.startswith("rfp4_qkva") for n in _kernels(e, prompt)):
            fused.append(hs)
        np.testing.assert_array_equal(e.generate(prompt, 0, 50), t0, err_msg=f"slices {hs}")
        np.testing.assert_array_equal(e.logits(), l0, err_msg=f"slices {hs}")
        e.close()
    assert len(fused) >= len(slices) - 1, f"fused launch used for slices {fused} of {slices}"


def test_fused_repeat_generation_same_positions(rf, orc):
    """A second generation at the same positions (the tagged q|k|v words of the
    first one carry the same tags until begin clears them) gives the oracle's
    tokens for its own prompt, and the first prompt again repeats its logits."""
    cfg = W64
    seed = 0x7A67
    e = _engine(rf, cfg, seed, fused=True)
    p1, p2 = [2, 9, 77, 401, 5, 6, 7], [13, 600, 3, 3, 250]
    t1 = e.generate(p1, 0, 30)
    l1 = e.logits()
    t2 = e.generate(p2, 0, 30)
    ref = orc.Model(cfg, seed)
    cpu2, margins = ref.generate(p2, 0, 30)
    assert list(t2) == list(cpu2), f"gpu {list(t2)}\ncpu {list(cpu2)}\nmargins {margins}"
    np.testing.assert_array_equal(e.generate(p1, 0, 30), t1)
    np.testing.assert_array_equal(e.logits(), l1)
    e.close()
    ref.close()


def test_fused_eager_equals_graph(rf):
    """The fused launch in eager steps (no graph) equals its graph replays."""
    cfg = W128
    seed = 0xE6E6
    prompt = [4, 8, 15, 16, 23, 42]
    g = _engine(rf, cfg, seed, fused=True, chunk=12)
    tg = g.generate(prompt, 0, 40)
    lg = g.logits()
    g.use_graph(False)
    np.testing.assert_array_equal(g.generate(prompt, 0, 40), tg)
    np.testing.assert_array_equal(g.logits(), lg)
    g.close()


@pytest.mark.parametrize("cfg", [W64, W128], ids=["hd64", "hd128"])
def test_default_policy_fuses_one_split_steps(rf, cfg):
    """The default engine fuses the q|k|v GEMV and the attention for steps
    whose attention is one split and keeps two launches past that."""
    c = {k: v for k, v in cfg.items() if k != "max_seq"}
    rf.debug_attn_chunk(30)
    try:
        e = rf.Engine(rf.model_config(max_seq=cfg["max_seq"], **c), 0x5151)
    finally:
        rf.debug_attn_chunk(0)
    prompt = [2, 9, 77]
    e.begin(prompt, 0, 8)
    one = [n for n, _ in e.time_steps(1)]
    e.begin(prompt, 200, 8)  # 7 splits of 30 tokens
    many = [n for n, _ in e.time_steps(1)]
    assert any(n.startswith("rfp4_qkva") for n in one), one
    assert not any(n.startswith("rfp4_qkva") for n in many), many
    e.close()


@pytest.mark.parametrize("cfg", [W64, W128], ids=["hd64", "hd128"])
def test_device_wait_error_reported_and_cleared(rf, cfg):
    """Every device-side wait of the step reports to the engine's error word:
    the fused launch's q|k|v poll at one split (where no tagged merge runs),
    the tagged merge past 8 splits, and the plain split kernel.  The word is
    set from the host (no kernel times out): the next read of the tokens
    fails with RFP4_E_WAIT, also from llama_engine_time_steps, and the next
    generation starts clean."""
    RFP4_E_WAIT = -9
    eng = _engine(rf, cfg, 0x9A12, fused=True, chunk=12)
    one = eng.debug_wait(1)
    assert one["fused"] and one["err_wired"] and one["checked"], one
    for ns in (2, 9, 20):
        w = eng.debug_wait(ns)
        assert w["err_wired"] and w["checked"], (ns, w)
    prompt = [3, 17, 200, 999]
    ref = eng.generate(prompt, 0, 8)
    eng.begin(prompt, 0, len(prompt) + 8)
    eng.run_steps(len(prompt) + 2)
    eng.debug_wait(1, set_error=True)
    with pytest.raises(rf.Rfp4Error) as ei:
        eng.read_ids(len(prompt) + 3)
    assert ei.value.code == RFP4_E_WAIT
    with pytest.raises(rf.Rfp4Error) as ei:
        eng.time_steps(1)
    assert ei.value.code == RFP4_E_WAIT
    # a new generation clears the word and reproduces the tokens
    np.testing.assert_array_equal(eng.generate(prompt, 0, 8), ref)
    eng.close()
