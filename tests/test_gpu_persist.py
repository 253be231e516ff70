"""Persistent decode (every layer of a step in one cooperative launch, grid
barriers between the stages; llama_engine_use_persistent) against the graph
step and the CPU oracle, at the Llama-3-8B widths it is compiled for.

The persistent step runs the stand-alone kernels' arithmetic (GEMV rows,
RMSNorm, attention) and merges attention splits in the merge kernel's
summation order, so past 8 splits its logits are bit-identical to the graph
step's; at 2-8 splits the graph step merges in the attention kernel in
another order (both within the attention bar), at one split there is no
merge."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# Llama-3-8B widths, two layers, a small vocabulary; max_seq 4224 gives the
# 8B configuration's split plan (144-token splits, 30 at most)
W8B = dict(dim=4096, n_layers=2, n_heads=32, n_kv_heads=8, head_dim=128, ffn=14336, vocab=2048,
           theta=500000.0, eps=1e-5)
MAX_SEQ = 4224


def _engine(rf, seed, n_layers=2):
    cfg = dict(W8B, n_layers=n_layers)
    return rf.Engine(rf.model_config(max_seq=MAX_SEQ, **cfg), seed)


def _run(eng, persistent, prompt, pos0, n_new, kv=None):
    eng.use_persistent(persistent)
    if kv:
        eng.prefill_kv(*kv)
    toks = eng.generate(prompt, pos0, n_new)
    return np.array(toks), eng.logits()


def test_persistent_available_for_8b_widths_off_by_default(rf):
    eng = _engine(rf, 1)
    assert not eng.persistent
    eng.use_persistent(True)
    assert eng.persistent
    eng.use_persistent(False)
    assert not eng.persistent
    eng.close()


def test_persistent_refused_elsewhere(rf):
    cfg = dict(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=1024, theta=1e4, eps=1e-5)
    eng = rf.Engine(rf.model_config(max_seq=64, **cfg), 1)
    assert not eng.persistent
    with pytest.raises(rf.Rfp4Error) as e:
        eng.use_persistent(True)
    assert e.value.code == -2
    eng.close()


@pytest.mark.parametrize("pos0,prompt", [(4096, [1]), (4000, [7, 99, 5])])
def test_persistent_bit_identical_to_graph_past_8_splits(rf, pos0, prompt):
    """Context ~4096 (29-30 splits): tokens and the last step's logits
    bit-identical to the graph step on the same weights and K/V."""
    print(f"persistent vs graph at pos0 {pos0}", flush=True)
    seed = 0x8B00 + pos0
    eng = _engine(rf, seed)
    kv = (seed ^ 0x55, pos0)
    tp, lp = _run(eng, True, prompt, pos0, 12, kv)
    tg, lg = _run(eng, False, prompt, pos0, 12, kv)
    np.testing.assert_array_equal(tp, tg)
    np.testing.assert_array_equal(lp, lg)
    eng.close()


@pytest.mark.parametrize("pos0,n_new", [(0, 8), (700, 6), (1300, 6)])
def test_persistent_tokens_match_oracle(rf, orc, pos0, n_new):
    """1 split (a fresh prompt), 5-6 splits and 9-10 splits: greedy tokens
    identical to the oracle's decode on the same weights and K/V."""
    print(f"persistent vs oracle at pos0 {pos0}", flush=True)
    seed = 0x9A00 + pos0
    cfg = dict(W8B, max_seq=MAX_SEQ)
    eng = _engine(rf, seed)
    ref = orc.Model(cfg, seed)
    prompt = [3, 1, 4, 1, 5][: 5 if pos0 == 0 else 2]
    kv = (seed ^ 0x77, pos0) if pos0 else None
    if kv:
        ref.prefill_kv(*kv)
    tp, lp = _run(eng, True, prompt, pos0, n_new, kv)
    cpu, margins = ref.generate(prompt, pos0, n_new)
    assert list(tp) == list(cpu), f"gpu {list(tp)}\ncpu {list(cpu)}\nmargins {margins}"
    eng.close()


def test_persistent_graph_within_attention_bar_at_few_splits(rf):
    """Context ~600 (5 splits): the graph step merges in the attention kernel
    in another order; tokens equal and logits within 1e-4 of their range."""
    seed = 0x5151
    eng = _engine(rf, seed)
    kv = (seed, 600)
    tp, lp = _run(eng, True, [11, 12], 600, 8, kv)
    tg, lg = _run(eng, False, [11, 12], 600, 8, kv)
    np.testing.assert_array_equal(tp, tg)
    assert np.max(np.abs(lp - lg)) <= 1e-4 * np.max(np.abs(lg))
    eng.close()


def test_persistent_harness_repeatable(rf):
    """The same steps twice (same K/V, same prompt): bit-identical logits,
    and the barrier generations carry over between launches."""
    seed = 0x7777
    eng = _engine(rf, seed)
    kv = (seed, 3000)
    t1, l1 = _run(eng, True, [5], 3000, 20, kv)
    t2, l2 = _run(eng, True, [5], 3000, 20, kv)
    np.testing.assert_array_equal(t1, t2)
    np.testing.assert_array_equal(l1, l2)
    eng.close()
