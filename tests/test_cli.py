"""Tokenizer-free text I/O: tok.py (the reference's tok/src/main.rs on the
same tokenizers library) and the llama_run command-line contract
(llama_run/src/main.rs:399-407, 536-587).  CPU: tok round trips, the CLI's
argument errors; GPU: llama_run's output ids against the oracle."""
import os
import re
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "rust-fp4-blackwell_amd")
TOK = os.path.join(PKG, "tok.py")
LLAMA_RUN = os.path.join(PKG, "llama_run")


def _tokenizer(path):
    """A small word-level tokenizer with a BOS post-processor, as TinyLlama's
    adds <s> (id 1) in front of every encoding."""
    from tokenizers import Tokenizer, models, pre_tokenizers, processors, decoders

    words = ["<unk>", "<s>", "</s>", "hello", "world", "the", "mi355x", "runs", "fp4", "fast", ","]
    tk = Tokenizer(models.WordLevel({w: i for i, w in enumerate(words)}, unk_token="<unk>"))
    tk.pre_tokenizer = pre_tokenizers.Sequence([pre_tokenizers.Whitespace()])
    tk.post_processor = processors.TemplateProcessing(single="<s> $A", special_tokens=[("<s>", 1)])
    tk.decoder = decoders.WordPiece(prefix="##")
    tk.save(path)
    return tk


def _tok(args, tokenizer):
    env = dict(os.environ, RFP4_TOKENIZER=tokenizer)
    return subprocess.run([sys.executable, TOK] + args, capture_output=True, text=True, env=env, timeout=60)


def test_tok_encode_decode(tmp_path):
    path = str(tmp_path / "tokenizer.json")
    tk = _tokenizer(path)
    r = _tok(["encode", "hello", "world", ",", "the", "mi355x", "runs", "fp4", "fast"], path)
    assert r.returncode == 0, r.stderr
    ids = [int(s) for s in r.stdout.split()]
    assert ids == tk.encode("hello world , the mi355x runs fp4 fast").ids
    assert ids[0] == 1 and ids[1:3] == [3, 4]           # BOS first
    r = _tok(["decode"] + [str(i) for i in ids], path)
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() == tk.decode(ids, skip_special_tokens=False)
    assert "hello world" in r.stdout and "<s>" in r.stdout   # special tokens kept, as the reference
    r = _tok(["encode", "hello", "zebra"], path)
    assert [int(s) for s in r.stdout.split()] == [1, 3, 0]   # unknown word -> <unk>


def test_tok_usage(tmp_path):
    r = _tok([], str(tmp_path / "none.json"))
    assert r.returncode == 0 and "usage: tok encode" in r.stderr


def test_llama_run_rejects_bad_ids():
    assert os.path.exists(LLAMA_RUN), "build first (make -C rust-fp4-blackwell_amd)"
    r = subprocess.run([LLAMA_RUN, "1", "x2"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "not a token id" in r.stderr
    r = subprocess.run([LLAMA_RUN], capture_output=True, text=True, timeout=60,
                       env=dict(os.environ, PROMPT_IDS="1 two"))
    assert r.returncode == 2 and "PROMPT_IDS" in r.stderr
    r = subprocess.run([LLAMA_RUN, "1"], capture_output=True, text=True, timeout=60,
                       env=dict(os.environ, RFP4_PRESET="gpt2"))
    assert r.returncode == 2 and "unknown preset" in r.stderr


def _parse(stdout):
    pm = re.search(r"^prompt ids: ((?:\d+ )*)$", stdout, re.M)
    om = re.search(r"^output ids: ((?:\d+ )*)$", stdout, re.M)
    assert pm and om, stdout
    return [int(s) for s in pm.group(1).split()], [int(s) for s in om.group(1).split()]


TINY = dict(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=1024,
            theta=10000.0, eps=1e-5, max_seq=2048)


@pytest.mark.gpu
def test_llama_run_contract_matches_oracle(rf, orc, tmp_path):
    """llama_run on a packed tiny model: the prompt from the arguments or
    PROMPT_IDS, greedy tokens identical to the oracle's, stopping after the
    first EOS (included) or max_new tokens."""
    seed = 0x51
    c = {k: v for k, v in TINY.items() if k != "max_seq"}
    eng = rf.Engine(rf.model_config(max_seq=2048, **c), seed)
    pack = str(tmp_path / "tiny.rfp4")
    eng.save(pack)
    eng.close()
    ref = orc.Model(TINY, seed)
    prompt = [1, 15, 300, 42]
    want, _ = ref.generate(prompt, 0, 40)
    want = [int(t) for t in want]
    eos = want[12]  # a token the run produces: the stop rule is exercised
    cut = want[: want.index(eos) + 1]
    env = dict(os.environ, RFP4_MODEL=pack, RFP4_EOS=str(eos), RFP4_MAX_NEW="40")
    print("llama_run with EOS", eos, flush=True)
    r = subprocess.run([LLAMA_RUN] + [str(t) for t in prompt], capture_output=True, text=True, env=env, timeout=120)
    assert r.returncode == 0, r.stderr
    p, out = _parse(r.stdout)
    assert p == prompt and out == cut
    assert "gen: " in r.stdout and "tokens/sec" in r.stdout
    # PROMPT_IDS path, no EOS in range: exactly max_new tokens
    env = dict(os.environ, RFP4_MODEL=pack, PROMPT_IDS=" ".join(map(str, prompt)), RFP4_EOS="100000",
               RFP4_MAX_NEW="40")
    r = subprocess.run([LLAMA_RUN], capture_output=True, text=True, env=env, timeout=120)
    assert r.returncode == 0, r.stderr
    p, out = _parse(r.stdout)
    assert p == prompt and out == want
    ref.close()


LLAMA_RUN_ASAN = os.path.join(PKG, "llama_run_asan")


@pytest.mark.gpu
def test_llama_run_graph_replays_under_host_asan(tmp_path):
    """The engine's host code under AddressSanitizer + UBSan (llama_run_asan
    over librfp4_asan.so; the gfx950 code object is the same): synthetic
    TinyLlama weights, the prompt, then greedy steps replayed as step graphs
    (capture, instantiation, replays with the device cursor, engine and
    runtime teardown through rfp4_shutdown).  No sanitizer report, and the
    tokens equal the plain build's."""
    if not os.path.exists(LLAMA_RUN_ASAN):
        pytest.skip("sanitizer build not present (make -C rust-fp4-blackwell_amd llama_run_asan)")
    base = dict(os.environ, RFP4_SEED="7", RFP4_MAX_NEW="48", RFP4_EOS="100000")
    # the harness may preload a library ahead of the ASan runtime; leaks of the
    # HIP runtime at exit are not this library's
    san = dict(base, ASAN_OPTIONS="verify_asan_link_order=0:detect_leaks=0:abort_on_error=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    prompt = ["1", "15043", "2787"]
    print("llama_run (plain) TinyLlama synthetic", flush=True)
    r0 = subprocess.run([LLAMA_RUN] + prompt, capture_output=True, text=True, env=base, timeout=300)
    assert r0.returncode == 0, r0.stderr
    print("llama_run_asan TinyLlama synthetic", flush=True)
    r1 = subprocess.run([LLAMA_RUN_ASAN] + prompt, capture_output=True, text=True, env=san, timeout=300)
    assert "AddressSanitizer" not in r1.stderr and "runtime error" not in r1.stderr, r1.stderr[-4000:]
    assert r1.returncode == 0, r1.stderr[-4000:]
    assert _parse(r1.stdout) == _parse(r0.stdout)
    assert len(_parse(r0.stdout)[1]) == 48
