"""Writes the golden fixtures of tests/golden/ from the CPU oracle.

Usage: python tests/golden/make_golden.py [small|tinyllama|llama3_8b|all]

The reference holds no stored vectors (its examples regenerate inputs from
seeds), so every fixture here is produced by the oracle on the BASELINE
configs' seeded synthetic inputs; the oracle itself is pinned by
tests/test_oracle*.py.  Fixtures are small: hashes of large tensors, outputs
of the small configs, and greedy token sequences with their top-1 minus top-2
logit margins.
"""
import hashlib
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import pyoracle as orc  # noqa: E402

TINYLLAMA = dict(dim=2048, n_layers=22, n_heads=32, n_kv_heads=4, head_dim=64, ffn=5632, vocab=32000,
                 theta=10000.0, eps=1e-5, max_seq=272)
LLAMA3_8B = dict(dim=4096, n_layers=32, n_heads=32, n_kv_heads=8, head_dim=128, ffn=14336, vocab=128256,
                 theta=500000.0, eps=1e-5, max_seq=4096 + 128)


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def config1_inputs(n=2048, k=2048, seed=0x12345678):
    """codes uniform over the 16 codes (xorshift32 words,
    8 codes each), E8M0 exponents uniform in [-6, 2], x ~ N(0,1) (Irwin-Hall
    from xorshift32 pairs)."""
    words, st = orc.xorshift32(seed, n * k // 8)
    codes = words.view(np.uint8).copy()
    r, st = orc.xorshift32(st, n * k // 32)
    scales = (127 - 6 + (r % 9)).astype(np.uint8)
    r2, st = orc.xorshift32(st, 2 * k)
    u = r2.astype(np.uint64).reshape(k, 2)
    x = np.array([orc.ih4_normal_from_u64(int((a << 32) | b), 1.0) for a, b in u], dtype=np.float32)
    return codes, scales, x


def small():
    codes, scales, x = config1_inputs()
    y = orc.gemv_e8m0(2048, 2048, codes, scales, x)
    y64, absy = orc.gemv_e8m0_f64(2048, 2048, codes, scales, x)
    np.savez_compressed(os.path.join(HERE, "config1_gemv.npz"), y=y, y64=y64, absy=absy,
                        sha_codes=sha(codes), sha_scales=sha(scales), sha_x=sha(x))
    # config 2 kernels at the reference harness seeds
    d = {}
    r, st = orc.xorshift32(0x9E3779B9, 2048)
    xn = (((r % 2001).astype(np.float32) - 1000.0) / 500.0).astype(np.float32)
    r, st = orc.xorshift32(st, 2048)
    wn = (0.5 + (r % 1000).astype(np.float32) / 1000.0).astype(np.float32)
    d["rmsnorm_y"] = orc.rmsnorm(xn, wn, 1e-5)
    r, _ = orc.xorshift32(0x13579BDF, 32 * 64)
    q = (((r % 2001).astype(np.float32) - 1000.0) / 500.0).astype(np.float32)
    c, s = orc.rope_table(2048, 64, 10000.0)
    d["rope_pos2047"] = orc.rope(q, 32, 64, c[2047 * 32:2048 * 32], s[2047 * 32:2048 * 32])
    r, _ = orc.xorshift32(0xABCD1234, 32 * 64 + 2 * 512 * 8 * 64)
    vals = (((r % 2001).astype(np.float32) - 1000.0) / 700.0).astype(np.float32)
    d["attn_harness_out"] = orc.attn_decode(32, 8, 64, 512, vals[:2048], vals[2048:2048 + 262144],
                                            vals[2048 + 262144:], 8 * 64, 64)
    np.savez_compressed(os.path.join(HERE, "config2_kernels.npz"), **d)
    print("small fixtures written")


def model_tokens(name, cfg, seed, prompt, pos0, n_new, prefill=None):
    orc.set_threads(0)
    t0 = time.time()
    m = orc.Model(cfg, seed)
    if prefill:
        m.prefill_kv(*prefill)
    hashes = {"lm_codes": sha(m.codes(-1, 0)), "l0_wq_codes": sha(m.codes(0, 0)),
              "l0_wd_scales": sha(m.scales(0, 6)), "embed": sha(m.embed())}
    t1 = time.time()
    toks, margins = m.generate(prompt, pos0, n_new)
    t2 = time.time()
    out = dict(config=cfg, seed=seed, prompt=[int(t) for t in prompt], pos0=pos0, n_new=n_new,
               prefill=list(prefill) if prefill else None, tokens=[int(t) for t in toks],
               margins=[float(v) for v in margins], hashes=hashes,
               oracle_seconds=dict(setup=round(t1 - t0, 1), generate=round(t2 - t1, 1),
                                   threads=orc.lib().orc_get_threads()))
    with open(os.path.join(HERE, f"{name}_tokens.json"), "w") as f:
        json.dump(out, f, indent=1)
    m.close()
    print(f"{name}: {len(toks)} tokens in {t2 - t1:.1f}s (setup {t1 - t0:.1f}s)")


def tinyllama():
    """16-token random prompt, 256 greedy steps from pos 0."""
    r, _ = orc.xorshift32(0xC0DE, 16)
    model_tokens("tinyllama", TINYLLAMA, 0x11B, (r % 32000).astype(np.uint32), 0, 256)


def llama3_8b():
    """context pre-filled to 4096, 128 greedy steps from
    token 1 at position 4096."""
    model_tokens("llama3_8b", LLAMA3_8B, 0x8B8B, np.array([1], np.uint32), 4096, 128, prefill=(0x4B56, 4096))


if __name__ == "__main__":
    what = sys.argv[1] if len(sys.argv) > 1 else "small"
    for w in (["small", "tinyllama", "llama3_8b"] if what == "all" else [what]):
        {"small": small, "tinyllama": tinyllama, "llama3_8b": llama3_8b}[w]()
