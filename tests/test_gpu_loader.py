"""Real-weight loading on the device: a safetensors checkpoint with the Llama
tensor names (the reference's loader, llama_run/src/main.rs:413-460) into
the engine, against the CPU oracle loaded with the same tensors.  The
projections are quantized by the OCP MX rules on both sides (bit-exact),
norm weights are held as fp16 (exact for these gains) and embeddings keep
the checkpoint's 16-bit values; greedy tokens must be identical.  Checkpoints are synthetic (no real weights in the image)."""
import numpy as np
import pytest

import st_writer as stw

pytestmark = pytest.mark.gpu

TINY = dict(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=1024,
            theta=10000.0, eps=1e-5, max_seq=64)
TINY128 = dict(dim=512, n_layers=2, n_heads=8, n_kv_heads=2, head_dim=128, ffn=1024, vocab=2048,
               theta=500000.0, eps=1e-5, max_seq=128)

PROJ = ("self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
        "self_attn.o_proj.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight")


def _shapes(c):
    qd, kvd = c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"]
    return [(qd, c["dim"]), (kvd, c["dim"]), (kvd, c["dim"]), (c["dim"], qd),
            (c["ffn"], c["dim"]), (c["ffn"], c["dim"]), (c["dim"], c["ffn"])]


def make_checkpoint(path, c, seed, dtype="BF16", tied=False, norm_dtype=None):
    """Write a checkpoint; return (f32 values, 16-bit bits for norms/embeds as
    the engine should hold them, embed_bf16)."""
    rng = np.random.default_rng(seed)
    norm_dtype = norm_dtype or dtype
    tensors, f32 = {}, {}

    def put(name, values, dt):
        raw = stw.as_stored(dt, values)
        tensors[name] = (dt, raw)
        f32[name] = stw.widen(dt, raw)

    for l in range(c["n_layers"]):
        for name, shape in zip(PROJ, _shapes(c)):
            put(f"model.layers.{l}.{name}", 0.02 * rng.standard_normal(shape), dtype)
        put(f"model.layers.{l}.input_layernorm.weight", 1 + 0.1 * rng.standard_normal(c["dim"]), norm_dtype)
        put(f"model.layers.{l}.post_attention_layernorm.weight", 1 + 0.1 * rng.standard_normal(c["dim"]), norm_dtype)
    put("model.norm.weight", 1 + 0.1 * rng.standard_normal(c["dim"]), norm_dtype)
    put("model.embed_tokens.weight", 0.02 * rng.standard_normal((c["vocab"], c["dim"])), norm_dtype)
    if not tied:
        put("lm_head.weight", 0.02 * rng.standard_normal((c["vocab"], c["dim"])), dtype)
    stw.write(path, tensors, metadata={"format": "pt"})
    # norms: fp16 (numpy's conversion rounds to nearest even, as the engine);
    # embeddings: as stored when BF16 / F16, F32 rounded to bf16
    half = {}
    for n in tensors:
        if n.endswith("norm.weight"):
            half[n] = f32[n].astype(np.float16).view(np.uint16).reshape(-1)
    dt, raw = tensors["model.embed_tokens.weight"]
    embed_bf16 = dt != "F16"
    half["model.embed_tokens.weight"] = (raw.reshape(-1).astype(np.uint16) if dt in ("BF16", "F16")
                                         else stw.bf16_bits(f32["model.embed_tokens.weight"]).reshape(-1))
    return f32, half, embed_bf16


def _cfg(rf, c):
    d = {k: v for k, v in c.items() if k != "max_seq"}
    return rf.model_config(max_seq=c["max_seq"], **d)


def _oracle(orc, c, f32, half, embed_bf16):
    m = orc.Model(c, 1)
    m.load_checkpoint(f32, half, embed_bf16)
    return m


def _check_same(eng, ref, c, prompt, n_new):
    gpu = eng.generate(prompt, 0, n_new)
    cpu, margins = ref.generate(prompt, 0, n_new)
    assert list(gpu) == list(cpu), f"gpu {list(gpu)}\ncpu {list(cpu)}\nmargins {margins}"


@pytest.mark.parametrize("c,dtype,norm_dtype,tied", [
    (TINY, "BF16", None, False),
    (TINY, "F16", None, False),
    (TINY, "F32", None, True),
    (TINY128, "BF16", None, True),
    (TINY, "BF16", "F32", False),
])
def test_checkpoint_tokens_match_oracle(rf, orc, tmp_path, c, dtype, norm_dtype, tied):
    path = str(tmp_path / "model.safetensors")
    f32, half, embed_bf16 = make_checkpoint(path, c, seed=len(dtype) + tied, dtype=dtype, tied=tied,
                                           norm_dtype=norm_dtype)
    print(f"checkpoint {dtype}/{norm_dtype} tied={tied} dim={c['dim']}", flush=True)
    eng = rf.Engine.from_safetensors(_cfg(rf, c), path)
    assert eng.embed_bf16() == embed_bf16
    ref = _oracle(orc, c, f32, half, embed_bf16)
    for layer in range(c["n_layers"]):
        for p in range(7):
            cg, sg = eng.weight_host(layer, p)
            np.testing.assert_array_equal(cg, ref.codes(layer, p))
            np.testing.assert_array_equal(sg, ref.scales(layer, p))
    cg, sg = eng.weight_host(-1, 0)
    np.testing.assert_array_equal(cg, ref.codes(-1, 0))
    np.testing.assert_array_equal(sg, ref.scales(-1, 0))
    _check_same(eng, ref, c, [1, 17, 300, 42, 7], 20)
    eng.close()
    ref.close()


def test_checkpoint_prefill_with_bf16_embeddings(rf, orc, tmp_path):
    """The batched prefill gathers bf16 embedding rows too."""
    c = TINY128
    path = str(tmp_path / "model.safetensors")
    f32, half, embed_bf16 = make_checkpoint(path, c, seed=9)
    eng = rf.Engine.from_safetensors(_cfg(rf, c), path)
    ref = _oracle(orc, c, f32, half, embed_bf16)
    prompt = list(range(5, 45))
    tok = eng.prefill(prompt, 0)
    rtok, rlog = ref.prefill(prompt, 0, want_logits=True)
    assert tok == rtok
    lg = eng.logits()
    assert np.max(np.abs(lg - rlog)) <= 2e-2 * np.max(np.abs(rlog))
    eng.close()
    ref.close()


def test_packed_cache_round_trip(rf, orc, tmp_path):
    """save() then load(): the same weights bit for bit, the same format flag
    and the same tokens, at another max_seq."""
    c = TINY
    path = str(tmp_path / "model.safetensors")
    make_checkpoint(path, c, seed=5)
    eng = rf.Engine.from_safetensors(_cfg(rf, c), path)
    pack = str(tmp_path / "model.rfp4")
    eng.save(pack)
    prompt = [3, 9, 27, 81]
    want = eng.generate(prompt, 0, 16)
    eng2 = rf.Engine.load(pack, max_seq=100)
    assert eng2.cfg.max_seq == 100 and eng2.cfg.dim == c["dim"] and eng2.embed_bf16()
    for layer in (-1, 0, 1):
        for p in (range(7) if layer >= 0 else [0]):
            a, b = eng.weight_host(layer, p), eng2.weight_host(layer, p)
            np.testing.assert_array_equal(a[0], b[0])
            np.testing.assert_array_equal(a[1], b[1])
    assert list(eng2.generate(prompt, 0, 16)) == list(want)
    eng.close()
    eng2.close()


def test_checkpoint_errors(rf, tmp_path):
    c = TINY
    path = str(tmp_path / "model.safetensors")
    make_checkpoint(path, c, seed=3)
    bad = dict(c, ffn=1024)                       # shapes do not match the config
    with pytest.raises(rf.Rfp4Error) as e:
        rf.Engine.from_safetensors(_cfg(rf, bad), path)
    assert e.value.code == -2 and b"mlp.gate_proj.weight" in rf.load().rfp4_last_error()
    more = dict(c, n_layers=3)                    # a layer the checkpoint lacks
    with pytest.raises(rf.Rfp4Error) as e:
        rf.Engine.from_safetensors(_cfg(rf, more), path)
    assert b"model.layers.2." in rf.load().rfp4_last_error()
    with pytest.raises(rf.Rfp4Error):
        rf.Engine.from_safetensors(_cfg(rf, c), str(tmp_path / "missing.safetensors"))
    junk = str(tmp_path / "junk.rfp4")
    open(junk, "wb").write(b"not a pack")
    with pytest.raises(rf.Rfp4Error):
        rf.Engine.load(junk, 64)
