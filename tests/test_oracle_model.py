"""Pins the oracle's decode loop (oracle.c orc_model_*) against an
independent float64 numpy Llama decoder run on the same packed weights:
layer order, GQA head mapping, rotate-half RoPE, fp16 KV rounding, SwiGLU and
the final norm + LM head (llama_run/src/main.rs:492-536).  CPU only."""
import math

import numpy as np

FP4 = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6], np.float64)
CFG = dict(dim=128, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=32, ffn=256, vocab=512,
           theta=10000.0, eps=1e-5, max_seq=32)


def _deq(orc, codes, scales, n, k):
    c = orc.unpack(codes).reshape(n, k)
    v = np.where(c & 8, -1.0, 1.0) * FP4[c & 7]
    return v * np.repeat(np.ldexp(1.0, scales.astype(np.int64) - 127).reshape(n, k // 32), 32, axis=1)


def _deq_f32(orc, codes, scales, n, k):
    """E2M1 codes times the reference's f32 per-32 scales (fp4_gemv/src/main.rs:136-142)."""
    c = orc.unpack(codes).reshape(n, k)
    v = np.where(c & 8, -1.0, 1.0) * FP4[c & 7]
    return v * np.repeat(np.asarray(scales, np.float64).reshape(n, k // 32), 32, axis=1)


def _f16(a):
    return np.asarray(a).view(np.float16).astype(np.float64)


class NumpyLlama:
    def __init__(self, orc, m, cfg):
        c = self.c = cfg
        qd, kvd = c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"]
        shapes = [(qd, c["dim"]), (kvd, c["dim"]), (kvd, c["dim"]), (c["dim"], qd),
                  (c["ffn"], c["dim"]), (c["ffn"], c["dim"]), (c["dim"], c["ffn"])]
        self.f32kv = c.get("kv_format", 0) == 1
        deq = _deq_f32 if c.get("scale_format", 0) == 1 else _deq
        self.W = [[deq(orc, m.codes(l, p), m.scales(l, p), *shapes[p]) for p in range(7)]
                  for l in range(c["n_layers"])]
        self.lm = deq(orc, m.codes(-1, 0), m.scales(-1, 0), c["vocab"], c["dim"])
        self.emb = _f16(m.embed()).reshape(c["vocab"], c["dim"])
        self.na = [_f16(m.norm(l, 0)) for l in range(c["n_layers"])]
        self.nf = [_f16(m.norm(l, 1)) for l in range(c["n_layers"])]
        self.nfinal = _f16(m.norm(-1, 0))
        self.K = [np.zeros((c["max_seq"], c["n_kv_heads"], c["head_dim"])) for _ in range(c["n_layers"])]
        self.V = [np.zeros_like(k) for k in self.K]

    def _norm(self, x, w):
        return x / np.sqrt(np.mean(x * x) + self.c["eps"]) * w

    def _rope(self, v, nh, pos):
        hd = self.c["head_dim"]
        half = hd // 2
        j = np.arange(half)
        ang = pos * (1.0 / np.power(self.c["theta"], 2.0 * j / hd))
        cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)  # f32 table
        v = v.reshape(nh, hd)
        a, b = v[:, :half], v[:, half:]
        return np.concatenate([a * cs - b * sn, b * cs + a * sn], axis=1)

    def step(self, tok, pos):
        return self.layers(self.emb[tok].copy(), pos)

    def _kv(self, v):
        v = v.astype(np.float32)
        return (v if self.f32kv else v.astype(np.float16)).astype(np.float64)

    def layers(self, x, pos):
        """The layers and LM head on activation x; returns (argmax, logits)
        and leaves the final residual stream in self.x."""
        c = self.c
        nh, nkv, hd = c["n_heads"], c["n_kv_heads"], c["head_dim"]
        for l in range(c["n_layers"]):
            Wq, Wk, Wv, Wo, Wg, Wu, Wd = self.W[l]
            h = self._norm(x, self.na[l])
            q = self._rope(Wq @ h, nh, pos)
            k = self._rope(Wk @ h, nkv, pos)
            # fp16 KV cache (round to nearest even via numpy's IEEE conversion), or f32
            self.K[l][pos] = self._kv(k)
            self.V[l][pos] = self._kv((Wv @ h).reshape(nkv, hd))
            att = np.zeros((nh, hd))
            for hh in range(nh):
                g = hh // (nh // nkv)
                s = self.K[l][:pos + 1, g] @ q[hh] / math.sqrt(hd)
                p = np.exp(s - s.max())
                att[hh] = (p / p.sum()) @ self.V[l][:pos + 1, g]
            x = x + Wo @ att.reshape(-1)
            h = self._norm(x, self.nf[l])
            gate, up = Wg @ h, Wu @ h
            x = x + Wd @ (gate / (1 + np.exp(-gate)) * up)
        self.x = x
        logits = self.lm @ self._norm(x, self.nfinal)
        return int(np.argmax(logits)), logits


    def prefill(self, orc, toks, pos0):
        """Batched prefill with MXFP4 activations: every projection input row
        quantized (OCP rules, the pinned quantizer), products in float64."""
        c = self.c
        nh, nkv, hd = c["n_heads"], c["n_kv_heads"], c["head_dim"]

        def q(rows):
            r = np.ascontiguousarray(rows, np.float32)
            codes, scales = orc.quant_mx(r)
            return _deq(orc, codes, scales, r.shape[0], r.shape[1])

        X = np.stack([self.emb[t] for t in toks])
        n = len(toks)
        for l in range(c["n_layers"]):
            Wq, Wk, Wv, Wo, Wg, Wu, Wd = self.W[l]
            Hq = q(np.stack([self._norm(x, self.na[l]) for x in X]))
            Q = (Hq @ Wq.T).astype(np.float32)
            K = (Hq @ Wk.T).astype(np.float32)
            V = (Hq @ Wv.T).astype(np.float32)
            att = np.zeros((n, nh * hd))
            for i in range(n):
                pos = pos0 + i
                k = self._rope(K[i].astype(np.float64), nkv, pos)
                self.K[l][pos] = k.astype(np.float32).astype(np.float16).astype(np.float64)
                self.V[l][pos] = V[i].reshape(nkv, hd).astype(np.float16).astype(np.float64)
            for i in range(n):
                pos = pos0 + i
                qi = self._rope(Q[i].astype(np.float64), nh, pos)
                for hh in range(nh):
                    g = hh // (nh // nkv)
                    sc = self.K[l][:pos + 1, g] @ qi[hh] / math.sqrt(hd)
                    p = np.exp(sc - sc.max())
                    att[i, hh * hd:(hh + 1) * hd] = (p / p.sum()) @ self.V[l][:pos + 1, g]
            X = X + q(att) @ Wo.T
            Hq = q(np.stack([self._norm(x, self.nf[l]) for x in X]))
            gate, up = Hq @ Wg.T, Hq @ Wu.T
            X = X + q(gate / (1 + np.exp(-gate)) * up) @ Wd.T
        logits = self.lm @ self._norm(X[-1], self.nfinal)
        return int(np.argmax(logits)), logits


def test_oracle_prefill_matches_numpy_llama(orc):
    """orc_model_prefill against the float64 numpy prefill: from position 0,
    and continuing a cache written by three decode steps (causal rows see the
    earlier positions); logits, next token and the prefilled fp16 K/V."""
    seed = 0x5EF1
    m = orc.Model(CFG, seed)
    ref = NumpyLlama(orc, m, CFG)
    toks = [3, 77, 150, 9, 300, 41]
    nxt, lg = m.prefill(toks, 0, want_logits=True)
    rn, rl = ref.prefill(orc, toks, 0)
    assert nxt == rn
    assert np.abs(lg - rl).max() <= 1e-4 * np.abs(rl).max()
    hd, nkv = CFG["head_dim"], CFG["n_kv_heads"]
    for l in range(CFG["n_layers"]):
        kc = m.kcache(l).reshape(nkv, CFG["max_seq"], hd)[:, :len(toks)].view(np.float16).astype(np.float64)
        np.testing.assert_allclose(kc.transpose(1, 0, 2), ref.K[l][:len(toks)], rtol=2e-3, atol=2e-3)
    m.close()

    m = orc.Model(CFG, seed)
    ref = NumpyLlama(orc, m, CFG)
    for pos, t in enumerate([5, 6, 7]):
        m.step(t, pos)
        ref.step(t, pos)
    nxt, lg = m.prefill(toks[:4], 3, want_logits=True)
    rn, rl = ref.prefill(orc, toks[:4], 3)
    assert nxt == rn
    assert np.abs(lg - rl).max() <= 1e-4 * np.abs(rl).max()
    m.close()


def test_oracle_decode_matches_numpy_llama(orc):
    seed = 0xBEEF
    m = orc.Model(CFG, seed)
    ref = NumpyLlama(orc, m, CFG)
    prompt = [5, 77, 300]
    tok = prompt[0]
    produced = 0
    for pos in range(14):
        t_orc, lo = m.step(tok, pos, want_logits=True)
        t_np, ln = ref.step(tok, pos)
        np.testing.assert_allclose(lo, ln, rtol=1e-4, atol=1e-4 * np.abs(ln).max())
        srt = np.sort(ln)
        if srt[-1] - srt[-2] > 1e-3 * np.abs(ln).max():
            assert t_orc == t_np, pos
        tok = prompt[pos + 1] if pos + 1 < len(prompt) else t_orc
        produced += pos + 1 >= len(prompt)
    assert produced > 8
    m.close()


def test_generate_equals_stepwise(orc):
    """orc_model_generate = the step loop of llama_run/src/main.rs:544-570
    (prompt fed token by token, then greedy feedback, no EOS stop)."""
    seed = 0xF00D
    prompt = [9, 8, 7, 6]
    a = orc.Model(CFG, seed)
    gen, margins = a.generate(prompt, 0, 10)
    b = orc.Model(CFG, seed)
    tok, out = prompt[0], []
    for pos in range(len(prompt) + 10 - 1):
        t = b.step(tok, pos)
        if pos + 1 < len(prompt):
            tok = prompt[pos + 1]
        else:
            out.append(t)
            tok = t
    assert list(gen) == out
    assert np.all(margins >= 0)
    a.close()
    b.close()


def test_kv_prefill_layout(orc):
    """Pre-filled context: element (t, kvh, d) is f16(0.1 * N) at counter index
    (t*NKV + kvh)*HD + d of the layer's stream, stored head-major."""
    m = orc.Model(CFG, 1)
    m.prefill_kv(0x4B56, 5)
    kc = m.kcache(1).reshape(CFG["n_kv_heads"], CFG["max_seq"], CFG["head_dim"])
    coef = orc.lib().orc_ih4_coef(0.1)
    t, kvh, d = 3, 1, 17
    idx = (t * CFG["n_kv_heads"] + kvh) * CFG["head_dim"] + d
    v = orc.lib().orc_ih4_normal(orc.mix64(0x4B56, 0x4B560000 + 2 * 1, idx), coef)
    assert kc[kvh, t, d] == orc.lib().orc_f32_to_f16(v)
    assert not kc[:, 5:].any()
    m.close()


def _xorshift(s, n):
    """xorshift32 13/17/5 (llama_decode/src/main.rs:300-305) in numpy."""
    out = np.empty(n, np.uint32)
    s = np.uint32(s)
    for i in range(n):
        s ^= np.uint32(s << np.uint32(13))
        s ^= np.uint32(s >> np.uint32(17))
        s ^= np.uint32(s << np.uint32(5))
        out[i] = s
    return out, int(s)


HCFG = dict(dim=64, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=32, ffn=128, vocab=96,
            theta=500000.0, eps=1e-5, max_seq=48, scale_format=1, kv_format=1)


def test_f32_scale_model_is_mk_fp4(orc):
    """An f32-scale oracle model holds the reference harness's weights
    (llama_decode/src/main.rs:307-325,369-393): per layer q, k, v, o, gate,
    up, down, then the LM head, each all its packed words then all its scales
    0.25 + (r % 8) * 0.03125, from one xorshift32 stream; norms 1.0."""
    c = HCFG
    qd, kvd = c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"]
    shapes = [(qd, c["dim"]), (kvd, c["dim"]), (kvd, c["dim"]), (c["dim"], qd),
              (c["ffn"], c["dim"]), (c["ffn"], c["dim"]), (c["dim"], c["ffn"])]
    m = orc.Model(c, 0xDEADBEEF)
    st = 0xDEADBEEF
    for l in range(c["n_layers"]):
        for p, (n, k) in enumerate(shapes):
            words, st = _xorshift(st, n * k // 8)
            r, st = _xorshift(st, n * k // 32)
            np.testing.assert_array_equal(m.codes(l, p).view(np.uint32), words)
            np.testing.assert_array_equal(m.scales(l, p), np.float32(0.25) + (r % 8).astype(np.float32) * np.float32(0.03125))
        assert np.all(m.norm(l, 0) == 0x3C00) and np.all(m.norm(l, 1) == 0x3C00)
    words, st = _xorshift(st, c["vocab"] * c["dim"] // 8)
    np.testing.assert_array_equal(m.codes(-1, 0).view(np.uint32), words)
    assert np.all(m.norm(-1, 0) == 0x3C00)
    m.close()


def test_harness_decode_matches_numpy_llama(orc):
    """The llama_decode harness (llama_decode/src/main.rs:356-492) on the
    oracle: f32 scales, f32 K/V with the context [0, P) at 0.01, the
    activation vector (r % 2001) / 1000 - 1 drawn after the weights, and steps
    at P, P+1, ... with no embedding (x carries over); against the float64
    numpy decoder on the same weights."""
    c = HCFG
    P = 20
    m = orc.Model(c, 0xDEADBEEF)
    ref = NumpyLlama(orc, m, c)
    # the stream position after the weights: replay the counts
    qd, kvd = c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"]
    per_layer = (qd + 2 * kvd) * c["dim"] + c["dim"] * qd + 3 * c["ffn"] * c["dim"]
    total = per_layer * c["n_layers"] + c["vocab"] * c["dim"]
    _, st = _xorshift(0xDEADBEEF, total // 8 + total // 32)
    r, _ = _xorshift(st, c["dim"])
    x = (r % 2001).astype(np.float32) / np.float32(1000.0) - np.float32(1.0)
    for l in range(c["n_layers"]):
        ref.K[l][:P] = np.float32(0.01)
        ref.V[l][:P] = np.float32(0.01)
    m.harness_begin(P)
    x = x.astype(np.float64)
    for i in range(6):
        t_orc, lo = m.step_noembed(P + i, want_logits=True)
        t_np, ln = ref.layers(x, P + i)
        x = ref.x
        np.testing.assert_allclose(lo, ln, rtol=1e-4, atol=1e-4 * np.abs(ln).max())
        srt = np.sort(ln)
        if srt[-1] - srt[-2] > 1e-3 * np.abs(ln).max():
            assert t_orc == t_np, i
    kc = m.kcache(0).reshape(c["n_kv_heads"], c["max_seq"], c["head_dim"])
    assert kc.dtype == np.float32 and np.all(kc[:, :P] == np.float32(0.01)) and np.any(kc[:, P] != np.float32(0.01))
    m.close()
