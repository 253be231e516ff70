"""ctypes wrapper of liboracle.so, the CPU restatement of the reference path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker.  The product never
imports it.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# RFP4_ORACLE_LIB selects another build (the sanitizer build of the CPU tests)
LIB_PATH = os.environ.get("RFP4_ORACLE_LIB") or os.path.join(HERE, "liboracle.so")

P = C.c_void_p
U8, U16, U32, U64, I32, F32, F64, SZ = C.c_uint8, C.c_uint16, C.c_uint32, C.c_uint64, C.c_int, C.c_float, C.c_double, C.c_size_t


class OrcModelConfig(C.Structure):
    _fields_ = [
        ("dim", U32), ("n_layers", U32), ("n_heads", U32), ("n_kv_heads", U32),
        ("head_dim", U32), ("ffn", U32), ("vocab", U32), ("max_seq", U32),
        ("theta", F64), ("eps", F32), ("scale_format", U16), ("kv_format", U16),
    ]


_SIGS = {
    "orc_set_threads": (None, [I32]),
    "orc_get_threads": (I32, []),
    "orc_xorshift32_next": (U32, [C.POINTER(U32)]),
    "orc_xorshift32_fill": (None, [C.POINTER(U32), P, SZ]),
    "orc_mix64": (U64, [U64, U64, U64]),
    "orc_ih4_coef": (F32, [F32]),
    "orc_ih4_normal": (F32, [U64, F32]),
    "orc_e2m1_decode": (F32, [U8]),
    "orc_e2m1_decode_arith": (F32, [U32]),
    "orc_e8m0_decode": (F32, [U8]),
    "orc_e8m0_encode_pow2": (U8, [F32]),
    "orc_e2m1_rne": (U8, [F32]),
    "orc_f16_to_f32": (F32, [U16]),
    "orc_f32_to_f16": (U16, [F32]),
    "orc_bf16_to_f32": (F32, [U16]),
    "orc_f32_to_bf16": (U16, [F32]),
    "orc_pack_codes": (None, [P, SZ, P]),
    "orc_unpack_codes": (None, [P, SZ, P]),
    "orc_model_set_embed_bf16": (None, [P, I32]),
    "orc_quant_fp4_absmax": (None, [P, I32, I32, P, P]),
    "orc_quant_mx": (None, [P, SZ, SZ, P, P]),
    "orc_synth_mx_weight": (None, [U64, U64, F32, SZ, SZ, SZ, P, P]),
    "orc_synth_f16": (None, [U64, U64, F32, F32, SZ, P]),
    "orc_gemv_f32scale": (None, [U32, U32, P, P, P, P]),
    "orc_gemv_e8m0": (None, [U32, U32, P, P, P, P]),
    "orc_gemv_e8m0_f64": (None, [U32, U32, P, P, P, P, P]),
    "orc_mma_m16n8k64_ref": (None, [P, P, P, P, P]),
    "orc_gemm_mx_f64": (None, [U32, U32, U32, P, P, P, P, P, P]),
    "orc_rmsnorm": (None, [U32, F32, P, P, P]),
    "orc_rope_table": (None, [U32, U32, F64, P, P]),
    "orc_rope": (None, [U32, U32, P, P, P]),
    "orc_attn_decode": (None, [U32, U32, U32, U32, P, P, P, SZ, SZ, P]),
    "orc_attn_decode_f16": (None, [U32, U32, U32, U32, P, P, P, SZ, SZ, P]),
    "orc_swiglu": (None, [U32, P, P, P]),
    "orc_residual": (None, [U32, P, P]),
    "orc_argmax": (U32, [U32, P]),
    "orc_model_create": (P, [C.POINTER(OrcModelConfig), U64]),
    "orc_model_destroy": (None, [P]),
    "orc_model_codes": (P, [P, I32, I32, C.POINTER(SZ)]),
    "orc_model_scales": (P, [P, I32, I32, C.POINTER(SZ)]),
    "orc_model_embed": (P, [P, C.POINTER(SZ)]),
    "orc_model_norm": (P, [P, I32, I32, C.POINTER(SZ)]),
    "orc_model_kcache": (P, [P, I32, C.POINTER(SZ)]),
    "orc_model_vcache": (P, [P, I32, C.POINTER(SZ)]),
    "orc_model_prefill_kv": (None, [P, U64, U32]),
    "orc_model_step": (U32, [P, U32, U32, P]),
    "orc_model_fill_kv": (None, [P, F32, U32]),
    "orc_model_harness_begin": (None, [P]),
    "orc_model_step_noembed": (U32, [P, U32, P]),
    "orc_model_generate": (None, [P, P, U32, U32, U32, P, P]),
    "orc_model_prefill": (U32, [P, P, U32, U32, P]),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} not built; run `make -C oracle`")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def ptr(a: np.ndarray):
    return a.ctypes.data


def set_threads(n: int):
    lib().orc_set_threads(n)


# ---------------------------------------------------------------- RNG / codecs
def xorshift32(seed: int, n: int) -> tuple[np.ndarray, int]:
    st = U32(seed)
    out = np.empty(n, dtype=np.uint32)
    lib().orc_xorshift32_fill(C.byref(st), ptr(out), n)
    return out, st.value


def mix64(seed, stream, index) -> int:
    return int(lib().orc_mix64(seed, stream, index))


def ih4_normal_from_u64(r: int, sigma: float) -> float:
    return float(lib().orc_ih4_normal(r, lib().orc_ih4_coef(sigma)))


def pack(codes: np.ndarray) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    out = np.empty(codes.size // 2, dtype=np.uint8)
    lib().orc_pack_codes(ptr(codes), codes.size, ptr(out))
    return out


def unpack(packed: np.ndarray) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.empty(packed.size * 2, dtype=np.uint8)
    lib().orc_unpack_codes(ptr(packed), out.size, ptr(out))
    return out


def quant_mx(w: np.ndarray):
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, k = w.shape
    packed = np.empty(rows * k // 2, dtype=np.uint8)
    scales = np.empty(rows * k // 32, dtype=np.uint8)
    lib().orc_quant_mx(ptr(w), rows, k, ptr(packed), ptr(scales))
    return packed, scales


def quant_fp4_absmax(w: np.ndarray):
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, k = w.shape
    packed = np.empty(rows * k // 2, dtype=np.uint8)
    scales = np.empty(rows * k // 32, dtype=np.float32)
    lib().orc_quant_fp4_absmax(ptr(w), rows, k, ptr(packed), ptr(scales))
    return packed, scales


def synth_mx_weight(seed, stream, sigma, k, r0, nrows):
    packed = np.empty(nrows * k // 2, dtype=np.uint8)
    scales = np.empty(nrows * k // 32, dtype=np.uint8)
    lib().orc_synth_mx_weight(seed, stream, sigma, k, r0, nrows, ptr(packed), ptr(scales))
    return packed, scales


def synth_f16(seed, stream, sigma, offset, n):
    out = np.empty(n, dtype=np.uint16)
    lib().orc_synth_f16(seed, stream, sigma, offset, n, ptr(out))
    return out


# ---------------------------------------------------------------- math
def gemv_f32scale(n, k, w_words, scales, x):
    y = np.empty(n, dtype=np.float32)
    lib().orc_gemv_f32scale(n, k, ptr(np.ascontiguousarray(w_words, np.uint32)),
                            ptr(np.ascontiguousarray(scales, np.float32)), ptr(np.ascontiguousarray(x, np.float32)), ptr(y))
    return y


def gemv_e8m0(n, k, codes, scales, x):
    y = np.empty(n, dtype=np.float32)
    lib().orc_gemv_e8m0(n, k, ptr(np.ascontiguousarray(codes, np.uint8)), ptr(np.ascontiguousarray(scales, np.uint8)),
                        ptr(np.ascontiguousarray(x, np.float32)), ptr(y))
    return y


def gemv_e8m0_f64(n, k, codes, scales, x):
    y = np.empty(n, dtype=np.float64)
    a = np.empty(n, dtype=np.float64)
    lib().orc_gemv_e8m0_f64(n, k, ptr(np.ascontiguousarray(codes, np.uint8)), ptr(np.ascontiguousarray(scales, np.uint8)),
                            ptr(np.ascontiguousarray(x, np.float32)), ptr(y), ptr(a))
    return y, a


def mma_m16n8k64_ref(A, B, SFA, SFB):
    D = np.empty((16, 8), dtype=np.float32)
    lib().orc_mma_m16n8k64_ref(*(ptr(np.ascontiguousarray(t, np.float32)) for t in (A, B, SFA, SFB)), ptr(D))
    return D


def gemm_mx_f64(M, N, K, a_codes, a_scales, w_codes, w_scales):
    c = np.empty((M, N), dtype=np.float64)
    ac = np.empty((M, N), dtype=np.float64)
    lib().orc_gemm_mx_f64(M, N, K, *(ptr(np.ascontiguousarray(t, np.uint8)) for t in (a_codes, a_scales, w_codes, w_scales)),
                          ptr(c), ptr(ac))
    return c, ac


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().orc_rmsnorm(x.size, eps, ptr(x), ptr(np.ascontiguousarray(w, np.float32)), ptr(y))
    return y


def rope_table(max_pos, head_dim, theta):
    half = head_dim // 2
    c = np.empty(max_pos * half, dtype=np.float32)
    s = np.empty(max_pos * half, dtype=np.float32)
    lib().orc_rope_table(max_pos, head_dim, theta, ptr(c), ptr(s))
    return c, s


def rope(q, num_heads, head_dim, cosp, sinp):
    q = np.array(q, dtype=np.float32, copy=True)
    lib().orc_rope(num_heads, head_dim, ptr(np.ascontiguousarray(cosp, np.float32)),
                   ptr(np.ascontiguousarray(sinp, np.float32)), ptr(q))
    return q


def attn_decode(nh, nkv, hd, seq, q, kc, vc, ts, hs):
    out = np.empty(nh * hd, dtype=np.float32)
    if kc.dtype == np.uint16:
        lib().orc_attn_decode_f16(nh, nkv, hd, seq, ptr(np.ascontiguousarray(q, np.float32)), ptr(kc), ptr(vc), ts, hs,
                                  ptr(out))
    else:
        lib().orc_attn_decode(nh, nkv, hd, seq, ptr(np.ascontiguousarray(q, np.float32)),
                              ptr(np.ascontiguousarray(kc, np.float32)), ptr(np.ascontiguousarray(vc, np.float32)),
                              ts, hs, ptr(out))
    return out


def swiglu(g, u):
    g = np.ascontiguousarray(g, np.float32)
    out = np.empty_like(g)
    lib().orc_swiglu(g.size, ptr(g), ptr(np.ascontiguousarray(u, np.float32)), ptr(out))
    return out


def residual(y, x):
    x = np.array(x, dtype=np.float32, copy=True)
    lib().orc_residual(x.size, ptr(np.ascontiguousarray(y, np.float32)), ptr(x))
    return x


def argmax(v) -> int:
    v = np.ascontiguousarray(v, np.float32)
    return int(lib().orc_argmax(v.size, ptr(v)))


def f32_to_f16(v: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(v, np.float32).ravel()
    f = lib().orc_f32_to_f16
    return np.array([f(float(t)) for t in v], dtype=np.uint16)


# ---------------------------------------------------------------- model
SCALE_E8M0, SCALE_F32 = 0, 1
KV_F16, KV_F32 = 0, 1


class Model:
    """The oracle decoder.  cfg may carry scale_format (SCALE_E8M0 or
    SCALE_F32: the reference's f32 per-32 scales and its mk_fp4 harness init)
    and kv_format (KV_F16 or KV_F32)."""

    def __init__(self, cfg: dict, seed: int):
        self.cfg = dict(cfg)
        self.scale_format = int(cfg.get("scale_format", SCALE_E8M0))
        self.kv_format = int(cfg.get("kv_format", KV_F16))
        c = OrcModelConfig(dim=cfg["dim"], n_layers=cfg["n_layers"], n_heads=cfg["n_heads"],
                           n_kv_heads=cfg["n_kv_heads"], head_dim=cfg["head_dim"], ffn=cfg["ffn"],
                           vocab=cfg["vocab"], max_seq=cfg["max_seq"], theta=cfg["theta"], eps=cfg["eps"],
                           scale_format=self.scale_format, kv_format=self.kv_format)
        self.h = lib().orc_model_create(C.byref(c), seed)
        if not self.h:
            raise RuntimeError("orc_model_create failed")

    def _view(self, fn, *args, dtype):
        n = SZ()
        p = fn(self.h, *args, C.byref(n))
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(np.ctypeslib.as_ctypes_type(dtype))), shape=(n.value,))

    def codes(self, layer, proj):
        return self._view(lib().orc_model_codes, layer, proj, dtype=np.uint8)

    def scales(self, layer, proj):
        """E8M0 bytes, or the f32 scales of a SCALE_F32 model."""
        b = self._view(lib().orc_model_scales, layer, proj, dtype=np.uint8)
        return b.view(np.float32) if self.scale_format == SCALE_F32 else b

    def embed(self):
        return self._view(lib().orc_model_embed, dtype=np.uint16)

    def norm(self, layer, which):
        return self._view(lib().orc_model_norm, layer, which, dtype=np.uint16)

    _PROJ = ("self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
             "self_attn.o_proj.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight")

    def load_checkpoint(self, f32, half_bits, embed_bf16):
        """Real weights: f32 (widened checkpoint values, name -> [rows][k]) for
        the projections, quantized by the OCP MX rules; half_bits (name ->
        uint16 bit patterns): f16 norms, embeddings bf16 or f16."""
        L = self.cfg["n_layers"]
        for l in range(L):
            for p, name in enumerate(self._PROJ):
                c, s = quant_mx(f32[f"model.layers.{l}.{name}"])
                self.codes(l, p)[:] = c.reshape(-1)
                self.scales(l, p)[:] = s.reshape(-1)
            self.norm(l, 0)[:] = half_bits[f"model.layers.{l}.input_layernorm.weight"]
            self.norm(l, 1)[:] = half_bits[f"model.layers.{l}.post_attention_layernorm.weight"]
        self.norm(-1, 0)[:] = half_bits["model.norm.weight"]
        self.embed()[:] = half_bits["model.embed_tokens.weight"].reshape(-1)
        lm = f32.get("lm_head.weight", f32["model.embed_tokens.weight"])
        c, s = quant_mx(lm)
        self.codes(-1, 0)[:] = c.reshape(-1)
        self.scales(-1, 0)[:] = s.reshape(-1)
        lib().orc_model_set_embed_bf16(self.h, 1 if embed_bf16 else 0)

    def _kv_dtype(self):
        return np.float32 if self.kv_format == KV_F32 else np.uint16

    def kcache(self, layer):
        return self._view(lib().orc_model_kcache, layer, dtype=self._kv_dtype())

    def vcache(self, layer):
        return self._view(lib().orc_model_vcache, layer, dtype=self._kv_dtype())

    def fill_kv(self, value, upto):
        lib().orc_model_fill_kv(self.h, value, upto)

    def harness_begin(self, ctx):
        """llama_decode's context: K/V positions [0, ctx) := 0.01 and x := the
        harness vector (llama_decode/src/main.rs:375-376,421)."""
        self.fill_kv(0.01, ctx)
        lib().orc_model_harness_begin(self.h)

    def step_noembed(self, pos, want_logits=False):
        logits = np.empty(self.cfg["vocab"], dtype=np.float32) if want_logits else None
        t = lib().orc_model_step_noembed(self.h, pos, ptr(logits) if want_logits else None)
        return (t, logits) if want_logits else t

    def prefill_kv(self, seed, upto):
        lib().orc_model_prefill_kv(self.h, seed, upto)

    def step(self, tok, pos, want_logits=False):
        logits = np.empty(self.cfg["vocab"], dtype=np.float32) if want_logits else None
        t = lib().orc_model_step(self.h, tok, pos, ptr(logits) if want_logits else None)
        return (t, logits) if want_logits else t

    def generate(self, prompt, pos0, n_new):
        pr = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.empty(n_new, dtype=np.uint32)
        margins = np.empty(n_new, dtype=np.float32)
        lib().orc_model_generate(self.h, ptr(pr), len(pr), pos0, n_new, ptr(out), ptr(margins))
        return out, margins

    def prefill(self, prompt, pos0, want_logits=False):
        """Batched prefill with MXFP4 activations; returns the next token (and logits)."""
        pr = np.ascontiguousarray(prompt, dtype=np.uint32)
        logits = np.empty(self.cfg["vocab"], dtype=np.float32) if want_logits else None
        t = lib().orc_model_prefill(self.h, ptr(pr), len(pr), pos0, ptr(logits) if want_logits else None)
        return (t, logits) if want_logits else t

    def close(self):
        if self.h:
            lib().orc_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
