"""ctypes binding of librfp4.so, the C ABI declared in include/rfp4.h.

Mirrors the reference's host API shape (cuda-oxide `CudaContext`,
`DeviceBuffer::{from_host, zeroed, to_host_vec}`, typed kernel launchers,
events; e.g. fp4_gemv/src/main.rs:144-191) so tests and the benchmark read like
the reference's self-checking examples.  Every call raises `Rfp4Error` on a
non-zero return code, the counterpart of the reference's `.unwrap()` panics.

There is no CPU fallback: if the library is missing or no gfx950 device is
present, the calls fail loudly.
"""
from __future__ import annotations

import atexit
import ctypes as C
import os
import re
import weakref

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# RFP4_LIB selects another build of the same library (the sanitizer build of
# the CPU tests); the default is the in-tree librfp4.so.
LIB_PATH = os.environ.get("RFP4_LIB") or os.path.join(HERE, "librfp4.so")
HEADER_PATH = os.path.join(os.path.dirname(HERE), "include", "rfp4.h")

P = C.c_void_p
U32 = C.c_uint32
U64 = C.c_uint64
I32 = C.c_int
F32 = C.c_float
SZ = C.c_size_t


class Rfp4Error(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"rfp4 error {code}: {msg}")
        self.code = code


class KernelTime(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("us", F32)]


class ModelConfig(C.Structure):
    _fields_ = [
        ("dim", U32), ("n_layers", U32), ("n_heads", U32), ("n_kv_heads", U32),
        ("head_dim", U32), ("ffn", U32), ("vocab", U32), ("max_seq", U32),
        ("theta", C.c_double), ("eps", F32), ("scale_format", C.c_uint16), ("kv_format", C.c_uint16),
    ]


SCALE_E8M0, SCALE_F32 = 0, 1   # RFP4_SCALE_*
EPI_STORE, EPI_RESIDUAL, EPI_SWIGLU, EPI_ARGMAX = 0, 1, 2, 3  # epilogues of rfp4_debug_gemv_fused
KV_F16, KV_F32 = 0, 1           # RFP4_KV_*


# name -> (restype, argtypes)
_SIGS = {
    "rfp4_last_error": (C.c_char_p, []),
    "rfp4_version": (I32, []),
    "rfp4_kernel_count": (I32, [C.POINTER(U32)]),
    "rfp4_kernel_name": (I32, [U32, C.c_char_p, SZ]),
    "rfp4_init": (I32, [I32]),
    "rfp4_shutdown": (I32, []),
    "rfp4_device_count": (I32, [C.POINTER(I32)]),
    "rfp4_device_info": (I32, [C.POINTER(I32), C.POINTER(SZ), C.POINTER(I32)]),
    "rfp4_stream_create": (I32, [C.POINTER(P)]),
    "rfp4_stream_destroy": (I32, [P]),
    "rfp4_stream_synchronize": (I32, [P]),
    "rfp4_malloc": (I32, [C.POINTER(P), SZ]),
    "rfp4_free": (I32, [P]),
    "rfp4_memset_zero": (I32, [P, SZ, P]),
    "rfp4_h2d": (I32, [P, P, SZ, P]),
    "rfp4_d2h": (I32, [P, P, SZ, P]),
    "rfp4_event_create": (I32, [C.POINTER(P)]),
    "rfp4_event_destroy": (I32, [P]),
    "rfp4_event_record": (I32, [P, P]),
    "rfp4_event_synchronize": (I32, [P]),
    "rfp4_event_elapsed_ms": (I32, [C.POINTER(F32), P, P]),
    "fp4_gemv": (I32, [P, U32, U32, P, P, P, P]),
    "mx4_gemv": (I32, [P, U32, U32, P, P, P, P]),
    "mx4_gemv_rmsnorm": (I32, [P, U32, U32, P, P, P, P, F32, P]),
    "mx4_gemv_residual": (I32, [P, U32, U32, P, P, P, P]),
    "mx4_gemv_swiglu": (I32, [P, U32, U32, U32, P, P, P, P]),
    "mx4_gemv_argmax_workspace": (SZ, [U32]),
    "mx4_gemv_argmax": (I32, [P, U32, U32, P, P, P, P, P, P]),
    "rmsnorm": (I32, [P, U32, F32, P, P, P]),
    "rmsnorm_f16w": (I32, [P, U32, F32, P, P, P]),
    "rope": (I32, [P, U32, U32, U32, P, P, P]),
    "copy_into": (I32, [P, U32, U32, P, P]),
    "kv_append_f16": (I32, [P, U32, U32, P, P]),
    "attn_decode": (I32, [P, U32, U32, U32, P, P, P, P]),
    "attn_decode_f16": (I32, [P, U32, U32, U32, U32, P, P, P, U64, U64, P]),
    "attn_decode_f16_noalloc": (I32, [P, U32, U32, U32, U32, P, P, P, U64, U64, P]),
    "attn_prefill_f16": (I32, [P, U32, U32, U32, U32, U32, P, U32, P, P, U64, U64, P, U32]),
    "swiglu": (I32, [P, U32, P, P, P]),
    "residual": (I32, [P, U32, P, P]),
    "argmax": (I32, [P, U32, P, P]),
    "fp4_mma_allones": (I32, [P, P]),
    "mx4_quantize": (I32, [P, U64, U64, P, I32, P, P]),
    "fp4_gemm": (I32, [P, U32, U32, U32, P, P, P, P, P]),
    "fp4_gemm_tiled": (I32, [P, U32, U32, U32, P, P, P, P, P, P, P]),
    "mx4_scales_tiled_bytes": (SZ, [U32, U32]),
    "mx4_scales_tile": (I32, [P, U32, U32, P, P]),
    "mx4_quantize_tiled": (I32, [P, U64, U64, P, I32, P, P, P]),
    "rfp4_debug_gemm_plan": (I32, [I32, I32]),
    "rfp4_debug_attn_chunk": (I32, [U32]),
    "rfp4_gemm_plan": (I32, [U32, U32, U32, P, P, P]),
    "rfp4_gemm_plan_kernel": (I32, [U32, U32, U32, C.c_char_p, SZ]),
    "rfp4_mma_tile16": (I32, [P, P, P, P, P, P]),
    "rfp4_mma_tile32": (I32, [P, P, P, P, P, P]),
    "rfp4_selftest_cvt_fp4": (I32, [P, U32, P, P]),
    "rfp4_debug_gemv_variant": (I32, [I32, I32]),
    "rfp4_debug_gemv_waves": (I32, [I32]),
    "rfp4_debug_attn_merge": (I32, [I32]),
    "rfp4_debug_prefill_attn": (I32, [I32]),
    "rfp4_debug_prefill_stop": (I32, [I32]),
    "rfp4_debug_prefill_swiglu": (I32, [I32]),
    "rfp4_debug_prefill_rope": (I32, [I32]),
    "rfp4_debug_prefill_attn_quant": (I32, [I32]),
    "rfp4_debug_prefill_ksplit": (I32, [I32]),
    "rfp4_debug_attn_head_split": (I32, [I32]),
    "rfp4_debug_qkv_attn": (I32, [I32]),
    "rfp4_debug_gemm_stages": (I32, [I32]),
    "rfp4_debug_gemm_pp": (I32, [I32]),
    "rfp4_debug_gemm_reduce_kernel": (I32, [I32]),
    "rfp4_debug_prefill_waves": (I32, [I32]),
    "rfp4_debug_prefill_pairing": (I32, [I32]),
    "rfp4_debug_fp4_encode_check": (I32, [P, C.c_int32, U32, P, P]),
    "rfp4_debug_gemv_fused": (I32, [P, I32, I32, U32, U32, U32, P, P, P, P, F32, P, P, P]),
    "rfp4_mma_bf16_tile": (I32, [P, P, P, P]),
    "rfp4_mma_f16_tile": (I32, [P, P, P, P]),
    "rfp4_synth_mx_weight": (I32, [P, U64, U64, F32, U64, U64, U64, P, P]),
    "rfp4_synth_f16": (I32, [P, U64, U64, F32, F32, U64, P]),
    "llama_engine_create": (I32, [C.POINTER(ModelConfig), U64, C.POINTER(P)]),
    "llama_engine_destroy": (I32, [P]),
    "llama_engine_prefill_kv": (I32, [P, U64, U32]),
    "llama_engine_create_from_safetensors": (I32, [C.POINTER(ModelConfig), C.c_char_p, C.POINTER(P)]),
    "llama_engine_save": (I32, [P, C.c_char_p]),
    "llama_engine_load": (I32, [C.c_char_p, U32, C.POINTER(P)]),
    "llama_engine_info": (I32, [P, C.POINTER(ModelConfig), C.POINTER(C.c_int)]),
    "fp4_quantize_absmax": (I32, [P, U32, U32, P, P]),
    "rfp4_st_open": (I32, [C.c_char_p, C.POINTER(P)]),
    "rfp4_st_close": (I32, [P]),
    "rfp4_st_count": (I32, [P, C.POINTER(U32)]),
    "rfp4_st_name": (I32, [P, U32, C.POINTER(C.c_char_p)]),
    "rfp4_st_info": (I32, [P, C.c_char_p, C.c_char_p, C.POINTER(U32), P, C.POINTER(U64)]),
    "rfp4_st_read_f32": (I32, [P, C.c_char_p, P, U64]),
    "rfp4_st_read_f16": (I32, [P, C.c_char_p, P, U64]),
    "llama_engine_prefill": (I32, [P, P, U32, U32, C.POINTER(U32)]),
    "llama_decode_step": (I32, [P, U32, U32, C.POINTER(U32)]),
    "llama_generate": (I32, [P, P, U32, U32, U32, P]),
    "llama_engine_begin": (I32, [P, P, U32, U32, U32]),
    "llama_engine_begin_harness": (I32, [P, U32, U32]),
    "llama_engine_run_steps": (I32, [P, U32]),
    "llama_engine_time_steps": (I32, [P, U32, P, U32, C.POINTER(U32)]),
    "llama_engine_read_ids": (I32, [P, P, U32]),
    "llama_engine_logits": (I32, [P, P]),
    "llama_engine_stream": (P, [P]),
    "llama_engine_use_graph": (I32, [P, I32]),
    "llama_engine_weight": (I32, [P, I32, I32, C.POINTER(P), C.POINTER(P), C.POINTER(SZ), C.POINTER(SZ)]),
    "llama_engine_weight_scales_tiled": (I32, [P, I32, I32, C.POINTER(P), C.POINTER(SZ)]),
    "llama_engine_kv": (I32, [P, I32, C.POINTER(P), C.POINTER(P), C.POINTER(SZ)]),
    "llama_engine_use_persistent": (I32, [P, I32]),
    "llama_engine_persistent": (I32, [P]),
    "llama_engine_prefill_buffers": (I32, [P, C.POINTER(P), C.POINTER(P), C.POINTER(P), C.POINTER(P), C.POINTER(P),
                                           C.POINTER(U32)]),
    "llama_engine_weight_bytes": (U64, [P]),
    "rfp4_debug_engine_wait": (I32, [P, I32, U32, C.POINTER(I32), C.POINTER(I32), C.POINTER(I32)]),
}

_lib = None


def load(path: str = LIB_PATH):
    """Load librfp4.so and attach signatures (no GPU call is made)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built; run __graft_entry__.build()")
    lib = C.CDLL(path)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def header_functions(path: str = HEADER_PATH) -> list[str]:
    """Function names declared in include/rfp4.h."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w \*]*?\b([A-Za-z_]\w*)\s*\(", text, flags=re.M)
    return sorted(set(n for n in names if n not in ("if", "while", "for", "return", "sizeof")))


def check(rc: int):
    if rc != 0:
        raise Rfp4Error(rc, load().rfp4_last_error().decode())


_inited = False
_atexit_registered = False
# Objects that own a library or HIP resource (engines, device buffers, events,
# owned streams), released by shutdown() if still alive.
_live = weakref.WeakSet()


def init(device: int = 0):
    """CudaContext::new(0) + kernels::load (llama_run/src/main.rs:432,488).
    Registers shutdown() to run at interpreter exit."""
    global _inited, _atexit_registered
    if not _inited:
        check(load().rfp4_init(device))
        _inited = True
        if not _atexit_registered:
            atexit.register(shutdown)
            _atexit_registered = True


def shutdown():
    """Release every resource held through the library, then the library's
    own (rfp4_shutdown): engines first (step graphs, their streams and memory),
    then device buffers, events and owned streams.  Runs at interpreter exit,
    before the HIP runtime's own teardown; the released objects' later
    free/close calls are no-ops.  init() may be called again afterwards."""
    global _inited
    if not _inited:
        return
    live = list(_live)
    for kind in (Engine, DeviceBuffer, Event, Stream):
        for o in live:
            if isinstance(o, kind):
                o._release()
    _inited = False
    check(load().rfp4_shutdown())


def kernel_names() -> list:
    """Every kernel of the embedded gfx950 code object (no device needed)."""
    lib = load()
    n = U32(0)
    check(lib.rfp4_kernel_count(C.byref(n)))
    buf = C.create_string_buffer(256)
    out = []
    for i in range(n.value):
        check(lib.rfp4_kernel_name(i, buf, 256))
        out.append(buf.value.decode())
    return out


def device_count() -> int:
    n = I32(0)
    rc = load().rfp4_device_count(C.byref(n))
    return n.value if rc == 0 else 0


class Stream:
    def __init__(self, handle=None):
        if handle is None:
            h = P()
            check(load().rfp4_stream_create(C.byref(h)))
            self.h = h.value
            self._own = True
            _live.add(self)
        else:
            self.h = handle
            self._own = False

    def synchronize(self):
        check(load().rfp4_stream_synchronize(self.h))

    def destroy(self):
        if self._own and self.h:
            load().rfp4_stream_destroy(self.h)
            self.h = None

    _release = destroy

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class DeviceBuffer:
    """Device allocation (reference DeviceBuffer<T>)."""

    def __init__(self, nbytes: int, dtype=np.uint8):
        self.nbytes = int(nbytes)
        self.dtype = np.dtype(dtype)
        p = P()
        check(load().rfp4_malloc(C.byref(p), max(self.nbytes, 16)))
        self.ptr = p.value
        _live.add(self)

    @classmethod
    def from_host(cls, arr: np.ndarray, stream: Stream | None = None):
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes, arr.dtype)
        s = stream.h if stream else None
        check(load().rfp4_h2d(buf.ptr, arr.ctypes.data, arr.nbytes, s))
        if stream:
            stream.synchronize()
        else:
            check(load().rfp4_stream_synchronize(None))
        return buf

    @classmethod
    def zeroed(cls, count: int, dtype=np.float32, stream: Stream | None = None):
        nbytes = int(count) * np.dtype(dtype).itemsize
        buf = cls((nbytes + 3) // 4 * 4, dtype)
        check(load().rfp4_memset_zero(buf.ptr, (nbytes + 3) // 4 * 4, stream.h if stream else None))
        return buf

    def to_host(self, count: int | None = None, dtype=None, stream: Stream | None = None) -> np.ndarray:
        dtype = np.dtype(dtype or self.dtype)
        if count is None:
            count = self.nbytes // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        check(load().rfp4_d2h(out.ctypes.data, self.ptr, out.nbytes, stream.h if stream else None))
        return out

    def free(self):
        if self.ptr:
            load().rfp4_free(self.ptr)
            self.ptr = None

    _release = free

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    def __init__(self):
        h = P()
        check(load().rfp4_event_create(C.byref(h)))
        self.h = h.value
        _live.add(self)

    def record(self, stream: Stream | None = None):
        check(load().rfp4_event_record(self.h, stream.h if stream else None))

    def synchronize(self):
        check(load().rfp4_event_synchronize(self.h))

    def elapsed_ms(self, end: "Event") -> float:
        ms = F32(0)
        check(load().rfp4_event_elapsed_ms(C.byref(ms), self.h, end.h))
        return ms.value

    def destroy(self):
        if self.h:
            load().rfp4_event_destroy(self.h)
            self.h = None

    _release = destroy

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


def _p(x):
    if x is None:
        return None
    if isinstance(x, DeviceBuffer):
        return x.ptr
    return x


def _s(stream):
    return stream.h if isinstance(stream, Stream) else stream


# ---------------------------------------------------------------- kernel launchers
def fp4_gemv(stream, n, k, w, scales, x, y):
    check(load().fp4_gemv(_s(stream), n, k, _p(w), _p(scales), _p(x), _p(y)))


def mx4_gemv(stream, n, k, codes, scales, x, y):
    check(load().mx4_gemv(_s(stream), n, k, _p(codes), _p(scales), _p(x), _p(y)))


def mx4_gemv_rmsnorm(stream, n, k, codes, scales, x, norm_w, eps, y):
    check(load().mx4_gemv_rmsnorm(_s(stream), n, k, _p(codes), _p(scales), _p(x), _p(norm_w), eps, _p(y)))


def mx4_gemv_residual(stream, n, k, codes, scales, x, x_res):
    check(load().mx4_gemv_residual(_s(stream), n, k, _p(codes), _p(scales), _p(x), _p(x_res)))


def mx4_gemv_swiglu(stream, n, k, pair_off, codes, scales, x, out):
    check(load().mx4_gemv_swiglu(_s(stream), n, k, pair_off, _p(codes), _p(scales), _p(x), _p(out)))


def mx4_gemv_argmax_workspace(n) -> int:
    return int(load().mx4_gemv_argmax_workspace(n))


def mx4_gemv_argmax(stream, n, k, codes, scales, x, y, workspace, best):
    check(load().mx4_gemv_argmax(_s(stream), n, k, _p(codes), _p(scales), _p(x), _p(y), _p(workspace), _p(best)))


def rmsnorm(stream, dim, eps, x, w, y):
    check(load().rmsnorm(_s(stream), dim, eps, _p(x), _p(w), _p(y)))


def rmsnorm_f16w(stream, dim, eps, x, w, y):
    check(load().rmsnorm_f16w(_s(stream), dim, eps, _p(x), _p(w), _p(y)))


def rope(stream, num_heads, head_dim, cos_base, cos_tab, sin_tab, q):
    check(load().rope(_s(stream), num_heads, head_dim, cos_base, _p(cos_tab), _p(sin_tab), _p(q)))


def copy_into(stream, n, off, src, dst):
    check(load().copy_into(_s(stream), n, off, _p(src), _p(dst)))


def kv_append_f16(stream, n, off, src, dst):
    check(load().kv_append_f16(_s(stream), n, off, _p(src), _p(dst)))


def attn_decode(stream, n_heads, n_kv_heads, seq, q, kc, vc, out):
    check(load().attn_decode(_s(stream), n_heads, n_kv_heads, seq, _p(q), _p(kc), _p(vc), _p(out)))


def attn_decode_f16(stream, n_heads, n_kv_heads, head_dim, seq, q, kc, vc, token_stride, head_stride, out):
    check(load().attn_decode_f16(_s(stream), n_heads, n_kv_heads, head_dim, seq, _p(q), _p(kc), _p(vc),
                                 token_stride, head_stride, _p(out)))


def attn_prefill_f16(stream, n_heads, n_kv_heads, head_dim, pos0, rows, q, q_row_stride, kc, vc, token_stride,
                     head_stride, out, out_row_stride):
    check(load().attn_prefill_f16(_s(stream), n_heads, n_kv_heads, head_dim, pos0, rows, _p(q), q_row_stride, _p(kc),
                                  _p(vc), token_stride, head_stride, _p(out), out_row_stride))


def swiglu(stream, n, gate, up, out):
    check(load().swiglu(_s(stream), n, _p(gate), _p(up), _p(out)))


def residual(stream, n, y, x):
    check(load().residual(_s(stream), n, _p(y), _p(x)))


def argmax(stream, n, logits, out):
    check(load().argmax(_s(stream), n, _p(logits), _p(out)))


def fp4_mma_allones(stream, out):
    check(load().fp4_mma_allones(_s(stream), _p(out)))


def mx4_quantize(stream, rows, k, src, src_is_bf16, codes, scales):
    check(load().mx4_quantize(_s(stream), rows, k, _p(src), int(src_is_bf16), _p(codes), _p(scales)))


def fp4_gemm(stream, m, n, k, a_codes, a_scales, w_codes, w_scales, c):
    check(load().fp4_gemm(_s(stream), m, n, k, _p(a_codes), _p(a_scales), _p(w_codes), _p(w_scales), _p(c)))


def fp4_gemm_tiled(stream, m, n, k, a_codes, a_scales, a_scales_tiled, w_codes, w_scales, w_scales_tiled, c):
    """fp4_gemm with the step-blocked scale copies supplied (no tiling launch)."""
    check(load().fp4_gemm_tiled(_s(stream), m, n, k, _p(a_codes), _p(a_scales), _p(a_scales_tiled), _p(w_codes),
                                _p(w_scales), _p(w_scales_tiled), _p(c)))


def mx4_scales_tiled_bytes(rows, k) -> int:
    return int(load().mx4_scales_tiled_bytes(rows, k))


def mx4_scales_tile(stream, rows, k, scales, scales_tiled):
    check(load().mx4_scales_tile(_s(stream), rows, k, _p(scales), _p(scales_tiled)))


def mx4_quantize_tiled(stream, rows, k, src, src_is_bf16, codes, scales, scales_tiled):
    check(load().mx4_quantize_tiled(_s(stream), rows, k, _p(src), int(src_is_bf16), _p(codes), _p(scales),
                                    _p(scales_tiled)))


def debug_attn_chunk(chunk=0):
    check(load().rfp4_debug_attn_chunk(chunk))


def debug_gemm_plan(tile=-1, kz=0):
    check(load().rfp4_debug_gemm_plan(tile, kz))


def gemm_plan(m, n, k):
    """(tile_m, tile_n, kz) fp4_gemm uses for this shape."""
    tm, tn, kz = C.c_int(), C.c_int(), C.c_int()
    check(load().rfp4_gemm_plan(m, n, k, C.byref(tm), C.byref(tn), C.byref(kz)))
    return tm.value, tn.value, kz.value


def gemm_plan_kernel(m, n, k) -> str:
    """The kernel (and K split) fp4_gemm launches for this shape."""
    buf = C.create_string_buffer(96)
    check(load().rfp4_gemm_plan_kernel(m, n, k, buf, 96))
    return buf.value.decode()


def mma_tile16(stream, a, b, sa, sb, out):
    check(load().rfp4_mma_tile16(_s(stream), _p(a), _p(b), _p(sa), _p(sb), _p(out)))


def mma_tile32(stream, a, b, sa, sb, out):
    check(load().rfp4_mma_tile32(_s(stream), _p(a), _p(b), _p(sa), _p(sb), _p(out)))


def selftest_cvt_fp4(stream, n, words, out):
    check(load().rfp4_selftest_cvt_fp4(_s(stream), n, _p(words), _p(out)))


def synth_mx_weight(stream, seed, stream_id, sigma, k, r0, nrows, codes, scales):
    check(load().rfp4_synth_mx_weight(_s(stream), seed, stream_id, sigma, k, r0, nrows, _p(codes), _p(scales)))


def synth_f16(stream, seed, stream_id, sigma, offset, n, out):
    check(load().rfp4_synth_f16(_s(stream), seed, stream_id, sigma, offset, n, _p(out)))


# ---------------------------------------------------------------- engine
PRESETS = {
    # TinyLlama-1.1B (llama_run/src/main.rs:318-332)
    "tinyllama-1.1b": dict(dim=2048, n_layers=22, n_heads=32, n_kv_heads=4, head_dim=64, ffn=5632,
                           vocab=32000, theta=10000.0, eps=1e-5),
    # Llama-3-8B architecture
    "llama3-8b": dict(dim=4096, n_layers=32, n_heads=32, n_kv_heads=8, head_dim=128, ffn=14336,
                      vocab=128256, theta=500000.0, eps=1e-5),
    # the reference's random-weight harness shape (llama_decode/src/main.rs:289-298)
    "llama3.2-1b": dict(dim=2048, n_layers=16, n_heads=32, n_kv_heads=8, head_dim=64, ffn=8192,
                        vocab=128256, theta=500000.0, eps=1e-5),
}


def model_config(preset=None, max_seq=2048, **kw) -> ModelConfig:
    d = dict(PRESETS[preset]) if preset else {}
    d.update(kw)
    d["max_seq"] = max_seq
    return ModelConfig(**d)


def fp4_quantize_absmax(w: np.ndarray):
    """The reference's host packer: (packed u32 [rows*k/8], f32 scales [rows*k/32])."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, k = w.shape
    packed = np.zeros(rows * k // 8, dtype=np.uint32)
    scales = np.zeros(rows * k // 32, dtype=np.float32)
    check(load().fp4_quantize_absmax(w.ctypes.data, rows, k, packed.ctypes.data, scales.ctypes.data))
    return packed, scales


class SafeTensors:
    """Read-only safetensors view (rfp4_st_*): names, dtype/shape, f32 widening."""

    def __init__(self, path: str):
        h = P()
        check(load().rfp4_st_open(os.fsencode(path), C.byref(h)))
        self.h = h.value

    def close(self):
        if self.h:
            check(load().rfp4_st_close(self.h))
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def names(self):
        n = U32(0)
        check(load().rfp4_st_count(self.h, C.byref(n)))
        out = []
        for i in range(n.value):
            p = C.c_char_p()
            check(load().rfp4_st_name(self.h, i, C.byref(p)))
            out.append(p.value.decode())
        return out

    def info(self, name: str):
        dt = C.create_string_buffer(8)
        nd = U32(0)
        shape = (U64 * 8)()
        nb = U64(0)
        check(load().rfp4_st_info(self.h, name.encode(), dt, C.byref(nd), C.cast(shape, P), C.byref(nb)))
        return dt.value.decode(), tuple(shape[i] for i in range(nd.value)), nb.value

    def read_f16(self, name: str) -> np.ndarray:
        """fp16 bit patterns (uint16): F16 as stored, BF16 / F32 rounded to nearest even."""
        _, shape, _ = self.info(name)
        out = np.empty(int(np.prod(shape)) if shape else 1, dtype=np.uint16)
        check(load().rfp4_st_read_f16(self.h, name.encode(), out.ctypes.data, out.size))
        return out.reshape(shape)

    def read_f32(self, name: str) -> np.ndarray:
        _, shape, _ = self.info(name)
        out = np.empty(int(np.prod(shape)) if shape else 1, dtype=np.float32)
        check(load().rfp4_st_read_f32(self.h, name.encode(), out.ctypes.data, out.size))
        return out.reshape(shape)


class Engine:
    """llama_engine: weights, KV caches and the captured step graphs."""

    def __init__(self, cfg: ModelConfig, seed: int, _handle=None):
        init()
        self.cfg = cfg
        if _handle is None:
            h = P()
            check(load().llama_engine_create(C.byref(cfg), seed, C.byref(h)))
            _handle = h.value
        self.h = _handle
        self.stream = Stream(load().llama_engine_stream(self.h))
        _live.add(self)

    @classmethod
    def from_safetensors(cls, cfg: ModelConfig, path: str) -> "Engine":
        """Real weights from a safetensors checkpoint (MXFP4 by the OCP rules)."""
        init()
        h = P()
        check(load().llama_engine_create_from_safetensors(C.byref(cfg), os.fsencode(path), C.byref(h)))
        return cls(cfg, 0, _handle=h.value)

    @classmethod
    def load(cls, path: str, max_seq: int) -> "Engine":
        """An engine rebuilt from a packed-weight file written by save()."""
        init()
        h = P()
        check(load().llama_engine_load(os.fsencode(path), max_seq, C.byref(h)))
        cfg = ModelConfig()
        check(load().llama_engine_info(h.value, C.byref(cfg), None))
        return cls(cfg, 0, _handle=h.value)

    def save(self, path: str):
        check(load().llama_engine_save(self.h, os.fsencode(path)))

    def embed_bf16(self) -> bool:
        b = C.c_int(0)
        check(load().llama_engine_info(self.h, None, C.byref(b)))
        return bool(b.value)

    def prefill_kv(self, seed: int, upto: int):
        check(load().llama_engine_prefill_kv(self.h, seed, upto))

    def prefill(self, prompt, pos0: int) -> int:
        """Batched prefill of prompt at positions pos0..; returns the next greedy token."""
        pr = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = U32(0)
        check(load().llama_engine_prefill(self.h, pr.ctypes.data, len(pr), pos0, C.byref(out)))
        return out.value

    def prefill_stop(self, prompt, pos0: int, after: int):
        """Test hook: the batched prefill stopped after one stage (-1: the
        embedding; 10 * layer + s: stage s of that layer); read the stage's
        output with prefill_buffer."""
        check(load().rfp4_debug_prefill_stop(after))
        try:
            self.prefill(prompt, pos0)
        finally:
            check(load().rfp4_debug_prefill_stop(-2))

    def prefill_buffer(self, name: str, shape, dtype=np.float32) -> np.ndarray:
        """Copy of the prefill workspace buffer `name` (x, codes, scales, c, a), first prod(shape) elements."""
        ptrs = [P() for _ in range(5)]
        cap = U32(0)
        check(load().llama_engine_prefill_buffers(self.h, *[C.byref(q) for q in ptrs], C.byref(cap)))
        src = dict(zip(("x", "codes", "scales", "c", "a"), ptrs))[name].value
        out = np.empty(shape, dtype=dtype)
        check(load().rfp4_d2h(out.ctypes.data, src, out.nbytes, self.stream.h))
        check(load().rfp4_stream_synchronize(self.stream.h))
        return out

    def decode_step(self, tok: int, pos: int) -> int:
        out = U32(0)
        check(load().llama_decode_step(self.h, tok, pos, C.byref(out)))
        return out.value

    def generate(self, prompt, pos0: int, n_new: int) -> np.ndarray:
        pr = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.zeros(n_new, dtype=np.uint32)
        check(load().llama_generate(self.h, pr.ctypes.data, len(pr), pos0, n_new, out.ctypes.data))
        return out

    def begin(self, prompt, pos0: int, ids_cap: int):
        pr = np.ascontiguousarray(prompt, dtype=np.uint32)
        check(load().llama_engine_begin(self.h, pr.ctypes.data, len(pr), pos0, ids_cap))

    def begin_harness(self, ctx: int, ids_cap: int):
        """llama_decode's harness (f32-scale engines): context [0, ctx) at 0.01,
        x = the harness vector; step i's argmax lands in ids[1 + i]."""
        check(load().llama_engine_begin_harness(self.h, ctx, ids_cap))

    def run_steps(self, n: int):
        check(load().llama_engine_run_steps(self.h, n))

    def time_steps(self, n: int, cap: int = 16384) -> list:
        """n more steps with every kernel timed in place: [(name, us)] in launch order."""
        buf = (KernelTime * cap)()
        cnt = U32(0)
        check(load().llama_engine_time_steps(self.h, n, buf, cap, C.byref(cnt)))
        return [(buf[i].name.decode(), float(buf[i].us)) for i in range(min(cnt.value, cap))]

    def read_ids(self, count: int) -> np.ndarray:
        out = np.zeros(count, dtype=np.uint32)
        check(load().llama_engine_read_ids(self.h, out.ctypes.data, count))
        return out

    def logits(self) -> np.ndarray:
        out = np.zeros(self.cfg.vocab, dtype=np.float32)
        check(load().llama_engine_logits(self.h, out.ctypes.data))
        return out

    def use_graph(self, on: bool):
        check(load().llama_engine_use_graph(self.h, int(on)))

    def use_persistent(self, on: bool):
        check(load().llama_engine_use_persistent(self.h, int(on)))

    @property
    def persistent(self) -> bool:
        return bool(load().llama_engine_persistent(self.h))

    @property
    def persistent_available(self) -> bool:
        """True where use_persistent(True) succeeds (the shape it is compiled for)."""
        if self.persistent:
            return True
        try:
            self.use_persistent(True)
        except Rfp4Error:
            return False
        self.use_persistent(False)
        return True

    def weight(self, layer: int, proj: int):
        c, s, cb, sb = P(), P(), SZ(), SZ()
        check(load().llama_engine_weight(self.h, layer, proj, C.byref(c), C.byref(s), C.byref(cb), C.byref(sb)))
        return c.value, s.value, cb.value, sb.value

    def weight_scales_tiled(self, layer: int, proj: int):
        """(device pointer, bytes) of the weight's step-blocked scale copy."""
        p, n = C.c_void_p(), SZ(0)
        check(load().llama_engine_weight_scales_tiled(self.h, layer, proj, C.byref(p), C.byref(n)))
        return p.value, n.value

    def weight_host(self, layer: int, proj: int):
        c, s, cb, sb = self.weight(layer, proj)
        codes = np.empty(cb, dtype=np.uint8)
        scales = np.empty(sb, dtype=np.uint8)
        check(load().rfp4_d2h(codes.ctypes.data, c, cb, self.stream.h))
        check(load().rfp4_d2h(scales.ctypes.data, s, sb, self.stream.h))
        return codes, (scales.view(np.float32) if self.cfg.scale_format == SCALE_F32 else scales)

    def kv_host(self, layer: int):
        k, v, n = P(), P(), SZ()
        check(load().llama_engine_kv(self.h, layer, C.byref(k), C.byref(v), C.byref(n)))
        dt = np.float32 if self.cfg.kv_format == KV_F32 else np.uint16
        ka = np.empty(n.value, dtype=dt)
        va = np.empty(n.value, dtype=dt)
        check(load().rfp4_d2h(ka.ctypes.data, k.value, ka.nbytes, self.stream.h))
        check(load().rfp4_d2h(va.ctypes.data, v.value, va.nbytes, self.stream.h))
        return ka, va

    def debug_wait(self, nsplit: int, set_error: bool = False) -> dict:
        """Test hook: whether the step's device-side waits report to the
        engine's error word (and, with set_error, set that word)."""
        w, c, f = I32(0), I32(0), I32(0)
        check(load().rfp4_debug_engine_wait(self.h, int(set_error), nsplit, C.byref(w), C.byref(c), C.byref(f)))
        return {"err_wired": bool(w.value), "checked": bool(c.value), "fused": bool(f.value)}

    def weight_bytes(self) -> int:
        return int(load().llama_engine_weight_bytes(self.h))

    def close(self):
        if self.h:
            load().llama_engine_destroy(self.h)
            self.h = None

    _release = close

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
