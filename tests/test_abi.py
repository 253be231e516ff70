"""The C-ABI boundary on the CPU: the library loads, exports every function
include/rfp4.h declares, validates arguments before touching a device, and
is built without any link to the oracle.  No GPU compute calls."""
import os
import re
import subprocess

import pytest

import rfp4

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "rust-fp4-blackwell_amd")


def test_library_exports_every_declared_function():
    lib = rfp4.load()
    names = rfp4.header_functions()
    assert len(names) > 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_the_header():
    names = set(rfp4.header_functions())
    assert names <= set(rfp4._SIGS), sorted(names - set(rfp4._SIGS))


def test_reference_entry_points_present():
    """The reference's kernel names (llama_run/src/main.rs:34-315,
    fp4_mma/src/main.rs:19) are all exported under the same names."""
    for n in ("fp4_gemv", "rmsnorm", "rope", "copy_into", "attn_decode", "swiglu", "residual", "argmax",
              "fp4_mma_allones"):
        assert n in rfp4.header_functions()


def _bundle_kernel_symbols():
    """Kernel descriptor symbols of the built code object, read with the LLVM
    tools (an independent reading of the same file)."""
    import tempfile
    hsaco = os.path.join(PKG, "build", "kernels.hsaco")
    llvm = "/opt/rocm/llvm/bin"
    if not os.path.exists(hsaco) or not os.path.exists(os.path.join(llvm, "llvm-readelf")):
        pytest.skip("built code object or LLVM tools not present")
    with tempfile.TemporaryDirectory() as d:
        elf = os.path.join(d, "k.elf")
        r = subprocess.run([os.path.join(llvm, "clang-offload-bundler"), "--unbundle", "--type=o",
                            "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--input={hsaco}", f"--output={elf}"],
                           capture_output=True, text=True)
        if r.returncode:
            pytest.skip("clang-offload-bundler failed: " + r.stderr[-200:])
        out = subprocess.run([os.path.join(llvm, "llvm-readelf"), "--syms", elf], capture_output=True,
                             text=True).stdout
    return sorted({w[:-3] for w in out.split() if w.endswith(".kd")})


def test_kernel_table_matches_the_code_object():
    """The runtime resolves every kernel handle at init from the embedded code
    object's symbol table (no lookup, and no map update, after init): its
    parser agrees with the LLVM tools on the built file, and every kernel the
    host launches by a literal name is present."""
    names = rfp4.kernel_names()
    assert len(names) == len(set(names)) and len(names) > 100
    assert sorted(names) == _bundle_kernel_symbols()
    literal = set()
    for f in ("runtime.cpp", "engine.cpp"):
        literal |= set(re.findall(r'"(rfp4_[a-z0-9_]+)"', open(os.path.join(PKG, "csrc", f)).read()))
    missing = sorted(n for n in literal if n not in names)
    assert not missing, missing
    for hd in (64, 128):
        for kv in ("f16", "f32"):
            for g in (1, 2, 4, 8):
                assert f"rfp4_attn_hd{hd}_{kv}_g{g}" in names


def test_shape_errors_need_no_device():
    lib = rfp4.load()
    p = 0x10000  # never dereferenced: validation fails first
    assert lib.mx4_gemv(None, 16, 33, p, p, p, p) == -2          # K not a multiple of 32
    assert b"multiple of the 32-element block" in lib.rfp4_last_error()
    assert lib.mx4_gemv(None, 0, 64, p, p, p, p) == -2            # N = 0
    assert lib.fp4_gemv(None, 16, 64, None, p, p, p) == -1         # null pointer
    assert lib.mx4_gemv(None, 16, 64, p + 4, p, p, p) == -6       # misaligned codes
    assert lib.mx4_gemv_swiglu(None, 16, 64, 8, p, p, p, p) == -2  # up rows overlap gate rows
    assert lib.fp4_gemm(None, 32, 4096, 4000, p, p, p, p, p) == -2  # K not a multiple of 256
    assert lib.fp4_gemm(None, 32, 4098, 4096, p, p, p, p, p) == -2  # N not a multiple of 4
    assert lib.fp4_gemm(None, 0, 4096, 4096, p, p, p, p, p) == -2   # M = 0
    assert lib.fp4_gemm(None, 32, 4096, 4096, p + 8, p, p, p, p) == -6  # misaligned codes
    assert lib.fp4_gemm(None, 32, 4096, 4096, p, p + 4, p, p, p) == -6  # misaligned scales
    assert lib.fp4_gemm(None, 32, 4096, 4096, None, p, p, p, p) == -1
    assert lib.rfp4_debug_gemm_plan(6, 0) == -1


@pytest.mark.parametrize("m", [1, 32, 80, 512, 2048, 4096])
@pytest.mark.parametrize("n,k", [(4096, 4096), (1024, 4096), (14336, 4096), (28672, 4096), (4096, 14336),
                                 (128256, 4096), (292, 1024)])
def test_gemm_plan_shapes(m, n, k):
    """The automatic GEMM plan (256 CUs without a device): a compiled tile, no
    empty K split, the split-K partials fit the workspace, and the CUs covered
    (at least 7/8 of them; at least half from 1024 rows or with a short K,
    under 32 steps, which runs unsplit from half the CUs) unless the K split
    is at its maximum."""
    tm, tn, kz = rfp4.gemm_plan(m, n, k)
    if m <= 32 and k % 512 == 0:   # few-row kernel: kz = W fragments per workgroup
        nf = next(f for f in (4, 2, 1) if f == 1 or (4 * -(-n // (16 * f)) >= 3 * 256 and k <= (4096 if f == 4 else 8192)))
        assert (tm, tn, kz) == (16 if m <= 16 else 32, 16 * nf, nf)
        return
    assert (tm, tn) in [(256, 256), (256, 128), (128, 128), (64, 128), (32, 128)]
    nsuper = k // 256
    per = -(-nsuper // kz)
    assert 1 <= kz <= nsuper and (kz - 1) * per < nsuper
    assert kz == 1 or kz * m * n <= (8 << 20)
    tiles = -(-m // tm) * -(-n // tn)
    cover = 128 if m >= 1024 or nsuper < 32 else 224
    assert tiles * kz >= cover or kz == nsuper or (kz + 1) * m * n > (8 << 20)
    if m > 32:
        assert -(-m // tm) * tm <= 1.25 * m or tm == 32   # bounded row padding


@pytest.mark.parametrize("m,n,k,plan", [
    (512, 28672, 4096, (256, 256, 1)),   # one round of 256x256 at 7/8 of the CUs (47.9 us, best of the sweep)
    (512, 4096, 14336, (128, 128, 2)),   # long K: one round of 128x128 in two splits, 3 stages (ahead inside the stack)
    (512, 14336, 4096, (256, 128, 1)),   # one round of 256x128, double-buffered (25.4 vs 29.2 us with 3 stages)
    (512, 6144, 4096, (128, 128, 1)),    # one round of 128x128 over 3/4 of the CUs (in the stack, 2 us per layer less than 64x128)
    (128, 28672, 4096, (128, 128, 1)),   # the same rule (18.5 vs 18.8 us for 64x128)
    (128, 6144, 4096, (32, 128, 1)),     # short K over 3/4 of the CUs unsplit (8.2 vs 11.1 us in two splits)
    (256, 28672, 4096, (256, 128, 1)),   # one round of 256x128 (26.4 vs 34.0 us for 128x128)
    (2048, 6144, 4096, (256, 256, 1)),   # fewest resident rounds (49.7 us, within 2 % of the best)
    (2048, 4096, 4096, (256, 128, 1)),   # (27.3 vs 34.0 us for 128x128)
    (2048, 4096, 14336, (256, 128, 1)),  # (77.7 vs 92.1 us for 128x128)
    (2048, 28672, 4096, (256, 256, 1)),
    (32, 28672, 4096, (32, 64, 4)),      # few rows, 4 W fragments (17.7 us vs 21.5 tiled)
    (32, 6144, 4096, (32, 32, 2)),       # few rows, 2 W fragments (6.9 vs 7.9 with one)
    (32, 4096, 14336, (32, 16, 1)),      # few rows, 4 segments per wave (11.7 vs 15.4 tiled)
    (32, 128256, 4096, (32, 64, 4)),     # very wide, 4 W fragments (62.5 vs 68.4 us tiled)
])
def test_gemm_plan_measured_choices(m, n, k, plan):
    """The planner's choices on the 8B prefill and decode-batch shapes that
    were measured on MI355X (tile sweeps; times in the comments)."""
    assert rfp4.gemm_plan(m, n, k) == plan


def test_calls_before_init_fail_loudly():
    if rfp4.device_count() > 0:
        pytest.skip("a device is present: init would succeed")
    lib = rfp4.load()
    assert lib.rfp4_init(0) == -8                                  # no device: loud failure
    p = 0x10000
    assert lib.mx4_gemv(None, 16, 64, p, p, p, p) == -5            # not initialised
    assert lib.rmsnorm(None, 16, 1e-5, p, p, p) == -5
    cfg = rfp4.model_config("tinyllama-1.1b", max_seq=64)
    import ctypes as C
    h = C.c_void_p()
    assert lib.llama_engine_create(C.byref(cfg), 1, C.byref(h)) == -5
    assert h.value is None


def test_product_does_not_link_or_name_the_oracle():
    so = os.path.join(PKG, "librfp4.so")
    out = subprocess.run(["readelf", "-d", so], capture_output=True, text=True).stdout
    needed = re.findall(r"Shared library: \[(.*?)\]", out)
    assert needed and not any("oracle" in n for n in needed), needed
    for dirpath, _, files in os.walk(os.path.join(PKG, "csrc")):
        for f in files:
            text = open(os.path.join(dirpath, f), errors="ignore").read()
            assert "orc_" not in text and "pyoracle" not in text, f
    assert "pyoracle" not in open(os.path.join(PKG, "rfp4.py")).read()


def test_test_hooks_validate_arguments():
    """The thread-local test hooks reject values that name no compiled
    variant or mode (no device needed) and accept their automatic setting."""
    lib = rfp4.load()
    assert lib.rfp4_debug_prefill_waves(6) == -1
    assert lib.rfp4_debug_prefill_waves(16) == -1
    assert lib.rfp4_debug_prefill_pairing(3) == -1
    assert lib.rfp4_debug_prefill_attn(2) == -1
    assert lib.rfp4_debug_attn_merge(4) == -1
    assert lib.rfp4_debug_gemv_waves(2) == -1
    for hook in (lib.rfp4_debug_prefill_waves, lib.rfp4_debug_prefill_pairing, lib.rfp4_debug_prefill_attn,
                 lib.rfp4_debug_attn_merge, lib.rfp4_debug_gemv_waves):
        assert hook(0) == 0

