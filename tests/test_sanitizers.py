"""The host code under AddressSanitizer + UndefinedBehaviorSanitizer: the
CPU tests of the C ABI (argument validation, the code-object parser, the
host packer) and of the safetensors reader (including malformed files), and
the oracle's own tests, rerun in a child process against the sanitizer
builds (`make asan` in the package and in oracle/; __graft_entry__.build()
makes them).  Any sanitizer report aborts the child, which fails this test.
CPU only."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "rust-fp4-blackwell_amd", "librfp4_asan.so")
ORC = os.path.join(ROOT, "oracle", "liboracle_asan.so")


def _runtime(name):
    r = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True)
    p = r.stdout.strip()
    return p if r.returncode == 0 and os.path.isabs(p) and os.path.exists(p) else None


@pytest.mark.parametrize("tests", [["tests/test_abi.py", "tests/test_loader.py"],
                                   ["tests/test_oracle.py", "tests/test_oracle_model.py"]])
def test_cpu_suite_under_asan_ubsan(tests):
    if not (os.path.exists(LIB) and os.path.exists(ORC)):
        pytest.skip("sanitizer builds not present (make asan)")
    asan = _runtime("libasan.so")
    if not asan:
        pytest.skip("libasan runtime not found")
    env = dict(os.environ, RFP4_LIB=LIB, RFP4_ORACLE_LIB=ORC, LD_PRELOAD=asan,
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-m", "not gpu", "-p", "no:cacheprovider",
                        "-k", "not sanitizer", *tests], cwd=ROOT, env=env, capture_output=True, text=True,
                       timeout=600)
    tail = (r.stdout + r.stderr)[-4000:]
    assert r.returncode == 0, tail
    assert "ERROR: AddressSanitizer" not in tail and "runtime error:" not in tail, tail
