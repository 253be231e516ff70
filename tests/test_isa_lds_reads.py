"""The tiled MXFP4 GEMM reads its LDS operands with inline-asm ds_read
instructions (device/gemm.h: the compiler would otherwise wait for every LDS
DMA in flight before each read) and waits for them with explicit lgkmcnt
waits, the fragments tied to each wait.  The compiler sees an asm read's
registers as written at once, so nothing but those ties keeps it from
reading, copying or spilling a register whose load has not returned.  This
test disassembles the built gfx950 code object (LLVM tools on this build's
own output) and checks every tiled GEMM kernel: no instruction may read or
overwrite a destination register of a ds_read before the s_waitcnt lgkmcnt
that completes that read (LDS reads retire in issue order, so lgkmcnt(N)
completes all but the last N), scanning each kernel in code order.  CPU only."""
import os
import re
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HSACO = os.path.join(ROOT, "rust-fp4-blackwell_amd", "build", "kernels.hsaco")
LLVM = "/opt/rocm/llvm/bin"
TILED = re.compile(r"^rfp4_gemm_\d+x\d+(_p\d|_pp|_ppsw)?(_rope)?$")


def _regs(text):
    out = set()
    for a, b, c in re.findall(r"\bv\[(\d+):(\d+)\]|\bv(\d+)\b", text):
        if c:
            out.add(int(c))
        else:
            out |= set(range(int(a), int(b) + 1))
    return out


def scan(lines):
    """[(line, instruction, registers)] of instructions that touch a register
    of an LDS read still in flight, over one kernel's disassembly."""
    fifo, bad = [], []
    for ln, raw in enumerate(lines):
        t = raw.split("//")[0].split(";")[0].strip()
        if not t or t.endswith(":") or t.startswith("."):
            continue
        op, _, rest = t.partition(" ")
        if op.startswith("ds_read"):
            dst = rest.split(",")[0]
            # an LDS read whose address register is still in flight is a touch too
            hit = _regs(rest.split(",", 1)[1] if "," in rest else "") & set().union(*fifo) if fifo else set()
            if hit:
                bad.append((ln, t, sorted(hit)))
            fifo.append(_regs(dst))
            continue
        m = re.match(r"s_waitcnt\b.*lgkmcnt\((\d+)\)", t)
        if m:
            n = int(m.group(1))
            del fifo[:max(0, len(fifo) - n)]
            continue
        if fifo:
            hit = _regs(rest) & set().union(*fifo)
            if hit:
                bad.append((ln, t, sorted(hit)))
    return bad


def test_scan_flags_planted_hazards():
    """The scanner itself: a use, a copy and a spill of an in-flight register
    are flagged; a use after the wait that completes it, or after a partial
    wait that leaves only later reads out, is not."""
    ok = ["ds_read_b128 v[0:3], v20", "ds_read_b128 v[4:7], v21", "s_waitcnt lgkmcnt(1)",
          "v_mfma_scale_f32_32x32x64_f8f6f4 a[0:15], v[0:3], v[8:11], a[0:15], v30, v31",
          "s_waitcnt lgkmcnt(0)", "v_mov_b32_e32 v40, v5"]
    assert scan(ok) == []
    for planted in ("v_mov_b32_e32 v40, v5", "scratch_store_dwordx4 off, v[4:7], off",
                    "v_mfma_scale_f32_32x32x64_f8f6f4 a[0:15], v[4:7], v[8:11], a[0:15], v30, v31"):
        lines = ok[:3] + [planted] + ok[3:]
        assert [b[1] for b in scan(lines)] == [planted], planted


def _disassembly():
    if not os.path.exists(HSACO) or not os.path.exists(os.path.join(LLVM, "llvm-objdump")):
        pytest.skip("built code object or LLVM tools not present")
    with tempfile.TemporaryDirectory() as d:
        elf = os.path.join(d, "k.elf")
        r = subprocess.run([os.path.join(LLVM, "clang-offload-bundler"), "--unbundle", "--type=o",
                            "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--input={HSACO}", f"--output={elf}"],
                           capture_output=True, text=True)
        if r.returncode:
            pytest.skip("clang-offload-bundler failed: " + r.stderr[-200:])
        return subprocess.run([os.path.join(LLVM, "llvm-objdump"), "-d", "--no-show-raw-insn", elf],
                              capture_output=True, text=True, check=True).stdout


def test_tiled_gemm_kernels_never_touch_registers_of_reads_in_flight():
    kernels, cur = {}, None
    for line in _disassembly().splitlines():
        m = re.match(r"^[0-9a-f]+ <([A-Za-z0-9_]+)>:", line)
        if m:
            cur = m.group(1)
            kernels[cur] = []
        elif cur:
            kernels[cur].append(line)
    tiled = sorted(k for k in kernels if TILED.match(k))
    assert len(tiled) >= 10, tiled
    bad = {}
    for k in tiled:
        assert sum(1 for l in kernels[k] if "ds_read" in l) > 20, k  # the scan sees the asm reads
        hits = scan(kernels[k])
        if hits:
            bad[k] = hits[:5]
    assert not bad, bad
