"""The kernels' inline-asm LDS reads are waited for before any use.

Several kernels read LDS with `ds_read` inside inline asm and wait for the
data with a separate `s_waitcnt lgkmcnt` statement (so the reads overlap
other work). The compiler takes an asm output as ready where the statement
ends: if it decides to copy such a register, or to reuse it, before the
wait, the kernel uses data that has not arrived, which no GPU run reports as
an error. This test compiles the sources that hold such reads to gfx950
assembly (hipcc, no GPU) and scans every kernel in straight-line order:
a register written by an asm `ds_read` stays pending until an
`s_waitcnt lgkmcnt(N)` retires it (LDS operations complete in order, so
lgkmcnt(N) retires all but the newest N), and no instruction may read or
write a pending register before that.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "tao-memory_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
SOURCES = ("prefill.hip", "local_attn.hip", "writer.hip")

_REG = re.compile(r"v\[(\d+):(\d+)\]|v(\d+)\b")


def _regs(text):
    out = set()
    for m in _REG.finditer(text):
        if m.group(1) is not None:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
        else:
            out.add(int(m.group(3)))
    return out


def scan(lines):
    """Hazards in one kernel's assembly lines: [(line, text, registers)]."""
    pending = []          # [(registers or empty set)] in issue order, LDS/SMEM ops
    in_asm = False
    found = []
    for i, raw in enumerate(lines):
        s = raw.strip()
        if s.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if s.startswith(";;#ASMEND"):
            in_asm = False
            continue
        s = s.split(";")[0].strip()
        if not s or s.endswith(":") or s.startswith("."):
            continue
        op, _, operands = s.partition(" ")
        if op == "s_waitcnt":
            m = re.search(r"lgkmcnt\((\d+)\)", operands)
            if m:
                n = int(m.group(1))
                pending = pending[len(pending) - n:] if 0 < n < len(pending) else (
                    [] if n == 0 else pending)
            continue
        counted = op.startswith("ds_") or op.startswith("s_load") or op.startswith("s_buffer_load")
        parts = [p.strip() for p in operands.split(",")]
        if op.startswith("ds_read") and in_asm:
            dst, srcs = _regs(parts[0]), _regs(",".join(parts[1:]))
        elif op.startswith("ds_read"):
            dst, srcs = set(), _regs(",".join(parts[1:]))
        else:
            dst, srcs = set(), _regs(operands)
        busy = set().union(*pending) if pending else set()
        hit = busy & srcs
        if hit:
            found.append((i, s, sorted(hit)))
        if counted:
            pending.append(dst)
    return found


def kernels(asm):
    names = re.findall(r"^(_Z\w+):", asm, re.M)
    for name in names:
        start = asm.index(name + ":")
        end = asm.find("s_endpgm", start)
        if end > start:
            yield name, asm[start:end].splitlines()


def test_scan_flags_a_copy_before_the_wait():
    lines = """
        ;;#ASMSTART
        ds_read_b128 v[2:5], v2
        ;;#ASMEND
        ;;#ASMSTART
        ds_read_b128 v[42:45], v31
        ;;#ASMEND
        v_mov_b32_e32 v30, v42
        ;;#ASMSTART
        s_waitcnt lgkmcnt(0)
        ;;#ASMEND
        v_mfma_f32_32x32x16_bf16 v[62:77], v[2:5], v[30:33], v[62:77]
    """.splitlines()
    found = scan(lines)
    assert len(found) == 1 and found[0][2] == [42]
    # The same reads with the wait first are clean; lgkmcnt(1) retires the
    # older read only.
    ok = """
        ;;#ASMSTART
        ds_read_b128 v[2:5], v2
        ;;#ASMEND
        ;;#ASMSTART
        ds_read_b128 v[42:45], v31
        ;;#ASMEND
        s_waitcnt lgkmcnt(1)
        v_mov_b32_e32 v30, v2
        s_waitcnt lgkmcnt(0)
        v_mov_b32_e32 v30, v42
    """.splitlines()
    assert scan(ok) == []


@pytest.mark.skipif(not shutil.which(HIPCC) and not os.path.exists(HIPCC), reason="no hipcc")
@pytest.mark.parametrize("source", SOURCES)
def test_asm_lds_reads_are_waited_for(source, tmp_path):
    out = tmp_path / (source + ".s")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "--cuda-device-only", "-S", os.path.join(CSRC, source), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    asm = out.read_text()
    checked, problems = 0, []
    for name, lines in kernels(asm):
        if not any(";;#ASMSTART" in ln for ln in lines):
            continue
        checked += 1
        for i, text, regs in scan(lines):
            problems.append(f"{name} line {i}: {text} uses {regs} before its wait")
    assert checked > 0
    assert not problems, "\n".join(problems[:20])
