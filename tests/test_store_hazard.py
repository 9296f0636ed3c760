"""Device-code check of the buffer stores (CPU: hipcc cross-compiles gfx950 assembly).

A buffer store of more than 64 bits needs one wait state before a VALU instruction may
overwrite its data registers. The compiler inserts that wait state only when the store's
scalar offset is a constant, not an SGPR; with an SGPR offset, gfx950 was measured to store the
overwritten values (the residual block of the fused head lost about 0.1 % of its entries to
address arithmetic issued right after the store). The kernels therefore keep every wide buffer
store's scalar offset constant; this test compiles each source that issues raw buffer stores
and checks the generated assembly for both conditions. Wide global stores (the head's staged
epilogues) are checked for the second condition too.
"""

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "algebraic-transformer_amd" / "csrc"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

WIDE_STORE = re.compile(r"^\s*buffer_store_(dwordx3|dwordx4|b96|b128)\s+(.*)$")
WIDE_GLOBAL_STORE = re.compile(r"^\s*global_store_(dwordx3|dwordx4|b96|b128)\s+(.*)$")


def _regs(tok):
    tok = tok.strip().rstrip(",")
    m = re.match(r"v\[(\d+):(\d+)\]$", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def _valu_dst(line):
    parts = line.split(None, 1)
    if len(parts) < 2 or not parts[0].startswith("v_") or parts[0].startswith("v_cmp"):
        return set()
    return _regs(re.split(r",\s*", parts[1])[0])


def _instructions(asm):
    out = []
    for raw in asm.split("\n"):
        s = raw.split(";")[0].strip()
        if not s or s.startswith("."):
            continue
        out.append("<label>" if s.endswith(":") else s)
    return out


def scan(asm):
    """Problems in gfx950 assembly: wide buffer stores with an SGPR scalar offset, and wide
    buffer stores whose data registers the next instruction overwrites."""
    ins = _instructions(asm)
    problems = []
    for k, s in enumerate(ins):
        g = WIDE_GLOBAL_STORE.match(s)
        if g:  # global_store vaddr, vdata, off
            data = _regs(re.split(r",\s*", g.group(2))[1])
            if k + 1 < len(ins) and _valu_dst(ins[k + 1]) & data:
                problems.append(f"data overwritten by the next instruction: {s} / {ins[k + 1]}")
            continue
        m = WIDE_STORE.match(s)
        if not m:
            continue
        ops = re.split(r",\s*", m.group(2))
        soffset = ops[3].split()[0] if len(ops) > 3 else "0"
        if re.match(r"s\d+$|s\[", soffset):
            problems.append(f"SGPR scalar offset: {s}")
        if k + 1 < len(ins) and _valu_dst(ins[k + 1]) & _regs(ops[0]):
            problems.append(f"data overwritten by the next instruction: {s} / {ins[k + 1]}")
    return problems


def test_scan_flags_the_hazard_forms():
    bad = """
        buffer_store_dwordx4 v[130:133], v149, s[0:3], s4 offen nt
        v_or_b32_e32 v130, 24, v148
    """
    good = """
        buffer_store_dwordx4 v[130:133], v149, s[0:3], 0 offen nt
        s_nop 0
        v_or_b32_e32 v130, 24, v148
        buffer_store_dwordx2 v[130:131], v149, s[0:3], s4 offen
    """
    assert len(scan(bad)) == 2
    assert scan(good) == []
    assert len(scan("global_store_dwordx4 v[2:3], v[8:11], off\nv_mov_b32_e32 v9, 0")) == 1
    assert scan("global_store_dwordx4 v[2:3], v[8:11], off\ns_nop 0\nv_mov_b32_e32 v9, 0") == []


SOURCES = sorted(p for p in CSRC.glob("*.hip") if "buffer_store" in p.read_text() or "store_block_bf16" in p.read_text())


@pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc not available")
@pytest.mark.parametrize("src", SOURCES, ids=[p.name for p in SOURCES])
def test_wide_buffer_stores_keep_a_constant_scalar_offset(src, tmp_path):
    out = tmp_path / (src.stem + ".s")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-munsafe-fp-atomics",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wno-unused-result",
           f"-I{ROOT / 'include'}", "--cuda-device-only", "-S", str(src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stderr[-2000:]
    problems = scan(out.read_text())
    assert not problems, "\n".join(problems[:10])
