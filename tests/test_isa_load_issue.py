"""Compiled-code check (CPU): the bandwidth kernels' row loads are in flight together.

Any if/else around a load (a per-lane length guard, a run-time dtype switch) makes the
compiler wait with `s_waitcnt vmcnt(0)` where the paths join, so the next load starts
only after the previous one returned: a row then costs one memory round trip per load
instead of one in all (the add-RMSNorm rows took twice as long that way).  The fast
paths take their dtypes as template arguments and clamp addresses instead of branching.

This test compiles the sources to gfx950 assembly and counts, for each listed kernel
instantiation, the global loads issued (in layout order) before its first vmcnt(0)
wait: at least the loads of one row's data (partial waits for older loads are fine).
"""

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "soupsuck_amd" / "csrc"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

pytestmark = pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc not available")


def loads_before_full_wait(asm, name):
    start = asm.index(name + ":")
    end = asm.index(".Lfunc_end", start)
    count = 0
    for raw in asm[start:end].split("\n"):
        line = raw.strip()
        if not line or line.startswith((";", ".")):
            continue
        op = line.split()[0]
        if op.startswith(("global_load", "buffer_load")):
            count += 1
        elif op.startswith("s_waitcnt") and "vmcnt(0)" in line and count:
            break
    return count


def assembly(tmp_path, source):
    out = tmp_path / (source + ".s")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off", "-Xclang",
           "-target-feature", "-Xclang", "-packed-fp32-ops", "--cuda-device-only", "-S",
           "-I", str(ROOT / "include"), "-o", str(out), str(CSRC / source)]
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, cwd=tmp_path)
    assert res.returncode == 0, res.stdout.decode(errors="replace")[-2000:]
    return out.read_text()


# (source, mangled-name pattern, loads of one row's data that must be in flight together)
CASES = [
    # add-RMSNorm fast forward, h = 1536 / 3584: r and d chunks (NCH = 3 / 7)
    ("add_rmsnorm.hip", r"add_rmsnorm_fwd_fast_kernelILi3ELb1ELb[01]E", 6),
    ("add_rmsnorm.hip", r"add_rmsnorm_fwd_fast_kernelILi7ELb1ELb[01]E", 14),
    # standalone RMSNorm fast forward: x chunks
    ("add_rmsnorm.hip", r"add_rmsnorm_fwd_fast_kernelILi3ELb0ELb[01]E", 3),
    # fast backward (plain and with dgamma): s, gy and gs chunks
    ("add_rmsnorm.hip", r"add_rmsnorm_bwd_kernelILi3ELi[12]E", 9),
    ("add_rmsnorm.hip", r"add_rmsnorm_bwd_dg_kernelILi3ELi[12]E", 9),
    ("add_rmsnorm.hip", r"add_rmsnorm_bwd_dg_kernelILi7ELi[12]E", 21),
    # RoPE vector kernel with template dtypes: x1, x2, c1, c2, s1, s2
    ("rope.hip", r"rope_vec_kernelILb[01]ELi[01]E", 6),
    # SwiGLU fp16 vector kernel: g, u (and da backward)
    ("swiglu.hip", r"swiglu_vec_kernelILb1ELb1E", 3),
    ("swiglu.hip", r"swiglu_vec_kernelILb0ELb1E", 2),
    # CE statistics: the lane's four 16-byte logit loads
    ("cross_entropy.hip", r"ce_stats_kernelILb1E", 4),
]


@pytest.mark.parametrize("source", sorted({c[0] for c in CASES}))
def test_row_loads_are_issued_together(tmp_path, source):
    asm = assembly(tmp_path, source)
    names = re.findall(r"^(_Z\w*):", asm, re.M)
    for src, pattern, need in CASES:
        if src != source:
            continue
        hits = [n for n in names if re.search(pattern, n)]
        assert hits, f"no instantiation matching {pattern} in {source}"
        for name in hits:
            got = loads_before_full_wait(asm, name)
            assert got >= need, f"{name}: {got} loads before the first vmcnt(0), need {need}"
