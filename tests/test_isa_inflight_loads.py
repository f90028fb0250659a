"""Compiled-code check (CPU): no register of an in-flight inline-asm load is reused.

The fused NF4 GEMMs (forward and dX) and the streaming kernels issue vector loads from inline
asm, which the compiler does not track: it takes their destination registers
as written at the asm statement.  A load whose result is never consumed is
then dead to the compiler, which may hand its registers to other values while
the load is still in flight; the late return overwrites them (this turned
epilogue store addresses into garbage once).  The kernels keep every such
register live until an explicit vmcnt wait has retired its load.

This test compiles the sources to gfx950 assembly and follows the vector
memory counter through each kernel in program order (s_waitcnt vmcnt(N)
retires all but the newest N operations): no VALU or LDS instruction may read
or write a destination register of an asm-issued load that is still
outstanding.  The scan is linear in layout order: it does not follow branches
or loop back-edges.  It is paired with a rule the kernels keep: every register
of an asm load ring is tied after the kernel's final vmcnt(0), so a load left
in flight on a loop exit (a skipped guarded issue, a wave without work) keeps
its registers allocated until that wait, and the code the scan checks between
an issue and its wait is the code that runs between them.
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


def _regs(tok):
    m = re.match(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def inflight_hazards(asm, name):
    """(line, instruction, load) triples where `name` touches a pending asm load's registers."""
    start = asm.index(name + ":")
    end = asm.index(".Lfunc_end", start)
    pending, found, in_asm = [], [], False
    for raw in asm[start:end].split("\n"):
        line = raw.strip()
        if ";;#ASMSTART" in line:
            in_asm = True
            continue
        if ";;#ASMEND" in line:
            in_asm = False
            continue
        if not line or line.startswith((";", ".")):
            continue
        parts = line.split(";")[0].replace(",", " ").split()
        op = parts[0]
        if op.startswith("s_waitcnt"):
            m = re.search(r"vmcnt\((\d+)\)", line)
            if m:
                keep = int(m.group(1))
                pending = pending[len(pending) - keep:] if keep < len(pending) else pending
            continue
        if op.startswith(("global_", "buffer_", "flat_")):
            dest = set() if ("lds" in op or "store" in op or not in_asm) else _regs(parts[1])
            pending.append((dest, line))
            continue
        if op.startswith(("v_", "ds_")) and len(parts) > 1:
            touched = set().union(*(_regs(t) for t in parts[1:]))
            for dest, load in pending:
                if touched & dest:
                    found.append((line, load))
                    break
    return found


@pytest.mark.parametrize("source,kernel", [("gemm_nf4.hip", "gemm_nf4_kernel"),
                                           ("gemm_nf4.hip", "gemm_nf4t_kernel"),
                                           ("nf4_stream.hip", "nf4_stream_fwd_kernel"),
                                           ("nf4_stream_dx.hip", "nf4_stream_dx_kernel")])
def test_no_register_reuse_under_inflight_asm_loads(tmp_path, source, kernel):
    out = tmp_path / (source + ".s")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off", "-Xclang",
           "-target-feature", "-Xclang", "-packed-fp32-ops", "--cuda-device-only", "-S",
           "-I", str(ROOT / "include"), "-o", str(out), str(CSRC / source)]
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, cwd=tmp_path)
    assert res.returncode == 0, res.stdout.decode(errors="replace")[-2000:]
    asm = out.read_text()
    names = [n for n in re.findall(r"^(_Z\w*):", asm, re.M) if kernel in n]
    assert names, f"no {kernel} instantiation in {source}"
    for name in names:
        hazards = inflight_hazards(asm, name)
        assert not hazards, f"{name}: {hazards[:3]}"
