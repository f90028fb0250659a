"""Build the gfx950 shared library ``libsoupsuck_amd.so`` in-tree with hipcc.

One hipcc invocation compiles every ``csrc/*.hip`` source for gfx950 only.
Flags:
  -ffp-contract=off   keep a*b+c as two roundings (the reference launches every
                      kernel with enable_fp_fusion=False); bit-exact NF4 decode
                      depends on it;
  -Xclang -target-feature -Xclang -packed-fp32-ops
                      no packed fp32 VALU instructions in device code.
"""

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
LIBRARY = PACKAGE / "libsoupsuck_amd.so"
ARCH = "gfx950"


def hipcc():
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found; the soupsuck_amd HIP library cannot be built")
    return found


def sources():
    return sorted(str(p) for p in CSRC.glob("*.hip"))


def build(verbose=False, jobs=None):
    """Compile all sources to objects in parallel, then link the shared library."""
    objdir = PACKAGE / "_build"
    objdir.mkdir(exist_ok=True)
    common = [hipcc(), f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
              "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
              "-Wall", "-Wno-unused-function", "-I", str(PACKAGE.parent / "include")]
    procs = []
    objects = []
    for src in sources():
        obj = objdir / (Path(src).stem + ".o")
        objects.append(str(obj))
        cmd = common + ["-c", src, "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
    failed = []
    for src, proc in procs:
        out, _ = proc.communicate()
        text = out.decode(errors="replace")
        # hipcc's host pass does not know the device-only feature flag.
        text = "\n".join(l for l in text.splitlines() if "packed-fp32-ops" not in l)
        if proc.returncode != 0:
            failed.append((src, text))
        elif verbose and text.strip():
            print(text)
    if failed:
        msg = "\n".join(f"--- {src}\n{text}" for src, text in failed)
        raise RuntimeError(f"hipcc failed:\n{msg}")
    tmp = str(LIBRARY) + ".tmp"
    link = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objects
    res = subprocess.run(link, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    if res.returncode != 0:
        raise RuntimeError("link failed:\n" + res.stdout.decode(errors="replace"))
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
