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


def build(verbose=False, jobs=None, address_sanitizer=False):
    """Compile all sources to objects in parallel, then link the shared library.

    address_sanitizer=True builds a copy with AddressSanitizer in the host code
    only (the device code is compiled as usual), for CPU runs of the C ABI's
    argument checks and host arithmetic, into _build/asan/libsoupsuck_amd.so;
    the GPU library is untouched.
    """
    objdir = PACKAGE / "_build" / ("asan" if address_sanitizer else "")
    objdir.mkdir(parents=True, exist_ok=True)
    common = [hipcc(), f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
              "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
              "-Wall", "-Wno-unused-function", "-I", str(PACKAGE.parent / "include")]
    sanitize = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer"]
    if address_sanitizer:
        common = common + ["-g"] + sanitize
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
    target = objdir / LIBRARY.name if address_sanitizer else LIBRARY
    tmp = str(target) + ".tmp"
    link = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objects
    if address_sanitizer:
        link += sanitize
    res = subprocess.run(link, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    if res.returncode != 0:
        raise RuntimeError("link failed:\n" + res.stdout.decode(errors="replace"))
    os.replace(tmp, target)
    return target


def built_library(address_sanitizer=False):
    """The library, built first if it is missing or older than a source or header."""
    target = (PACKAGE / "_build" / "asan" / LIBRARY.name) if address_sanitizer else LIBRARY
    inputs = [Path(p) for p in sources()] + list(CSRC.glob("*.h")) + \
        list((PACKAGE.parent / "include").glob("*.h"))
    if not target.exists() or target.stat().st_mtime < max(p.stat().st_mtime for p in inputs):
        return build(address_sanitizer=address_sanitizer)
    return target


def asan_runtime():
    """Path of the compiler's AddressSanitizer runtime (to preload into a host process)."""
    found = sorted(Path("/opt/rocm/llvm/lib/clang").glob("*/lib/linux/libclang_rt.asan-x86_64.so"))
    return found[-1] if found else None


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv, address_sanitizer="--asan" in sys.argv))
