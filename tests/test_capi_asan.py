"""The C ABI's host code under AddressSanitizer (CPU, no GPU).

Builds a host-only copy of the library with AddressSanitizer in the host code
(soupsuck_amd.build, address_sanitizer=True: no device code), preloads the
compiler's ASan runtime into a fresh Python process, and drives every host
path that runs without a GPU: argument rejection with its formatted error
message (including messages longer than the message buffer), workspace and
scratch sizing arithmetic, the no-alloc entry point's size limit, and error
messages raised from several threads at once (the message is per thread).  A
heap or stack error in that code makes the child process fail.
"""

import os
import subprocess
import sys
import textwrap
from pathlib import Path

import pytest

from soupsuck_amd import build

ROOT = Path(__file__).resolve().parents[1]

CHILD = textwrap.dedent("""
    import ctypes, sys, threading
    sys.path.insert(0, {root!r})
    from soupsuck_amd import _lib
    lib = _lib.load({lib!r})
    E = _lib.ERR_INVALID_ARGUMENT
    assert lib.ss_nf4_dequant_nested(None, None, None, None, None, None, -1, None) == E
    assert b"n=-1" in lib.ss_last_error()
    # the longest formatted messages (shapes near int64 limits)
    big = 2 ** 62
    assert lib.ss_nf4_gemm_fwd_noalloc(None, 64, big, None, None, None, None, None, big, 64,
                                       None, None, big, None) != 0
    assert len(lib.ss_last_error()) > 0
    for t in (1, 16, 128, 255, 256, 990, 16384):
        for n, k in ((3584, 3584), (512, 3584), (18944, 3584), (3584, 18944), (8960, 1536)):
            lib.ss_nf4_gemm_workspace_size(t, n, k)
            lib.ss_qlora_rank_workspace_size(t, n, k)
            lib.ss_lora_workspace_size(t, n)
            lib.ss_gemm_f16_workspace_size(0, 1, t, n, k)
        lib.ss_add_rmsnorm_dgamma_waves(t)
    buf = (ctypes.c_uint8 * 4096)()
    p = (ctypes.addressof(buf) + 255) // 256 * 256
    # no-alloc forward: a shape beyond its fixed scratch is rejected before any HIP call
    rc = lib.ss_nf4_gemm_fwd_noalloc(p, 3584, 4096, p, p, p, p, p, 18944, 3584, None, p, 18944,
                                     None)
    assert rc == E and b"scratch" in lib.ss_last_error(), lib.ss_last_error()
    errors = []
    def worker(i):
        for _ in range(200):
            rc = lib.ss_nf4_dequant_nested(None, None, None, None, None, None, -i - 1, None)
            msg = lib.ss_last_error()
            if rc != E or ("n=%d" % (-i - 1)).encode() not in msg:
                errors.append(msg)
    threads = [threading.Thread(target=worker, args=(i,)) for i in range(8)]
    [t.start() for t in threads]
    [t.join() for t in threads]
    assert not errors, errors[:2]
    print("asan-child-ok")
""")


@pytest.mark.skipif(build.asan_runtime() is None, reason="no AddressSanitizer runtime")
def test_host_paths_clean_under_address_sanitizer(tmp_path):
    library = build.built_library(address_sanitizer=True)
    script = tmp_path / "child.py"
    script.write_text(CHILD.format(root=str(ROOT), lib=str(library)))
    env = dict(os.environ, LD_PRELOAD=str(build.asan_runtime()),
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0")
    res = subprocess.run([sys.executable, str(script)], env=env, stdout=subprocess.PIPE,
                         stderr=subprocess.STDOUT, timeout=300)
    out = res.stdout.decode(errors="replace")
    assert res.returncode == 0 and "asan-child-ok" in out, out[-3000:]
    assert "AddressSanitizer" not in out, out[-3000:]
