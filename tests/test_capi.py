"""The C-ABI library loads on a CPU-only host and exports every declared symbol.

No compute call is made here: only entry points whose argument checks reject
the input before any HIP call (documented in include/soupsuck_amd.h: invalid
arguments are rejected before any launch), plus pure host queries.
"""

import ctypes
import re
from pathlib import Path

import pytest

from soupsuck_amd import _lib

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    text = (ROOT / "include" / "soupsuck_amd.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ss_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIBRARY.exists():
        from soupsuck_amd import build

        build.build()
    return _lib.load()


def test_every_declared_symbol_is_exported_and_bound(lib):
    names = declared_functions()
    assert len(names) >= 20
    for name in names:
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)


def test_abi_version(lib):
    assert lib.ss_abi_version() == 1


def test_workspace_policy_is_host_only(lib):
    # Large T: the decoded fp16 W (plus any split-K partials).  Small and middle T: room
    # for the backward's decoded W^T as well as the forward's split partials.  Pure host
    # arithmetic.
    dense = 8960 * 1536 * 2
    assert lib.ss_nf4_gemm_workspace_size(16384, 8960, 1536) >= dense
    assert lib.ss_nf4_gemm_workspace_size(16, 8960, 1536) >= dense
    assert lib.ss_nf4_gemm_workspace_size(200, 8960, 1536) >= dense
    assert lib.ss_nf4_gemm_workspace_size(200, 8960, 1536) % 256 == 0
    assert lib.ss_nf4_gemm_workspace_size(16, 8960, 1536) % 256 == 0
    assert lib.ss_nf4_gemm_workspace_size(0, 8960, 1536) == 0


@pytest.mark.parametrize("name,args,needle", [
    ("ss_nf4_dequant_nested", (None, None, None, None, None, None, -1, None), "n=-1"),
    ("ss_nf4_dequant_flat", (None, None, None, 5, None), "null pointer"),
    ("ss_nf4_gemm_fwd", (None, 64, 4, None, None, None, None, None, 8, 64, None, None, 8,
                         None, 0, None), "null NF4"),
    ("ss_gemm_f16", (0, 1, 4, 4, 4, 1.0, None, 4, None, 4, None, 0.5, None, 0, 4, None),
     "beta"),
    ("ss_lora_epilogue_fwd", (None, 0, None, 1, None, 0, 4, 2.0, 0, None), "out dtype"),
    ("ss_add_rmsnorm_fwd", (None, 0, None, 0, None, 0, 1, None, 1, None, 0, None, 4, 8, 1e-6,
                            None), "promote"),
    ("ss_unpad_gather", (None, 4, None, None, 2, 3, None), "even"),
    ("ss_ce_stats", (None, 4, None, None, None, 2, 8, 8192, 0, 0, 1, -100, None), "bad sizes"),
    ("ss_ce_stats", (None, 8, None, None, None, 2, 8, 8193, 0, 0, 1, -100, None), "piece"),
    ("ss_ce_stats", (None, 8, None, None, None, 2, 8, 4, 0, 0, 1, -100, None), "partial row"),
    ("ss_ce_outputs", (None, None, 0, None, None, None, None, None, 2, -100, None),
     "bad sizes"),
    ("ss_ce_rows", (None, 4, 10, -100, None, 2, None, None, None), "bad sizes"),
    ("ss_ce_head_gain", (None, 3, None, None), "null pointer"),
    ("ss_ce_derivative", (None, 8, None, None, None, None, None, None, None, 4, 2, 8, 0, -100,
                          None), "global_rows"),
])
def test_invalid_arguments_are_rejected_before_launch(lib, name, args, needle):
    rc = getattr(lib, name)(*args)
    assert rc == _lib.ERR_INVALID_ARGUMENT
    assert needle in lib.ss_last_error().decode()


def test_unsupported_shape_is_reported(lib):
    buf = ctypes.create_string_buffer(64)
    addr = ctypes.addressof(buf)
    aligned = (addr + 15) // 16 * 16
    rc = lib.ss_nf4_gemm_fwd(aligned, 100, 4, aligned, aligned, aligned, aligned, aligned, 8,
                             100, None, aligned, 8, None, 0, None)
    assert rc == _lib.ERR_UNSUPPORTED
    assert "K % 64" in lib.ss_last_error().decode()


def test_python_call_raises_value_error(lib):
    with pytest.raises(ValueError, match="n=-1"):
        _lib.call("ss_nf4_dequant_nested", None, None, None, None, None, None, -1, None)
