"""The C-ABI library loads and exports every function include/*.h declares; argument
validation runs on the host (no GPU needed) and reports through flour_hip_last_error."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from flour_amd import _lib

ROOT = Path(__file__).resolve().parent.parent


def declared_functions() -> list[str]:
    names = []
    for h in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names += re.findall(r"\b(flour_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_the_boundary():
    names = declared_functions()
    for want in ("flour_hip_kv_write", "flour_hip_paged_decode", "flour_hip_varlen_prefill",
                 "flour_hip_paged_decode_workspace_size", "flour_hip_last_error"):
        assert want in names


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert missing == []
    assert b"gfx950" in lib.flour_hip_version()


def test_host_validation_errors_without_gpu():
    lib = _lib.lib()
    rc = lib.flour_hip_kv_write(None, None, 0, 0, None, None, None, 4, 2, 8, 16, 9, None)
    assert rc == _lib.ERR_INVALID_ARGUMENT
    assert "dtype" in _lib.last_error()
    rc = lib.flour_hip_paged_decode(None, 1, None, None, None, None, 4, None, 2, 6, 4, 128, 16,
                                    64, 32, 1.0, 1, None, 0, None)
    assert rc == _lib.ERR_INVALID_ARGUMENT  # 6 heads not a multiple of 4 kv heads
    n = ctypes.c_size_t(0)
    assert lib.flour_hip_paged_decode_workspace_size(64, 32, 8, 128, 4096, ctypes.byref(n)) == 0
    assert n.value > 0
    rc = lib.flour_hip_varlen_prefill(None, 1, 0, 0, None, 0, 0, None, None, None, None, None, 4,
                                      2, 8, 16, 32, 8, 128, 0, 64, 1.0, 1, None)
    assert rc == _lib.ERR_INVALID_ARGUMENT  # block_size 0
    # zero-size work is a no-op that touches nothing
    assert lib.flour_hip_kv_write(None, None, 0, 0, None, None, None, 0, 2, 8, 16, 1, None) == 0
    with pytest.raises(_lib.FlourError):
        _lib.check(-1)
