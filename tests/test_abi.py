"""The C ABI: libneedle_hip.so loads, exports every entry point that
include/needle_hip.h declares, and maps failures to NeedleError codes.
Runs without a GPU (no compute calls)."""

import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

from needle_hip import HipBackend, NeedleError
from needle_hip import lib as L

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "needle_hip.h"


def declared():
    text = HEADER.read_text()
    return re.findall(r"^(?:nd_status|const char\*|void\*|nd_kv\*|uint32_t)\s+(nd_\w+)\(", text, re.M)


def test_header_declarations_are_bound_and_exported():
    names = declared()
    assert len(names) >= 20
    assert set(names) == set(L.SIGNATURES), set(names) ^ set(L.SIGNATURES)
    lib = L.load_library()
    for name in names:
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(L.library_path())],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (nd_\w+)$", out, re.M))
    assert set(names) <= exported


def test_library_carries_gfx950_code_objects():
    data = L.library_path().read_bytes()
    assert b"amdgcn-amd-amdhsa--gfx950" in data
    for other in (b"--gfx942", b"--gfx90a", b"--gfx1100"):
        assert other not in data


def test_null_context_errors_do_not_touch_the_device():
    lib = L.load_library()
    assert lib.nd_sync(None) == L.ND_ERR_BACKEND
    assert lib.nd_matvec(None, None, None, 1, 0, 1, None) == L.ND_ERR_BACKEND
    assert lib.nd_destroy(None) == L.ND_OK
    assert lib.nd_create(0, None) == L.ND_ERR_INVALID
    assert b"NULL" in lib.nd_last_error(None)


def test_status_mapping():
    lib = L.load_library()
    with pytest.raises(NeedleError) as e:
        L.check(lib, None, L.ND_ERR_OVERFLOW)
    assert e.value.code == "CONTEXT_OVERFLOW"
    with pytest.raises(NeedleError) as e:
        L.check(lib, None, L.ND_ERR_INVALID)
    assert e.value.code == "INVALID_CACT"
    L.check(lib, None, L.ND_OK)


def test_backend_unavailable_without_device():
    lib = L.load_library()
    ctx = C.c_void_p()
    if lib.nd_create(0, C.byref(ctx)) == L.ND_OK:
        lib.nd_destroy(ctx)
        pytest.skip("a device is present")
    with pytest.raises(NeedleError) as e:
        HipBackend()
    assert e.value.code == "BACKEND_UNAVAILABLE"


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(L, "_LIB", None)
    monkeypatch.setenv("NEEDLE_HIP_LIB", str(tmp_path / "absent.so"))
    with pytest.raises(NeedleError) as e:
        L.load_library()
    assert e.value.code == "BACKEND_UNAVAILABLE"
