"""The C ABI library loads on a GPU-less host and exports every entry point
include/wisp_hip.h declares (no device calls are made here)."""
import re
from pathlib import Path

from wisp_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "wisp_hip.h"


def declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(wisp_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared()
    assert len(names) >= 15
    assert "wisp_layer_forward" in names and "wisp_pager_decide" in names


def test_library_exports_every_declared_symbol(hiplib):
    missing = [n for n in declared() if not hasattr(hiplib, n)]
    assert not missing, missing


def test_binding_covers_header():
    assert set(declared()) == set(_lib.SIGNATURES)


def test_host_only_entry_points(hiplib):
    assert hiplib.wisp_abi_version() == 4
    # record: 8 header words + 8 per group + 4 per (token, k) pair
    assert hiplib.wisp_record_words(1, 8) == 8 + 8 + 4 * 8
    assert hiplib.wisp_record_words(0, 8) == 8 + 8 + 4


def test_struct_layout_mismatch_is_refused(hiplib):
    """A descriptor whose struct_bytes is not this library's sizeof (a caller
    built against another header) is refused before anything is read past
    it or allocated."""
    import ctypes as C
    from wisp_amd import _lib
    d = _lib.LayerDesc()
    h = C.c_void_p()
    for bad in (0, C.sizeof(_lib.LayerDesc) - 8):
        d.struct_bytes = bad
        assert hiplib.wisp_layer_create(C.byref(d), C.byref(h)) == _lib.WISP_ERR_INVALID
        assert b"struct_bytes" in hiplib.wisp_last_error()
    assert not h.value


def test_noalloc_array_size_is_reported(hiplib):
    """The size of the no-allocation entry point's static device array (held
    per GPU by every process that loads the library) is the header's default
    unless the build set WISP_NOALLOC_SCRATCH_MIB."""
    import os
    from wisp_amd import _lib
    mib = os.environ.get("WISP_NOALLOC_SCRATCH_MIB")
    want = int(mib) << 20 if mib else _lib.WISP_NOALLOC_SCRATCH_BYTES
    assert hiplib.wisp_noalloc_scratch_bytes() == want
