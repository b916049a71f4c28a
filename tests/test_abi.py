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
    assert hiplib.wisp_abi_version() == 2
    # record: 8 header words + 8 per group + 4 per (token, k) pair
    assert hiplib.wisp_record_words(1, 8) == 8 + 8 + 4 * 8
    assert hiplib.wisp_record_words(0, 8) == 8 + 8 + 4
