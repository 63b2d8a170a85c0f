"""CPU checks of the drop-in boundary: libva_hip.so loads and exports every entry point that
include/va_hip.h declares, the Python binding types all of them, and argument validation
that needs no device rejects bad input.  No kernel is launched here."""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "va_hip.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b(va_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib():
    from vectoraccelerate_amd import _lib
    from vectoraccelerate_amd import build as b

    if not _lib.LIB_PATH.exists():
        b.build()
    return _lib.load()


def test_header_declares_the_search_path():
    names = declared_functions()
    for required in ["va_context_create", "va_fused_topk", "va_topk_select", "va_sq_quantize_i8", "va_i8_scan_topk",
                     "va_bq_pack", "va_hamming_topk", "va_ivf_build", "va_ivf_search"]:
        assert required in names


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"libva_hip.so lacks {missing}"


def test_binding_types_every_declared_symbol():
    from vectoraccelerate_amd import _lib

    assert sorted(_lib.SIGNATURES) == declared_functions()


def test_abi_version_and_status_strings(lib):
    assert lib.va_abi_version() == 5
    assert lib.va_status_string(0) == b"ok"
    assert lib.va_status_string(1) == b"invalid argument"


def test_null_context_is_rejected_without_a_device(lib):
    assert lib.va_context_synchronize(None) == 1
    assert lib.va_fused_topk(None, 0, None, None, 1, 1, 1, 1, None, None) == 1
    assert lib.va_context_destroy(None) == 1
    out = C.c_void_p()
    assert lib.va_context_create(0, None) == 1
    del out
