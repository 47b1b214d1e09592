"""CPU-side checks of the C ABI: the library loads and exports every entry point
that include/mtpx.h declares (no compute call is made without a GPU)."""
import ctypes as C
import os

import pytest

from mtpx import _lib


def test_header_symbols_exported():
    L = C.CDLL(_lib.LIB_PATH)
    syms = _lib.header_symbols()
    assert len(syms) >= 25
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing


def test_binding_covers_header():
    assert set(_lib.header_symbols()) == set(_lib._SIGS)


def test_version_and_error_string():
    L = _lib.lib()
    assert L.mtpx_version().decode().startswith("mtpx")
    assert isinstance(L.mtpx_last_error(), bytes)


def test_struct_sizes_match_header_layout():
    # offsets of the pointer block after five ints (padded to 8)
    assert C.sizeof(_lib.MoEWeights) == 24 + 20 * 8
    assert _lib.LayerWeights.moe.offset == 12 * 8
