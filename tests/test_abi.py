"""The C ABI library loads without a GPU and exports every symbol its header declares."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "texelator_hip.h"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(tx_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_boundary():
    names = declared_symbols()
    for required in ("tx_pack_encoded", "tx_linear", "tx_set_lookahead", "tx_set_prefill",
                     "tx_set_prefill_backend", "tx_handle_info", "tx_free", "tx_palette_probe",
                     "tx_kernel_info", "tx_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from texelator_amd import _lib

    if not _lib.LIBRARY_PATH.exists():
        pytest.fail("libtexelator_hip.so is not built; run python -m texelator_amd.build")
    lib = ctypes.CDLL(str(_lib.LIBRARY_PATH))
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert set(declared_symbols()) == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"


def test_errors_without_gpu_are_reported_not_crashing():
    from texelator_amd import _lib

    lib = _lib.load()
    assert lib.tx_set_lookahead(0, 2) == _lib.TX_ERR_INVALID
    assert b"null" in lib.tx_last_error()
    assert lib.tx_free(0) == _lib.TX_ERR_INVALID
    assert lib.tx_candidate_name(5) == b"large_256x128x128"
    assert lib.tx_candidate_name(4) is None


def test_kernel_info_wrapper_reads_nine_fields(monkeypatch):
    """``_hip.kernel_info`` asks the library for the reference's nine fields
    (``cutlass_texture_mainloop.cu:251-267``: ..., tile M/N/K, active blocks)."""
    from texelator_amd import _hip, _lib

    requested = []

    class FakeLibrary:
        def tx_kernel_info(self, candidate, out, n):
            requested.append((candidate, n))
            for i in range(n):
                out[i] = 10 * candidate + i
            return _lib.TX_OK

    monkeypatch.setattr(_lib, "load", lambda: FakeLibrary())
    assert _hip.kernel_info(7) == [70 + i for i in range(9)]
    assert _hip.cutlass_smalln_kernel_info() == [90 + i for i in range(9)]
    assert requested == [(7, 9), (9, 9)]


def test_candidate_names_are_the_tile_table():
    from texelator_amd import _lib, autotune

    lib = _lib.load()
    names = [lib.tx_candidate_name(c).decode() for c in range(5, 10)]
    assert names == list(autotune.CANDIDATES)
    assert [autotune.CANDIDATES[n] for n in names] == list(range(5, 10))
