"""CPU checks of the C ABI library: it loads, exports every declared symbol,
and its host-only entry points behave (no device calls here)."""
import ctypes as C

import numpy as np
import pytest


def test_exports_every_declared_symbol(awa):
    names = awa.header_symbols()
    assert "awa_forward" in names and "awa_geom_build" in names and len(names) >= 12
    lib = C.CDLL(awa.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_plan_windows_rejects_bad_sizes(awa):
    with pytest.raises(awa.AwaError):
        awa.plan_windows(0, 4, 4, (1, 1, 1), 0)
    with pytest.raises(awa.AwaError):
        awa.plan_windows(1, 4, 4, (1, 0, 1), 1)


def test_plan_windows_reference_counts(awa):
    for grid, nw, n0, n1 in [((1, 68, 80), (4, 3, 3), 16, 25), ((1, 23, 27), (4, 3, 3), 4, 4),
                             ((1, 71, 97), (1, 4, 4), 36, 36), ((1, 71, 97), (4, 4, 4), 36, 36)]:
        assert awa.plan_windows(*grid, nw, 0).shape[0] == n0
        assert awa.plan_windows(*grid, nw, 1).shape[0] == n1


def test_binding_fails_loudly_without_library(awa, monkeypatch, tmp_path):
    monkeypatch.setattr(awa, "_lib", None)
    monkeypatch.setattr(awa, "LIB_PATH", str(tmp_path / "missing.so"))
    with pytest.raises(ImportError):
        awa.lib()
