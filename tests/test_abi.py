"""CPU checks of the boundary: the C-ABI library loads and exports every
function include/indecis_hip.h declares (no GPU call is made)."""
import os
import re

import pytest

from indecis_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    text = open(os.path.join(ROOT, "include", "indecis_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ixh_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_bound_functions():
    assert declared() == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_symbol():
    if not os.path.exists(_lib.SO_PATH):
        pytest.fail(f"{_lib.SO_PATH} not built: run __graft_entry__.build()")
    L = _lib.lib()
    for name in declared():
        assert hasattr(L, name), name


def test_last_error_is_callable_without_gpu():
    assert isinstance(_lib.lib().ixh_last_error(), bytes)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "SO_PATH", str(tmp_path / "absent.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        _lib.lib()
