"""The C-ABI libraries load and export every symbol the headers declare
(no compute calls: this runs without a GPU)."""
import ctypes
import os
import re

from foundry_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared(header: str, prefix: str) -> set[str]:
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(" + prefix + r"[a-z0-9_]+)\s*\(", text))


def test_restore_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.RESTORE_LIB)
    declared = _declared("foundry_restore.h", "fdy_")
    assert len(declared) >= 25
    missing = [s for s in sorted(declared) if not hasattr(lib, s)]
    assert not missing, missing
    # ...and the Python bindings cover them all.
    assert declared == set(_lib.exported_symbols())


def test_synth_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.SYNTH_LIB)
    declared = _declared("fdy_synth.h", "fdy_synth_")
    missing = [s for s in sorted(declared) if not hasattr(lib, s)]
    assert not missing, missing


def test_version_string_without_gpu():
    assert b"gfx950" in _lib.restore_lib().fdy_version()


def test_library_raises_when_missing(tmp_path, monkeypatch):
    monkeypatch.setattr(_lib, "_restore", None)
    monkeypatch.setattr(_lib, "RESTORE_LIB", str(tmp_path / "absent.so"))
    try:
        _lib.restore_lib()
    except _lib.FoundryError as e:
        assert "not built" in str(e)
    else:
        raise AssertionError("missing library did not raise")
