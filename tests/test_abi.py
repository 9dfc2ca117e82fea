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


def test_graph_half_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.RESTORE_LIB)
    declared = _declared("foundry_graph.h", "fdy_")
    assert len(declared) >= 10
    missing = [s for s in sorted(declared) if not hasattr(lib, s)]
    assert not missing, missing
    assert declared == set(_lib.graph_symbols())


def test_region_half_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.RESTORE_LIB)
    declared = _declared("foundry_region.h", "fdy_")
    assert len(declared) >= 15
    missing = [s for s in sorted(declared) if not hasattr(lib, s)]
    assert not missing, missing
    assert declared == set(_lib.region_symbols())


def test_code_object_hash_is_crc64_xz_without_gpu():
    """fdy_code_object_hash is CRC-64/XZ (the identity of csrc/hook.cpp:315-321):
    the standard check value, and agreement with the bit-serial reference."""
    from refcrc import crc64_xz

    lib = _lib.restore_lib()
    check = b"123456789"
    assert lib.fdy_code_object_hash(check, len(check)) == 0x995DC9BBDF1939FA
    blob = bytes((i * 131 + 7) & 0xFF for i in range(1237))
    for n in (0, 1, 7, 8, 9, 63, 64, 1237):
        assert lib.fdy_code_object_hash(blob[:n], n) == crc64_xz(blob[:n])


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
