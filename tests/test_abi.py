"""The C-ABI library loads and exports every symbol include/sa_hip.h declares.

CPU-only: no compute call is made (there is no GPU here); the Python binding's
signature table must cover exactly the header's entry points.
"""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sa_hip.h")


def _declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(sa_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = _declared_symbols()
    assert "sa_ssu_fwd" in syms and "sa_last_error" in syms


def test_library_exports_declared_symbols():
    from selective_attention import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} missing: run python selective-attention_amd/build.py")
    lib = _lib.load()
    for name in _declared_symbols():
        assert hasattr(lib, name), f"libsa_hip.so does not export {name}"
    assert lib.sa_version() >= 1


def test_binding_table_matches_header():
    from selective_attention import _lib
    assert sorted(_lib.SIGNATURES) == _declared_symbols()


def test_missing_library_fails_loudly(tmp_path):
    from selective_attention import _lib
    with pytest.raises(_lib.LibraryNotBuilt):
        _lib.load(str(tmp_path / "nope.so"))
