"""The C-ABI library loads and exports exactly the entry points include/vsplat.h declares."""
import re
from pathlib import Path

import vauss_amd
from vauss_amd import _lib

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "vsplat.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(vs_[a-z0-9_]+)\s*\(", text))


def test_header_declares_the_binding_surface():
    assert declared_symbols() == set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = vauss_amd.load()
    for name in declared_symbols():
        assert hasattr(lib, name), name


def test_version_and_error_strings():
    lib = vauss_amd.load()
    assert lib.vs_version().decode().startswith("vsplat-gfx950")
    assert isinstance(lib.vs_last_error(), bytes)
