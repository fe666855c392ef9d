"""The C-ABI library loads and exports every entry point the header declares."""

from __future__ import annotations

import re
from pathlib import Path

import pytest

from opake_amd import _native

HEADER = Path(__file__).resolve().parents[1] / "include" / "opake_amd.h"


def declared_functions() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(dpc_[a-z0-9_]+)\s*\(", text))


def test_header_declares_the_bound_functions():
    assert declared_functions() == set(_native.SIGNATURES)


def test_library_exports_every_declared_symbol():
    if not _native.LIB_PATH.exists():
        pytest.skip("native library not built")
    lib = _native.load()
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_version_and_size_queries():
    if not _native.LIB_PATH.exists():
        pytest.skip("native library not built")
    lib = _native.load()
    assert lib.dpc_version() == _native.ABI_VERSION == 200
    assert lib.dpc_clip_plan_bytes(32) == 16 + 32 * 4
    assert lib.dpc_gram_workspace_bytes(0, 5) == 0
    assert lib.dpc_gram_workspace_bytes(2, 128) > 0
