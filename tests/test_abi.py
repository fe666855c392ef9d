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
    assert lib.dpc_version() == _native.ABI_VERSION == 207
    assert lib.dpc_clip_plan_bytes(32) == 16 + 32 * 4
    # Grouped Gram workspace: the records, then the split kernel's tickets and
    # accumulator exchange (2 x 224 KiB per set), each 256-byte aligned.
    assert lib.dpc_grouped_gram_workspace_bytes(10, 0) == 1024
    assert lib.dpc_grouped_gram_workspace_bytes(10, 3) == 1024 + 256 + 3 * 2 * 229376
    assert lib.dpc_gram_workspace_bytes(0, 5) == 0
    assert lib.dpc_gram_workspace_bytes(2, 128) > 0


def test_tables_used_under_keep_alive_survive_eviction():
    # A graph owner holds the tables its capture used: filling the content
    # cache past its bound afterwards evicts the cache's entries but not the
    # owner's references (CPU tables: the cache logic is device-independent).
    import gc
    import weakref

    from opake_amd import _tables

    with _tables.keep_alive() as kept:
        t1 = _tables.device_table([1, 2, 3], "int32", "cpu")
        t2 = _tables.device_table([1, 2, 3], "int32", "cpu")  # a cache hit
    assert t1 is t2 and any(x is t1 for x in kept)
    ref = weakref.ref(t1)
    del t1, t2
    for i in range(_tables._MAX_ENTRIES + 10):
        _tables.device_table([i, i + 1, 7777], "int32", "cpu")
    gc.collect()
    assert ref() is not None  # evicted from the cache, alive through `kept`
    del kept
    gc.collect()
    assert ref() is None


def test_err_less_accumulation_must_be_explicit():
    # Accumulating norms into `out` without `err` drops the bound of the sum;
    # the norm helpers refuse it unless return_error=False says so.
    from opake_amd import ops
    from opake_amd.exceptions import ConfigurationError

    out, err = object(), object()
    assert ops._wants_error(None, None, None) is False
    assert ops._wants_error(None, None, True) is True
    assert ops._wants_error(out, err, None) is True
    assert ops._wants_error(out, None, False) is False
    with pytest.raises(ConfigurationError, match="drops the rounding-error bound"):
        ops._wants_error(out, None, None)
    with pytest.raises(ConfigurationError, match="return_error=False"):
        ops._wants_error(out, err, False)


def _kernarg_setting(env_value):
    """HIP_FORCE_DEV_KERNARG as seen after `import opake_amd` in a fresh
    interpreter whose environment holds `env_value` (None: unset)."""
    import os
    import subprocess
    import sys

    env = {k: v for k, v in os.environ.items() if k != "HIP_FORCE_DEV_KERNARG"}
    if env_value is not None:
        env["HIP_FORCE_DEV_KERNARG"] = env_value
    code = "import os, opake_amd; print(os.environ.get('HIP_FORCE_DEV_KERNARG'))"
    out = subprocess.run([sys.executable, "-c", code], env=env, check=True, text=True,
                         capture_output=True, cwd=Path(__file__).resolve().parents[1])
    return out.stdout.strip()


def test_import_asks_for_device_kernel_arguments_unless_set():
    assert _kernarg_setting(None) == "1"
    assert _kernarg_setting("0") == "0"
