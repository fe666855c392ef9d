"""Small read-only index and pointer tables on the device, cached by content.

The kernels take their per-call metadata (leaf pointers, tile tables, segment
tables, per-problem leaf ids) as device arrays.  A table is built once per
distinct content and kept in a bounded LRU together with the pinned host buffer
it was copied from: repeated calls with the same operands issue no host to
device copy, and a HIP graph that recorded the copy can replay it (its source
buffer stays alive and unchanged).  A table first needed while a graph is being
captured is written by a kernel that carries its words as arguments
(``dpc_write_words``).  Entries are never written after creation.  A graph
owner collects the tables its capture used with :func:`keep_alive`.
"""

from __future__ import annotations

import contextlib
import threading
from collections import OrderedDict

import numpy as np
import torch

_MAX_ENTRIES = 1024
_cache: OrderedDict = OrderedDict()
_lock = threading.Lock()
_recording = threading.local()


@contextlib.contextmanager
def keep_alive():
    """Collects every table (and its host source) handed out on this thread
    inside the block into the yielded list.  A HIP graph captured inside the
    block reads those tables on every replay: its owner keeps the list for the
    graph's lifetime, so an entry evicted from the cache later is not freed
    while the graph can still read it."""
    kept: list = []
    stack = getattr(_recording, "stack", None)
    if stack is None:
        stack = _recording.stack = []
    stack.append(kept)
    try:
        yield kept
    finally:
        stack.pop()


def _record(*objs) -> None:
    for kept in getattr(_recording, "stack", ()):
        kept.extend(objs)


def device_table(values, np_dtype, device) -> torch.Tensor:
    """The device copy of ``values`` (1-D, ``np_dtype``); cached by content."""
    arr = np.ascontiguousarray(np.asarray(values, dtype=np_dtype).reshape(-1))
    dev = torch.device(device)
    key = (str(dev), arr.dtype.str, arr.tobytes())
    with _lock:
        hit = _cache.get(key)
        if hit is not None:
            _cache.move_to_end(key)
            _record(*hit)
            return hit[1]
    if dev.type == "cuda" and torch.cuda.is_current_stream_capturing():
        # Under graph capture: the words travel as kernel arguments (no host
        # buffer to keep alive; every replay rewrites the table); the table is
        # not cached.
        table = _write_table(arr, dev)
        _record(table)
        return table
    host = torch.from_numpy(arr.copy())
    if dev.type == "cuda":
        host = host.pin_memory()
        table = host.to(dev, non_blocking=True)
    else:
        table = host
    with _lock:
        _cache[key] = (host, table)
        while len(_cache) > _MAX_ENTRIES:
            _cache.popitem(last=False)
    _record(host, table)
    return table


def _write_table(arr: np.ndarray, dev: torch.device) -> torch.Tensor:
    import ctypes

    from opake_amd import _native as nat

    words = np.frombuffer(arr.tobytes(), dtype=np.uint32)
    table = torch.empty(arr.shape, dtype=torch.from_numpy(arr[:0].copy()).dtype, device=dev)
    buf = (ctypes.c_uint32 * max(len(words), 1))(*words.tolist())
    nat.call("dpc_write_words", nat.ptr(table), buf, len(words), nat.stream_handle(dev))
    return table


def pointer_table(tensors, device) -> torch.Tensor:
    """int64 device table of the tensors' data pointers (cached by content)."""
    return device_table([t.data_ptr() for t in tensors], np.int64, device)


__all__ = ["device_table", "keep_alive", "pointer_table"]
