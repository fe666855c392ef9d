"""ctypes binding of ``libopake_amd.so`` (the C ABI in ``include/opake_amd.h``).

The library is loaded from this package directory.  There is no fallback:
if it is missing, or the tensors are not on a ROCm device, calls raise
:class:`~opake_amd.exceptions.OperationError` / ``ConfigurationError``.
Status codes map to the reference's error classes: ``DPC_EINVAL`` ->
``ConfigurationError`` (a ``ValueError``), anything else -> ``OperationError``.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

from opake_amd.exceptions import ConfigurationError, OperationError

LIB_PATH = Path(__file__).resolve().parent / "libopake_amd.so"

DPC_OK = 0
DPC_EINVAL = -22
DPC_ENOTSUP = -95
DPC_ENOSPC = -28
DPC_EHIP = -1000

DPC_F32 = 0
DPC_BF16 = 1
DPC_F16 = 2
DPC_F64 = 3
SCALE_FIXED = 0
SCALE_AUTO_S = 1
NOISE_NONE = 0
NOISE_INJECTED = 1
NOISE_PHILOX = 2

_c_void_p = ctypes.c_void_p
_c_int = ctypes.c_int
_c_double = ctypes.c_double
_c_float = ctypes.c_float
_c_size_t = ctypes.c_size_t
_c_u32 = ctypes.c_uint32
_c_u64 = ctypes.c_uint64
_c_i64 = ctypes.c_int64

ABI_VERSION = 207  # dpc_version() of the library these signatures describe

# name -> (restype, argtypes)
SIGNATURES = {
    "dpc_version": (_c_int, []),
    "dpc_calib_mfma_bf16": (_c_int, [_c_void_p, _c_int, _c_int, _c_void_p, _c_void_p]),
    "dpc_last_error": (ctypes.c_char_p, []),
    "dpc_write_words": (_c_int, [_c_void_p, _c_void_p, _c_int, _c_void_p]),
    "dpc_gram_workspace_bytes": (_c_size_t, [_c_int, _c_int]),
    "dpc_gram_sqnorms": (
        _c_int,
        [_c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
         _c_void_p, _c_void_p, _c_void_p, _c_size_t, _c_void_p],
    ),
    "dpc_gram_sqnorms_noalloc": (
        _c_int,
        [_c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
         _c_void_p, _c_void_p, _c_void_p],
    ),
    "dpc_flat_sqnorms": (
        _c_int,
        [_c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_void_p,
         _c_void_p, _c_void_p],
    ),
    "dpc_clip_plan_bytes": (_c_size_t, [_c_int]),
    "dpc_clip_factors_groups": (
        _c_int,
        [_c_void_p, _c_void_p, _c_int, _c_int, ctypes.POINTER(_c_double), _c_int, _c_double,
         ctypes.POINTER(_c_double), ctypes.POINTER(_c_double), ctypes.POINTER(_c_int), _c_int,
         ctypes.POINTER(_c_float), _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _c_void_p, _c_void_p],
    ),
    "dpc_clip_factors": (
        _c_int,
        [_c_void_p, _c_void_p, _c_int, _c_double, _c_int, _c_double, ctypes.POINTER(_c_double),
         ctypes.POINTER(_c_double), ctypes.POINTER(_c_int), _c_int, _c_float, _c_void_p,
         _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p],
    ),
    "dpc_clipped_sum_workspace_bytes": (_c_size_t, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "dpc_clipped_sum": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_int, _c_int,
         _c_double, _c_int, _c_void_p, _c_void_p, _c_u64, _c_u32, _c_u32, _c_double, _c_int,
         _c_void_p, _c_int, _c_void_p, _c_void_p, _c_size_t, _c_void_p],
    ),
    "dpc_timing_event_create": (_c_int, [_c_void_p]),
    "dpc_timing_event_record": (_c_int, [_c_void_p, _c_void_p]),
    "dpc_timing_event_elapsed_ms": (_c_int, [_c_void_p, _c_void_p, _c_void_p]),
    "dpc_timing_event_destroy": (_c_int, [_c_void_p]),
    "dpc_gram_sqnorms_multi_workspace_bytes": (
        _c_size_t, [_c_int, _c_void_p, _c_void_p, _c_int, _c_int, _c_int],
    ),
    "dpc_gram_clip_workspace_bytes": (_c_size_t, [_c_int, _c_int]),
    "dpc_gram_clip_counter_bytes": (_c_size_t, [_c_int, _c_int]),
    "dpc_gram_clip_factors": (
        _c_int,
        [_c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_double, _c_int,
         _c_double, ctypes.POINTER(_c_double), ctypes.POINTER(_c_double), ctypes.POINTER(_c_int),
         _c_int, _c_float, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _c_void_p, _c_void_p, _c_void_p, _c_size_t, _c_void_p, _c_size_t, _c_void_p],
    ),
    "dpc_gram_sqnorms_multi": (
        _c_int,
        [_c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_int,
         _c_void_p, _c_void_p, _c_void_p, _c_size_t, _c_void_p],
    ),
    "dpc_clipped_sum_multi": (
        _c_int,
        [_c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int,
         _c_int, _c_double, _c_int, _c_void_p, _c_u64, _c_void_p, _c_void_p, _c_int, _c_void_p,
         _c_void_p],
    ),
    "dpc_add_noise": (
        _c_int,
        [_c_void_p, _c_void_p, _c_i64, _c_i64, _c_int, _c_double, _c_int, _c_void_p, _c_u64,
         _c_u32, _c_void_p],
    ),
    "dpc_philox4x32_10": (
        _c_int,
        [_c_u32, _c_u32, _c_u32, _c_u32, _c_u32, _c_u32, _c_int, _c_void_p, _c_void_p],
    ),
    "dpc_leaves_sqnorm": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int,
         _c_int, _c_int, _c_void_p, _c_void_p, _c_int, _c_void_p],
    ),
    "dpc_leaves_apply": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_void_p,
         _c_void_p, _c_void_p, _c_void_p, _c_int, _c_void_p, _c_void_p],
    ),
    "dpc_sanitize_columns": (
        _c_int, [_c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_int, _c_void_p],
    ),
    "dpc_leaves_apply_ex": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_int,
         _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_void_p,
         _c_void_p],
    ),
    "dpc_add_noise_ex": (
        _c_int,
        [_c_void_p, _c_void_p, _c_i64, _c_i64, _c_int, _c_int, _c_double, _c_int, _c_void_p,
         _c_u64, _c_u32, _c_void_p],
    ),
    "dpc_group_sum_f64": (
        _c_int,
        [_c_void_p, _c_int, _c_int, _c_int, _c_int, _c_void_p, _c_int, _c_void_p, _c_int,
         _c_void_p],
    ),
    "dpc_row_sum_f64": (_c_int, [_c_void_p, _c_int, _c_int, _c_int, _c_void_p, _c_void_p]),
    "dpc_per_example_grads_workspace_bytes": (_c_size_t, [_c_int, _c_int, _c_int, _c_int]),
    "dpc_per_example_grads": (
        _c_int,
        [_c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_void_p, _c_int,
         _c_void_p, _c_size_t, _c_void_p],
    ),
    "dpc_per_example_grads_grouped_workspace_bytes": (
        _c_size_t, [_c_int, _c_void_p, _c_void_p, _c_int, _c_int, _c_int]),
    "dpc_per_example_grads_grouped": (
        _c_int,
        [_c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int,
         _c_int, _c_void_p, _c_size_t, _c_void_p],
    ),
    "dpc_add_noise_leaves": (
        _c_int,
        [_c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_u64,
         _c_void_p],
    ),
    "dpc_grouped_gram_workspace_bytes": (_c_size_t, [_c_int, _c_int]),
    "dpc_grouped_gram_sqnorms": (
        _c_int,
        [_c_void_p, _c_void_p, ctypes.POINTER(_c_int), _c_int, _c_int, _c_void_p, _c_int, _c_int,
         _c_void_p, _c_int, _c_int, _c_int, _c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p,
         _c_size_t, _c_void_p],
    ),
    "dpc_segment_plan": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_void_p,
         _c_void_p, _c_void_p],
    ),
    "dpc_grouped_clipped_sum": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_void_p,
         _c_void_p, _c_void_p, _c_double, _c_int, _c_void_p, _c_u64, _c_void_p, _c_void_p, _c_int,
         _c_void_p, _c_void_p],
    ),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load (once) and return the native library; raise if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise OperationError(
                f"native library {LIB_PATH} is missing; build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` (needs hipcc)"
            )
        try:
            lib = ctypes.CDLL(str(LIB_PATH))
        except OSError as exc:
            raise OperationError(f"cannot load {LIB_PATH}: {exc}") from exc
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.dpc_version()
        if version != ABI_VERSION:
            raise OperationError(
                f"{LIB_PATH} has ABI version {version}, these bindings need {ABI_VERSION}; "
                "rebuild it")
        _lib = lib
        return lib


def call(name: str, *args) -> None:
    """Call a status-returning entry point and raise on failure."""
    lib = load()
    status = getattr(lib, name)(*args)
    if status == DPC_OK:
        return
    if status == DPC_EINVAL:
        raise ConfigurationError(f"{name}: invalid argument (DPC_EINVAL)")
    if status == DPC_ENOSPC:
        raise OperationError(f"{name}: workspace too small (DPC_ENOSPC)")
    if status == DPC_ENOTSUP:
        raise OperationError(f"{name}: unsupported configuration (DPC_ENOTSUP)")
    detail = lib.dpc_last_error().decode(errors="replace")
    raise OperationError(f"{name}: HIP error ({status}): {detail}")


def ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def stream_handle(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


class TimingEvent:
    """A timing event recorded without the system-scope fence
    (``dpc_timing_event_*``), with the ``record`` / ``elapsed_time`` methods
    of ``torch.cuda.Event`` that the timing hooks use: recording one adds no
    cache writeback or invalidation around the launch it brackets."""

    def __init__(self):
        self._h = ctypes.c_void_p()
        call("dpc_timing_event_create", ctypes.addressof(self._h))

    def record(self) -> None:
        call("dpc_timing_event_record", self._h,
             stream_handle(torch.device("cuda", torch.cuda.current_device())))

    def elapsed_time(self, end: "TimingEvent") -> float:
        ms = ctypes.c_float()
        call("dpc_timing_event_elapsed_ms", self._h, end._h, ctypes.addressof(ms))
        return ms.value

    def __del__(self):
        try:
            if self._h:
                load().dpc_timing_event_destroy(self._h)
        except Exception:  # interpreter shutdown
            pass


_CODES = {torch.float32: DPC_F32, torch.bfloat16: DPC_BF16, torch.float16: DPC_F16,
          torch.float64: DPC_F64}


def dtype_code(dtype: torch.dtype, *, wide: bool = False) -> int:
    """The library's code of ``dtype``: float32 or bfloat16 for the linear-layer
    kernels; with ``wide`` (the materialised-leaf, clip-guard and noise entry
    points) also float16 and float64."""
    code = _CODES.get(dtype)
    if code is None or (not wide and code not in (DPC_F32, DPC_BF16)):
        supported = "float16, bfloat16, float32, float64" if wide else "float32, bfloat16"
        raise ConfigurationError(f"unsupported dtype {dtype} (supported: {supported})")
    return code


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors on one ROCm device; returns it."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ConfigurationError(
                f"opake_amd kernels need tensors on a ROCm device, got {t.device}"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ConfigurationError("tensors span more than one device")
    if dev is None:
        raise ConfigurationError("no tensor argument to infer the device from")
    if torch.version.hip is None:
        raise OperationError("opake_amd requires a ROCm build of PyTorch")
    return dev


__all__ = ["LIB_PATH", "SIGNATURES", "call", "load", "ptr", "stream_handle"]
