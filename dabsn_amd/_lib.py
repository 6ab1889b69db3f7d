"""ctypes binding of the C ABI in ``include/dabsn_hip.h``.

The library is ``dabsn_amd/_build/libdabsn_hip.so`` (built by ``dabsn_amd.build``). It is
loaded lazily on first use; a missing library is a hard error on any GPU call, never a
silent fallback.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_build" / "libdabsn_hip.so"
ABI_VERSION = 18

_lock = threading.Lock()
_lib = None
_load_error: str | None = None

vp = ctypes.c_void_p
i64 = ctypes.c_int64
i32 = ctypes.c_int
sz = ctypes.c_size_t


class CoreParams(ctypes.Structure):
    """Mirror of ``dabsn_core_params``."""

    _fields_ = [("vec", vp * 16), ("scal", vp * 3)]


PTR4 = vp * 4
PTR8 = vp * 8


class CoreFwdCall(ctypes.Structure):
    """Mirror of ``dabsn_core_fwd_call``."""

    _fields_ = ([("dtype", i32), ("B", i64), ("T", i64), ("H", i64), ("ldt", i64), ("ldx", i64),
                 ("Wx", vp), ("Wgx", vp), ("GA", vp), ("params", ctypes.POINTER(CoreParams))]
                + [(n, vp) for n in ("b0", "e0", "c0", "U", "nov", "plast", "expr", "write",
                                     "energy", "sat", "gate", "bF", "eF", "cF", "workspace")]
                + [("workspace_bytes", sz), ("state_dtype", i32), ("coresident_cus", i32)])


class CoreBwdCall(ctypes.Structure):
    """Mirror of ``dabsn_core_bwd_call``."""

    _fields_ = ([("dtype", i32), ("B", i64), ("T", i64), ("H", i64), ("ldt", i64), ("GAT", vp),
                 ("params", ctypes.POINTER(CoreParams))]
                + [(n, vp) for n in ("b0", "c0", "U", "plast", "expr", "energy", "sat", "gate",
                                     "gU", "gNov", "gP", "gAy", "gW", "gE", "gC", "gbF", "geF",
                                     "gcF", "gWx", "gWgx", "day", "part_vec", "part_scal", "gb0",
                                     "ge0", "gc0", "workspace")]
                + [("workspace_bytes", sz), ("coresident_cus", i32)])

_SIGNATURES = {
    "dabsn_hip_abi_version": ([], i32),
    "dabsn_hip_last_error": ([], ctypes.c_char_p),
    "dabsn_hip_zero": ([vp, sz, vp], i32),
    "dabsn_hip_core_scan_workspace_bytes": ([i32, i64, i64, i32], sz),
    "dabsn_hip_core_scan_layout": ([i32, i64, i64, ctypes.POINTER(i64), ctypes.POINTER(i64)], i32),
    "dabsn_hip_core_scan_config": (
        [i32, i64, i64, ctypes.POINTER(i32), ctypes.POINTER(i32), ctypes.POINTER(i32)], i32),
    "dabsn_hip_core_scan_fwd": (
        [i32, i64, i64, i64, vp, vp, vp, ctypes.POINTER(CoreParams), vp, vp, vp]
        + [vp] * 8 + [vp, vp, vp, vp, sz, vp],
        i32,
    ),
    "dabsn_hip_core_scan_bwd": (
        [i32, i64, i64, i64, vp, ctypes.POINTER(CoreParams), vp, vp]
        + [vp] * 6 + [vp] * 7 + [vp] * 3 + [vp] * 3 + [vp, vp] + [vp] * 3 + [vp, sz, vp],
        i32,
    ),
    "dabsn_hip_stream_pair": (
        [ctypes.POINTER(vp), ctypes.POINTER(vp), ctypes.POINTER(i32), ctypes.POINTER(i32)], i32),
    "dabsn_hip_stream_destroy": ([vp], i32),
    "dabsn_hip_tape_stats_window": (
        [i32, i64, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, i64, vp], i32),
    "dabsn_hip_tape_stats_bwd_window": (
        [i32, i64, i64, i64, i64, vp, i64, i32, vp, vp, vp, vp, vp], i32),
    "dabsn_hip_core_scan_fwd_call": ([ctypes.POINTER(CoreFwdCall), vp], i32),
    "dabsn_hip_core_scan_bwd_call": ([ctypes.POINTER(CoreBwdCall), vp], i32),
    "dabsn_hip_linrec_fwd": ([i32, i64, i64, i64, vp, vp, vp, vp, vp], i32),
    "dabsn_hip_linrec_workspace_bytes": ([i32, i64, i64, i64], sz),
    "dabsn_hip_linrec_bwd": ([i32, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp], i32),
    "dabsn_hip_long_workspace_bytes": ([i64, i64, i64, i32], sz),
    "dabsn_hip_long_fwd": (
        [i32, i64, i64, i64, i64, vp, vp, PTR4, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp], i32),
    "dabsn_hip_long_partials": ([i64, i64, i64], i64),
    "dabsn_hip_long_bwd": (
        [i32, i64, i64, i64, i64, vp, vp, PTR4, vp, vp, vp, vp, vp, vp, vp, i64, i32, vp, vp, vp,
         vp, vp, sz, vp],
        i32,
    ),
    "dabsn_hip_tape_stats": ([i32, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, vp], i32),
    "dabsn_hip_tape_stats_bwd": ([i32, i64, i64, i64, vp, i32, vp, vp, vp, vp, vp], i32),
    "dabsn_hip_read_output": ([i32, i32, i32, i32, i64, vp, vp, vp, vp, vp], i32),
    "dabsn_hip_read_output_partials": ([i64], sz),
    "dabsn_hip_read_output_bwd": (
        [i32, i32, i32, i32, i64, vp, vp, vp, vp, vp, vp, vp, sz, vp], i32),
    "dabsn_hip_read_output_window": (
        [i32, i32, i32, i32, i64, i64, i64, i64, i64, vp, vp, vp, vp, vp], i32),
    "dabsn_hip_read_output_bwd_window": (
        [i32, i32, i32, i32, i64, i64, i64, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, sz, vp],
        i32),
    "dabsn_hip_read_mix": ([i32, i64, vp, vp, vp, vp, vp, vp, vp], i32),
    "dabsn_hip_rms_norm": ([i32, i64, i64, vp, vp, ctypes.c_float, vp, vp], i32),
    "dabsn_hip_relu_square": ([i32, i64, vp, vp, vp], i32),
    "dabsn_hip_normalize_rows": ([i32, i64, i64, vp, vp, vp, vp], i32),
    "dabsn_hip_normalize_rows_bwd": ([i32, i64, i64, vp, vp, vp, vp, vp], i32),
    "dabsn_hip_bank_select": ([i32, i32, i64, i64, vp, vp, vp, vp, vp, vp], i32),
    "dabsn_hip_admit_step": (
        [i32, i64, i64, i64, i64, vp, i64, PTR8, vp, i32, vp, vp, vp, vp, vp, vp, vp], i32),
    "dabsn_hip_bank_fold": ([i64, i64, i64, vp, vp, vp, vp, vp], i32),
    "dabsn_hip_bank_width": ([i64, i64, vp, vp, i32, vp, vp], i32),
    "dabsn_hip_window_add": ([i32, i64, i64, i64, vp, i64, i64, vp, i64, i64, vp, i64, i64, vp],
                             i32),
    "dabsn_hip_bank_slots": ([i64, i64, i64, vp, vp, i64, vp, vp, vp, vp, vp, vp], i32),
    "dabsn_hip_glue_slots": ([i64, i64, i64, i64, vp, vp, i64, PTR8, i32, vp, vp, vp, vp], i32),
    "dabsn_hip_glue_slots_partials": ([i64, i64], sz),
    "dabsn_hip_glue_slots_bwd": (
        [i64, i64, i64, i64, vp, vp, i64, PTR8, i32, vp, vp, vp, vp, i64, vp, vp, vp], i32),
    "dabsn_hip_glue_rows_bwd": ([i64, i64, i64, vp, i32, vp, vp, i64, vp], i32),
    "dabsn_hip_bank_gather_bwd_prefix": (
        [i32, i64, i64, i64, i64, i64, vp, vp, vp, vp, vp, vp, i32, vp, vp], i32),
    "dabsn_hip_bank_gather": ([i32, i64, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, vp], i32),
    "dabsn_hip_bank_gather_bwd": (
        [i32, i64, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, vp, vp], i32),
    "dabsn_hip_core_scan_launches": ([i32, i64, i64, i64, i32, vp], i32),
    "dabsn_hip_read3_workspace_bytes": ([i32, i64, i64, i64, i64, i32], sz),
    "dabsn_hip_read3_fwd": (
        [i32, i64, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, PTR4, vp, vp,
         sz, vp],
        i32,
    ),
    "dabsn_hip_read3_fwd_keep": (
        [i32, i64, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, PTR4, vp,
         vp, sz, vp, sz, vp],
        i32,
    ),
    "dabsn_hip_read3_decode_workspace_bytes": ([i32, i64, i64, i64, i64], sz),
    "dabsn_hip_read_dense_workspace_bytes": ([i64, i64, i64, i64, i32], sz),
    "dabsn_hip_read_dense_fwd": ([i64] * 4 + [vp] * 8 + [vp] * 4 + [vp, vp, vp, sz, vp], i32),
    "dabsn_hip_read_dense_fwd_weights": (
        [i64] * 4 + [vp] * 8 + [vp] * 4 + [vp, vp, vp, vp, vp, vp, sz, vp], i32),
    "dabsn_hip_read_dense_bwd": (
        [i64] * 4 + [vp] + [vp] * 8 + [vp] * 4 + [vp] + [vp] * 9 + [vp, sz, vp], i32),
    "dabsn_hip_permanent_scan_fwd": ([i64, i64, i64, vp, vp, vp, vp, vp], i32),
    "dabsn_hip_permanent_scan_workspace_bytes": ([i64, i64, i64], sz),
    "dabsn_hip_permanent_scan_bwd": ([i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp], i32),
    "dabsn_hip_local_field_workspace_bytes": ([i64, i64, i64, i32], sz),
    "dabsn_hip_local_field_gather": ([i32, i64, i64, i64, i64, i64, vp, vp, vp, vp, sz, vp], i32),
    "dabsn_hip_local_field_gather_bwd": (
        [i32, i64, i64, i64, i64, i64, vp, vp, vp, vp, sz, vp], i32),
    "dabsn_hip_means_glue": ([i64, i64, i64, vp, i64, PTR8, i32, vp, vp, vp, vp], i32),
    "dabsn_hip_ce_fwd": ([i32, i64, i64, vp, i64, vp, i64, vp, vp, vp, vp], i32),
    "dabsn_hip_ce_bwd": ([i32, i64, i64, vp, i64, vp, i64, vp, vp, vp, vp, vp], i32),
    "dabsn_hip_read3_decode": (
        [i32, i64, i64, i64, i64, vp, vp, i64, i64, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, PTR4,
         vp, vp, sz, vp],
        i32,
    ),
    "dabsn_hip_read3_decode_members": (
        [i32, i64, i64, i64, vp, vp, i64, i64, vp, vp, vp, i64, vp, vp, vp, vp, PTR4, vp, vp, sz,
         vp],
        i32,
    ),
    "dabsn_hip_read3_decode_noalloc": (
        [i32, i64, i64, i64, i64, vp, vp, i64, i64, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, PTR4,
         vp, vp],
        i32,
    ),
    "dabsn_hip_read3_bwd": (
        [i32, i64, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, PTR4]
        + [vp] * 4 + [vp] * 5 + [vp, sz, vp],
        i32,
    ),
    "dabsn_hip_read3_bwd_after_fwd": (
        [i32, i64, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, PTR4]
        + [vp] * 4 + [vp] * 5 + [vp, sz, vp, sz, vp],
        i32,
    ),
}

EXPORTED = tuple(_SIGNATURES)


def load():
    """Load (once) and return the ctypes library; raises if it is missing."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = Path(os.environ.get("DABSN_HIP_LIB", str(LIB_PATH)))
        if not path.exists():
            _load_error = f"{path} is not built (run dabsn_amd.build.build())"
            raise RuntimeError(f"DABSN HIP library unavailable: {_load_error}")
        lib = ctypes.CDLL(str(path))
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        version = lib.dabsn_hip_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"DABSN HIP library ABI {version} != expected {ABI_VERSION}")
        _lib = lib
        return lib


def available() -> bool:
    try:
        load()
        return True
    except Exception:  # noqa: BLE001 - reported by status()
        return False


def load_error() -> str | None:
    return _load_error


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = _lib.dabsn_hip_last_error().decode(errors="replace") if _lib else "library not loaded"
        raise RuntimeError(f"DABSN HIP {what} failed (status {rc}): {msg}")
