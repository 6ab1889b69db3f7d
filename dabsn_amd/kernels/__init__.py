"""Backend selection, status and primitive map for the ROCm (gfx950) backend.

Mirrors the reference backend API (src/dabsn/kernels/__init__.py:38-163):
``enable(backend, required=...)`` is process-wide and refuses to switch backends in
one process; ``status()`` reports what is actually loaded; ``PRIMITIVES`` maps each
hot-path primitive to its implementation. This package provides one backend, the
hand-written HIP kernels (``"rocm"``; ``"auto"`` and ``"cuda"`` select it too, since
PyTorch-ROCm names the device ``cuda``). There is no CPU product path: CPU tensors
raise in every operator.
"""

from __future__ import annotations

from dataclasses import asdict, dataclass

import torch
import torch.nn.functional as F
from torch import Tensor

from .. import _lib
from . import ops
from . import vmap_rules  # noqa: F401  (registers the operators' vmap rules)
from .ops import (
    admitted_three_way_read_compact_flash,
    bank_gather,
    bank_select,
    check_errors,
    core_scan_batched,
    linear_recurrence,
    local_field_gather_backward,
    long_scan_fused,
    normalize_rows,
    parameters_changed,
    permanent_delta_scan,
    read_tape_stats,
)

_ACTIVE_BACKEND = "none"


@dataclass(frozen=True)
class Primitive:
    name: str
    reference: str
    rocm: str
    backward: str
    geometries: tuple[str, ...]
    validation: str


PRIMITIVES = (
    Primitive("core_scan", "DABSNCore.forward / DABSNCore.forward_from_state",
              "persistent cooperative HIP scan, MFMA recurrent product, sc1 step exchange",
              "persistent cooperative HIP reverse scan + hipBLASLt weight-gradient GEMM",
              ("seq",), "oracle (C restatement of cpu_runtime.cpp) forward/backward parity"),
    Primitive("admitted_three_way_read", "DABSNRead._three_way_read",
              "MFMA score GEMM + masked softmax rows + MFMA value GEMM",
              "MFMA GEMMs for dP, dQ, dK, dV + score-gradient rows",
              ("seq", "field"), "oracle (cpu_runtime.cpp:321-662 restatement) parity"),
    Primitive("recurrent_long_read", "DABSNRead._long_scan_from_state",
              "fused three-recurrence HIP scan with fp32 checkpoints",
              "segment-replay HIP reverse scan", ("seq",),
              "oracle long-scan forward/backward parity"),
    Primitive("linear_recurrence", ops._q("linear_recurrence"), "HIP channel scan",
              "HIP analytic reverse", ("seq",), "oracle linrec parity"),
    Primitive("admitted_selection", "DABSNRead._unified_forward (read.py:185-239)",
              "HIP cummax/stable-partition kernel", "none (integer)", ("seq",),
              "bit-exact against the oracle stable partition"),
    Primitive("permanent_delta_read", "permanent_delta_scan",
              "HIP delta scan: one wave per value row, state row in registers",
              "HIP state-tape recompute + reverse adjoint, deterministic row sums", ("seq",),
              "oracle (cpu_runtime.cpp:1075-1188 restatement) forward/backward parity"),
    Primitive("local_field_gather", "inputs[:, patch]", "HIP 16-byte row gather",
              "HIP inverse-index scatter-add in the reference loop's order", ("field", "hybrid"),
              "bit-exact against the oracle gather/scatter"),
)

_PRIMITIVE_HITS = {"permanent_delta_scan": 0, "local_field_gather": 0}


def permanent_delta_read(expression: Tensor, long_state: Tensor, progress: Tensor,
                         plasticity: Tensor, energy: Tensor, saturation: Tensor, *,
                         phase_gain: Tensor, progress_gain: Tensor, beta_gain: Tensor,
                         consolidation_energy_gain: Tensor,
                         consolidation_saturation_gain: Tensor, beta_bias: Tensor) -> Tensor:
    """Permanent read (reference permanent.py:457-484): keys are the normalised
    expression shifted by the long state and progress, the write strength is a sigmoid of
    the mean plasticity, energy and saturation, and the scan runs on the HIP kernel."""
    key = F.normalize(expression + phase_gain * long_state + progress_gain * progress, dim=-1)
    beta = torch.sigmoid(beta_gain * plasticity.mean(dim=-1)
                         + consolidation_energy_gain * energy.mean(dim=-1)
                         + consolidation_saturation_gain * saturation.mean(dim=-1) + beta_bias)
    _PRIMITIVE_HITS["permanent_delta_scan"] += 1
    return permanent_delta_scan(key, expression, beta)


def local_field_gather(inputs: Tensor, patch: Tensor) -> tuple[Tensor, str]:
    """``inputs[:, patch]`` with the route label the reference's helper returns
    (local_field.py:257-274)."""
    _PRIMITIVE_HITS["local_field_gather"] += 1
    return ops.local_field_gather(inputs, patch), "rocm_hip_patch_gather_then_shared_core"



def primitive_map() -> list[dict[str, object]]:
    return [asdict(p) for p in PRIMITIVES]


def enable(backend: str = "auto", *, required: bool = False) -> dict[str, object]:
    """Enable the ROCm backend process-wide (see module docstring)."""
    global _ACTIVE_BACKEND
    normalized = backend.lower()
    if normalized in {"auto", "cuda", "hip"}:
        normalized = "rocm"
    if normalized != "rocm":
        raise ValueError("backend must be one of: auto, rocm, cuda, hip")
    if _ACTIVE_BACKEND not in {"none", normalized}:
        raise RuntimeError(f"DABSN backend already selected as {_ACTIVE_BACKEND}; "
                           "select a different backend in a fresh process")
    ok = _lib.available() and torch.cuda.is_available()
    if required and not ok:
        reason = _lib.load_error() or "no ROCm device is visible"
        raise RuntimeError(f"required ROCm DABSN backend unavailable: {reason}")
    if ok:
        from ..core import DABSNCore
        from ..read import DABSNRead

        DABSNCore._rocm_native_enabled = True
        DABSNRead._rocm_native_enabled = True
        _ACTIVE_BACKEND = normalized
    return status()


def status() -> dict[str, object]:
    lib_ok = _lib.available()
    arch = None
    if torch.cuda.is_available():
        arch = getattr(torch.cuda.get_device_properties(0), "gcnArchName", None)
    return {
        "active_backend": _ACTIVE_BACKEND,
        "torch_version": torch.__version__,
        "hip_version": getattr(torch.version, "hip", None),
        "device_available": torch.cuda.is_available(),
        "device_arch": arch,
        "rocm": {
            "library": str(_lib.LIB_PATH),
            "library_loaded": lib_ok,
            "load_error": _lib.load_error(),
            "abi_version": _lib.ABI_VERSION,
            "namespace": ops.NAMESPACE,
            "operators": list(ops.OPERATORS),
        },
        "permanent": {"hip_available": lib_ok, "hits": _PRIMITIVE_HITS["permanent_delta_scan"]},
        "local_field": {"hip_available": lib_ok, "hits": _PRIMITIVE_HITS["local_field_gather"]},
        "primitives": primitive_map(),
    }


__all__ = [
    "PRIMITIVES",
    "Primitive",
    "admitted_three_way_read_compact_flash",
    "bank_gather",
    "bank_select",
    "check_errors",
    "core_scan_batched",
    "enable",
    "linear_recurrence",
    "local_field_gather",
    "local_field_gather_backward",
    "long_scan_fused",
    "normalize_rows",
    "parameters_changed",
    "permanent_delta_read",
    "permanent_delta_scan",
    "primitive_map",
    "read_tape_stats",
    "status",
]
