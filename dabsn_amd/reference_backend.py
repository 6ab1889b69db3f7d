"""The reference-side binding: run the reference package's registered ``dabsn::`` operators
and its core / read / long-memory dispatch on this library's HIP kernels.

The reference attaches per-device kernels to its own operator objects with
``register_kernel(device)`` (kernels/cpu.py:1020-1044, triton.py:504,
compact_flash.py:332-333) and routes its modules with class flags set by its enable hooks
(``enable_triton_kernels``, triton.py:486-510; ``enable_fused_long_read``, long.py:582-589).
Imported into a process where the reference's operators are already registered, this
package registers its own under ``dabsn_amd::`` (the reference owns ``dabsn::``; set
``DABSN_AMD_OP_NAMESPACE=dabsn_amd`` when this package is imported first), so both live
side by side.

``enable_rocm()`` is the hook a maintainer exposes as ``dabsn.kernels.rocm.enable_rocm``
(called from ``dabsn.kernels.enable("rocm")``). It

* attaches the HIP bodies of this package's operators to the reference's ten replaced
  operators (``attach``), and the HIP reverse scans as the autograd of the three whose
  backward is not an operator there (the core op's Python reverse loop,
  batched_runtime.py:1589-1634; the permanent scan's Triton backward, permanent.py:402-433;
  the local field's atomic scatter, local_field.py:224-236);
* sets the routing flags ``DABSNCore._cuda_native_enabled``,
  ``DABSNRead._cuda_native_enabled`` and ``DABSNRead._long_native_enabled`` (with their
  ``*_required`` companions), so device tensors take the compact read
  (read.py:278, 461, 758) and the native long channel (read.py:586);
* installs the read dispatcher the compact path imports at call time
  (``dabsn.kernels.triton.cuda_compact_three_way_read``, read.py:465): every compact
  read, training and inference, goes to the registered
  ``dabsn::admitted_three_way_read_compact_flash`` (HIP forward, HIP backward through
  ``dabsn::_admitted_three_way_read_compact_flash_backward``) instead of the composite
  dense-BMM operator or the Triton-runtime density heuristics (triton.py:344-480);
* installs the long-channel entry the flag selects
  (``dabsn.kernels.long.fused_long_scan_from_state``, read.py:586-596): the three
  recurrences and their glue run as one fused HIP scan (``dabsn::long_scan_fused``, the
  same math as long.py:492-579) with its HIP backward.

The flag-off dense path (read.py:498-558, ``dabsn::admitted_three_way_read``) is attached
too, so a caller that clears the flags still runs its forward on the device (the
reference's own autograd differentiates it from the weights the forward returns).
"""

from __future__ import annotations

import dataclasses
import types
from typing import Mapping, Optional

import torch

from .kernels import ops

# Reference operator name -> this package's operator with the same schema.
KERNELS = {
    "core_scan_batched": ops.core_scan_batched,
    "admitted_three_way_read_compact_flash": ops.admitted_three_way_read_compact_flash,
    "_admitted_three_way_read_compact_flash_backward":
        ops.admitted_three_way_read_compact_flash_backward,
    "linear_recurrence": ops.linear_recurrence,
    "_linrec_backward": ops.linrec_backward,
    "permanent_delta_scan": ops.permanent_delta_scan,
    "local_field_gather": ops.local_field_gather,
    "admitted_three_way_read_native": ops.admitted_three_way_read_native,
    "_admitted_three_way_read_backward": ops.admitted_three_way_read_native_backward,
    "admitted_three_way_read": ops.admitted_three_way_read,
}

# Reference operator name -> (backward, setup_context) that replace its autograd.
AUTOGRAD = {
    "core_scan_batched": (ops._core_backward, ops._core_setup),
    "permanent_delta_scan": (ops._permanent_bwd, ops._permanent_setup),
    "local_field_gather": (ops._field_bwd, ops._field_setup),
}

_READ_MODES = {"seq": 0, "field": 1}
# The long channel's four coefficient logits, in the order of dabsn::long_scan_fused.
_LONG_LOGITS = ("logit_expect_retain", "logit_retention_decay", "logit_retain",
                "logit_retention_strength")


def attach(targets: Mapping[str, object], device: str = "cuda") -> list[str]:
    """Register this library's kernels as the ``device`` kernels of the given operators
    (reference name -> operator object or qualified name) and, for the three operators in
    ``AUTOGRAD``, their HIP backward. Returns the names attached; an unknown name raises."""
    done = []
    for name, target in targets.items():
        if name not in KERNELS:
            raise KeyError(f"no HIP kernel for operator {name!r}")
        body = getattr(KERNELS[name], "_init_fn")  # the operator's undecorated device body
        torch.library.register_kernel(target, device, body)
        if name in AUTOGRAD:
            backward, setup = AUTOGRAD[name]
            torch.library.register_autograd(target, backward, setup_context=setup)
        done.append(name)
    return done


@dataclasses.dataclass
class ReferenceSide:
    """Where the binding reaches into the reference: its two module classes, the module
    holding the compact-read dispatcher, the module holding the long-channel entry, and
    the namespace of its operators."""

    core: type
    read: type
    dispatch: types.ModuleType
    long: types.ModuleType
    namespace: str = "dabsn"

    @classmethod
    def imported(cls) -> "ReferenceSide":
        """The reference package itself (``import dabsn``); importing its kernel modules
        registers its operators."""
        import dabsn.kernels.admitted  # noqa: F401
        import dabsn.kernels.batched_runtime  # noqa: F401
        import dabsn.kernels.compact_flash  # noqa: F401
        import dabsn.kernels.local_field  # noqa: F401
        import dabsn.kernels.long as long_module
        import dabsn.kernels.permanent  # noqa: F401
        import dabsn.kernels.triton as dispatch
        from dabsn.core import DABSNCore
        from dabsn.read import DABSNRead

        return cls(DABSNCore, DABSNRead, dispatch, long_module)


def compact_read(namespace: str):
    """The compact-read dispatcher (the signature of triton.py:314-330) running every read
    on ``namespace``'s registered compact operator."""
    op = getattr(getattr(torch.ops, namespace), "admitted_three_way_read_compact_flash")

    def rocm_compact_three_way_read(read, query, bank_keys, bank_writes, next_writes, cocktail,
                                    bank_cocktail, bank_key_bias, bank_admission, scale,
                                    bank_idx, bank_valid, *, mode: str):
        if not query.is_cuda:
            raise TypeError("the ROCm compact admitted read requires device tensors")
        if mode not in _READ_MODES:
            raise ValueError("compact admitted-read mode must be seq or field")
        out = op(query, bank_keys, bank_writes, next_writes, cocktail, bank_cocktail,
                 bank_key_bias, bank_admission, scale, bank_idx, bank_valid, _READ_MODES[mode],
                 read.short_gain, read.pad_gain, read.induct_gain, read.cocktail_gain)
        read._last_three_way_backend = ("registered_compact_flash_rocm_trainable"
                                        if torch.is_grad_enabled() else
                                        "registered_compact_flash_rocm_infer")
        return out

    return rocm_compact_three_way_read


def rocm_long_scan_from_state(read, write, plasticity, novelty, *, initial_state=None,
                              return_final_state: bool = False):
    """The long channel (the signature and results of long.py:492-579) as one fused HIP
    scan with its HIP backward. The state is carried in fp32 (as long.py:507-511 does for
    inference; the three linear recurrences there accumulate in fp32 either way)."""
    del novelty  # unused by the long channel (long.py:501)
    if bool(getattr(type(read), "_long_native_required", False)) and not write.is_cuda:
        raise RuntimeError("the ROCm long-memory recurrence was required, but received a CPU tensor")
    batch, _, hidden = write.shape
    if initial_state is None:
        z = torch.zeros(batch, hidden, device=write.device, dtype=torch.float32)
        initial_state = (z, torch.zeros_like(z), torch.ones_like(z))
    else:
        if any(s.shape != (batch, hidden) for s in initial_state):
            raise ValueError(f"initial long-scan state must have shape {(batch, hidden)}")
        initial_state = tuple(s.to(device=write.device, dtype=torch.float32) for s in initial_state)
    logits = [getattr(read, n) for n in _LONG_LOGITS]
    long, lf, ef, rf, _ = ops.direct.long_scan_fused(write, plasticity, *logits, *initial_state)
    read._last_long_backend = "rocm_hip"
    if return_final_state:
        return long, (lf, ef, rf)
    return long


def enable_rocm(side: Optional[ReferenceSide] = None, *, required: bool = False) -> dict:
    """Attach the HIP kernels to the reference and route its modules to them (see the
    module docstring). ``side`` defaults to the imported reference package. Returns the
    status entries the reference's ``status()`` reports for a device backend."""
    if required and not torch.cuda.is_available():
        raise RuntimeError("ROCm was required for the DABSN HIP kernels, but no device is available")
    side = side or ReferenceSide.imported()
    attached = attach({name: f"{side.namespace}::{name}" for name in KERNELS})
    for cls, flags in ((side.core, ("_cuda_native",)),
                       (side.read, ("_cuda_native", "_long_native"))):
        for flag in flags:
            setattr(cls, f"{flag}_enabled", True)
            setattr(cls, f"{flag}_required", bool(required))
    side.dispatch.cuda_compact_three_way_read = compact_read(side.namespace)
    side.long.fused_long_scan_from_state = rocm_long_scan_from_state
    return {"core_scan": True, "admitted_three_way_read": True, "long": True,
            "operators": sorted(attached)}
