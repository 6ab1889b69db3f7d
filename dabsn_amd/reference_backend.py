"""The reference-side binding: run the reference package's registered ``dabsn::`` operators
on this library's HIP kernels.

The reference attaches per-device kernels to its own operator objects with
``register_kernel(device)`` (kernels/cpu.py:1020-1044, triton.py:504,
compact_flash.py:332-333). A ROCm backend does the same with the operators below, whose
schemas this package reproduces exactly (tests/golden/ref/op_schemas.json holds the
reference's; tests check them equal). Imported into a process where the reference's
operators are already registered, this package registers its own under ``dabsn_amd::``
(the reference owns ``dabsn::``; set ``DABSN_AMD_OP_NAMESPACE=dabsn_amd`` when this package
is imported first), so both live side by side; ``attach`` then hands the reference's
operator objects the device bodies of this package's operators:

    # src/dabsn/kernels/rocm.py (the file a maintainer adds to the reference)
    def enable_rocm(required: bool = False) -> bool:
        from dabsn_amd import reference_backend
        from .admitted import (_admitted_three_way_read_native_backward_op,
                               _admitted_three_way_read_native_op)
        from .batched_runtime import _core_scan_batched_op
        from .compact_flash import _compact_flash_backward_op, _compact_flash_op
        from .local_field import _local_field_gather_op
        from .long import _linear_recurrence_op, _linrec_bwd_op
        from .permanent import _permanent_delta_scan_op
        reference_backend.attach({
            "core_scan_batched": _core_scan_batched_op,
            "admitted_three_way_read_compact_flash": _compact_flash_op,
            "_admitted_three_way_read_compact_flash_backward": _compact_flash_backward_op,
            "linear_recurrence": _linear_recurrence_op,
            "_linrec_backward": _linrec_bwd_op,
            "permanent_delta_scan": _permanent_delta_scan_op,
            "local_field_gather": _local_field_gather_op,
            "admitted_three_way_read_native": _admitted_three_way_read_native_op,
            "_admitted_three_way_read_backward": _admitted_three_way_read_native_backward_op,
        })
        return True

Three of the reference's autograd formulas do their device work outside a registered
backward operator -- the core op's Python reverse loop (batched_runtime.py:1589-1634), the
permanent scan's Triton backward (permanent.py:402-433) and the local field's atomic
scatter (local_field.py:224-236) -- so ``attach`` re-registers those three with the HIP
reverse scans; the other operators keep the reference's autograd, which calls backward
operators that now run here.
"""

from __future__ import annotations

from typing import Mapping

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
}

# Reference operator name -> (backward, setup_context) that replace its autograd.
AUTOGRAD = {
    "core_scan_batched": (ops._core_backward, ops._core_setup),
    "permanent_delta_scan": (ops._permanent_bwd, ops._permanent_setup),
    "local_field_gather": (ops._field_bwd, ops._field_setup),
}


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
