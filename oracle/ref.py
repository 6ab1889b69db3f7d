"""The reference's own CPU backend, compiled from its source -- TEST INFRASTRUCTURE ONLY.

``oracle/ref.mk`` compiles ``src/dabsn/kernels/cpu_runtime.cpp`` from the reference tree
(present only in the build container) into ``oracle/_ref/``. The tests use the module it
builds to pin the C restatement in ``dabsn_oracle.c`` function by function:

  * ``dabsn_core_scan_fwd_train`` (cpu_runtime.cpp:672-837) and the analytic reverse
    ``dabsn_core_scan_bwd`` (cpu_runtime.cpp:844-1072);
  * ``three_way_read_cpu`` / ``three_way_read_bwd`` (cpu_runtime.cpp:321-438, 479-662);
  * ``linrec_forward_cpu`` / ``linrec_backward_cpu`` (cpu_runtime.cpp:92-143, 440-477);
  * ``permanent_delta_scan_cpu`` / ``_bwd_cpu`` (cpu_runtime.cpp:1075-1188);
  * ``local_field_gather_cpu`` / ``_bwd_cpu`` (cpu_runtime.cpp:1191-1237).

Nothing in the product package loads it. The module is a pybind11 torch extension, so it
is imported after torch.
"""

from __future__ import annotations

import importlib.util
import subprocess
from pathlib import Path

_HERE = Path(__file__).resolve().parent
_OUT = _HERE / "_ref"
REFERENCE_SOURCE = Path("/root/reference/src/dabsn/kernels/cpu_runtime.cpp")
_MOD = None


def build() -> bool:
    """Compile the reference CPU backend when its source is present. Returns whether a
    build ran."""
    if not REFERENCE_SOURCE.exists():
        return False
    subprocess.run(["make", "-s", "-f", str(_HERE / "ref.mk")], check=True)
    return True


def path() -> Path | None:
    found = sorted(_OUT.glob("dabsn_ref_cpu*.so"))
    return found[0] if found else None


def load():
    """The compiled reference module, or None when it has not been built."""
    global _MOD
    if _MOD is None:
        so = path()
        if so is None:
            return None
        import torch  # noqa: F401  (the extension links against libtorch)

        spec = importlib.util.spec_from_file_location("dabsn_ref_cpu", so)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        _MOD = mod
    return _MOD
