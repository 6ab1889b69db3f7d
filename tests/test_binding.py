"""The drop-in boundary from the reference's side.

  * Every operator this build replaces has exactly the reference's dispatcher schema
    (tests/golden/ref/op_schemas.json, printed by the reference's own registration).
  * With the reference's operators already registered in the process, this package
    registers its own under ``dabsn_amd::`` and both coexist.
  * GPU: ``dabsn_amd.reference_backend.attach`` -- the binding a maintainer adds to the
    reference -- run against stand-in operators defined from the reference's schemas (the
    reference cannot be imported here) and wired as the reference wires its autograd
    (compact_flash.py, long.py, admitted.py: the forward op's backward calls its backward
    op). Outputs and gradients through the stand-ins equal this package's own operators
    bit for bit: the same kernels run.
"""

from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from dabsn_amd.kernels import ops

ROOT = Path(__file__).resolve().parents[1]
SCHEMAS = json.loads((ROOT / "tests" / "golden" / "ref" / "op_schemas.json").read_text())


def test_operator_schemas_equal_the_reference():
    for name, ref in SCHEMAS.items():
        mine = str(getattr(getattr(torch.ops, ops.NAMESPACE), name).default._schema)
        assert mine.replace(f"{ops.NAMESPACE}::", "dabsn::", 1) == ref, name


def test_coexists_with_the_reference_operators():
    code = (
        "import torch\n"
        "@torch.library.custom_op('dabsn::core_scan_batched', mutates_args=())\n"
        "def f(x: torch.Tensor) -> torch.Tensor:\n"
        "    return x.clone()\n"
        "import dabsn_amd\n"
        "from dabsn_amd.kernels import ops\n"
        "assert ops.NAMESPACE == 'dabsn_amd', ops.NAMESPACE\n"
        "assert dabsn_amd.kernels.status()['rocm']['namespace'] == 'dabsn_amd'\n"
        "assert hasattr(torch.ops.dabsn_amd, 'core_scan_batched')\n"
        "x = torch.ones(2)\n"
        "assert torch.equal(torch.ops.dabsn.core_scan_batched(x), x)\n"
        "print('ok')\n")
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stderr[-2000:]


# ---- GPU: the binding on stand-ins of the reference's operators -------------------------
_LIB = None
NS = "dabsn_refsim"


def _standins():
    """Define the reference's operators (its schemas) under NS once, wire the autograd the
    reference registers for the three ops whose backward is an operator, then attach."""
    global _LIB
    if _LIB is not None:
        return
    from dabsn_amd import reference_backend

    lib = torch.library.Library(NS, "DEF")
    for name, schema in SCHEMAS.items():
        lib.define(schema.split("::", 1)[1])

    def q(name):
        return getattr(getattr(torch.ops, NS), name)

    def read_setup(ctx, inputs, output):
        ctx.save_for_backward(*inputs[:11], *inputs[12:])
        ctx.mode = int(inputs[11])

    def read_bwd(ctx, g):
        t = ctx.saved_tensors
        r = q("_admitted_three_way_read_compact_flash_backward")(g, *t[:11], ctx.mode, *t[11:])
        return (*r[:9], None, None, None, *r[9:])

    def lin_setup(ctx, inputs, output):
        ctx.save_for_backward(*inputs)

    def lin_bwd(ctx, g):
        return tuple(q("_linrec_backward")(*ctx.saved_tensors, g))

    def dense_setup(ctx, inputs, output):
        ctx.save_for_backward(*inputs)

    def dense_bwd(ctx, g):
        r = q("_admitted_three_way_read_backward")(g, *ctx.saved_tensors)
        return (*r[:9], None, None, None, None, *r[9:])

    torch.library.register_autograd(f"{NS}::admitted_three_way_read_compact_flash", read_bwd,
                                    setup_context=read_setup, lib=lib)
    torch.library.register_autograd(f"{NS}::linear_recurrence", lin_bwd, setup_context=lin_setup,
                                    lib=lib)
    torch.library.register_autograd(f"{NS}::admitted_three_way_read_native", dense_bwd,
                                    setup_context=dense_setup, lib=lib)
    attached = reference_backend.attach({name: f"{NS}::{name}" for name in SCHEMAS})
    assert sorted(attached) == sorted(SCHEMAS)
    _LIB = lib


def _same_through_both(mine, theirs, args, float_idx):
    """Forward outputs and the gradients of the float inputs in ``float_idx`` agree."""
    a = [x.detach().clone().requires_grad_(i in float_idx) if torch.is_tensor(x) else x
         for i, x in enumerate(args)]
    b = [x.detach().clone().requires_grad_(i in float_idx) if torch.is_tensor(x) else x
         for i, x in enumerate(args)]
    out_a, out_b = mine(*a), theirs(*b)
    outs_a = list(out_a) if isinstance(out_a, (tuple, list)) else [out_a]
    outs_b = list(out_b) if isinstance(out_b, (tuple, list)) else [out_b]
    for x, y in zip(outs_a, outs_b):
        assert torch.equal(x, y)
    gen = torch.Generator().manual_seed(1)
    diff = [i for i, o in enumerate(outs_a) if o.is_floating_point() and o.requires_grad]
    seeds = [torch.randn(outs_a[i].shape, generator=gen).to(outs_a[i]) for i in diff]
    ga = torch.autograd.grad([outs_a[i] for i in diff], [a[i] for i in float_idx], seeds,
                             allow_unused=True)
    gb = torch.autograd.grad([outs_b[i] for i in diff], [b[i] for i in float_idx], seeds,
                             allow_unused=True)
    for i, x, y in zip(float_idx, ga, gb):
        assert (x is None) == (y is None), i
        if x is not None:
            assert torch.equal(x, y), f"gradient of input {i}"


@pytest.mark.gpu
def test_reference_binding_on_stand_in_operators(cuda_device):
    from helpers import core_case
    from test_dense_read import dense_case

    _standins()
    ref = getattr(torch.ops, NS)
    d = cuda_device
    core = [t.to(d) for t in core_case(5, 3, 9, 16)]
    _same_through_both(ops.core_scan_batched, ref.core_scan_batched, core, list(range(26)))

    g = torch.Generator().manual_seed(2)
    lin = [torch.rand(2, 40, 8, generator=g).to(d), torch.randn(2, 40, 8, generator=g).to(d),
           torch.randn(2, 8, generator=g).to(d)]
    _same_through_both(ops.linear_recurrence, ref.linear_recurrence, lin, [0, 1, 2])

    perm = [torch.nn.functional.normalize(torch.randn(2, 12, 16, generator=g), dim=-1).to(d),
            torch.randn(2, 12, 16, generator=g).to(d), torch.rand(2, 12, generator=g).to(d)]
    _same_through_both(ops.permanent_delta_scan, ref.permanent_delta_scan, perm, [0, 1, 2])

    field = [torch.randn(2, 10, 8, generator=g).to(d),
             torch.randint(0, 10, (10, 3), generator=g).to(d)]
    _same_through_both(ops.local_field_gather, ref.local_field_gather, field, [0])

    dense = [t.to(d) for t in dense_case(6, 2, 20, 17, 12)]
    _same_through_both(ops.admitted_three_way_read_native, ref.admitted_three_way_read_native,
                       dense, [0, 1, 2, 3, 4, 5, 6, 7, 8, 13, 14, 15, 16])

    # compact read: a causal bank over the query positions (seq mode)
    B, T, H = 2, 24, 16
    x = dense_case(7, B, T, T, H)
    idx = torch.arange(T).expand(B, T).contiguous()
    valid = torch.rand(B, T, generator=g) < 0.8
    compact = [x[0], x[1], x[2], x[3], x[4], x[5], x[6], x[7], x[8], idx, valid, 0, *x[13:]]
    compact = [t.to(d) if torch.is_tensor(t) else t for t in compact]
    _same_through_both(ops.admitted_three_way_read_compact_flash,
                       ref.admitted_three_way_read_compact_flash, compact,
                       [0, 1, 2, 3, 4, 5, 6, 7, 8, 12, 13, 14, 15])
