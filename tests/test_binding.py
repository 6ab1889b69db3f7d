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
    bit for bit: the same kernels run. The 4-output dense operator of the flag-off path
    returns the same read and its three softmaxes.
  * GPU: ``reference_backend.enable_rocm`` on stand-ins of the reference's side: the
    routing flags are set and the compact read (training and inference, seq and field) and
    the long channel reach the HIP operators.
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

    lib = _define_standins(NS)
    attached = reference_backend.attach({name: f"{NS}::{name}" for name in SCHEMAS})
    assert sorted(attached) == sorted(SCHEMAS)
    _LIB = lib


def _define_standins(ns):
    """The reference's operators (its schemas) under ``ns``, with the autograd the reference
    registers for the three ops whose backward is an operator (compact_flash.py:275-296,
    long.py:418-437, admitted.py:590-622)."""
    lib = torch.library.Library(ns, "DEF")
    for name, schema in SCHEMAS.items():
        lib.define(schema.split("::", 1)[1])

    def q(name):
        return getattr(getattr(torch.ops, ns), name)

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

    torch.library.register_autograd(f"{ns}::admitted_three_way_read_compact_flash", read_bwd,
                                    setup_context=read_setup, lib=lib)
    torch.library.register_autograd(f"{ns}::linear_recurrence", lin_bwd, setup_context=lin_setup,
                                    lib=lib)
    torch.library.register_autograd(f"{ns}::admitted_three_way_read_native", dense_bwd,
                                    setup_context=dense_setup, lib=lib)
    return lib


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
    # the 4-output dense op of the flag-off path: the same output, and its softmaxes
    with torch.no_grad():
        out4 = ref.admitted_three_way_read(*dense)
        assert torch.equal(out4[0], ops.admitted_three_way_read_native(*dense))
        assert torch.equal(out4[1], ops.admitted_three_way_read(*dense)[1])
        elig, ielig = dense[11].bool(), dense[12].bool()
        ones = torch.ones_like(out4[1][..., 0])
        for w, e in ((out4[1], elig), (out4[2], elig), (out4[3], ielig)):
            rows = w.sum(-1)[e]
            assert torch.allclose(rows, ones[e], atol=1e-5)
            assert float(w[~e].abs().max() if (~e).any() else 0.0) == 0.0

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


@pytest.mark.gpu
def test_enable_rocm_routes_the_reference_modules(cuda_device):
    """``reference_backend.enable_rocm`` on stand-ins of the reference's side (its operators
    under their schemas, its two module classes, the dispatcher module the compact read
    imports and the long-channel module): the routing flags are set, every compact read --
    with and without autograd, seq and field -- and the long channel run the HIP
    operators, bit for bit the same outputs and gradients as this package's own."""
    import types

    from dabsn_amd import reference_backend
    from test_dense_read import dense_case

    ns = "dabsn_refsim_routing"
    lib = _define_standins(ns)  # noqa: F841  (kept alive for the test)
    sentinel = lambda *a, **k: (_ for _ in ()).throw(AssertionError("not routed"))  # noqa: E731
    side = reference_backend.ReferenceSide(
        core=type("DABSNCore", (), {}), read=type("DABSNRead", (), {}),
        dispatch=types.ModuleType("triton_standin"), long=types.ModuleType("long_standin"),
        namespace=ns)
    side.dispatch.cuda_compact_three_way_read = sentinel
    side.long.fused_long_scan_from_state = sentinel
    status = reference_backend.enable_rocm(side, required=True)
    assert status["operators"] == sorted(SCHEMAS)
    assert side.core._cuda_native_enabled and side.core._cuda_native_required
    assert side.read._cuda_native_enabled and side.read._long_native_enabled
    assert side.read._long_native_required

    d = cuda_device
    g = torch.Generator().manual_seed(3)
    B, T, H = 2, 24, 16
    x = dense_case(7, B, T, T, H)
    idx = torch.arange(T).expand(B, T).contiguous().to(d)
    valid = (torch.rand(B, T, generator=g) < 0.8).to(d)
    gains = [t.to(d) for t in x[13:]]
    stub = types.SimpleNamespace(short_gain=gains[0], pad_gain=gains[1], induct_gain=gains[2],
                                 cocktail_gain=gains[3])
    route = side.dispatch.cuda_compact_three_way_read
    for mode, code in (("seq", 0), ("field", 1)):
        args = [t.to(d) for t in x[:9]]
        with torch.no_grad():
            got = route(stub, *args, idx, valid, mode=mode)
        assert stub._last_three_way_backend.endswith("infer")
        assert torch.equal(got, ops.admitted_three_way_read_compact_flash(
            *args, idx, valid, code, *gains))
        a = [t.clone().requires_grad_(True) for t in args]
        b = [t.clone().requires_grad_(True) for t in args]
        out_a = route(stub, *a, idx, valid, mode=mode)
        out_b = ops.admitted_three_way_read_compact_flash(*b, idx, valid, code, *gains)
        assert stub._last_three_way_backend.endswith("trainable")
        seed = torch.randn(out_a.shape, generator=g).to(d)
        for ga, gb in zip(torch.autograd.grad(out_a, a, seed), torch.autograd.grad(out_b, b, seed)):
            assert torch.equal(ga, gb)

    w = torch.randn(B, 30, H, generator=g).to(d)
    p = torch.rand(B, 30, H, generator=g).to(d)
    logits = {n: torch.tensor([v], device=d, requires_grad=True) for n, v in (
        ("logit_expect_retain", 2.2), ("logit_retention_decay", 2.0), ("logit_retain", 1.7),
        ("logit_retention_strength", 1.4))}
    rstub = types.SimpleNamespace(**logits)
    wl = w.clone().requires_grad_(True)
    long, final = side.long.fused_long_scan_from_state(rstub, wl, p, None, return_final_state=True)
    assert rstub._last_long_backend == "rocm_hip"
    z = torch.zeros(B, H, device=d)
    wr = w.clone().requires_grad_(True)
    mine = ops.long_scan_fused(wr, p, *logits.values(), z, z.clone(), torch.ones_like(z))
    assert torch.equal(long, mine[0]) and all(torch.equal(a, b) for a, b in zip(final, mine[1:4]))
    seed = torch.randn(long.shape, generator=g).to(d)
    ga = torch.autograd.grad(long, [wl, *logits.values()], seed)
    gb = torch.autograd.grad(mine[0], [wr, *logits.values()], seed)
    for a_, b_ in zip(ga, gb):
        assert torch.equal(a_, b_)
