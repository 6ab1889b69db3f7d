"""Write golden vectors produced by the reference implementation itself.

Runs ONLY in the build container, where the reference source tree is present
(default ``/root/reference``; override with ``DABSN_REFERENCE_SRC``). It imports the
reference's ``dabsn`` package on the CPU, in its default pure-torch backend, evaluates the
functions listed below on small seeded inputs, and writes inputs, parameters and outputs
(plus autograd gradients) as ``.npz`` files under ``tests/golden/ref/``. Only those data
files are committed; nothing of the reference travels with them.

    TORCH_EXTENSIONS_DIR=/tmp/refext python tests/golden/make_ref_golden.py

Fixtures (reference file:line of the function evaluated):

* ``core_op_fp32`` -- the registered op ``dabsn::core_scan_batched``
  forward (kernels/batched_runtime.py:1507-1560) and its registered autograd, i.e. the
  Python reverse recurrence ``DABSNCoreScanBatched.backward`` (batched_runtime.py:1333-1504),
  from a random carried state with every per-unit term active.
* ``core_op_bf16`` -- the same op with bf16 activations and recurrent weights (the
  reference's own bf16 path, tests/test_batched_runtime.py:83-162) and, on the same
  values, in fp32: outputs and gradients of both, so the reference's bf16-vs-fp32 gap is
  known per gradient.
* ``core_bf16_gap`` -- the reference's bf16-vs-fp32 distance of the same op at B=2 T=256
  H=512 and B=1 T=1024 H=2048, per output and gradient, with seeded sketches of its fp32
  results; the inputs are rebuilt from ``golden_cases.bf16_gap_case``.
* ``core_loop_fp64`` -- ``DABSNCore._reference_forward_from_state`` (core.py:111-246), the
  per-step torch loop, differentiated by autograd.
* ``read_seq_fp32`` -- ``DABSNRead.forward`` in seq geometry (read.py:139-438) on a
  partially admitted bank (admission window shrunk), with the slot order and counts the
  call produced, ``last_n_max`` and the gradients of every tape and parameter.
* ``read_field_fp32``, ``read_hybrid_fp32`` -- the same read in field geometry
  (whole-sequence admission floor, every admitted slot visible to every query,
  read.py:185-191, 283-314, 346-367) and in hybrid geometry (both reads over the
  whole-sequence bank mixed by sigmoid(hybrid_gate), read.py:368-420).
* ``read_seq_bf16`` -- the same read with the module and tapes in bfloat16: the admission
  values, the selection order and counts it made (bf16 tape means, read.py:58-72,
  161-192) and its output.
* ``query_bank_fp32`` -- ``DABSNRead.forward_query_bank`` (read.py:650-838): a query
  chunk read against an external bank with ``query_start > 0`` and a carried long state.
* ``model_c1`` -- a config-1-shaped ``DABSNModel`` (input 24, out 10, seq blocks 128/96
  and 192/128, residual, mlp_ratio 4, token head; model.py:572-665) at B=2, T=64: each
  block's input and output, the gradient flowing into each block output, and each
  block's parameter gradients under a random linear loss on the model output.
* ``memory_lm.dmem`` + ``memory_lm.npz`` -- a ``.dmem`` file written by the reference's
  ``memory.save`` after ``ingest`` of a prompt into a small ``DABSNSequenceLM``
  (memory.py:389-470), the LM's state dict, the prompt, and the logits of the next
  ``forward_with_memory`` token.
* ``op_schemas.json`` -- the dispatcher schema of every registered ``dabsn::`` operator
  this build replaces (kernels/batched_runtime.py:1507, compact_flash.py:71 and 182,
  long.py:392 and 410, permanent.py:384, local_field.py:208, admitted.py:16, 384 and 509), as
  ``torch`` prints it: the interface a backend's kernels must accept.

``python tests/golden/make_ref_golden.py NAME ...`` writes only the named fixtures.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
OUT = HERE / "ref"
REF_SRC = Path(os.environ.get("DABSN_REFERENCE_SRC", "/root/reference/src"))


def _np(t):
    import torch

    if t is None:
        return None
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.float().numpy()  # exact: every bf16 value is an fp32 value
    return t.numpy()


def _save(name: str, arrays: dict) -> None:
    arrays = {k: v for k, v in arrays.items() if v is not None}
    OUT.mkdir(parents=True, exist_ok=True)
    np.savez_compressed(OUT / f"{name}.npz", **arrays)
    size = (OUT / f"{name}.npz").stat().st_size
    print(f"wrote {name}.npz ({len(arrays)} arrays, {size / 1024:.1f} KiB)")


VEC_ATTRS = ("beta", "log_kappa", "logit_recover", "k_s", "k_y", "k_b", "k_n", "k_bias",
             "r_s", "r_y", "r_b", "r_n", "r_bias", None, "k_saturation", "r_saturation")


def _perturbed_core(core, gen, scale=0.3):
    """Add noise to every core parameter so each term of the recurrence is active."""
    import torch

    with torch.no_grad():
        for _, p in core.named_parameters():
            p.add_(scale * torch.randn(p.shape, generator=gen, dtype=p.dtype))


def _core_op_inputs(core, B, T, gen, dtype):
    import torch

    H = core.hidden_dim
    Wx = (0.8 * torch.randn(B, T, H, generator=gen)).to(dtype)
    Wgx = (0.8 * torch.randn(B, T, H, generator=gen) + 0.5).to(dtype)
    b0 = (0.5 * torch.randn(B, H, generator=gen)).to(dtype)
    e0 = (0.2 + 0.8 * torch.rand(B, H, generator=gen)).to(dtype)
    c0 = (0.6 * torch.rand(B, H, generator=gen)).to(dtype)
    vecs = [getattr(core, a) if a else core.logit_saturation_decay.expand(H) for a in VEC_ATTRS]
    scal = [core.logit_alpha.reshape(()), core.log_lambda.reshape(()),
            core.logit_saturation_suppress.reshape(())]
    return Wx, Wgx, b0, e0, c0, vecs, scal


def core_op(dtype_name: str) -> None:
    import torch
    from dabsn.core import DABSNCore

    dtype = {"fp32": torch.float32, "fp64": torch.float64}[dtype_name]
    torch.manual_seed(0)
    gen = torch.Generator().manual_seed(11)
    B, T, H = 2, 9, 12
    core = DABSNCore(input_dim=5, hidden_dim=H)
    _perturbed_core(core, gen)
    core = core.to(dtype)
    Wx, Wgx, b0, e0, c0, vecs, scal = _core_op_inputs(core, B, T, gen, dtype)
    leaves = [Wx, Wgx, core.Ug.weight, core.A.weight, *vecs, *scal, b0, e0, c0]
    leaves = [x.detach().clone().requires_grad_(True) for x in leaves]
    outs = torch.ops.dabsn.core_scan_batched(*leaves)
    grads_out = [torch.randn(o.shape, generator=gen, dtype=dtype) for o in outs]
    loss = sum((o * g).sum() for i, (o, g) in enumerate(zip(outs, grads_out)) if i != 7)
    grads = torch.autograd.grad(loss, leaves, allow_unused=True)
    arrays = {f"in{i}": _np(x) for i, x in enumerate(leaves)}
    arrays.update({f"out{i}": _np(o) for i, o in enumerate(outs)})
    arrays.update({f"gout{i}": _np(g) for i, g in enumerate(grads_out) if i != 7})
    arrays.update({f"grad{i}": _np(g) for i, g in enumerate(grads) if g is not None})
    _save(f"core_op_{dtype_name}", arrays)


def core_op_bf16() -> None:
    """The registered core op with the reference's bf16 activations (Wx, Wgx, Ug, A in
    bf16, as tests/test_batched_runtime.py:83-113 drives it; fp32 state and vectors), and
    the same op on the same values in fp32: how far the reference's own bf16 path lands
    from fp32."""
    import torch
    from dabsn.core import DABSNCore

    os.environ["DABSN_BATCHED_STEP_COMPILE"] = "0"
    torch.manual_seed(0)
    gen = torch.Generator().manual_seed(13)
    B, T, H = 4, 48, 32
    core = DABSNCore(input_dim=5, hidden_dim=H)
    _perturbed_core(core, gen)
    Wx, Wgx, b0, e0, c0, vecs, scal = _core_op_inputs(core, B, T, gen, torch.float32)
    bf = torch.bfloat16
    base = [Wx.to(bf), Wgx.to(bf), core.Ug.weight.to(bf), core.A.weight.to(bf), *vecs, *scal,
            b0, e0, c0]
    leaves16 = [x.detach().clone().requires_grad_(True) for x in base]
    leaves32 = [x.detach().float().clone().requires_grad_(True) for x in base]
    outs16 = torch.ops.dabsn.core_scan_batched(*leaves16)
    outs32 = torch.ops.dabsn.core_scan_batched(*leaves32)
    gout = [torch.randn(o.shape, generator=gen) for o in outs32]

    def loss(outs):
        return sum((o.float() * g).sum() for i, (o, g) in enumerate(zip(outs, gout)) if i != 7)

    g16 = torch.autograd.grad(loss(outs16), leaves16, allow_unused=True)
    g32 = torch.autograd.grad(loss(outs32), leaves32, allow_unused=True)
    arrays = {f"in{i}": _np(x) for i, x in enumerate(leaves32)}
    arrays.update({f"out16_{i}": _np(o) for i, o in enumerate(outs16)})
    arrays.update({f"out32_{i}": _np(o) for i, o in enumerate(outs32)})
    arrays.update({f"gout{i}": _np(g) for i, g in enumerate(gout) if i != 7})
    arrays.update({f"grad16_{i}": _np(g) for i, g in enumerate(g16) if g is not None})
    arrays.update({f"grad32_{i}": _np(g) for i, g in enumerate(g32) if g is not None})
    _save("core_op_bf16", arrays)


def core_bf16_gap() -> None:
    """The reference's own bf16-vs-fp32 distance of dabsn::core_scan_batched at two larger
    shapes (B=2 T=256 H=512 and B=1 T=1024 H=2048), per output (normwise max) and per
    gradient (Frobenius): the bf16 run casts Wx, Wgx, Ug and A (tests/test_batched_runtime.py
    :83-113), the fp32 run takes the same values in fp32. Inputs and upstream gradients come
    from the seeded recipe ``golden_cases.bf16_gap_case`` (no large tensor is stored);
    the fp32 outputs and gradients are kept as seeded sketches and norms, which pin the CPU
    oracle to the reference's fp32 run at these shapes."""
    import torch

    import dabsn.kernels.batched_runtime  # noqa: F401  (registers dabsn::core_scan_batched)

    sys.path.insert(0, str(HERE.parent))
    import golden_cases as gc

    os.environ["DABSN_BATCHED_STEP_COMPILE"] = "0"
    arrays = {}
    for name in gc.BF16_GAP_SHAPES:
        inputs, gout = gc.bf16_gap_case(name)
        leaves16 = [(x.to(torch.bfloat16) if i < 4 else x).clone().requires_grad_(True)
                    for i, x in enumerate(inputs)]
        leaves32 = [x.clone().requires_grad_(True) for x in inputs]
        outs16 = torch.ops.dabsn.core_scan_batched(*leaves16)
        outs32 = torch.ops.dabsn.core_scan_batched(*leaves32)

        def loss(outs):
            return sum((o.float() * g).sum() for o, g in zip(outs, gout) if g is not None)

        g16 = torch.autograd.grad(loss(outs16), leaves16, allow_unused=True)
        g32 = torch.autograd.grad(loss(outs32), leaves32, allow_unused=True)
        arrays[f"{name}.checksum_in"] = np.array([float(x.double().sum()) for x in inputs])
        for i, (a, b) in enumerate(zip(outs16, outs32)):
            a64, b64 = _np(a).astype(np.float64), _np(b).astype(np.float64)
            arrays[f"{name}.gap_out{i}"] = np.array(
                np.abs(a64 - b64).max() / max(np.abs(b64).max(), 1e-30))
            arrays[f"{name}.sketch_out{i}"] = gc.sketch(b64, 1000 + i)
            arrays[f"{name}.norm_out{i}"] = np.array(np.linalg.norm(b64))
        for i, (a, b) in enumerate(zip(g16, g32)):
            if b is None:
                continue
            a64, b64 = _np(a).astype(np.float64), _np(b).astype(np.float64)
            arrays[f"{name}.gap_grad{i}"] = np.array(
                np.linalg.norm(a64 - b64) / max(np.linalg.norm(b64), 1e-30))
            arrays[f"{name}.sketch_grad{i}"] = gc.sketch(b64, 2000 + i)
            arrays[f"{name}.sketch16_grad{i}"] = gc.sketch(a64, 2000 + i)
            arrays[f"{name}.norm_grad{i}"] = np.array(np.linalg.norm(b64))
            if b64.size == 1:
                arrays[f"{name}.val16_grad{i}"] = a64.reshape(())
                arrays[f"{name}.val32_grad{i}"] = b64.reshape(())
        worst = max((float(arrays[k]), k) for k in arrays if k.startswith(f"{name}.gap_grad"))
        print(f"  {name}: worst reference bf16 gradient gap {worst[0]:.3e} ({worst[1]})")
    # The end-to-end bf16 cases of tests/test_gpu_ops.py: inputs helpers.core_case(200 + H,
    # B, T, H) with Wx, Wgx, Ug, A cast to bf16 for the bf16 run and unrounded for the fp32
    # run, upstream gradients seeded 9 and rounded to bf16 values for both.
    sys.path.insert(0, str(HERE.parent.parent))
    from helpers import core_case

    for B, T, H in gc.OPS_BF16_CASES:
        name = f"ops_B{B}_T{T}_H{H}"
        inputs = core_case(200 + H, B, T, H)
        g = torch.Generator().manual_seed(9)
        shapes = [(B, T, 2 * H)] + [(B, T, H)] * 7 + [(B, H)] * 3
        ups = [torch.randn(sh, generator=g).to(torch.bfloat16).float() for sh in shapes]
        leaves16 = [(x.to(torch.bfloat16) if i < 4 else x).clone().requires_grad_(True)
                    for i, x in enumerate(inputs)]
        leaves32 = [x.clone().requires_grad_(True) for x in inputs]
        outs16 = torch.ops.dabsn.core_scan_batched(*leaves16)
        outs32 = torch.ops.dabsn.core_scan_batched(*leaves32)

        def loss2(outs):
            return sum((o.float() * u).sum() for i, (o, u) in enumerate(zip(outs, ups)) if i != 7)

        g16 = torch.autograd.grad(loss2(outs16), leaves16, allow_unused=True)
        g32 = torch.autograd.grad(loss2(outs32), leaves32, allow_unused=True)
        for i, (a, b) in enumerate(zip(g16, g32)):
            if b is None:
                continue
            a64, b64 = _np(a).astype(np.float64), _np(b).astype(np.float64)
            arrays[f"{name}.gap_grad{i}"] = np.array(
                np.linalg.norm(a64 - b64) / max(np.linalg.norm(b64), 1e-30))
            arrays[f"{name}.sketch16_grad{i}"] = gc.sketch(a64, 2000 + i)
            arrays[f"{name}.sketch_grad{i}"] = gc.sketch(b64, 2000 + i)
            if b64.size == 1:
                arrays[f"{name}.val16_grad{i}"] = a64.reshape(())
                arrays[f"{name}.val32_grad{i}"] = b64.reshape(())
        worst = max((float(arrays[k]), k) for k in arrays if k.startswith(f"{name}.gap_grad"))
        print(f"  {name}: worst reference bf16 gradient gap {worst[0]:.3e} ({worst[1]})")
    _save("core_bf16_gap", arrays)


def core_loop() -> None:
    import torch
    from dabsn.core import DABSNCore

    torch.manual_seed(0)
    gen = torch.Generator().manual_seed(12)
    B, T, D, H = 2, 8, 5, 10
    core = DABSNCore(input_dim=D, hidden_dim=H)
    _perturbed_core(core, gen)
    core = core.double()
    x = torch.randn(B, T, D, generator=gen, dtype=torch.float64).requires_grad_(True)
    b0 = (0.5 * torch.randn(B, H, generator=gen, dtype=torch.float64)).requires_grad_(True)
    e0 = (0.2 + 0.8 * torch.rand(B, H, generator=gen, dtype=torch.float64)).requires_grad_(True)
    c0 = (0.6 * torch.rand(B, H, generator=gen, dtype=torch.float64)).requires_grad_(True)
    result, final = core._reference_forward_from_state(
        x, initial_state=(b0, e0, c0), return_writes=True, return_cocktail=True,
        return_final_state=True)
    outs = list(result) + list(final)
    gouts = [torch.randn(o.shape, generator=gen, dtype=torch.float64) for o in outs]
    loss = sum((o * g).sum() for o, g in zip(outs, gouts))
    names = [n for n, _ in core.named_parameters()]
    params = [p for _, p in core.named_parameters()]
    grads = torch.autograd.grad(loss, [x, b0, e0, c0, *params], allow_unused=True)
    arrays = {"x": _np(x), "b0": _np(b0), "e0": _np(e0), "c0": _np(c0)}
    arrays.update({f"param.{n}": _np(p) for n, p in zip(names, params)})
    arrays.update({f"out{i}": _np(o) for i, o in enumerate(outs)})
    arrays.update({f"gout{i}": _np(g) for i, g in enumerate(gouts)})
    for n, g in zip(["x", "b0", "e0", "c0"] + [f"param.{n}" for n in names], grads):
        if g is not None:
            arrays[f"grad.{n}"] = _np(g)
    _save("core_loop_fp64", arrays)


def _read_tapes(B, T, H, gen, dtype):
    import torch

    y = torch.tanh(torch.randn(B, T, H, generator=gen))
    budget = 0.5 * torch.randn(B, T, H, generator=gen)
    ay = torch.randn(B, T, H, generator=gen)
    nov = torch.rand(B, T, H, generator=gen)
    pl = torch.rand(B, T, H, generator=gen) * torch.rand(B, T, 1, generator=gen)
    w = pl * ay
    en = torch.rand(B, T, H, generator=gen)
    sat = torch.rand(B, T, H, generator=gen) * 0.7
    return [t.to(dtype) for t in (y, budget, ay, w, nov, pl, en, sat)]


TAPE_NAMES = ("y", "budget", "expression", "write", "novelty", "plasticity", "energy",
              "saturation")


class _ArgsortSpy:
    """Records what torch.argsort returns inside one reference call (the slot order)."""

    def __init__(self):
        import torch

        self.torch = torch
        self.calls = []
        self._orig = torch.argsort

    def __enter__(self):
        orig = self._orig

        def spy(*args, **kwargs):
            out = orig(*args, **kwargs)
            self.calls.append(out.detach().clone())
            return out

        self.torch.argsort = spy
        return self

    def __exit__(self, *exc):
        self.torch.argsort = self._orig


def _perturbed_read(read, gen, scale=0.2):
    import torch

    with torch.no_grad():
        for name, p in read.named_parameters():
            if name.startswith("short_read.out"):
                continue
            p.add_(scale * torch.randn(p.shape, generator=gen, dtype=p.dtype))


def read_seq(geometry: str = "seq") -> None:
    import torch
    from dabsn.read import DABSNRead

    torch.manual_seed(0)
    gen = torch.Generator().manual_seed(13)
    B, T, H = 2, 24, 16
    read = DABSNRead(hidden_dim=H, read_geometry=geometry)
    _perturbed_read(read, gen)
    with torch.no_grad():
        read.admit_window.fill_(-1.2)  # softplus = 0.26: a partially admitted bank
    tapes = [t.requires_grad_(True) for t in _read_tapes(B, T, H, gen, torch.float32)]
    with _ArgsortSpy() as spy:
        out = read(*tapes)
    order = spy.calls[-1]
    gout = torch.randn(out.shape, generator=gen)
    names = [n for n, _ in read.named_parameters()]
    params = [p for _, p in read.named_parameters()]
    grads = torch.autograd.grad((out * gout).sum(), [*tapes, *params], allow_unused=True)
    arrays = {n: _np(t) for n, t in zip(TAPE_NAMES, tapes)}
    arrays.update({f"param.{n}": _np(p) for n, p in zip(names, params)})
    arrays.update({"out": _np(out), "gout": _np(gout), "order": order.numpy(),
                   "n_max": np.array(read.last_n_max, dtype=np.int64)})
    for n, g in zip(list(TAPE_NAMES) + [f"param.{n}" for n in names], grads):
        if g is not None:
            arrays[f"grad.{n}"] = _np(g)
    print(f"  read_{geometry}: n_max={read.last_n_max} of T={T}")
    _save(f"read_{geometry}_fp32", arrays)


def read_seq_bf16() -> None:
    import torch
    from dabsn.read import DABSNRead

    torch.manual_seed(0)
    gen = torch.Generator().manual_seed(14)
    B, T, H = 3, 256, 16
    read = DABSNRead(hidden_dim=H, read_geometry="seq")
    _perturbed_read(read, gen)
    with torch.no_grad():
        read.admit_window.fill_(-2.0)
    read = read.to(torch.bfloat16)
    tapes = _read_tapes(B, T, H, gen, torch.bfloat16)
    # The admission values themselves (read.py:58-72), in the module's dtype.
    _, _, _, _, nov, pl, en, sat = tapes
    with torch.no_grad():
        adm = read.short_read.admission(nov, pl, en, sat)
        with _ArgsortSpy() as spy:
            out = read(*tapes)
    order = spy.calls[-1]
    # bf16 values stored as their 16-bit patterns (exact, half the bytes of fp32).
    arrays = {f"{n}_bf16": t.view(torch.int16).numpy() for n, t in zip(TAPE_NAMES, tapes)}
    arrays.update({f"param.{n}_bf16": p.detach().view(torch.int16).numpy()
                   for n, p in read.named_parameters()})
    arrays.update({"admission_bf16": adm.view(torch.int16).numpy(), "order": order.numpy(),
                   "n_max": np.array(read.last_n_max, dtype=np.int64), "out": _np(out)})
    print(f"  read_seq_bf16: n_max={read.last_n_max} of T={T}")
    _save("read_seq_bf16", arrays)


def query_bank() -> None:
    import torch
    from dabsn.read import DABSNRead

    torch.manual_seed(0)
    gen = torch.Generator().manual_seed(15)
    B, T, H, start = 2, 20, 12, 14
    read = DABSNRead(hidden_dim=H, read_geometry="seq")
    _perturbed_read(read, gen)
    with torch.no_grad():
        read.admit_window.fill_(-0.5)
    tapes = _read_tapes(B, T, H, gen, torch.float32)
    y, budget, ay, w, nov, pl, en, sat = tapes
    q = [t[:, start:] for t in tapes]
    long0 = tuple(x for x in (0.3 * torch.randn(B, H, generator=gen),
                              0.3 * torch.randn(B, H, generator=gen),
                              0.5 + 0.5 * torch.rand(B, H, generator=gen)))
    with torch.no_grad(), _ArgsortSpy() as spy:
        out, state = read.forward_query_bank(
            *q, bank_y=y, bank_b=budget, bank_ay=ay, bank_write=w, bank_novelty=nov,
            bank_p=pl, bank_energy=en,
            bank_saturation=sat, query_start=start, initial_long_state=long0,
            return_long_state=True)
    arrays = {n: _np(t) for n, t in zip(TAPE_NAMES, tapes)}
    arrays.update({f"param.{n}": _np(p) for n, p in read.named_parameters()})
    arrays.update({"query_start": np.array(start, dtype=np.int64), "out": _np(out),
                   "order": spy.calls[-1].numpy(),
                   "n_max": np.array(read.last_n_max, dtype=np.int64)})
    arrays.update({f"long0_{i}": _np(x) for i, x in enumerate(long0)})
    arrays.update({f"long1_{i}": _np(x) for i, x in enumerate(state)})
    _save("query_bank_fp32", arrays)


def model_c1() -> None:
    import torch
    from dabsn.model import DABSNLayerSpec, DABSNModel

    torch.manual_seed(0)
    gen = torch.Generator().manual_seed(16)
    model = DABSNModel(24, 10, [DABSNLayerSpec(128, 96, "seq"), DABSNLayerSpec(192, 128, "seq")],
                       output_adapter="token", residual=True, mlp_ratio=4.0)
    with torch.no_grad():
        for blk in model.backbone.blocks:
            _perturbed_core(blk.core, gen, 0.1)
            blk.mlp_fc2.weight.normal_(0.0, 0.02, generator=gen)  # zero-init otherwise
        # Every parameter is rounded to a bf16-representable fp32 value, so the fixture
        # stores it exactly as a 16-bit pattern. The model itself still runs in fp32.
        for p in model.parameters():
            p.copy_(p.to(torch.bfloat16).float())
    B, T = 2, 64
    x = torch.randn(B, T, 24, generator=gen).requires_grad_(True)
    # Block chain as the backbone evaluates it: each block's world view (core, read,
    # state_to_hidden, residual skip; model.py:309-337) then its inline MLP. The fixture
    # keeps each world view's input, output and incoming gradient; the MLP sits outside
    # the scan+read path and its weights are not stored.
    xs, ws = [], []
    h = x
    for blk in model.backbone.blocks:
        if h is not x:
            h.retain_grad()
        xs.append(h)
        w = blk.forward_world(h)
        w.retain_grad()
        ws.append(w)
        h = blk.forward_mlp(w)
    out = model.project_sequence(h)
    ref = model.forward_sequence(x)
    assert torch.equal(out, ref), "block chain differs from DABSNModel.forward_sequence"
    gout = torch.randn(out.shape, generator=gen)
    (out * gout).sum().backward()
    arrays = {"x": _np(x), "grad.x": _np(x.grad)}
    for k, blk in enumerate(model.backbone.blocks):
        arrays[f"b{k}.in"] = _np(xs[k])
        arrays[f"b{k}.out"] = _np(ws[k])
        arrays[f"b{k}.gout"] = _np(ws[k].grad)
        arrays[f"b{k}.n_max"] = np.array(blk.read.last_n_max, dtype=np.int64)
        for n, p in blk.named_parameters():
            if n.startswith("mlp_"):
                continue
            arrays[f"b{k}.param.{n}_bf16"] = p.detach().to(torch.bfloat16).view(torch.int16).numpy()
            if p.grad is not None:
                arrays[f"b{k}.grad.{n}"] = _np(p.grad)
    # d loss / d (input of block 1) is what block 1's world view passes back.
    arrays["b1.grad_in"] = _np(xs[1].grad) if xs[1].grad is not None else None
    _save("model_c1", arrays)


def memory_lm() -> None:
    import torch
    from dabsn import memory as ref_memory
    from dabsn.model import DABSNSequenceLM

    torch.manual_seed(0)
    gen = torch.Generator().manual_seed(17)
    model = DABSNSequenceLM(vocab=40, hidden_dim=24, depth=2, layers="seq:24:24,seq:32:16",
                            residual=True, mlp_ratio=2.0).eval()
    with torch.no_grad():
        for blk in model.backbone.blocks:
            blk.mlp_fc2.weight.normal_(0.0, 0.02, generator=gen)
    prompt = torch.randint(0, 40, (2, 13), generator=gen)
    nxt = torch.randint(0, 40, (2, 1), generator=gen)
    with torch.no_grad():
        mem = ref_memory.ingest(model, prompt, chunk_size=5)
        ref_memory.save(mem, OUT / "memory_lm.dmem")
        logits, _ = ref_memory.forward_with_memory(model, nxt, mem)
    arrays = {f"param.{n}": _np(p) for n, p in model.state_dict().items()}
    arrays.update({"prompt": prompt.numpy(), "next": nxt.numpy(), "logits": _np(logits),
                   "position": np.array(mem.position, dtype=np.int64)})
    _save("memory_lm", arrays)
    print(f"  fingerprint: {mem.fingerprint}")


SCHEMA_OPS = ("core_scan_batched", "admitted_three_way_read_compact_flash",
              "_admitted_three_way_read_compact_flash_backward", "linear_recurrence",
              "_linrec_backward", "permanent_delta_scan", "local_field_gather",
              "admitted_three_way_read_native", "_admitted_three_way_read_backward",
              "admitted_three_way_read")


def op_schemas() -> None:
    import json

    import torch

    import dabsn.kernels.admitted  # noqa: F401  (each import registers its operators)
    import dabsn.kernels.batched_runtime  # noqa: F401
    import dabsn.kernels.compact_flash  # noqa: F401
    import dabsn.kernels.local_field  # noqa: F401
    import dabsn.kernels.long  # noqa: F401
    import dabsn.kernels.permanent  # noqa: F401

    schemas = {name: str(getattr(torch.ops.dabsn, name).default._schema) for name in SCHEMA_OPS}
    OUT.mkdir(parents=True, exist_ok=True)
    (OUT / "op_schemas.json").write_text(json.dumps(schemas, indent=1) + "\n")
    print(f"wrote op_schemas.json ({len(schemas)} operators)")


FIXTURES = {"core_op": lambda: core_op("fp32"), "core_op_bf16": core_op_bf16,
            "core_bf16_gap": core_bf16_gap,
            "core_loop": core_loop, "read_seq": read_seq,
            "read_field": lambda: read_seq("field"), "read_hybrid": lambda: read_seq("hybrid"),
            "read_seq_bf16": read_seq_bf16, "query_bank": query_bank, "model_c1": model_c1,
            "memory_lm": memory_lm, "op_schemas": op_schemas}


def main() -> None:
    if not REF_SRC.exists():
        raise SystemExit(f"reference source not found at {REF_SRC}")
    os.environ.setdefault("TORCH_EXTENSIONS_DIR", "/tmp/dabsn_ref_ext")
    sys.path.insert(0, str(REF_SRC))
    import torch

    torch.set_num_threads(min(8, os.cpu_count() or 1))
    for name in sys.argv[1:] or list(FIXTURES):
        FIXTURES[name]()


if __name__ == "__main__":
    main()
