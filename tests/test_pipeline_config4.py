"""The benchmarked path -- the pipelined scan + read (dabsn_amd/kernels/pipeline.py) on
bench.py's exact config-4 workload -- against the CPU oracle.

Workload: ``bench.build_workload`` (B=16, T=4096, state 2048, input width 4096, chunk 1024,
bf16 autocast over fp32 parameters, the initialised read whose bank admits every position).
Checks:
  * trajectory: y and budget bit-identical to ``chunked_core_scan`` on the same inputs, whose
    windows are checked against the oracle here too (2e-2, the bf16 bar);
  * read output: query windows inside every chunk and across each chunk boundary and each
    boundary of the pipeline's own windows (``pipeline.windows``), rows 0 and 15, against the oracle's composition on the same tapes -- the product's statistics,
    selection and gather checked against the oracle (1e-5, bit-exact, bit-exact), the
    oracle's three-way read of the window, the oracle's long channel of the row, and the
    output projection in fp64: 2e-2 normwise;
  * backward of one window: upstream gradients on steps [t0, t1) of one batch row only,
    through the pipeline at full size, against the oracle on the GPU's own bf16 tapes of
    that row over [0, t1): the read module on the CPU oracle's kernels (bf16 tapes, means
    and projection under bf16 autocast, as the pipeline), then the oracle's reverse scan
    of the row with the read's tape gradients. Causality makes the row's first t1 steps the
    same problem: the admission floor (a prefix maximum), the bank, the long channel and
    the scan are causal, and the bank admits every position of the window (asserted).
    Every gradient the window reaches -- its Wx / Wgx rows (exactly zero elsewhere), every
    core and read parameter -- within 2e-2 (Frobenius; scalar gradients relative), on
    window [0, 16) of the 1024-step pipeline and on [56, 72) across a chunk boundary of a
    64-step pipeline;
  * whole tensors: bench.py's random upstream gradients on every position, every gradient
    of the pipeline within 2e-2 (Frobenius) of the sequential run on the same HIP kernels
    (chunked scan, then the whole-sequence read).

Two read parameters shift every score of a softmax row equally (null_bias, adm_bias): their
exact gradient is zero and both runs hold rounding noise of the row sums. They are bounded
by 2e-2 of the largest scalar gradient of the read instead of relative to their own value.
"""

from __future__ import annotations

import copy
import types

import numpy as np
import pytest
import torch

import bench
import config_checks as cc
import oracle
from dabsn_amd import kernels
from dabsn_amd.kernels import ops
from dabsn_amd.kernels.chunked import chunked_core_scan
from helpers import np32, rel_err
from oracle import torch_backend

pytestmark = pytest.mark.gpu

C4 = types.SimpleNamespace(vocab=32000, hidden=4096, state=2048, chunk=1024, batch=16, seq=4096)
TOL = 2e-2
SHIFT_INVARIANT = ("read.short_read.null_bias", "read.short_read.adm_bias")


@pytest.fixture(scope="module", autouse=True)
def _setup(cuda_device):
    kernels.enable("rocm", required=True)
    torch_backend.register()


@pytest.fixture(scope="module")
def c4p(cuda_device):
    model, Wx, Wgx, gy, gr = bench.build_workload(C4, cuda_device, torch.bfloat16, C4.batch,
                                                  C4.seq)
    return {"model": model, "Wx": Wx, "Wgx": Wgx, "gy": gy, "gr": gr}


def _gpu_step(model, Wx, Wgx, gy, gr, *, pipelined=True, chunk=None):
    """Forward + backward of bench's ScanRead under bf16 autocast; returns (y, read output,
    gradients by name)."""
    model.pipelined = pipelined
    saved_chunk = model.chunk
    if chunk is not None:
        model.chunk = chunk
    try:
        model.zero_grad(set_to_none=True)
        Wx.grad = None
        Wgx.grad = None
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y, out = model(Wx, Wgx)
        torch.autograd.backward([y, out], [gy, gr.to(out.dtype)])
    finally:
        model.pipelined = True
        model.chunk = saved_chunk
    grads = {"Wx": Wx.grad, "Wgx": Wgx.grad}
    for prefix, m in (("core", model.core), ("read", model.read)):
        for n, p in m.named_parameters():
            if p.grad is not None:
                grads[f"{prefix}.{n}"] = p.grad.detach().clone()
    torch.cuda.synchronize()
    return y.detach(), out.detach(), grads


@pytest.fixture(scope="module")
def piped(c4p):
    y, out, grads = _gpu_step(c4p["model"], c4p["Wx"], c4p["Wgx"], c4p["gy"], c4p["gr"])
    return {"y": y, "out": out, "grads": grads}


@pytest.fixture(scope="module")
def tapes(c4p):
    """The chunked scan's outputs on the pipeline's inputs (autocast bf16, as the bench)."""
    model = c4p["model"]
    B, H = C4.batch, C4.state
    z = torch.zeros(B, H, device=c4p["Wx"].device)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        outs = chunked_core_scan(C4.chunk, c4p["Wx"], c4p["Wgx"], *model.core.scan_inputs(), z,
                                 torch.ones_like(z), z.clone())
    return [o.detach() for o in outs]


def test_pipeline_trajectory_equals_chunked_scan(c4p, piped, tapes):
    H = C4.state
    assert torch.equal(piped["y"], tapes[0][..., :H])
    counts = _dense_counts(c4p, tapes)
    assert int(counts.min()) == C4.seq, "the initialised read admits every position"
    wins = [(1016, 1032), (3064, 3080)] + [(b - 8, b + 8) for _, b in _pipeline_windows()[:-1]]
    worst = cc.check_core_windows(c4p["model"].core, c4p["Wx"].detach(), c4p["Wgx"].detach(),
                                  tapes, rows=(0, 15), windows=wins, tol=TOL)
    print(f"config4 pipeline trajectory: bit-identical; core windows {worst:.2e}")


def _pipeline_windows():
    from dabsn_amd.kernels.pipeline import windows

    w = windows(C4.seq, C4.chunk)
    assert len(w) > C4.seq // C4.chunk, "the pipeline's windows differ from the chunks here"
    return w


def _pieces(c4p, tapes):
    if "P" not in c4p:
        H = C4.state
        o = tapes
        t = (o[0][..., :H], o[0][..., H:], o[3], o[4], o[1], o[2], o[5], o[6])
        with torch.no_grad():
            c4p["P"] = cc.read_pieces(c4p["model"].read, t)
        c4p["T8"] = t
    return c4p["P"], c4p["T8"]


def _dense_counts(c4p, tapes):
    P, _ = _pieces(c4p, tapes)
    return P["bank_valid"].sum(1)


def test_pipeline_read_output_windows_vs_oracle(c4p, piped, tapes):
    """Rows 0 and 15, windows inside each of the four chunks and across each boundary of the
    chunks and of the pipeline's windows."""
    read = c4p["model"].read
    P, t = _pieces(c4p, tapes)
    y, budget, ay, w, nov, pl, en, sat = t
    rows = (0, 15)
    cc.check_stats_rows(P, t, rows=rows)
    cc.check_selection(P, read)
    cc.check_gather(P, w, rows=rows)
    Wo = read.short_read.out.weight.detach().double().cpu().numpy()
    bo = read.short_read.out.bias.detach().double().cpu().numpy()
    gain = float(read.long_gain.detach())
    coef = np.array([float(torch.sigmoid(p.detach())) for p in (
        read.logit_expect_retain, read.logit_retention_decay, read.logit_retain,
        read.logit_retention_strength)], np.float32)
    windows = [(0, 32), (500, 532), (1008, 1040), (1500, 1532), (2032, 2064), (2500, 2532),
               (3056, 3088), (3500, 3532), (4064, 4096)]
    windows += [(b - 16, b + 16) for _, b in _pipeline_windows()[:-1]]
    H = C4.state
    worst = 0.0
    for r in rows:
        z = np.zeros((1, H), np.float32)
        long_row, _ = oracle.long_fwd(np32(w[r:r + 1]), np32(pl[r:r + 1]), coef, z, z,
                                      np.ones((1, H), np.float32))
        for t0, t1 in windows:
            retr = oracle.read3_fwd(*cc._oracle_read_args(P, read, r, t0, t1), query_offset=t0,
                                    total_steps=C4.seq)[0].astype(np.float64)
            x = np.concatenate([np32(y[r, t0:t1]), np32(budget[r, t0:t1]), retr], axis=-1)
            want = x.astype(np.float64) @ Wo.T + bo + gain * long_row[0, t0:t1].astype(np.float64)
            err = rel_err(piped["out"][r, t0:t1], want)
            worst = max(worst, err)
            assert err <= TOL, f"read output row {r}, window [{t0},{t1}): {err:.3e}"
    print(f"config4 pipeline read output windows: worst normwise error {worst:.2e}")


CORE_VECS = ("beta", "log_kappa", "logit_recover", "k_s", "k_y", "k_b", "k_n", "k_bias", "r_s",
             "r_y", "r_b", "r_n", "r_bias", "logit_saturation_decay", "k_saturation",
             "r_saturation")
CORE_SCALARS = ("logit_alpha", "log_lambda", "logit_saturation_suppress")


def _oracle_window_grads(model, tapes, gy, gr, r, t1):
    """Every gradient the window reaches, from the oracle on the GPU's own bf16 tapes of
    row r over [0, t1): the read module on the CPU oracle's kernels under bf16 autocast
    (bf16 tapes, means and projection, as the pipeline and the reference's bf16 read), its
    tape gradients (bf16, as the pipeline keeps them) then through the oracle's reverse
    scan of row r with [Ug; A] at its bf16 values (the scan's recurrent GEMM operand)."""
    H = C4.state
    read = copy.deepcopy(model.read).cpu()
    U = tapes[0][r:r + 1, :t1].cpu().requires_grad_(True)
    ay, w, nov, pl, en, sat = (tapes[k][r:r + 1, :t1].cpu().requires_grad_(True)
                               for k in (3, 4, 1, 2, 5, 6))
    with torch.autocast("cpu", dtype=torch.bfloat16):
        out = read(U[..., :H], U[..., H:], ay, w, nov, pl, en, sat)
    assert read.last_n_max == t1, "the bank admits every position of the window"
    torch.autograd.backward([U[..., :H], out], [gy[r:r + 1, :t1].cpu(),
                                                gr[r:r + 1, :t1].cpu().to(out.dtype)])
    grads = {f"read.{n}": p.grad for n, p in read.named_parameters() if p.grad is not None}
    core = model.core
    GA = np32(torch.cat([core.Ug.weight, core.A.weight], 0).to(torch.bfloat16))
    _, vec, scal = cc.core_params_np(core)
    saved = tuple(np32(tapes[k][r:r + 1, :t1]) for k in (0, 2, 3, 5, 6, 7))
    up = [np32(x.grad if x.grad is not None else torch.zeros_like(x))
          for x in (U, nov, pl, ay, w, en, sat)]
    z = np.zeros((1, H), np.float32)
    gWx, gWgx, gGA, gvec, gscal, _, _, _ = oracle.core_scan_bwd(GA, vec, *scal, z, z, saved,
                                                                up + [None] * 3)
    grads.update({"Wx": torch.from_numpy(gWx), "Wgx": torch.from_numpy(gWgx),
                  "core.Ug.weight": torch.from_numpy(gGA[:H]),
                  "core.A.weight": torch.from_numpy(gGA[H:])})
    for i, n in enumerate(CORE_VECS):
        g = torch.from_numpy(np.asarray(gvec[i], np.float32))
        grads[f"core.{n}"] = g.sum().reshape(1) if n == "logit_saturation_decay" else g
    for i, n in enumerate(CORE_SCALARS):
        grads[f"core.{n}"] = torch.tensor([float(gscal[i])])
    return grads


def _window_upstream(c4p, r, t0, t1, seed):
    g = torch.Generator().manual_seed(seed)
    B, T, H = C4.batch, C4.seq, C4.state
    gy = torch.zeros(B, T, H)
    gr = torch.zeros(B, T, H)
    gy[r, t0:t1] = torch.randn(t1 - t0, H, generator=g) * 1e-3
    gr[r, t0:t1] = torch.randn(t1 - t0, H, generator=g) * 1e-3
    dev = c4p["Wx"].device
    return gy.to(dev, torch.bfloat16), gr.to(dev)


def _check_window_backward(c4p, tapes, r, t0, t1, chunk, seed):
    gy, gr = _window_upstream(c4p, r, t0, t1, seed)
    model = c4p["model"]
    _, _, gpu = _gpu_step(model, c4p["Wx"], c4p["Wgx"], gy, gr, chunk=chunk)
    cpu = _oracle_window_grads(model, tapes, gy, gr, r, t1)
    assert gpu.keys() == cpu.keys(), (sorted(gpu), sorted(cpu))
    for name in ("Wx", "Wgx"):
        g = gpu[name].float()
        outside = torch.ones(g.shape[:2], dtype=torch.bool, device=g.device)
        outside[r, :t1] = False
        assert float(g[outside].abs().max()) == 0.0, f"{name} outside the window's row"
    scalars = [float(cpu[n].abs().max()) for n in cpu if n.startswith("read.") and cpu[n].numel() == 1]
    floor = max(scalars)
    res = {}
    for name, want in cpu.items():
        got = gpu[name].detach().float().cpu()
        if name in ("Wx", "Wgx"):
            got = got[r:r + 1, :t1]
        if name in SHIFT_INVARIANT:
            res[name] = float((got - want).abs().max()) / floor
        elif want.numel() == 1:
            res[name] = abs(float(got) - float(want)) / max(abs(float(want)), 1e-30)
        else:
            res[name] = cc.rel_fro(got, want)
    bad = {n: e for n, e in res.items() if e > TOL}
    worst = max(res.items(), key=lambda kv: kv[1])
    print(f"config4 pipeline backward window [{t0},{t1}) row {r}, chunk {chunk}: "
          f"worst {worst[0]} {worst[1]:.2e}; "
          + ", ".join(f"{n} {e:.1e}" for n, e in sorted(res.items(), key=lambda kv: -kv[1])[:6]))
    assert not bad, f"gradients above {TOL}: {bad}"


def test_pipeline_backward_window_vs_oracle(c4p, tapes):
    _check_window_backward(c4p, tapes, r=3, t0=0, t1=16, chunk=C4.chunk, seed=21)


def test_pipeline_backward_across_chunk_boundary_vs_oracle(c4p, tapes):
    """The same config-4 tensors through a 64-step pipeline (64 chunks, same H = 2048 kernel
    instances), upstream on [56, 72): the window's gradients cross the boundary at 64 through
    the reverse scans of chunks 1 and 0, the read of query chunks 0 and 1 and the long
    channel's window carry."""
    _check_window_backward(c4p, tapes, r=11, t0=56, t1=72, chunk=64, seed=22)


def test_pipeline_gradients_equal_sequential(c4p, piped):
    _, out0, seq = _gpu_step(c4p["model"], c4p["Wx"], c4p["Wgx"], c4p["gy"], c4p["gr"],
                             pipelined=False)
    err_out = cc.rel_fro(piped["out"].cpu(), out0.cpu())
    assert err_out <= TOL, f"read output {err_out:.3e}"
    pip = piped["grads"]
    assert pip.keys() == seq.keys()
    scalars = [float(seq[n].abs().max()) for n in seq if n.startswith("read.") and seq[n].numel() == 1]
    floor = max(scalars)
    res = {}
    for n in seq:
        a, b = pip[n].detach().double().cpu(), seq[n].detach().double().cpu()
        if n in SHIFT_INVARIANT:
            res[n] = float((a - b).abs().max()) / floor
        else:
            res[n] = float((a - b).norm() / max(float(b.norm()), 1e-30))
    bad = {n: e for n, e in res.items() if e > TOL}
    print("config4 pipeline vs sequential: output %.2e; " % err_out
          + ", ".join(f"{n} {e:.1e}" for n, e in sorted(res.items(), key=lambda kv: -kv[1])[:8]))
    assert not bad, f"gradients above {TOL}: {bad}"
