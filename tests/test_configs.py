"""Every BASELINE configuration under a GPU test.

Configurations (BASELINE.json ``configs``; test ids carry the config number):

  * config 1 -- the config-1 model: tests/test_block.py (GPU vs the CPU oracle model) and
    tests/test_gpu_ref.py (vectors from the reference itself);
  * config 2 -- copy-task LM, 2 seq layers of state 256, fp32, batch 32:
      - training shape T=64: forward, chunked cross-entropy and backward of the whole LM
        on the GPU against the same LM on the CPU oracle (loss 1e-5, logits and every
        parameter gradient 1e-5);
      - evaluation shape T=3200: layer 0 at full size, piece by piece against the oracle
        (tests/config_checks.py): core windows 1e-5, statistics 1e-5, selection and
        gather bit-exact, read query windows 1e-5, long scan 1e-5;
  * config 3 -- A5 group-tracking LM, 2 seq layers of state 512, fp32, batch 16:
      - training shape T=256: the whole LM against the CPU oracle LM, as config 2;
      - long-evaluation shape T=16384: layer 0 at full size, piece by piece;
  * config 4 -- the benchmark workload (one seq layer, state 2048, input width 4096, bf16
    activations under autocast with fp32 parameters, batch 16, T=4096, block chunking
    1024), piece by piece at full size: the chunked forward equals one unchunked scan bit
    for bit; core windows (including one across a chunk boundary) within the bf16 bar
    2e-2 of the fp32 oracle restarted from the GPU's state; tape statistics 1e-5;
    selection over the whole sequence bit-exact; gather bit-exact; read query windows
    2e-2; the read backward of one query window (Frobenius 2e-2, scalar gradients 2e-2);
    the chunked core backward of windows (one across a chunk boundary) against the
    oracle's reverse scan on the same bf16 tapes (Frobenius 2e-2); the 1024-step chunked
    backward against the unchunked one at full size (5e-3); long scan 1e-2;
  * config 5 -- streaming decode, 4 seq layers of state 2048 with MLPs, bf16, batch 256:
    a prompt ingested in chunks, then token-by-token decode with carried memory, against
    one dense GPU pass over prompt + decoded tokens and against the CPU oracle LM on two
    of the 256 rows (bf16 bar 2e-2).
"""

from __future__ import annotations

import copy
import itertools

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import config_checks as cc
import dabsn_amd
from dabsn_amd import kernels
from dabsn_amd import memory as mem
from dabsn_amd.kernels import ops
from dabsn_amd.kernels.chunked import chunked_core_scan
from dabsn_amd.loss import chunked_linear_cross_entropy
from helpers import grad_err, rel_err
from oracle import torch_backend

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _setup(cuda_device):
    kernels.enable("rocm", required=True)
    torch_backend.register()


# ---------------------------------------------------------------------------
# Task data (configs 2 and 3)
# ---------------------------------------------------------------------------
def copy_task(B, L, seed=1):
    """Vocab 64 + delimiter 64: L random tokens, the delimiter, then L positions whose
    targets are the prefix (inputs are the prefix shifted by one); positions before the
    delimiter are ignored."""
    g = torch.Generator().manual_seed(seed)
    prefix = torch.randint(0, 64, (B, L), generator=g)
    ids = torch.cat([prefix, torch.full((B, 1), 64), prefix[:, :-1]], dim=1)
    targets = torch.cat([torch.full((B, L), -100), prefix], dim=1)
    return ids, targets


def _a5():
    """The 60 even permutations of 5 points, in lexicographic order, and their product
    table (g * h)(i) = g(h(i))."""
    perms = [p for p in itertools.permutations(range(5))
             if sum(p[i] > p[j] for i in range(5) for j in range(i + 1, 5)) % 2 == 0]
    index = {p: k for k, p in enumerate(perms)}
    table = np.array([[index[tuple(g[h[i]] for i in range(5))] for h in perms] for g in perms])
    return table


def a5_task(B, T, seed=2):
    table = _a5()
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, 60, (B, T), generator=g)
    labels = np.empty((B, T), np.int64)
    run = ids[:, 0].numpy().copy()
    labels[:, 0] = run
    for t in range(1, T):
        run = table[ids[:, t].numpy(), run]  # left product: token_t * running
        labels[:, t] = run
    return ids, torch.from_numpy(labels)


def _lm_step(model, ids, targets):
    h = model.forward_hidden(ids)
    loss = chunked_linear_cross_entropy(h, model.readout.weight, model.readout.bias, targets)
    loss.backward()
    return loss.detach(), h.detach()


def lm_against_oracle(model, ids, targets, device, tol=1e-5):
    """The whole LM step on the GPU against the same LM on the CPU oracle kernels."""
    gpu = copy.deepcopy(model).to(device)
    loss_g, h_g = _lm_step(gpu, ids.to(device), targets.to(device))
    loss_c, h_c = _lm_step(model, ids, targets)
    assert abs(float(loss_g) - float(loss_c)) <= 1e-5 * abs(float(loss_c))
    assert rel_err(h_g.cpu(), h_c) <= tol
    grads_c = {n: p.grad for n, p in model.named_parameters() if p.grad is not None}
    scale = max(float(g.abs().max()) for g in grads_c.values())
    worst = 0.0
    for n, p in gpu.named_parameters():
        if n in grads_c:
            err = grad_err(p.grad.cpu(), grads_c[n], scale)
            worst = max(worst, err)
            assert err <= tol, f"{n}: {err:.3e}"
    return worst


def layer0_at_size(model, ids, device, *, rows, core_windows, read_windows, tol):
    """Layer 0 of ``model`` at the full input size, piece by piece against the oracle."""
    blk = model.blocks[0]
    with torch.no_grad():
        x = model.embed(ids.to(device))
        Wx, Wgx = blk.core.W(x), blk.core.Wg(x)
        T = x.shape[1]
        z = torch.zeros(x.shape[0], blk.state_dim, device=device)
        outs = ops.core_scan_batched(Wx, Wgx, *blk.core.scan_inputs(), z, torch.ones_like(z), z)
        for o in outs:
            assert torch.isfinite(o).all()
        cc.check_core_windows(blk.core, Wx, Wgx, outs, rows, core_windows, tol)
        H = blk.state_dim
        y, budget = outs[0][..., :H], outs[0][..., H:]
        tapes = (y, budget, outs[3], outs[4], outs[1], outs[2], outs[5], outs[6])
        P = cc.read_pieces(blk.read, tapes)
        cc.check_stats_rows(P, tapes, rows)
        cc.check_selection(P, blk.read)
        cc.check_gather(P, tapes[3], rows)
        out = ops.admitted_three_way_read_compact_flash(
            *cc._read_args(P, blk.read), 0, *cc.read_gains(blk.read))
        assert torch.isfinite(out).all()
        cc.check_read_windows(P, blk.read, out, rows, [(max(0, T - 32), T), *read_windows], tol)
        long = blk.read._long_scan(tapes[3], tapes[5], tapes[4])
        cc.check_long_rows(blk.read, tapes[3], tapes[5], long, rows, tol)
        return P["bank_n_max"]


# ---------------------------------------------------------------------------
# Config 2: copy task
# ---------------------------------------------------------------------------
def _config2_model():
    torch.manual_seed(0)
    return dabsn_amd.DABSNSequenceLM(65, 256, 2, layers="seq:256:256,seq:256:256")


def test_config2_copy_train_T64_vs_oracle(cuda_device):
    ids, targets = copy_task(32, 32)
    worst = lm_against_oracle(_config2_model(), ids, targets, cuda_device)
    print(f"config2 T=64: worst parameter-gradient error {worst:.2e}")


def test_config2_copy_eval_T3200_layer0_at_size(cuda_device):
    ids, _ = copy_task(32, 1600)
    model = _config2_model().to(cuda_device).eval()
    n_max = layer0_at_size(model, ids, cuda_device, rows=(0, 31),
                           core_windows=[(0, 32), (1584, 1616), (3168, 3200)],
                           read_windows=[(1600, 1632)], tol=1e-5)
    with torch.no_grad():
        logits = model(ids.to(cuda_device))
    assert torch.isfinite(logits).all()
    print(f"config2 T=3200: n_max {n_max}")


# ---------------------------------------------------------------------------
# Config 3: A5 group-state tracking
# ---------------------------------------------------------------------------
def _config3_model():
    torch.manual_seed(0)
    return dabsn_amd.DABSNSequenceLM(60, 512, 2, layers="seq:512:512,seq:512:512")


def test_config3_a5_train_T256_vs_oracle(cuda_device):
    ids, labels = a5_task(16, 256)
    worst = lm_against_oracle(_config3_model(), ids, labels, cuda_device)
    print(f"config3 T=256: worst parameter-gradient error {worst:.2e}")


def test_config3_a5_eval_T16384_layer0_at_size(cuda_device):
    ids, _ = a5_task(16, 16384)
    model = _config3_model().to(cuda_device).eval()
    n_max = layer0_at_size(model, ids, cuda_device, rows=(0, 15),
                           core_windows=[(0, 32), (8176, 8208), (16352, 16384)],
                           read_windows=[(8192, 8224)], tol=1e-5)
    print(f"config3 T=16384: n_max {n_max}")


# ---------------------------------------------------------------------------
# Config 4: the benchmark workload
# ---------------------------------------------------------------------------
C4 = dict(B=16, T=4096, H=2048, D=4096, vocab=32000, chunk=1024)


@pytest.fixture(scope="module")
def c4(cuda_device):
    B, T, H, D = C4["B"], C4["T"], C4["H"], C4["D"]
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, C4["vocab"], (B, T), generator=g)
    torch.manual_seed(0)
    core = dabsn_amd.DABSNCore(D, H).to(cuda_device)
    read = dabsn_amd.DABSNRead(H).to(cuda_device)
    embed = (torch.randn(C4["vocab"], D, generator=g) * 0.02).to(torch.bfloat16)
    x = embed[ids].to(cuda_device)
    with torch.no_grad():
        Wx = F.linear(x, core.W.weight.to(torch.bfloat16))
        Wgx = F.linear(x, core.Wg.weight.to(torch.bfloat16), core.Wg.bias.to(torch.bfloat16))
    del x
    Wx = Wx.requires_grad_(True)
    Wgx = Wgx.requires_grad_(True)
    prm = [p.detach().clone().requires_grad_(True) for p in core.scan_inputs()]
    z = torch.zeros(B, H, device=cuda_device)
    outs = chunked_core_scan(C4["chunk"], Wx, Wgx, *prm, z, torch.ones_like(z), z.clone())
    return {"core": core, "read": read, "Wx": Wx, "Wgx": Wgx, "prm": prm, "outs": outs, "z": z}


def test_config4_chunked_forward_equals_unchunked_scan(c4):
    with torch.no_grad():
        z = c4["z"]
        full = ops.core_scan_batched(c4["Wx"], c4["Wgx"], *c4["prm"], z, torch.ones_like(z), z)
    for k in range(11):
        assert torch.equal(full[k], c4["outs"][k]), f"output {k}"
    e, s = c4["outs"][5].detach(), c4["outs"][7].detach()
    assert float(e.min()) >= 0.0 and float(e.max()) <= 1.0
    assert float(s.min()) >= 0.0 and float(s.max()) <= 1.0
    for o in c4["outs"]:
        assert torch.isfinite(o).all()


def test_config4_core_windows_vs_oracle(c4):
    outs = [o.detach() for o in c4["outs"]]
    worst = cc.check_core_windows(c4["core"], c4["Wx"].detach(), c4["Wgx"].detach(), outs,
                                  rows=(0, 15), windows=[(0, 16), (1016, 1032), (4080, 4096)],
                                  tol=2e-2)
    print(f"config4 core windows: worst normwise error {worst:.2e}")


@pytest.fixture(scope="module")
def c4_read(c4):
    outs = [o.detach() for o in c4["outs"]]
    H = C4["H"]
    tapes = (outs[0][..., :H], outs[0][..., H:], outs[3], outs[4], outs[1], outs[2], outs[5],
             outs[6])
    with torch.no_grad():
        P = cc.read_pieces(c4["read"], tapes)
    return tapes, P


def test_config4_stats_selection_gather_at_size(c4, c4_read):
    tapes, P = c4_read
    cc.check_stats_rows(P, tapes, rows=(0, 15))
    n_max = cc.check_selection(P, c4["read"])
    cc.check_gather(P, tapes[3], rows=(0, 15))
    print(f"config4 n_max {n_max} of T={C4['T']}")


def test_config4_read_windows_vs_oracle(c4, c4_read):
    _, P = c4_read
    read = c4["read"]
    with torch.no_grad():
        out = ops.admitted_three_way_read_train(*cc._read_args(P, read), 0, *cc.read_gains(read))
    assert torch.isfinite(out).all()
    worst = cc.check_read_windows(P, read, out, rows=(0,),
                                  windows=[(0, 32), (2032, 2064), (4064, 4096)], tol=2e-2)
    print(f"config4 read windows: worst normwise error {worst:.2e}")


def test_config4_read_backward_window_vs_oracle(c4, c4_read):
    _, P = c4_read
    worst = cc.check_read_backward_window(P, c4["read"], r=5, t0=4064, t1=4096, tol=2e-2,
                                          scalar_tol=2e-2)
    print(f"config4 read backward window: worst error {worst:.2e}")


def _window_upstream(outs, r, t0, t1, seed):
    g = torch.Generator().manual_seed(seed)
    ups = []
    for k in range(7):
        up = torch.zeros(outs[k].shape, dtype=torch.float32)
        up[r, t0:t1] = torch.randn(t1 - t0, outs[k].shape[-1], generator=g) * 1e-2
        ups.append(up.to(outs[k].device, outs[k].dtype))
    return ups


def test_config4_core_backward_window_vs_oracle(c4):
    """Upstream gradients on row 3, steps [0, 16), through the 1024-step
    chunked backward, against the oracle's reverse scan of row 3 over those steps on the
    same bf16 tapes."""
    outs = c4["outs"]
    r, t0, t1 = 3, 0, 16
    ups = _window_upstream(outs, r, t0, t1, 3)
    leaves = [c4["Wx"], c4["Wgx"], *c4["prm"]]
    grads = torch.autograd.grad(outs[:7], leaves, ups, retain_graph=True)
    worst = cc.check_core_backward_window(c4["core"], c4["Wx"].detach(), c4["Wgx"].detach(),
                                          [o.detach() for o in outs], ups, grads, r, t1, 2e-2)
    print(f"config4 core backward window [0,16): worst error {worst:.2e}")


def test_config4_core_backward_across_chunk_boundary_vs_oracle(c4):
    """The same config-4 tensors scanned in 64-step chunks, so a window across a chunk
    boundary, [56, 72), is reached by a short reverse scan: the backward runs the reverse
    scans of chunks 1 and 0 on the kept tapes, with the same H = 2048 kernel instances as
    the 1024-step schedule.
    The oracle's reverse scan covers [0, 72) of row 3 (the oracle takes ~70 s per 1000
    steps at this width, so a boundary at 1024 is out of a test's reach)."""
    z = c4["z"]
    Wx, Wgx = c4["Wx"], c4["Wgx"]
    outs = chunked_core_scan(64, Wx, Wgx, *c4["prm"], z, torch.ones_like(z), z.clone())
    for k in range(11):
        assert torch.equal(outs[k].detach(), c4["outs"][k].detach()), f"output {k}"
    r, t0, t1 = 3, 56, 72
    ups = _window_upstream(outs, r, t0, t1, 4)
    grads = torch.autograd.grad(outs[:7], [Wx, Wgx, *c4["prm"]], ups)
    worst = cc.check_core_backward_window(c4["core"], Wx.detach(), Wgx.detach(),
                                          [o.detach() for o in outs], ups, grads, r, t1, 2e-2)
    print(f"config4 core backward across a chunk boundary: worst error {worst:.2e}")


def test_config4_chunked_backward_equals_unchunked(c4):
    """Random upstream gradients on every output at full size: the 1024-step chunked
    backward against the unchunked op's backward. They differ
    only by the bf16 rounding of the carried state gradient at the chunk boundaries:
    Frobenius 5e-3."""
    outs = c4["outs"]
    g = torch.Generator().manual_seed(6)
    ups = [(torch.randn(o.shape, generator=g) * 1e-2).to(o.device, o.dtype) for o in outs[:7]]
    leaves = [c4["Wx"], c4["Wgx"], *c4["prm"]]
    chunked = torch.autograd.grad(outs[:7], leaves, ups, retain_graph=True)
    z = c4["z"]
    full = ops.core_scan_batched(*leaves, z, torch.ones_like(z), z)
    unchunked = torch.autograd.grad(full[:7], leaves, ups)
    worst = 0.0
    for i, (a, b) in enumerate(zip(chunked, unchunked)):
        err = cc.rel_fro(a.float().cpu(), b.float().cpu())
        worst = max(worst, err)
        assert err <= 5e-3, f"gradient {i}: {err:.3e}"
    print(f"config4 chunked vs unchunked backward: worst error {worst:.2e}")


def test_config4_long_scan_rows_vs_oracle(c4, c4_read):
    tapes, _ = c4_read
    with torch.no_grad():
        long = c4["read"]._long_scan(tapes[3], tapes[5], tapes[4])
    cc.check_long_rows(c4["read"], tapes[3], tapes[5], long, rows=(0, 15), tol=1e-2)


# ---------------------------------------------------------------------------
# Config 5: streaming decode
# ---------------------------------------------------------------------------
def test_config5_decode_vs_dense_and_oracle(cuda_device):
    B, H, L, prompt, steps = 256, 2048, 4, 48, 6
    torch.manual_seed(0)
    model = dabsn_amd.DABSNSequenceLM(32000, H, L, layers=[(H, H)] * L, residual=True,
                                      mlp_ratio=4.0)
    g = torch.Generator().manual_seed(5)
    with torch.no_grad():
        for blk in model.blocks:
            blk.mlp_fc2.weight.normal_(0.0, 0.02, generator=g)
    model = model.to(torch.bfloat16).eval()
    ids = torch.randint(0, 32000, (B, prompt + steps), generator=g)
    gpu = copy.deepcopy(model).to(cuda_device)
    idg = ids.to(cuda_device)
    with torch.no_grad():
        dense = gpu(idg)[:, prompt:].float()
        memory = mem.ingest(gpu, idg[:, :prompt], chunk_size=16)
        memory.reserve(prompt + steps)
        dec = []
        for t in range(prompt, prompt + steps):
            logits, memory = mem.forward_with_memory(gpu, idg[:, t:t + 1], memory, extend=True)
            dec.append(logits.float())
        dec = torch.cat(dec, dim=1)
    assert memory.position == prompt + steps
    err_dense = rel_err(dec.cpu(), dense.cpu())
    assert err_dense <= 2e-2, f"decode vs dense GPU pass: {err_dense:.3e}"
    rows = [0, B - 1]
    with torch.no_grad():
        want = model(ids[rows])[:, prompt:].float()
    err_oracle = rel_err(dec[rows].cpu(), want)
    assert err_oracle <= 2e-2, f"decode vs CPU oracle: {err_oracle:.3e}"
    print(f"config5 decode: vs dense {err_dense:.2e}, vs oracle {err_oracle:.2e}")


def test_config5_decode_after_long_prompt_vs_oracle(cuda_device):
    """Config-5 widths (H=2048) decoding 32 tokens after a 1,024-token prompt, so each read
    runs against a bank of about a thousand rows: every decode step's logits against the CPU
    oracle's full forward over the same tokens (drift over many steps would show as a
    growing per-step error)."""
    B, H, L, prompt, steps = 2, 2048, 2, 1024, 32
    torch.manual_seed(1)
    model = dabsn_amd.DABSNSequenceLM(32000, H, L, layers=[(H, H)] * L, residual=True,
                                      mlp_ratio=4.0)
    g = torch.Generator().manual_seed(9)
    with torch.no_grad():
        for blk in model.blocks:
            blk.mlp_fc2.weight.normal_(0.0, 0.02, generator=g)
    model = model.to(torch.bfloat16).eval()
    ids = torch.randint(0, 32000, (B, prompt + steps), generator=g)
    gpu = copy.deepcopy(model).to(cuda_device)
    idg = ids.to(cuda_device)
    with torch.no_grad():
        memory = mem.ingest(gpu, idg[:, :prompt], chunk_size=256)
        memory.reserve(prompt + steps)
        dec = []
        for t in range(prompt, prompt + steps):
            logits, memory = mem.forward_with_memory(gpu, idg[:, t:t + 1], memory, extend=True)
            dec.append(logits.float())
        dec = torch.cat(dec, dim=1).cpu()
        want = model(ids)[:, prompt:].float()
    assert memory.position == prompt + steps
    per_step = [rel_err(dec[:, i], want[:, i]) for i in range(steps)]
    worst = max(per_step)
    assert worst <= 2e-2, f"decode step {per_step.index(worst)} vs CPU oracle: {worst:.3e}"
    print(f"config5 long-prompt decode vs oracle: first step {per_step[0]:.2e}, "
          f"last {per_step[-1]:.2e}, worst {worst:.2e}")
