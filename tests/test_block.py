"""Block-level behaviour of the seq DABSN block built on the dabsn:: operators.

CPU variants run the block through the test-only oracle backend (oracle/torch_backend.py
registers the C oracle as the ops' CPU kernels); GPU variants run the HIP kernels and are
compared with the CPU oracle evaluation of the same module.

  * block time-chunking with carried state equals the full scan (reference
    tests/test_block_chunking.py:20-51): forward to fp32 rounding, grads to 1e-5;
  * forward_query_bank on a query chunk against the full bank equals the unified read
    for those rows (reference tests/test_read_chunking.py:23-109): 1e-5; on the GPU the
    chunk read runs on the device and the unified read is the CPU oracle run;
  * config 1 (two seq layers 128/96 and 192/128, input 24, residual, MLP 4.0, fp32)
    forward+backward on GPU against the CPU oracle: normwise 1e-5 for every output and
    parameter gradient (several fp32 ops in sequence, each within 1e-5).
"""

from __future__ import annotations

import copy

import pytest
import torch

import dabsn_amd
from helpers import rel_err
from oracle import torch_backend


@pytest.fixture(scope="module", autouse=True)
def _oracle_cpu_kernels():
    torch_backend.register()


def _block(seed, din, hidden, state, chunk=None):
    torch.manual_seed(seed)
    blk = dabsn_amd.DABSNBlock(din, hidden, state, "seq", residual=True, mlp_ratio=2.0,
                               block_chunk_t=chunk)
    blk.read.admit_window.data.fill_(0.3)  # a partially admitted bank
    return blk


def _fwd_bwd(block, x, w):
    x = x.clone().requires_grad_(True)
    out = block(x)
    (out * w).sum().backward()
    grads = {n: p.grad.detach().clone() for n, p in block.named_parameters() if p.grad is not None}
    return out.detach(), x.grad.detach(), grads


def _check_same(a, b, tol):
    """Outputs and input gradients relative to their own size; parameter gradients relative
    to max(|grad|, 1e-3 x the largest parameter gradient): null_bias and adm_bias shift every
    logit of a softmax equally, so their exact gradient is zero and both runs hold rounding
    noise."""
    out_a, gx_a, g_a = a
    out_b, gx_b, g_b = b
    assert rel_err(out_a.cpu(), out_b.cpu()) <= tol
    assert rel_err(gx_a.cpu(), gx_b.cpu()) <= tol
    assert g_a.keys() == g_b.keys()
    floor = 1e-3 * max(float(g.abs().max()) for g in g_b.values())
    for n in g_a:
        d = float((g_a[n].cpu() - g_b[n].cpu()).abs().max())
        err = d / max(float(g_b[n].abs().max()), floor)
        assert err <= tol, f"{n}: {err:.3e}"


def _chunk_case(device):
    full = _block(1, 16, 24, 24).to(device)
    chunked = copy.deepcopy(full)
    chunked.block_chunk_t = 7
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 30, 16, generator=g).to(device)
    w = torch.randn(2, 30, 24, generator=g).to(device)
    return _fwd_bwd(full, x, w), _fwd_bwd(chunked, x, w)


def test_block_chunking_equals_full_cpu():
    a, b = _chunk_case("cpu")
    _check_same(a, b, 1e-5)


@pytest.mark.gpu
def test_block_chunking_equals_full_gpu(cuda_device):
    a, b = _chunk_case(cuda_device)
    _check_same(a, b, 1e-5)


def _query_bank_case(device):
    """The unified read of the full sequence on the CPU oracle, and on ``device`` the query
    chunk [25, 40) read against the whole bank with the long state carried to 25."""
    torch.manual_seed(3)
    blk = _block(3, 16, 24, 24)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 40, 16, generator=g)
    with torch.no_grad():
        traj, nov, p, ay, wr, en, sat = blk.core_tapes(x)
        y, b = traj.split(24, dim=-1)
        full = blk.read(y, b, ay, wr, nov, p, en, sat)
        dev = copy.deepcopy(blk).to(device)
        y, b, ay, wr, nov, p, en, sat = (t.to(device) for t in (y, b, ay, wr, nov, p, en, sat))
        t0 = 25
        _, long_state = dev.read._long_scan_from_state(wr[:, :t0], p[:, :t0], nov[:, :t0],
                                                        return_final_state=True)
        sl = slice(t0, None)
        part = dev.read.forward_query_bank(
            y[:, sl], b[:, sl], ay[:, sl], wr[:, sl], nov[:, sl], p[:, sl], en[:, sl], sat[:, sl],
            bank_write=wr, bank_novelty=nov, bank_p=p, bank_energy=en, bank_saturation=sat,
            query_start=t0, initial_long_state=long_state)
    return full[:, t0:], part.cpu()


def test_forward_query_bank_matches_unified_read_cpu():
    full, part = _query_bank_case("cpu")
    assert rel_err(part, full) <= 1e-5


@pytest.mark.gpu
def test_forward_query_bank_matches_oracle_unified_read_gpu(cuda_device):
    full, part = _query_bank_case(cuda_device)
    assert rel_err(part, full) <= 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("geometry", ["field", "hybrid"])
def test_field_and_hybrid_read_gpu_match_cpu_oracle(cuda_device, geometry):
    """The field and hybrid reads at T=300 (several 256-row tiles, a partially admitted
    whole-sequence bank) on the GPU against the same module on the CPU oracle kernels:
    output, tape gradients and the output projection's gradients 1e-5 normwise. A scalar
    gain's gradient sums O(T * N) signed terms that partly cancel (here every query reads
    every admitted slot): |diff| <= 1e-5 x the largest scalar gradient of the module."""
    torch.manual_seed(3)
    B, T, H = 2, 300, 64
    read = dabsn_amd.DABSNRead(H, read_geometry=geometry)
    with torch.no_grad():
        read.admit_window.fill_(-2.0)  # about 45 of 300 positions admitted
        if geometry == "hybrid":
            read.hybrid_gate.fill_(0.4)
    g = torch.Generator().manual_seed(4)
    tapes = [torch.randn(B, T, H, generator=g) for _ in range(3)]
    tapes += [torch.rand(B, T, H, generator=g) for _ in range(5)]
    tapes[3] = tapes[5] * tapes[2]  # write = plasticity * expression
    gout = torch.randn(B, T, H, generator=g)

    def run(module, device):
        xs = [t.to(device).requires_grad_(True) for t in tapes]
        out = module(*xs)
        grads = torch.autograd.grad((out * gout.to(device)).sum(), [*xs, *module.parameters()],
                                    allow_unused=True)
        return out.detach().cpu(), [None if x is None else x.cpu() for x in grads], module.last_n_max

    out_c, g_c, n_c = run(read, "cpu")
    out_g, g_g, n_g = run(copy.deepcopy(read).to(cuda_device), cuda_device)
    assert n_c == n_g and 1 < n_c < T
    assert rel_err(out_g, out_c) <= 1e-5
    scalar = [b for b in g_c[8:] if b is not None and b.numel() == 1]
    s_max = max(float(b.abs()) for b in scalar)
    worst = 0.0
    for i, (a, b) in enumerate(zip(g_g, g_c)):
        if b is None:
            continue
        if b.numel() == 1:
            worst = max(worst, float((a - b).abs()) / s_max)
            assert float((a - b).abs()) <= 1e-5 * s_max, f"grad {i}: {float(a)} vs {float(b)}"
        else:
            assert rel_err(a, b) <= 1e-5, f"grad {i}: {rel_err(a, b):.3e}"
    print(f"{geometry} read: worst scalar gradient difference {worst:.2e} of the largest")


@pytest.mark.gpu
def test_config1_two_layer_model_gpu_matches_cpu_oracle(cuda_device):
    """input 24, layers (hidden 128, state 96) and (192, 128)."""
    torch.manual_seed(0)
    layers = torch.nn.Sequential(
        dabsn_amd.DABSNBlock(24, 128, 96, "seq", residual=True, mlp_ratio=4.0),
        dabsn_amd.DABSNBlock(128, 192, 128, "seq", residual=True, mlp_ratio=4.0),
        torch.nn.Linear(192, 10))
    gpu = copy.deepcopy(layers).to(cuda_device)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(8, 256, 24, generator=g)
    target = torch.randint(0, 10, (8, 256), generator=g)

    def run(model, xx, tt):
        xx = xx.clone().requires_grad_(True)
        logits = model(xx)
        loss = torch.nn.functional.cross_entropy(logits.reshape(-1, 10), tt.reshape(-1))
        loss.backward()
        return loss.detach(), {n: p.grad.detach().clone() for n, p in model.named_parameters()
                               if p.grad is not None}

    loss_c, grads_c = run(layers, x, target)
    loss_g, grads_g = run(gpu, x.to(cuda_device), target.to(cuda_device))
    assert abs(float(loss_g) - float(loss_c)) <= 1e-5 * abs(float(loss_c))
    assert grads_c.keys() == grads_g.keys()
    # Some parameters have an exactly zero gradient in exact arithmetic (null_bias shifts
    # every logit of a softmax equally), so both sides hold rounding noise there; the
    # normwise denominator is floored at 1e-3 of the largest gradient in the model.
    floor = 1e-3 * max(float(g.abs().max()) for g in grads_c.values())
    worst = 0.0
    for n in grads_c:
        a, e = grads_g[n].cpu().double(), grads_c[n].double()
        err = float((a - e).abs().max()) / max(float(e.abs().max()), floor)
        worst = max(worst, err)
        assert err <= 1e-5, f"{n}: {err:.3e} (max|grad| {float(e.abs().max()):.3e})"
    print(f"config-1 model vs oracle: worst parameter gradient error {worst:.2e}")
