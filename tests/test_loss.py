"""Chunked readout + cross-entropy (dabsn_amd.loss) against F.cross_entropy.

Mirrors the reference's tests/test_loss_chunking.py cases (forward, gradients for several
chunk budgets, ignore_index, the single-chunk path, the from-logits variant, the ``off``
switch) on this package's device path: the row kernels run as HIP on the GPU, and on the
CPU through the test-only oracle kernels, which checks the chunking, masking and gradient
assembly of loss.py itself. fp32 throughout (the HIP kernels take fp32/bf16): loss relative
1e-5 and gradients normwise 1e-5 against fp64 torch on the same fp32 values; bf16 logits
relative 1e-2 against the fp32 loss of the same bf16 hidden/weight.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from dabsn_amd import loss as L
from helpers import rel_err
from oracle import torch_backend


@pytest.fixture(scope="module", autouse=True)
def _oracle_cpu_kernels():
    torch_backend.register()


def _case(seed, B, T, H, V, bias=True, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    hidden = torch.randn(B, T, H, generator=g).to(dtype)
    weight = (torch.randn(V, H, generator=g) / H ** 0.5).to(dtype)
    b = torch.randn(V, generator=g).to(dtype) if bias else None
    targets = torch.randint(0, V, (B, T), generator=g)
    return hidden, weight, b, targets


def _naive(hidden, weight, bias, targets, ignore_index=-100):
    """fp64 F.linear + F.cross_entropy on the same values, with gradients."""
    leaves = [None if x is None else x.detach().double().requires_grad_(True)
              for x in (hidden, weight, bias)]
    logits = F.linear(leaves[0], leaves[1], leaves[2])
    loss = F.cross_entropy(logits.reshape(-1, logits.shape[-1]), targets.reshape(-1),
                           ignore_index=ignore_index)
    loss.backward()
    return loss.detach(), [None if x is None else x.grad for x in leaves]


def _run(hidden, weight, bias, targets, device, **kw):
    leaves = [None if x is None else x.detach().to(device).requires_grad_(True)
              for x in (hidden, weight, bias)]
    loss = L.chunked_linear_cross_entropy(leaves[0], leaves[1], leaves[2], targets.to(device), **kw)
    loss.backward()
    return loss.detach().cpu(), [None if x is None else x.grad.cpu() for x in leaves]


def _check(got, want, tol=1e-5):
    loss, grads = got
    ref_loss, ref_grads = want
    assert abs(float(loss) - float(ref_loss)) <= tol * abs(float(ref_loss))
    for a, b in zip(grads, ref_grads):
        assert (a is None) == (b is None)
        if a is not None:
            assert rel_err(a, b) <= tol


DEVICES = ["cpu", pytest.param("cuda", marks=pytest.mark.gpu)]


@pytest.mark.parametrize("device", DEVICES)
@pytest.mark.parametrize("budget", [1, 7 * 50, 10_000])
def test_loss_and_gradients_match_cross_entropy_for_any_chunking(device, budget):
    """reference test_loss_chunking.py:45-65 (budgets 1 row, 7 rows, everything)."""
    h, w, b, t = _case(1, 3, 5, 7, 50)
    _check(_run(h, w, b, t, device, chunk_budget=budget), _naive(h, w, b, t))


@pytest.mark.parametrize("device", DEVICES)
def test_ignore_index_masks_positions(device):
    """reference test_loss_chunking.py:68-89."""
    h, w, b, t = _case(2, 2, 8, 6, 30)
    t[:, ::2] = -100
    _check(_run(h, w, b, t, device, chunk_budget=1, ignore_index=-100),
           _naive(h, w, b, t, ignore_index=-100))


@pytest.mark.parametrize("device", DEVICES)
def test_no_bias_and_single_chunk(device):
    h, w, _, t = _case(3, 2, 4, 5, 16, bias=False)
    _check(_run(h, w, None, t, device, chunk_budget=1 << 30), _naive(h, w, None, t))


@pytest.mark.parametrize("device", DEVICES)
def test_from_logits_variant_matches(device):
    """reference test_loss_chunking.py:108-117, with its gradient."""
    g = torch.Generator().manual_seed(4)
    logits = torch.randn(37, 60, generator=g)
    t = torch.randint(0, 60, (37,), generator=g)
    x = logits.detach().to(device).clone().requires_grad_(True)
    got = L.chunked_cross_entropy_from_logits(x, t.to(device), chunk_budget=1)
    got.backward()
    xl = logits.detach().double().requires_grad_(True)
    ref = F.cross_entropy(xl, t)
    ref.backward()
    assert abs(float(got.detach()) - float(ref.detach())) <= 1e-5 * float(ref.detach())
    assert rel_err(x.grad.cpu(), xl.grad) <= 1e-5


def test_off_switch_uses_full_cross_entropy(monkeypatch):
    """reference test_loss_chunking.py:120-131."""
    monkeypatch.setenv("DABSN_LOSS_CHUNK_SCORES", "off")
    h, w, b, t = _case(5, 2, 6, 8, 40)
    got = L.chunked_linear_cross_entropy(h, w, b, t)
    assert abs(float(got) - float(_naive(h, w, b, t)[0])) <= 1e-5 * float(got)


@pytest.mark.gpu
def test_readout_size_loss_on_device_bf16(cuda_device):
    """Vocabulary 32000 at bf16 with several chunks: against the fp32 loss and gradients of
    the same bf16 hidden and weight."""
    h, w, b, t = _case(6, 2, 512, 256, 32000, dtype=torch.bfloat16)
    leaves = [x.to(cuda_device).requires_grad_(True) for x in (h, w, b)]
    loss = L.chunked_linear_cross_entropy(*leaves, t.to(cuda_device), chunk_budget=1 << 22)
    loss.backward()
    ref = [x.float().to(cuda_device).requires_grad_(True) for x in (h, w, b)]
    want = F.cross_entropy(F.linear(*ref).reshape(-1, 32000), t.to(cuda_device).reshape(-1))
    want.backward()
    assert loss.dtype == torch.float32
    assert abs(float(loss.detach()) - float(want.detach())) <= 1e-2 * float(want.detach())
    for a, r in zip(leaves, ref):
        assert rel_err(a.grad.float().cpu(), r.grad.cpu()) <= 2e-2


@pytest.mark.gpu
def test_out_of_range_target_is_reported(cuda_device):
    x = torch.randn(3, 10, device=cuda_device)
    with pytest.raises(RuntimeError, match="outside"):
        L.chunked_cross_entropy_from_logits(x, torch.tensor([1, 10, 2], device=cuda_device))
