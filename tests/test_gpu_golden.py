"""The HIP operators (fp32) against the committed golden fixtures.

Same bars as the oracle's own golden test: tensors normwise relative 1e-5 against the
fp64 fixture, scalar reductions relative 1e-5, selection bit-exact.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import golden_cases as gc
from helpers import rel_err

pytestmark = pytest.mark.gpu


def _scalar_close(a, b, tol, name):
    a, b = float(a), float(b)
    assert abs(a - b) <= tol * max(abs(b), 1e-6), f"{name}: {a} vs {b}"


@pytest.mark.parametrize("name", gc.CORE)
def test_hip_core_matches_golden(cuda_device, name):
    d = gc.load(name)
    out, grads = gc.core_hip(d, cuda_device)
    for i, o in enumerate(out):
        assert rel_err(o, d[f"out{i}"]) <= 1e-5, f"out{i}: {rel_err(o, d[f'out{i}']):.3e}"
    for i, g in enumerate(grads):
        want = d[f"gin{i}"]
        if want.ndim == 0:
            _scalar_close(g, want, 1e-5, f"gin{i}")
        else:
            assert rel_err(g, want) <= 1e-5, f"gin{i}: {rel_err(g, want):.3e}"


@pytest.mark.parametrize("name", gc.READ3)
def test_hip_read3_matches_golden(cuda_device, name):
    d = gc.load(name)
    out, grads = gc.read3_hip(d, cuda_device)
    assert rel_err(out, d["out"]) <= 1e-5
    for i, (g, n) in enumerate(zip(grads, gc.READ3_GRAD_NAMES)):
        want = d[f"g{i}"]
        if i >= 8:
            _scalar_close(g, want, 1e-5, n)
        else:
            assert rel_err(g, want) <= 1e-5, f"{n}: {rel_err(g, want):.3e}"


def test_hip_long_and_linrec_match_golden(cuda_device):
    d = gc.load(gc.LONG)
    out, fin, grads = gc.long_hip(d, cuda_device)
    assert rel_err(out, d["out"]) <= 1e-5
    for f, k in zip(fin, ("fL", "fE", "fR")):
        assert rel_err(f, d[k]) <= 1e-5, k
    for g, k in zip(grads, gc.LONG_GRAD_NAMES):
        assert rel_err(g, d[k]) <= 1e-5, k
    d = gc.load(gc.LINREC)
    y, grads = gc.linrec_hip(d, cuda_device)
    assert rel_err(y, d["y"]) <= 1e-6
    for g, k in zip(grads, ("da", "dg", "dy0")):
        assert rel_err(g, d[k]) <= 1e-6, k


def test_hip_selection_matches_golden_bit_exact(cuda_device):
    from dabsn_amd.kernels import ops

    d = gc.load(gc.SELECT)
    order, counts, _rank = ops.bank_select(torch.from_numpy(d["adm"]).to(cuda_device),
                                           torch.tensor([float(d["window"])], device=cuda_device))
    np.testing.assert_array_equal(order.cpu().numpy(), d["order"])
    np.testing.assert_array_equal(counts.cpu().numpy(), d["counts"])
