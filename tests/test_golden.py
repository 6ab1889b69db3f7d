"""The CPU oracle against the committed golden fixtures (CPU only).

The fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py) hold fp64
results of the reference math in loop form with autograd gradients; the oracle is fp32,
so tensors must agree to normwise relative 1e-5 and the reductions to scalars (sums of
O(B*T*H) signed terms) to relative 1e-4. Selection order and counts are bit-exact.
"""

from __future__ import annotations

import numpy as np
import pytest

import golden_cases as gc
import oracle
from helpers import rel_err


def _scalar_close(a, b, tol, name):
    a, b = float(a), float(b)
    assert abs(a - b) <= tol * max(abs(b), 1e-6), f"{name}: {a} vs {b}"


@pytest.mark.parametrize("name", gc.CORE)
def test_oracle_core_matches_golden(name):
    d = gc.load(name)
    out, grads = gc.core_oracle(d)
    for i, o in enumerate(out):
        assert rel_err(o, d[f"out{i}"]) <= 1e-5, f"out{i}: {rel_err(o, d[f'out{i}']):.3e}"
    for i, g in enumerate(grads):
        want = d[f"gin{i}"]
        if want.ndim == 0:
            _scalar_close(g, want, 1e-4, f"gin{i}")
        else:
            assert rel_err(g, want) <= 1e-5, f"gin{i}: {rel_err(g, want):.3e}"


@pytest.mark.parametrize("name", gc.READ3)
def test_oracle_read3_matches_golden(name):
    d = gc.load(name)
    out, grads = gc.read3_oracle(d)
    assert rel_err(out, d["out"]) <= 1e-5
    for i, (g, n) in enumerate(zip(grads, gc.READ3_GRAD_NAMES)):
        want = d[f"g{i}"]
        if i >= 8:
            _scalar_close(g, want, 1e-4, n)
        else:
            assert rel_err(g, want) <= 1e-5, f"{n}: {rel_err(g, want):.3e}"


def test_oracle_long_matches_golden():
    d = gc.load(gc.LONG)
    out, fin, grads = gc.long_oracle(d)
    assert rel_err(out, d["out"]) <= 1e-5
    for f, k in zip(fin, ("fL", "fE", "fR")):
        assert rel_err(f, d[k]) <= 1e-5, k
    for g, k in zip(grads, gc.LONG_GRAD_NAMES):
        assert rel_err(g, d[k]) <= (1e-4 if k == "g_logits" else 1e-5), k


def test_oracle_linrec_matches_golden():
    d = gc.load(gc.LINREC)
    y, grads = gc.linrec_oracle(d)
    assert rel_err(y, d["y"]) <= 1e-6
    for g, k in zip(grads, ("da", "dg", "dy0")):
        assert rel_err(g, d[k]) <= 1e-6, k


def test_oracle_selection_matches_golden_bit_exact():
    d = gc.load(gc.SELECT)
    order, counts = oracle.bank_select(d["adm"], float(d["window"]))
    np.testing.assert_array_equal(order, d["order"])
    np.testing.assert_array_equal(counts, d["counts"])


def test_golden_fixtures_hold_only_plain_arrays():
    for p in sorted(gc.GOLDEN.glob("*.npz")):
        with np.load(p, allow_pickle=False) as z:
            for k in z.files:
                assert z[k].dtype.kind in "fiub", f"{p.name}:{k} has dtype {z[k].dtype}"
