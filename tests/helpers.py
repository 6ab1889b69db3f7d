"""Shared input builders and comparison helpers for the parity tests."""

from __future__ import annotations

import math

import numpy as np
import torch

import oracle


def core_case(seed: int, B: int, T: int, H: int, *, param_scale: float = 0.3, init: bool = True):
    """Random core-op inputs as fp32 CPU tensors (op input order, 26 tensors)."""
    g = torch.Generator().manual_seed(seed)
    Wx = torch.randn(B, T, H, generator=g) * 0.8
    Wgx = torch.randn(B, T, H, generator=g) * 1.5 - 0.5
    Ug = torch.randn(H, H, generator=g) / math.sqrt(H)
    A = torch.randn(H, H, generator=g) * 0.5 / math.sqrt(H)
    vec = []
    for name in oracle.VEC_NAMES:
        base = {"log_kappa": -2.25, "logit_recover": -4.6, "logit_c_decay": 2.2}.get(name, 0.0)
        vec.append(base + param_scale * torch.randn(H, generator=g))
    scal = [torch.tensor(-2.0) + 0.2 * torch.randn((), generator=g),
            torch.tensor(-1.0) + 0.2 * torch.randn((), generator=g),
            torch.tensor(-6.0) + 0.5 * torch.randn((), generator=g)]
    if init:
        b0 = 0.3 * torch.randn(B, H, generator=g)
        e0 = torch.rand(B, H, generator=g) * 0.5 + 0.5
        c0 = torch.rand(B, H, generator=g) * 0.3
    else:
        b0, e0, c0 = torch.zeros(B, H), torch.ones(B, H), torch.zeros(B, H)
    return [Wx, Wgx, Ug, A, *vec, *scal, b0, e0, c0]


def oracle_core_fwd(inputs):
    Wx, Wgx, Ug, A = inputs[:4]
    vec = inputs[4:20]
    la, ll, ls = inputs[20:23]
    b0, e0, c0 = inputs[23:26]
    GA = torch.cat([Ug, A], 0)
    return oracle.core_scan_fwd(np32(Wx), np32(Wgx), np32(GA), [np32(v) for v in vec], float(la),
                                float(ll), float(ls), np32(b0), np32(e0), np32(c0))


def oracle_core_bwd(inputs, fwd, grads):
    Ug, A = inputs[2], inputs[3]
    vec = inputs[4:20]
    la, ll, ls = inputs[20:23]
    b0, c0 = inputs[23], inputs[25]
    saved = (fwd[0], fwd[2], fwd[3], fwd[5], fwd[6], fwd[7])
    return oracle.core_scan_bwd(np32(torch.cat([Ug, A], 0)), [np32(v) for v in vec], float(la),
                                float(ll), float(ls), np32(b0), np32(c0), saved,
                                [None if g is None else np32(g) for g in grads])


def np32(x) -> np.ndarray:
    if isinstance(x, torch.Tensor):
        return x.detach().float().cpu().numpy()
    return np.asarray(x, dtype=np.float32)


def rel_err(actual, expected) -> float:
    """Normwise relative error max|a - e| / max(max|e|, tiny)."""
    a = np.asarray(np32(actual), dtype=np.float64)
    e = np.asarray(np32(expected), dtype=np.float64)
    denom = max(float(np.abs(e).max()) if e.size else 0.0, 1e-30)
    return float(np.abs(a - e).max()) / denom if e.size else 0.0


def assert_close(actual, expected, *, rtol: float, atol: float, name: str = "") -> None:
    a = np.asarray(np32(actual), dtype=np.float64)
    e = np.asarray(np32(expected), dtype=np.float64)
    assert a.shape == e.shape, f"{name}: shape {a.shape} != {e.shape}"
    if not np.isfinite(a).all():
        raise AssertionError(f"{name}: non-finite values in the HIP result")
    err = np.abs(a - e)
    bound = atol + rtol * np.abs(e)
    excess = err - bound
    if excess.size and excess.max() > 0:
        i = np.unravel_index(int(excess.argmax()), excess.shape)
        raise AssertionError(
            f"{name}: max|diff|={err.max():.3e} (at {i}: got {a[i]:.6e} want {e[i]:.6e}); "
            f"rtol={rtol} atol={atol}; normwise rel={rel_err(a, e):.3e}")


def assert_rel(actual, expected, tol: float, name: str = "") -> None:
    r = rel_err(actual, expected)
    a = np.asarray(np32(actual))
    if not np.isfinite(a).all():
        raise AssertionError(f"{name}: non-finite values in the HIP result")
    assert r <= tol, f"{name}: normwise relative error {r:.3e} > {tol}"


def grad_err(got, want, scale: float) -> float:
    """Normwise error of a parameter gradient, relative to max(max|want|, 1e-3 * scale)
    where ``scale`` is the largest parameter gradient of the module. A scalar gain's
    gradient is a sum over all (query, slot) terms; where those cancel (null_bias and
    adm_bias shift every score of a softmax row equally, so their exact gradient is 0;
    cocktail_gain sums O(1) terms to O(1e-3)), both sides carry fp32 rounding of the
    terms, not of the small total."""
    g = np.asarray(np32(got), np.float64)
    w = np.asarray(np32(want), np.float64)
    return float(np.abs(g - w).max()) / max(float(np.abs(w).max()), 1e-3 * scale, 1e-30)
