"""Pins for the CPU oracle (CPU only).

The oracle is what every GPU parity test compares against, so each oracle function
is checked here against something independent of its own formulas:
fp64 autograd of the reference's loop-form math (oracle/autograd_ref.py), closed
forms, brute force, and special cases that reduce the recurrence to scalar math.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from oracle import autograd_ref as ar

@pytest.fixture(autouse=True)
def _fp64_default():
    """fp64 factory default inside this module only (restored for other modules)."""
    previous = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(previous)


def _core_case(seed, B, T, H, din=None, scale_params=0.3):
    """Random inputs/params for the core op, fp64 torch tensors."""
    g = torch.Generator().manual_seed(seed)
    Wx = torch.randn(B, T, H, generator=g) * 0.8
    Wgx = torch.randn(B, T, H, generator=g) * 1.5 - 0.5
    Ug = torch.randn(H, H, generator=g) / math.sqrt(H)
    A = torch.randn(H, H, generator=g) * 0.5 / math.sqrt(H)
    vec = []
    for name in oracle.VEC_NAMES:
        base = {"log_kappa": -2.25, "logit_recover": -4.6, "logit_c_decay": 2.2}.get(name, 0.0)
        vec.append(base + scale_params * torch.randn(H, generator=g))
    scal = (torch.tensor(-2.0) + 0.2 * torch.randn((), generator=g),
            torch.tensor(-1.0) + 0.2 * torch.randn((), generator=g),
            torch.tensor(-6.0) + 0.5 * torch.randn((), generator=g))
    b0 = 0.3 * torch.randn(B, H, generator=g)
    e0 = torch.rand(B, H, generator=g) * 0.5 + 0.5
    c0 = torch.rand(B, H, generator=g) * 0.3
    return Wx, Wgx, Ug, A, vec, scal, b0, e0, c0


def _np(x):
    return x.detach().cpu().numpy().astype(np.float32)


def _oracle_fwd(Wx, Wgx, Ug, A, vec, scal, b0, e0, c0):
    GA = torch.cat([Ug, A], 0)
    return oracle.core_scan_fwd(_np(Wx), _np(Wgx), _np(GA), [_np(v) for v in vec],
                                float(scal[0]), float(scal[1]), float(scal[2]),
                                _np(b0), _np(e0), _np(c0))


def _close(actual, expected, rtol, atol, what=""):
    actual = np.asarray(actual, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    err = np.abs(actual - expected)
    bound = atol + rtol * np.abs(expected)
    worst = float((err - bound).max()) if err.size else 0.0
    assert worst <= 0.0, f"{what}: max|diff|={err.max():.3e} exceeds atol={atol} rtol={rtol}"


@pytest.mark.parametrize("seed,B,T,H", [(7, 3, 5, 6), (8, 2, 9, 7), (9, 1, 1, 4)])
def test_core_forward_matches_fp64_reference_loop(seed, B, T, H):
    case = _core_case(seed, B, T, H)
    got = _oracle_fwd(*case)
    want = ar.core_loop(*case[:4], case[4], *case[5], *case[6:])
    names = ("U", "novelty", "plasticity", "expression", "write", "energy", "saturation",
             "gate", "final_b", "final_e", "final_c")
    for name, a, b in zip(names, got, want):
        _close(a, b.numpy(), 2e-5, 2e-6, name)


def test_core_forward_special_case_zero_recurrence_is_scalar_math():
    """With Ug = A = 0 the recurrent product vanishes: ug = ay = 0, so every unit is an
    independent scalar recurrence that plain Python math can evaluate."""
    B, T, H = 1, 4, 3
    case = list(_core_case(11, B, T, H))
    case[2] = torch.zeros(H, H)
    case[3] = torch.zeros(H, H)
    got = _oracle_fwd(*case)
    Wx, Wgx = case[0][0].numpy(), case[1][0].numpy()
    vec = [v.numpy() for v in case[4]]
    la, ll, ls = (float(s) for s in case[5])
    sig = lambda x: 1.0 / (1.0 + math.exp(-x))
    sp = lambda x: math.log1p(math.exp(x))
    for i in range(H):
        b, e, c = float(case[6][0, i]), float(case[7][0, i]), float(case[8][0, i])
        for t in range(T):
            y = math.tanh(Wx[t, i] + b)
            s = min(max(Wgx[t, i] + 3.0, 0.0), 6.0) / 6.0
            nov = math.tanh(abs(0.0 - b))
            d = sig(vec[13][i])
            c = d * c + (1 - d) * nov * (1 - e)
            ne = nov * (1 - sig(ls) * c)
            tb = math.tanh(b)
            ks = vec[3][i] * s + vec[4][i] * y + vec[5][i] * tb + vec[6][i] * ne + vec[7][i] + vec[14][i] * c
            rs = vec[8][i] * s + vec[9][i] * y + vec[10][i] * tb + vec[11][i] * ne + vec[12][i] + vec[15][i] * c
            wc = sp(vec[1][i]) * math.exp(0.5 * math.tanh(ks))
            rec = min(max(sig(vec[2][i]) * math.exp(0.5 * math.tanh(rs)), 0.0), 1.0)
            p = s * e
            assert got[2][0, t, i] == pytest.approx(p, rel=1e-5, abs=1e-7)
            assert got[3][0, t, i] == 0.0 and got[4][0, t, i] == 0.0
            b = (1 - sig(la)) * b + vec[0][i] + sp(ll) * (p * 0.0)
            e = min(max(e + rec * (1 - e) - wc * p, 0.0), 1.0)
            assert got[0][0, t, H + i] == pytest.approx(b, rel=1e-5, abs=1e-6)
            assert got[6][0, t, i] == pytest.approx(c, rel=1e-5, abs=1e-7)
        assert got[9][0, i] == pytest.approx(e, rel=1e-5, abs=1e-6)


def test_core_forward_invariants_hold():
    case = _core_case(21, 2, 40, 8, scale_params=1.0)
    U, nov, p, ay, w, e, c, s, bF, eF, cF = _oracle_fwd(*case)
    assert (e >= 0).all() and (e <= 1).all() and (eF >= 0).all() and (eF <= 1).all()
    assert (s >= 0).all() and (s <= 1).all()
    np.testing.assert_array_equal(w, p * ay)
    np.testing.assert_array_equal(U[:, -1, 8:], bF)
    np.testing.assert_array_equal(c[:, -1], cF)


def test_core_forward_chunked_equals_full():
    """Carried state: scanning [0,k) then [k,T) from the carried (b,e,c) equals one pass."""
    Wx, Wgx, Ug, A, vec, scal, b0, e0, c0 = _core_case(31, 2, 9, 5)
    full = _oracle_fwd(Wx, Wgx, Ug, A, vec, scal, b0, e0, c0)
    left = _oracle_fwd(Wx[:, :4], Wgx[:, :4], Ug, A, vec, scal, b0, e0, c0)
    carry = [torch.from_numpy(x).double() for x in left[8:]]
    right = _oracle_fwd(Wx[:, 4:], Wgx[:, 4:], Ug, A, vec, scal, *carry)
    for k in range(8):
        np.testing.assert_array_equal(np.concatenate([left[k], right[k]], 1), full[k])
    for k in range(8, 11):
        np.testing.assert_array_equal(right[k], full[k])


@pytest.mark.parametrize("seed,B,T,H", [(41, 2, 6, 5), (42, 3, 4, 8)])
def test_core_backward_matches_fp64_autograd(seed, B, T, H):
    Wx, Wgx, Ug, A, vec, scal, b0, e0, c0 = _core_case(seed, B, T, H)
    leaves = [Wx, Wgx, Ug, A, *vec, *scal, b0, e0, c0]
    leaves = [x.clone().requires_grad_(True) for x in leaves]
    Wx_, Wgx_, Ug_, A_ = leaves[:4]
    vec_ = leaves[4:20]
    scal_ = leaves[20:23]
    b0_, e0_, c0_ = leaves[23:26]
    outs = ar.core_loop(Wx_, Wgx_, Ug_, A_, vec_, *scal_, b0_, e0_, c0_)
    g = torch.Generator().manual_seed(seed + 1000)
    # upstream grads for the 10 public outputs (gate tape excluded, as the op drops it)
    up = [torch.randn(o.shape, generator=g) for o in outs]
    loss = sum((o * u).sum() for k, (o, u) in enumerate(zip(outs, up)) if k != 7)
    grads = torch.autograd.grad(loss, leaves)

    fwd = _oracle_fwd(Wx, Wgx, Ug, A, vec, scal, b0, e0, c0)
    saved = (fwd[0], fwd[2], fwd[3], fwd[5], fwd[6], fwd[7])
    gin = [_np(up[k]) for k in (0, 1, 2, 3, 4, 5, 6, 8, 9, 10)]
    gWx, gWgx, gGA, gvec, gscal, gb0, ge0, gc0 = oracle.core_scan_bwd(
        _np(torch.cat([Ug, A], 0)), [_np(v) for v in vec], float(scal[0]), float(scal[1]),
        float(scal[2]), _np(b0), _np(c0), saved, gin)
    tol = dict(rtol=2e-4, atol=2e-5)
    _close(gWx, grads[0].numpy(), what="Wx", **tol)
    _close(gWgx, grads[1].numpy(), what="Wgx", **tol)
    _close(gGA[:H], grads[2].numpy(), what="Ug", **tol)
    _close(gGA[H:], grads[3].numpy(), what="A", **tol)
    for k, name in enumerate(oracle.VEC_NAMES):
        _close(gvec[k], grads[4 + k].numpy(), what=name, **tol)
    for k, name in enumerate(("logit_alpha", "log_lambda", "logit_c_suppress")):
        _close(gscal[k], grads[20 + k].numpy(), what=name, **tol)
    _close(gb0, grads[23].numpy(), what="b0", **tol)
    _close(ge0, grads[24].numpy(), what="e0", **tol)
    _close(gc0, grads[25].numpy(), what="c0", **tol)


def _read_case(seed, B, T, H, window=0.6, C=4):
    g = torch.Generator().manual_seed(seed)
    q = torch.nn.functional.normalize(torch.randn(B, T, H, generator=g), dim=-1)
    w = torch.randn(B, T, H, generator=g)
    ck = torch.nn.functional.normalize(torch.rand(B, T, C, generator=g), dim=-1)
    kbt = torch.randn(B, T, generator=g) * 0.3
    admt = torch.randn(B, T, generator=g) * 0.5
    order, counts = oracle.bank_select(_np(admt), window)
    n_max, idx, valid, nidx = oracle.bank_from_order(order, counts)
    idx_t = torch.from_numpy(idx)
    gather = lambda x: torch.gather(x, 1, idx_t.unsqueeze(-1).expand(-1, -1, x.shape[-1]))
    V = gather(w)
    K = torch.nn.functional.normalize(V, dim=-1)
    Vn = torch.gather(w, 1, torch.from_numpy(nidx).unsqueeze(-1).expand(-1, -1, H))
    cb = gather(ck)
    kb = torch.gather(kbt, 1, idx_t)
    adm = torch.gather(admt, 1, idx_t)
    return q, K, V, Vn, ck, cb, kb, adm, idx, valid


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("seed,B,T,H", [(51, 2, 7, 5), (52, 3, 12, 4)])
def test_read3_forward_backward_match_fp64_dense_autograd(seed, B, T, H, mode):
    q, K, V, Vn, ck, cb, kb, adm, idx, valid = _read_case(seed, B, T, H)
    gains = (torch.tensor(1.0), torch.tensor(0.7), torch.tensor(0.1), torch.tensor(1.3))
    scale = torch.tensor(1.9)
    allow, induct, _, _ = ar.compact_masks(torch.from_numpy(idx), torch.from_numpy(valid), T, mode)
    leaves = [x.clone().requires_grad_(True) for x in (q, K, V, Vn, ck, cb, kb, adm, scale, *gains)]
    out = ar.dense_read(*leaves[:9], allow, induct, leaves[9:])
    got = oracle.read3_fwd(_np(q), _np(K), _np(V), _np(Vn), _np(ck), _np(cb), _np(kb), _np(adm),
                           float(scale), idx, valid, mode, [float(x) for x in gains])
    _close(got, out.detach().numpy(), 2e-5, 2e-6, "read3 forward")
    go = torch.randn(out.shape, generator=torch.Generator().manual_seed(seed + 7))
    grads = torch.autograd.grad((out * go).sum(), leaves)
    mine = oracle.read3_bwd(_np(go), _np(q), _np(K), _np(V), _np(Vn), _np(ck), _np(cb), _np(kb),
                            _np(adm), float(scale), idx, valid, mode, [float(x) for x in gains])
    names = ("q", "K", "V", "Vn", "cocktail", "bank_cocktail", "key_bias", "admission", "scale",
             "short_gain", "pad_gain", "induct_gain", "cocktail_gain")
    for name, a, b in zip(names, mine, grads):
        _close(a, b.numpy(), 1e-4, 1e-5, name)


def test_read3_rows_with_nothing_allowed_are_zero():
    """A query before every admitted index has no eligible entry: its output is 0."""
    B, T, H = 1, 5, 3
    q, K, V, Vn, ck, cb, kb, adm, idx, valid = _read_case(3, B, T, H)
    idx = np.array([[2, 3, 4, 0, 1]])[:, : K.shape[1]]
    valid = np.ones_like(idx, dtype=bool)
    out = oracle.read3_fwd(_np(q), _np(K), _np(V), _np(Vn), _np(ck), _np(cb), _np(kb), _np(adm),
                           1.0, idx, valid, 0, (1.0, 1.0, 1.0, 1.0))
    if idx.shape[1] and idx[0].min() > 0:
        assert np.all(out[0, : idx[0].min()] == 0.0)


def test_linrec_closed_form_and_backward():
    g = torch.Generator().manual_seed(61)
    B, T, H = 2, 11, 3
    a = torch.rand(B, T, H, generator=g) * 1.2 - 0.1
    gg = torch.randn(B, T, H, generator=g)
    y0 = torch.randn(B, H, generator=g)
    got = oracle.linrec_fwd(_np(a), _np(gg), _np(y0))
    # closed form y_t = (prod_{s<=t} a_s) y0 + sum_{s<=t} (prod_{s<r<=t} a_r) g_s
    an, gn, y0n = a.numpy(), gg.numpy(), y0.numpy()
    want = np.zeros((B, T, H))
    for t in range(T):
        acc = np.prod(an[:, : t + 1], axis=1) * y0n
        for s in range(t + 1):
            acc = acc + np.prod(an[:, s + 1 : t + 1], axis=1) * gn[:, s]
        want[:, t] = acc
    _close(got, want, 1e-5, 1e-6, "linrec closed form")
    leaves = [x.clone().requires_grad_(True) for x in (a, gg, y0)]
    out = ar.linrec_loop(*leaves)
    gy = torch.randn(out.shape, generator=g)
    da, dg, dy0 = torch.autograd.grad((out * gy).sum(), leaves)
    mine = oracle.linrec_bwd(_np(a), _np(gg), _np(y0), _np(gy))
    for name, x, y in zip(("da", "dg", "dy0"), mine, (da, dg, dy0)):
        _close(x, y.numpy(), 1e-5, 1e-6, name)


def test_long_scan_forward_backward_match_fp64_autograd():
    g = torch.Generator().manual_seed(71)
    B, T, H = 2, 13, 4
    w = torch.randn(B, T, H, generator=g) * 0.7
    p = torch.rand(B, T, H, generator=g)
    logits = torch.tensor([2.2, 2.2, 2.2, 1.4]) + 0.3 * torch.randn(4, generator=g)
    L0 = 0.1 * torch.randn(B, H, generator=g)
    E0 = 0.1 * torch.randn(B, H, generator=g)
    R0 = 1.0 - 0.1 * torch.rand(B, H, generator=g)
    coef = torch.sigmoid(logits)
    leaves = [x.clone().requires_grad_(True) for x in (w, p, coef, L0, E0, R0)]
    out, fin = ar.long_loop(leaves[0], leaves[1], *leaves[2].unbind(0), *leaves[3:])
    got, gfin = oracle.long_fwd(_np(w), _np(p), _np(coef), _np(L0), _np(E0), _np(R0))
    _close(got, out.detach().numpy(), 2e-5, 2e-6, "long forward")
    for a, b in zip(gfin, fin):
        _close(a, b.detach().numpy(), 2e-5, 2e-6, "long final")
    gout = torch.randn(out.shape, generator=g)
    gf = [torch.randn(B, H, generator=g) for _ in range(3)]
    loss = (out * gout).sum() + sum((f * u).sum() for f, u in zip(fin, gf))
    grads = torch.autograd.grad(loss, leaves)
    gw, gp, (gL0, gE0, gR0), gcoef = oracle.long_bwd(
        _np(w), _np(p), _np(coef), _np(L0), _np(E0), _np(R0), _np(gout), [_np(x) for x in gf])
    for name, a, b in zip(("w", "p", "coef", "L0", "E0", "R0"),
                          (gw, gp, gcoef, gL0, gE0, gR0), grads):
        _close(a, b.numpy(), 1e-4, 1e-5, name)


def _brute_select(adm, window):
    B, T = adm.shape
    order = np.zeros((B, T), np.int64)
    counts = np.zeros((B,), np.int64)
    for b in range(B):
        run = -np.inf
        member = []
        for t in range(T):
            run = max(run, float(adm[b, t]))
            member.append(bool(np.float32(adm[b, t]) >= np.float32(np.float32(run) - np.float32(window))))
        order[b] = sorted(range(T), key=lambda t: not member[t])
        counts[b] = sum(member)
    return order, counts


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_bank_select_is_a_stable_partition(seed):
    rng = np.random.default_rng(seed)
    B, T = 4, 300
    # quantised values make exact ties with the floor (adm == cummax - window) common
    adm = (rng.integers(-40, 40, size=(B, T)) / 8.0).astype(np.float32)
    window = 1.5
    order, counts = oracle.bank_select(adm, window)
    bo, bc = _brute_select(adm, window)
    np.testing.assert_array_equal(counts, bc)
    np.testing.assert_array_equal(order, bo)
    n_max, idx, valid, nidx = oracle.bank_from_order(order, counts)
    assert n_max == max(int(counts.max()), 1)
    assert (nidx == np.minimum(idx + 1, T - 1)).all()
    for b in range(B):
        assert valid[b].sum() == max(counts[b], 1) or valid[b].sum() == n_max


def test_tape_stats_match_numpy():
    rng = np.random.default_rng(5)
    B, T, H = 2, 6, 9
    tapes = [rng.standard_normal((B, T, H)).astype(np.float32) for _ in range(6)]
    tapes[1] = np.abs(tapes[1])
    gains = (1.0, 0.5, -2.0, 1.0, 0.5, 0.5, 0.25, -2.0)
    st = oracle.tape_stats(*tapes, gains)
    nov, pl, en, sat, ay, wr = (t.astype(np.float64) for t in tapes)
    mn, mp, me, mc = nov.mean(-1), pl.mean(-1), en.mean(-1), sat.mean(-1)
    _close(st["means"], np.stack([me, mc, mn, mp], -1), 1e-6, 1e-7, "means")
    _close(st["norm_ay"], np.sqrt((ay ** 2).sum(-1)), 1e-6, 1e-7, "norm_ay")
    _close(st["norm_w"], np.sqrt((wr ** 2).sum(-1)), 1e-6, 1e-7, "norm_w")
    lp = np.log1p(mp * H)
    _close(st["key_bias"], 1.0 * lp + 0.5 * mn - 2.0, 1e-5, 1e-6, "key_bias")
    _close(st["admission"], lp + 0.5 * mn + 0.5 * mc + 0.25 * me - 2.0, 1e-5, 1e-6, "admission")
    ck = np.stack([me, mc, mn, mp], -1)
    ck = ck / np.maximum(np.linalg.norm(ck, axis=-1, keepdims=True), 1e-12)
    _close(st["cocktail"], ck, 1e-5, 1e-7, "cocktail")


def _permanent_case(seed, B, T, H, unit_keys=False):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(B, T, H, generator=g)
    if unit_keys:
        k = k / k.norm(dim=-1, keepdim=True)
    v = torch.randn(B, T, H, generator=g)
    beta = torch.sigmoid(torch.randn(B, T, generator=g))
    return k, v, beta


@pytest.mark.parametrize("seed,B,T,H,unit", [(81, 2, 7, 6, False), (82, 3, 12, 9, True),
                                             (83, 1, 1, 4, False)])
def test_permanent_scan_matches_fp64_loop_and_autograd(seed, B, T, H, unit):
    """Release-gate shape (2, 7, 6) with raw keys, as in tools/release_gate.py:456-472."""
    k, v, beta = _permanent_case(seed, B, T, H, unit)
    want = ar.permanent_loop(k, v, beta)
    got = oracle.permanent_fwd(_np(k), _np(v), _np(beta))
    scale = float(want.abs().max()) + 1e-30
    _close(got, want.numpy(), 1e-5, 1e-6 * scale, "permanent forward")
    leaves = [x.clone().requires_grad_(True) for x in (k, v, beta)]
    out = ar.permanent_loop(*leaves)
    up = torch.randn(out.shape, generator=torch.Generator().manual_seed(seed + 100))
    grads = torch.autograd.grad((out * up).sum(), leaves, allow_unused=True)  # T = 1: no v, beta
    grads = [torch.zeros_like(x) if d is None else d for x, d in zip(leaves, grads)]
    mine = oracle.permanent_bwd(_np(k), _np(v), _np(beta), _np(up))
    for name, x, y in zip(("dk", "dv", "dbeta"), mine, grads):
        _close(x, y.numpy(), 1e-4, 1e-5 * (float(y.abs().max()) + 1e-30), name)


def test_permanent_scan_closed_forms():
    """T = 1 reads the empty state (0); the second step reads beta_0 (k_0 . k_1) v_0; with
    beta = 0 nothing is ever written."""
    k, v, beta = _permanent_case(84, 3, 2, 5)
    out = oracle.permanent_fwd(_np(k), _np(v), _np(beta))
    assert np.all(out[:, 0] == 0.0)
    want = (beta[:, 0] * (k[:, 0] * k[:, 1]).sum(-1))[:, None] * v[:, 0]
    _close(out[:, 1], want.numpy(), 1e-6, 1e-7, "second step")
    k, v, beta = _permanent_case(85, 2, 6, 4)
    assert np.all(oracle.permanent_fwd(_np(k), _np(v), _np(beta * 0.0)) == 0.0)


def test_field_gather_and_scatter_match_numpy():
    """Release-gate patch (tools/release_gate.py:474-493: 9 cells, neighbours n, n+1, n+3)
    and a random patch with more rows than cells; the scatter is np.add.at, which adds in
    index order, so fp32 results agree exactly."""
    g = np.random.default_rng(86)
    gate = np.array([[n, (n + 1) % 9, (n + 3) % 9] for n in range(9)], np.int64)
    for B, N, D, patch in ((2, 9, 6, gate), (3, 7, 5, g.integers(0, 7, size=(11, 4)))):
        x = g.standard_normal((B, N, D)).astype(np.float32)
        assert np.array_equal(oracle.field_gather(x, patch), x[:, patch])
        gout = g.standard_normal((B,) + patch.shape + (D,)).astype(np.float32)
        want = np.zeros((B, N, D), np.float32)
        for b in range(B):
            np.add.at(want[b], patch.reshape(-1), gout[b].reshape(-1, D))
        assert np.array_equal(oracle.field_gather_bwd(gout, patch, N), want)
    with pytest.raises(IndexError):
        oracle.field_gather(np.zeros((1, 3, 2), np.float32), np.array([[3]]))


def test_cross_entropy_rows_match_fp64_torch():
    """lse and masked NLL against torch.logsumexp / F.cross_entropy(reduction='none'); the
    backward against autograd of scale * sum(NLL)."""
    g = torch.Generator().manual_seed(91)
    rows, V = 13, 37
    x = torch.randn(rows, V, generator=g) * 3
    t = torch.randint(0, V, (rows,), generator=g)
    t[::4] = -100
    lse, nll = oracle.ce_fwd(_np(x), t.numpy(), -100)
    _close(lse, torch.logsumexp(x, -1).numpy(), 1e-6, 1e-6, "lse")
    want = torch.nn.functional.cross_entropy(x, t, ignore_index=-100, reduction="none")
    _close(nll, want.numpy(), 1e-5, 1e-6, "nll")
    xl = x.clone().requires_grad_(True)
    (0.37 * torch.nn.functional.cross_entropy(xl, t, ignore_index=-100, reduction="sum")).backward()
    d = oracle.ce_bwd(_np(x), t.numpy(), -100, lse, 0.37)
    _close(d, xl.grad.numpy(), 1e-5, 1e-7, "dlogits")
