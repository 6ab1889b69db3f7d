"""Checks of the HIP path at the BASELINE configurations' full sizes against the CPU oracle.

A whole config-4 step is minutes of work for the oracle (the read alone is 9*N*H
multiply-adds per query), so full-size runs are checked piece by piece, each piece on the
GPU's own inputs so that differences do not compound from one piece to the next:

  * core scan forward: windows of W steps, the oracle restarted from the state the GPU's
    tapes hold at the window start -- budget from U[:, t0-1, H:], energy from the
    (pre-update) energy tape at t0, saturation from the (post-update) tape at t0-1;
  * core scan backward: upstream gradients non-zero only inside one window of one batch
    row, so the oracle's reverse scan over [0, window end) of that row gives every
    gradient the GPU produced for the whole batch;
  * tape statistics: the oracle's means and norms of the GPU's tapes;
  * slot selection: the oracle's stable partition of the GPU's admission values, over the
    full length, bit-exact;
  * three-way read forward: query windows (the oracle reads them with query_offset);
  * three-way read backward: upstream gradient non-zero only inside one query window of
    one batch row, so the oracle's window backward gives every gradient;
  * long scan: the oracle over whole rows (three linear passes are cheap).
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

import oracle
from dabsn_amd.kernels import ops
from helpers import np32, rel_err


def rel_fro(a, b) -> float:
    a = np.asarray(np32(a), np.float64)
    b = np.asarray(np32(b), np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def core_params_np(core):
    """(GA [2H, H], 16 vectors, 3 scalars) of a DABSNCore as fp32 numpy."""
    prm = core.scan_inputs()
    GA = np32(torch.cat([prm[0], prm[1]], 0))
    vec = [np32(v) for v in prm[2:18]]
    scal = [float(x.detach()) for x in prm[18:21]]
    return GA, vec, scal


def core_window_state(U, energy, sat, r, t0, H):
    """The (b, e, c) entering step t0 of row r, read from the forward tapes."""
    if t0 == 0:
        return (np.zeros((1, H), np.float32), np.ones((1, H), np.float32),
                np.zeros((1, H), np.float32))
    return (np32(U[r:r + 1, t0 - 1, H:]), np32(energy[r:r + 1, t0]), np32(sat[r:r + 1, t0 - 1]))


def check_core_windows(core, Wx, Wgx, outs, rows, windows, tol, metric=rel_err):
    """outs = (U, nov, p, ay, w, e, c, gate) of the GPU scan."""
    GA, vec, scal = core_params_np(core)
    U, energy, sat = outs[0], outs[5], outs[6]
    H = Wx.shape[-1]
    worst = 0.0
    for r in rows:
        for t0, t1 in windows:
            b0, e0, c0 = core_window_state(U, energy, sat, r, t0, H)
            want = oracle.core_scan_fwd(np32(Wx[r:r + 1, t0:t1]), np32(Wgx[r:r + 1, t0:t1]), GA,
                                        vec, *scal, b0, e0, c0)
            for k in range(8):
                err = metric(outs[k][r:r + 1, t0:t1], want[k])
                worst = max(worst, err)
                assert err <= tol, f"core output {k}, row {r}, window [{t0},{t1}): {err:.3e}"
    return worst


def check_core_backward_window(core, Wx, Wgx, outs, grads_in, gpu_grads, r, t1, tol):
    """The GPU's gradients (gWx, gWgx, gUg, gA, 16 vectors, 3 scalars) for upstream
    ``grads_in`` (7 tape gradients, non-zero only in row r before t1) against the oracle's
    reverse scan of row r over [0, t1) on the GPU's own tapes (zero initial state)."""
    GA, vec, scal = core_params_np(core)
    H = Wx.shape[-1]
    saved = tuple(np32(outs[k][r:r + 1, :t1]) for k in (0, 2, 3, 5, 6, 7))
    grads = [np32(g[r:r + 1, :t1]) for g in grads_in] + [None, None, None]
    zeros = np.zeros((1, H), np.float32)
    gWx, gWgx, gGA, gvec, gscal, _, _, _ = oracle.core_scan_bwd(GA, vec, *scal, zeros, zeros,
                                                                saved, grads)
    res = {}
    res["gWx"] = rel_fro(gpu_grads[0][r:r + 1, :t1], gWx)
    res["gWgx"] = rel_fro(gpu_grads[1][r:r + 1, :t1], gWgx)
    res["gUg"] = rel_fro(gpu_grads[2], gGA[:H])
    res["gA"] = rel_fro(gpu_grads[3], gGA[H:])
    for i, n in enumerate(oracle.VEC_NAMES):
        res[f"g_{n}"] = rel_fro(gpu_grads[4 + i], gvec[i])
    for i, n in enumerate(("logit_alpha", "log_lambda", "logit_c_suppress")):
        res[f"g_{n}"] = abs(float(gpu_grads[20 + i]) - float(gscal[i])) / max(abs(float(gscal[i])), 1e-6)
    # Nothing outside row r / before t1 may receive gradient.
    others = [gpu_grads[k] for k in (0, 1)]
    for g in others:
        mask = torch.ones(g.shape[:2], dtype=torch.bool)
        mask[r, :t1] = False
        assert float(g.detach().float().cpu()[mask].abs().max()) == 0.0
    for n, err in res.items():
        assert err <= tol, f"core backward {n}: {err:.3e} > {tol}"
    return max(res.values())


def read_pieces(read, tapes):
    """The product's read pieces for full tapes: glue, selection, bank gather."""
    y, budget, ay, w, nov, pl, en, sat = tapes
    T = int(ay.shape[1])
    stats, q, glue = read._glue(ay, w, nov, pl, en, sat)
    bank = read._bank(glue, T, 0)
    K, V, Vn = ops.bank_gather(w, stats[..., 5], bank["idx"], bank["next_idx"], bank["rank"])
    return {"stats": stats, "q": q, "admission": glue.admission_for_select(),
            "cocktail": bank["query_cocktail"], "K": K, "V": V, "Vn": Vn,
            **{f"bank_{k}": v for k, v in bank.items()}, "T": T}


def read_gains(read):
    return (read.short_gain, read.pad_gain, read.induct_gain, read.cocktail_gain)


def check_stats_rows(P, tapes, rows, tol=1e-5):
    y, budget, ay, w, nov, pl, en, sat = tapes
    for r in rows:
        sl = slice(r, r + 1)
        want = oracle.tape_stats(np32(nov[sl]), np32(pl[sl]), np32(en[sl]), np32(sat[sl]),
                                 np32(ay[sl]), np32(w[sl]), [0.0] * 8)
        got = np32(P["stats"][sl])
        assert rel_err(got[..., :4], want["means"]) <= tol
        assert rel_err(got[..., 4], want["norm_ay"]) <= tol
        assert rel_err(got[..., 5], want["norm_w"]) <= tol


def check_selection(P, read):
    adm = P["admission"]
    window = float(F.softplus(read.admit_window.detach()))
    order, counts = oracle.bank_select(np32(adm), window, floor_bf16=adm.dtype == torch.bfloat16)
    n_max = max(int(counts.max()), 1)
    assert P["bank_n_max"] == n_max
    assert np.array_equal(P["bank_idx"].cpu().numpy(), order[:, :n_max])
    valid = np.arange(n_max)[None, :] < np.maximum(counts, 1)[:, None]
    assert np.array_equal(P["bank_valid"].cpu().numpy(), valid)
    return n_max


def check_gather(P, write, rows):
    idx, nidx = P["bank_idx"], P["bank_next_idx"]
    for r in rows:
        assert torch.equal(P["V"][r], write[r, idx[r]])
        assert torch.equal(P["Vn"][r], write[r, nidx[r]])


def _read_args(P, read):
    return (P["q"], P["K"], P["V"], P["Vn"], P["cocktail"], P["bank_cocktail"],
            P["bank_key_bias"], P["bank_admission"], P["bank_scale"], P["bank_read_idx"],
            P["bank_valid"])


def _oracle_read_args(P, read, r, t0, t1):
    sl = slice(r, r + 1)
    gains = tuple(float(x.detach()) for x in read_gains(read))
    return (np32(P["q"][sl, t0:t1]), np32(P["K"][sl]), np32(P["V"][sl]), np32(P["Vn"][sl]),
            np32(P["cocktail"][sl, t0:t1]), np32(P["bank_cocktail"][sl]),
            np32(P["bank_key_bias"][sl]), np32(P["bank_admission"][sl]),
            float(P["bank_scale"]), P["bank_read_idx"][sl].cpu().numpy(),
            P["bank_valid"][sl].cpu().numpy(), 0, gains)


def check_read_windows(P, read, out, rows, windows, tol, metric=rel_err):
    worst = 0.0
    for r in rows:
        for t0, t1 in windows:
            want = oracle.read3_fwd(*_oracle_read_args(P, read, r, t0, t1), query_offset=t0,
                                    total_steps=P["T"])
            err = metric(out[r:r + 1, t0:t1], want)
            worst = max(worst, err)
            assert err <= tol, f"read row {r}, window [{t0},{t1}): {err:.3e}"
    return worst


def check_read_backward_window(P, read, r, t0, t1, tol, scalar_tol, seed=0):
    """Upstream gradient on rows [t0, t1) of batch row r only, through the training read
    (the op that keeps its forward workspace), against the oracle's window backward."""
    args = list(_read_args(P, read))
    leaves = [a.detach().clone().requires_grad_(True) for a in args[:9]]
    gains = [g.detach().clone().requires_grad_(True) for g in read_gains(read)]
    out = ops.admitted_three_way_read_train(*leaves, args[9], args[10], 0, *gains)
    g = torch.Generator().manual_seed(seed)
    go = torch.zeros(out.shape, dtype=torch.float32)
    go[r, t0:t1] = torch.randn(t1 - t0, out.shape[-1], generator=g)
    go = go.to(out.device, out.dtype)
    out.backward(go)
    want = oracle.read3_bwd(np32(go[r:r + 1, t0:t1]), *_oracle_read_args(P, read, r, t0, t1),
                            query_offset=t0, total_steps=P["T"])
    gq, gK, gV, gVn, gck, gcb, gkb, gadm, gscale = (x.grad for x in leaves)
    res = {
        "q": rel_fro(gq[r:r + 1, t0:t1], want[0]), "K": rel_fro(gK[r:r + 1], want[1]),
        "V": rel_fro(gV[r:r + 1], want[2]), "Vn": rel_fro(gVn[r:r + 1], want[3]),
        "bank_cocktail": rel_fro(gcb[r:r + 1], want[5]),
        "key_bias": rel_fro(gkb[r:r + 1], want[6]), "admission": rel_fro(gadm[r:r + 1], want[7]),
    }
    g64, terms = read_window_fp64(P, read, r, t0, t1, go)
    # Cancelling sums, against fp64 (the fp32 oracle must meet the same bound).
    for name, got, ora in (("cocktail", gck[r:r + 1, t0:t1], want[4]),
                           ("scale", gscale, want[8]), ("cocktail_gain", gains[3].grad, want[12])):
        bound = cancelling_bound(g64[name], terms[name], tol)
        err = float(np.linalg.norm(np32(got).astype(np.float64) - g64[name]))
        err_oracle = float(np.linalg.norm(np.asarray(ora, np.float64) - g64[name]))
        assert err_oracle <= bound, f"oracle {name} gradient: {err_oracle:.3e} > {bound:.3e}"
        assert err <= bound, f"read backward {name}: {err:.3e} > {bound:.3e}"
        res[name] = err / bound * tol
    scal = {"short_gain": (gains[0].grad, want[9]), "pad_gain": (gains[1].grad, want[10]),
            "induct_gain": (gains[2].grad, want[11])}
    outside = torch.ones(gq.shape[:2], dtype=torch.bool)
    outside[r, t0:t1] = False
    assert float(gq.detach().float().cpu()[outside].abs().max()) == 0.0
    for n, err in res.items():
        assert err <= tol, f"read backward {n}: {err:.3e} > {tol}"
    for n, (a, b) in scal.items():
        err = abs(float(a.reshape(())) - float(b)) / max(abs(float(b)), 1e-6)
        res[n] = err
        assert err <= scalar_tol, f"read backward {n}: {float(a.reshape(()))} vs {float(b)}"
    return max(res.values())


def read_window_fp64(P, read, r, t0, t1, go):
    """The read of query rows [t0, t1) of batch row r evaluated in fp64 and differentiated
    by autograd (oracle/autograd_ref.dense_read), with the magnitudes of the terms that
    the cancelling gradients sum: cocktail (cg sum_j |dS_perm| |cb_j|), scale
    (sum |dS| |q.k|) and cocktail gain (sum |dS_perm| |ck.cb|)."""
    from oracle import autograd_ref

    sl = slice(r, r + 1)
    d = lambda x: torch.from_numpy(np32(x)).double()  # noqa: E731
    leaves = [d(x).requires_grad_(True) for x in (
        P["q"][sl, t0:t1], P["K"][sl], P["V"][sl], P["Vn"][sl], P["cocktail"][sl, t0:t1],
        P["bank_cocktail"][sl], P["bank_key_bias"][sl], P["bank_admission"][sl])]
    scale = torch.tensor(float(P["bank_scale"]), dtype=torch.float64, requires_grad=True)
    gains = [torch.tensor(float(x.detach()), dtype=torch.float64, requires_grad=True)
             for x in read_gains(read)]
    idx = P["bank_read_idx"][sl].cpu()
    valid = P["bank_valid"][sl].cpu().bool()
    allow, induct = autograd_ref.compact_masks(idx, valid, t1 - t0, 0, query_offset=t0,
                                               total_steps=P["T"])[:2]
    cap: dict = {}
    out = autograd_ref.dense_read(*leaves, scale, allow, induct, gains, capture=cap)
    out.backward(d(go[sl, t0:t1]))
    dperm = cap["perm"].grad.abs()
    cg = float(gains[3].detach())
    terms = {
        "cocktail": (abs(cg) * (dperm @ leaves[5].detach().abs())).numpy(),
        "scale": float((cap["compat"].grad.abs() * cap["qk"].abs()).sum()),
        "cocktail_gain": float((dperm * cap["cocktail_compat"].abs()).sum()) / max(abs(cg), 1e-30)
        if cap["cocktail_compat"] is not None else 0.0,
    }
    grads = {"cocktail": leaves[4].grad.numpy(), "scale": float(scale.grad),
             "short_gain": float(gains[0].grad), "pad_gain": float(gains[1].grad),
             "induct_gain": float(gains[2].grad), "cocktail_gain": float(gains[3].grad)}
    return grads, terms


def cancelling_bound(g64, terms, tol):
    """``tol`` of the fp64 value plus 1e-4 of the summed terms' magnitudes (about a
    thousand fp32 roundings of the terms, for sums taken in different orders)."""
    return tol * float(np.linalg.norm(g64)) + 1e-4 * float(np.linalg.norm(terms))


def check_long_rows(read, write, plasticity, long, rows, tol):
    coef = np.array([float(torch.sigmoid(p.detach())) for p in (
        read.logit_expect_retain, read.logit_retention_decay, read.logit_retain,
        read.logit_retention_strength)], np.float32)
    H = write.shape[-1]
    for r in rows:
        z = np.zeros((1, H), np.float32)
        want, _ = oracle.long_fwd(np32(write[r:r + 1]), np32(plasticity[r:r + 1]), coef, z, z,
                                  np.ones((1, H), np.float32))
        err = rel_err(long[r:r + 1], want)
        assert err <= tol, f"long row {r}: {err:.3e}"
