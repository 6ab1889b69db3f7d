"""CPU oracle for the DABSN recurrent hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
import this package, and only as the checker. The product package ``dabsn_amd``
never imports it.

The numeric work lives in ``dabsn_oracle.c`` (a plain-C restatement of the
reference CPU backend, built by ``oracle/Makefile`` into ``oracle/_build``). This
module is a thin numpy/ctypes wrapper around it plus the pure-Python pieces of the
read glue. Each wrapper names the reference code it restates.

Parity pins (what checks this oracle, see ``tests/test_oracle_pins.py``):
  * core scan fwd/bwd: fp64 autograd of the reference loop (core.py:171-221),
    hand-computed special cases (Ug=A=0, T=1), invariants (e, s in [0,1]).
  * three-way read fwd/bwd: fp64 autograd of the dense masked-softmax op
    (admitted.py:16-65), brute-force mask construction.
  * linear recurrence / long scan: closed form y_t = prod(a) y0 + sum prod(a) g,
    fp64 autograd of the loop at read.py:625-636.
  * bank selection: Python ``sorted`` stable partition (read.py:198-203).
  * tape stats: numpy means/norms (read.py:58-72, 154-183).
  * permanent delta scan fwd/bwd: fp64 autograd of the reference's einsum loop
    (permanent.py:39-51), closed forms (T = 1 gives 0; T = 2 gives beta_0 (k_0 . k_1) v_0;
    beta = 0 gives 0).
  * local field gather/scatter: numpy fancy indexing and ``np.add.at``.
  * cross-entropy rows: fp64 torch ``F.cross_entropy`` and its autograd gradient.
The reference ships no golden vectors for this path, and its C++ backend needs
libtorch to build, so it is not compiled here.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "liboracle.so"
_LIB = None

_F = ctypes.POINTER(ctypes.c_float)
_I64 = ctypes.POINTER(ctypes.c_int64)
_U8 = ctypes.POINTER(ctypes.c_uint8)

VEC_NAMES = (
    "beta",
    "log_kappa",
    "logit_recover",
    "k_s",
    "k_y",
    "k_b",
    "k_n",
    "k_bias",
    "r_s",
    "r_y",
    "r_b",
    "r_n",
    "r_bias",
    "logit_c_decay",
    "k_c",
    "r_c",
)


def build() -> Path:
    """Compile the oracle library (idempotent: make only rebuilds when stale)."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def lib():
    global _LIB
    if _LIB is None:
        if not _LIB_PATH.exists():
            build()
        _LIB = ctypes.CDLL(str(_LIB_PATH))
        _LIB.oracle_num_threads.restype = ctypes.c_int
    return _LIB


def set_num_threads(n: int) -> None:
    lib().oracle_set_num_threads(int(n))


def num_threads() -> int:
    return int(lib().oracle_num_threads())


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    if a.dtype == np.float32:
        return a.ctypes.data_as(_F)
    if a.dtype == np.int64:
        return a.ctypes.data_as(_I64)
    if a.dtype == np.uint8:
        return a.ctypes.data_as(_U8)
    raise TypeError(a.dtype)


def _vec_array(vec) -> tuple[ctypes.Array, list[np.ndarray]]:
    arrays = [_f32(v) for v in vec]
    if len(arrays) != 16:
        raise ValueError("core scan takes 16 per-unit vectors")
    table = (_F * 16)(*[_ptr(a) for a in arrays])
    return table, arrays


def core_scan_fwd(Wx, Wgx, GA, vec, logit_alpha, log_lambda, logit_c_suppress, b0, e0, c0):
    """Restates cpu_runtime.cpp:672-837 (+ gate tape, cpu.py:866-869).

    Returns the registered op's 11 outputs (batched_runtime.py:1193-1205):
    U, novelty, plasticity, expression, write, energy, saturation, gate,
    final_b, final_e, final_c.
    """
    Wx, Wgx, GA = _f32(Wx), _f32(Wgx), _f32(GA)
    B, T, H = Wx.shape
    b0, e0, c0 = _f32(b0), _f32(e0), _f32(c0)
    table, keep = _vec_array(vec)
    U = np.empty((B, T, 2 * H), np.float32)
    tapes = [np.empty((B, T, H), np.float32) for _ in range(7)]
    finals = [np.empty((B, H), np.float32) for _ in range(3)]
    lib().oracle_core_scan_fwd(
        ctypes.c_int64(B), ctypes.c_int64(T), ctypes.c_int64(H),
        _ptr(Wx), _ptr(Wgx), _ptr(GA), table,
        ctypes.c_float(logit_alpha), ctypes.c_float(log_lambda), ctypes.c_float(logit_c_suppress),
        _ptr(b0), _ptr(e0), _ptr(c0), _ptr(U), *[_ptr(t) for t in tapes], *[_ptr(f) for f in finals],
    )
    del keep
    return (U, *tapes, *finals)


def core_scan_bwd(GA, vec, logit_alpha, log_lambda, logit_c_suppress, b0, c0, saved, grads):
    """Restates the registered reverse scan (batched_runtime.py:299-466, 501-622)
    and the recurrent-weight gradient GEMM (batched_runtime.py:1475-1482).

    ``saved`` = (U, plasticity, expression, energy, saturation, gate).
    ``grads`` = (gU, gnovelty, gplasticity, gexpression, gwrite, genergy,
    gsaturation, gfinal_b, gfinal_e, gfinal_c); entries may be None.
    Returns (gWx, gWgx, gGA [2H,H], gvec [16,H], gscal [3], gb0, ge0, gc0).
    """
    GA = _f32(GA)
    U, Pl, Ay, Et, Ct, St = (_f32(x) for x in saved)
    B, T, H = Pl.shape
    g = [None if x is None else _f32(x) for x in grads]
    table, keep = _vec_array(vec)
    gWx = np.empty((B, T, H), np.float32)
    gWgx = np.empty((B, T, H), np.float32)
    day = np.empty((B, T, H), np.float32)
    gGA = np.empty((2 * H, H), np.float32)
    gvec = np.empty((16, H), np.float32)
    gscal = np.empty((3,), np.float32)
    gb0, ge0, gc0 = (np.empty((B, H), np.float32) for _ in range(3))
    lib().oracle_core_scan_bwd(
        ctypes.c_int64(B), ctypes.c_int64(T), ctypes.c_int64(H), _ptr(GA), table,
        ctypes.c_float(logit_alpha), ctypes.c_float(log_lambda), ctypes.c_float(logit_c_suppress),
        _ptr(_f32(b0)), _ptr(_f32(c0)),
        _ptr(U), _ptr(Pl), _ptr(Ay), _ptr(Et), _ptr(Ct), _ptr(St),
        *[_ptr(x) for x in g],
        _ptr(gWx), _ptr(gWgx), _ptr(day), _ptr(gGA), _ptr(gvec), _ptr(gscal),
        _ptr(gb0), _ptr(ge0), _ptr(gc0),
    )
    del keep
    return gWx, gWgx, gGA, gvec, gscal, gb0, ge0, gc0


def _read_common(q, K, V, Vn, ck, cb, kb, adm, idx, valid):
    q, K, V, Vn, ck, cb, kb, adm = (_f32(x) for x in (q, K, V, Vn, ck, cb, kb, adm))
    idx = np.ascontiguousarray(np.asarray(idx, dtype=np.int64))
    valid = np.ascontiguousarray(np.asarray(valid, dtype=np.uint8))
    return q, K, V, Vn, ck, cb, kb, adm, idx, valid


def read3_fwd(q, K, V, Vn, ck, cb, kb, adm, scale, idx, valid, mode, gains,
              query_offset=0, total_steps=None):
    """Restates cpu_runtime.cpp:321-438 with compact masks (compact_admitted.py:176-198).

    gains = (short_gain, pad_gain, induct_gain, cocktail_gain).
    """
    q, K, V, Vn, ck, cb, kb, adm, idx, valid = _read_common(q, K, V, Vn, ck, cb, kb, adm, idx, valid)
    B, T, H = q.shape
    N = K.shape[1]
    C = ck.shape[2]
    total = T if total_steps is None else int(total_steps)
    out = np.empty((B, T, H), np.float32)
    sg, pg, ig, cg = (float(x) for x in gains)
    lib().oracle_read3_fwd(
        ctypes.c_int64(B), ctypes.c_int64(T), ctypes.c_int64(N), ctypes.c_int64(H), ctypes.c_int64(C),
        _ptr(q), _ptr(K), _ptr(V), _ptr(Vn), _ptr(ck), _ptr(cb), _ptr(kb), _ptr(adm),
        ctypes.c_float(scale), _ptr(idx), _ptr(valid), ctypes.c_int(mode),
        ctypes.c_int64(query_offset), ctypes.c_int64(total),
        ctypes.c_float(sg), ctypes.c_float(pg), ctypes.c_float(ig), ctypes.c_float(cg), _ptr(out),
    )
    return out


def read3_bwd(go, q, K, V, Vn, ck, cb, kb, adm, scale, idx, valid, mode, gains,
              query_offset=0, total_steps=None):
    """Restates cpu_runtime.cpp:479-662. Returns
    (gq, gK, gV, gVn, gck, gcb, gkb, gadm, gscale, gshort, gpad, ginduct, gcocktail_gain)."""
    go = _f32(go)
    q, K, V, Vn, ck, cb, kb, adm, idx, valid = _read_common(q, K, V, Vn, ck, cb, kb, adm, idx, valid)
    B, T, H = q.shape
    N = K.shape[1]
    C = ck.shape[2]
    total = T if total_steps is None else int(total_steps)
    gq = np.empty_like(q)
    gK, gV, gVn = np.empty_like(K), np.empty_like(V), np.empty_like(Vn)
    gck, gcb = np.empty_like(ck), np.empty_like(cb)
    gkb, gadm = np.empty_like(kb), np.empty_like(adm)
    gsc = np.empty((5,), np.float32)
    sg, pg, ig, cg = (float(x) for x in gains)
    lib().oracle_read3_bwd(
        ctypes.c_int64(B), ctypes.c_int64(T), ctypes.c_int64(N), ctypes.c_int64(H), ctypes.c_int64(C),
        _ptr(go), _ptr(q), _ptr(K), _ptr(V), _ptr(Vn), _ptr(ck), _ptr(cb), _ptr(kb), _ptr(adm),
        ctypes.c_float(scale), _ptr(idx), _ptr(valid), ctypes.c_int(mode),
        ctypes.c_int64(query_offset), ctypes.c_int64(total),
        ctypes.c_float(sg), ctypes.c_float(pg), ctypes.c_float(ig), ctypes.c_float(cg),
        _ptr(gq), _ptr(gK), _ptr(gV), _ptr(gVn), _ptr(gck), _ptr(gcb), _ptr(gkb), _ptr(gadm), _ptr(gsc),
    )
    return (gq, gK, gV, gVn, gck, gcb, gkb, gadm, gsc[0], gsc[1], gsc[2], gsc[3], gsc[4])


def linrec_fwd(a, g, y0):
    """Restates cpu_runtime.cpp:92-108."""
    a, g, y0 = _f32(a), _f32(g), _f32(y0)
    B, T, H = a.shape
    out = np.empty_like(a)
    lib().oracle_linrec_fwd(ctypes.c_int64(B), ctypes.c_int64(T), ctypes.c_int64(H),
                            _ptr(a), _ptr(g), _ptr(y0), _ptr(out))
    return out


def linrec_bwd(a, g, y0, gy):
    """Restates cpu_runtime.cpp:110-143. Returns (da, dg, dy0)."""
    a, g, y0, gy = _f32(a), _f32(g), _f32(y0), _f32(gy)
    B, T, H = a.shape
    da, dg, dy0 = np.empty_like(a), np.empty_like(g), np.empty_like(y0)
    lib().oracle_linrec_bwd(ctypes.c_int64(B), ctypes.c_int64(T), ctypes.c_int64(H),
                            _ptr(a), _ptr(g), _ptr(y0), _ptr(gy), _ptr(da), _ptr(dg), _ptr(dy0))
    return da, dg, dy0


def long_fwd(w, p, coef, L0, E0, R0):
    """Restates long.py:492-579 (equivalently the loop at read.py:625-636).

    coef = sigmoid of (logit_expect_retain, logit_retention_decay, logit_retain,
    logit_retention_strength). Returns (long [B,T,H], (L, E, R) final)."""
    w, p = _f32(w), _f32(p)
    B, T, H = w.shape
    coef = _f32(coef)
    out = np.empty_like(w)
    LF, EF, RF = (np.empty((B, H), np.float32) for _ in range(3))
    lib().oracle_long_fwd(ctypes.c_int64(B), ctypes.c_int64(T), ctypes.c_int64(H),
                          _ptr(w), _ptr(p), _ptr(coef), _ptr(_f32(L0)), _ptr(_f32(E0)), _ptr(_f32(R0)),
                          _ptr(out), _ptr(LF), _ptr(EF), _ptr(RF))
    return out, (LF, EF, RF)


def long_bwd(w, p, coef, L0, E0, R0, gout, gfinal=(None, None, None)):
    """Chain rule through the three recurrences of long.py:492-579.

    Returns (gw, gp, (gL0, gE0, gR0), gcoef[4]) with gcoef w.r.t. the sigmoid outputs."""
    w, p, gout = _f32(w), _f32(p), _f32(gout)
    B, T, H = w.shape
    coef = _f32(coef)
    gf = [None if x is None else _f32(x) for x in gfinal]
    gw, gp = np.empty_like(w), np.empty_like(p)
    gL0, gE0, gR0 = (np.empty((B, H), np.float32) for _ in range(3))
    gcoef = np.empty((4,), np.float32)
    lib().oracle_long_bwd(ctypes.c_int64(B), ctypes.c_int64(T), ctypes.c_int64(H),
                          _ptr(w), _ptr(p), _ptr(coef), _ptr(_f32(L0)), _ptr(_f32(E0)), _ptr(_f32(R0)),
                          _ptr(gout), *[_ptr(x) for x in gf],
                          _ptr(gw), _ptr(gp), _ptr(gL0), _ptr(gE0), _ptr(gR0), _ptr(gcoef))
    return gw, gp, (gL0, gE0, gR0), gcoef


def tape_stats(nov, pl, en, sat, ay, wr, gains):
    """Restates read.py:58-72, 154-183. gains = (p_gain, novelty_gain, null_bias,
    adm_p, adm_n, adm_s, adm_e, adm_bias). Returns a dict of per-position arrays."""
    nov, pl, en, sat, ay, wr = (_f32(x) for x in (nov, pl, en, sat, ay, wr))
    B, T, H = nov.shape
    g = np.zeros(10, np.float32)
    g[: len(gains)] = np.asarray(gains, np.float32)
    means = np.empty((B, T, 4), np.float32)
    norm_ay, norm_w, kb, adm = (np.empty((B, T), np.float32) for _ in range(4))
    cock = np.empty((B, T, 4), np.float32)
    lib().oracle_tape_stats(ctypes.c_int64(B), ctypes.c_int64(T), ctypes.c_int64(H),
                            _ptr(nov), _ptr(pl), _ptr(en), _ptr(sat), _ptr(ay), _ptr(wr), _ptr(g),
                            _ptr(means), _ptr(norm_ay), _ptr(norm_w), _ptr(kb), _ptr(adm), _ptr(cock))
    return {"means": means, "norm_ay": norm_ay, "norm_w": norm_w, "key_bias": kb,
            "admission": adm, "cocktail": cock}


def round_bf16(x) -> np.ndarray:
    """fp32 -> nearest bf16 (ties to even), returned as fp32 values: what
    ``tensor.to(torch.bfloat16)`` stores for finite inputs."""
    bits = _f32(x).view(np.uint32).astype(np.uint64)
    bits = (bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000
    return bits.astype(np.uint32).view(np.float32)


def bank_select(adm, window, floor_bf16: bool = False, whole: bool = False):
    """Restates read.py:185-239. Returns (order [B,T] int64, counts [B] int64).

    The floor is ``cummax(adm) - window`` (seq geometry) or, with ``whole``, the row's
    ``max(adm) - window`` (field and hybrid, read.py:189-191). With ``floor_bf16`` the
    admission values are bf16 values and the floor is rounded to bf16, as the reference's
    bf16 subtraction does (its result is computed in fp32 and rounded once)."""
    if floor_bf16 or whole:
        a = _f32(adm)
        top = (np.max(a, axis=1, keepdims=True) if whole else np.maximum.accumulate(a, axis=1))
        floor = top - np.float32(window)
        if floor_bf16:
            floor = round_bf16(floor)
        member = a >= floor
        order = np.argsort(~member, axis=1, kind="stable").astype(np.int64)
        return order, member.sum(axis=1).astype(np.int64)
    adm = _f32(adm)
    B, T = adm.shape
    order = np.empty((B, T), np.int64)
    counts = np.empty((B,), np.int64)
    lib().oracle_bank_select(ctypes.c_int64(B), ctypes.c_int64(T), _ptr(adm),
                             ctypes.c_float(window), _ptr(order), _ptr(counts))
    return order, counts


def bank_from_order(order, counts):
    """n_max, idx, valid, next_idx exactly as read.py:233-239, 298."""
    order = np.asarray(order)
    counts = np.asarray(counts)
    T = order.shape[1]
    n_max = max(int(counts.max()), 1)
    idx = order[:, :n_max].copy()
    valid = np.arange(n_max)[None, :] < np.maximum(counts, 1)[:, None]
    next_idx = np.minimum(idx + 1, T - 1)
    return n_max, idx, valid, next_idx


def normalize_rows(x, eps=1e-12):
    """F.normalize(x, dim=-1) in float32."""
    x = _f32(x)
    n = np.sqrt((x.astype(np.float64) ** 2).sum(-1, keepdims=True)).astype(np.float32)
    return (x / np.maximum(n, np.float32(eps))).astype(np.float32)


def _ensure_env():
    os.environ.setdefault("OMP_NUM_THREADS", str(min(16, os.cpu_count() or 1)))


_ensure_env()


def permanent_fwd(k, v, beta):
    """Restates cpu_runtime.cpp:1075-1109 (permanent.py:39-51). Returns out [B,T,H]."""
    k, v, beta = _f32(k), _f32(v), _f32(beta)
    B, T, H = k.shape
    out = np.empty_like(k)
    lib().oracle_permanent_fwd(ctypes.c_int64(B), ctypes.c_int64(T), ctypes.c_int64(H),
                               _ptr(k), _ptr(v), _ptr(beta), _ptr(out))
    return out


def permanent_bwd(k, v, beta, g):
    """Restates cpu_runtime.cpp:1112-1188 (permanent.py:70-119). Returns (dk, dv, dbeta)."""
    k, v, beta, g = _f32(k), _f32(v), _f32(beta), _f32(g)
    B, T, H = k.shape
    dk, dv, db = np.empty_like(k), np.empty_like(v), np.empty_like(beta)
    lib().oracle_permanent_bwd(ctypes.c_int64(B), ctypes.c_int64(T), ctypes.c_int64(H),
                               _ptr(k), _ptr(v), _ptr(beta), _ptr(g), _ptr(dk), _ptr(dv), _ptr(db))
    return dk, dv, db


def field_gather(x, patch):
    """Restates cpu_runtime.cpp:1191-1211: x [B,N,D], patch [P,K] -> [B,P,K,D]."""
    x = _f32(x)
    patch = np.ascontiguousarray(np.asarray(patch, dtype=np.int64))
    B, N, D = x.shape
    P, K = patch.shape
    if patch.size and (patch.min() < 0 or patch.max() >= N):
        raise IndexError("patch index outside [0, N)")
    out = np.empty((B, P, K, D), np.float32)
    lib().oracle_field_gather(ctypes.c_int64(B), ctypes.c_int64(N), ctypes.c_int64(D),
                              ctypes.c_int64(P), ctypes.c_int64(K), _ptr(x), _ptr(patch), _ptr(out))
    return out


def field_gather_bwd(gout, patch, cells):
    """Restates cpu_runtime.cpp:1214-1237: scatter-add of gout [B,P,K,D] -> [B,cells,D]."""
    gout = _f32(gout)
    patch = np.ascontiguousarray(np.asarray(patch, dtype=np.int64))
    B, P, K, D = gout.shape
    if patch.size and (patch.min() < 0 or patch.max() >= cells):
        raise IndexError("patch index outside [0, N)")
    gx = np.empty((B, cells, D), np.float32)
    lib().oracle_field_gather_bwd(ctypes.c_int64(B), ctypes.c_int64(cells), ctypes.c_int64(D),
                                  ctypes.c_int64(P), ctypes.c_int64(K), _ptr(gout), _ptr(patch),
                                  _ptr(gx))
    return gx


def ce_fwd(logits, targets, ignore_index):
    """Restates runtime/loss.py:83-93 for one chunk. Returns (lse, nll) per row."""
    x = _f32(logits)
    t = np.ascontiguousarray(np.asarray(targets, dtype=np.int64))
    rows, V = x.shape
    bad = (t != ignore_index) & ((t < 0) | (t >= V))
    if bad.any():
        raise IndexError("target outside [0, V)")
    lse, nll = np.empty(rows, np.float32), np.empty(rows, np.float32)
    lib().oracle_ce_fwd(ctypes.c_int64(rows), ctypes.c_int64(V), _ptr(x), _ptr(t),
                        ctypes.c_int64(ignore_index), _ptr(lse), _ptr(nll))
    return lse, nll


def ce_bwd(logits, targets, ignore_index, lse, scale):
    """Restates runtime/loss.py:105-133 for one chunk: (softmax - onehot) * scale."""
    x = _f32(logits)
    t = np.ascontiguousarray(np.asarray(targets, dtype=np.int64))
    rows, V = x.shape
    d = np.empty_like(x)
    lib().oracle_ce_bwd(ctypes.c_int64(rows), ctypes.c_int64(V), _ptr(x), _ptr(t),
                        ctypes.c_int64(ignore_index), _ptr(_f32(lse)), ctypes.c_float(scale),
                        _ptr(d))
    return d
