"""Write the golden fixtures in this directory (run: python tests/golden/make_golden.py).

The reference ships no stored vectors for the hot path, so these fixtures are computed
from the fp64 loop-form restatement of the reference math (oracle/autograd_ref.py:
core.py:171-221, admitted.py:16-65 with the compact masks of compact_admitted.py:176-198,
read.py:625-636, long.py:24-32). Gradients come from fp64 torch autograd, independently
of the analytic backward passes in the C oracle and the HIP kernels. Selection order comes
from Python's stable ``sorted`` (read.py:198-203).

Every array is stored as float64 / int64 / uint8 in an ``.npz`` (no pickled objects).
"""

from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import VEC_NAMES  # noqa: E402
from oracle import autograd_ref as ar  # noqa: E402

torch.set_default_dtype(torch.float64)


def _np(x):
    return x.detach().cpu().numpy()


def core_fixture(seed: int, B: int, T: int, H: int) -> dict[str, np.ndarray]:
    g = torch.Generator().manual_seed(seed)
    Wx = torch.randn(B, T, H, generator=g) * 0.8
    Wgx = torch.randn(B, T, H, generator=g) * 1.5 - 0.5
    Ug = torch.randn(H, H, generator=g) / math.sqrt(H)
    A = torch.randn(H, H, generator=g) * 0.5 / math.sqrt(H)
    vec = []
    for name in VEC_NAMES:
        base = {"log_kappa": -2.25, "logit_recover": -4.6, "logit_c_decay": 2.2}.get(name, 0.0)
        vec.append(base + 0.3 * torch.randn(H, generator=g))
    scal = [torch.tensor(-2.0) + 0.2 * torch.randn((), generator=g),
            torch.tensor(-1.0) + 0.2 * torch.randn((), generator=g),
            torch.tensor(-6.0) + 0.5 * torch.randn((), generator=g)]
    b0 = 0.3 * torch.randn(B, H, generator=g)
    e0 = torch.rand(B, H, generator=g) * 0.5 + 0.5
    c0 = torch.rand(B, H, generator=g) * 0.3
    inputs = [Wx, Wgx, Ug, A, *vec, *scal, b0, e0, c0]
    leaves = [x.clone().requires_grad_(True) for x in inputs]
    out = ar.core_loop(leaves[0], leaves[1], leaves[2], leaves[3], leaves[4:20], leaves[20],
                       leaves[21], leaves[22], leaves[23], leaves[24], leaves[25])
    ups = [torch.randn(o.shape, generator=g) for o in out]
    ups[7] = torch.zeros_like(ups[7])  # the gate tape has no gradient path in the op
    grads = torch.autograd.grad(sum((o * u).sum() for o, u in zip(out, ups)), leaves)
    d = {f"in{i}": _np(x) for i, x in enumerate(inputs)}
    d.update({f"out{i}": _np(o) for i, o in enumerate(out)})
    d.update({f"up{i}": _np(u) for i, u in enumerate(ups)})
    d.update({f"gin{i}": _np(x) for i, x in enumerate(grads)})
    return d


def _selection(adm: np.ndarray, window: float):
    """read.py:185-239: cummax floor, member, stable partition (members first)."""
    B, T = adm.shape
    order = np.zeros((B, T), dtype=np.int64)
    counts = np.zeros(B, dtype=np.int64)
    for b in range(B):
        run = -math.inf
        member = []
        for t in range(T):
            run = max(run, float(adm[b, t]))
            member.append(float(adm[b, t]) >= run - window)
        order[b] = sorted(range(T), key=lambda t: not member[t])
        counts[b] = sum(member)
    return order, counts


def read_fixture(seed: int, B: int, T: int, H: int, mode: int) -> dict[str, np.ndarray]:
    g = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(B, T, H, generator=g), dim=-1)
    w = torch.randn(B, T, H, generator=g)
    ck = F.normalize(torch.rand(B, T, 4, generator=g), dim=-1)
    kbt = torch.randn(B, T, generator=g) * 0.3
    admt = torch.randn(B, T, generator=g) * 0.5
    window = 0.7
    order, counts = _selection(_np(admt).astype(np.float32).astype(np.float64), window)
    n_max = max(int(counts.max()), 1)
    idx = order[:, :n_max]
    valid = (np.arange(n_max)[None, :] < np.maximum(counts, 1)[:, None]).astype(np.uint8)
    nidx = np.minimum(idx + 1, T - 1)
    it = torch.from_numpy(idx)
    gat = lambda x: torch.gather(x, 1, it.unsqueeze(-1).expand(-1, -1, x.shape[-1]))  # noqa: E731
    V = gat(w)
    K = F.normalize(V, dim=-1)
    Vn = torch.gather(w, 1, torch.from_numpy(nidx).unsqueeze(-1).expand(-1, -1, H))
    cb, kb, adm = gat(ck), torch.gather(kbt, 1, it), torch.gather(admt, 1, it)
    scale, gains = 1.9, (1.0, 0.7, 0.1, 1.3)
    tens = [q, K, V, Vn, ck, cb, kb, adm]
    leaves = [x.clone().requires_grad_(True) for x in tens]
    sl = [torch.tensor(v).requires_grad_(True) for v in (scale, *gains)]
    allow, induct, _, _ = ar.compact_masks(it, torch.from_numpy(valid).bool(), T, mode)
    out = ar.dense_read(*leaves, sl[0], allow, induct, sl[1:])
    go = torch.randn(B, T, H, generator=g)
    grads = torch.autograd.grad((out * go).sum(), leaves + sl)
    names = ("q", "K", "V", "Vn", "ck", "cb", "kb", "adm")
    d = {n: _np(x) for n, x in zip(names, tens)}
    d.update(idx=idx, valid=valid, mode=np.array(mode, dtype=np.int64),
             scale=np.array(scale), gains=np.array(gains), out=_np(out), go=_np(go))
    d.update({f"g{i}": _np(x) for i, x in enumerate(grads)})
    return d


def long_fixture(seed: int, B: int, T: int, H: int) -> dict[str, np.ndarray]:
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(B, T, H, generator=g) * 0.7
    p = torch.rand(B, T, H, generator=g)
    logits = torch.tensor([2.2, 2.0, 2.4, 1.4]) + 0.1 * torch.randn(4, generator=g)
    L0, E0 = 0.1 * torch.randn(B, H, generator=g), 0.1 * torch.randn(B, H, generator=g)
    R0 = torch.ones(B, H)
    tens = [w, p, logits, L0, E0, R0]
    lv = [x.clone().requires_grad_(True) for x in tens]
    coef = torch.sigmoid(lv[2])
    out, fin = ar.long_loop(lv[0], lv[1], coef[0], coef[1], coef[2], coef[3], lv[3], lv[4], lv[5])
    gout = torch.randn(B, T, H, generator=g)
    gf = [torch.randn(B, H, generator=g) for _ in range(3)]
    loss = (out * gout).sum() + sum((f * u).sum() for f, u in zip(fin, gf))
    grads = torch.autograd.grad(loss, lv)
    d = {n: _np(x) for n, x in zip(("w", "p", "logits", "L0", "E0", "R0"), tens)}
    d.update(out=_np(out), fL=_np(fin[0]), fE=_np(fin[1]), fR=_np(fin[2]), gout=_np(gout),
             gfL=_np(gf[0]), gfE=_np(gf[1]), gfR=_np(gf[2]))
    d.update({f"g_{n}": _np(x) for n, x in zip(("w", "p", "logits", "L0", "E0", "R0"), grads)})
    return d


def linrec_fixture(seed: int, B: int, T: int, H: int) -> dict[str, np.ndarray]:
    g = torch.Generator().manual_seed(seed)
    a = torch.rand(B, T, H, generator=g) * 1.1 - 0.05
    x = torch.randn(B, T, H, generator=g)
    y0 = torch.randn(B, H, generator=g)
    lv = [t.clone().requires_grad_(True) for t in (a, x, y0)]
    y = ar.linrec_loop(*lv)
    gy = torch.randn(B, T, H, generator=g)
    grads = torch.autograd.grad((y * gy).sum(), lv)
    return dict(a=_np(a), g=_np(x), y0=_np(y0), y=_np(y), gy=_np(gy), da=_np(grads[0]),
                dg=_np(grads[1]), dy0=_np(grads[2]))


def select_fixture(seed: int, B: int, T: int) -> dict[str, np.ndarray]:
    rng = np.random.default_rng(seed)
    adm = (rng.integers(-24, 24, size=(B, T)) / 8.0).astype(np.float32)  # many exact ties
    adm[0] = np.sort(adm[0])
    adm[1] = adm[1][0]
    window = np.float32(1.25)
    order, counts = _selection(adm.astype(np.float64), float(window))
    return dict(adm=adm, window=np.array(window), order=order, counts=counts)


FIXTURES = {
    "core_B3_T16_H12": lambda: core_fixture(1, 3, 16, 12),
    "core_B2_T9_H40": lambda: core_fixture(2, 2, 9, 40),
    "read3_seq_B2_T12_H6": lambda: read_fixture(3, 2, 12, 6, 0),
    "read3_field_B2_T12_H6": lambda: read_fixture(4, 2, 12, 6, 1),
    "long_B2_T40_H5": lambda: long_fixture(5, 2, 40, 5),
    "linrec_B2_T30_H4": lambda: linrec_fixture(6, 2, 30, 4),
    "select_B4_T50": lambda: select_fixture(7, 4, 50),
}


def main() -> None:
    for name, make in FIXTURES.items():
        path = HERE / f"{name}.npz"
        np.savez_compressed(path, **make())
        print(f"wrote {path.name} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
