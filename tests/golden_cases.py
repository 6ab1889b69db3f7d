"""Golden fixtures (tests/golden/*.npz) and runners that evaluate them on the CPU oracle
or on the HIP operators, returning results in the fixture's layout."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"

CORE = ("core_B3_T16_H12", "core_B2_T9_H40")
READ3 = ("read3_seq_B2_T12_H6", "read3_field_B2_T12_H6")
LONG = "long_B2_T40_H5"
LINREC = "linrec_B2_T30_H4"
SELECT = "select_B4_T50"


def load(name: str) -> dict[str, np.ndarray]:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def f32(x) -> np.ndarray:
    a = np.asarray(x, dtype=np.float32)
    return a if a.ndim == 0 else np.ascontiguousarray(a)


# ---- core ---------------------------------------------------------------------------
def core_grads_in(d):
    """Upstream grads in op order (U, nov, p, ay, w, e, c, final b, e, c); gate has none."""
    return [d[f"up{i}"] for i in (0, 1, 2, 3, 4, 5, 6, 8, 9, 10)]


def core_oracle(d):
    import oracle

    x = [f32(d[f"in{i}"]) for i in range(26)]
    GA = np.concatenate([x[2], x[3]], 0)
    out = oracle.core_scan_fwd(x[0], x[1], GA, x[4:20], float(x[20]), float(x[21]), float(x[22]),
                               x[23], x[24], x[25])
    saved = (out[0], out[2], out[3], out[5], out[6], out[7])
    ob = oracle.core_scan_bwd(GA, x[4:20], float(x[20]), float(x[21]), float(x[22]), x[23], x[25],
                              saved, [f32(g) for g in core_grads_in(d)])
    H = x[0].shape[-1]
    grads = [ob[0], ob[1], ob[2][:H], ob[2][H:], *[ob[3][i] for i in range(16)],
             *[ob[4][i] for i in range(3)], ob[5], ob[6], ob[7]]
    return list(out), grads


def core_hip(d, device):
    from dabsn_amd.kernels import ops

    x = [torch.from_numpy(f32(d[f"in{i}"])).to(device) for i in range(26)]
    out = ops.core_scan_batched(*x)
    ups = [torch.from_numpy(f32(g)).to(device) for g in core_grads_in(d)]
    res = ops.core_scan_batched_backward(
        x[2], x[3], x[4:20], x[20], x[21], x[22], x[23], x[25], out[0], out[2], out[3], out[5],
        out[6], out[7], *ups)
    return [o.cpu() for o in out], [r.cpu() for r in res]


# ---- three-way read -------------------------------------------------------------------
def read3_oracle(d):
    import oracle

    a = [f32(d[k]) for k in ("q", "K", "V", "Vn", "ck", "cb", "kb", "adm")]
    args = (*a, float(d["scale"]), d["idx"], d["valid"], int(d["mode"]),
            tuple(float(v) for v in d["gains"]))
    out = oracle.read3_fwd(*args)
    grads = oracle.read3_bwd(f32(d["go"]), *args)
    return out, list(grads)


def read3_hip(d, device):
    from dabsn_amd.kernels import ops

    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(device)  # noqa: E731
    s = lambda v: torch.tensor([float(v)], device=device)  # noqa: E731
    args = (*[t(f32(d[k])) for k in ("q", "K", "V", "Vn", "ck", "cb", "kb", "adm")],
            s(d["scale"]), t(d["idx"]), t(d["valid"]), int(d["mode"]),
            *[s(v) for v in d["gains"]])
    out = ops.admitted_three_way_read_compact_flash(*args)
    grads = ops.admitted_three_way_read_compact_flash_backward(t(f32(d["go"])), *args)
    return out.cpu(), [g.cpu() for g in grads]


# ---- long scan / linear recurrence -------------------------------------------------
def _sig(x):
    return 1.0 / (1.0 + np.exp(-np.asarray(x, dtype=np.float64)))


def long_oracle(d):
    import oracle

    coef = f32(_sig(d["logits"]))
    out, fin = oracle.long_fwd(f32(d["w"]), f32(d["p"]), coef, f32(d["L0"]), f32(d["E0"]),
                               f32(d["R0"]))
    gw, gp, g0, gcoef = oracle.long_bwd(f32(d["w"]), f32(d["p"]), coef, f32(d["L0"]),
                                        f32(d["E0"]), f32(d["R0"]), f32(d["gout"]),
                                        [f32(d["gfL"]), f32(d["gfE"]), f32(d["gfR"])])
    glog = np.asarray(gcoef, np.float64) * coef * (1.0 - coef)
    return out, list(fin), [gw, gp, glog, *g0]


def long_hip(d, device):
    from dabsn_amd.kernels import ops

    t = lambda x: torch.from_numpy(f32(x)).to(device)  # noqa: E731
    logits = [torch.tensor([float(v)], device=device) for v in d["logits"]]
    out = ops.long_scan_fused(t(d["w"]), t(d["p"]), *logits, t(d["L0"]), t(d["E0"]), t(d["R0"]))
    res = ops.long_scan_fused_backward(t(d["w"]), t(d["p"]), logits, out[4], t(d["gout"]),
                                       t(d["gfL"]), t(d["gfE"]), t(d["gfR"]))
    glog = np.array([float(res[2 + i]) for i in range(4)])
    return (out[0].cpu(), [o.cpu() for o in out[1:4]],
            [res[0].cpu(), res[1].cpu(), glog, *[r.cpu() for r in res[6:9]]])


def linrec_oracle(d):
    import oracle

    y = oracle.linrec_fwd(f32(d["a"]), f32(d["g"]), f32(d["y0"]))
    return y, list(oracle.linrec_bwd(f32(d["a"]), f32(d["g"]), f32(d["y0"]), f32(d["gy"])))


def linrec_hip(d, device):
    from dabsn_amd.kernels import ops

    t = lambda x: torch.from_numpy(f32(x)).to(device)  # noqa: E731
    y = ops.linear_recurrence(t(d["a"]), t(d["g"]), t(d["y0"]))
    return y.cpu(), [r.cpu() for r in ops.linrec_backward(t(d["a"]), t(d["g"]), t(d["y0"]), t(d["gy"]))]


LONG_GRAD_NAMES = ("g_w", "g_p", "g_logits", "g_L0", "g_E0", "g_R0")
READ3_GRAD_NAMES = ("q", "K", "V", "Vn", "cocktail", "bank_cocktail", "key_bias", "admission",
                    "scale", "short_gain", "pad_gain", "induct_gain", "cocktail_gain")
