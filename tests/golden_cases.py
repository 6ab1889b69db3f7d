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


# ---- bf16 distance of the core op at larger shapes ----------------------------------
# The reference's own bf16-vs-fp32 distance of dabsn::core_scan_batched is recorded at
# these shapes (tests/golden/ref/core_bf16_gap.npz, written by make_ref_golden.py); the
# inputs are rebuilt from this seeded recipe wherever the fixture is checked, so no large
# tensor is stored.
BF16_GAP_SHAPES = {"B2_T256_H512": (2, 256, 512, 31), "B1_T1024_H2048": (1, 1024, 2048, 32)}
# Centres of the 16 per-unit vectors in op order (beta, log_kappa, logit_recover, k_s, k_y,
# k_b, k_n, k_bias, r_s, r_y, r_b, r_n, r_bias, logit_c_decay, k_saturation, r_saturation).
# The end-to-end bf16 cases of tests/test_gpu_ops.py whose reference gaps are recorded too.
OPS_BF16_CASES = ((40, 1, 2048), (8, 64, 128), (16, 64, 2048))
CORE_VEC_BASE = (0.0, -2.25, -4.6, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 2.2, 0.0, 0.0)
SKETCHES = 4
# Scalar gradients of the core op that sum B*T*H terms (op input order 20-22).
CORE_SCALAR_GRADS = (20, 21, 22)


def bf16_gap_case(name: str):
    """(26 op inputs, 11 upstream gradients with None for the gate tape) as fp32 CPU
    tensors; Wx, Wgx, Ug and A hold bf16 values (the reference's bf16 path casts exactly
    these four, tests/test_batched_runtime.py:83-113, so its fp32 run on the same values
    differs from its bf16 run only by the bf16 arithmetic)."""
    import math

    B, T, H, seed = BF16_GAP_SHAPES[name]
    g = torch.Generator().manual_seed(seed)
    bf = lambda x: x.to(torch.bfloat16).float()  # noqa: E731
    Wx = bf(torch.randn(B, T, H, generator=g) * 0.8)
    Wgx = bf(torch.randn(B, T, H, generator=g) * 1.5 - 0.5)
    Ug = bf(torch.randn(H, H, generator=g) / math.sqrt(H))
    A = bf(torch.randn(H, H, generator=g) * 0.5 / math.sqrt(H))
    vec = [base + 0.3 * torch.randn(H, generator=g) for base in CORE_VEC_BASE]
    scal = [torch.tensor(-2.0) + 0.2 * torch.randn((), generator=g),
            torch.tensor(-1.0) + 0.2 * torch.randn((), generator=g),
            torch.tensor(-6.0) + 0.5 * torch.randn((), generator=g)]
    b0 = 0.3 * torch.randn(B, H, generator=g)
    e0 = torch.rand(B, H, generator=g) * 0.5 + 0.5
    c0 = torch.rand(B, H, generator=g) * 0.3
    inputs = [Wx, Wgx, Ug, A, *vec, *scal, b0, e0, c0]
    shapes = [(B, T, 2 * H)] + [(B, T, H)] * 7 + [(B, H)] * 3
    gout = [None if i == 7 else torch.randn(s, generator=g) for i, s in enumerate(shapes)]
    return inputs, gout


def sketch(x, seed: int) -> np.ndarray:
    """SKETCHES seeded random projections <x, R_k> in fp64: a small fingerprint that pins a
    large tensor to a recorded one (a plausible error moves it by far more than fp32
    rounding does)."""
    a = np.asarray(x, np.float64).reshape(-1)
    g = np.random.default_rng(seed)
    return np.array([float(a @ g.standard_normal(a.size)) for _ in range(SKETCHES)])


def core_oracle_case(inputs, gout):
    """The fp32 oracle's 11 outputs and 26 input gradients (op order, None where the op has
    no gradient) for op inputs and upstream gradients as CPU tensors."""
    import oracle

    x = [f32(t.numpy()) for t in inputs]
    GA = np.concatenate([x[2], x[3]], 0)
    out = oracle.core_scan_fwd(x[0], x[1], GA, x[4:20], float(x[20]), float(x[21]),
                               float(x[22]), x[23], x[24], x[25])
    saved = (out[0], out[2], out[3], out[5], out[6], out[7])
    ups = [None if gout[i] is None else f32(gout[i].numpy()) for i in (0, 1, 2, 3, 4, 5, 6, 8, 9, 10)]
    ob = oracle.core_scan_bwd(GA, x[4:20], float(x[20]), float(x[21]), float(x[22]), x[23], x[25],
                              saved, ups)
    H = x[0].shape[-1]
    grads = [ob[0], ob[1], ob[2][:H], ob[2][H:], *[ob[3][i] for i in range(16)],
             *[np.asarray(ob[4][i]) for i in range(3)], ob[5], ob[6], ob[7]]
    return list(out), grads


def bf16_gap_verdict(gaps, name: str, i: int, err: float, value=None):
    """The bf16 bar of gradient i of a core-op case recorded in core_bf16_gap.npz, given the
    HIP bf16 result's distance ``err`` from the fp32 oracle (Frobenius, relative) and, for a
    scalar gradient, its ``value``. Returns (ok, bar description).

    * tensors: err <= max(2e-2, 1.2 x the reference's own bf16 distance from fp32). Where
      the reference misses 2e-2 the distance is made of elements that cross a clamp or sign
      boundary (hard-sigmoid gate, energy and recovery clamps, the novelty sign) under bf16
      rounding; two bf16 evaluations share most such crossings but not all (37 gate
      crossings in the HIP run at B=40 T=1 H=2048 against 39 in the reference's rounding, 8
      of them not shared), so their distances from fp32 differ by up to ~20% either way.
    * the three scalar gradients that sum all B*T*H terms (logit_alpha, log_lambda,
      logit_c_suppress) cancel to a small total, so a relative distance from fp32 is
      dominated by bf16 tape rounding common to both implementations: within 2e-2 of fp32,
      or nearer to the reference's own bf16 value than that value is to fp32."""
    gap = float(gaps[f"{name}.gap_grad{i}"])
    if i in CORE_SCALAR_GRADS and value is not None:
        v16 = float(gaps[f"{name}.val16_grad{i}"])
        v32 = float(gaps[f"{name}.val32_grad{i}"])
        ok = err <= 2e-2 or abs(float(value) - v16) <= abs(v16 - v32)
        return ok, f"2e-2 or |hip - ref16| {abs(float(value) - v16):.3e} <= {abs(v16 - v32):.3e}"
    bar = max(2e-2, 1.2 * gap)
    return err <= bar, f"{bar:.3e}"
