"""fp64 autograd restatements used to pin the C oracle -- TEST INFRASTRUCTURE ONLY.

These are direct, loop-form restatements of the reference's mathematical oracles.
Their gradients come from torch autograd, independently of the hand-derived
analytic backward passes in ``dabsn_oracle.c``, so a dropped term, a wrong sign or
a transposed operand in the C backward shows up as a mismatch.

  core_loop      core.py:171-221 (DABSNCore._reference_forward_from_state loop); core_op
                 and core_module_forward wrap it as the registered op and the module
  dense_read     admitted.py:9-65 (dense-mask three-way read)
  long_loop      read.py:625-636 (DABSNRead._long_scan_from_state loop)
  linrec_loop    long.py:24-32 (_linrec_reference)
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def core_loop(Wx, Wgx, Ug, A, vec, logit_alpha, log_lambda, logit_c_suppress, b0, e0, c0):
    """Returns the 11 registered-op outputs computed by the reference loop."""
    (beta, log_kappa, logit_recover, k_s, k_y, k_b, k_n, k_bias,
     r_s, r_y, r_b, r_n, r_bias, logit_c_decay, k_c, r_c) = vec
    B, T, H = Wx.shape
    gate_alpha = torch.sigmoid(logit_alpha)
    lam = F.softplus(log_lambda)
    kappa = F.softplus(log_kappa)
    recover = torch.sigmoid(logit_recover)
    decay = torch.sigmoid(logit_c_decay)
    suppress = torch.sigmoid(logit_c_suppress)
    fused = torch.cat([Ug, A], dim=0)
    budget, energy, saturation = b0, e0, c0
    outs = {k: [] for k in ("U", "n", "p", "ay", "w", "e", "c", "s")}
    for t in range(T):
        y = torch.tanh(Wx[:, t] + budget)
        gate_rec, expression = F.linear(y, fused).chunk(2, dim=1)
        gate = F.hardsigmoid(Wgx[:, t] + gate_rec)
        novelty = torch.tanh((expression - budget).abs())
        stress = novelty * (1.0 - energy)
        saturation = decay * saturation + (1.0 - decay) * stress
        nov_eff = novelty * (1.0 - suppress * saturation)
        tb = torch.tanh(budget)
        k_sig = k_s * gate + k_y * y + k_b * tb + k_n * nov_eff + k_bias + k_c * saturation
        r_sig = r_s * gate + r_y * y + r_b * tb + r_n * nov_eff + r_bias + r_c * saturation
        write_cost = kappa * torch.exp(0.5 * torch.tanh(k_sig))
        recovery = torch.clamp(recover * torch.exp(0.5 * torch.tanh(r_sig)), 0.0, 1.0)
        plasticity = gate * energy
        outs["e"].append(energy)
        outs["c"].append(saturation)
        budget = (1.0 - gate_alpha) * budget + beta + lam * (plasticity * expression)
        energy = torch.clamp(energy + recovery * (1.0 - energy) - write_cost * plasticity, 0.0, 1.0)
        outs["U"].append(torch.cat([y, budget], dim=-1))
        outs["n"].append(novelty)
        outs["p"].append(plasticity)
        outs["ay"].append(expression)
        outs["w"].append(plasticity * expression)
        outs["s"].append(gate)
    st = {k: torch.stack(v, dim=1) for k, v in outs.items()}
    return (st["U"], st["n"], st["p"], st["ay"], st["w"], st["e"], st["c"], st["s"],
            budget, energy, saturation)


def core_op(*inputs):
    """The registered op's 26 inputs in schema order (batched_runtime.py:1507-1535) ->
    its 11 outputs, through ``core_loop``."""
    Wx, Wgx, Ug, A = inputs[:4]
    vec = inputs[4:20]
    la, ll, ls = inputs[20:23]
    b0, e0, c0 = inputs[23:26]
    return core_loop(Wx, Wgx, Ug, A, vec, la, ll, ls, b0, e0, c0)


_MODULE_VECS = ("beta", "log_kappa", "logit_recover", "k_s", "k_y", "k_b", "k_n", "k_bias",
                "r_s", "r_y", "r_b", "r_n", "r_bias", None, "k_saturation", "r_saturation")


def core_module_forward(params, x, state):
    """``DABSNCore._reference_forward_from_state`` with return_writes, return_cocktail and
    return_final_state (core.py:111-246, projections at 281-282): ``params`` maps the
    module's parameter names to tensors. Returns (trajectory, novelty, plasticity,
    expression, write, energy, saturation, final b, final e, final c)."""
    H = params["beta"].shape[0]
    Wx = F.linear(x, params["W.weight"])
    Wgx = F.linear(x, params["Wg.weight"], params["Wg.bias"])
    vec = [params[n] if n else params["logit_saturation_decay"].expand(H) for n in _MODULE_VECS]
    out = core_loop(Wx, Wgx, params["Ug.weight"], params["A.weight"], vec,
                    params["logit_alpha"].reshape(()), params["log_lambda"].reshape(()),
                    params["logit_saturation_suppress"].reshape(()), *state)
    return out[:7] + out[8:]


def _masked_softmax(scores, allow, eligible):
    masked = scores.masked_fill(~allow, float("-inf"))
    masked = masked.masked_fill(~eligible.unsqueeze(-1), 0.0)
    weights = torch.softmax(masked, dim=-1)
    return torch.where(eligible.unsqueeze(-1), weights, torch.zeros_like(weights))


def compact_masks(idx, valid, T, mode, query_offset=0, total_steps=None):
    """compact_admitted.py:176-198."""
    total = T if total_steps is None else total_steps
    B, N = idx.shape
    v = valid.unsqueeze(1)
    pos_b = idx.unsqueeze(1)
    if mode == 0:
        qp = (torch.arange(T) + query_offset).view(1, T, 1)
        allow = v & (pos_b <= qp)
        induct = v & (pos_b < qp)
    else:
        allow = v.expand(B, T, N)
        induct = (v & (pos_b < total - 1)).expand(B, T, N)
    return allow, induct, allow.any(-1), induct.any(-1)


def dense_read(q, K, V, Vn, ck, cb, kb, adm, scale, allow, induct, gains, capture=None,
               eligible=None, induct_eligible=None):
    """admitted.py:16-65 output (gains = short, pad, induct, cocktail). The row
    eligibilities default to "any slot allowed" (what the compact read derives,
    compact_admitted.py:176-198). With a ``capture`` dict, the permanent pathway's scores
    ("perm") and the scaled query-key products ("compat") are stored there with their
    gradients retained, plus the unscaled products "qk" and "cocktail_compat": the terms
    that the cocktail, scale and cocktail-gain gradients sum."""
    sg, pg, ig, cg = gains
    if eligible is None:
        eligible = allow.any(-1)
    if induct_eligible is None:
        induct_eligible = induct.any(-1)
    compat = torch.bmm(q, K.transpose(1, 2)) * scale
    cocktail_compat = torch.bmm(ck, cb.transpose(1, 2)) * cg
    content = compat + kb.unsqueeze(1)
    short = content + adm.unsqueeze(1)
    perm = content + cocktail_compat + adm.unsqueeze(1)
    if capture is not None and perm.requires_grad:
        for name, t in (("perm", perm), ("compat", compat)):
            t.retain_grad()
            capture[name] = t
        capture["qk"] = (compat / scale).detach()
        capture["cocktail_compat"] = (cocktail_compat / cg).detach() if cg else None
    ws = _masked_softmax(short, allow, eligible)
    wp = _masked_softmax(perm, allow, eligible)
    wi = _masked_softmax(short, induct, induct_eligible)
    return sg * torch.bmm(ws, V) + pg * torch.bmm(wp, V) + ig * torch.bmm(wi, Vn)


def long_loop(w, p, er, rd, ret, rs, L0, E0, R0):
    """read.py:625-636 with sigmoid-ed coefficients passed in."""
    L, E, R = L0, E0, R0
    outs = []
    for t in range(w.shape[1]):
        pe = torch.tanh((w[:, t] - E).abs())
        sal = p[:, t] * pe
        E = er * E + (1.0 - er) * w[:, t]
        R = rd * R + (1.0 - rd) * (1.0 - pe)
        eff = ret + (1.0 - ret) * rs * R
        L = eff * L + (1.0 - eff) * (sal * w[:, t])
        outs.append(L)
    return torch.stack(outs, dim=1), (L, E, R)


def linrec_loop(a, g, y0):
    """long.py:24-32."""
    y = y0
    outs = []
    for i in range(a.shape[1]):
        y = a[:, i] * y + g[:, i]
        outs.append(y)
    return torch.stack(outs, dim=1)


def permanent_loop(k, v, beta):
    """permanent.py:39-51: S = 0; per step out = S k, S += beta (v - out) k^T."""
    B, T, H = k.shape
    S = torch.zeros(B, H, H, dtype=k.dtype)
    outs = []
    for t in range(T):
        kt = k[:, t]
        r = torch.matmul(S, kt.unsqueeze(-1)).squeeze(-1)
        outs.append(r)
        S = S + (beta[:, t, None] * (v[:, t] - r)).unsqueeze(-1) * kt.unsqueeze(1)
    return torch.stack(outs, dim=1)
