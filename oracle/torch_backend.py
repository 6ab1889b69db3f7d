"""CPU kernels for the ``dabsn::`` operators backed by the CPU oracle -- TEST INFRASTRUCTURE ONLY.

Registering these lets the product's module code (DABSNCore/DABSNRead/DABSNBlock) run on
CPU tensors through the oracle, so a whole block can be compared HIP-vs-oracle end to
end. The product package never registers CPU kernels; only tests/, smoke() and the
benchmark's cpu_baseline leg import this module.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

import oracle
from oracle import autograd_ref
from dabsn_amd.kernels import ops

_DONE = False


def _np(x):
    return x.detach().float().cpu().numpy()


def _t(a, like_dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(like_dtype)


def _core_fwd(*inputs):
    Wx, Wgx, Ug, A = inputs[:4]
    vec = inputs[4:20]
    la, ll, ls = inputs[20:23]
    b0, e0, c0 = inputs[23:26]
    out = oracle.core_scan_fwd(_np(Wx), _np(Wgx), _np(torch.cat([Ug, A], 0)),
                               [_np(v) for v in vec], float(la), float(ll), float(ls),
                               _np(b0), _np(e0), _np(c0))
    dt = Wx.dtype
    res = [_t(o, dt) for o in out[:8]]
    res += [_t(o, s.dtype) for o, s in zip(out[8:], (b0, e0, c0))]
    return tuple(res)


def _core_bwd(Ug, A, vecs, la, ll, ls, ib, ic, U, plasticity, expression, energy, saturation,
              gate, gU, gn, gp, ga, gw, ge, gc, gbF, geF, gcF):
    saved = tuple(_np(x) for x in (U, plasticity, expression, energy, saturation, gate))
    grads = [None if g is None else _np(g) for g in (gU, gn, gp, ga, gw, ge, gc, gbF, geF, gcF)]
    gWx, gWgx, gGA, gvec, gscal, gb0, ge0, gc0 = oracle.core_scan_bwd(
        _np(torch.cat([Ug, A], 0)), [_np(v) for v in vecs], float(la), float(ll), float(ls),
        _np(ib), _np(ic), saved, grads)
    H = Ug.shape[0]
    dt = plasticity.dtype
    return [_t(gWx, dt), _t(gWgx, dt), _t(gGA[:H]), _t(gGA[H:]),
            *[_t(gvec[i].copy()) for i in range(16)], *[_t(np.array(gscal[i])) for i in range(3)],
            _t(gb0), _t(ge0), _t(gc0)]


def _linrec(a, g, y0):
    return _t(oracle.linrec_fwd(_np(a), _np(g), _np(y0)), a.dtype)


def _linrec_bwd(a, g, y0, gy):
    da, dg, dy = oracle.linrec_bwd(_np(a), _np(g), _np(y0), _np(gy))
    return [_t(da, a.dtype), _t(dg, g.dtype), _t(dy, y0.dtype)]


def _coef(l1, l2, l3, l4):
    return np.array([float(torch.sigmoid(x.float()).reshape(())) for x in (l1, l2, l3, l4)],
                    np.float32)


def _long(write, plasticity, l1, l2, l3, l4, L0, E0, R0):
    out, (LF, EF, RF) = oracle.long_fwd(_np(write), _np(plasticity), _coef(l1, l2, l3, l4),
                                        _np(L0), _np(E0), _np(R0))
    B, T, H = write.shape
    # The op's checkpoint [B, ceil(T/32), 3, H]; the oracle backward only needs the states
    # entering the first chunk (the initial state) and replays the rest itself.
    ckpt = torch.zeros((B, -(-T // 32), 3, H))
    if T > 0:
        ckpt[:, 0, 0] = L0.float()
        ckpt[:, 0, 1] = E0.float()
        ckpt[:, 0, 2] = R0.float()
    return _t(out, write.dtype), _t(LF), _t(EF), _t(RF), ckpt


def _long_bwd(write, plasticity, logits, checkpoint, grad_long, gLF, gEF, gRF):
    coef = _coef(*logits)
    L0, E0, R0 = (_np(checkpoint[:, 0, k]) for k in range(3))
    gw, gp, (gL0, gE0, gR0), gcoef = oracle.long_bwd(
        _np(write), _np(plasticity), coef, L0, E0, R0, _np(grad_long),
        [None if g is None else _np(g) for g in (gLF, gEF, gRF)])
    glog = gcoef * coef * (1.0 - coef)
    return [_t(gw, write.dtype), _t(gp, plasticity.dtype),
            *[_t(np.array(glog[i])) for i in range(4)], _t(gL0), _t(gE0), _t(gR0)]


_STATS_GAINS = (1.0, 0.5, -2.0, 1.0, 0.5, 0.5, 0.25, -2.0)


def _stats(nov, pl, en, sat, ay, wr):
    st = oracle.tape_stats(_np(nov), _np(pl), _np(en), _np(sat), _np(ay), _np(wr), _STATS_GAINS)
    out = np.concatenate([st["means"], st["norm_ay"][..., None], st["norm_w"][..., None]], -1)
    return _t(out)


def _stats_bwd(gstats, like):
    H = like.shape[-1]
    g = gstats.float() / H
    return [g[..., k:k + 1].expand(like.shape).to(like.dtype).contiguous() for k in (2, 3, 0, 1)]


def _normalize(x, norms):
    return (x.float() / norms.float().clamp_min(1e-12).unsqueeze(-1)).to(x.dtype)


def _normalize_grad(q, n, gq):
    """Gradient of x / max(|x|, eps) (F.normalize): (gq - q (q.gq)) / |x| above eps."""
    q64, g64 = q.astype(np.float64), gq.astype(np.float64)
    n = n.astype(np.float64)[..., None]
    dot = (q64 * g64).sum(-1, keepdims=True)
    return np.where(n > 1e-12, (g64 - q64 * dot) / np.maximum(n, 1e-12), g64 / 1e-12)


def _normalize_bwd(q, norms, gq):
    return _t(_normalize_grad(_np(q), _np(norms), _np(gq)).astype(np.float32), q.dtype)


def _select(adm, window, whole=0):
    order, counts = oracle.bank_select(_np(adm), float(window.reshape(())),
                                       floor_bf16=adm.dtype == torch.bfloat16, whole=bool(whole))
    rank = np.empty_like(order, dtype=np.int32)
    rows = np.arange(order.shape[0])[:, None]
    rank[rows, order] = np.arange(order.shape[1], dtype=np.int32)[None, :]
    return torch.from_numpy(order), torch.from_numpy(counts), torch.from_numpy(rank)


def _gather(write, norm_w, idx, next_idx, rank):
    H = write.shape[-1]
    V = torch.gather(write, 1, idx.unsqueeze(-1).expand(-1, -1, H))
    n = torch.gather(norm_w.float(), 1, idx).clamp_min(1e-12).unsqueeze(-1)
    K = (V.float() / n).to(write.dtype)
    Vn = torch.gather(write, 1, next_idx.unsqueeze(-1).expand(-1, -1, H))
    return K, V.clone(), Vn


def _gather_bwd(write, norm_w, rank, K, gK, gV, gVn):
    B, T, H = write.shape
    N = K.shape[1]
    order = np.argsort(rank.cpu().numpy().astype(np.int64), axis=1)
    idx = order[:, :N]
    next_idx = np.minimum(idx + 1, T - 1)
    nrm = np.take_along_axis(_np(norm_w), idx, 1)
    Kn = _np(K).astype(np.float64)
    gKV = _normalize_grad(Kn, nrm, _np(gK)) + _np(gV)
    gw = np.zeros((B, T, H), np.float64)
    rows = np.arange(B)[:, None]
    np.add.at(gw, (rows, idx), gKV)
    if gVn is not None:
        np.add.at(gw, (rows, next_idx), _np(gVn).astype(np.float64))
    return _t(gw.astype(np.float32), write.dtype)


def _read_args(query, K, V, Vn, ck, cb, kb, adm, scale, idx, valid, mode, sg, pg, ig, cg):
    return (_np(query), _np(K), _np(V), _np(Vn), _np(ck), _np(cb), _np(kb), _np(adm),
            float(scale.reshape(())), idx.cpu().numpy(), valid.cpu().numpy(), int(mode),
            [float(x.reshape(())) for x in (sg, pg, ig, cg)])


def _read(query, K, V, Vn, ck, cb, kb, adm, scale, idx, valid, mode, sg, pg, ig, cg):
    a = _read_args(query, K, V, Vn, ck, cb, kb, adm, scale, idx, valid, mode, sg, pg, ig, cg)
    return _t(oracle.read3_fwd(*a), query.dtype)


def _read_bwd(go, query, K, V, Vn, ck, cb, kb, adm, scale, idx, valid, mode, sg, pg, ig, cg):
    a = _read_args(query, K, V, Vn, ck, cb, kb, adm, scale, idx, valid, mode, sg, pg, ig, cg)
    g = oracle.read3_bwd(_np(go), *a)
    like = (query, K, V, Vn, ck, cb, kb, adm, scale, sg, pg, ig, cg)
    out = []
    for val, ref in zip(g, like):
        out.append(_t(np.array(val, dtype=np.float32)).reshape(ref.shape).to(ref.dtype))
    return tuple(out)


def _permanent(k, v, beta):
    return _t(oracle.permanent_fwd(_np(k), _np(v), _np(beta)), v.dtype)


def _permanent_bwd(k, v, beta, g):
    dk, dv, db = oracle.permanent_bwd(_np(k), _np(v), _np(beta), _np(g))
    return [_t(dk, k.dtype), _t(dv, v.dtype), _t(db, beta.dtype)]


def _field(inputs, patch):
    return _t(oracle.field_gather(_np(inputs), patch.cpu().numpy()), inputs.dtype)


def _field_bwd(grad_out, patch, cells):
    return _t(oracle.field_gather_bwd(_np(grad_out), patch.cpu().numpy(), cells), grad_out.dtype)


def _ce(logits, targets, ignore_index):
    lse, nll = oracle.ce_fwd(_np(logits), targets.cpu().numpy(), ignore_index)
    return _t(lse), _t(nll)


def _ce_bwd(logits, targets, ignore_index, lse, scale):
    return _t(oracle.ce_bwd(_np(logits), targets.cpu().numpy(), ignore_index, _np(lse),
                            float(scale.reshape(()))))


def _read_output(proj, long, gain):
    """The reference's expression ``out(...) + long_gain * long`` (read.py:435-438)."""
    return proj + gain * long


def _read_output_bwd(grad, long, gain, proj_dtype):
    """What autograd forms for ``proj + gain * long``: the sum passes the gradient through
    (cast to each operand's dtype), the product multiplies it by the other factor."""
    pdt = ops._DTYPE_OF_CODE[int(proj_dtype)]
    gp = grad.to(torch.result_type(gain, long))
    ggain = (gp * long).sum().reshape(gain.shape).to(gain.dtype)
    return grad.to(pdt, copy=True), (gp * gain).to(long.dtype), ggain


def _dense_floats(inputs):
    (q, K, V, Vn, ck, cb, kb, adm, scale, allow, iallow, elig, ielig, sg, pg, ig, cg) = inputs
    return [x.float() for x in (q, K, V, Vn, ck, cb, kb, adm, scale, sg, pg, ig, cg)], \
        (allow, iallow, elig, ielig)


def _dense_eval(f, masks):
    q, K, V, Vn, ck, cb, kb, adm, scale, sg, pg, ig, cg = f
    allow, iallow, elig, ielig = masks
    return autograd_ref.dense_read(q, K, V, Vn, ck, cb, kb, adm, scale, allow, iallow,
                                   (sg, pg, ig, cg), eligible=elig, induct_eligible=ielig)


def _dense_read(*inputs):
    """admitted.py:16-65 restated in fp32 (the reference's compute dtype)."""
    f, masks = _dense_floats(inputs)
    return _dense_eval(f, masks).to(inputs[0].dtype)


def _dense_read_bwd(grad_output, *inputs):
    """The analytic backward of admitted.py:126-236 in fp32 (autograd is not available
    inside an operator's kernel): the 13 float inputs' gradients in their dtypes."""
    f, (allow, iallow, elig, ielig) = _dense_floats(inputs)
    q, K, V, Vn, ck, cb, kb, adm, scale, sg, pg, ig, cg = f
    go = grad_output.float()
    compat = torch.bmm(q, K.transpose(1, 2))
    ccomp = torch.bmm(ck, cb.transpose(1, 2))
    content = compat * scale + kb.unsqueeze(1)
    short = content + adm.unsqueeze(1)
    perm = content + ccomp * cg + adm.unsqueeze(1)
    sm = autograd_ref._masked_softmax
    ws, wp, wi = sm(short, allow, elig), sm(perm, allow, elig), sm(short, iallow, ielig)
    G, Gn = torch.bmm(go, V.transpose(1, 2)), torch.bmm(go, Vn.transpose(1, 2))

    def soft_bwd(gw, w, a, e):
        d = w * (gw - (gw * w).sum(-1, keepdim=True))
        return d.masked_fill(~a, 0.0).masked_fill(~e.unsqueeze(-1), 0.0)

    ds, dp, di = soft_bwd(G * sg, ws, allow, elig), soft_bwd(G * pg, wp, allow, elig), \
        soft_bwd(Gn * ig, wi, iallow, ielig)
    D = ds + dp + di
    grads = [torch.bmm(D, K) * scale, torch.bmm(D.transpose(1, 2), q) * scale,
             torch.bmm(ws.transpose(1, 2), go) * sg + torch.bmm(wp.transpose(1, 2), go) * pg,
             torch.bmm(wi.transpose(1, 2), go) * ig, torch.bmm(dp, cb) * cg,
             torch.bmm(dp.transpose(1, 2), ck) * cg, D.sum(1), D.sum(1), (D * compat).sum(),
             (ws * G).sum(), (wp * G).sum(), (wi * Gn).sum(), (dp * ccomp).sum()]
    like = [x for i, x in enumerate(inputs) if i not in (9, 10, 11, 12)]
    return tuple(g.reshape(x.shape).to(x.dtype) for g, x in zip(grads, like))


def register() -> None:
    """Attach the oracle as the CPU kernel of every dabsn:: operator (idempotent)."""
    global _DONE
    if _DONE:
        return
    ops.core_scan_batched.register_kernel("cpu")(_core_fwd)
    ops.core_scan_batched_backward.register_kernel("cpu")(_core_bwd)
    ops.linear_recurrence.register_kernel("cpu")(_linrec)
    ops.linrec_backward.register_kernel("cpu")(_linrec_bwd)
    ops.long_scan_fused.register_kernel("cpu")(_long)
    ops.long_scan_fused_backward.register_kernel("cpu")(_long_bwd)
    ops.read_tape_stats.register_kernel("cpu")(_stats)
    ops.read_tape_stats_backward.register_kernel("cpu")(_stats_bwd)
    ops.normalize_rows.register_kernel("cpu")(_normalize)
    ops.normalize_rows_backward.register_kernel("cpu")(_normalize_bwd)
    ops.bank_select.register_kernel("cpu")(_select)
    ops.bank_gather.register_kernel("cpu")(_gather)
    ops.bank_gather_backward.register_kernel("cpu")(_gather_bwd)
    ops.admitted_three_way_read_compact_flash.register_kernel("cpu")(_read)
    ops.admitted_three_way_read_compact_flash_backward.register_kernel("cpu")(_read_bwd)
    ops.permanent_delta_scan.register_kernel("cpu")(_permanent)
    ops.permanent_delta_scan_backward.register_kernel("cpu")(_permanent_bwd)
    ops.local_field_gather.register_kernel("cpu")(_field)
    ops.local_field_gather_backward.register_kernel("cpu")(_field_bwd)
    ops.ce_rows.register_kernel("cpu")(_ce)
    ops.ce_rows_backward.register_kernel("cpu")(_ce_bwd)
    ops.read_output.register_kernel("cpu")(_read_output)
    ops.read_output_backward.register_kernel("cpu")(_read_output_bwd)
    ops.admitted_three_way_read_native.register_kernel("cpu")(_dense_read)
    ops.admitted_three_way_read_native_backward.register_kernel("cpu")(_dense_read_bwd)
    _DONE = True
