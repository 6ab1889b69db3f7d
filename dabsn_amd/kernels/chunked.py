"""Time-chunked core scan with a checkpointed, pipelined reverse pass.

Reference behaviour: src/dabsn/model.py:274-307. The block scan runs in time chunks of
``chunk_t`` steps with the (b, e, c) state carried from chunk to chunk, and every chunk is
checkpointed, so the backward recomputes a chunk's forward scan right before running its
reverse scan. The same work is scheduled differently here: the recompute of chunk k - 1
depends only on the saved start state of that chunk, not on the reverse scan of chunk k,
so the two run as one cooperative launch on disjoint halves of the device
(``dabsn_hip_core_scan_pair``). When the device cannot hold both grids at once the two
launches run one after the other. Outputs and gradients are the same either way.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Sequence

import torch
from torch import Tensor

from .. import _lib
from . import ops


def _empty(shape, like: Tensor, dtype=None) -> Tensor:
    return torch.empty(shape, device=like.device, dtype=dtype or like.dtype)


class _Fwd:
    """Outputs, workspace and C call descriptor of one forward scan."""

    def __init__(self, code: int, Wx: Tensor, Wgx: Tensor, GA: Tensor, params, b0: Tensor,
                 e0: Tensor, c0: Tensor) -> None:
        lib = _lib.load()
        B, T, H = Wx.shape
        self.inputs = (Wx, Wgx, GA, b0, e0, c0)
        self.U = _empty((B, T, 2 * H), Wx)
        self.tapes = [_empty((B, T, H), Wx) for _ in range(7)]
        self.finals = [_empty((B, H), Wx, torch.float32) for _ in range(3)]
        nbytes = lib.dabsn_hip_core_scan_workspace_bytes(code, B, H, 0)
        self.ws = _empty((nbytes,), Wx, torch.uint8)
        self.params = params
        self.call = _lib.CoreFwdCall(
            code, B, T, H, Wx.data_ptr(), Wgx.data_ptr(), GA.data_ptr(), ctypes.pointer(params),
            b0.data_ptr(), e0.data_ptr(), c0.data_ptr(), self.U.data_ptr(),
            *[t.data_ptr() for t in self.tapes], *[f.data_ptr() for f in self.finals],
            self.ws.data_ptr(), nbytes)

    def launch(self, stream) -> None:
        c = self.call
        _lib.check(_lib.load().dabsn_hip_core_scan_fwd(
            c.dtype, c.B, c.T, c.H, c.Wx, c.Wgx, c.GA, c.params, c.b0, c.e0, c.c0, c.U, c.nov,
            c.plast, c.expr, c.write, c.energy, c.sat, c.gate, c.bF, c.eF, c.cF, c.workspace,
            c.workspace_bytes, stream), "core scan forward")


class _Bwd:
    """Outputs, workspace and C call descriptor of one reverse scan."""

    def __init__(self, code: int, GAT: Tensor, params, b0: Tensor, c0: Tensor,
                 saved: Sequence[Tensor], grads: Sequence[Optional[Tensor]],
                 gfin: Sequence[Optional[Tensor]]) -> None:
        lib = _lib.load()
        U, plast = saved[0], saved[1]
        B, T, H = plast.shape
        self.keep = (GAT, b0, c0, *saved, *[g for g in grads if g is not None],
                     *[g for g in gfin if g is not None])
        self.gWx = _empty((B, T, H), plast)
        self.gWgx = _empty((B, T, H), plast)
        self.day = _empty((B, T, H), plast)
        nbg, nwg = _lib.i64(), _lib.i64()
        _lib.check(lib.dabsn_hip_core_scan_layout(code, B, H, ctypes.byref(nbg), ctypes.byref(nwg)),
                   "core scan layout")
        self.part_vec = _empty((nbg.value, 16, H), plast, torch.float32)
        self.part_scal = _empty((nwg.value, 3), plast, torch.float32)
        self.g0 = [_empty((B, H), plast, torch.float32) for _ in range(3)]
        nbytes = lib.dabsn_hip_core_scan_workspace_bytes(code, B, H, 1)
        self.ws = _empty((nbytes,), plast, torch.uint8)
        self.params = params
        ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        self.call = _lib.CoreBwdCall(
            code, B, T, H, GAT.data_ptr(), ctypes.pointer(params), b0.data_ptr(), c0.data_ptr(),
            *[x.data_ptr() for x in saved], *[ptr(g) for g in grads], *[ptr(g) for g in gfin],
            self.gWx.data_ptr(), self.gWgx.data_ptr(), self.day.data_ptr(),
            self.part_vec.data_ptr(), self.part_scal.data_ptr(), *[g.data_ptr() for g in self.g0],
            self.ws.data_ptr(), nbytes)

    def launch(self, stream) -> None:
        c = self.call
        _lib.check(_lib.load().dabsn_hip_core_scan_bwd(
            c.dtype, c.B, c.T, c.H, c.GAT, c.params, c.b0, c.c0, c.U, c.plast, c.expr, c.energy,
            c.sat, c.gate, c.gU, c.gNov, c.gP, c.gAy, c.gW, c.gE, c.gC, c.gbF, c.geF, c.gcF,
            c.gWx, c.gWgx, c.day, c.part_vec, c.part_scal, c.gb0, c.ge0, c.gc0, c.workspace,
            c.workspace_bytes, stream), "core scan backward")


def _launch_pair(fwd: _Fwd, bwd: _Bwd, stream) -> None:
    """Recompute `fwd` while `bwd` runs; one after the other if the device is too small."""
    lib = _lib.load()
    rc = lib.dabsn_hip_core_scan_pair(ctypes.byref(fwd.call), ctypes.byref(bwd.call), stream)
    if rc == -3:  # DABSN_ERR_UNSUPPORTED: nothing was enqueued
        fwd.launch(stream)
        bwd.launch(stream)
    else:
        _lib.check(rc, "core scan pair")


def _chunks(T: int, chunk: int) -> list[tuple[int, int]]:
    return [(t0, min(T, t0 + chunk)) for t0 in range(0, T, chunk)]


class _ChunkedCoreScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx, chunk: int, *inputs: Tensor):
        Wx, Wgx, Ug, A = inputs[:4]
        vecs, scal = inputs[4:20], inputs[20:23]
        b0, e0, c0 = inputs[23:26]
        ops._require_cuda(Wx)
        B, T, H = Wx.shape
        dt = Wx.dtype
        code = ops._code(dt)
        stream = ops._stream(Wx)
        GA = torch.cat((Ug, A), dim=0).to(dt).contiguous()
        params, keep = ops._core_params(vecs, scal)
        carry = [x.float().contiguous() for x in (b0, e0, c0)]
        starts, outs = [], []
        Wx_c, Wgx_c = Wx.contiguous(), Wgx.to(dt).contiguous()
        for t0, t1 in _chunks(T, chunk):
            starts.append(torch.stack(carry))
            f = _Fwd(code, Wx_c[:, t0:t1].contiguous(), Wgx_c[:, t0:t1].contiguous(), GA, params,
                     *carry)
            tk = ops.KernelTimer.begin("core_scan_fwd", Wx)
            f.launch(stream)
            ops.KernelTimer.end(tk)
            ops._record_error_word(f.ws, "core scan forward")
            outs.append(f)
            carry = f.finals
        del keep
        U = torch.cat([f.U for f in outs], 1)
        tapes = [torch.cat([f.tapes[i] for f in outs], 1) for i in range(7)]
        finals = [f.to(x.dtype) for f, x in zip(carry, (b0, e0, c0))]
        ctx.chunk = chunk
        ctx.meta = [(x.dtype, tuple(x.shape)) for x in inputs]
        ctx.save_for_backward(Wx_c, Wgx_c, Ug, A, *vecs, *scal, torch.stack(starts))
        ctx.set_materialize_grads(False)
        return (U, *tapes, *finals)

    @staticmethod
    def backward(ctx, *grads):
        saved = ctx.saved_tensors
        Wx, Wgx, Ug, A = saved[:4]
        vecs, scal = saved[4:20], saved[20:23]
        starts = saved[23]  # [K, 3, B, H]
        B, T, H = Wx.shape
        dt = Wx.dtype
        code = ops._code(dt)
        stream = ops._stream(Wx)
        GA = torch.cat((Ug, A), dim=0).to(dt).contiguous()
        GAT = GA.t().contiguous()
        params, keep = ops._core_params(vecs, scal)
        bounds = _chunks(T, ctx.chunk)
        K = len(bounds)

        def slice_grad(g: Optional[Tensor], t0: int, t1: int) -> Optional[Tensor]:
            return None if g is None else g[:, t0:t1].to(dt).contiguous()

        def fwd_of(k: int) -> _Fwd:
            t0, t1 = bounds[k]
            return _Fwd(code, Wx[:, t0:t1].contiguous(), Wgx[:, t0:t1].contiguous(), GA, params,
                        starts[k, 0].contiguous(), starts[k, 1].contiguous(),
                        starts[k, 2].contiguous())

        carry = [None if g is None else g.float().contiguous() for g in grads[8:11]]
        gWx, gWgx = [None] * K, [None] * K
        gvec = torch.zeros((16, H), device=Wx.device, dtype=torch.float32)
        gscal = torch.zeros((3,), device=Wx.device, dtype=torch.float32)
        gUg = torch.zeros((H, H), device=Wx.device, dtype=torch.float32)
        gA = torch.zeros((H, H), device=Wx.device, dtype=torch.float32)
        rec = fwd_of(K - 1)
        tk = ops.KernelTimer.begin("core_scan_fwd", Wx)
        rec.launch(stream)
        ops.KernelTimer.end(tk)
        ops._record_error_word(rec.ws, "core scan forward")
        for k in range(K - 1, -1, -1):
            t0, t1 = bounds[k]
            up = [slice_grad(g, t0, t1) for g in grads[:7]]
            saved_k = (rec.U, rec.tapes[1], rec.tapes[2], rec.tapes[4], rec.tapes[5], rec.tapes[6])
            bw = _Bwd(code, GAT, params, starts[k, 0].contiguous(), starts[k, 2].contiguous(),
                      saved_k, up, carry)
            nxt = fwd_of(k - 1) if k > 0 else None
            if nxt is not None:
                tk = ops.KernelTimer.begin("core_scan_pair", Wx)
                _launch_pair(nxt, bw, stream)
                ops.KernelTimer.end(tk)
                ops._record_error_word(nxt.ws, "core scan forward")
            else:
                tk = ops.KernelTimer.begin("core_scan_bwd", Wx)
                bw.launch(stream)
                ops.KernelTimer.end(tk)
            ops._record_error_word(bw.ws, "core scan backward")
            gWx[k], gWgx[k] = bw.gWx, bw.gWgx
            gvec += bw.part_vec.sum(0)
            gscal += bw.part_scal.sum(0)
            y = rec.U[..., :H].reshape(-1, H)
            gUg += (bw.gWgx.reshape(-1, H).t() @ y).float()
            gA += (bw.day.reshape(-1, H).t() @ y).float()
            carry = bw.g0
            rec = nxt
        del keep
        out = [torch.cat(gWx, 1), torch.cat(gWgx, 1), gUg, gA, *[gvec[i] for i in range(16)],
               *[gscal[i] for i in range(3)], *carry]
        return (None, *[g.reshape(shape).to(dtype) for g, (dtype, shape) in zip(out, ctx.meta)])


def chunked_core_scan(chunk: int, Wx: Tensor, Wgx: Tensor, Ug: Tensor, A: Tensor,
                      *rest: Tensor) -> tuple[Tensor, ...]:
    """dabsn::core_scan_batched over time chunks of `chunk` steps (checkpointed: the
    backward recomputes each chunk's forward scan). Same 26 inputs and 11 outputs as the op."""
    if len(rest) != 22:
        raise TypeError("chunked_core_scan takes the 26 inputs of dabsn::core_scan_batched")
    if Wx.shape[1] == 0:
        return ops.core_scan_batched(Wx, Wgx, Ug, A, *rest)
    return _ChunkedCoreScan.apply(max(1, int(chunk)), Wx, Wgx, Ug, A, *rest)
