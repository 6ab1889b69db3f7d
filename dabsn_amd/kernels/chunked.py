"""Time-chunked core scan: one launch per chunk, carried state, reverse scans on kept tapes.

Reference behaviour: src/dabsn/model.py:274-307. The block scan runs in time chunks of
``chunk_t`` steps with the (b, e, c) state carried from chunk to chunk, and every chunk is
checkpointed, so the reference's backward recomputes a chunk's forward scan right before
running its reverse scan. Checkpointing is a memory policy, not part of the result, and
the three-way read needs the tapes of the whole sequence at once, so here:

* every chunk reads and writes its time window of full-length tensors in place (the C call
  descriptors carry a time stride ``ldt``), so there are no per-chunk copies or
  concatenations;
* the full-length tapes stay resident in HBM from the forward to the backward (config 4
  holds 2.3 GB of them on a 288 GB device) and every chunk's reverse scan reads its window
  there, so no chunk is recomputed.

Outputs equal the single full-length scan bit for bit; gradients equal it up to the
rounding of the carried state gradient at chunk boundaries.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Sequence

import torch
from torch import Tensor

from .. import _lib, events
from . import ops


def _ptr(t: Optional[Tensor], off: int = 0) -> Optional[int]:
    """Device address of element `off` of `t` (None for an absent tensor)."""
    return None if t is None else t.data_ptr() + off * t.element_size()


def _empty(shape, like: Tensor, dtype=None) -> Tensor:
    return torch.empty(shape, device=like.device, dtype=dtype or like.dtype)


class _Tapes:
    """Full-length forward outputs: U [B, T, 2H] and the 7 tapes [B, T, H] (novelty,
    plasticity, expression, write, energy, saturation, gate); new, or existing tensors."""

    def __init__(self, like: Tensor, B: int, T: int, H: int, existing=None) -> None:
        if existing is not None:
            self.U, self.tapes = existing[0], list(existing[1:])
            return
        self.U = _empty((B, T, 2 * H), like)
        self.tapes = [_empty((B, T, H), like) for _ in range(7)]


class _Fwd:
    """C call descriptor, workspace and final state of the forward scan of steps [t0, t1)."""

    def __init__(self, code: int, Wx: Tensor, Wgx: Tensor, GA: Tensor, params, b0: Tensor,
                 e0: Tensor, c0: Tensor, out: _Tapes, t0: int, t1: int, ldx: int,
                 coresident_cus: int = 0) -> None:
        lib = _lib.load()
        B, T, H = Wx.shape
        self.keep = (Wx, Wgx, GA, b0, e0, c0, out)
        self.finals = [_empty((B, H), Wx, torch.float32) for _ in range(3)]
        nbytes = lib.dabsn_hip_core_scan_workspace_bytes(code, B, H, 0)
        self.ws = _empty((nbytes,), Wx, torch.uint8)
        self.params = params
        o, ox = t0 * H, t0 * ldx  # first step of the window in the tapes / in Wx, Wgx
        self.call = _lib.CoreFwdCall(
            code, B, t1 - t0, H, T, ldx, _ptr(Wx, ox), _ptr(Wgx, ox), _ptr(GA),
            ctypes.pointer(params), _ptr(b0), _ptr(e0), _ptr(c0), _ptr(out.U, 2 * o),
            *[_ptr(t, o) for t in out.tapes], *[_ptr(f) for f in self.finals], _ptr(self.ws),
            nbytes)
        self.call.coresident_cus = int(coresident_cus)

    def launch(self, stream) -> None:
        _lib.check(_lib.load().dabsn_hip_core_scan_fwd_call(ctypes.byref(self.call), stream),
                   "core scan forward")


class _Bwd:
    """C call descriptor, workspace and partial sums of the reverse scan of steps [t0, t1).

    `outs` = (gWx, gWgx, day), full-length [B, T, H]; the scan writes its window of each."""

    def __init__(self, code: int, GAT: Tensor, params, b0: Tensor, c0: Tensor, src: _Tapes,
                 grads: Sequence[Optional[Tensor]], gfin: Sequence[Optional[Tensor]],
                 outs: Sequence[Tensor], t0: int, t1: int, coresident_cus: int = 0) -> None:
        lib = _lib.load()
        B, T, H = outs[0].shape
        self.keep = (GAT, b0, c0, src, *[g for g in grads if g is not None],
                     *[g for g in gfin if g is not None], *outs)
        nbg, nwg = _lib.i64(), _lib.i64()
        _lib.check(lib.dabsn_hip_core_scan_layout(code, B, H, ctypes.byref(nbg), ctypes.byref(nwg)),
                   "core scan layout")
        like = outs[0]
        self.part_vec = _empty((nbg.value, 16, H), like, torch.float32)
        self.part_scal = _empty((nwg.value, 3), like, torch.float32)
        self.g0 = [_empty((B, H), like, torch.float32) for _ in range(3)]
        nbytes = lib.dabsn_hip_core_scan_workspace_bytes(code, B, H, 1)
        self.ws = _empty((nbytes,), like, torch.uint8)
        self.params = params
        o = t0 * H
        saved = (src.tapes[1], src.tapes[2], src.tapes[4], src.tapes[5], src.tapes[6])
        self.call = _lib.CoreBwdCall(
            code, B, t1 - t0, H, T, _ptr(GAT), ctypes.pointer(params), _ptr(b0), _ptr(c0),
            _ptr(src.U, 2 * o), *[_ptr(x, o) for x in saved],
            _ptr(grads[0], 2 * o), *[_ptr(g, o) for g in grads[1:]],
            *[_ptr(g) for g in gfin], *[_ptr(x, o) for x in outs], _ptr(self.part_vec),
            _ptr(self.part_scal), *[_ptr(g) for g in self.g0], _ptr(self.ws), nbytes)
        self.call.coresident_cus = int(coresident_cus)

    def launch(self, stream) -> None:
        _lib.check(_lib.load().dabsn_hip_core_scan_bwd_call(ctypes.byref(self.call), stream),
                   "core scan backward")


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
        events.announce("core_scan_chunked", "rocm_chunked_kept_tapes", B=B, H=H,
                        chunk=int(chunk), dtype="bf16" if code == 1 else "fp32")
        ops.core_launch_check(code, B, min(T, chunk), H, False)
        GA = torch.cat((Ug, A), dim=0).to(dt).contiguous()
        params, keep = ops._core_params(vecs, scal)
        carry = [x.float().contiguous() for x in (b0, e0, c0)]
        Wx_c, Wgx_c, ldx = ops.scan_inputs(Wx, Wgx, dt)
        out = _Tapes(Wx_c, B, T, H)
        starts, calls = [], []
        for t0, t1 in _chunks(T, chunk):
            starts.append(torch.stack(carry))
            f = _Fwd(code, Wx_c, Wgx_c, GA, params, *carry, out, t0, t1, ldx)
            tk = ops.KernelTimer.begin("core_scan_fwd", Wx)
            f.launch(stream)
            ops.KernelTimer.end(tk)
            calls.append(f)
            carry = f.finals
        # Error words after every chunk is enqueued (a checking sync per chunk would leave
        # the device idle between chunks).
        for f in calls:
            ops._record_error_word(f.ws, "core scan forward")
        del keep
        finals = [f.to(x.dtype) for f, x in zip(carry, (b0, e0, c0))]
        ctx.chunk = chunk
        ctx.ldx = ldx
        ctx.meta = [(x.dtype, tuple(x.shape)) for x in inputs]
        # The forward's own outputs are kept for the backward: every chunk's reverse scan
        # reads its window of them, and the grad [Ug; A] GEMM reads y from U. Only the chunk
        # start states are added (the reverse step of a chunk's first step needs them).
        ctx.save_for_backward(Wx_c, Wgx_c, Ug, A, *vecs, *scal, torch.stack(starts), out.U,
                              *out.tapes)
        ctx.set_materialize_grads(False)
        return (out.U, *out.tapes, *finals)

    @staticmethod
    def backward(ctx, *grads):
        saved = ctx.saved_tensors
        Wx, Wgx, Ug, A = saved[:4]
        vecs, scal = saved[4:20], saved[20:23]
        starts = saved[23]  # [K, 3, B, H] chunk start states
        fwd_out = _Tapes(None, 0, 0, 0, existing=saved[24:32])
        B, T, H = Wx.shape
        dt = Wx.dtype
        code = ops._code(dt)
        stream = ops._stream(Wx)
        GA = torch.cat((Ug, A), dim=0).to(dt).contiguous()
        GAT = GA.t().contiguous()
        params, keep = ops._core_params(vecs, scal)
        bounds = _chunks(T, ctx.chunk)
        K = len(bounds)
        ops.core_launch_check(code, B, min(T, ctx.chunk), H, True)
        up = [None if g is None else g.to(dt).contiguous() for g in grads[:7]]
        carry = [None if g is None else g.float().contiguous() for g in grads[8:11]]
        gWx, gWgx, day = (_empty((B, T, H), Wx) for _ in range(3))
        gvec = torch.zeros((16, H), device=Wx.device, dtype=torch.float32)
        gscal = torch.zeros((3,), device=Wx.device, dtype=torch.float32)
        calls = []
        for k in range(K - 1, -1, -1):
            bw = _Bwd(code, GAT, params, starts[k, 0].contiguous(), starts[k, 2].contiguous(),
                      fwd_out, up, carry, (gWx, gWgx, day), *bounds[k])
            tk = ops.KernelTimer.begin("core_scan_bwd", Wx)
            bw.launch(stream)
            ops.KernelTimer.end(tk)
            calls.append(bw)
            gvec += bw.part_vec.sum(0)
            gscal += bw.part_scal.sum(0)
            carry = bw.g0
        for bw in calls:
            ops._record_error_word(bw.ws, "core scan backward")
        del keep
        # grad [Ug; A] = [gWgx; day]^T y over the whole sequence (y = first half of U).
        y = fwd_out.U.reshape(B * T, 2 * H)[:, :H]
        gUg = (gWgx.view(B * T, H).t() @ y).float()
        gA = (day.view(B * T, H).t() @ y).float()
        out = [gWx, gWgx, gUg, gA, *[gvec[i] for i in range(16)], *[gscal[i] for i in range(3)],
               *carry]
        return (None, *[g.reshape(shape).to(dtype) for g, (dtype, shape) in zip(out, ctx.meta)])


def chunked_core_scan(chunk: int, Wx: Tensor, Wgx: Tensor, Ug: Tensor, A: Tensor,
                      *rest: Tensor) -> tuple[Tensor, ...]:
    """dabsn::core_scan_batched over time chunks of `chunk` steps with the (b, e, c) state
    carried between them; the backward runs the chunks' reverse scans, last chunk first, on
    the tapes the forward kept. Same 26 inputs and 11 outputs as the op."""
    if len(rest) != 22:
        raise TypeError("chunked_core_scan takes the 26 inputs of dabsn::core_scan_batched")
    if Wx.shape[1] == 0:
        return ops.core_scan_batched(Wx, Wgx, Ug, A, *rest)
    return _ChunkedCoreScan.apply(max(1, int(chunk)), Wx, Wgx, Ug, A, *rest)
