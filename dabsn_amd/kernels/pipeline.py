"""Scan + read of one seq block, pipelined over time chunks on the two halves of the device.

Reference behaviour: the block's time-chunked scan (src/dabsn/model.py:274-307) followed by
its read over the whole sequence (read.py:139-438), and the read of a query chunk against
the bank that ends with it (read.py:650-838), which gives the same rows as the whole-sequence
read. The core scan is a persistent kernel that needs half of MI355X's CUs (128 workgroups
at B = 16, H = 2048) and is bound by its per-step exchange, so the other half is idle while
it runs. Here the scan runs on one CU-masked stream (16 CUs of every XCD, plain launches with
``coresident_cus``) and the read on the other:

* forward: the scan of chunk k + 1 runs while the read of query chunk k (its statistics,
  selection, bank gather, three-way read and output projection against the bank of
  positions [0, end of chunk k)) and the long channel over window k (its recurrent state
  carried from window k - 1) run beside it; the last chunk's read and the read output
  follow on the whole device, the last window's long channel beside them;
* backward: the read output first, the long channel's last window on the read half
  beside the last chunk's projection and read backward, then per chunk, last chunk first,
  the projection, read and long-channel backward of window k complete its tape gradients
  (its query rows, and the bank rows of window k, which only query chunks >= k read), the
  reverse scan of chunk k starts on the scan's half, and the backward of chunk k - 1 runs
  beside it, as do the core weight gradients of the windows whose reverse scans have
  finished.

Each query chunk's read is its own small autograd graph built under ``enable_grad`` inside
this function's forward, on detached leaves (the chunk's y, budget and expression windows,
the statistics rows, the write tape and the read's parameters); the backward walks those
graphs in reverse chunk order on the streams their forwards ran on. The bank-write gradient
of a chunk (its bank gather's backward) is added in place into a full-length buffer over
the bank's positions only, so no stream writes a window that the reverse scan is reading.
Outputs equal the unpipelined block's up to summation order (the read of a query chunk is
the whole-sequence read's rows; the tape gradients sum their chunk contributions).
"""

from __future__ import annotations

import atexit
import contextlib
import ctypes
import os
from typing import Optional, Sequence

import torch
import torch.nn.functional as F
from torch import Tensor

from .. import _lib, events
from . import chunked, ops

_PAIRS: dict[int, tuple] = {}
# The long channel's four coefficient logits, in the order of dabsn::long_scan_fused.
_LONG_LOGITS = ("logit_expect_retain", "logit_retention_decay", "logit_retain",
                "logit_retention_strength")


def stream_pair(device: torch.device):
    """(scan stream, read stream, CUs of the scan stream, whole-device stream) for
    ``device``: two CU-masked streams on complementary halves of the device
    (``dabsn_hip_stream_pair``) and a non-blocking stream for the pipeline's whole-device
    work, created once per device and kept for the process.

    HIP creates CU-masked streams as blocking streams: work on the legacy default stream
    waits for all of their earlier work and they wait for it. The pipeline therefore keeps
    its own work off the default stream (on the third stream) between its entry and exit
    synchronisations, or the scan half would hold the read half back."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    pair = _PAIRS.get(idx)
    if pair is None:
        lib = _lib.load()
        a, b = ctypes.c_void_p(), ctypes.c_void_p()
        ca, cb = _lib.i32(), _lib.i32()
        with torch.cuda.device(idx):
            _lib.check(lib.dabsn_hip_stream_pair(ctypes.byref(a), ctypes.byref(b), ctypes.byref(ca),
                                                 ctypes.byref(cb)), "stream pair")
        dev = torch.device("cuda", idx)
        pair = (torch.cuda.ExternalStream(a.value, device=dev),
                torch.cuda.ExternalStream(b.value, device=dev), int(ca.value),
                torch.cuda.Stream(device=dev))
        if not _PAIRS:
            atexit.register(release_streams)
        _PAIRS[idx] = pair
    return pair


def release_streams() -> None:
    """Wait for and destroy the CU-masked stream pairs (each is a hardware queue of its own).
    Registered to run at interpreter exit, ahead of the HIP runtime's own teardown: a
    process that still holds such queues when the runtime's library destructors run ends
    with a fault there under a profiler."""
    lib = _lib.load()
    for idx, (S, R, _, _) in list(_PAIRS.items()):
        with torch.cuda.device(idx):
            torch.cuda.synchronize()
            for st in (S, R):
                _lib.check(lib.dabsn_hip_stream_destroy(ctypes.c_void_p(st.cuda_stream)),
                           "stream destroy")
        del _PAIRS[idx]


@contextlib.contextmanager
def _parameters_as(module: torch.nn.Module, leaves: dict[str, Tensor]):
    """Run ``module`` with its parameters replaced by ``leaves`` (same names)."""
    saved = []
    try:
        for name, leaf in leaves.items():
            path, _, attr = name.rpartition(".")
            mod = module.get_submodule(path) if path else module
            saved.append((mod, attr, mod._parameters[attr]))
            mod._parameters[attr] = leaf
        yield
    finally:
        for mod, attr, p in reversed(saved):
            mod._parameters[attr] = p


class _SinkGather(torch.autograd.Function):
    """Bank gather over a prefix of a full-length write tape whose backward adds the bank
    rows' gradient into ``sink`` (the write tape's gradient buffer) over the bank's positions
    only, instead of returning a full-length gradient. Returns (K, V, Vn or None).
    ``wait[0]``, when an event at backward time, is waited for before the add (another
    stream's earlier writes into the same rows)."""

    @staticmethod
    def forward(ctx, sink: Tensor, write: Tensor, norm_w: Tensor, idx: Tensor,
                next_idx: Optional[Tensor], rank: Tensor, wait: list):
        lib = _lib.load()
        B, T, H = write.shape
        N = idx.shape[1]
        nw = norm_w.float().contiguous()
        ic = idx.to(torch.int64).contiguous()
        nc = None if next_idx is None else next_idx.to(torch.int64).contiguous()
        K, V = (torch.empty((B, N, H), device=write.device, dtype=write.dtype) for _ in range(2))
        Vn = None if nc is None else torch.empty_like(K)
        _lib.check(lib.dabsn_hip_bank_gather(ops._code(write.dtype), B, T, N, H, ops._p(write),
                                             ops._p(nw), ops._p(ic), ops._p(nc), ops._p(K),
                                             ops._p(V), ops._p(Vn), ops._stream(write)),
                   "bank gather")
        ctx.save_for_backward(nw, rank, K)
        ctx.sink = sink
        ctx.wait = wait
        ctx.shape = (B, T, H)
        ctx.set_materialize_grads(False)
        return K, V, Vn

    @staticmethod
    def backward(ctx, gK, gV, gVn):
        nw, rank, K = ctx.saved_tensors
        B, T, H = ctx.shape
        N = K.shape[1]
        dt = K.dtype
        z = lambda g: torch.zeros_like(K) if g is None else g.to(dt).contiguous()  # noqa: E731
        gKc, gVc = z(gK), z(gV)
        gVnc = None if gVn is None else gVn.to(dt).contiguous()
        rk = rank.to(torch.int32).contiguous()
        if ctx.wait[0] is not None:
            torch.cuda.current_stream(K.device).wait_event(ctx.wait[0])
        lib = _lib.load()
        _lib.check(lib.dabsn_hip_bank_gather_bwd_prefix(
            ops._code(dt), B, int(rk.shape[1]), T, N, H, ops._p(nw), ops._p(rk), ops._p(K),
            ops._p(gKc), ops._p(gVc), ops._p(gVnc), 1, ops._p(ctx.sink), ops._stream(K)),
            "bank gather backward")
        return None, None, None, None, None, None, None


def _stats_window(tapes: chunked._Tapes, stats: Tensor, t0: int, t1: int, stream) -> None:
    """stats[:, t0:t1] = read_tape_stats of the tapes' window [t0, t1), in place."""
    lib = _lib.load()
    B, T, H = tapes.tapes[0].shape
    o = t0 * H
    nov, pl, ay, w, en, sat = (tapes.tapes[i] for i in (0, 1, 2, 3, 4, 5))
    ptr = lambda t: t.data_ptr() + o * t.element_size()  # noqa: E731
    _lib.check(lib.dabsn_hip_tape_stats_window(
        ops._code(nov.dtype), B, t1 - t0, H, T, ptr(nov), ptr(pl), ptr(en), ptr(sat), ptr(ay),
        ptr(w), stats.data_ptr() + t0 * 6 * 4, T, stream), "tape statistics")


def _stats_bwd_window(gstats: Tensor, outs: Sequence[Optional[Tensor]], accumulate: bool,
                      t0: int, t1: int, stream) -> None:
    """Mean gradients of window [t0, t1) broadcast into the full-length gradients
    outs = (g_novelty, g_plasticity, g_energy, g_saturation) (None to skip)."""
    lib = _lib.load()
    like = next(x for x in outs if x is not None)
    B, T, H = like.shape
    o = t0 * H
    ptr = lambda t: None if t is None else t.data_ptr() + o * t.element_size()  # noqa: E731
    gs = gstats.data_ptr() + t0 * 6 * 4
    _lib.check(lib.dabsn_hip_tape_stats_bwd_window(
        ops._code(like.dtype), B, t1 - t0, H, T, gs, T, 1 if accumulate else 0, *map(ptr, outs),
        stream), "tape statistics backward")


def windows(T: int, chunk: int) -> list[tuple[int, int]]:
    """The pipeline's time windows for a block chunked every ``chunk`` steps: one window more
    than the chunks, of lengths in multiples of 128 that do not grow toward the end (the
    scan and read results do not depend on where the windows fall). The read of window k
    runs beside the scan of window k + 1 and costs more per query the later the window (the
    bank grows), while the last window's read and its backward run alone: shorter late
    windows shrink that exposed part, the extra window's fixed costs bound how short they
    get. Lengths: the 256-multiple below T / n for every window, the remainder added in
    128-step units from the front. At B=16, T=4096, H=2048, chunk 1024 (windows 896, 896,
    768, 768, 768) this measured 0.4-0.5 ms per step faster than 4 x 1024 and than the other
    five- and six-window schedules tried. Fewer than 256 steps per window: the chunks as
    they are."""
    n = -(-T // chunk) + 1
    base = (T // n) // 256 * 256
    if chunk >= T or base < 256:
        return chunked._chunks(T, chunk)
    lens = [base] * n
    extra = T - n * base
    i = 0
    while extra >= 128:
        lens[i % n] += 128
        extra -= 128
        i += 1
    lens[0] += extra
    out, t = [], 0
    for length in lens:
        out.append((t, t + length))
        t += length
    return out


def _check_scans(S, calls, what: str) -> None:
    """The scans' error words, read on the scan stream once everything is enqueued: a
    checking read then waits for the scans only (not for the read half's work), and none
    sits between two launches."""
    with torch.cuda.stream(S):
        for c in calls:
            ops._record_error_word(c.ws, what)


class _PipelinedScanRead(torch.autograd.Function):
    @staticmethod
    def forward(ctx, read, chunk: int, names: tuple, Wx: Tensor, Wgx: Tensor, *rest: Tensor):
        core_in, read_params = rest[:21], rest[21:]
        Ug, A = core_in[:2]
        vecs, scal = core_in[2:18], core_in[18:21]
        ops._require_cuda(Wx)
        B, T, H = Wx.shape
        dt = Wx.dtype
        code = ops._code(dt)
        dev = Wx.device
        S, R, cus, M = stream_pair(dev)
        ambient = torch.cuda.current_stream(dev)
        events.announce("core_scan_chunked", "rocm_pipelined_scan_read", B=B, H=H,
                        chunk=int(chunk), dtype="bf16" if code == 1 else "fp32")
        ops.core_launch_check(code, B, min(T, chunk), H, False)
        # Buffers that outlive the call come from the caller's stream, before any work.
        GA = torch.cat((Ug, A), dim=0).to(dt).contiguous()
        # Transposed copies the backward takes as they are: [Ug; A]^T for the reverse scans
        # and the output projection's weight as [3H, H] for its input-gradient product (the
        # layout hipBLASLt runs fastest), filled on the read half before its first chunk.
        W_out = read.short_read.out.weight
        GAT = torch.empty((H, 2 * H), device=dev, dtype=dt)
        WdT = torch.empty((W_out.shape[1], W_out.shape[0]), device=dev, dtype=dt)
        params, keep = ops._core_params(vecs, scal)
        Wx_c, Wgx_c, ldx = ops.scan_inputs(Wx, Wgx, dt)
        out = chunked._Tapes(Wx_c, B, T, H)
        stats = torch.empty((B, T, 6), device=dev, dtype=torch.float32)
        # Chunk-major row blocks (window k: rows [B t0, B t1), batch-major inside), kept for
        # the backward: the projection's [y, budget] input and the three-way read, each
        # window a contiguous matrix for the products that take it.
        U_rows = torch.empty((B * T, 2 * H), device=dev, dtype=dt)
        retr_rows = torch.empty((B * T, H), device=dev, dtype=dt)
        sink = torch.zeros((B, T, H), device=dev, dtype=dt)    # bank-write gradient (backward)
        gain = read_params[names.index("long_gain")]
        logits = [read_params[names.index(n)] for n in _LONG_LOGITS]
        long_state0 = read.initial_long_scan_state(B, H, device=dev)
        like = Wx.new_empty((1, 1, 1))
        read_out = torch.empty((B, T, H), device=dev,  # short + long_gain * long
                               dtype=ops._read_output_dtypes(like, like, gain)[1])
        bounds = windows(T, chunk)
        K = len(bounds)
        for st in (M, S, R):
            st.wait_stream(ambient)

        try:
            with torch.cuda.stream(M):
                # Scan of every chunk on the scan half; an event after each.
                scan_done, starts, fwd_calls = [], [], []
                with torch.cuda.stream(S):
                    zeros = torch.zeros(B, H, device=dev, dtype=torch.float32)
                    carry = [zeros, torch.ones_like(zeros), zeros.clone()]
                    for t0, t1 in bounds:
                        starts.append(torch.stack(carry))
                        f = chunked._Fwd(code, Wx_c, Wgx_c, GA, params, *carry, out, t0, t1, ldx, cus)
                        tk = ops.KernelTimer.begin("core_scan_fwd", Wx)
                        f.launch(S)
                        ops.KernelTimer.end(tk)
                        e = torch.cuda.Event()
                        e.record(S)
                        scan_done.append(e)
                        fwd_calls.append(f)
                        carry = f.finals
                    starts = torch.stack(starts)

                U = out.U
                ay, w, pl = out.tapes[2], out.tapes[3], out.tapes[1]
                # Leaves of the per-chunk read graphs, one set for the chunks read on the read
                # half and one for the last chunk's read on the whole-device stream: a leaf's
                # gradient accumulator belongs to the stream of the graph that first uses it,
                # and a gradient produced on another stream makes the engine synchronise the
                # two. The backward sums the two sets.
                def leaf_set():
                    return (w.detach().requires_grad_(True), stats.detach().requires_grad_(True),
                            {n: p.detach().requires_grad_(p.requires_grad)
                             for n, p in zip(names, read_params)})

                sets = (leaf_set(), leaf_set())
                norms = stats[..., 5]
                Wd = read.short_read.out.weight.detach().to(dt)
                bd = read.short_read.out.bias.detach().to(dt)

                sink_wait: list = [None]

                def gather(bank_write, norm_w, idx, next_idx, rank, fold):
                    return _SinkGather.apply(sink, bank_write, norm_w, idx,
                                             None if fold is not None else next_idx, rank,
                                             sink_wait)

                shorts: dict = {}

                def read_chunk(k: int, leaves):
                    # Statistics of window k, the three-way read of query chunk k against the
                    # bank [0, t1) (its own autograd graph) and, without autograd, its output
                    # projection (differentiated by hand in the backward): the [y, budget] block
                    # with the bias (enqueued while the read's host read of the bank width is
                    # in flight, so the device has it to run while the host waits), then the
                    # retrieved block added.
                    t0, t1 = bounds[k]
                    C = t1 - t0
                    st = torch.cuda.current_stream(dev)
                    _stats_window(out, stats, t0, t1, st.cuda_stream)
                    pre = []

                    def project_y_budget():
                        with torch.no_grad():
                            Uk = U_rows[B * t0:B * t1]
                            ops.window_add(Uk.view(B, C, 2 * H), U[:, t0:t1])
                            pre.append(F.linear(Uk, Wd[:, :2 * H], bd))

                    w_leaf, stats_leaf, _ = leaves
                    with torch.enable_grad(), read.during_width_read(project_y_budget):
                        # A contiguous copy of the expression window as the leaf (the read's
                        # normalisation reads it densely).
                        ay_leaf = ops.window_copy(ay[:, t0:t1]).requires_grad_(True)
                        r = read.query_bank_retrieved(
                            ay_leaf, query_stats=stats_leaf[:, t0:t1], bank_write=w_leaf,
                            bank_norms=norms, bank_stats=stats_leaf[:, :t1], query_start=t0,
                            gather=gather)
                    rd = r.detach().to(dt)
                    ops.window_add(retr_rows[B * t0:B * t1].view(B, C, H), rd)
                    sh = pre[0].addmm_(rd.reshape(B * C, H), Wd[:, 2 * H:].t())
                    shorts[k] = sh.view(B, C, H)
                    return r, ay_leaf

                # The long channel (long.py:492-579) window by window from the state the previous
                # window ends in, differentiated by hand: per window its write and plasticity
                # rows (windows of the tapes, read in place), the checkpoint its backward
                # replays from and its output, kept.
                events.announce("recurrent_long_read", "rocm_chunk_parallel_scan", B=B, T=T, H=H,
                                dtype="bf16" if code == 1 else "fp32")
                longs = []
                carried = long_state0

                def long_window(k: int) -> None:
                    nonlocal carried
                    t0, t1 = bounds[k]
                    wk, pk = w[:, t0:t1], pl[:, t0:t1]
                    lk, lf, ef, rf, ckpt = ops.long_scan_window(wk, pk, logits, *carried)
                    carried = (lf, ef, rf)
                    longs.append((wk, pk, ckpt, lk))

                def read_output(k: int) -> None:
                    # short + long_gain * long over window k, into the full-length output.
                    t0, t1 = bounds[k]
                    lk = longs[k][3]
                    lk.record_stream(torch.cuda.current_stream(dev))
                    ops.read_output_window(shorts.pop(k), lk, gain, read_out[:, t0:t1])

                chunks = []
                with _parameters_as(read, sets[0][2]):
                    with torch.cuda.stream(R):
                        GAT.copy_(GA.t())
                        WdT.copy_(W_out.detach().t())
                        for k in range(K - 1):
                            R.wait_event(scan_done[k])
                            chunks.append(read_chunk(k, sets[0]))
                            if k == K - 2:
                                r_chunks = torch.cuda.Event()
                                r_chunks.record(R)
                            long_window(k)
                            read_output(k)
                        # The last window's long channel beside the last chunk's read.
                        R.wait_event(scan_done[K - 1])
                        long_window(K - 1)
                        r_long = torch.cuda.Event()
                        r_long.record(R)
                M.wait_event(scan_done[K - 1])
                M.wait_event(r_chunks)
                with _parameters_as(read, sets[1][2]):
                    chunks.append(read_chunk(K - 1, sets[1]))
                    M.wait_event(r_long)
                    read_output(K - 1)
                M.wait_stream(S)
            _check_scans(S, fwd_calls, "core scan forward")
        finally:
            # Also when an exception leaves: the caller's stream waits for all three
            # streams, so buffers allocated on it are not reused while work still runs.
            M.wait_stream(R)
            ambient.wait_stream(S)
            ambient.wait_stream(M)
        read_out.record_stream(ambient)
        del keep

        ctx.read, ctx.chunk, ctx.names = read, chunk, names
        ctx.bounds = bounds
        ctx.meta = [(x.dtype, tuple(x.shape)) for x in (Wx, Wgx, *core_in)]
        ctx.graph = (chunks, longs, sets, sink, sink_wait)
        ctx.transposed = (GAT, WdT)
        ctx.out_dtype = read_out.dtype
        ctx.save_for_backward(Wx_c, Wgx_c, Ug, A, *vecs, *scal, starts, retr_rows, U_rows, out.U,
                              *out.tapes)
        ctx.set_materialize_grads(False)
        return U[..., :H], U[..., H:], read_out

    @staticmethod
    def backward(ctx, g_y, g_budget, g_read):
        if ctx.graph is None:
            raise RuntimeError(
                "pipelined scan + read: the backward runs once per forward (it walks and frees "
                "the per-chunk read graphs); DABSN_PIPELINE=0 gives the block a backward that "
                "can run again on a retained graph")
        saved = ctx.saved_tensors
        Wx, Wgx, Ug, A = saved[:4]
        vecs, scal = saved[4:20], saved[20:23]
        starts, retr_rows, U_rows = saved[23], saved[24], saved[25]
        fwd_out = chunked._Tapes(None, 0, 0, 0, existing=saved[26:34])
        chunks, longs, sets, sink, sink_wait = ctx.graph
        GAT, WdT = ctx.transposed
        # Leaves of the read-half chunks, and of the last chunk (whole-device stream): the
        # hand-differentiated parameters' gradients go to the first set, and the second
        # set's gradients are added to it at the end.
        (_, stats_leaf, param_leaves), (_, stats_last, last_leaves) = sets
        read = ctx.read
        B, T, H = Wx.shape
        dt = Wx.dtype
        code = ops._code(dt)
        dev = Wx.device
        S, R, cus, M = stream_pair(dev)
        ambient = torch.cuda.current_stream(dev)
        bounds = ctx.bounds
        K = len(bounds)
        ops.core_launch_check(code, B, min(T, ctx.chunk), H, True)
        params, keep = ops._core_params(vecs, scal)
        pleaves = list(param_leaves.values())
        trainable = [[p for p in s[2].values() if p.requires_grad] for s in sets]
        W = param_leaves["short_read.out.weight"]
        bias = param_leaves["short_read.out.bias"]
        # Tape gradients of the reverse scans, full length, filled window by window.
        gU = torch.empty((B, T, 2 * H), device=dev, dtype=dt)
        g_halves = [None if g is None else g.to(dt) for g in (g_y, g_budget)]
        g_nov, g_p, g_ay, g_e, g_c = (torch.empty((B, T, H), device=dev, dtype=dt)
                                      for _ in range(5))
        gWx, gWgx, day = (torch.empty((B, T, H), device=dev, dtype=dt) for _ in range(3))
        g_read = (torch.zeros((B, T, H), device=dev, dtype=ctx.out_dtype) if g_read is None
                  else g_read.to(ctx.out_dtype).contiguous())
        # The read output's gradients, window by window: the projection's and the long
        # channel's (chunk-major rows, as the forward's kept rows), and the gain's share of
        # each window.
        gs_rows = torch.empty((B * T, H), device=dev, dtype=dt)
        gl_rows = torch.empty((B * T, H), device=dev, dtype=dt)
        gain_leaf = param_leaves["long_gain"]
        gain_parts = torch.zeros((K,), device=dev, dtype=torch.float32)
        out_done = [False] * K
        # dL/d[Ug; A] summed over windows as their reverse scans finish, with the scans'
        # per-workgroup parameter partials.
        gUA_sum = torch.zeros((2 * H, H), device=dev, dtype=torch.float32)
        vec_parts: list = []
        scal_parts: list = []
        for st in (M, S, R):
            st.wait_stream(ambient)

        def fill_gU(prod: Tensor, k: int) -> None:
            # y's and budget's projection gradients (columns [0, 2H) of prod) plus their own
            # upstream gradients fill U's gradient window k.
            t0, t1 = bounds[k]
            C = t1 - t0
            for i, g_in in enumerate(g_halves):
                g_proj = prod[:, i * H:(i + 1) * H].view(B, C, H)
                dst = gU[:, t0:t1, i * H:(i + 1) * H]
                if g_in is None:
                    ops.window_add(dst, g_proj)
                elif g_in.stride(2) == 1:
                    ops.window_add(dst, g_in[:, t0:t1], g_proj)
                else:
                    torch.add(g_in[:, t0:t1], g_proj, out=dst)

        def projection_grads(k: int, u_stream=None) -> Tensor:
            # out(cat[y, budget, retrieved]) over query chunk k: the retrieved rows' gradient
            # (returned, each row contiguous for the read's backward), then the [y, budget]
            # rows' gradient into U's (on u_stream when given, after which the read's
            # backward can start).
            t0, t1 = bounds[k]
            C = t1 - t0
            gs = gs_rows[B * t0:B * t1]
            g_r = F.linear(gs, WdT[2 * H:]).view(B, C, H)
            if u_stream is None:
                fill_gU(F.linear(gs, WdT[:2 * H]), k)
                return g_r
            ready = torch.cuda.Event()
            ready.record(torch.cuda.current_stream(dev))
            u_stream.wait_event(ready)
            gs.record_stream(u_stream)
            with torch.cuda.stream(u_stream):
                fill_gU(F.linear(gs, WdT[:2 * H]), k)
            return g_r

        def core_weight_grads(k: int) -> None:
            # dL/d[Ug; A] over window k: the reverse scan's [dWgx, da_y] rows times the
            # trajectory's y rows, summed over the window's rows (one GEMM), and the scan's
            # parameter partials reduced.
            t0, t1 = bounds[k]
            y = U_rows[B * t0:B * t1, :H]
            gd = torch.empty((B, t1 - t0, 2 * H), device=dev, dtype=dt)
            ops.window_add(gd[..., :H], gWgx[:, t0:t1])
            ops.window_add(gd[..., H:], day[:, t0:t1])
            gUA_sum.add_(gd.view(-1, 2 * H).t() @ y)
            vec_parts.append(bw_of[k].part_vec.sum(0))
            scal_parts.append(bw_of[k].part_scal.sum(0))

        def read_out_backward(k: int) -> None:
            if not out_done[k]:
                t0, t1 = bounds[k]
                C = t1 - t0
                lk = longs[k][3]
                lk.record_stream(torch.cuda.current_stream(dev))
                ops.read_output_bwd_window(g_read[:, t0:t1], lk, gain_leaf,
                                           gs_rows[B * t0:B * t1].view(B, C, H),
                                           gl_rows[B * t0:B * t1].view(B, C, H),
                                           gain_parts[k:k + 1])
                out_done[k] = True

        logit_leaves = [param_leaves[n] for n in _LONG_LOGITS]
        logit_sum: list = [None]          # the four logits' gradients, summed window by window
        state_grad: list = [None, None, None]

        def long_backward(k: int) -> None:
            # Window k of the long channel: its rows' gradient plus the gradient of the state
            # it ends in (from window k + 1's backward); leaves the gradient of the state it
            # starts from for window k - 1. The write gradient is added into the sink's rows
            # (the gather backward of every query chunk >= k adds into them too) and the
            # plasticity gradient written into g_p's (the statistics backward then adds to
            # it), both in place.
            wk, pk, ckpt, _ = longs[k]
            t0, t1 = bounds[k]
            _, _, part, g0 = ops.long_scan_backward_parts(
                wk, pk, logit_leaves, ckpt, gl_rows[B * t0:B * t1].view(B, t1 - t0, H),
                *state_grad, gw_into=sink[:, t0:t1], gp_into=g_p[:, t0:t1])
            logit_sum[0] = part if logit_sum[0] is None else logit_sum[0] + part
            state_grad[:] = g0

        try:
            with torch.cuda.stream(M):
                # The read output's backward over the last window; then the long channel's last
                # window on the read half (enqueued first, so that its kernels hold their CUs)
                # beside the last chunk's projection and read backward on the whole device. The
                # other windows' long channel runs in the read half's per-chunk work (measured:
                # a second window at the head slows the last chunk's read backward by 0.45 ms,
                # more than it saves later).
                read_out_backward(K - 1)
                head = torch.cuda.Event()
                head.record(M)
                R.wait_event(head)
                with torch.cuda.stream(R):
                    # With its shares of the last window's write and plasticity gradients,
                    # ahead of the last chunk's gather backward (which waits for them) and
                    # statistics backward, off the path to the last reverse scan.
                    long_backward(K - 1)
                    last_shares = torch.cuda.Event()
                    last_shares.record(R)
                sink_wait[0] = last_shares

                carry = [None, None, None]
                bws = []
                scan_back: list[Optional[torch.cuda.Event]] = [None] * K
                bw_of: dict = {}
                for k in range(K - 1, -1, -1):
                    t0, t1 = bounds[k]
                    r, ay_leaf = chunks[k]
                    st = M if k == K - 1 else R
                    side = 1 if k == K - 1 else 0
                    with torch.cuda.stream(st):
                        read_out_backward(k)
                        # The last chunk's [y, budget] product on the scan half, idle until
                        # that chunk's reverse scan, which the scan stream's order puts after it.
                        g_r = projection_grads(k, S if k == K - 1 else None)
                        # The write leaf is listed so that the engine runs the gather's backward,
                        # whose gradient goes to the sink (it returns none for the leaf itself).
                        torch.autograd.backward([r], [g_r], inputs=[ay_leaf, sets[side][0],
                                                                     sets[side][1], *trainable[side]])
                        if ay_leaf.grad is not None:
                            ops.window_add(g_ay[:, t0:t1], ay_leaf.grad.to(dt))
                        else:
                            g_ay[:, t0:t1].zero_()
                    if st is not R:
                        done = torch.cuda.Event()
                        done.record(st)
                        R.wait_event(done)
                    with torch.cuda.stream(R):
                        if k < K - 1:
                            long_backward(k)
                        if k == K - 1:
                            # Later chunks of the read half add theirs to the last chunk's.
                            stats_leaf.grad = stats_last.grad
                        gs = stats_leaf.grad
                        gs = torch.zeros_like(stats_leaf) if gs is None else gs.contiguous()
                        _stats_bwd_window(gs, (g_nov, None, g_e, g_c), False, t0, t1, R.cuda_stream)
                        _stats_bwd_window(gs, (None, g_p, None, None), True, t0, t1, R.cuda_stream)
                        tapes_ready = torch.cuda.Event()
                        tapes_ready.record(R)
                        # The reverse scan of window k + 2 finished before that of k + 1 began.
                        if k + 2 < K:
                            R.wait_event(scan_back[k + 2])
                            core_weight_grads(k + 2)
                    with torch.cuda.stream(S):
                        S.wait_event(tapes_ready)
                        up = [gU, g_nov, g_p, g_ay, sink, g_e, g_c]
                        bw = chunked._Bwd(code, GAT, params, starts[k, 0].contiguous(),
                                          starts[k, 2].contiguous(), fwd_out, up, carry,
                                          (gWx, gWgx, day), t0, t1, cus)
                        tk = ops.KernelTimer.begin("core_scan_bwd", Wx)
                        bw.launch(S)
                        ops.KernelTimer.end(tk)
                        bws.append(bw)
                        bw_of[k] = bw
                        carry = bw.g0
                        ev = torch.cuda.Event()
                        ev.record(S)
                        scan_back[k] = ev
                with torch.cuda.stream(R):
                    # The projection's weight gradients, beside the last reverse scan (rows
                    # paired in the chunk-major order of all three).
                    gw = torch.empty((H, 3 * H), device=dev, dtype=W.dtype)
                    gw[:, :2 * H] = gs_rows.t() @ U_rows
                    gw[:, 2 * H:] = gs_rows.t() @ retr_rows
                    W.grad = gw
                    bias.grad = torch.sum(gs_rows, dim=0, dtype=torch.float32).to(bias.dtype)
                    # The read's parameter gradients are final here (every chunk's read
                    # backward has run, the last chunk's on the whole-device stream, which
                    # this stream waited for): the two leaf sets summed, the read output's
                    # gain and the long channel's logits, beside the last reverse scan
                    # rather than after it.
                    if gain_leaf.requires_grad:
                        gain_leaf.grad = gain_parts.sum().reshape(gain_leaf.shape).to(
                            gain_leaf.dtype)
                    for i, leaf in enumerate(logit_leaves):
                        if leaf.requires_grad:
                            leaf.grad = logit_sum[0][i].reshape(leaf.shape).to(leaf.dtype)
                    for n, leaf in last_leaves.items():
                        if leaf.grad is not None:
                            mine = param_leaves[n]
                            mine.grad = leaf.grad if mine.grad is None else mine.grad + leaf.grad
                    if K > 1:
                        R.wait_event(scan_back[1])
                        core_weight_grads(1)
                    # The scans' parameter partials of windows 1.. summed ahead of window 0's.
                    vec_rest = torch.stack(vec_parts).sum(0) if vec_parts else None
                    scal_rest = torch.stack(scal_parts).sum(0) if scal_parts else None
                M.wait_stream(S)
                M.wait_stream(R)
                vec_parts.clear()
                scal_parts.clear()
                core_weight_grads(0)
                gvec, gscal = vec_parts[0], scal_parts[0]
                if vec_rest is not None:
                    gvec, gscal = gvec + vec_rest, gscal + scal_rest
                core = [gWx, gWgx, gUA_sum[:H], gUA_sum[H:], *[gvec[i] for i in range(16)],
                        *[gscal[i] for i in range(3)]]
                core = [g.reshape(shape).to(dtype) for g, (dtype, shape) in zip(core, ctx.meta)]
                grads = [p.grad for p in pleaves]
            _check_scans(S, bws, "core scan backward")
        finally:
            # Also when an exception leaves: the caller's stream waits for all three
            # streams, so buffers allocated on it are not reused while work still runs.
            M.wait_stream(R)
            ambient.wait_stream(S)
            ambient.wait_stream(M)
        for g in (*core, *grads):
            if g is not None:
                g.record_stream(ambient)
        del keep
        ctx.graph = None
        return (None, None, None, *core, *grads)


def pipelined_scan_read(read, chunk: int, Wx: Tensor, Wgx: Tensor,
                        core_params: Sequence[Tensor]) -> tuple[Tensor, Tensor, Tensor]:
    """(y, budget, read output), each [B, T, H], of a seq block's core scan over
    ``chunk``-step windows from the zero state and its read, with the read of query chunk k
    overlapping the scan of chunk k + 1 (forward) and the reverse scan of chunk k
    overlapping the read backward of chunk k - 1 (backward). y and budget are the two halves
    of the trajectory U [B, T, 2H] (views), returned apart so that a caller that uses one
    of them hands back no gradient for the other. ``core_params``: the 21 parameter inputs
    of dabsn::core_scan_batched (``DABSNCore.scan_inputs()``)."""
    if read.read_geometry != "seq":
        raise ValueError("the pipelined scan + read is the seq geometry's (causal banks)")
    names = tuple(n for n, _ in read.named_parameters())
    params = [p for _, p in read.named_parameters()]
    return _PipelinedScanRead.apply(read, int(chunk), names, Wx, Wgx, *core_params, *params)


def enabled() -> bool:
    """``DABSN_PIPELINE=0`` runs the block's scan and read one after the other instead."""
    return os.environ.get("DABSN_PIPELINE", "1") != "0"


def pipeline_applies(read, Wx: Tensor, chunk: int, state: Optional[int] = None,
                     dtype: Optional[torch.dtype] = None) -> bool:
    """The pipelined path serves training of a seq block on the device with 2+ chunks whose
    scan fits one CU-masked half: the channel tiles of a batch group must be resident there
    together (fp32 beyond H = 1024 needs the whole device). ``state`` and ``dtype``: the
    scan's width and activation dtype when ``Wx`` stands for the block input."""
    if not (Wx.is_cuda and torch.is_grad_enabled() and read.read_geometry == "seq"
            and 0 < chunk < int(Wx.shape[1])):
        return False
    H = int(state if state is not None else Wx.shape[-1])
    dt = dtype if dtype is not None else Wx.dtype
    tiles = ops.core_channel_tiles(ops._code(dt), int(Wx.shape[0]), H)
    half = stream_pair(Wx.device)[2]
    if tiles > half:
        events.report_fallback(
            "core_scan_chunked", "the scan's channel tiles do not fit one half of the device",
            requested_path="rocm_pipelined_scan_read",
            selected_path="chunked scan, then the read, on the whole device",
            corrective_action="train in bf16 (16-unit tiles) or at H <= 1024 in fp32",
            H=H, dtype=str(dt), tiles=tiles, half_cus=half)
        return False
    return True
