"""Registered ``dabsn::`` operators backed by the gfx950 HIP library.

Each operator keeps the reference's schema where the reference has one, so callers
written against the reference see the same boundary:

  dabsn::core_scan_batched                    batched_runtime.py:1507-1586 (26 in, 11 out)
  dabsn::_core_scan_batched_backward          new: the reference's core op has no registered
                                              backward (its autograd is a Python loop,
                                              batched_runtime.py:1589-1634)
  dabsn::linear_recurrence / _linrec_backward long.py:392-437
  dabsn::permanent_delta_scan and its backward op
                                              permanent.py:384-433
  dabsn::local_field_gather and its backward op
                                              local_field.py:208-244
  dabsn::admitted_three_way_read_compact_flash and its backward op
                                              compact_flash.py:71-107, 181-224
plus fused operators for the rest of the read (long-memory scan, tape statistics,
query normalisation, admitted-slot selection, bank gather).

Only a device ("cuda" = ROCm) kernel is registered: on a CPU tensor these ops raise
instead of silently falling back.

The operators live in the ``dabsn`` namespace, the reference's own, unless the process has
already registered the reference's operators (``dabsn::core_scan_batched`` exists when
this module is imported) or ``DABSN_AMD_OP_NAMESPACE`` names another namespace: then they
register under ``dabsn_amd`` (or the named one), a ``PROVIDER_RESOLUTION`` event records
it, and the two packages share the process. ``NAMESPACE`` holds the one in use.
"""

from __future__ import annotations

import ctypes
import os
import weakref
from typing import Callable, Optional, Sequence

import torch
from torch import Tensor

from .. import _lib, events


def _choose_namespace() -> str:
    named = os.environ.get("DABSN_AMD_OP_NAMESPACE")
    if named:
        return named
    try:
        taken = hasattr(torch.ops.dabsn, "core_scan_batched")
    except Exception:  # noqa: BLE001 - an unknown namespace reads as free
        taken = False
    return "dabsn_amd" if taken else "dabsn"


NAMESPACE = _choose_namespace()


def _q(name: str) -> str:
    """Qualified operator name in this module's namespace."""
    return f"{NAMESPACE}::{name}"


_DTYPES = {torch.float32: 0, torch.bfloat16: 1}

# Sticky device-side error words of persistent kernels (int32 [1] per device): a kernel's
# error word is OR-ed in on the device after each launch, and read by check_errors() or,
# at no extra synchronisation, together with the read's bank width (pending_error_word).
_STICKY: dict[int, Tensor] = {}


def _code(dt: torch.dtype) -> int:
    try:
        return _DTYPES[dt]
    except KeyError:
        raise TypeError(f"DABSN HIP kernels support float32 and bfloat16, not {dt}") from None


def _stream(t: Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _p(t: Optional[Tensor]) -> Optional[int]:
    """Device pointer of `t`. The caller must keep `t` referenced until the launch is
    enqueued: a temporary (e.g. ``x.contiguous()`` inline in the call) may be freed and its
    block handed to another allocation of the same call before the kernel runs."""
    return None if t is None else t.data_ptr()


def _sync_mode(input_check: bool = False) -> str:
    """How a kernel's error word is read. ``DABSN_HIP_ERROR_CHECK=sync`` reads every op's
    word right after it (one host synchronisation per op); ``deferred`` keeps every word on
    the device until ``check_errors()`` or the next read's bank-width read. Unset, the
    persistent scans' barrier word is deferred (no host synchronisation inside the scan
    ops, so they can be captured in a graph) and the words that validate caller input
    (target and patch indices) are read at once, so a bad argument raises from the call
    that received it. Under graph capture every word is deferred."""
    mode = os.environ.get("DABSN_HIP_ERROR_CHECK")
    if mode is None:
        mode = "sync" if input_check else "deferred"
    if mode == "sync" and torch.cuda.is_initialized() and torch.cuda.is_current_stream_capturing():
        return "deferred"
    return mode


def _capture_cus(device: torch.device) -> int:
    """CUs a persistent scan may assume it owns when launched as a plain kernel: all of the
    device's while the current stream is being captured into a graph (a cooperative launch
    is not recorded as such; a captured scan must not run beside other work on the device
    when the graph is replayed), else 0 (cooperative launch)."""
    if not torch.cuda.is_current_stream_capturing():
        return 0
    return int(torch.cuda.get_device_properties(device).multi_processor_count)


# Derived copies of parameters (fp32 copies of bf16 parameter vectors and scalars, the
# [Ug; A] concatenation). Streaming decode calls every op once per token with the same
# parameters, and these copies were a third of its kernel launches. Inside
# `reuse_parameter_copies()` (the carried-memory inference entry points) an entry is
# reused while every source is the same nn.Parameter object with the same storage and
# version counter: an in-place update (load_state_dict's copy included), a `.data` swap or
# a new module rebuilds it. An edit through `p.data` in place (`p.data.copy_(...)`,
# `p.data.add_(...)`, an EMA swap) leaves the version counter alone: whoever edits weights
# that way calls `parameters_changed()` before the next call. Elsewhere nothing is cached.
_DERIVED: dict[tuple, tuple] = {}
_REUSE_DEPTH = 0
# Bumped by parameters_changed(): part of every kept copy's stamp and of a carried bank's
# admission key (memory.BankStore), so both are rebuilt after such an edit.
_GENERATION = 0


def parameters_changed() -> None:
    """Declare that parameters were edited in place without their version counter moving
    (through ``p.data``): drops every kept parameter copy, and carried banks rebuild their
    admission glue and admitted-slot lists on their next use."""
    global _GENERATION
    _GENERATION += 1
    _DERIVED.clear()


def parameter_generation() -> int:
    return _GENERATION


class reuse_parameter_copies:
    """Context manager enabling the parameter-copy reuse described above."""

    def __enter__(self):
        global _REUSE_DEPTH
        _REUSE_DEPTH += 1
        return self

    def __exit__(self, *exc):
        global _REUSE_DEPTH
        _REUSE_DEPTH -= 1
        return False


def clear_parameter_copies() -> None:
    """Alias of ``parameters_changed()``."""
    parameters_changed()


def _derived(tag: str, sources: Sequence[Tensor], build: Callable[..., object]):
    if _REUSE_DEPTH == 0:
        return build(*sources)
    # Each source is a parameter or a view of one (``p.reshape(())``, ``p.expand(H)``): the
    # entry is tied to the parameter, and a view adds its geometry to the key.
    owners, key = [], [tag]
    for t in sources:
        if isinstance(t, torch.nn.Parameter):
            owners.append(t)
            key.append(id(t))
        else:
            o = t._base
            if not isinstance(o, torch.nn.Parameter):
                return build(*sources)
            owners.append(o)
            key.append((id(o), tuple(t.shape), t.stride(), t.storage_offset()))
    key = tuple(key)
    # Device pointers are unique across devices, so the pointer also stands for the device.
    stamp = (_GENERATION, tuple((o.data_ptr(), o._version, o.dtype) for o in owners))
    hit = _DERIVED.get(key)
    if hit is not None and hit[1] == stamp and all(r() is o for r, o in zip(hit[0], owners)):
        return hit[2]
    value = build(*sources)
    if len(_DERIVED) >= 4096:  # drop entries whose parameters are gone
        for k in [k for k, v in _DERIVED.items() if any(r() is None for r in v[0])]:
            del _DERIVED[k]
    # An entry goes when one of its parameters does (values hold no reference to them).
    drop = lambda _ref, k=key: _DERIVED.pop(k, None)  # noqa: E731
    _DERIVED[key] = (tuple(weakref.ref(o, drop) for o in owners), stamp, value)
    return value


def _f32(t: Tensor) -> Tensor:
    """t as a contiguous fp32 tensor (a cached copy for a bf16 parameter)."""
    if t.dtype == torch.float32 and t.is_contiguous():
        return t
    return _derived("f32", (t,), lambda x: x.detach().float().contiguous())


def _f32_scalar(t: Tensor) -> Tensor:
    return _f32(t).reshape(())


def _record_error_word(ws: Tensor, what: str, meaning: str | None = None) -> None:
    """Check a launch's error word (the first 4 bytes of ``ws``). ``meaning`` describes an
    input-validation word (see _sync_mode); without it the word is a persistent scan's
    barrier timeout."""
    word = ws[:4].view(torch.int32)
    if _sync_mode(input_check=meaning is not None) == "sync":
        value = int(word.item())
        if value != 0:
            raise RuntimeError(
                f"DABSN HIP {what}: "
                + (meaning or "a device-wide step barrier timed out; the workgroups of the "
                   "persistent scan were not all co-resident") + f" (error word {value})"
            )
        return
    sticky = _sticky(ws.device)
    torch.bitwise_or(sticky, word, out=sticky)


def _sticky(device: torch.device) -> Tensor:
    dev = device.index if device.index is not None else torch.cuda.current_device()
    sticky = _STICKY.get(dev)
    if sticky is None:
        sticky = torch.zeros(1, dtype=torch.int32, device=device)
        _STICKY[dev] = sticky
    return sticky


def pending_error_word(device: torch.device) -> Optional[Tensor]:
    """The device's sticky error word as an int64 [1] tensor (None when nothing was
    launched in deferred mode), for a caller that reads it together with another value
    in one host read."""
    dev = device.index if device.index is not None else torch.cuda.current_device()
    sticky = _STICKY.get(dev)
    return None if sticky is None else sticky.to(torch.int64)


def raise_error_word(value: int, device: torch.device) -> None:
    """Clear the device's sticky word and raise for a non-zero ``value`` read from it."""
    if value != 0:
        _sticky(device).zero_()
        raise RuntimeError(
            f"DABSN HIP kernel on {device} reported error word {value} (a persistent scan's "
            "step barrier timed out, or an index argument was out of range; see the op's "
            "documentation)")


def check_errors() -> None:
    """Raise if any kernel launched in deferred-check mode reported an error (a persistent
    scan's barrier timeout, or an out-of-range local-field patch index or target). The
    documented check point of the default deferred mode; the training read also carries
    the word along with its bank-width read."""
    for dev, sticky in _STICKY.items():
        raise_error_word(int(sticky.item()), torch.device("cuda", dev))


class KernelTimer:
    """Optional per-operator device timing: HIP events recorded on the launch stream
    around each library call (enabled by ``timing(True)``; used by the benchmark)."""

    enabled = False
    records: list = []

    @classmethod
    def begin(cls, name: str, t: Tensor):
        if not cls.enabled:
            return None
        stream = torch.cuda.current_stream(t.device)
        start = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        return (name, start, stream)

    @classmethod
    def end(cls, token) -> None:
        if token is None:
            return
        name, start, stream = token
        stop = torch.cuda.Event(enable_timing=True)
        stop.record(stream)
        cls.records.append((name, start, stop))

    @classmethod
    def summary(cls) -> dict[str, dict[str, float]]:
        torch.cuda.synchronize()
        out: dict[str, dict[str, float]] = {}
        for name, start, stop in cls.records:
            d = out.setdefault(name, {"calls": 0, "total_ms": 0.0})
            d["calls"] += 1
            d["total_ms"] += start.elapsed_time(stop)
        for d in out.values():
            d["avg_ms"] = d["total_ms"] / max(d["calls"], 1)
        return out


def timing(enabled: bool) -> None:
    KernelTimer.enabled = bool(enabled)
    KernelTimer.records = []


def _require_cuda(*tensors: Tensor) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError("DABSN HIP operators need ROCm device tensors")


# ---------------------------------------------------------------------------
# Core scan
# ---------------------------------------------------------------------------
CoreScanOutputs = tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor,
                        Tensor, Tensor]


def _separate(v: Tensor, n: int) -> list[Tensor]:
    """The n elements of a 1-D fp32 tensor as n separate scalar tensors (operator outputs
    must not alias each other), copied in one fused launch instead of n."""
    outs = [torch.empty((), device=v.device, dtype=v.dtype) for _ in range(n)]
    torch._foreach_copy_(outs, list(v.unbind(0)))
    return outs


def _core_params(vecs: Sequence[Tensor], scal: Sequence[Tensor]):
    """The kernel's parameter table (fp32 copies of the 16 vectors and 3 scalars and the
    ctypes struct pointing at them), one cache entry for all 19 parameters."""

    def build(*ts):
        vec_f = [v.detach().float().contiguous() for v in ts[:16]]
        scal_f = [x.detach().float().reshape(()).contiguous() for x in ts[16:]]
        params = _lib.CoreParams()
        for i, v in enumerate(vec_f):
            params.vec[i] = v.data_ptr()
        for i, x in enumerate(scal_f):
            params.scal[i] = x.data_ptr()
        return params, (vec_f, scal_f)

    return _derived("core_params", (*vecs, *scal), build)


# Cooperative launches per scan, by (device, dtype code, B, H, backward, one-step forward).
_LAUNCHES: dict[tuple, int] = {}


def core_launch_check(code: int, B: int, T: int, H: int, backward: bool) -> int:
    """Announce the core scan's path and report the batch-slab fallback: a batch whose
    groups of 16 rows do not all fit one cooperative launch runs as consecutive launches
    over slabs of the batch (each slab re-walks every time step). Returns the number of
    launches one scan makes."""
    key = (torch.cuda.current_device(), code, B, H, bool(backward), T == 1 and not backward)
    n = _LAUNCHES.get(key)
    if n is None:
        out = ctypes.c_int64(0)
        _lib.check(_lib.load().dabsn_hip_core_scan_launches(code, B, T, H, int(backward),
                                                            ctypes.byref(out)),
                   "core scan launch count")
        n = _LAUNCHES[key] = int(out.value)
    dtype = "bf16" if code == 1 else "fp32"
    path = ("rocm_one_step_gemm" if key[-1] else
            "rocm_cooperative_reverse_scan" if backward else "rocm_cooperative_scan")
    events.announce("core_scan", path, B=B, H=H, dtype=dtype)
    if n > 1:
        events.report_fallback(
            "core_scan", "the batch's row groups do not all fit one cooperative launch",
            requested_path="one cooperative launch per scan",
            selected_path=f"{n} consecutive cooperative launches over batch slabs",
            corrective_action="call with fewer batch rows per device (the rows are "
                              "independent, so the batch can be split across calls or GPUs)",
            B=B, H=H, dtype=dtype, backward=bool(backward))
    return n


def core_channel_tiles(code: int, B: int, H: int) -> int:
    """Workgroups of one batch group of the core scan (its channel tiles) for dtype code
    ``code`` at width ``H`` (a large number when the width is unsupported)."""
    ch, ks, nw = _lib.i32(), _lib.i32(), _lib.i32()
    rc = _lib.load().dabsn_hip_core_scan_config(code, B, H, ctypes.byref(ch), ctypes.byref(ks),
                                               ctypes.byref(nw))
    return -(-H // ch.value) if rc == 0 and ch.value > 0 else 1 << 30


def scan_inputs(Wx: Tensor, Wgx: Tensor, dt: torch.dtype) -> tuple[Tensor, Tensor, int]:
    """(Wx, Wgx, ldx) as the scan reads them: unchanged when both are row-strided views
    with unit element stride and a common time stride ldx (the two halves of one
    [B, T, 2H] projection over [W; Wg]), else contiguous copies with ldx = H."""
    B, T, H = Wx.shape
    ldx = Wx.stride(1)
    if (Wx.dtype == dt and Wgx.dtype == dt and Wx.stride(2) == 1 and Wgx.stride(2) == 1
            and Wgx.stride(1) == ldx and ldx >= H and ldx % 8 == 0
            and (B == 1 or (Wx.stride(0) == T * ldx and Wgx.stride(0) == T * ldx))):
        return Wx, Wgx, ldx
    return Wx.contiguous(), Wgx.to(dt).contiguous(), H


@torch.library.custom_op(_q("core_scan_batched"), mutates_args=(), device_types="cuda")
def core_scan_batched(
    Wx: Tensor, Wgx: Tensor, Ug: Tensor, A: Tensor, beta: Tensor, log_kappa: Tensor,
    logit_recover: Tensor, k_s: Tensor, k_y: Tensor, k_b: Tensor, k_n: Tensor, k_bias: Tensor,
    r_s: Tensor, r_y: Tensor, r_b: Tensor, r_n: Tensor, r_bias: Tensor, logit_c_decay: Tensor,
    k_c: Tensor, r_c: Tensor, logit_alpha: Tensor, log_lambda: Tensor, logit_c_suppress: Tensor,
    initial_b: Tensor, initial_e: Tensor, initial_c: Tensor,
) -> CoreScanOutputs:
    """Forward core scan (reference math core.py:171-221; CPU kernel cpu_runtime.cpp:672-837)."""
    _require_cuda(Wx)
    lib = _lib.load()
    B, T, H = Wx.shape
    if Wgx.shape != Wx.shape or Ug.shape != (H, H) or A.shape != (H, H):
        raise ValueError("batched DABSN core received incompatible tensor shapes")
    dt = Wx.dtype
    code = _code(dt)
    Wx_c, Wgx_c, ldx = scan_inputs(Wx, Wgx, dt)
    GA = _derived(f"GA:{dt}", (Ug, A), lambda u, a: torch.cat((u, a), dim=0).to(dt).contiguous())
    params, keep = _core_params(
        (beta, log_kappa, logit_recover, k_s, k_y, k_b, k_n, k_bias, r_s, r_y, r_b, r_n, r_bias,
         logit_c_decay, k_c, r_c),
        (logit_alpha, log_lambda, logit_c_suppress),
    )
    states = (initial_b, initial_e, initial_c)
    # A state carried in bf16 is read and written in bf16 by the kernels (the final state
    # rounded as the fp32 result's conversion would round it); any other mix runs in fp32.
    sdt = (torch.bfloat16 if all(x.dtype == torch.bfloat16 for x in states) else torch.float32)
    b0, e0, c0 = (x.to(sdt).contiguous() for x in states)
    for x in (b0, e0, c0):
        if x.shape != (B, H):
            raise ValueError(f"initial state must have shape {(B, H)}, got {tuple(x.shape)}")
    U = torch.empty((B, T, 2 * H), device=Wx.device, dtype=dt)
    tapes = [torch.empty((B, T, H), device=Wx.device, dtype=dt) for _ in range(7)]
    if T == 0:
        return (U, *tapes, *(s.clone() for s in states))
    finals = [torch.empty((B, H), device=Wx.device, dtype=sdt) for _ in range(3)]
    nbytes = lib.dabsn_hip_core_scan_workspace_bytes(code, B, H, 0)
    if nbytes == 0:
        raise RuntimeError(f"DABSN HIP core scan does not support H={H} for {dt}")
    core_launch_check(code, B, T, H, False)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=Wx.device)
    call = _lib.CoreFwdCall(code, B, T, H, T, ldx, _p(Wx_c), _p(Wgx_c), _p(GA),
                            ctypes.pointer(params), _p(b0), _p(e0), _p(c0), _p(U),
                            *[_p(t) for t in tapes], *[_p(f) for f in finals], _p(ws), nbytes,
                            _code(sdt), _capture_cus(Wx.device))
    tk = KernelTimer.begin("core_scan_fwd", Wx)
    rc = lib.dabsn_hip_core_scan_fwd_call(ctypes.byref(call), _stream(Wx))
    KernelTimer.end(tk)
    _lib.check(rc, "core scan forward")
    if T > 1:  # one-step scans have no step barrier that could time out
        _record_error_word(ws, "core scan forward")
    del keep
    fb, fe, fc = (f.to(s.dtype) for f, s in zip(finals, states))
    return (U, *tapes, fb, fe, fc)


@core_scan_batched.register_fake
def _core_scan_batched_fake(*inputs: Tensor) -> CoreScanOutputs:
    Wx = inputs[0]
    ib, ie, ic = inputs[-3:]
    B, T, H = Wx.shape
    sig = Wx.new_empty((B, T, H))
    return (Wx.new_empty((B, T, 2 * H)), sig, sig.clone(), sig.clone(), sig.clone(), sig.clone(),
            sig.clone(), sig.clone(), ib.new_empty(ib.shape), ie.new_empty(ie.shape),
            ic.new_empty(ic.shape))


@torch.library.custom_op(_q("_core_scan_batched_backward"), mutates_args=(),
                         device_types="cuda")
def core_scan_batched_backward(
    Ug: Tensor, A: Tensor, vecs: list[Tensor], logit_alpha: Tensor, log_lambda: Tensor,
    logit_c_suppress: Tensor, initial_b: Tensor, initial_c: Tensor, U: Tensor,
    plasticity: Tensor, expression: Tensor, energy: Tensor, saturation: Tensor, gate: Tensor,
    gU: Optional[Tensor], gnovelty: Optional[Tensor], gplasticity: Optional[Tensor],
    gexpression: Optional[Tensor], gwrite: Optional[Tensor], genergy: Optional[Tensor],
    gsaturation: Optional[Tensor], gfinal_b: Optional[Tensor], gfinal_e: Optional[Tensor],
    gfinal_c: Optional[Tensor],
) -> list[Tensor]:
    """Reverse scan of the core (reference batched_runtime.py:299-466, 1333-1504).

    Returns [gWx, gWgx, gUg, gA, 16 vector grads, 3 scalar grads, gb0, ge0, gc0] in fp32
    for parameters/states and in the tape dtype for gWx, gWgx.
    """
    _require_cuda(U)
    lib = _lib.load()
    B, T, H = plasticity.shape
    dt = plasticity.dtype
    code = _code(dt)
    if T == 0:
        z = lambda *s: torch.zeros(s, device=U.device, dtype=torch.float32)  # noqa: E731
        fin = [z(B, H) if g is None else g.float().clone() for g in (gfinal_b, gfinal_e, gfinal_c)]
        return [torch.zeros((B, 0, H), device=U.device, dtype=dt),
                torch.zeros((B, 0, H), device=U.device, dtype=dt), z(H, H), z(H, H),
                *[z(H) for _ in range(16)], *[z() for _ in range(3)], *fin]
    GAT = torch.cat((Ug, A), dim=0).to(dt).t().contiguous()
    params, keep = _core_params(vecs, (logit_alpha, log_lambda, logit_c_suppress))
    b0 = initial_b.float().contiguous()
    c0 = initial_c.float().contiguous()
    saved = [x.to(dt).contiguous() for x in (U, plasticity, expression, energy, saturation, gate)]
    grads = [None if g is None else g.to(dt).contiguous()
             for g in (gU, gnovelty, gplasticity, gexpression, gwrite, genergy, gsaturation)]
    gfin = [None if g is None else g.float().contiguous() for g in (gfinal_b, gfinal_e, gfinal_c)]
    gWx = torch.empty((B, T, H), device=U.device, dtype=dt)
    gWgx = torch.empty_like(gWx)
    day = torch.empty_like(gWx)
    nbg, nwg = _lib.i64(), _lib.i64()
    _lib.check(lib.dabsn_hip_core_scan_layout(code, B, H, ctypes.byref(nbg), ctypes.byref(nwg)),
               "core scan layout")
    part_vec = torch.empty((nbg.value, 16, H), device=U.device, dtype=torch.float32)
    part_scal = torch.empty((nwg.value, 3), device=U.device, dtype=torch.float32)
    gb0, ge0, gc0 = (torch.empty((B, H), device=U.device, dtype=torch.float32) for _ in range(3))
    nbytes = lib.dabsn_hip_core_scan_workspace_bytes(code, B, H, 1)
    core_launch_check(code, B, T, H, True)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=U.device)
    call = _lib.CoreBwdCall(code, B, T, H, T, _p(GAT), ctypes.pointer(params), _p(b0), _p(c0),
                            *[_p(x) for x in saved], *[_p(g) for g in grads],
                            *[_p(g) for g in gfin], _p(gWx), _p(gWgx), _p(day), _p(part_vec),
                            _p(part_scal), _p(gb0), _p(ge0), _p(gc0), _p(ws), nbytes,
                            _capture_cus(U.device))
    tk = KernelTimer.begin("core_scan_bwd", U)
    rc = lib.dabsn_hip_core_scan_bwd_call(ctypes.byref(call), _stream(U))
    KernelTimer.end(tk)
    _lib.check(rc, "core scan backward")
    _record_error_word(ws, "core scan backward")
    del keep
    gvec = part_vec.sum(0)
    gscal = part_scal.sum(0)
    # grad [Ug; A] = [gWgx; day]^T y: one plain GEMM per half (hipBLASLt through torch).
    tk = KernelTimer.begin("core_weight_grad_gemm", U)
    y = U[..., :H].to(dt).reshape(B * T, H)
    gUg = (gWgx.reshape(B * T, H).t() @ y).float()
    gA = (day.reshape(B * T, H).t() @ y).float()
    KernelTimer.end(tk)
    # operator outputs must not alias each other: split into separate tensors
    return [gWx, gWgx, gUg, gA, *[gvec[i].clone() for i in range(16)],
            *[gscal[i].clone() for i in range(3)], gb0, ge0, gc0]


@core_scan_batched_backward.register_fake
def _core_scan_batched_backward_fake(Ug, A, vecs, la, ll, ls, ib, ic, U, plasticity, *rest):
    B, T, H = plasticity.shape
    g = plasticity.new_empty((B, T, H))
    f = lambda *s: plasticity.new_empty(s, dtype=torch.float32)  # noqa: E731
    return [g, g.clone(), f(H, H), f(H, H), *[f(H) for _ in range(16)], *[f() for _ in range(3)],
            f(B, H), f(B, H), f(B, H)]


def _core_setup(ctx, inputs, output) -> None:
    (U, _nov, plasticity, expression, _write, energy, saturation, gate, *_finals) = output
    ctx.save_for_backward(inputs[2], inputs[3], *inputs[4:20], inputs[20], inputs[21],
                          inputs[22], inputs[23], inputs[25], U, plasticity, expression, energy,
                          saturation, gate)
    ctx.input_meta = [(x.dtype, tuple(x.shape)) for x in inputs]


def _core_backward(ctx, *grad_outputs):
    saved = ctx.saved_tensors
    Ug, A = saved[0], saved[1]
    vecs = list(saved[2:18])
    la, ll, ls, ib, ic = saved[18:23]
    U, plasticity, expression, energy, saturation, gate = saved[23:29]
    g = list(grad_outputs)
    # the gate tape (output 7) has no gradient path in the reference op (batched_runtime.py:1619-1627)
    grads = core_scan_batched_backward(
        Ug, A, vecs, la, ll, ls, ib, ic, U, plasticity, expression, energy, saturation, gate,
        g[0], g[1], g[2], g[3], g[4], g[5], g[6], g[8], g[9], g[10])
    out = []
    for value, (dtype, shape) in zip(grads, ctx.input_meta):
        out.append(value.reshape(shape).to(dtype))
    return tuple(out)


torch.library.register_autograd(_q("core_scan_batched"), _core_backward,
                                setup_context=_core_setup)


# ---------------------------------------------------------------------------
# Linear recurrence (drop-in for dabsn::linear_recurrence)
# ---------------------------------------------------------------------------
@torch.library.custom_op(_q("linear_recurrence"), mutates_args=(), device_types="cuda")
def linear_recurrence(a: Tensor, g: Tensor, y_init: Tensor) -> Tensor:
    """y_t = a_t y_{t-1} + g_t (reference long.py:392-396; CPU cpu_runtime.cpp:92-108)."""
    _require_cuda(a)
    lib = _lib.load()
    if a.dim() != 3 or g.shape != a.shape or y_init.shape != (a.shape[0], a.shape[2]):
        raise ValueError("expected a/g [B,T,H] and y_init [B,H]")
    dt = a.dtype
    B, T, H = a.shape
    a_c, g_c, y0 = a.contiguous(), g.to(dt).contiguous(), y_init.to(dt).contiguous()
    out = torch.empty_like(a_c)
    _lib.check(lib.dabsn_hip_linrec_fwd(_code(dt), B, T, H, _p(a_c), _p(g_c), _p(y0), _p(out),
                                        _stream(a)), "linear recurrence")
    return out


@linear_recurrence.register_fake
def _linear_recurrence_fake(a, g, y_init):
    if a.dim() != 3 or g.shape != a.shape or y_init.shape != (a.shape[0], a.shape[2]):
        raise ValueError("expected a/g [B,T,H] and y_init [B,H]")
    return torch.empty_like(a)


@torch.library.custom_op(_q("_linrec_backward"), mutates_args=(), device_types="cuda")
def linrec_backward(a: Tensor, g: Tensor, y_init: Tensor, grad_out: Tensor) -> list[Tensor]:
    """Analytic reverse of the linear recurrence (reference long.py:58-98, 410-417)."""
    _require_cuda(a)
    lib = _lib.load()
    dt = a.dtype
    B, T, H = a.shape
    a_c, g_c, y0, gy = (x.to(dt).contiguous() for x in (a, g, y_init, grad_out))
    da, dg, dy0 = torch.empty_like(a_c), torch.empty_like(a_c), torch.empty_like(y0)
    nbytes = lib.dabsn_hip_linrec_workspace_bytes(_code(dt), B, T, H)
    ws = torch.empty(max(nbytes, 4), dtype=torch.uint8, device=a.device)
    _lib.check(lib.dabsn_hip_linrec_bwd(_code(dt), B, T, H, _p(a_c), _p(g_c), _p(y0), _p(gy),
                                        _p(da), _p(dg), _p(dy0), _p(ws), nbytes, _stream(a)),
               "linear recurrence backward")
    return [da, dg.to(g.dtype), dy0.to(y_init.dtype)]


@linrec_backward.register_fake
def _linrec_backward_fake(a, g, y_init, grad_out):
    return [torch.empty_like(a), torch.empty_like(g), torch.empty_like(y_init)]


def _linrec_setup(ctx, inputs, output):
    ctx.save_for_backward(*inputs)


def _linrec_bwd(ctx, grad_out):
    a, g, y0 = ctx.saved_tensors
    da, dg, dy = linrec_backward(a, g, y0, grad_out.contiguous())
    return da, dg, dy


torch.library.register_autograd(_q("linear_recurrence"), _linrec_bwd, setup_context=_linrec_setup)


# ---------------------------------------------------------------------------
# Permanent associative delta scan (drop-in for dabsn::permanent_delta_scan)
# ---------------------------------------------------------------------------
def _permanent_shapes(k: Tensor, v: Tensor, beta: Tensor) -> tuple[int, int, int]:
    if k.dim() != 3 or v.shape != k.shape or beta.shape != k.shape[:2]:
        raise ValueError("expected k/v [B,T,H] and beta [B,T]")
    return tuple(int(x) for x in k.shape)


@torch.library.custom_op(_q("permanent_delta_scan"), mutates_args=(), device_types="cuda")
def permanent_delta_scan(k: Tensor, v: Tensor, beta: Tensor) -> Tensor:
    """out_t = S k_t, S += beta_t (v_t - out_t) k_t^T from S = 0 (reference permanent.py:39-51,
    op 384-397; CPU cpu_runtime.cpp:1075-1109). fp32 state and arithmetic; the output takes
    v's dtype."""
    _require_cuda(k)
    B, T, H = _permanent_shapes(k, v, beta)
    lib = _lib.load()
    kf, vf, bf = (x.float().contiguous() for x in (k, v, beta))
    out = torch.empty((B, T, H), device=k.device, dtype=torch.float32)
    tk = KernelTimer.begin("permanent_scan_fwd", k)
    _lib.check(lib.dabsn_hip_permanent_scan_fwd(B, T, H, _p(kf), _p(vf), _p(bf), _p(out),
                                                _stream(k)), "permanent scan")
    KernelTimer.end(tk)
    return out.to(v.dtype)


@permanent_delta_scan.register_fake
def _permanent_delta_scan_fake(k, v, beta):
    _permanent_shapes(k, v, beta)
    return torch.empty_like(v)


@torch.library.custom_op(_q("_permanent_delta_scan_backward"), mutates_args=(),
                         device_types="cuda")
def permanent_delta_scan_backward(k: Tensor, v: Tensor, beta: Tensor,
                                  grad_out: Tensor) -> list[Tensor]:
    """Analytic reverse of the delta scan (reference permanent.py:70-119, 403-426; CPU
    cpu_runtime.cpp:1112-1188): (dk, dv, dbeta) in the inputs' dtypes."""
    _require_cuda(k)
    B, T, H = _permanent_shapes(k, v, beta)
    lib = _lib.load()
    kf, vf, bf, gf = (x.float().contiguous() for x in (k, v, beta, grad_out))
    dk, dv = torch.empty_like(kf), torch.empty_like(vf)
    db = torch.empty_like(bf)
    nbytes = lib.dabsn_hip_permanent_scan_workspace_bytes(B, T, H)
    ws = torch.empty(max(nbytes, 4), dtype=torch.uint8, device=k.device)
    tk = KernelTimer.begin("permanent_scan_bwd", k)
    _lib.check(lib.dabsn_hip_permanent_scan_bwd(B, T, H, _p(kf), _p(vf), _p(bf), _p(gf), _p(dk),
                                                _p(dv), _p(db), _p(ws), nbytes, _stream(k)),
               "permanent scan backward")
    KernelTimer.end(tk)
    return [dk.to(k.dtype), dv.to(v.dtype), db.to(beta.dtype)]


@permanent_delta_scan_backward.register_fake
def _permanent_delta_scan_backward_fake(k, v, beta, grad_out):
    return [torch.empty_like(k), torch.empty_like(v), torch.empty_like(beta)]


def _permanent_setup(ctx, inputs, output):
    ctx.save_for_backward(*inputs)


def _permanent_bwd(ctx, grad_out):
    k, v, beta = ctx.saved_tensors
    dk, dv, db = permanent_delta_scan_backward(k, v, beta, grad_out.contiguous())
    return dk, dv, db


torch.library.register_autograd(_q("permanent_delta_scan"), _permanent_bwd,
                                setup_context=_permanent_setup)


# ---------------------------------------------------------------------------
# Local field patch gather (drop-in for dabsn::local_field_gather)
# ---------------------------------------------------------------------------
_FIELD_INDEX_ERROR = "a patch index lies outside [0, N)"


def _field_shapes(inputs: Tensor, patch: Tensor) -> tuple[int, int, int, int, int]:
    if inputs.dim() != 3 or patch.dim() != 2:
        raise ValueError("expected inputs [B,N,D] and patch [N,K]")
    B, N, D = (int(x) for x in inputs.shape)
    P, K = (int(x) for x in patch.shape)
    return B, N, D, P, K


def _field_dtype(t: Tensor) -> torch.dtype:
    """Storage dtype of the HIP kernels for t: fp32 and bf16 natively, fp16 through fp32."""
    if t.dtype in (torch.float32, torch.bfloat16):
        return t.dtype
    if t.dtype == torch.float16:
        return torch.float32
    raise TypeError(f"local field gather on the HIP path supports fp32/bf16/fp16, not {t.dtype}")


@torch.library.custom_op(_q("local_field_gather"), mutates_args=(), device_types="cuda")
def local_field_gather(inputs: Tensor, patch: Tensor) -> Tensor:
    """inputs[:, patch] -> [B, P, K, D] (reference local_field.py:208-214; CPU
    cpu_runtime.cpp:1191-1211)."""
    _require_cuda(inputs)
    B, N, D, P, K = _field_shapes(inputs, patch)
    lib = _lib.load()
    dt = _field_dtype(inputs)
    x = inputs.to(dt).contiguous()
    idx = patch.to(device=inputs.device, dtype=torch.int64).contiguous()
    out = torch.empty((B, P, K, D), device=inputs.device, dtype=dt)
    nbytes = lib.dabsn_hip_local_field_workspace_bytes(N, P, K, 0)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=inputs.device)
    tk = KernelTimer.begin("local_field_gather", inputs)
    _lib.check(lib.dabsn_hip_local_field_gather(_code(dt), B, N, D, P, K, _p(x), _p(idx), _p(out),
                                                _p(ws), nbytes, _stream(inputs)),
               "local field gather")
    KernelTimer.end(tk)
    _record_error_word(ws, "local field gather", _FIELD_INDEX_ERROR)
    return out.to(inputs.dtype)


@local_field_gather.register_fake
def _local_field_gather_fake(inputs, patch):
    B, N, D, P, K = _field_shapes(inputs, patch)
    return inputs.new_empty((B, P, K, D))


@torch.library.custom_op(_q("_local_field_gather_backward"), mutates_args=(),
                         device_types="cuda")
def local_field_gather_backward(grad_out: Tensor, patch: Tensor, cells: int) -> Tensor:
    """Scatter-add of grad_out [B, P, K, D] into [B, cells, D], each source cell summed over
    its entries in increasing (p, j) order (reference local_field.py:230-236; CPU
    cpu_runtime.cpp:1214-1237)."""
    _require_cuda(grad_out)
    B, P, K, D = (int(x) for x in grad_out.shape)
    if tuple(patch.shape) != (P, K):
        raise ValueError("patch does not match grad_out")
    lib = _lib.load()
    dt = _field_dtype(grad_out)
    g = grad_out.to(dt).contiguous()
    idx = patch.to(device=grad_out.device, dtype=torch.int64).contiguous()
    gx = torch.empty((B, cells, D), device=grad_out.device, dtype=dt)
    nbytes = lib.dabsn_hip_local_field_workspace_bytes(cells, P, K, 1)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=grad_out.device)
    tk = KernelTimer.begin("local_field_scatter", grad_out)
    _lib.check(lib.dabsn_hip_local_field_gather_bwd(_code(dt), B, cells, D, P, K, _p(g), _p(idx),
                                                    _p(gx), _p(ws), nbytes, _stream(grad_out)),
               "local field gather backward")
    KernelTimer.end(tk)
    _record_error_word(ws, "local field gather backward", _FIELD_INDEX_ERROR)
    return gx.to(grad_out.dtype)


@local_field_gather_backward.register_fake
def _local_field_gather_backward_fake(grad_out, patch, cells):
    return grad_out.new_empty((grad_out.shape[0], cells, grad_out.shape[3]))


def _field_setup(ctx, inputs, output):
    values, patch = inputs
    ctx.save_for_backward(patch)
    ctx.cells = int(values.shape[1])


def _field_bwd(ctx, grad_out):
    (patch,) = ctx.saved_tensors
    return local_field_gather_backward(grad_out.contiguous(), patch, ctx.cells), None


torch.library.register_autograd(_q("local_field_gather"), _field_bwd, setup_context=_field_setup)


# ---------------------------------------------------------------------------
# Key bias, admission and cocktail from tape statistics (no autograd)
# ---------------------------------------------------------------------------
def means_glue(stats: Tensor, hidden: int, params: Sequence[Tensor],
               tape_dtype: torch.dtype = torch.float32) -> tuple[Tensor, Tensor, Tensor]:
    """(key_bias [B, N], admission [B, N], cocktail [B, N, 4]) of statistics rows
    ``stats`` [B, N, 6] (rows contiguous within a batch row; the batch stride may be
    longer, e.g. the live prefix of a bank buffer): read.py:58-72, 155-180, 680-700 in one
    kernel, for callers without autograd. ``params`` = (p_gain, novelty_gain, null_bias,
    adm_p_gain, adm_novelty_gain, adm_saturation_gain, adm_energy_gain, adm_bias).

    The values are those of the reference's expressions in the dtype they run in there:
    with bf16 tapes (``tape_dtype``) the means and tape-dtype intermediates are bf16, and
    with bf16 gains as well every step is; the outputs are returned as fp32 holding those
    values."""
    _require_cuda(stats)
    if stats.dim() != 3 or stats.shape[-1] != 6 or stats.dtype != torch.float32 \
            or stats.stride(2) != 1 or stats.stride(1) != 6:
        raise ValueError("means_glue: stats must be fp32 [B, N, 6] with contiguous rows")
    B, N, _ = (int(d) for d in stats.shape)
    lib = _lib.load()
    prm = [_f32_scalar(x) for x in params]
    kb = torch.empty((B, N), device=stats.device, dtype=torch.float32)
    adm = torch.empty_like(kb)
    ck = torch.empty((B, N, 4), device=stats.device, dtype=torch.float32)
    ptrs = _lib.PTR8(*[x.data_ptr() for x in prm])
    mode = 0
    if tape_dtype == torch.bfloat16:
        mode = 1 | (2 if all(x.dtype == torch.bfloat16 for x in params) else 0)
    _lib.check(lib.dabsn_hip_means_glue(B, N, int(stats.stride(0)), _p(stats), int(hidden), ptrs,
                                        mode, _p(kb), _p(adm), _p(ck), _stream(stats)),
               "means glue")
    return kb, adm, ck


def glue_mode(tape_dtype: torch.dtype, params: Sequence[Tensor]) -> int:
    """The dtype code of the glue kernels: bit 0 = bf16 tapes, bit 1 = bf16 gains too."""
    if tape_dtype != torch.bfloat16:
        return 0
    return 1 | (2 if all(x.dtype == torch.bfloat16 for x in params) else 0)


def _stats_rows(stats: Tensor) -> Tensor:
    """Statistics rows as the glue kernels read them: fp32 [B, L, 6] with contiguous rows
    (any batch stride)."""
    if (stats.dim() != 3 or stats.shape[-1] != 6 or stats.dtype != torch.float32
            or stats.stride(2) != 1 or stats.stride(1) != 6):
        stats = stats.float().contiguous()
    return stats


class _SlotGlue(torch.autograd.Function):
    """(key bias [B, N], admission [B, N], cocktail [B, N, 4]) of the bank rows idx of
    ``bank_stats`` and the cocktails [B, C, 4] of ``query_stats`` (read.py:58-72, 155-183,
    241-256), with the statistics rows' and the eight gains' gradients."""

    @staticmethod
    def forward(ctx, bank_stats: Tensor, query_stats: Tensor, idx: Tensor, hidden: int, mode: int,
                *params: Tensor):
        lib = _lib.load()
        bs, qs = _stats_rows(bank_stats), _stats_rows(query_stats)
        B, L, _ = bs.shape
        C = qs.shape[1]
        N = idx.shape[1]
        ic = idx.to(torch.int64).contiguous()
        prm = [_f32_scalar(x) for x in params]
        ptrs = _lib.PTR8(*[x.data_ptr() for x in prm])
        kb = torch.empty((B, N), device=bs.device, dtype=torch.float32)
        adm = torch.empty_like(kb)
        cb = torch.empty((B, N, 4), device=bs.device, dtype=torch.float32)
        ck = torch.empty((B, C, 4), device=bs.device, dtype=torch.float32)
        st = _stream(bs)
        _lib.check(lib.dabsn_hip_glue_slots(B, N, L, int(bs.stride(0)), _p(bs), _p(ic), int(hidden),
                                            ptrs, mode, _p(kb), _p(adm), _p(cb), st), "slot glue")
        _lib.check(lib.dabsn_hip_means_glue(B, C, int(qs.stride(0)), _p(qs), int(hidden), ptrs, mode,
                                            None, None, _p(ck), st), "query cocktail")
        ctx.save_for_backward(bs, qs, ic, *prm)
        ctx.hidden, ctx.mode = int(hidden), int(mode)
        ctx.meta = [(x.dtype, tuple(x.shape)) for x in params]
        ctx.set_materialize_grads(False)
        return kb, adm, cb, ck

    @staticmethod
    def backward(ctx, gkb, gadm, gcb, gck):
        bs, qs, ic, *prm = ctx.saved_tensors
        lib = _lib.load()
        B, L, _ = bs.shape
        C = qs.shape[1]
        N = ic.shape[1]
        z = lambda g, shape: (torch.zeros(shape, device=bs.device, dtype=torch.float32) if g is None  # noqa: E731
                              else g.float().contiguous())
        gkb, gadm = z(gkb, (B, N)), z(gadm, (B, N))
        gcb, gck = z(gcb, (B, N, 4)), z(gck, (B, C, 4))
        gbank = torch.zeros((B, L, 6), device=bs.device, dtype=torch.float32)
        gquery = torch.zeros((B, C, 6), device=bs.device, dtype=torch.float32)
        partial = torch.empty(max(lib.dabsn_hip_glue_slots_partials(B, N) // 4, 1),
                              device=bs.device, dtype=torch.float32)
        gparams = torch.empty((8,), device=bs.device, dtype=torch.float32)
        ptrs = _lib.PTR8(*[x.data_ptr() for x in prm])
        st = _stream(bs)
        _lib.check(lib.dabsn_hip_glue_slots_bwd(
            B, N, L, int(bs.stride(0)), _p(bs), _p(ic), ctx.hidden, ptrs, ctx.mode, _p(gkb),
            _p(gadm), _p(gcb), _p(gbank), 6 * L, _p(partial), _p(gparams), st), "slot glue backward")
        _lib.check(lib.dabsn_hip_glue_rows_bwd(B, C, int(qs.stride(0)), _p(qs), ctx.mode, _p(gck),
                                               _p(gquery), 6 * C, st), "query cocktail backward")
        gp = [gparams[k].reshape(shape).to(dtype) for k, (dtype, shape) in enumerate(ctx.meta)]
        return (gbank, gquery, None, None, None, *gp)


def slot_glue(bank_stats: Tensor, query_stats: Tensor, idx: Tensor, hidden: int,
              params: Sequence[Tensor], tape_dtype: torch.dtype) -> tuple[Tensor, ...]:
    """The read's per-slot glue in one kernel and its backward in two (see _SlotGlue):
    returns (key bias, admission, bank cocktail [B, N, 4], query cocktail [B, C, 4]) as
    fp32 holding the values of the reference's expressions in their dtypes. ``params`` =
    (p_gain, novelty_gain, null_bias, adm_p_gain, adm_novelty_gain, adm_saturation_gain,
    adm_energy_gain, adm_bias)."""
    _require_cuda(bank_stats)
    return _SlotGlue.apply(bank_stats, query_stats, idx, int(hidden),
                           glue_mode(tape_dtype, params), *params)


# ---------------------------------------------------------------------------
# Cross-entropy row kernels of the chunked readout loss (loss.py)
# ---------------------------------------------------------------------------
_TARGET_ERROR = "a target lies outside [0, V) and is not ignore_index"


def _ce_logits(logits: Tensor) -> Tensor:
    if logits.dim() != 2:
        raise ValueError("expected logits [rows, V]")
    if logits.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"cross-entropy rows on the HIP path take fp32/bf16 logits, not {logits.dtype}")
    return logits if logits.stride(1) == 1 else logits.contiguous()


@torch.library.custom_op(_q("_ce_rows"), mutates_args=(), device_types="cuda")
def ce_rows(logits: Tensor, targets: Tensor, ignore_index: int) -> tuple[Tensor, Tensor]:
    """Per row of logits [rows, V]: (logsumexp, lse - logit[target] or 0 where ignored), fp32
    (reference loss.py:83-93 for one chunk)."""
    _require_cuda(logits)
    x = _ce_logits(logits)
    rows, V = (int(d) for d in x.shape)
    lib = _lib.load()
    t = targets.to(device=x.device, dtype=torch.int64).contiguous()
    lse = torch.empty(rows, device=x.device, dtype=torch.float32)
    nll = torch.empty_like(lse)
    err = torch.zeros(1, device=x.device, dtype=torch.int32)
    tk = KernelTimer.begin("ce_rows_fwd", x)
    _lib.check(lib.dabsn_hip_ce_fwd(_code(x.dtype), rows, V, _p(x), int(x.stride(0)) if rows else V,
                                    _p(t), int(ignore_index), _p(lse), _p(nll), _p(err),
                                    _stream(x)), "cross entropy")
    KernelTimer.end(tk)
    _record_error_word(err, "cross entropy", _TARGET_ERROR)
    return lse, nll


@ce_rows.register_fake
def _ce_rows_fake(logits, targets, ignore_index):
    rows = logits.shape[0]
    return (logits.new_empty((rows,), dtype=torch.float32),
            logits.new_empty((rows,), dtype=torch.float32))


@torch.library.custom_op(_q("_ce_rows_backward"), mutates_args=(), device_types="cuda")
def ce_rows_backward(logits: Tensor, targets: Tensor, ignore_index: int, lse: Tensor,
                     scale: Tensor) -> Tensor:
    """(softmax(logits) - onehot(target)) * scale, fp32 [rows, V], zero rows where ignored
    (reference loss.py:105-133 for one chunk); scale is a device scalar."""
    _require_cuda(logits)
    x = _ce_logits(logits)
    rows, V = (int(d) for d in x.shape)
    lib = _lib.load()
    t = targets.to(device=x.device, dtype=torch.int64).contiguous()
    l = lse.to(torch.float32).contiguous()
    sc = scale.to(device=x.device, dtype=torch.float32).reshape(1).contiguous()
    d = torch.empty((rows, V), device=x.device, dtype=torch.float32)
    err = torch.zeros(1, device=x.device, dtype=torch.int32)
    tk = KernelTimer.begin("ce_rows_bwd", x)
    _lib.check(lib.dabsn_hip_ce_bwd(_code(x.dtype), rows, V, _p(x), int(x.stride(0)) if rows else V,
                                    _p(t), int(ignore_index), _p(l), _p(sc), _p(d), _p(err),
                                    _stream(x)), "cross entropy backward")
    KernelTimer.end(tk)
    _record_error_word(err, "cross entropy backward", _TARGET_ERROR)
    return d


@ce_rows_backward.register_fake
def _ce_rows_backward_fake(logits, targets, ignore_index, lse, scale):
    return logits.new_empty(logits.shape, dtype=torch.float32)


# ---------------------------------------------------------------------------
# Read output: proj + long_gain * long (read.py:435-438, 821-823)
# ---------------------------------------------------------------------------
def _read_output_dtypes(proj: Tensor, long: Tensor, gain: Tensor) -> tuple[torch.dtype, torch.dtype]:
    prod = torch.result_type(gain, long)
    return prod, torch.promote_types(proj.dtype, prod)


@torch.library.custom_op(_q("read_output"), mutates_args=(), device_types="cuda")
def read_output(proj: Tensor, long: Tensor, gain: Tensor) -> Tensor:
    """``proj + gain * long`` as the reference evaluates ``out(...) + long_gain * long``: two
    tensor operations under type promotion (the product in the dtype of gain and long, the
    sum in the dtype of proj and the product), here in one pass over the elements."""
    _require_cuda(proj)
    if proj.shape != long.shape or gain.numel() != 1:
        raise ValueError("read_output: proj and long must match and gain hold one value")
    lib = _lib.load()
    prod_dt, out_dt = _read_output_dtypes(proj, long, gain)
    pc, lc = proj.contiguous(), long.contiguous()
    g = _f32_scalar(gain)
    out = torch.empty(proj.shape, device=proj.device, dtype=out_dt)
    _lib.check(lib.dabsn_hip_read_output(_code(pc.dtype), _code(lc.dtype), _code(prod_dt),
                                         _code(out_dt), pc.numel(), _p(pc), _p(lc), _p(g), _p(out),
                                         _stream(pc)), "read output")
    return out


@read_output.register_fake
def _read_output_fake(proj, long, gain):
    return proj.new_empty(proj.shape, dtype=_read_output_dtypes(proj, long, gain)[1])


def _row_blocks(what: str, *xs: Tensor) -> tuple[int, int, list[int]]:
    """(B, C * H, per-tensor batch strides) of [B, C, H] views whose (C, H) block is
    contiguous: time windows of [B, T, H] tensors or contiguous [B, C, H] tensors."""
    B, C, H = xs[0].shape
    for x in xs:
        if (x.dim() != 3 or tuple(x.shape) != (B, C, H) or x.stride(2) != 1
                or (C > 1 and x.stride(1) != H)):
            raise ValueError(f"{what}: [B, C, H] views of one shape with contiguous (C, H) "
                             "blocks")
    return B, C * H, [x.stride(0) for x in xs]


def read_output_window(proj: Tensor, long: Tensor, gain: Tensor, out: Tensor) -> None:
    """out = proj + gain * long over [B, C, H] views with contiguous (C, H) blocks (time
    windows of [B, T, H] tensors or contiguous blocks, each its own batch stride), in place
    (``dabsn_hip_read_output_window``; ``read_output``'s arithmetic). ``gain``: the parameter
    (one value)."""
    B, n, ld = _row_blocks("read_output_window", proj, long, out)
    prod_dt, out_dt = _read_output_dtypes(proj, long, gain)
    if out.dtype != out_dt:
        raise TypeError(f"read_output_window: out must be {out_dt}")
    lib = _lib.load()
    g = _f32_scalar(gain)
    _lib.check(lib.dabsn_hip_read_output_window(
        _code(proj.dtype), _code(long.dtype), _code(prod_dt), _code(out_dt), B, n, *ld,
        _p(proj), _p(long), _p(g), _p(out), _stream(proj)), "read output window")


def read_output_bwd_window(grad: Tensor, long: Tensor, gain: Tensor, gproj: Tensor,
                           glong: Tensor, ggain: Tensor) -> None:
    """``read_output``'s backward over [B, C, H] views as ``read_output_window`` takes, in
    place: gproj and glong written, ``ggain`` (one fp32 value) the views' share of the gain
    gradient, summed in a fixed order."""
    B, n, ld = _row_blocks("read_output_bwd_window", grad, long, gproj, glong)
    prod_dt = torch.result_type(gain, long)
    lib = _lib.load()
    g = _f32_scalar(gain)
    count = lib.dabsn_hip_read_output_partials(B * n)
    partials = torch.empty((max(count, 1),), device=grad.device, dtype=torch.float32)
    _lib.check(lib.dabsn_hip_read_output_bwd_window(
        _code(grad.dtype), _code(gproj.dtype), _code(long.dtype), _code(prod_dt), B, n, *ld,
        _p(grad), _p(long), _p(g), _p(gproj), _p(glong), _p(ggain), _p(partials),
        partials.numel(), _stream(grad)), "read output window backward")


_DTYPE_OF_CODE = {0: torch.float32, 1: torch.bfloat16}


@torch.library.custom_op(_q("_read_output_backward"), mutates_args=(), device_types="cuda")
def read_output_backward(grad: Tensor, long: Tensor, gain: Tensor,
                         proj_dtype: int) -> tuple[Tensor, Tensor, Tensor]:
    """(g_proj, g_long, g_gain) of ``read_output`` (``proj_dtype`` = the dtype code of proj):
    the gradients autograd forms for the two tensor operations, the gain's summed in a fixed
    order."""
    lib = _lib.load()
    pdt = _DTYPE_OF_CODE[int(proj_dtype)]
    prod_dt = torch.result_type(gain, long)
    out_dt = torch.promote_types(pdt, prod_dt)
    go = grad.to(out_dt).contiguous()
    lc = long.contiguous()
    g = _f32_scalar(gain)
    n = go.numel()
    gproj = torch.empty(go.shape, device=go.device, dtype=pdt)
    glong = torch.empty_like(lc)
    ggain = torch.empty((1,), device=go.device, dtype=torch.float32)
    count = lib.dabsn_hip_read_output_partials(n)
    partials = torch.empty((max(count, 1),), device=go.device, dtype=torch.float32)
    _lib.check(lib.dabsn_hip_read_output_bwd(
        _code(out_dt), _code(pdt), _code(lc.dtype), _code(prod_dt), n, _p(go), _p(lc), _p(g),
        _p(gproj), _p(glong), _p(ggain), _p(partials), partials.numel(), _stream(go)),
        "read output backward")
    return gproj, glong, ggain.reshape(gain.shape).to(gain.dtype)


@read_output_backward.register_fake
def _read_output_backward_fake(grad, long, gain, proj_dtype):
    return (grad.new_empty(grad.shape, dtype=_DTYPE_OF_CODE[int(proj_dtype)]),
            torch.empty_like(long), torch.empty_like(gain))


def _read_output_setup(ctx, inputs, output):
    proj, long, gain = inputs
    ctx.save_for_backward(long, gain)
    ctx.proj_dtype = _code(proj.dtype)


def _read_output_bwd(ctx, grad):
    long, gain = ctx.saved_tensors
    return read_output_backward(grad, long, gain, ctx.proj_dtype)


torch.library.register_autograd(_q("read_output"), _read_output_bwd,
                                setup_context=_read_output_setup)


# ---------------------------------------------------------------------------
# Fused recurrent long-memory scan
# ---------------------------------------------------------------------------
LONG_CKPT = 32  # steps per chunk of the long scan (DABSN_LONG_CKPT)


def long_segments(T: int) -> int:
    """Chunks of the long scan over T steps (rows of its checkpoint)."""
    return -(-int(T) // LONG_CKPT)


def _long_inputs(write: Tensor, plasticity: Tensor) -> tuple[Tensor, Tensor, int]:
    """(w, p, batch stride) for the long scan: [B, T, H] views with contiguous (T, H) blocks
    and one batch stride (time windows of longer tapes) pass as they are, anything else as
    contiguous copies."""
    dt = write.dtype
    w, p = write, plasticity.to(dt)
    B, T, H = w.shape
    ok = all(x.stride(2) == 1 and (T <= 1 or x.stride(1) == H) and x.stride(0) >= T * H
             for x in (w, p)) and w.stride(0) == p.stride(0)
    if not ok:
        w, p = w.contiguous(), p.contiguous()
    return w, p, (w.stride(0) if B > 1 else T * H)


@torch.library.custom_op(_q("long_scan_fused"), mutates_args=(), device_types="cuda")
def long_scan_fused(
    write: Tensor, plasticity: Tensor, logit_expect_retain: Tensor,
    logit_retention_decay: Tensor, logit_retain: Tensor, logit_retention_strength: Tensor,
    long0: Tensor, expected0: Tensor, retention0: Tensor,
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """The three recurrences of long.py:492-579, chunked over time. Returns (long [B,T,H],
    final long, final expected, final retention [B,H] fp32, and the checkpoint the backward
    replays from: the states (L, E, R) entering every 32-step chunk, [B, ceil(T/32), 3, H]
    fp32)."""
    _require_cuda(write)
    return long_scan_window(write, plasticity, [logit_expect_retain, logit_retention_decay,
                                                logit_retain, logit_retention_strength],
                            long0, expected0, retention0)


def long_scan_window(write: Tensor, plasticity: Tensor, logits: list[Tensor], long0: Tensor,
                     expected0: Tensor, retention0: Tensor
                     ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """long_scan_fused's results for inputs that may be time windows of longer [B, T', H]
    tapes (read in place, ``dabsn_hip_long_fwd``'s input batch stride); the outputs are
    contiguous."""
    lib = _lib.load()
    B, T, H = write.shape
    dt = write.dtype
    w, p, ldx = _long_inputs(write, plasticity)
    logits = [_f32_scalar(x) for x in logits]
    ptrs = _lib.PTR4(*[x.data_ptr() for x in logits])
    L0, E0, R0 = (x.float().contiguous() for x in (long0, expected0, retention0))
    out = torch.empty((B, T, H), device=w.device, dtype=dt)
    LF, EF, RF = (torch.empty((B, H), device=w.device, dtype=torch.float32) for _ in range(3))
    ckpt = torch.empty((B, long_segments(T), 3, H), device=w.device, dtype=torch.float32)
    nbytes = lib.dabsn_hip_long_workspace_bytes(B, T, H, 0)
    ws = torch.empty(max(nbytes, 4), dtype=torch.uint8, device=w.device)
    tk = KernelTimer.begin("long_scan_fwd", w)
    _lib.check(lib.dabsn_hip_long_fwd(_code(dt), B, T, H, ldx, _p(w), _p(p), ptrs, _p(L0),
                                      _p(E0), _p(R0), _p(out), _p(LF), _p(EF), _p(RF), _p(ckpt),
                                      _p(ws), nbytes, _stream(w)), "long scan")
    KernelTimer.end(tk)
    return out, LF, EF, RF, ckpt


@long_scan_fused.register_fake
def _long_scan_fused_fake(write, plasticity, l1, l2, l3, l4, long0, expected0, retention0):
    B, T, H = write.shape
    f = lambda *s: write.new_empty(s, dtype=torch.float32)  # noqa: E731
    return torch.empty_like(write), f(B, H), f(B, H), f(B, H), f(B, long_segments(T), 3, H)


def long_scan_backward_parts(
    write: Tensor, plasticity: Tensor, logits: list[Tensor], checkpoint: Tensor,
    grad_long: Tensor, g_long_final: Optional[Tensor], g_expected_final: Optional[Tensor],
    g_retention_final: Optional[Tensor], gw_into: Optional[Tensor] = None,
    gp_into: Optional[Tensor] = None,
) -> tuple[Tensor, Tensor, Tensor, list[Tensor]]:
    """long_scan_fused_backward's results as (g_write, g_plasticity in the write dtype, the
    four logit gradients as one [4] fp32 tensor, [gL0, gE0, gR0]), for callers that need
    no separate tensor per logit. write and plasticity may be time windows of longer tapes
    (read in place, as ``long_scan_window``). ``gw_into`` / ``gp_into`` (together, [B, T, H]
    views in the write dtype with contiguous (T, H) blocks and one batch stride, e.g. time
    windows of full-length gradient buffers): the write gradient is added into ``gw_into``
    (rounded to the dtype, the sum formed in fp32 and rounded once, as a tensor add) and the
    plasticity gradient written into ``gp_into``; they are returned in place of new
    tensors."""
    _require_cuda(write)
    lib = _lib.load()
    B, T, H = write.shape
    dt = write.dtype
    w, p, ldx = _long_inputs(write, plasticity)
    lg = [_f32_scalar(x) for x in logits]
    ptrs = _lib.PTR4(*[x.data_ptr() for x in lg])
    gout = grad_long.to(dt).contiguous()
    gf = [None if x is None else x.float().contiguous()
          for x in (g_long_final, g_expected_final, g_retention_final)]
    if (gw_into is None) != (gp_into is None):
        raise ValueError("long scan backward: gw_into and gp_into go together")
    if gw_into is None:
        gw, gp = (torch.empty((B, T, H), device=w.device, dtype=dt) for _ in range(2))
        ldo, acc = T * H, 0
    else:
        gw, gp = gw_into, gp_into
        if any(tuple(x.shape) != (B, T, H) or x.dtype != dt or x.stride(2) != 1
               or (T > 1 and x.stride(1) != H) or x.stride(0) < T * H for x in (gw, gp)) \
                or gw.stride(0) != gp.stride(0):
            raise ValueError("long scan backward: gw_into / gp_into must be [B, T, H] views of "
                             "the write dtype with contiguous (T, H) blocks and one batch stride")
        ldo, acc = (gw.stride(0) if B > 1 else T * H), 1
    g0 = [torch.empty((B, H), device=w.device, dtype=torch.float32) for _ in range(3)]
    nparts = lib.dabsn_hip_long_partials(B, T, H)
    part = torch.empty((max(nparts, 1), 4), device=w.device, dtype=torch.float32)
    part[nparts:].zero_()
    nbytes = lib.dabsn_hip_long_workspace_bytes(B, T, H, 1)
    ws = torch.empty(max(nbytes, 4), dtype=torch.uint8, device=w.device)
    tk = KernelTimer.begin("long_scan_bwd", w)
    st = checkpoint.float().contiguous()
    if tuple(st.shape) != (B, long_segments(T), 3, H):
        raise ValueError(f"long scan backward: checkpoint shape {tuple(st.shape)}, expected "
                         f"{(B, long_segments(T), 3, H)}")
    _lib.check(lib.dabsn_hip_long_bwd(_code(dt), B, T, H, ldx, _p(w), _p(p), ptrs, _p(st),
                                      _p(gout), *[_p(x) for x in gf], _p(gw), _p(gp), ldo, acc,
                                      *[_p(x) for x in g0], _p(part), _p(ws), nbytes,
                                      _stream(w)), "long scan backward")
    KernelTimer.end(tk)
    # The partials as four contiguous rows: a reduction along rows spreads each sum over many
    # threads (summing down the columns in place runs serially).
    return gw, gp, part.t().contiguous().sum(1), g0


@torch.library.custom_op(_q("_long_scan_fused_backward"), mutates_args=(),
                         device_types="cuda")
def long_scan_fused_backward(
    write: Tensor, plasticity: Tensor, logits: list[Tensor], checkpoint: Tensor,
    grad_long: Tensor, g_long_final: Optional[Tensor], g_expected_final: Optional[Tensor],
    g_retention_final: Optional[Tensor],
) -> list[Tensor]:
    """Reverse of long_scan_fused from its checkpoint: [g_write, g_plasticity, 4 logit
    grads, gL0, gE0, gR0]."""
    gw, gp, glog, g0 = long_scan_backward_parts(write, plasticity, logits, checkpoint,
                                                grad_long, g_long_final, g_expected_final,
                                                g_retention_final)
    return [gw, gp.to(plasticity.dtype), *_separate(glog, 4), *g0]


@long_scan_fused_backward.register_fake
def _long_scan_fused_backward_fake(write, plasticity, logits, checkpoint, grad_long, a, b, c):
    B, T, H = write.shape
    f = lambda *s: write.new_empty(s, dtype=torch.float32)  # noqa: E731
    return [torch.empty_like(write), torch.empty_like(plasticity), f(), f(), f(), f(),
            f(B, H), f(B, H), f(B, H)]


def _long_setup(ctx, inputs, output):
    write, plasticity, l1, l2, l3, l4, L0, E0, R0 = inputs
    ctx.save_for_backward(write, plasticity, l1, l2, l3, l4, output[4])
    ctx.meta = [(x.dtype, tuple(x.shape)) for x in inputs]
    # The checkpoint is saved for the backward, not a result anyone differentiates;
    # with grads left unmaterialised, unused outputs bring None instead of zero tensors.
    ctx.mark_non_differentiable(output[4])
    ctx.set_materialize_grads(False)


def _long_bwd(ctx, g_long, g_lf, g_ef, g_rf, _g_ckpt):
    write, plasticity, l1, l2, l3, l4, ckpt = ctx.saved_tensors
    if g_long is None:
        g_long = torch.zeros_like(write)
    grads = long_scan_fused_backward(write, plasticity, [l1, l2, l3, l4], ckpt, g_long, g_lf,
                                     g_ef, g_rf)
    return tuple(g.reshape(shape).to(dtype) for g, (dtype, shape) in zip(grads, ctx.meta))


torch.library.register_autograd(_q("long_scan_fused"), _long_bwd, setup_context=_long_setup)


# ---------------------------------------------------------------------------
# Read glue
# ---------------------------------------------------------------------------
@torch.library.custom_op(_q("read_tape_stats"), mutates_args=(), device_types="cuda")
def read_tape_stats(novelty: Tensor, plasticity: Tensor, energy: Tensor, saturation: Tensor,
                    expression: Tensor, write: Tensor) -> Tensor:
    """Per-position (mean e, mean c, mean n, mean p, |expression|, |write|), fp32 [B,T,6]
    (reference read.py:58-72, 154-183). The two norms carry no gradient here: their
    dependence is part of the normalisation operators' backward."""
    _require_cuda(novelty)
    lib = _lib.load()
    B, T, H = novelty.shape
    dt = novelty.dtype
    xs = [x.to(dt).contiguous() for x in (novelty, plasticity, energy, saturation, expression, write)]
    stats = torch.empty((B, T, 6), device=novelty.device, dtype=torch.float32)
    _lib.check(lib.dabsn_hip_tape_stats(_code(dt), B, T, H, *[_p(x) for x in xs], _p(stats),
                                        _stream(novelty)), "tape statistics")
    return stats


@read_tape_stats.register_fake
def _read_tape_stats_fake(novelty, plasticity, energy, saturation, expression, write):
    B, T, _ = novelty.shape
    return novelty.new_empty((B, T, 6), dtype=torch.float32)


@torch.library.custom_op(_q("_read_tape_stats_backward"), mutates_args=(),
                         device_types="cuda")
def read_tape_stats_backward(gstats: Tensor, like: Tensor) -> list[Tensor]:
    """Broadcast mean gradients back to the four averaged tapes [g_n, g_p, g_e, g_c]."""
    lib = _lib.load()
    B, T, H = like.shape
    dt = like.dtype
    gs = gstats.float().contiguous()
    gn, gp, ge, gc = (torch.empty((B, T, H), device=like.device, dtype=dt) for _ in range(4))
    _lib.check(lib.dabsn_hip_tape_stats_bwd(_code(dt), B, T, H, _p(gs), 0, _p(gn), _p(gp),
                                            _p(ge), _p(gc), _stream(like)),
               "tape statistics backward")
    return [gn, gp, ge, gc]


@read_tape_stats_backward.register_fake
def _read_tape_stats_backward_fake(gstats, like):
    return [torch.empty_like(like) for _ in range(4)]


def _stats_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[0])
    ctx.dtypes = [x.dtype for x in inputs]


def _stats_bwd(ctx, gstats):
    (like,) = ctx.saved_tensors
    gn, gp, ge, gc = read_tape_stats_backward(gstats, like)
    d = ctx.dtypes
    return gn.to(d[0]), gp.to(d[1]), ge.to(d[2]), gc.to(d[3]), None, None


torch.library.register_autograd(_q("read_tape_stats"), _stats_bwd, setup_context=_stats_setup)


@torch.library.custom_op(_q("normalize_rows"), mutates_args=(), device_types="cuda")
def normalize_rows(x: Tensor, norms: Tensor) -> Tensor:
    """x / max(norms, 1e-12) along the last dim, norms = |x| rows (F.normalize, read.py:154)."""
    lib = _lib.load()
    H = x.shape[-1]
    rows = x.numel() // H
    xc = x.contiguous()
    n = norms.float().contiguous()
    q = torch.empty_like(xc)
    _lib.check(lib.dabsn_hip_normalize_rows(_code(x.dtype), rows, H, _p(xc), _p(n), _p(q),
                                            _stream(x)), "normalize rows")
    return q


@normalize_rows.register_fake
def _normalize_rows_fake(x, norms):
    return torch.empty_like(x)


@torch.library.custom_op(_q("_normalize_rows_backward"), mutates_args=(), device_types="cuda")
def normalize_rows_backward(q: Tensor, norms: Tensor, gq: Tensor) -> Tensor:
    lib = _lib.load()
    H = q.shape[-1]
    rows = q.numel() // H
    qc = q.contiguous()
    gqc = gq.to(q.dtype).contiguous()
    nc = norms.float().contiguous()
    gx = torch.zeros_like(qc)
    _lib.check(lib.dabsn_hip_normalize_rows_bwd(_code(q.dtype), rows, H, _p(qc),
                                                _p(nc), _p(gqc), _p(gx),
                                                _stream(q)), "normalize rows backward")
    return gx


@normalize_rows_backward.register_fake
def _normalize_rows_backward_fake(q, norms, gq):
    return torch.empty_like(q)


def _norm_setup(ctx, inputs, output):
    ctx.save_for_backward(output, inputs[1])


def _norm_bwd(ctx, gq):
    q, norms = ctx.saved_tensors
    return normalize_rows_backward(q, norms, gq), None


torch.library.register_autograd(_q("normalize_rows"), _norm_bwd, setup_context=_norm_setup)


@torch.library.custom_op(_q("bank_select"), mutates_args=(), device_types="cuda")
def bank_select(admission: Tensor, window: Tensor,
                whole: int = 0) -> tuple[Tensor, Tensor, Tensor]:
    """Admitted-slot selection (read.py:185-239): (order [B,T] int64, counts [B] int64,
    rank [B,T] int32). Bit-exact integer work given the admission values. The floor
    ``cummax(admission) - window`` (``whole`` = 0, seq geometry) or ``max(admission) -
    window`` over the whole row (``whole`` = 1, field and hybrid geometry) is evaluated in
    the admission's dtype, as the reference does (bf16 admission: the difference is rounded
    to bf16)."""
    lib = _lib.load()
    B, T = admission.shape
    if admission.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"bank_select: admission must be fp32 or bf16, not {admission.dtype}")
    adm_code = 1 if admission.dtype == torch.bfloat16 else 0
    adm = admission.float().contiguous()
    win = window.float().reshape(()).contiguous()
    order = torch.empty((B, T), device=adm.device, dtype=torch.int64)
    counts = torch.empty((B,), device=adm.device, dtype=torch.int64)
    rank = torch.empty((B, T), device=adm.device, dtype=torch.int32)
    _lib.check(lib.dabsn_hip_bank_select(adm_code, int(whole), B, T, _p(adm), _p(win), _p(order),
                                         _p(counts), _p(rank), _stream(adm)), "bank selection")
    return order, counts, rank


def admit_step(stats: Optional[Tensor], hidden: int, params: Sequence[Tensor],
               tape_dtype: torch.dtype, window: Tensor, base: int, n: int, key_bias: Tensor,
               admission: Tensor, cocktail: Tensor, amax: Tensor, mcount: Tensor,
               members: Tensor, adm_bf16: bool) -> None:
    """Incremental admission of a carried bank (streaming decode, inference only), in
    place: for positions ``base`` .. ``base + n - 1``, their glue from the statistics rows
    ``stats`` [B, cap, 6] (as ``means_glue``; with ``stats`` None the values already in
    ``admission`` are used) into ``key_bias`` / ``admission`` [B, cap] and ``cocktail``
    [B, cap, 4], then their membership under the causal floor, extending each row's slot
    list ``members`` [B, cap] int64, the counts ``mcount`` [B] int64 and the running prefix
    max ``amax`` [B] fp32. ``adm_bf16``: the reference's admission is a bf16 tensor, so the
    floor is rounded to bf16 (as ``bank_select``)."""
    _require_cuda(admission)
    lib = _lib.load()
    B, cap = (int(d) for d in admission.shape)
    for t, shape, dt in ((key_bias, (B, cap), torch.float32), (admission, (B, cap), torch.float32),
                         (cocktail, (B, cap, 4), torch.float32), (amax, (B,), torch.float32),
                         (mcount, (B,), torch.int64), (members, (B, cap), torch.int64)):
        if tuple(t.shape) != shape or t.dtype != dt or not t.is_contiguous():
            raise ValueError(f"admit_step: expected a contiguous {dt} tensor of shape {shape}")
    if stats is not None and (tuple(stats.shape) != (B, cap, 6) or stats.dtype != torch.float32
                              or not stats.is_contiguous()):
        raise ValueError("admit_step: stats must be contiguous fp32 [B, cap, 6]")
    prm = [_f32_scalar(x) for x in params]
    ptrs = _lib.PTR8(*[x.data_ptr() for x in prm])
    mode = 0
    if tape_dtype == torch.bfloat16:
        mode = 1 | (2 if all(x.dtype == torch.bfloat16 for x in params) else 0)
    win = _f32_scalar(window)
    _lib.check(lib.dabsn_hip_admit_step(mode, B, int(n), int(base), cap, _p(stats), int(hidden),
                                        ptrs, _p(win), 1 if adm_bf16 else 0, _p(key_bias),
                                        _p(admission), _p(cocktail), _p(amax), _p(mcount),
                                        _p(members), _stream(admission)),
               "incremental admission")


@bank_select.register_fake
def _bank_select_fake(admission, window, whole=0):
    B, T = admission.shape
    return (admission.new_empty((B, T), dtype=torch.int64),
            admission.new_empty((B,), dtype=torch.int64),
            admission.new_empty((B, T), dtype=torch.int32))


@torch.library.custom_op(_q("bank_gather"), mutates_args=(), device_types="cuda")
def bank_gather(write: Tensor, norm_w: Tensor, idx: Tensor, next_idx: Tensor,
                rank: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """(normalize(write[idx]), write[idx], write[next_idx]) as in read.py:241-256, 298-303."""
    lib = _lib.load()
    B, T, H = write.shape
    N = idx.shape[1]
    w = write.contiguous()
    nw = norm_w.float().contiguous()
    ic = idx.to(torch.int64).contiguous()
    nc = next_idx.to(torch.int64).contiguous()
    K, V, Vn = (torch.empty((B, N, H), device=w.device, dtype=w.dtype) for _ in range(3))
    _lib.check(lib.dabsn_hip_bank_gather(_code(w.dtype), B, T, N, H, _p(w), _p(nw), _p(ic),
                                         _p(nc), _p(K), _p(V), _p(Vn), _stream(w)), "bank gather")
    return K, V, Vn


@bank_gather.register_fake
def _bank_gather_fake(write, norm_w, idx, next_idx, rank):
    B, T, H = write.shape
    N = idx.shape[1]
    return tuple(write.new_empty((B, N, H)) for _ in range(3))


@torch.library.custom_op(_q("_bank_gather_backward"), mutates_args=(), device_types="cuda")
def bank_gather_backward(write: Tensor, norm_w: Tensor, rank: Tensor, K: Tensor, gK: Tensor,
                         gV: Tensor, gVn: Optional[Tensor]) -> Tensor:
    """Deterministic inverse gather of the bank gradients onto the write tape (gVn None: no
    successor-row gradients)."""
    lib = _lib.load()
    B, T, H = write.shape
    N = K.shape[1]
    dt = write.dtype
    gw = torch.empty((B, T, H), device=write.device, dtype=dt)
    nw = norm_w.float().contiguous()
    rk = rank.to(torch.int32).contiguous()
    Kc = K.to(dt).contiguous()
    gKc, gVc = (g.to(dt).contiguous() for g in (gK, gV))
    gVnc = None if gVn is None else gVn.to(dt).contiguous()
    _lib.check(lib.dabsn_hip_bank_gather_bwd(_code(dt), B, T, N, H, None, _p(nw), _p(rk), _p(Kc),
                                             _p(gKc), _p(gVc), _p(gVnc), _p(gw), _stream(write)),
               "bank gather backward")
    return gw


@bank_gather_backward.register_fake
def _bank_gather_backward_fake(write, norm_w, rank, K, gK, gV, gVn):
    return torch.empty_like(write)


def _gather_setup(ctx, inputs, output):
    write, norm_w, idx, next_idx, rank = inputs
    ctx.save_for_backward(write, norm_w, rank, output[0])


def _gather_bwd(ctx, gK, gV, gVn):
    write, norm_w, rank, K = ctx.saved_tensors
    z = lambda g: torch.zeros_like(K) if g is None else g  # noqa: E731
    gw = bank_gather_backward(write, norm_w, rank, K, z(gK), z(gV), gVn)
    return gw, None, None, None, None


torch.library.register_autograd(_q("bank_gather"), _gather_bwd, setup_context=_gather_setup)


@torch.library.custom_op(_q("bank_gather_kv"), mutates_args=(), device_types="cuda")
def bank_gather_kv(write: Tensor, norm_w: Tensor, idx: Tensor, rank: Tensor) -> tuple[Tensor, Tensor]:
    """(normalize(write[idx]), write[idx]): ``bank_gather`` without the successor rows, for
    a read that folds them into V (``bank_fold``)."""
    lib = _lib.load()
    B, T, H = write.shape
    N = idx.shape[1]
    w = write.contiguous()
    nw = norm_w.float().contiguous()
    ic = idx.to(torch.int64).contiguous()
    K, V = (torch.empty((B, N, H), device=w.device, dtype=w.dtype) for _ in range(2))
    _lib.check(lib.dabsn_hip_bank_gather(_code(w.dtype), B, T, N, H, _p(w), _p(nw), _p(ic), None,
                                         _p(K), _p(V), None, _stream(w)), "bank gather")
    return K, V


@bank_gather_kv.register_fake
def _bank_gather_kv_fake(write, norm_w, idx, rank):
    B, T, H = write.shape
    N = idx.shape[1]
    return write.new_empty((B, N, H)), write.new_empty((B, N, H))


def _gather_kv_setup(ctx, inputs, output):
    write, norm_w, idx, rank = inputs
    ctx.save_for_backward(write, norm_w, rank, output[0])


def _gather_kv_bwd(ctx, gK, gV):
    write, norm_w, rank, K = ctx.saved_tensors
    z = lambda g: torch.zeros_like(K) if g is None else g  # noqa: E731
    gw = bank_gather_backward(write, norm_w, rank, K, z(gK), z(gV), None)
    return gw, None, None, None


torch.library.register_autograd(_q("bank_gather_kv"), _gather_kv_bwd, setup_context=_gather_kv_setup)


def bank_fold(order: Tensor, counts: Tensor, width: Optional[int] = None):
    """Successor-fold codes of a ``bank_select`` result (``dabsn_hip_bank_fold``).

    width None: returns a one-element int32 device tensor, 1 when some admitted slot's next
    position (min(idx + 1, T - 1)) is neither the next slot's position nor its own, else 0
    (no host sync). width N: returns the int8 codes [B, N] (1: the next position is slot
    j + 1's; 0: its own, or past the row's count; 2: neither)."""
    lib = _lib.load()
    B, T = order.shape
    o = order.contiguous()
    c = counts.contiguous()
    if width is None:
        flag = torch.empty((1,), device=order.device, dtype=torch.int32)
        _lib.check(lib.dabsn_hip_bank_fold(B, T, T, _p(o), _p(c), None, _p(flag), _stream(o)),
                   "bank fold")
        return flag
    codes = torch.empty((B, int(width)), device=order.device, dtype=torch.int8)
    _lib.check(lib.dabsn_hip_bank_fold(B, T, int(width), _p(o), _p(c), _p(codes), None,
                                       _stream(o)), "bank fold")
    return codes


def window_add(out: Tensor, a: Tensor, x: Optional[Tensor] = None) -> Tensor:
    """out = a (+ x) for [B, R, C] views with contiguous columns and any batch and row
    strides (``dabsn_hip_window_add``): time windows of [B, T, C] tensors, column blocks of
    wider rows. Returns out."""
    ops_ = [t for t in (out, a, x) if t is not None]
    if any(t.dim() != 3 or t.shape != out.shape or t.dtype != out.dtype or t.stride(2) != 1
           or t.device != out.device for t in ops_):
        raise ValueError("window_add: [B, R, C] views of one shape and dtype, columns contiguous")
    lib = _lib.load()
    B, R, C = out.shape
    xs = (0, 0) if x is None else (x.stride(0), x.stride(1))
    _lib.check(lib.dabsn_hip_window_add(_code(out.dtype), B, R, C, _p(a), a.stride(0), a.stride(1),
                                        _p(x), *xs, _p(out), out.stride(0), out.stride(1),
                                        _stream(out)), "window add")
    return out


def window_copy(a: Tensor) -> Tensor:
    """A contiguous copy of the [B, R, C] view ``a`` (``window_add`` with no second term)."""
    return window_add(torch.empty(a.shape, device=a.device, dtype=a.dtype), a)


def bank_width(order: Tensor, counts: Tensor, check_fold: bool) -> Tensor:
    """[largest admitted count, unfoldable flag] of a ``bank_select`` result as one int64
    device tensor of two values (``dabsn_hip_bank_width``; the flag is 0 without
    ``check_fold``), for one host read."""
    lib = _lib.load()
    B, T = order.shape
    o, c = order.contiguous(), counts.contiguous()
    out = torch.empty((2,), device=order.device, dtype=torch.int64)
    _lib.check(lib.dabsn_hip_bank_width(B, T, _p(o), _p(c), 1 if check_fold else 0, _p(out),
                                        _stream(o)), "bank width")
    return out


def bank_slots(order: Tensor, counts: Tensor, width: int, query_start: int,
               fold: bool) -> tuple[Tensor, Tensor, Tensor, Tensor, Optional[Tensor]]:
    """(idx, valid, next_idx, read_idx, fold codes or None), each [B, width], of a read of
    ``width`` slots from a ``bank_select`` result in one launch (``dabsn_hip_bank_slots``):
    idx = order[:, :width], valid = slot < max(count, 1), next_idx = min(idx + 1, T - 1),
    read_idx = idx - query_start."""
    lib = _lib.load()
    B, T = order.shape
    N = int(width)
    o, c = order.contiguous(), counts.contiguous()
    dev = order.device
    idx, next_idx, read_idx = (torch.empty((B, N), device=dev, dtype=torch.int64)
                               for _ in range(3))
    valid = torch.empty((B, N), device=dev, dtype=torch.bool)
    codes = torch.empty((B, N), device=dev, dtype=torch.int8) if fold else None
    _lib.check(lib.dabsn_hip_bank_slots(B, T, N, _p(o), _p(c), int(query_start), _p(idx),
                                        _p(valid), _p(next_idx), _p(read_idx), _p(codes),
                                        _stream(o)), "bank slots")
    return idx, valid, next_idx, read_idx, codes


# ---------------------------------------------------------------------------
# Three-way admitted read (compact ABI)
# ---------------------------------------------------------------------------
def _read_common(query, bank_keys, bank_writes, next_writes, cocktail, bank_cocktail,
                 bank_key_bias, bank_admission, scale, bank_idx, bank_valid, gains):
    dt = query.dtype
    q = query.contiguous()
    K, V = (x.to(dt).contiguous() for x in (bank_keys, bank_writes))
    Vn = None if next_writes is None else next_writes.to(dt).contiguous()
    ck, cb, kb, adm = (x.float().contiguous() for x in (cocktail, bank_cocktail, bank_key_bias,
                                                       bank_admission))
    sc = scale.float().reshape(()).contiguous()
    g = [_f32_scalar(x) for x in gains]
    idx = bank_idx.to(torch.int64).contiguous()
    # A bool mask is already one 0/1 byte per slot: reinterpreted, not converted.
    valid = (bank_valid.view(torch.uint8) if bank_valid.dtype == torch.bool
             else bank_valid.to(torch.uint8)).contiguous()
    if cocktail.shape[-1] != 4 or bank_cocktail.shape[-1] != 4:
        raise ValueError("the HIP read expects a 4-component cocktail")
    return dt, q, K, V, Vn, ck, cb, kb, adm, sc, g, idx, valid


@torch.library.custom_op(_q("admitted_three_way_read_compact_flash"), mutates_args=(),
                         device_types="cuda")
def admitted_three_way_read_compact_flash(
    query: Tensor, bank_keys: Tensor, bank_writes: Tensor, next_writes: Tensor, cocktail: Tensor,
    bank_cocktail: Tensor, bank_key_bias: Tensor, bank_admission: Tensor, scale: Tensor,
    bank_idx: Tensor, bank_valid: Tensor, mode: int, short_gain: Tensor, pad_gain: Tensor,
    induct_gain: Tensor, cocktail_gain: Tensor,
) -> Tensor:
    """Three-way admitted read (reference compact_flash.py:71-107; math admitted.py:16-65)."""
    _require_cuda(query)
    lib = _lib.load()
    if mode not in (0, 1):
        raise ValueError("compact admitted-read mode must be 0 (seq) or 1 (field)")
    dt, q, K, V, Vn, ck, cb, kb, adm, sc, g, idx, valid = _read_common(
        query, bank_keys, bank_writes, next_writes, cocktail, bank_cocktail, bank_key_bias,
        bank_admission, scale, bank_idx, bank_valid,
        (short_gain, pad_gain, induct_gain, cocktail_gain))
    B, T, H = q.shape
    N = K.shape[1]
    code = _code(dt)
    out = torch.empty_like(q)
    nbytes = lib.dabsn_hip_read3_workspace_bytes(code, B, T, N, H, 0)
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=q.device)
    ptrs = _lib.PTR4(*[x.data_ptr() for x in g])
    tk = KernelTimer.begin("read3_fwd", q)
    _lib.check(lib.dabsn_hip_read3_fwd(code, B, T, N, H, _p(q), _p(K), _p(V), _p(Vn), _p(ck),
                                       _p(cb), _p(kb), _p(adm), _p(sc), _p(idx), _p(valid), mode,
                                       ptrs, _p(out), _p(ws), ws.numel(), _stream(q)),
               "three-way read")
    KernelTimer.end(tk)
    return out


@admitted_three_way_read_compact_flash.register_fake
def _read_fake(query, *rest):
    return torch.empty_like(query)


def read3_decode(query: Tensor, bank_write: Tensor, norm_w: Tensor, idx: Tensor,
                 next_idx: Tensor, read_idx: Tensor, valid: Tensor, cocktail: Tensor,
                 bank_cocktail: Tensor, bank_key_bias: Tensor, bank_admission: Tensor,
                 scale: Tensor, gains: tuple[Tensor, Tensor, Tensor, Tensor]) -> Tensor:
    """The seq three-way read of a few query rows (T <= 8) against a bank read in place
    (inference only; no autograd). Equals bank_gather followed by
    admitted_three_way_read_compact_flash in mode 0 up to the summation order of the dot
    products and of the slot sum.

    ``bank_write`` [B, N_bank, H] may be a view of a longer per-row buffer (unit stride over
    H, rows H apart); ``norm_w`` [B, N_bank] are its write norms; ``idx`` / ``next_idx``
    [B, N] address the bank, ``read_idx`` [B, N] are the query-relative slot indices the
    masks use. ``gains`` = (short, pad, induct, cocktail)."""
    _require_cuda(query)
    lib = _lib.load()
    dt = query.dtype
    q = query.contiguous()
    B, T, H = q.shape
    N = idx.shape[1]
    if bank_write.dtype != dt or bank_write.stride(2) != 1 or bank_write.stride(1) != H \
            or bank_write.stride(0) % H != 0:
        raise ValueError("read3_decode: bank_write must be rows of H contiguous elements")
    bank_len, bank_ld = int(bank_write.shape[1]), int(bank_write.stride(0) // H)
    nw = norm_w.float().contiguous()
    ic, nc, rc = (x.to(torch.int64).contiguous() for x in (idx, next_idx, read_idx))
    vc = valid.to(torch.uint8).contiguous()
    ck, cb, kb, adm = (x.float().contiguous() for x in (cocktail, bank_cocktail, bank_key_bias,
                                                       bank_admission))
    sc = scale.float().reshape(()).contiguous()
    g = [_f32_scalar(x) for x in gains]
    out = torch.empty_like(q)
    code = _code(dt)
    nbytes = lib.dabsn_hip_read3_decode_workspace_bytes(code, B, T, N, H)
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=q.device)
    ptrs = _lib.PTR4(*[x.data_ptr() for x in g])
    tk = KernelTimer.begin("read3_decode", q)
    _lib.check(lib.dabsn_hip_read3_decode(code, B, T, N, H, _p(q), _p(bank_write), bank_len,
                                          bank_ld, _p(nw), _p(ic), _p(nc), _p(rc), _p(vc),
                                          _p(ck), _p(cb), _p(kb), _p(adm), _p(sc), ptrs, _p(out),
                                          _p(ws), ws.numel(), _stream(q)), "three-way decode read")
    KernelTimer.end(tk)
    return out


def read3_decode_members(query: Tensor, write: Tensor, stats: Tensor, length: int, width: int,
                         members: Tensor, counts: Tensor, query_start: int, cocktail: Tensor,
                         key_bias: Tensor, admission: Tensor, scale: Tensor,
                         gains: tuple[Tensor, Tensor, Tensor, Tensor]) -> Tensor:
    """``read3_decode`` of one query row per batch row with the slots taken from a carried
    bank's admitted-slot lists: ``write`` [B, cap, H], ``stats`` [B, cap, 6], ``members``
    [B, cap], ``cocktail`` [B, cap, 4], ``key_bias`` / ``admission`` [B, cap] are the bank's
    whole storage (the first ``length`` positions live), ``counts`` [B] the members per row;
    the read covers the first ``width`` slots. Equals ``read3_decode`` on idx =
    members[:, :width], valid = j < max(count, 1), next_idx = min(idx + 1, length - 1),
    read_idx = idx - query_start and the glue gathered at idx, without materialising them."""
    _require_cuda(query)
    lib = _lib.load()
    dt = query.dtype
    B, T, H = query.shape
    cap = int(write.shape[1])
    if T != 1 or not query.is_contiguous() or write.dtype != dt or not write.is_contiguous():
        raise ValueError("read3_decode_members: one contiguous query row per batch row and a "
                         "contiguous bank of the query's dtype")
    for t, shape, tdt in ((stats, (B, cap, 6), torch.float32), (members, (B, cap), torch.int64),
                          (counts, (B,), torch.int64), (cocktail, (B, cap, 4), torch.float32),
                          (key_bias, (B, cap), torch.float32),
                          (admission, (B, cap), torch.float32)):
        if tuple(t.shape) != shape or t.dtype != tdt or not t.is_contiguous():
            raise ValueError(f"read3_decode_members: expected a contiguous {tdt} tensor of "
                             f"shape {shape}, got {tuple(t.shape)} {t.dtype}")
    g = [_f32_scalar(x) for x in gains]
    sc = _f32_scalar(scale)
    out = torch.empty_like(query)
    code = _code(dt)
    nbytes = lib.dabsn_hip_read3_decode_workspace_bytes(code, B, 1, width, H)
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=query.device)
    ptrs = _lib.PTR4(*[x.data_ptr() for x in g])
    tk = KernelTimer.begin("read3_decode", query)
    _lib.check(lib.dabsn_hip_read3_decode_members(
        code, B, int(width), H, _p(query), _p(write), int(length), cap, _p(stats), _p(members),
        _p(counts), int(query_start), _p(cocktail), _p(key_bias), _p(admission), _p(sc), ptrs,
        _p(out), _p(ws), ws.numel(), _stream(query)), "three-way decode read (members)")
    KernelTimer.end(tk)
    return out


CompactGradients = tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor,
                         Tensor, Tensor, Tensor, Tensor]


@torch.library.custom_op(_q("_admitted_three_way_read_compact_flash_backward"),
                         mutates_args=(), device_types="cuda")
def admitted_three_way_read_compact_flash_backward(
    grad_output: Tensor, query: Tensor, bank_keys: Tensor, bank_writes: Tensor,
    next_writes: Tensor, cocktail: Tensor, bank_cocktail: Tensor, bank_key_bias: Tensor,
    bank_admission: Tensor, scale: Tensor, bank_idx: Tensor, bank_valid: Tensor, mode: int,
    short_gain: Tensor, pad_gain: Tensor, induct_gain: Tensor, cocktail_gain: Tensor,
) -> CompactGradients:
    """13 gradients (compact_flash.py:181-224 order): query, bank_keys, bank_writes,
    next_writes, cocktail, bank_cocktail, bank_key_bias, bank_admission, scale, short_gain,
    pad_gain, induct_gain, cocktail_gain."""
    _require_cuda(query)
    lib = _lib.load()
    dt, q, K, V, Vn, ck, cb, kb, adm, sc, g, idx, valid = _read_common(
        query, bank_keys, bank_writes, next_writes, cocktail, bank_cocktail, bank_key_bias,
        bank_admission, scale, bank_idx, bank_valid,
        (short_gain, pad_gain, induct_gain, cocktail_gain))
    B, T, H = q.shape
    N = K.shape[1]
    code = _code(dt)
    go = grad_output.to(dt).contiguous()
    gq = torch.empty_like(q)
    gK, gV, gVn = (torch.empty((B, N, H), device=q.device, dtype=dt) for _ in range(3))
    gck = torch.empty((B, T, 4), device=q.device, dtype=torch.float32)
    gcb = torch.empty((B, N, 4), device=q.device, dtype=torch.float32)
    gkb = torch.empty((B, N), device=q.device, dtype=torch.float32)
    gadm = torch.empty((B, N), device=q.device, dtype=torch.float32)
    g5 = torch.empty((5,), device=q.device, dtype=torch.float32)
    nbytes = lib.dabsn_hip_read3_workspace_bytes(code, B, T, N, H, 1)
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=q.device)
    ptrs = _lib.PTR4(*[x.data_ptr() for x in g])
    tk = KernelTimer.begin("read3_bwd", q)
    _lib.check(lib.dabsn_hip_read3_bwd(code, B, T, N, H, _p(go), _p(q), _p(K), _p(V), _p(Vn),
                                       _p(ck), _p(cb), _p(kb), _p(adm), _p(sc), _p(idx),
                                       _p(valid), mode, ptrs, _p(gq), _p(gK), _p(gV), _p(gVn),
                                       _p(gck), _p(gcb), _p(gkb), _p(gadm), _p(g5), _p(ws),
                                       ws.numel(), _stream(q)), "three-way read backward")
    KernelTimer.end(tk)
    return (gq, gK.to(bank_keys.dtype), gV.to(bank_writes.dtype), gVn.to(next_writes.dtype),
            gck.to(cocktail.dtype), gcb.to(bank_cocktail.dtype), gkb.to(bank_key_bias.dtype),
            gadm.to(bank_admission.dtype),
            *(g.reshape_as(x).to(x.dtype) for g, x in zip(
                _separate(g5, 5), (scale, short_gain, pad_gain, induct_gain, cocktail_gain))))


@admitted_three_way_read_compact_flash_backward.register_fake
def _read_backward_fake(grad_output, query, bank_keys, bank_writes, next_writes, cocktail,
                        bank_cocktail, bank_key_bias, bank_admission, scale, bank_idx, bank_valid,
                        mode, short_gain, pad_gain, induct_gain, cocktail_gain):
    return tuple(torch.empty_like(v) for v in (
        query, bank_keys, bank_writes, next_writes, cocktail, bank_cocktail, bank_key_bias,
        bank_admission, scale, short_gain, pad_gain, induct_gain, cocktail_gain))


def _read_setup(ctx, inputs, output):
    ctx.save_for_backward(*inputs[:11], *inputs[12:])
    ctx.mode = int(inputs[11])


def _read_bwd(ctx, grad_output):
    t = ctx.saved_tensors
    g = admitted_three_way_read_compact_flash_backward(grad_output, *t[:11], ctx.mode, *t[11:])
    return (*g[:9], None, None, None, *g[9:])


torch.library.register_autograd(_q("admitted_three_way_read_compact_flash"), _read_bwd,
                                setup_context=_read_setup)


# ---------------------------------------------------------------------------
# Dense-mask three-way read (admitted.py:383-622)
# ---------------------------------------------------------------------------
def _dense_inputs(query, bank_keys, bank_writes, next_writes, cocktail, bank_cocktail,
                  bank_key_bias, bank_admission, scale, allow, induct_allow, eligible,
                  induct_eligible, short_gain, pad_gain, induct_gain, cocktail_gain):
    """fp32 contiguous operands (the reference's compute dtype), byte masks and the [5]
    device scalars in schema order, after the reference's shape contract."""
    _require_cuda(query)
    if query.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise TypeError(f"admitted_three_way_read_native: unsupported dtype {query.dtype} on "
                        "the device (fp32, bf16 and fp16 compute in fp32)")
    B, T, H = query.shape
    N = bank_keys.shape[1]
    shapes = {"bank_keys": (B, N, H), "bank_writes": (B, N, H), "next_writes": (B, N, H),
              "cocktail": (B, T, 4), "bank_cocktail": (B, N, 4), "bank_key_bias": (B, N),
              "bank_admission": (B, N), "allow": (B, T, N), "induct_allow": (B, T, N),
              "eligible": (B, T), "induct_eligible": (B, T)}
    given = dict(bank_keys=bank_keys, bank_writes=bank_writes, next_writes=next_writes,
                 cocktail=cocktail, bank_cocktail=bank_cocktail, bank_key_bias=bank_key_bias,
                 bank_admission=bank_admission, allow=allow, induct_allow=induct_allow,
                 eligible=eligible, induct_eligible=induct_eligible)
    for name, want in shapes.items():
        if tuple(given[name].shape) != want:
            raise ValueError(f"admitted_three_way_read_native: {name} has shape "
                             f"{tuple(given[name].shape)}, expected {want}")
    for name in ("allow", "induct_allow", "eligible", "induct_eligible"):
        if given[name].dtype != torch.bool:
            raise TypeError(f"admitted_three_way_read_native: {name} must be torch.bool")
    floats = [x.float().contiguous() for x in (query, bank_keys, bank_writes, next_writes,
                                               cocktail, bank_cocktail, bank_key_bias,
                                               bank_admission)]
    masks = [x.contiguous().view(torch.uint8) for x in (allow, induct_allow, eligible,
                                                        induct_eligible)]
    scal = torch.stack([_f32_scalar(x) for x in (scale, short_gain, pad_gain, induct_gain,
                                                 cocktail_gain)])
    return (B, T, N, H), floats, masks, scal


@torch.library.custom_op(_q("admitted_three_way_read_native"), mutates_args=(),
                         device_types="cuda")
def admitted_three_way_read_native(
    query: Tensor, bank_keys: Tensor, bank_writes: Tensor, next_writes: Tensor, cocktail: Tensor,
    bank_cocktail: Tensor, bank_key_bias: Tensor, bank_admission: Tensor, scale: Tensor,
    allow: Tensor, induct_allow: Tensor, eligible: Tensor, induct_eligible: Tensor,
    short_gain: Tensor, pad_gain: Tensor, induct_gain: Tensor, cocktail_gain: Tensor,
) -> Tensor:
    """The three-way admitted read with explicit dense masks (reference admitted.py:509-546;
    math admitted.py:16-65): fp32 compute, output in the query's dtype."""
    (B, T, N, H), f, m, scal = _dense_inputs(
        query, bank_keys, bank_writes, next_writes, cocktail, bank_cocktail, bank_key_bias,
        bank_admission, scale, allow, induct_allow, eligible, induct_eligible, short_gain,
        pad_gain, induct_gain, cocktail_gain)
    if min(B, T, N, H) == 0:
        return torch.zeros(query.shape, device=query.device, dtype=query.dtype)
    lib = _lib.load()
    out = torch.empty((B, T, H), device=query.device, dtype=torch.float32)
    nbytes = lib.dabsn_hip_read_dense_workspace_bytes(B, T, N, H, 0)
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=query.device)
    tk = KernelTimer.begin("read_dense_fwd", out)
    _lib.check(lib.dabsn_hip_read_dense_fwd(B, T, N, H, *[_p(x) for x in f], *[_p(x) for x in m],
                                            _p(scal), _p(out), _p(ws), ws.numel(), _stream(out)),
               "dense three-way read")
    KernelTimer.end(tk)
    return out.to(query.dtype)


@admitted_three_way_read_native.register_fake
def _dense_read_fake(query, *rest):
    return torch.empty_like(query)


@torch.library.custom_op(_q("admitted_three_way_read"), mutates_args=(), device_types="cuda")
def admitted_three_way_read(
    query: Tensor, bank_keys: Tensor, bank_writes: Tensor, next_writes: Tensor, cocktail: Tensor,
    bank_cocktail: Tensor, bank_key_bias: Tensor, bank_admission: Tensor, scale: Tensor,
    allow: Tensor, induct_allow: Tensor, eligible: Tensor, induct_eligible: Tensor,
    short_gain: Tensor, pad_gain: Tensor, induct_gain: Tensor, cocktail_gain: Tensor,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """The reference's 4-output dense read (admitted.py:16-65): (output in the query's dtype,
    short, permanent and induction softmax weights [B, T, N] in fp32 for bf16/fp16 queries,
    else in the query's dtype). Registered without autograd here: the reference's own
    formula (admitted.py:126-247) differentiates it from the saved weights in a process
    that binds this kernel to the reference's operator (``reference_backend``); this
    package's reads use the compact and dense-mask operators, which have HIP backwards."""
    (B, T, N, H), f, m, scal = _dense_inputs(
        query, bank_keys, bank_writes, next_writes, cocktail, bank_cocktail, bank_key_bias,
        bank_admission, scale, allow, induct_allow, eligible, induct_eligible, short_gain,
        pad_gain, induct_gain, cocktail_gain)
    wdt = torch.float32 if query.dtype in (torch.float16, torch.bfloat16) else query.dtype
    if min(B, T, N, H) == 0:
        z = torch.zeros((B, T, N), device=query.device, dtype=wdt)
        return (torch.zeros(query.shape, device=query.device, dtype=query.dtype), z, z.clone(),
                z.clone())
    lib = _lib.load()
    out = torch.empty((B, T, H), device=query.device, dtype=torch.float32)
    w = [torch.empty((B, T, N), device=query.device, dtype=torch.float32) for _ in range(3)]
    nbytes = lib.dabsn_hip_read_dense_workspace_bytes(B, T, N, H, 0)
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=query.device)
    _lib.check(lib.dabsn_hip_read_dense_fwd_weights(
        B, T, N, H, *[_p(x) for x in f], *[_p(x) for x in m], _p(scal), _p(out),
        *[_p(x) for x in w], _p(ws), ws.numel(), _stream(out)), "dense three-way read")
    return (out.to(query.dtype), *[x.to(wdt) for x in w])


@admitted_three_way_read.register_fake
def _dense_read4_fake(query, bank_keys, *rest):
    B, T, _ = query.shape
    N = bank_keys.shape[1]
    wdt = torch.float32 if query.dtype in (torch.float16, torch.bfloat16) else query.dtype
    w = query.new_empty((B, T, N), dtype=wdt)
    return torch.empty_like(query), w, w.clone(), w.clone()


@torch.library.custom_op(_q("_admitted_three_way_read_backward"), mutates_args=(),
                         device_types="cuda")
def admitted_three_way_read_native_backward(
    grad_output: Tensor, query: Tensor, bank_keys: Tensor, bank_writes: Tensor,
    next_writes: Tensor, cocktail: Tensor, bank_cocktail: Tensor, bank_key_bias: Tensor,
    bank_admission: Tensor, scale: Tensor, allow: Tensor, induct_allow: Tensor,
    eligible: Tensor, induct_eligible: Tensor, short_gain: Tensor, pad_gain: Tensor,
    induct_gain: Tensor, cocktail_gain: Tensor,
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor,
           Tensor, Tensor, Tensor]:
    """Gradients of the 13 float inputs (reference admitted.py:383-453, math :126-236), each
    in its input's dtype: query, bank_keys, bank_writes, next_writes, cocktail,
    bank_cocktail, bank_key_bias, bank_admission, scale, short_gain, pad_gain, induct_gain,
    cocktail_gain."""
    inputs = (query, bank_keys, bank_writes, next_writes, cocktail, bank_cocktail, bank_key_bias,
              bank_admission)
    gains = (scale, short_gain, pad_gain, induct_gain, cocktail_gain)
    (B, T, N, H), f, m, scal = _dense_inputs(*inputs, scale, allow, induct_allow, eligible,
                                             induct_eligible, short_gain, pad_gain, induct_gain,
                                             cocktail_gain)
    dev = query.device
    grads = [torch.zeros(x.shape, device=dev, dtype=torch.float32) for x in inputs]
    gscal = torch.zeros(5, device=dev, dtype=torch.float32)
    if min(B, T, N, H) > 0:
        lib = _lib.load()
        go = grad_output.float().contiguous()
        nbytes = lib.dabsn_hip_read_dense_workspace_bytes(B, T, N, H, 1)
        ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=dev)
        tk = KernelTimer.begin("read_dense_bwd", go)
        _lib.check(lib.dabsn_hip_read_dense_bwd(
            B, T, N, H, _p(go), *[_p(x) for x in f], *[_p(x) for x in m], _p(scal),
            *[_p(g) for g in grads], _p(gscal), _p(ws), ws.numel(), _stream(go)),
            "dense three-way read backward")
        KernelTimer.end(tk)
    out = [g.to(x.dtype) for g, x in zip(grads, inputs)]
    out += [gscal[i].reshape(x.shape).to(x.dtype, copy=True) for i, x in enumerate(gains)]
    return tuple(out)


@admitted_three_way_read_native_backward.register_fake
def _dense_read_backward_fake(grad_output, query, bank_keys, bank_writes, next_writes, cocktail,
                              bank_cocktail, bank_key_bias, bank_admission, scale, allow,
                              induct_allow, eligible, induct_eligible, short_gain, pad_gain,
                              induct_gain, cocktail_gain):
    return tuple(torch.empty_like(x) for x in (
        query, bank_keys, bank_writes, next_writes, cocktail, bank_cocktail, bank_key_bias,
        bank_admission, scale, short_gain, pad_gain, induct_gain, cocktail_gain))


def _dense_read_setup(ctx, inputs, output):
    ctx.save_for_backward(*inputs)


def _dense_read_bwd(ctx, grad_output):
    g = admitted_three_way_read_native_backward(grad_output, *ctx.saved_tensors)
    return (*g[:9], None, None, None, None, *g[9:])


torch.library.register_autograd(_q("admitted_three_way_read_native"), _dense_read_bwd,
                                setup_context=_dense_read_setup)


# The training path of the read: the forward keeps its workspace (tile ranges, scores and
# row statistics) for the backward, which then skips the recompute of the score GEMM and
# the softmax rows. The registered op above keeps the reference's one-output schema for
# external callers; the read module uses ``admitted_three_way_read_train``.
@torch.library.custom_op(_q("_read3_fwd_keep"), mutates_args=(), device_types="cuda")
def read3_fwd_keep(
    query: Tensor, bank_keys: Tensor, bank_writes: Tensor, next_writes: Optional[Tensor],
    cocktail: Tensor, bank_cocktail: Tensor, bank_key_bias: Tensor, bank_admission: Tensor,
    scale: Tensor, bank_idx: Tensor, bank_valid: Tensor, mode: int, short_gain: Tensor,
    pad_gain: Tensor, induct_gain: Tensor, cocktail_gain: Tensor, fold: Optional[Tensor] = None,
) -> tuple[Tensor, Tensor]:
    """The three-way read forward; returns (out, kept) where ``kept`` holds the scores, tile
    ranges and row statistics that ``read3_bwd_kept`` reads (the forward's other scratch is
    released when the call returns). ``fold`` (int8 [B, N], ``bank_fold`` codes 0/1 only)
    states next_writes[j] = bank_writes[j + fold[j]]; next_writes may then be None."""
    _require_cuda(query)
    lib = _lib.load()
    if mode not in (0, 1):
        raise ValueError("compact admitted-read mode must be 0 (seq) or 1 (field)")
    dt, q, K, V, Vn, ck, cb, kb, adm, sc, g, idx, valid = _read_common(
        query, bank_keys, bank_writes, next_writes, cocktail, bank_cocktail, bank_key_bias,
        bank_admission, scale, bank_idx, bank_valid,
        (short_gain, pad_gain, induct_gain, cocktail_gain))
    B, T, H = q.shape
    N = K.shape[1]
    code = _code(dt)
    fc = _fold_codes(fold, B, N, Vn)
    out = torch.empty_like(q)
    kept = torch.empty(max(lib.dabsn_hip_read3_workspace_bytes(code, B, T, N, H, 2), 256),
                       dtype=torch.uint8, device=q.device)
    scratch = torch.empty(max(lib.dabsn_hip_read3_workspace_bytes(code, B, T, N, H, 3), 256),
                          dtype=torch.uint8, device=q.device)
    ptrs = _lib.PTR4(*[x.data_ptr() for x in g])
    tk = KernelTimer.begin("read3_fwd", q)
    _lib.check(lib.dabsn_hip_read3_fwd_keep(
        code, B, T, N, H, _p(q), _p(K), _p(V), _p(Vn), _p(ck), _p(cb), _p(kb), _p(adm), _p(sc),
        _p(idx), _p(valid), _p(fc), mode, ptrs, _p(out), _p(kept), kept.numel(), _p(scratch),
        scratch.numel(), _stream(q)), "three-way read")
    KernelTimer.end(tk)
    return out, kept


@read3_fwd_keep.register_fake
def _read3_fwd_keep_fake(query, *rest):
    return torch.empty_like(query), query.new_empty((256,), dtype=torch.uint8)


def _fold_codes(fold: Optional[Tensor], B: int, N: int, Vn: Optional[Tensor]) -> Optional[Tensor]:
    """The fold codes as the kernels take them (int8 [B, N], contiguous), or None; without
    them the successor rows must be given."""
    if fold is None:
        if Vn is None:
            raise ValueError("three-way read: next_writes may be None only with a fold")
        return None
    if fold.shape != (B, N):
        raise ValueError(f"three-way read: fold must be [B, N] = {(B, N)}, got {tuple(fold.shape)}")
    return fold.to(torch.int8).contiguous()


@torch.library.custom_op(_q("_read3_bwd_kept"), mutates_args=(), device_types="cuda")
def read3_bwd_kept(
    grad_output: Tensor, query: Tensor, bank_keys: Tensor, bank_writes: Tensor,
    next_writes: Optional[Tensor], cocktail: Tensor, bank_cocktail: Tensor, bank_key_bias: Tensor,
    bank_admission: Tensor, scale: Tensor, bank_idx: Tensor, bank_valid: Tensor, mode: int,
    short_gain: Tensor, pad_gain: Tensor, induct_gain: Tensor, cocktail_gain: Tensor,
    workspace: Tensor, fold: Optional[Tensor] = None,
) -> CompactGradients:
    """``admitted_three_way_read_compact_flash_backward`` on the kept buffer of a
    ``read3_fwd_keep`` call with the same inputs (``dabsn_hip_read3_bwd_after_fwd``). The
    kept buffer is only read, so a second backward through the same graph sees it
    unchanged. With ``fold`` the successor-row gradient is part of the bank-write gradient
    and the next_writes gradient comes back empty ([0])."""
    _require_cuda(query)
    lib = _lib.load()
    dt, q, K, V, Vn, ck, cb, kb, adm, sc, g, idx, valid = _read_common(
        query, bank_keys, bank_writes, next_writes, cocktail, bank_cocktail, bank_key_bias,
        bank_admission, scale, bank_idx, bank_valid,
        (short_gain, pad_gain, induct_gain, cocktail_gain))
    B, T, H = q.shape
    N = K.shape[1]
    fc = _fold_codes(fold, B, N, Vn)
    go = grad_output.to(dt).contiguous()
    gq = torch.empty_like(q)
    gK, gV = (torch.empty((B, N, H), device=q.device, dtype=dt) for _ in range(2))
    gVn = (torch.empty((B, N, H), device=q.device, dtype=dt) if fc is None
           else q.new_empty((0,)))
    gck = torch.empty((B, T, 4), device=q.device, dtype=torch.float32)
    gcb = torch.empty((B, N, 4), device=q.device, dtype=torch.float32)
    gkb = torch.empty((B, N), device=q.device, dtype=torch.float32)
    gadm = torch.empty((B, N), device=q.device, dtype=torch.float32)
    g5 = torch.empty((5,), device=q.device, dtype=torch.float32)
    scratch = torch.empty(max(lib.dabsn_hip_read3_workspace_bytes(_code(dt), B, T, N, H, 4), 256),
                          dtype=torch.uint8, device=q.device)
    ptrs = _lib.PTR4(*[x.data_ptr() for x in g])
    tk = KernelTimer.begin("read3_bwd", q)
    _lib.check(lib.dabsn_hip_read3_bwd_after_fwd(
        _code(dt), B, T, N, H, _p(go), _p(q), _p(K), _p(V), _p(Vn), _p(ck), _p(cb), _p(kb),
        _p(adm), _p(sc), _p(idx), _p(valid), _p(fc), mode, ptrs, _p(gq), _p(gK), _p(gV),
        None if fc is not None else _p(gVn), _p(gck), _p(gcb), _p(gkb), _p(gadm), _p(g5),
        _p(workspace), workspace.numel(), _p(scratch), scratch.numel(), _stream(q)),
        "three-way read backward")
    KernelTimer.end(tk)
    return (gq, gK.to(bank_keys.dtype), gV.to(bank_writes.dtype),
            gVn if next_writes is None else gVn.to(next_writes.dtype),
            gck.to(cocktail.dtype), gcb.to(bank_cocktail.dtype), gkb.to(bank_key_bias.dtype),
            gadm.to(bank_admission.dtype),
            *(g.reshape_as(x).to(x.dtype) for g, x in zip(
                _separate(g5, 5), (scale, short_gain, pad_gain, induct_gain, cocktail_gain))))


@read3_bwd_kept.register_fake
def _read3_bwd_kept_fake(grad_output, query, bank_keys, bank_writes, next_writes, cocktail,
                         bank_cocktail, bank_key_bias, bank_admission, scale, bank_idx, bank_valid,
                         mode, short_gain, pad_gain, induct_gain, cocktail_gain, workspace,
                         fold=None):
    gvn = query.new_empty((0,)) if fold is not None else torch.empty_like(next_writes)
    return tuple(torch.empty_like(v) if v is not None else gvn for v in (
        query, bank_keys, bank_writes, None, cocktail, bank_cocktail, bank_key_bias,
        bank_admission, scale, short_gain, pad_gain, induct_gain, cocktail_gain))


class _Read3Train(torch.autograd.Function):
    """Inputs: the 16 of the compact read (next_writes may be None with a fold), then the
    fold codes or None."""

    @staticmethod
    def forward(ctx, *inputs):
        fold = inputs[16]
        out, ws = read3_fwd_keep(*inputs[:16], fold)
        ctx.save_for_backward(*inputs[:11], *inputs[12:16], ws, fold)
        ctx.mode = int(inputs[11])
        return out

    @staticmethod
    def backward(ctx, grad_output):
        t = ctx.saved_tensors
        fold = t[16]
        g = read3_bwd_kept(grad_output.contiguous(), *t[:11], ctx.mode, *t[11:15], t[15], fold)
        gvn = None if fold is not None else g[3]
        return (*g[:3], gvn, *g[4:9], None, None, None, *g[9:], None)


def admitted_three_way_read_train(*inputs, fold: Optional[Tensor] = None) -> Tensor:
    """``admitted_three_way_read_compact_flash`` (same 16 inputs and result) for callers
    that will differentiate it: under autograd the forward's workspace is kept for the
    backward; otherwise this is the registered op. ``fold``: successor-fold codes
    (``bank_fold``) for a bank whose successor rows are bank rows; inputs[3] (next_writes)
    may then be None."""
    if inputs[0].is_cuda and torch.is_grad_enabled() and any(
            isinstance(x, Tensor) and x.requires_grad for x in inputs):
        return _Read3Train.apply(*inputs, fold)
    if fold is not None:
        return read3_fwd_keep(*inputs, fold)[0]
    return admitted_three_way_read_compact_flash(*inputs)


def kernel_symbol(kernel: str, B: int, H: int, dtype: torch.dtype = torch.bfloat16) -> Optional[str]:
    """Profiler symbol of the core-scan kernel instance used for (B, H, dtype)."""
    if kernel not in ("core_scan_fwd", "core_scan_bwd"):
        return None
    lib = _lib.load()
    ch, ks, nw = _lib.i32(), _lib.i32(), _lib.i32()
    if lib.dabsn_hip_core_scan_config(_code(dtype), B, H, ctypes.byref(ch), ctypes.byref(ks),
                                      ctypes.byref(nw)) != 0:
        return None
    e = "unsigned short" if dtype == torch.bfloat16 else "float"
    which, args = ("fwd", "FwdArgs") if kernel == "core_scan_fwd" else ("bwd", "BwdArgs")
    return (f"void dabsn::core::core_{which}_kernel<{e}, {ch.value}, {ks.value}, {nw.value}>"
            f"(dabsn::core::{args}<{e}>)")


OPERATORS = (
    _q("core_scan_batched"),
    _q("_core_scan_batched_backward"),
    _q("linear_recurrence"),
    _q("_linrec_backward"),
    _q("permanent_delta_scan"),
    _q("_permanent_delta_scan_backward"),
    _q("local_field_gather"),
    _q("_local_field_gather_backward"),
    _q("_ce_rows"),
    _q("_ce_rows_backward"),
    _q("long_scan_fused"),
    _q("_long_scan_fused_backward"),
    _q("read_tape_stats"),
    _q("_read_tape_stats_backward"),
    _q("normalize_rows"),
    _q("_normalize_rows_backward"),
    _q("bank_select"),
    _q("bank_gather"),
    _q("bank_gather_kv"),
    _q("_bank_gather_backward"),
    _q("admitted_three_way_read_compact_flash"),
    _q("_admitted_three_way_read_compact_flash_backward"),
    _q("_read3_fwd_keep"),
    _q("_read3_bwd_kept"),
    _q("read_output"),
    _q("_read_output_backward"),
    _q("admitted_three_way_read_native"),
    _q("_admitted_three_way_read_backward"),
)


if NAMESPACE != "dabsn":
    events.emit_event(events.EventCode.PROVIDER_RESOLUTION, component_id="dabsn_amd.kernels.ops",
                      namespace=NAMESPACE,
                      reason="DABSN_AMD_OP_NAMESPACE is set" if os.environ.get(
                          "DABSN_AMD_OP_NAMESPACE") else
                      "the reference's dabsn:: operators are registered in this process")


# ---- block glue (inference on the device, no autograd) ----------------------------------
def _same_dtype(*ts: Tensor) -> bool:
    dt = ts[0].dtype
    return dt in _DTYPES and all(t.dtype == dt and t.is_cuda for t in ts)


def read_mix(proj: Tensor, long: Tensor, long_gain: Tensor, y: Tensor,
             read_gain: Tensor) -> Tensor:
    """``y + read_gain * (proj + long_gain * long)`` in one pass: the read's output
    (read.py:435, 821) fed into the block's mix (model.py:336), each product and sum
    rounded to the common dtype as the unfused tensor operations round them. All five
    tensors share one dtype (the gains hold one element each)."""
    if not _same_dtype(proj, long, long_gain, y, read_gain) or proj.shape != long.shape \
            or proj.shape != y.shape or long_gain.numel() != 1 or read_gain.numel() != 1:
        raise ValueError("read_mix: proj, long and y must match and share the gains' dtype")
    lib = _lib.load()
    pc, lc, yc = proj.contiguous(), long.contiguous(), y.contiguous()
    # held until the launch: a temporary's block could be handed to the next allocation
    lg, rg = _f32_scalar(long_gain), _f32_scalar(read_gain)
    out = torch.empty_like(yc)
    _lib.check(lib.dabsn_hip_read_mix(_code(pc.dtype), pc.numel(), _p(pc), _p(lc), _p(lg),
                                      _p(yc), _p(rg), _p(out), _stream(pc)), "read mix")
    return out


def rms_norm(x: Tensor, weight: Tensor, eps: float) -> Tensor:
    """MLPRMSNorm (model.py:35-45) in one kernel: ``(x.float() * rsqrt(mean(x^2) + eps))``
    rounded to x's dtype, times ``weight`` (same dtype as x)."""
    if not _same_dtype(x, weight) or weight.dim() != 1 or weight.shape[0] != x.shape[-1]:
        raise ValueError("rms_norm: x and weight [H] must share a dtype on the device")
    lib = _lib.load()
    xc, wc = x.contiguous(), weight.contiguous()
    H = int(x.shape[-1])
    out = torch.empty_like(xc)
    _lib.check(lib.dabsn_hip_rms_norm(_code(xc.dtype), xc.numel() // H, H, _p(xc), _p(wc),
                                      float(eps), _p(out), _stream(xc)), "rms norm")
    return out


def relu_square(x: Tensor) -> Tensor:
    """``F.relu(x).square()`` in one kernel."""
    if not _same_dtype(x):
        raise ValueError("relu_square: a float32 or bfloat16 device tensor is required")
    lib = _lib.load()
    xc = x.contiguous()
    out = torch.empty_like(xc)
    _lib.check(lib.dabsn_hip_relu_square(_code(xc.dtype), xc.numel(), _p(xc), _p(out),
                                         _stream(xc)), "relu square")
    return out


def _direct(op):
    """``op`` with the dispatcher skipped where nothing needs it: inside
    ``reuse_parameter_copies()`` with autograd off and device inputs, the op's body is
    called as a plain function (about 15 µs less host time per call, and streaming decode
    makes ~30 such calls per token); anywhere else the registered operator runs."""
    body = getattr(op, "_init_fn", None)  # the undecorated function (torch's CustomOpDef)
    if body is None:
        return op

    def call(*args):
        if _REUSE_DEPTH and not torch.is_grad_enabled() and args[0].is_cuda:
            return body(*args)
        return op(*args)

    call.__name__ = call.__qualname__ = body.__name__
    return call


class direct:
    """The inference call sites' entry to the operators above (see ``_direct``)."""

    core_scan_batched = staticmethod(_direct(core_scan_batched))
    long_scan_fused = staticmethod(_direct(long_scan_fused))
    read_tape_stats = staticmethod(_direct(read_tape_stats))
    normalize_rows = staticmethod(_direct(normalize_rows))
    bank_select = staticmethod(_direct(bank_select))
    read_output = staticmethod(_direct(read_output))
