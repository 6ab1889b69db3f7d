"""The pipelined scan + read (``dabsn_amd/kernels/pipeline.py``) against the same block run
one piece after the other (time-chunked core scan, then the whole-sequence read).

The pipeline reads each query chunk against the bank that ends with it (read.py:650-838,
the same rows as the whole-sequence read) and sums the tape gradients chunk by chunk, so
only summation orders differ:
  * the trajectory halves y and budget: bit-identical (the same scan kernels, launched
    plainly on a CU-masked stream instead of cooperatively);
  * fp32: read output and every gradient (input projections, core and read parameters)
    normwise 1e-5, the scalar parameter gradients (sums of O(B*T*N) terms) included;
  * bf16 at state width 2048 (the config-4 kernel instances): read output and gradients
    Frobenius 2e-2 from the sequential bf16 run;
  * bf16 at width 512, where the fp32 scan runs too: every gradient within max(2e-2, 1.5 x
    the sequential bf16 run's own distance) of the block run in fp32 (scalar gradients that
    sum many cancelling terms move by up to a few 1e-2 under bf16 rounding in either
    schedule);
  * dense banks (the successor fold) and partially admitted ones (no fold, a bank width
    that grows chunk by chunk); losses with and without budget (a block mixes only y into
    its output); a DABSNBlock with block chunking, pipelined or not;
  * the window entry points the pipeline hands its pieces through (read output and its
    backward per window, window copies and adds) against the whole-tensor operations.
"""

from __future__ import annotations


import pytest
import torch

import dabsn_amd
from dabsn_amd.kernels import pipeline
from dabsn_amd.kernels.chunked import chunked_core_scan

pytestmark = pytest.mark.gpu


def _modules(seed, din, H, window, dev):
    torch.manual_seed(seed)
    core = dabsn_amd.DABSNCore(din, H).to(dev)
    read = dabsn_amd.DABSNRead(H).to(dev)
    read.admit_window.data.fill_(window)
    return core, read


def _sequential(core, read, chunk, Wx, Wgx):
    B, T, H = Wx.shape
    z = torch.zeros(B, H, device=Wx.device, dtype=torch.float32)
    outs = chunked_core_scan(chunk, Wx, Wgx, *core.scan_inputs(), z, torch.ones_like(z), z.clone())
    U, nov, p, ay, w, e, c = outs[:7]
    y, budget = U.split(H, dim=-1)
    return y, budget, read(y, budget, ay, w, nov, p, e, c)


def _run(fn, core, read, x, ups, dtype):
    """Outputs (y, budget, read) of ``fn`` and every gradient of a backward from the
    upstream gradients ``ups`` (None: that output takes no part in the loss)."""
    core.zero_grad(set_to_none=True)
    read.zero_grad(set_to_none=True)
    xl = x.clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=dtype, enabled=dtype != torch.float32):
        Wx, Wgx = core.projections(xl)
        outs = fn(core, read, Wx, Wgx)
    pairs = [(o, u.to(o.dtype)) for o, u in zip(outs, ups) if u is not None]
    torch.autograd.backward([o for o, _ in pairs], [u for _, u in pairs])
    grads = {"x": xl.grad}
    for prefix, m in (("core", core), ("read", read)):
        for n, p in m.named_parameters():
            if p.grad is not None:
                grads[f"{prefix}.{n}"] = p.grad.detach().clone()
    return [o.detach() for o in outs], grads, read.last_n_max


def _rel(a, b, fro, floor=1e-30):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    if fro:
        return float((a - b).norm() / max(float(b.norm()), floor * b.numel() ** 0.5))
    return float((a - b).abs().max() / max(float(b.abs().max()), floor))


def _floor(grads):
    """Parameters such as null_bias and adm_bias shift every logit of a softmax equally: their
    exact gradient is zero and both runs hold rounding noise, so gradient errors are taken
    relative to max(|grad|, 1e-3 x the largest parameter gradient)."""
    return 1e-3 * max(float(g.abs().max()) for g in grads.values())


@pytest.mark.parametrize("dtype,B,T,H,chunk,window,ref32,budget_grad", [
    (torch.float32, 3, 96, 64, 32, 50.0, False, True),
    (torch.float32, 3, 96, 64, 32, 0.3, False, False),
    (torch.float32, 2, 100, 48, 24, 50.0, False, True),
    (torch.bfloat16, 16, 512, 2048, 128, 50.0, False, True),
    (torch.bfloat16, 16, 384, 2048, 128, 0.3, False, False),
    (torch.bfloat16, 16, 512, 512, 128, 50.0, True, True),
])
def test_pipelined_scan_read_matches_sequential(cuda_device, dtype, B, T, H, chunk, window,
                                                ref32, budget_grad):
    din = 32
    core, read = _modules(11 + T, din, H, window, cuda_device)
    g = torch.Generator().manual_seed(12)
    x = torch.randn(B, T, din, generator=g).to(cuda_device)
    gy, gb = ((torch.randn(B, T, H, generator=g) * 1e-2).to(cuda_device) for _ in range(2))
    gr = torch.randn(B, T, H, generator=g).to(cuda_device)
    ups = (gy, gb if budget_grad else None, gr)

    def piped(c, r, Wx, Wgx):
        return pipeline.pipelined_scan_read(r, chunk, Wx, Wgx, c.scan_inputs())

    def seq(c, r, Wx, Wgx):
        return _sequential(c, r, chunk, Wx, Wgx)

    (y1, b1, r1), g1, n1 = _run(piped, core, read, x, ups, dtype)
    (y0, b0, r0), g0, n0 = _run(seq, core, read, x, ups, dtype)
    assert n1 == n0
    assert torch.equal(y1, y0) and torch.equal(b1, b0), "trajectory"
    fro = dtype != torch.float32
    tol = 2e-2 if fro else 1e-5
    assert _rel(r1, r0, fro) <= tol, f"read output {_rel(r1, r0, fro):.3e}"
    assert g1.keys() == g0.keys()
    worst = ("", 0.0)
    if not ref32:
        floor = _floor(g0)
        for n in g0:
            err = _rel(g1[n], g0[n], fro, floor)
            assert err <= tol, f"gradient {n}: {err:.3e}"
            worst = max(worst, (n, err), key=lambda v: v[1])
    else:
        _, gf, _ = _run(seq, core, read, x, ups, torch.float32)
        floor = _floor(gf)
        for n in gf:
            err = _rel(g1[n], gf[n], True, floor)
            ref = _rel(g0[n], gf[n], True, floor)
            assert err <= max(tol, 1.5 * ref), f"gradient {n}: {err:.3e} (sequential bf16 {ref:.3e})"
            worst = max(worst, (n, err), key=lambda v: v[1])
    print(f"pipelined vs sequential ({dtype}, B={B} T={T} H={H}, n_max={n1}): "
          f"output {_rel(r1, r0, fro):.2e}, worst gradient {worst[0]} {worst[1]:.2e}")


def test_block_pipelined_matches_sequential(cuda_device, monkeypatch):
    """A seq DABSNBlock with block chunking in training mode takes the pipeline; with
    DABSN_PIPELINE=0 it runs the chunked scan and then the read (fp32, 1e-5, scalars included)."""
    torch.manual_seed(3)
    blk = dabsn_amd.DABSNBlock(24, 48, 40, "seq", residual=True, mlp_ratio=2.0,
                               block_chunk_t=32).to(cuda_device)
    blk.train()
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 100, 24, generator=g).to(cuda_device)
    w = torch.randn(2, 100, 48, generator=g).to(cuda_device)

    def run(flag):
        monkeypatch.setenv("DABSN_PIPELINE", flag)
        blk.zero_grad(set_to_none=True)
        xl = x.clone().requires_grad_(True)
        out = blk(xl)
        (out * w).sum().backward()
        grads = {n: p.grad.detach().clone() for n, p in blk.named_parameters() if p.grad is not None}
        return out.detach(), xl.grad, grads

    o1, gx1, g1 = run("1")
    o0, gx0, g0 = run("0")
    assert _rel(o1, o0, False) <= 1e-5
    assert _rel(gx1, gx0, False) <= 1e-5
    assert g1.keys() == g0.keys()
    floor = _floor(g0)
    for n in g0:
        err = _rel(g1[n], g0[n], False, floor)
        assert err <= 1e-5, f"{n}: {err:.3e}"


@pytest.mark.parametrize("dtypes", [(torch.bfloat16, torch.bfloat16, torch.float32),
                                    (torch.float32, torch.float32, torch.float32),
                                    (torch.bfloat16, torch.bfloat16, torch.bfloat16)])
@pytest.mark.parametrize("B,T,H,bounds", [(3, 40, 24, [(0, 16), (16, 31), (31, 40)]),
                                          (2, 17, 5, [(0, 9), (9, 17)])])
def test_read_output_windows_equal_the_whole_op(cuda_device, dtypes, B, T, H, bounds):
    """``ops.read_output_window`` / ``read_output_bwd_window`` over a partition of the time
    axis against ``read_output`` and its backward on the whole tensors: outputs and the
    projection / long gradients bit for bit (the same arithmetic per element, vector path at
    H = 24, scalar path at H = 5), the gain gradient as the sum of the window shares (another
    summation order: within 1e-6 of the sum of its terms' magnitudes). Every other window
    passes its inputs (forward) or outputs (backward) as contiguous [B, C, H] blocks beside
    time-window views of the full tensors, so the tensors' batch strides differ."""
    from dabsn_amd.kernels import ops

    pd, ld, gd = dtypes
    g = torch.Generator().manual_seed(T + H)
    proj = torch.randn(B, T, H, generator=g).to(cuda_device, pd)
    lng = torch.randn(B, T, H, generator=g).to(cuda_device, ld)
    gain = torch.tensor([0.37], device=cuda_device, dtype=gd).reshape(())
    whole = ops.read_output(proj, lng, gain)
    out = torch.full_like(whole, float("nan"))
    for k, (t0, t1) in enumerate(bounds):
        p_k, l_k = proj[:, t0:t1], lng[:, t0:t1]
        if k % 2:
            p_k, l_k = p_k.contiguous(), l_k.contiguous()
        ops.read_output_window(p_k, l_k, gain, out[:, t0:t1])
    assert torch.equal(out, whole)

    grad = torch.randn(B, T, H, generator=g).to(cuda_device, whole.dtype)
    gp_w, gl_w, gg_w = ops.read_output_backward(grad, lng, gain, ops._code(pd))
    gp, gl = torch.empty_like(proj), torch.empty_like(lng)
    shares = torch.zeros(len(bounds), device=cuda_device, dtype=torch.float32)
    for k, (t0, t1) in enumerate(bounds):
        if k % 2:
            gp_k, gl_k = torch.empty_like(gp[:, t0:t1]), torch.empty_like(gl[:, t0:t1])
        else:
            gp_k, gl_k = gp[:, t0:t1], gl[:, t0:t1]
        ops.read_output_bwd_window(grad[:, t0:t1], lng[:, t0:t1], gain, gp_k, gl_k,
                                   shares[k:k + 1])
        if k % 2:
            gp[:, t0:t1], gl[:, t0:t1] = gp_k, gl_k
    assert torch.equal(gp, gp_w) and torch.equal(gl, gl_w)
    want = float(gg_w.float())
    # Relative to the sum of |terms|: the gain's gradient sums B*T*H products of both signs.
    scale = float((grad.double() * lng.double()).abs().sum())
    # read_output_backward returns the gain's gradient in the gain's dtype (bf16: rounded).
    rounding = abs(want) * 2.0 ** -8 if gd == torch.bfloat16 else 0.0
    assert abs(float(shares.sum()) - want) <= 1e-6 * scale + rounding


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("B,T,H,t0,t1", [(3, 100, 24, 37, 90), (2, 70, 5, 0, 33),
                                         (1, 40, 8, 8, 40)])
def test_long_scan_on_tape_windows_equals_contiguous_copies(cuda_device, dtype, B, T, H, t0, t1):
    """``ops.long_scan_window`` and ``long_scan_backward_parts`` read time windows of longer
    tapes in place (the batch stride passed to the library): the same outputs, final states,
    checkpoint and gradients as on contiguous copies of the windows, bit for bit; and with
    ``gw_into`` / ``gp_into`` windows of full-length buffers, the write gradient added into
    its window as ``window_add`` adds it and the plasticity gradient written into its own,
    bit for bit, the rows outside the windows untouched."""
    from dabsn_amd.kernels import ops

    g = torch.Generator().manual_seed(T + H + t0)
    w = torch.randn(B, T, H, generator=g).to(cuda_device, dtype)
    pl = torch.rand(B, T, H, generator=g).to(cuda_device, dtype)
    logits = [torch.tensor([v], device=cuda_device) for v in (0.3, -0.2, 0.5, 0.1)]
    state = [torch.randn(B, H, generator=g).to(cuda_device) for _ in range(3)]
    wk, pk = w[:, t0:t1], pl[:, t0:t1]
    a = ops.long_scan_window(wk, pk, logits, *state)
    b = ops.long_scan_window(wk.contiguous(), pk.contiguous(), logits, *state)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    gl = torch.randn(B, t1 - t0, H, generator=g).to(cuda_device, dtype)
    gf = [torch.randn(B, H, generator=g).to(cuda_device) for _ in range(3)]
    ga = ops.long_scan_backward_parts(wk, pk, logits, a[4], gl, *gf)
    gb = ops.long_scan_backward_parts(wk.contiguous(), pk.contiguous(), logits, a[4], gl, *gf)
    for x, y in zip(ga[:3], gb[:3]):
        assert torch.equal(x, y)
    for x, y in zip(ga[3], gb[3]):
        assert torch.equal(x, y)
    sink = torch.randn(B, T, H, generator=g).to(cuda_device, dtype)
    gpb = torch.randn(B, T, H, generator=g).to(cuda_device, dtype)
    want_sink, want_gp = sink.clone(), gpb.clone()
    ops.window_add(want_sink[:, t0:t1], want_sink[:, t0:t1], ga[0])
    want_gp[:, t0:t1] = ga[1]
    gc = ops.long_scan_backward_parts(wk, pk, logits, a[4], gl, *gf, gw_into=sink[:, t0:t1],
                                      gp_into=gpb[:, t0:t1])
    assert torch.equal(sink, want_sink) and torch.equal(gpb, want_gp)
    assert torch.equal(gc[2], ga[2])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("H", [24, 5])
def test_window_add_equals_torch(cuda_device, dtype, H):
    """``ops.window_add`` / ``window_copy`` on time windows and column blocks of strided
    tensors against torch's copy and add: bit for bit (the bf16 sum formed in fp32 and
    rounded once, as torch's add), on the 16-byte path (H = 24) and the scalar path (H = 5),
    in place (out aliasing a) and with the operands' strides all different."""
    from dabsn_amd.kernels import ops

    g = torch.Generator().manual_seed(H)
    B, T = 3, 37
    a = torch.randn(B, T, 2 * H, generator=g).to(cuda_device, dtype)
    x = torch.randn(B, T + 5, H, generator=g).to(cuda_device, dtype)
    out = torch.randn(B, T, H, generator=g).to(cuda_device, dtype)
    t0, t1 = 9, 30
    want = out.clone()
    want[:, t0:t1] = a[:, t0:t1, H:] + x[:, t0 + 2:t1 + 2]
    ops.window_add(out[:, t0:t1], a[:, t0:t1, H:], x[:, t0 + 2:t1 + 2])
    assert torch.equal(out, want)
    before = out.clone()
    ops.window_add(out[:, t0:t1], out[:, t0:t1], x[:, :t1 - t0])  # in place
    assert torch.equal(out[:, t0:t1], before[:, t0:t1] + x[:, :t1 - t0])
    assert torch.equal(out[:, :t0], before[:, :t0]) and torch.equal(out[:, t1:], before[:, t1:])
    c = ops.window_copy(a[:, t0:t1, :H])
    assert c.is_contiguous() and torch.equal(c, a[:, t0:t1, :H])


def test_pipeline_needs_the_scan_to_fit_one_half(cuda_device):
    """The scan runs on the CU-masked half: fp32 at width 2048 (256 channel tiles of 8
    units) does not fit there, so the block keeps the sequential path and a performance
    fallback event says why; bf16 at the same width (128 tiles of 16) pipelines."""
    from dabsn_amd import events

    seen = []
    listen = seen.append
    events.add_event_listener(listen)
    try:
        _, read = _modules(1, 8, 2048, 0.7, cuda_device)
        x = torch.zeros(2, 64, 2048, device=cuda_device)
        with torch.enable_grad():
            assert pipeline.pipeline_applies(read, x.bfloat16(), 32)
            events.reset_routing_log()
            assert not pipeline.pipeline_applies(read, x, 32)
        falls = [e for e in seen if e.fallback and e.component_id == "core_scan_chunked"]
        assert falls and "half" in falls[0].fields["reason"]
    finally:
        events.remove_event_listener(listen)


def test_width_read_work_runs_inside_the_read(cuda_device):
    """DABSNRead.during_width_read on the device: the work runs once, inside the read's host
    read of the bank width (before the read returns), and the read's output is the same."""
    core, read = _modules(5, 8, 64, 0.7, cuda_device)
    x = torch.randn(2, 48, 8, generator=torch.Generator().manual_seed(5)).to(cuda_device)
    with torch.no_grad():
        Wx, Wgx = core.projections(x)
        _, _, ref = _sequential(core, read, 16, Wx, Wgx)
        order = []
        side = torch.zeros(4, device=cuda_device)
        with read.during_width_read(lambda: (order.append("work"), side.add_(1.0))):
            _, _, out = _sequential(core, read, 16, Wx, Wgx)
            order.append("read returned")
    assert order == ["work", "read returned"]
    assert torch.equal(out, ref) and torch.equal(side.cpu(), torch.ones(4))
