"""Benchmark: DABSN scan+read forward+backward on one MI355X.

Workload ("config 4"): one seq DABSN layer, state width 2048,
read/hidden width 4096, vocabulary 32,000, batch 16, T = 4096, bf16, block chunking
enabled (chunk 1024; the chunks' tapes are kept for the reverse scans instead of
recomputed). One step = forward + backward of the scan+read region: the chunked core scan
(op dabsn::core_scan_batched), read statistics, admitted-slot selection, bank gather,
three-way read, read output projection and the long-memory scan, pipelined over the
chunks on the two halves of the device (--no-pipeline: one after the other), from input projections
Wx = W x, Wgx = Wg x that are already resident in HBM (the input projections are plain
GEMMs timed separately, as the metric excludes them). Synthetic data: random token ids
through a random embedding, random-initialised weights.

Prints one JSON line (see the repository's benchmark contract).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "scan+read tokens/sec (B×T) fwd+bwd, state 2048 T=4096 bf16; % HBM roofline"
HBM_PEAK_GBS = 8000.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--batch", type=int, default=None, help="default 16 (train), 256 (decode)")
    p.add_argument("--seq", type=int, default=4096)
    p.add_argument("--state", type=int, default=2048)
    p.add_argument("--hidden", type=int, default=4096)
    p.add_argument("--vocab", type=int, default=32000)
    p.add_argument("--chunk", type=int, default=1024)
    p.add_argument("--cpu-seq", type=int, default=256, help="T of the bounded CPU sample")
    p.add_argument("--no-pipeline", action="store_true",
                   help="train: scan and read one after the other on the whole device")
    p.add_argument("--no-proj", action="store_true",
                   help="skip the separate timing of the input projections (profiling runs)")
    p.add_argument("--cpu-trials", type=int, default=3,
                   help="timed CPU steps after one untimed warm-up step")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--workload", choices=("train", "decode", "primitives"), default="train",
                   help="train: the config-4 headline step (default); decode: config-5 streaming "
                        "decode through the carried memory; primitives: the permanent delta "
                        "scan and local field gather kernels")
    p.add_argument("--prompt", type=int, default=2048, help="decode: prompt tokens ingested")
    p.add_argument("--layers", type=int, default=4, help="decode: seq layers")
    args = p.parse_args()
    if args.batch is None:
        args.batch = 256 if args.workload == "decode" else 16
    return args


class ScanRead(torch.nn.Module):
    """The scan+read region of one seq block (core + read), driven from Wx/Wgx."""

    def __init__(self, hidden: int, state: int, chunk: int):
        super().__init__()
        from dabsn_amd import DABSNCore, DABSNRead

        self.core = DABSNCore(hidden, state)
        self.read = DABSNRead(state)
        self.state = state
        self.chunk = chunk
        self.pipelined = True

    def scan(self, Wx, Wgx):
        from torch.utils.checkpoint import checkpoint

        from dabsn_amd.kernels.chunked import chunked_core_scan
        from dabsn_amd.kernels.ops import core_scan_batched

        B, T, H = Wx.shape
        zeros = torch.zeros(B, H, device=Wx.device, dtype=torch.float32)
        carry = (zeros, torch.ones_like(zeros), zeros.clone())
        params = self.core.scan_inputs()
        if Wx.is_cuda and 0 < self.chunk < T and torch.is_grad_enabled():
            # Checkpointed chunks; the backward overlaps each recompute with a reverse scan.
            return list(chunked_core_scan(self.chunk, Wx, Wgx, *params, *carry)[:7])
        tapes = [[] for _ in range(7)]

        def run(wx, wgx, b, e, c):
            out = core_scan_batched(wx, wgx, *params, b, e, c)
            return (*out[:7], *out[8:11])

        chunk = self.chunk if 0 < self.chunk < T else T
        for t0 in range(0, T, chunk):
            sl = slice(t0, min(T, t0 + chunk))
            if chunk < T and torch.is_grad_enabled():
                outs = checkpoint(run, Wx[:, sl], Wgx[:, sl], *carry, use_reentrant=False)
            else:
                outs = run(Wx[:, sl], Wgx[:, sl], *carry)
            for i in range(7):
                tapes[i].append(outs[i])
            carry = outs[7:10]
        return [torch.cat(p, 1) if len(p) > 1 else p[0] for p in tapes]

    def forward(self, Wx, Wgx):
        from dabsn_amd.kernels import pipeline

        if self.pipelined and pipeline.pipeline_applies(self.read, Wx, self.chunk):
            # The read of query chunk k beside the scan of chunk k + 1 (and in reverse in the
            # backward), on the two halves of the device.
            y, _, read = pipeline.pipelined_scan_read(self.read, self.chunk, Wx, Wgx,
                                                      self.core.scan_inputs())
            return y, read
        U, nov, p, ay, w, e, c = self.scan(Wx, Wgx)
        y, budget = U.split(self.state, dim=-1)
        return y, self.read(y, budget, ay, w, nov, p, e, c)


def build_workload(args, device, dtype, batch, seq):
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, args.vocab, (batch, seq), generator=g)
    torch.manual_seed(0)
    model = ScanRead(args.hidden, args.state, args.chunk).to(device)
    embed = (torch.randn(args.vocab, args.hidden, generator=g) * 0.02).to(dtype)
    x = embed[ids].to(device)
    with torch.no_grad():
        Wx = torch.nn.functional.linear(x, model.core.W.weight.to(dtype))
        Wgx = torch.nn.functional.linear(x, model.core.Wg.weight.to(dtype), model.core.Wg.bias.to(dtype))
    Wx = Wx.detach().requires_grad_(True)
    Wgx = Wgx.detach().requires_grad_(True)
    gy = (torch.randn(batch, seq, args.state, generator=g) * 1e-3).to(device=device, dtype=dtype)
    # The read output is fp32 under the reference's type promotion (bf16 projection plus the
    # fp32 gain times the long channel, read.py:435-438), so its upstream gradient is too.
    gr = (torch.randn(batch, seq, args.state, generator=g) * 1e-3).to(device=device,
                                                                      dtype=torch.float32)
    return model, Wx, Wgx, gy, gr


def step(model, Wx, Wgx, gy, gr, device_type, dtype):
    model.zero_grad(set_to_none=True)
    Wx.grad = None
    Wgx.grad = None
    with torch.autocast(device_type, dtype=dtype, enabled=dtype != torch.float32):
        y, read = model(Wx, Wgx)
    torch.autograd.backward([y, read], [gy, gr if gr.dtype == read.dtype else gr.to(read.dtype)])


PMC_FILE = os.path.join(ROOT, "profiles", "core_scan_config4_pmc.json")


def measured_traffic(kernel: str, args, chunk: int):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
    summary (copy-kernel calibrated), when it was measured on this workload and kernel."""
    try:
        with open(PMC_FILE) as fh:
            doc = json.load(fh)
    except OSError:
        return None, None
    w = doc.get("workload", {})
    if (w.get("batch"), w.get("seq_len"), w.get("state"), w.get("chunk_t")) != (
            args.batch, args.seq, args.state, chunk):
        return None, None
    entry = doc.get("kernels", {}).get(kernel)
    if not entry:
        return None, None
    from dabsn_amd.kernels import ops

    symbol = ops.kernel_symbol(kernel, args.batch, args.state)
    if symbol is not None and symbol != entry.get("kernel_symbol"):
        return None, None  # the counters were taken on a different kernel configuration
    return int(entry["traffic_bytes"]), "profiles/core_scan_config4_pmc.md"


def time_projections(args, model, device, dtype, reps: int = 5):
    """The block's input projections Wx = W x and Wgx = Wg x + b (core.py:281-282), which
    the scan+read step takes as resident inputs, timed on their own: forward (two GEMMs)
    and backward (input gradient as two accumulating GEMMs, two weight-gradient GEMMs) on
    hipBLASLt through torch, bf16, [B*T, hidden] x [hidden, state]; and the block combine's
    state_to_hidden (model.py:336-337, [B*T, state] x [state, hidden]): forward one GEMM,
    backward two (input and weight gradients)."""
    F = torch.nn.functional
    rows, D, H = args.batch * args.seq, args.hidden, args.state
    g = torch.Generator(device=device).manual_seed(3)
    x = torch.randn(rows, D, device=device, dtype=dtype, generator=g)
    gy = torch.randn(rows, H, device=device, dtype=dtype, generator=g)
    gz = torch.randn(rows, H, device=device, dtype=dtype, generator=g)
    W = model.core.W.weight.detach().to(dtype)
    Wg = model.core.Wg.weight.detach().to(dtype)
    bg = model.core.Wg.bias.detach().to(dtype)

    def fwd():
        return F.linear(x, W), F.linear(x, Wg, bg)

    def bwd():
        gx = torch.addmm(gy @ W, gz, Wg)
        return gx, gy.t() @ x, gz.t() @ x

    Wsh = (torch.randn(D, H, device=device, generator=g) / H ** 0.5).to(dtype)
    ysh = torch.randn(rows, H, device=device, dtype=dtype, generator=g)
    gsh = torch.randn(rows, D, device=device, dtype=dtype, generator=g)

    def sh_fwd():
        return F.linear(ysh, Wsh)

    def sh_bwd():
        return gsh @ Wsh, gsh.t() @ ysh

    out = {}
    for name, fn, gemms in (("forward", fwd, 2), ("backward", bwd, 4),
                            ("state_to_hidden_forward", sh_fwd, 1),
                            ("state_to_hidden_backward", sh_bwd, 2)):
        fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / reps
        tflops = gemms * 2.0 * rows * D * H / (ms / 1e3) / 1e12
        out[name] = {"ms": round(ms, 3), "tflops": round(tflops, 1),
                     "frac_bf16_peak": round(tflops / 2500.0, 4)}
    out["note"] = ("not part of value: the scan+read step starts from resident Wx, Wgx and "
                   "ends at the read output; input projections [rows, hidden] x [hidden, state] "
                   "and state_to_hidden [rows, state] x [state, hidden], "
                   f"rows {rows}, hidden {D}, state {H}, bf16, hipBLASLt via torch")
    return out


def cpu_baseline(args):
    """The oracle (C restatement of the reference CPU backend, fp32, OpenMP over batch)
    running the same scan+read step on a bounded sample: config-4 widths, T=cpu_seq."""
    import oracle
    from oracle import torch_backend

    oracle.build()
    torch_backend.register()
    omp_env = os.environ.get("OMP_NUM_THREADS")
    threads = int(omp_env or min(16, os.cpu_count() or 1))
    oracle.set_num_threads(threads)
    torch.set_num_threads(threads)
    seq = int(args.cpu_seq)

    def sample(T, trials):
        model, Wx, Wgx, gy, gr = build_workload(args, torch.device("cpu"), torch.float32,
                                                args.batch, T)
        step(model, Wx, Wgx, gy, gr, "cpu", torch.float32)  # warm-up (page-in, thread pools)
        out = []
        for _ in range(max(1, trials)):
            t0 = time.perf_counter()
            step(model, Wx, Wgx, gy, gr, "cpu", torch.float32)
            out.append(time.perf_counter() - t0)
        return model, out

    model, times = sample(seq, int(args.cpu_trials))
    # A second, half-length sample fixes the two terms of the step time t(T) = a T + b T^2:
    # the scan, the glue and the long channel are linear in T, the dense-bank read (every
    # query against every earlier slot) quadratic. The fit extrapolates to the workload's T.
    seq_half = max(1, seq // 2)
    _, times_half = sample(seq_half, max(2, int(args.cpu_trials) // 2))
    t1, t2 = sum(times_half) / len(times_half), sum(times) / len(times)
    b_coef = (t2 / seq - t1 / seq_half) / (seq - seq_half)
    a_coef = t1 / seq_half - b_coef * seq_half
    if b_coef < 0 or a_coef < 0:  # timing noise on a tiny sample: keep the fit's sign sane
        a_coef, b_coef = (t2 / seq, 0.0) if b_coef < 0 else (0.0, t2 / seq ** 2)
    t_full = a_coef * args.seq + b_coef * args.seq ** 2
    tokens = args.batch * seq
    rates = [tokens / t for t in times]
    n = len(rates)
    mean = sum(rates) / n
    sd = (sum((r - mean) ** 2 for r in rates) / (n - 1)) ** 0.5 if n > 1 else 0.0
    # Student t, 95 %, n - 1 degrees of freedom (n <= 10 here)
    t95 = {1: 12.71, 2: 4.303, 3: 3.182, 4: 2.776, 5: 2.571, 6: 2.447, 7: 2.365, 8: 2.306,
           9: 2.262}.get(n - 1, 2.0)
    half = t95 * sd / n ** 0.5 if n > 1 else None
    return {
        "value": mean,
        "unit": "tokens/s",
        "cores": threads,
        "threads": {"os_cpu_count": os.cpu_count(), "OMP_NUM_THREADS": omp_env,
                    "torch_get_num_threads": torch.get_num_threads(),
                    "oracle_threads": oracle.num_threads()},
        "extrapolated": {"seq_len": args.seq, "tokens_per_s": args.batch * args.seq / t_full,
                         "seconds_per_step": t_full, "linear_s_per_token_step": a_coef,
                         "quadratic_s": b_coef, "fit": f"t(T) = a T + b T^2 through the mean "
                         f"step times at T={seq_half} ({t1:.2f} s) and T={seq} ({t2:.2f} s)"},
        "kind": "port",
        "ci95": [mean - half, mean + half] if half is not None else None,
        "trials": n,
        "sample": (f"oracle C/OpenMP fp32 (restates reference cpu_runtime.cpp + registered reverse scan), "
                   f"fwd+bwd steps at B={args.batch}, T={seq}, H={args.state}, D={args.hidden}, "
                   f"n_max={model.read.last_n_max}: 1 warm-up + {n} timed, mean "
                   f"{sum(times) / n:.2f} s each; T-truncated proxy of the T={args.seq} workload "
                   f"(scan cost scales with T, read with T*n_max)"),
        "seconds": sum(times) + sum(times_half),
    }


DECODE_METRIC = "decode tokens/sec (B x steps), config 5: 4 seq layers 2048/2048, prompt 2048"


def decode_main(args):
    """Config 5: DABSNSequenceLM(vocab 32000, hidden 2048, 4 x
    seq 2048/2048, residual, MLP ratio 4.0) in bf16, B=256 (pass --batch 256). A prompt of
    --prompt random tokens is ingested in chunks of 512 (``dabsn_amd.ingest``), the banks are
    reserved for the whole run, then each timed step decodes one token per row with
    ``forward_with_memory(extend=True)``: the core steps from the carried state, the read
    scans each layer's bank in place (``dabsn_hip_read3_decode``) and the bank grows by one
    row. value = B x steps / time. The timed steps run without per-kernel timers (their
    event records cost host time in a host-bound step); --steps further steps then run with
    them to measure the kernels."""
    import dabsn_amd
    from dabsn_amd import memory as mem
    from dabsn_amd.kernels import ops

    dabsn_amd.kernels.enable("rocm", required=True)
    os.environ.setdefault("DABSN_HIP_ERROR_CHECK", "deferred")
    device = torch.device("cuda:0")
    H, B, L = args.state, args.batch, args.layers
    torch.manual_seed(0)
    model = dabsn_amd.DABSNSequenceLM(args.vocab, H, L, layers=[(H, H)] * L, residual=True, mlp_ratio=4.0)
    model = model.to(device).to(torch.bfloat16).eval()
    meas = min(args.steps, 8)  # steps with per-kernel timers, after the timed ones
    total = args.prompt + args.warmup + args.steps + meas
    ids = torch.randint(0, args.vocab, (B, total), generator=torch.Generator().manual_seed(1))
    ids = ids.to(device)
    memory = mem.ingest(model, ids[:, :args.prompt], chunk_size=512)
    memory.reserve(total)
    pos = args.prompt
    for _ in range(args.warmup):
        _, memory = mem.forward_with_memory(model, ids[:, pos:pos + 1], memory, extend=True)
        pos += 1
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        _, memory = mem.forward_with_memory(model, ids[:, pos:pos + 1], memory, extend=True)
        pos += 1
    stop.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / args.steps
    ops.timing(True)
    for _ in range(meas):
        _, memory = mem.forward_with_memory(model, ids[:, pos:pos + 1], memory, extend=True)
        pos += 1
    torch.cuda.synchronize()
    kernels = ops.KernelTimer.summary()
    ops.timing(False)
    ops.check_errors()
    # bank rows per layer, mean over the measured steps
    n_mean = args.prompt + args.warmup + args.steps + (meas + 1) / 2
    bank_bytes = B * n_mean * H * 2  # one pass over one layer's bank
    dec = kernels.get("read3_decode")
    roofline = None
    if dec:
        # One query row per batch row: the single-pass read streams every admitted slot's
        # write row once (its induction value is the next slot's row, already in registers):
        # algorithmic bytes = one bank pass per launch when every slot is admitted.
        achieved = bank_bytes / (dec["avg_ms"] / 1e3) / 1e9
        roofline = {"bound": "hbm", "kernel": "read3_decode", "achieved": round(achieved, 2),
                    "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 5),
                    "traffic": None, "alg_bytes_per_launch": int(bank_bytes),
                    "avg_launch_ms": round(dec["avg_ms"], 4)}
    result = {
        "metric": DECODE_METRIC, "value": round(B * 1e3 / ms, 1), "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: uniform random token ids, random-init weights",
        "config": {"workload": "config5 streaming decode: 4 seq layers 2048/2048, MLP 4.0, "
                               "vocab 32000, prompt ingested in chunks of 512",
                   "batch": B, "prompt": args.prompt, "layers": L, "state": H,
                   "bank_rows_mean": n_mean},
        "roofline": roofline,
        "kernel_ms": {k: {"avg": round(v["avg_ms"], 4), "calls_per_step": v["calls"] / meas,
                          "per_step": round(v["total_ms"] / meas, 3)}
                      for k, v in sorted(kernels.items(), key=lambda kv: -kv[1]["total_ms"])},
    }
    print(json.dumps(result), flush=True)


PRIMITIVES_METRIC = ("standalone primitives: permanent delta scan, local field gather, chunked "
                     "readout cross-entropy rows")
FP32_VALU_PEAK_TFLOPS = 78.6  # non-packed fp32 FMA rate (packed fp32 is not used)


def primitives_main(args):
    """The two primitives outside the model path (reference PRIMITIVES, kernels/__init__.py:
    56-83), at sizes of their own: permanent_delta_scan fwd + bwd at B=16, T=1024, H=256
    (unit keys), fp32; local_field_gather fwd + bwd on a 256 x 256 torus with 3 x 3
    neighbourhoods (K = 9), B=8, D=64, fp32; and the row kernels of the chunked readout
    cross-entropy (``dabsn_amd.loss``, forward + backward, N=8192 rows, V=32000, hidden 2048,
    bf16, 2**24-element chunks). Prints per-kernel averages over --steps and each kernel's
    roofline: the delta scan against the fp32 VALU rate (algorithmic flops: 4 H^2 per
    (b, t) forward, 14 H^2 backward with its recompute), the gather and its scatter-add
    against HBM (algorithmic bytes: every gathered element written once and every source
    element read once; the backward the reverse), the cross-entropy rows against HBM
    (forward: the bf16 logits read once; backward: read once, fp32 gradient written)."""
    import dabsn_amd
    from dabsn_amd import loss as dloss
    from dabsn_amd.kernels import ops

    dabsn_amd.kernels.enable("rocm", required=True)
    os.environ.setdefault("DABSN_HIP_ERROR_CHECK", "deferred")
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(3)
    B, T, H = 16, 1024, 256
    k = torch.randn(B, T, H, generator=g)
    k = (k / k.norm(dim=-1, keepdim=True)).to(dev)
    v = torch.randn(B, T, H, generator=g).to(dev)
    beta = torch.sigmoid(torch.randn(B, T, generator=g)).to(dev)
    up = torch.randn(B, T, H, generator=g).to(dev)
    side = 256
    n = torch.arange(side * side)
    r, c = n // side, n % side
    patch = torch.stack([((r + dr) % side) * side + (c + dc) % side
                         for dr in (-1, 0, 1) for dc in (-1, 0, 1)], dim=1).to(dev)
    FB, D = 8, 64
    x = torch.randn(FB, side * side, D, generator=g).to(dev)
    gout = torch.randn(FB, side * side, 9, D, generator=g).to(dev)

    NR, V, HR = 8192, 32000, 2048
    hid = torch.randn(NR, HR, generator=g).to(dev, torch.bfloat16).requires_grad_(True)
    wro = (torch.randn(V, HR, generator=g) / HR ** 0.5).to(dev, torch.bfloat16).requires_grad_(True)
    tgt = torch.randint(0, V, (NR,), generator=g).to(dev)

    def run():
        ops.permanent_delta_scan(k, v, beta)
        ops.permanent_delta_scan_backward(k, v, beta, up)
        ops.local_field_gather(x, patch)
        ops.local_field_gather_backward(gout, patch, side * side)
        dloss.chunked_linear_cross_entropy(hid, wro, None, tgt).backward()

    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    ops.timing(True)
    for _ in range(args.steps):
        run()
    torch.cuda.synchronize()
    kernels = ops.KernelTimer.summary()
    ops.timing(False)
    ops.check_errors()
    cells = side * side
    work = {
        "permanent_scan_fwd": ("valu", 4.0 * B * T * H * H),
        "permanent_scan_bwd": ("valu", 14.0 * B * T * H * H),
        "local_field_gather": ("hbm", 4.0 * FB * cells * D * (9 + 1)),
        "local_field_scatter": ("hbm", 4.0 * FB * cells * D * (9 + 1)),
        # per launch: one 2**24-element chunk (524 rows of 32000)
        "ce_rows_fwd": ("hbm", 2.0 * (1 << 24) // V * V),
        "ce_rows_bwd": ("hbm", 6.0 * (1 << 24) // V * V),
    }
    out = {}
    for name, (bound, amount) in work.items():
        avg = kernels[name]["avg_ms"] / 1e3
        if bound == "hbm":
            ach = amount / avg / 1e9
            out[name] = {"avg_ms": round(avg * 1e3, 4), "bound": "hbm", "achieved": round(ach, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(ach / HBM_PEAK_GBS, 4), "alg_bytes": int(amount)}
        else:
            ach = amount / avg / 1e12
            out[name] = {"avg_ms": round(avg * 1e3, 4), "bound": "fp32 valu",
                         "achieved": round(ach, 3), "peak": FP32_VALU_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(ach / FP32_VALU_PEAK_TFLOPS, 4),
                         "alg_flops": int(amount)}
    result = {"metric": PRIMITIVES_METRIC, "unit": "ms", "n_gpus": 1, "steps": args.steps,
              "warmup": args.warmup, "dtype": "f32", "data": "synthetic",
              "config": {"workload": "permanent B=16 T=1024 H=256; local field 256x256 torus, "
                                     "K=9, B=8, D=64; readout CE N=8192 V=32000 H=2048 bf16"},
              "kernels": out}
    print(json.dumps(result), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested).", file=sys.stderr)
        sys.exit(2)
    import dabsn_amd
    from dabsn_amd.kernels import ops

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    if args.workload == "decode":
        decode_main(args)
        return
    if args.workload == "primitives":
        primitives_main(args)
        return
    dabsn_amd.kernels.enable("rocm", required=True)
    os.environ.setdefault("DABSN_HIP_ERROR_CHECK", "deferred")
    device = torch.device("cuda:0")
    dtype = torch.bfloat16
    model, Wx, Wgx, gy, gr = build_workload(args, device, dtype, args.batch, args.seq)
    model.pipelined = not args.no_pipeline
    for _ in range(args.warmup):
        step(model, Wx, Wgx, gy, gr, "cuda", dtype)
    torch.cuda.synchronize()
    ops.timing(True)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(args.steps):
        step(model, Wx, Wgx, gy, gr, "cuda", dtype)
    stop.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / args.steps
    kernels = ops.KernelTimer.summary()
    ops.timing(False)
    ops.check_errors()
    tokens = args.batch * args.seq
    value = tokens / (ms / 1e3)

    # Dominant kernel and its roofline (algorithmic bytes per launch / measured duration).
    dom = max(kernels, key=lambda k: kernels[k]["total_ms"])
    H = args.state
    el = 2  # bf16
    n_max = int(model.read.last_n_max or 0)
    chunk = args.chunk if 0 < args.chunk < args.seq else args.seq
    per_token = {
        # reads U (2H), plasticity, expression, energy, saturation, gate (5H), grads of
        # U (2H) and of 6 [B,T,H] outputs (6H); writes gWx, gWgx, d_expression (3H)
        "core_scan_bwd": 18 * H * el,
        # reads Wx, Wgx (2H); writes U (2H) + 7 tapes (7H)
        "core_scan_fwd": 11 * H * el,
    }
    weights_bytes = 2 * H * H * el
    if dom in per_token:
        # The launches of one step cover the sequence once (the pipeline's windows, or the
        # block's chunks): the average launch scans tokens / launches-per-step tokens.
        launches = kernels[dom]["calls"] / args.steps
        launch_tokens = int(round(tokens / launches))
        alg_bytes = per_token[dom] * launch_tokens + weights_bytes
        achieved = alg_bytes / (kernels[dom]["avg_ms"] / 1e3) / 1e9
        traffic, traffic_src = measured_traffic(dom, args, chunk)
        roofline = {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 2),
                    "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 5),
                    "traffic": traffic, "traffic_source": traffic_src,
                    "alg_bytes_per_launch": alg_bytes,
                    "avg_launch_ms": round(kernels[dom]["avg_ms"], 4),
                    "launch_tokens": launch_tokens}
    else:
        roofline = {"bound": "mfma", "kernel": dom, "achieved": None, "peak": 2500.0,
                    "unit": "TFLOP/s", "frac": None, "traffic": None}
    # Whole-step fraction of the HBM roofline on the algorithmic bytes of the step.
    step_bytes = (55 + 18 * (n_max / args.seq)) * H * el * tokens + 3 * weights_bytes

    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: uniform random token ids, random embedding, random-init weights",
        "config": {"workload": "config4 scan+read fwd+bwd: one seq layer, state 2048, read/hidden 4096, "
                               "vocab 32000, block chunking 1024 (tapes kept in HBM for the reverse scans)",
                   "batch": args.batch, "seq_len": args.seq, "state": H, "hidden": args.hidden,
                   "chunk_t": chunk, "n_max": n_max},
        "roofline": roofline,
        "step_hbm_roofline_frac": round(step_bytes / (ms / 1e3) / 1e9 / HBM_PEAK_GBS, 5),
        "kernel_ms": {k: {"avg": round(v["avg_ms"], 4), "calls_per_step": v["calls"] / args.steps,
                          "per_step": round(v["total_ms"] / args.steps, 3)}
                      for k, v in sorted(kernels.items(), key=lambda kv: -kv[1]["total_ms"])},
    }
    if not args.no_proj:
        result["projections"] = time_projections(args, model, device, dtype)
    if not args.no_cpu:
        try:
            result["cpu_baseline"] = cpu_baseline(args)
        except Exception as exc:  # noqa: BLE001 - reported, the GPU figure stands
            result["cpu_baseline"] = {"error": f"{type(exc).__name__}: {exc}"}
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
