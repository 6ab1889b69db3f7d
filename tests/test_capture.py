"""Graph capture of the registered operators.

The reference captures its scan chunks in CUDA graphs (kernels/batched_runtime.py:892-1021)
and gives the read a static, synchronisation-free bank width for capture (read.py:224-231).
Here the ops run without a host synchronisation in the default error mode (deferred error
words), the persistent scans launch as plain kernels under capture (a graph replays them on
an otherwise idle device), and the library clears its workspaces with its own kernel, never
with hipMemsetAsync. Each graph is checked to hold no memset node, replayed several times
with eager work, new input values and synchronisations between the replays, and every
replay compared bit for bit with the eager op on the same inputs.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from dabsn_amd.kernels import ops
from helpers import core_case

pytestmark = pytest.mark.gpu

MEMSET_NODE = 2  # hipGraphNodeTypeMemset


def _hip_runtime():
    """The HIP runtime library this process loaded (the one torch's graphs belong to)."""
    with open("/proc/self/maps") as fh:
        paths = sorted({line.split()[-1] for line in fh if "libamdhip64" in line})
    assert paths, "no HIP runtime mapped"
    return ctypes.CDLL(paths[0])


def _node_types(graph: torch.cuda.CUDAGraph) -> list[int]:
    hip = _hip_runtime()
    hip.hipGraphGetNodes.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_size_t)]
    hip.hipGraphNodeGetType.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int)]
    g = ctypes.c_void_p(graph.raw_cuda_graph())
    n = ctypes.c_size_t(0)
    assert hip.hipGraphGetNodes(g, None, ctypes.byref(n)) == 0
    nodes = (ctypes.c_void_p * n.value)()
    assert hip.hipGraphGetNodes(g, nodes, ctypes.byref(n)) == 0
    types = []
    for node in nodes:
        t = ctypes.c_int(-1)
        assert hip.hipGraphNodeGetType(ctypes.c_void_p(node), ctypes.byref(t)) == 0
        types.append(t.value)
    return types


def _capture(fn):
    """Warm ``fn`` up on a side stream, then capture it; returns (graph, static outputs)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph(keep_graph=True)
    with torch.cuda.graph(graph):
        outs = fn()
    types = _node_types(graph)
    assert types and MEMSET_NODE not in types, f"graph node types {types}"
    return graph, outs


def _replays(graph, outs, static_inputs, cases, eager):
    """For each case (a list of new input values): copy it into the static inputs, replay,
    run unrelated eager work and synchronise, and compare the graph's outputs with the
    eager op on the same values, bit for bit."""
    for values in cases:
        with torch.no_grad():
            for dst, src in zip(static_inputs, values):
                dst.copy_(src)
        graph.replay()
        noise = torch.randn(1 << 20, device=outs[0].device).square().sum()
        torch.cuda.synchronize()
        want = eager(values)
        assert torch.isfinite(noise)
        for i, (a, b) in enumerate(zip(outs, want)):
            if a is None and b is None:
                continue
            assert torch.equal(a, b), f"output {i} differs from the eager op"
    ops.check_errors()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_core_scan_forward_and_backward_capture(cuda_device, dtype):
    B, T, H = 16, 48, 256
    cases = []
    for seed in (1, 2, 3):
        x = [t.to(cuda_device) for t in core_case(seed, B, T, H)]
        x[0], x[1] = x[0].to(dtype), x[1].to(dtype)
        cases.append(x)
    static = [t.clone() for t in cases[0]]
    g = torch.Generator().manual_seed(7)
    ups = [(torch.randn(B, T, 2 * H, generator=g)).to(cuda_device, dtype)]
    ups += [(torch.randn(B, T, H, generator=g)).to(cuda_device, dtype) for _ in range(6)]
    ups += [torch.randn(B, H, generator=g).to(cuda_device) for _ in range(3)]

    def run(x):
        out = ops.core_scan_batched(*x)
        grads = ops.core_scan_batched_backward(
            x[2], x[3], x[4:20], x[20], x[21], x[22], x[23], x[25], out[0], out[2], out[3],
            out[5], out[6], out[7], *ups)
        return [*out, *grads]

    graph, outs = _capture(lambda: run(static))
    _replays(graph, outs, static, cases[1:] + cases[:1], run)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_read_at_static_bank_width_capture(cuda_device, dtype):
    B, T, N, H = 2, 96, 96, 64

    def case(seed):
        g = torch.Generator().manual_seed(seed)
        q = torch.nn.functional.normalize(torch.randn(B, T, H, generator=g), dim=-1)
        V = torch.randn(B, N, H, generator=g)
        K = torch.nn.functional.normalize(V, dim=-1)
        Vn = torch.roll(V, -1, dims=1)
        ck = torch.nn.functional.normalize(torch.rand(B, T, 4, generator=g), dim=-1)
        cb = torch.nn.functional.normalize(torch.rand(B, N, 4, generator=g), dim=-1)
        kb = torch.randn(B, N, generator=g) * 0.3
        adm = torch.randn(B, N, generator=g) * 0.3
        vals = [v.to(cuda_device, dtype) for v in (q, K, V, Vn)]
        vals += [v.to(cuda_device) for v in (ck, cb, kb, adm)]
        vals += [torch.tensor([3.0 + seed], device=cuda_device)]
        vals += [torch.tensor([s], device=cuda_device) for s in (1.0, 0.9, 0.1, 1.1)]
        return vals

    idx = torch.arange(N, device=cuda_device).expand(B, N).contiguous()
    valid = torch.ones(B, N, dtype=torch.bool, device=cuda_device)
    cases = [case(s) for s in (4, 5, 6)]
    static = [t.clone() for t in cases[0]]

    def run(v):
        out = ops.admitted_three_way_read_compact_flash(*v[:9], idx, valid, 0, *v[9:])
        return [out]

    graph, outs = _capture(lambda: run(static))
    _replays(graph, outs, static, cases[1:] + cases[:1], run)
