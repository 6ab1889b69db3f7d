"""``torch.vmap`` over the ``dabsn::`` operators (the reference registers a per-index loop
rule on each public op: batched_runtime.py:1639, compact_flash.py:300, long.py:440,
admitted.py:635, permanent.py:435, local_field.py:246).

The rules here fold the vmapped dim into the operators' row dim when only row-batched
arguments carry it, and loop otherwise. Both must give what calling the operator once per
index and stacking gives: on the CPU (oracle kernels) to fp32 rounding of the same kernel
(equal, since the oracle is row-independent), on the GPU bit for bit (every HIP operator
computes each row independently of which other rows share its launch).
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from dabsn_amd.kernels import ops
from helpers import core_case
from oracle import torch_backend
from test_dense_read import dense_case


@pytest.fixture(scope="module", autouse=True)
def _oracle_cpu_kernels():
    torch_backend.register()


def _stacked(op, per_index):
    outs = [op(*args) for args in per_index]
    if isinstance(outs[0], (tuple, list)):
        return [torch.stack([o[k] for o in outs]) for k in range(len(outs[0]))]
    return torch.stack(outs)


def _same(a, b, exact):
    if isinstance(a, (tuple, list)):
        for x, y in zip(a, b):
            _same(x, y, exact)
        return
    assert a.shape == b.shape
    if exact:
        assert torch.equal(a, b)
    else:
        torch.testing.assert_close(a, b, rtol=1e-6, atol=1e-6)


def _core_cases(V, device, batched_param=False):
    cases = [core_case(40 + v, 2, 6, 8) for v in range(V)]
    if not batched_param:
        for c in cases[1:]:
            c[2:23] = cases[0][2:23]  # shared weights and gains
    return [[t.to(device) for t in c] for c in cases]


def _vmap_vs_loop(op, cases, in_dims, exact):
    stacked_args = [torch.stack([c[i] for c in cases]) if d == 0 else cases[0][i]
                    for i, d in enumerate(in_dims)]
    got = torch.vmap(op, in_dims=tuple(in_dims))(*stacked_args)
    _same(got, _stacked(op, cases), exact)


@pytest.mark.parametrize("batched_param", [False, True])
def test_vmap_core_scan_cpu(batched_param):
    cases = _core_cases(3, "cpu", batched_param)
    dims = [0 if i in (0, 1, 23, 24, 25) or batched_param else None for i in range(26)]
    _vmap_vs_loop(ops.core_scan_batched, cases, dims, exact=False)


def test_vmap_linrec_permanent_field_cpu():
    g = torch.Generator().manual_seed(3)
    lin = [[torch.rand(2, 9, 5, generator=g), torch.randn(2, 9, 5, generator=g),
            torch.randn(2, 5, generator=g)] for _ in range(3)]
    _vmap_vs_loop(ops.linear_recurrence, lin, [0, 0, 0], exact=False)
    perm = [[F.normalize(torch.randn(2, 7, 6, generator=g), dim=-1),
             torch.randn(2, 7, 6, generator=g), torch.rand(2, 7, generator=g)] for _ in range(2)]
    _vmap_vs_loop(ops.permanent_delta_scan, perm, [0, 0, 0], exact=False)
    patch = torch.randint(0, 10, (10, 3), generator=g)
    field = [[torch.randn(2, 10, 4, generator=g), patch] for _ in range(3)]
    _vmap_vs_loop(ops.local_field_gather, field, [0, None], exact=False)


def test_vmap_dense_read_cpu():
    cases = [dense_case(60 + v, 2, 5, 4, 6) for v in range(3)]
    for c in cases[1:]:
        for i in (8, 13, 14, 15, 16):
            c[i] = cases[0][i]
    dims = [0 if i not in (8, 13, 14, 15, 16) else None for i in range(17)]
    _vmap_vs_loop(ops.admitted_three_way_read_native, cases, dims, exact=False)


def test_vmap_long_scan_cpu():
    g = torch.Generator().manual_seed(8)
    logits = [torch.tensor([v]) for v in (2.2, 2.0, 2.4, 1.4)]
    cases = [[torch.randn(2, 9, 5, generator=g), torch.rand(2, 9, 5, generator=g), *logits,
              torch.randn(2, 5, generator=g), torch.randn(2, 5, generator=g), torch.ones(2, 5)]
             for _ in range(2)]
    _vmap_vs_loop(ops.long_scan_fused, cases, [0, 0, None, None, None, None, 0, 0, 0],
                  exact=False)


@pytest.mark.gpu
def test_vmap_fold_is_bit_exact_on_gpu(cuda_device):
    cases = _core_cases(3, cuda_device)
    dims = [0 if i in (0, 1, 23, 24, 25) else None for i in range(26)]
    _vmap_vs_loop(ops.core_scan_batched, cases, dims, exact=True)
    dense = [[t.to(cuda_device) for t in dense_case(70 + v, 2, 33, 40, 24)] for v in range(2)]
    for c in dense[1:]:
        for i in (8, 13, 14, 15, 16):
            c[i] = dense[0][i]
    ddims = [0 if i not in (8, 13, 14, 15, 16) else None for i in range(17)]
    _vmap_vs_loop(ops.admitted_three_way_read_native, dense, ddims, exact=True)
