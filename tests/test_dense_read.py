"""The dense-mask three-way read op pair, ``dabsn::admitted_three_way_read_native`` and
``dabsn::_admitted_three_way_read_backward`` (reference admitted.py:383-622).

Checkers, none of them the HIP path:

  * the reference's own C++ dense read (``three_way_read_cpu`` / ``three_way_read_bwd``
    in src/dabsn/kernels/cpu_runtime.cpp, compiled into ``oracle/_ref``) on masks where
    every eligible row has an allowed slot;
  * the fp64 autograd restatement of admitted.py:16-65 (``oracle.autograd_ref.dense_read``
    with explicit row eligibilities), itself pinned to that C++ here (CPU tests).

Tolerances: fp32 outputs and tensor gradients normwise 1e-5 against the C++ (fp32 on
both sides, different summation orders); scalar gradients (sums over every (query, slot)
term) 5e-5 relative to a floor of 1e-3 x the largest scalar gradient (worst seen on the
GPU 2.4e-5, the cocktail gain at B=1, T=96, N=1000); against fp64, the same. Semantics
the C++ does not share: an eligible row with no allowed slot gives NaN weights in the
reference's registered Python op (softmax over all -inf), which is what runs on a device
in the reference; the C++ CPU kernel returns zeros for such a row. The HIP op follows the
registered op and is checked against the fp64 restatement there.
bf16 inputs compute in fp32 (the reference's compute dtype), so they must equal the fp32
op on the same values, rounded to bf16, bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from dabsn_amd.kernels import ops
from helpers import np32, rel_err
from oracle import autograd_ref
from oracle import ref as oracle_ref
from oracle import torch_backend

NAMES = ("query", "bank_keys", "bank_writes", "next_writes", "cocktail", "bank_cocktail",
         "bank_key_bias", "bank_admission", "scale", "short_gain", "pad_gain", "induct_gain",
         "cocktail_gain")
SCALARS = (8, 9, 10, 11, 12)
# The C++ backward's order: ..., scale, cocktail_gain, short, pad, induct.
CPP_ORDER = (0, 1, 2, 3, 4, 5, 6, 7, 8, 10, 11, 12, 9)


@pytest.fixture(scope="module", autouse=True)
def _oracle_cpu_kernels():
    torch_backend.register()


@pytest.fixture(scope="module")
def R():
    mod = oracle_ref.load()
    if mod is None:
        pytest.skip("oracle/_ref not built: it compiles the reference's cpu_runtime.cpp, "
                    "which only the build container has (make -f oracle/ref.mk)")
    return mod


def dense_case(seed, B, T, N, H, *, empty_eligible_row=False):
    """Op inputs in schema order (fp32 CPU): random masks, some rows ineligible although
    they have allowed slots; every eligible row has at least one allowed slot unless
    ``empty_eligible_row``."""
    g = torch.Generator().manual_seed(seed)
    q = torch.nn.functional.normalize(torch.randn(B, T, H, generator=g), dim=-1)
    K = torch.nn.functional.normalize(torch.randn(B, N, H, generator=g), dim=-1)
    V = torch.randn(B, N, H, generator=g)
    Vn = torch.randn(B, N, H, generator=g)
    ck = torch.nn.functional.normalize(torch.rand(B, T, 4, generator=g), dim=-1)
    cb = torch.nn.functional.normalize(torch.rand(B, N, 4, generator=g), dim=-1)
    kb = torch.randn(B, N, generator=g) * 0.3
    adm = torch.randn(B, N, generator=g) * 0.5
    allow = torch.rand(B, T, N, generator=g) < 0.6
    induct = allow & (torch.rand(B, T, N, generator=g) < 0.7)
    elig = allow.any(-1) & (torch.rand(B, T, generator=g) < 0.9)
    ielig = induct.any(-1) & (torch.rand(B, T, generator=g) < 0.9)
    if empty_eligible_row:
        allow[0, 1] = False
        elig[0, 1] = True
        induct[0, 2] = False
        ielig[0, 2] = True
    scal = [torch.tensor(v) for v in (2.7, 1.1, 0.9, 0.3, 0.8)]  # scale, short, pad, induct, cocktail
    return [q, K, V, Vn, ck, cb, kb, adm, scal[0], allow, induct, elig, ielig, *scal[1:]]


def _cpp(R, x, go):
    q, K, V, Vn, ck, cb, kb, adm, scale, allow, induct, elig, ielig, sg, pg, ig, cg = x
    s = [float(v) for v in (scale, cg, sg, pg, ig)]
    out = R.three_way_read_cpu(q, K, V, Vn, ck, cb, kb, adm, allow, induct, elig, ielig, *s)
    gr = R.three_way_read_bwd(go, q, K, V, Vn, ck, cb, kb, adm, allow, induct, elig, ielig, *s)
    return out, [gr[i] for i in CPP_ORDER]


def _fp64(x, go):
    """Output and the 13 gradients of the fp64 restatement."""
    floats = [v.double().clone().requires_grad_(True) for i, v in enumerate(x)
              if i not in (9, 10, 11, 12)]
    q, K, V, Vn, ck, cb, kb, adm, scale, sg, pg, ig, cg = floats
    out = autograd_ref.dense_read(q, K, V, Vn, ck, cb, kb, adm, scale, x[9], x[10],
                                  (sg, pg, ig, cg), eligible=x[11], induct_eligible=x[12])
    grads = torch.autograd.grad(out, floats, go.double())
    return out.detach(), list(grads)


def _check_grads(got, want, tol, label):
    scalar_floor = 1e-3 * max(float(np.abs(np32(want[i])).max()) for i in SCALARS)
    for i, name in enumerate(NAMES):
        a, b = np.asarray(np32(got[i]), np.float64), np.asarray(np32(want[i]), np.float64)
        assert a.shape == b.shape, f"{label} {name}: shape {a.shape} != {b.shape}"
        if i in SCALARS:
            err = float(np.abs(a - b).max()) / max(float(np.abs(b).max()), scalar_floor)
            assert err <= 5e-5, f"{label} g_{name}: {err:.3e}"
        else:
            assert rel_err(a, b) <= tol, f"{label} g_{name}: {rel_err(a, b):.3e} > {tol}"


def test_fp64_restatement_matches_reference_cpp(R):
    """The restatement with explicit eligibilities against the reference's C++."""
    x = dense_case(1, 2, 13, 9, 11)
    go = torch.randn(2, 13, 11, generator=torch.Generator().manual_seed(2))
    out, grads = _cpp(R, x, go)
    out64, g64 = _fp64(x, go)
    assert rel_err(out, out64) <= 1e-6
    _check_grads(grads, g64, 1e-5, "cpp vs fp64")


def test_fp64_restatement_nan_row_follows_the_registered_op():
    """An eligible row without an allowed slot: NaN in the registered Python op (softmax
    over all -inf, admitted.py:9-13); the short/permanent row here and the induct row."""
    x = dense_case(3, 1, 5, 4, 6, empty_eligible_row=True)
    out, _ = _fp64(x, torch.ones(1, 5, 6))
    assert torch.isnan(out[0, 1]).all() and torch.isnan(out[0, 2]).all()
    assert not torch.isnan(out[0, 0]).any()


def test_op_registration_on_cpu_kernels():
    """Schema, fake kernel and autograd wiring of the op pair (the CPU kernels are the
    oracle restatement registered for tests)."""
    x = dense_case(4, 2, 6, 5, 8)
    for i in (0, 1, 2, 3, 4, 5, 6, 7, 8, 13, 14, 15, 16):
        x[i] = x[i].double().requires_grad_(True)
    torch.library.opcheck(torch.ops.dabsn.admitted_three_way_read_native.default, x,
                          test_utils=("test_schema", "test_autograd_registration",
                                      "test_faketensor"))
    out = ops.admitted_three_way_read_native(*x)
    go = torch.randn(out.shape, dtype=out.dtype, generator=torch.Generator().manual_seed(5))
    floats = [v for i, v in enumerate(x) if i not in (9, 10, 11, 12)]
    got = torch.autograd.grad(out, floats, go)
    _, want = _fp64([v.detach() for v in x], go)
    for a, b in zip(got, want):
        assert a.dtype == torch.float64
        assert rel_err(a, b) <= 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("B,T,N,H", [(2, 11, 7, 9), (2, 300, 257, 64), (1, 96, 1000, 128)])
def test_dense_read_gpu_matches_reference_cpp(cuda_device, R, B, T, N, H):
    x = dense_case(10 + T, B, T, N, H)
    go = torch.randn(B, T, H, generator=torch.Generator().manual_seed(11))
    out_ref, g_ref = _cpp(R, x, go)
    xd = [v.to(cuda_device) for v in x]
    leaves = [v.requires_grad_(True) for i, v in enumerate(xd) if i not in (9, 10, 11, 12)]
    out = ops.admitted_three_way_read_native(*xd)
    assert out.dtype == torch.float32 and out.shape == (B, T, H)
    assert rel_err(out.cpu(), out_ref) <= 1e-5, rel_err(out.cpu(), out_ref)
    grads = torch.autograd.grad(out, leaves, go.to(cuda_device))
    _check_grads([g.cpu() for g in grads], g_ref, 1e-5, f"B={B} T={T} N={N} H={H}")


@pytest.mark.gpu
def test_dense_read_gpu_nan_rows_and_ineligible_rows(cuda_device):
    x = dense_case(20, 1, 5, 40, 16, empty_eligible_row=True)
    go = torch.randn(1, 5, 16, generator=torch.Generator().manual_seed(21))
    out64, _ = _fp64(x, go)
    out = ops.admitted_three_way_read_native(*[v.to(cuda_device) for v in x]).cpu()
    assert torch.equal(torch.isnan(out), torch.isnan(out64))
    ok = ~torch.isnan(out64)
    assert rel_err(out[ok], out64[ok].float()) <= 1e-5


@pytest.mark.gpu
def test_dense_read_gpu_bf16_computes_in_fp32(cuda_device):
    x = dense_case(30, 2, 40, 33, 24)
    for i in (0, 1, 2, 3, 4, 5, 6, 7):
        x[i] = x[i].to(torch.bfloat16)
    xd = [v.to(cuda_device) for v in x]
    leaves = [v.requires_grad_(True) for i, v in enumerate(xd) if i not in (9, 10, 11, 12)]
    out = ops.admitted_three_way_read_native(*xd)
    x32 = [v.float() if i in (0, 1, 2, 3, 4, 5, 6, 7) else v for i, v in enumerate(xd)]
    x32 = [v.detach() for v in x32]
    out32 = ops.admitted_three_way_read_native(*x32)
    assert out.dtype == torch.bfloat16 and torch.equal(out, out32.to(torch.bfloat16))
    go = torch.randn(out.shape, generator=torch.Generator().manual_seed(31)).to(cuda_device)
    grads = torch.autograd.grad(out, leaves, go.to(torch.bfloat16))
    g32 = ops.admitted_three_way_read_native_backward(go.to(torch.bfloat16), *x32)
    for g, w, leaf in zip(grads, g32, leaves):
        assert g.dtype == leaf.dtype
        assert torch.equal(g, w.to(leaf.dtype))
