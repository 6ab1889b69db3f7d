"""The read's fused glue (``ops.slot_glue``, ``dabsn_hip_glue_slots`` and its backward)
against the torch expressions it replaces (read.py:58-72, 155-183, 241-256: means in the tape
dtype, key bias, admission, cocktails, gathered per admitted slot), evaluated by the CPU
path of the read module (``_ArrayGlue``) on the same statistics rows.

  * key bias and admission: bit-exact (the slot selection reads the admission; the kernel
    uses the same log1p and the torch operation order without contraction);
  * cocktails: 1e-6 relative (the norm of four values may be summed in another order);
  * gradients (statistics rows' means, the eight gains): against fp64 autograd of the same
    expressions at the same rounded values (with bf16 tapes the means, mean_p * H and its
    log1p are rounded to bf16 as the forward rounds them), 1e-5 relative (the backward is
    evaluated in fp32).
"""

from __future__ import annotations

import pytest
import torch

import dabsn_amd
from dabsn_amd.kernels import ops
from dabsn_amd.read import _cocktail

pytestmark = pytest.mark.gpu

PARAM_NAMES = ("p_gain", "novelty_gain", "null_bias", "adm_p_gain", "adm_novelty_gain",
               "adm_saturation_gain", "adm_energy_gain", "adm_bias")


def _case(seed, B, L, C, N):
    g = torch.Generator().manual_seed(seed)
    bank = torch.rand(B, L, 6, generator=g)
    bank[..., 3] *= 0.05  # plasticity means: small, as the core produces them
    query = torch.rand(B, C, 6, generator=g)
    idx = torch.stack([torch.randperm(L, generator=g)[:N].sort().values for _ in range(B)])
    params = [torch.randn(1, generator=g) for _ in range(8)]
    return bank, query, idx, params


def _torch_glue(bank, query, idx, params, H, tape_dtype):
    """read.py's expressions on the statistics rows, gathered by slot."""
    rp = dabsn_amd.DABSNRead(H).short_read.to(bank.device)
    for n, p in zip(PARAM_NAMES, params):
        getattr(rp, n).data.copy_(p)
    be, bc, bn, bp = (m.to(tape_dtype) for m in bank.unbind(-1)[:4])
    qe, qc, qn, qp = (m.to(tape_dtype) for m in query.unbind(-1)[:4])
    kb = rp.key_bias_from_means(bn, bp, H)
    adm = rp.admission_from_means(be, bc, bn, bp, H)
    cb = _cocktail(be, bc, bn, bp)
    ck = _cocktail(qe, qc, qn, qp)
    e = idx.unsqueeze(-1)
    return (torch.gather(kb, 1, idx), torch.gather(adm, 1, idx),
            torch.gather(cb, 1, e.expand(-1, -1, 4)), ck), rp


@pytest.mark.parametrize("tape_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,L,C,N", [(2, 40, 40, 31), (3, 300, 64, 250)])
def test_slot_glue_matches_torch_expressions(cuda_device, tape_dtype, B, L, C, N):
    H = 96
    bank, query, idx, params = _case(5 + L, B, L, C, N)
    d = lambda x: x.to(cuda_device)  # noqa: E731
    bank_d = d(bank).requires_grad_(True)
    query_d = d(query).requires_grad_(True)
    prm_d = [d(p).requires_grad_(True) for p in params]
    kb, adm, cb, ck = ops.slot_glue(bank_d, query_d, d(idx), H, prm_d, tape_dtype)

    # Forward against the torch expressions on the device (same math library).
    bank_t = d(bank).requires_grad_(True)
    query_t = d(query).requires_grad_(True)
    (kb_t, adm_t, cb_t, ck_t), _ = _torch_glue(bank_t, query_t, d(idx), params, H, tape_dtype)
    assert torch.equal(adm, adm_t.float()), "admission"
    assert torch.equal(kb, kb_t.float()), "key bias"
    for name, a, b in (("bank cocktail", cb, cb_t), ("query cocktail", ck, ck_t)):
        err = float((a - b.float()).abs().max() / b.float().abs().max())
        assert err <= (1e-6 if tape_dtype == torch.float32 else 8e-3), f"{name}: {err:.3e}"

    # Backward against autograd of the same expressions, in fp64 from the rounded means.
    g = torch.Generator().manual_seed(9)
    gk, ga = torch.randn(B, N, generator=g), torch.randn(B, N, generator=g)
    gc, gq = torch.randn(B, N, 4, generator=g), torch.randn(B, C, 4, generator=g)
    torch.autograd.backward([kb, adm, cb, ck], [d(gk), d(ga), d(gc), d(gq)])
    b64 = bank.double().requires_grad_(True)
    q64 = query.double().requires_grad_(True)
    p64 = [p.double().requires_grad_(True) for p in params]
    # Every value the forward rounds to the tape dtype is rounded here too, with an identity
    # gradient (the kernel differentiates at the rounded values).
    rb = lambda x: x.to(tape_dtype).double() if tape_dtype != torch.float32 else x  # noqa: E731
    st = lambda x: x + (rb(x.detach()) - x.detach())  # noqa: E731
    be, bc, bn, bp = (st(m) for m in b64.unbind(-1)[:4])
    qe, qc, qn, qp = (st(m) for m in q64.unbind(-1)[:4])
    lp = st(torch.log1p(st(bp * H)))
    kb64 = p64[0] * lp + p64[1] * bn + p64[2]
    adm64 = p64[3] * lp + p64[4] * bn + p64[5] * bc + p64[6] * be + p64[7]
    cb64 = _cocktail(be, bc, bn, bp)
    ck64 = _cocktail(qe, qc, qn, qp)
    e = idx.unsqueeze(-1).expand(-1, -1, 4)
    outs = (torch.gather(kb64, 1, idx), torch.gather(adm64, 1, idx), torch.gather(cb64, 1, e), ck64)
    torch.autograd.backward(outs, [gk.double(), ga.double(), gc.double(), gq.double()])

    def rel(a, b):
        a, b = a.detach().double().cpu(), b.detach().double()
        return float((a - b).abs().max() / max(float(b.abs().max()), 1e-30))

    assert rel(bank_d.grad, b64.grad) <= 1e-5, f"bank rows: {rel(bank_d.grad, b64.grad):.3e}"
    assert rel(query_d.grad, q64.grad) <= 1e-5, f"query rows: {rel(query_d.grad, q64.grad):.3e}"
    for n, a, b in zip(PARAM_NAMES, prm_d, p64):
        assert rel(a.grad, b.grad) <= 1e-5, f"{n}: {rel(a.grad, b.grad):.3e}"
