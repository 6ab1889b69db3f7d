"""The successor fold of the training read (``ops.bank_fold``, the ``fold`` argument of the
kept-workspace read ops, ``bank_gather_kv``).

A bank's successor row of slot j is write[min(idx[j] + 1, T - 1)]. When every admitted
slot's successor is itself a bank row (slot j + 1's, or its own at the clamped last
position) the read moves the induction weights onto those V columns: out = P_V' V, no
successor rows, no gO Vn^T and no P_Vn^T gO GEMM. The reference computes the two products
separately (admitted.py:16-65); the fold changes the summation order only.

  * fold codes and the unfoldable flag against a brute-force restatement of their
    definition on random, dense and suffix banks: bit-exact; likewise the bank width read
    and the slot arrays (idx, valid, next_idx, read_idx, codes) built in one launch;
  * the folded read against the oracle's unfolded read (fp32, 1e-5 normwise), with the
    successor-row gradients of the oracle mapped onto the rows they fold into;
  * bf16 folded against unfolded on the same inputs (2e-2 Frobenius, the bf16 bar);
  * a DABSNRead forward and backward with the fold against the same module with the fold
    switched off (fp32 1e-5 for the output and every gradient).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from dabsn_amd.kernels import ops
from helpers import assert_rel, np32

pytestmark = pytest.mark.gpu


def _brute_fold(order, counts, N):
    """Codes of fold_kernel from their definition: 1 when slot j's next position
    min(i + 1, T - 1) is slot j + 1's position, 0 when it is its own or j >= counts, 2
    otherwise; the flag is any 2 among the admitted slots."""
    B, T = order.shape
    codes = np.zeros((B, N), np.int8)
    bad = 0
    for b in range(B):
        for j in range(int(counts[b])):
            i = int(order[b, j])
            nx = min(i + 1, T - 1)
            if nx == i:
                code = 0
            elif j + 1 < counts[b] and int(order[b, j + 1]) == nx:
                code = 1
            else:
                code = 2
            bad |= code == 2
            if j < N:
                codes[b, j] = code
    return codes, bad


def _admissions(kind, B, T, g):
    if kind == "random":
        return torch.randn(B, T, generator=g) * 0.5, 0.7, 0
    if kind == "dense":
        return torch.randn(B, T, generator=g) * 0.5, 50.0, 0
    # field geometry (whole-row floor) with a contiguous admitted suffix
    adm = torch.full((B, T), -10.0)
    adm[:, T // 3:] = torch.rand(B, T - T // 3, generator=g) * 0.1
    return adm, 1.0, 1


@pytest.mark.parametrize("kind", ["random", "dense", "suffix"])
@pytest.mark.parametrize("B,T", [(3, 1), (2, 37), (4, 300)])
def test_fold_codes_match_their_definition(cuda_device, kind, B, T):
    g = torch.Generator().manual_seed(7 + T)
    adm, window, whole = _admissions(kind, B, T, g)
    order, counts, _ = ops.bank_select(adm.to(cuda_device), torch.tensor([window], device=cuda_device),
                                       whole)
    flag = ops.bank_fold(order, counts)
    n_max = max(int(counts.max()), 1)
    codes = ops.bank_fold(order, counts, n_max)
    want, bad = _brute_fold(order.cpu().numpy(), counts.cpu().numpy(), n_max)
    assert int(flag[0]) == int(bad)
    assert np.array_equal(codes.cpu().numpy(), want)
    if kind != "random" or T == 1:
        assert not bad, "dense and suffix banks fold"


@pytest.mark.parametrize("kind", ["random", "dense", "suffix"])
@pytest.mark.parametrize("B,T", [(3, 1), (2, 37), (4, 300)])
def test_bank_width_and_slots_match_their_definition(cuda_device, kind, B, T):
    """``ops.bank_width`` / ``ops.bank_slots`` (the selection's host read and slot arrays in
    one launch each) against the same values from their definitions on the bank_select
    result: the largest count, the unfoldable flag, order[:, :N], valid = j < max(count, 1),
    min(idx + 1, T - 1), idx - query_start and the fold codes; bit-exact, at the bank's own
    width and at a fixed larger width."""
    g = torch.Generator().manual_seed(11 + T)
    adm, window, whole = _admissions(kind, B, T, g)
    order, counts, _ = ops.bank_select(adm.to(cuda_device), torch.tensor([window], device=cuda_device),
                                       whole)
    o, c = order.cpu().numpy(), counts.cpu().numpy()
    want_codes, bad = _brute_fold(o, c, T)
    top, flag = ops.bank_width(order, counts, True).tolist()
    assert (top, flag) == (int(c.max()), int(bad))
    assert ops.bank_width(order, counts, False).tolist() == [int(c.max()), 0]
    for N in sorted({max(int(c.max()), 1), T}):
        for qs in (0, T // 2):
            idx, valid, nxt, rid, codes = (x.cpu().numpy() if x is not None else None
                                           for x in ops.bank_slots(order, counts, N, qs, True))
            assert np.array_equal(idx, o[:, :N])
            assert np.array_equal(valid, np.arange(N)[None, :] < np.maximum(c, 1)[:, None])
            assert np.array_equal(nxt, np.minimum(o[:, :N] + 1, T - 1))
            assert np.array_equal(rid, o[:, :N] - qs)
            assert np.array_equal(codes, want_codes[:, :N])
    assert ops.bank_slots(order, counts, 1, 0, False)[4] is None


def _case(seed, B, T, H, kind):
    """Bank tensors of a foldable bank as the read module builds them."""
    g = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(B, T, H, generator=g), dim=-1)
    w = torch.randn(B, T, H, generator=g)
    ck = F.normalize(torch.rand(B, T, 4, generator=g), dim=-1)
    kbt = torch.randn(B, T, generator=g) * 0.3
    adm, window, whole = _admissions(kind, B, T, g)
    adm = adm + torch.randn(B, T, generator=g) * 1e-3
    order, counts = oracle.bank_select(np32(adm), window, whole=bool(whole))
    n_max, idx, valid, nidx = oracle.bank_from_order(order, counts)
    codes, bad = _brute_fold(order, counts, n_max)
    assert not bad
    it = torch.from_numpy(idx)
    gat = lambda x: torch.gather(x, 1, it.unsqueeze(-1).expand(-1, -1, x.shape[-1]))  # noqa: E731
    V = gat(w)
    Vn = torch.gather(w, 1, torch.from_numpy(nidx).unsqueeze(-1).expand(-1, -1, H))
    return dict(q=q, K=F.normalize(V, dim=-1), V=V, Vn=Vn, ck=ck, cb=gat(ck),
                kb=torch.gather(kbt, 1, it), adm=torch.gather(adm, 1, it), idx=idx, valid=valid,
                fold=torch.from_numpy(codes), mode=whole)


def _args(c, dev, dtype, with_next):
    d = lambda x: x.to(dev)  # noqa: E731
    act = lambda x: d(x).to(dtype)  # noqa: E731
    return (act(c["q"]), act(c["K"]), act(c["V"]), act(c["Vn"]) if with_next else None,
            d(c["ck"]), d(c["cb"]), d(c["kb"]), d(c["adm"]), torch.tensor([1.9], device=dev),
            d(torch.from_numpy(c["idx"])), d(torch.from_numpy(c["valid"])), c["mode"],
            *[torch.tensor([v], device=dev) for v in (1.0, 0.7, 0.1, 1.3)])


def _fold_rows(gV, gVn, fold):
    """Successor-row gradients added to the rows they fold into (gV[j + fold[j]] +=
    gVn[j]), which is where the folded read puts them."""
    out = gV.astype(np.float64).copy()
    B, N, _ = gV.shape
    for b in range(B):
        for j in range(N):
            out[b, j + int(fold[b, j])] += gVn[b, j]
    return out


@pytest.mark.parametrize("kind", ["dense", "suffix"])
@pytest.mark.parametrize("B,T,H", [(2, 40, 24), (2, 300, 136)])
def test_folded_read_fp32_matches_oracle(cuda_device, kind, B, T, H):
    c = _case(61 + T, B, T, H, kind)
    gains = (1.0, 0.7, 0.1, 1.3)
    a = _args(c, cuda_device, torch.float32, with_next=False)
    fold = c["fold"].to(cuda_device)
    out, ws = ops.read3_fwd_keep(*a, fold)
    host = [np32(c[k]) for k in ("q", "K", "V", "Vn", "ck", "cb", "kb", "adm")]
    ref = oracle.read3_fwd(*host, 1.9, c["idx"], c["valid"], c["mode"], gains)
    assert_rel(out, ref, 1e-5, "folded read output")
    go = torch.randn(B, T, H, generator=torch.Generator().manual_seed(3))
    g = ops.read3_bwd_kept(go.to(cuda_device), *a, ws, fold)
    refb = oracle.read3_bwd(np32(go), *host, 1.9, c["idx"], c["valid"], c["mode"], gains)
    assert g[3].numel() == 0, "no successor-row gradient under the fold"
    assert_rel(g[0], refb[0], 1e-5, "q")
    assert_rel(g[1], refb[1], 1e-5, "K")
    assert_rel(g[2], _fold_rows(refb[2], refb[3], c["fold"].numpy()), 1e-5, "V (+ folded Vn)")
    for n, i in (("cocktail", 4), ("bank_cocktail", 5), ("key_bias", 6), ("admission", 7)):
        assert_rel(g[i], refb[i], 1e-5, n)


@pytest.mark.parametrize("kind", ["dense", "suffix"])
def test_folded_read_bf16_matches_unfolded(cuda_device, kind):
    B, T, H = 2, 520, 256
    c = _case(97, B, T, H, kind)
    fold = c["fold"].to(cuda_device)
    plain = _args(c, cuda_device, torch.bfloat16, with_next=True)
    folded = _args(c, cuda_device, torch.bfloat16, with_next=False)
    out0, ws0 = ops.read3_fwd_keep(*plain)
    out1, ws1 = ops.read3_fwd_keep(*folded, fold)
    assert_rel(out1.float(), out0.float(), 2e-2, "output")
    go = torch.randn(B, T, H, generator=torch.Generator().manual_seed(4)).to(cuda_device, torch.bfloat16)
    g0 = ops.read3_bwd_kept(go, *plain, ws0)
    g1 = ops.read3_bwd_kept(go, *folded, ws1, fold)
    gv0 = _fold_rows(g0[2].float().cpu().numpy(), g0[3].float().cpu().numpy(), c["fold"].numpy())
    pairs = [("q", g1[0], g0[0]), ("K", g1[1], g0[1]), ("V", g1[2], torch.from_numpy(gv0)),
             *[(f"grad {i}", g1[i], g0[i]) for i in range(4, 13)]]
    for name, a, b in pairs:
        a, b = a.float().cpu().double(), b.float().cpu().double()
        err = float((a - b).norm() / max(float(b.norm()), 1e-30))
        assert err <= 2e-2, f"{name}: {err:.3e}"


def test_read_module_fold_equals_unfolded(cuda_device):
    """A dense seq bank (every position admitted): the module's training read takes the fold;
    with the fold switched off it gathers successor rows and runs both products."""
    import dabsn_amd

    torch.manual_seed(5)
    B, T, H = 2, 96, 40
    read = dabsn_amd.DABSNRead(H).to(cuda_device)
    read.admit_window.data.fill_(50.0)
    g = torch.Generator().manual_seed(8)
    # tapes in [0, 1) as the core produces them: finite admissions, all within the window
    tapes = [torch.rand(B, T, H, generator=g).to(cuda_device) for _ in range(8)]
    w = torch.randn(B, T, H, generator=g).to(cuda_device)

    def run(fold: bool):
        leaves = [t.clone().requires_grad_(True) for t in tapes]
        read.zero_grad(set_to_none=True)
        if not fold:
            orig = read._select
            read._select = (lambda a, n, width=None, want_fold=False, query_start=0:
                            orig(a, n, width, False, query_start))
        try:
            out = read(*leaves)
            (out * w).sum().backward()
        finally:
            if not fold:
                del read._select
        grads = [x.grad for x in leaves] + [p.grad for p in read.parameters() if p.grad is not None]
        return out.detach(), grads, read.last_n_max

    out1, g1, n1 = run(True)
    out0, g0, n0 = run(False)
    assert n1 == n0 == T
    assert_rel(out1, out0, 1e-5, "output")
    assert len(g1) == len(g0)
    scale = max(float(x.abs().max()) for x in g0)
    for i, (a, b) in enumerate(zip(g1, g0)):
        err = float((a - b).abs().max()) / max(float(b.abs().max()), 1e-3 * scale)
        assert err <= 1e-5, f"gradient {i}: {err:.3e}"
