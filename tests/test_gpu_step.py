"""GPU kernels of the streaming step's glue against the tensor operations they replace.

  * ``read3_decode_members`` (slots read from a carried bank's admitted-slot lists inside
    the kernel) against ``read3_decode`` on the slot arrays the read module builds from the
    same lists with torch (read.py:185-256 as ``DABSNRead._bank`` evaluates it): bit-exact,
    the two run the same single-pass kernels on identical slot metadata.
  * ``read_mix`` and ``relu_square`` against the unfused torch operations: bit-exact (each
    intermediate rounded to the activation dtype where the unfused tensors are stored).
  * ``rms_norm`` against MLPRMSNorm: fp32 normwise 2e-7 (the mean is summed in another
    order); bf16 results at most one bf16 ulp apart, on at most 1% of the elements.
  * The core scan with its state carried in bf16 (read and written by the kernels) against
    the same scan with the state converted to fp32 and the final state converted back:
    bit-exact, on the one-step path, the persistent scan and a batch split over several
    cooperative launches.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from dabsn_amd.kernels import ops
from dabsn_amd.model import MLPRMSNorm
from helpers import core_case, rel_err

pytestmark = pytest.mark.gpu


def _bank_case(dev, dtype, B, H, cap, Nb, counts, seed):
    """A carried bank as BankStore holds it: [B, cap, .] storage with Nb live positions,
    ascending admitted positions per row (zeros past the count), and glue arrays."""
    g = torch.Generator().manual_seed(seed)
    write = torch.randn(B, cap, H, generator=g).to(dtype)
    stats = torch.rand(B, cap, 6, generator=g) + 0.5
    stats[..., 5] = write.float().norm(dim=-1) * (0.5 + torch.rand(B, cap, generator=g))
    members = torch.zeros(B, cap, dtype=torch.int64)
    for b, c in enumerate(counts):
        members[b, :c] = torch.sort(torch.randperm(Nb, generator=g)[:c]).values
    cocktail = F.normalize(torch.randn(B, cap, 4, generator=g), dim=-1)
    kb, adm = 0.3 * torch.randn(B, cap, generator=g), 0.3 * torch.randn(B, cap, generator=g)
    q = F.normalize(torch.randn(B, 1, H, generator=g), dim=-1).to(dtype)
    d = lambda x: x.to(dev)  # noqa: E731
    return (d(q), d(write), d(stats), d(members), d(torch.tensor(counts, dtype=torch.int64)),
            d(cocktail), d(kb), d(adm))


@pytest.mark.parametrize("dtype,B,H,cap,Nb,width,counts", [
    (torch.bfloat16, 4, 2048, 300, 260, 260, [260, 131, 0, 1]),   # a row with no member
    (torch.float32, 3, 1000, 64, 40, 40, [40, 17, 5]),            # lanes past the row
    (torch.bfloat16, 4, 512, 50, 50, 20, [50, 33, 20, 2]),        # width below the counts
    (torch.bfloat16, 64, 2048, 1100, 1024, 1024, [1024, 700, 3, 512] * 16),
])
def test_decode_members_equals_decode_on_gathered_slots(cuda_device, dtype, B, H, cap, Nb,
                                                        width, counts):
    q, write, stats, members, cnt, cocktail, kb, adm = _bank_case(
        cuda_device, dtype, B, H, cap, Nb, counts, 100 + H)
    scale = torch.tensor(2.5, device=cuda_device)
    gains = tuple(torch.tensor(v, device=cuda_device) for v in (1.0, 0.7, 0.2, 0.9))
    qs = Nb - 1
    with torch.no_grad():
        got = ops.read3_decode_members(q, write, stats, Nb, width, members, cnt, qs, cocktail,
                                       kb, adm, scale, gains)
        # the slot arrays as DABSNRead._bank builds them from the same lists
        idx = members[:, :width]
        valid = torch.arange(width, device=cuda_device).unsqueeze(0) < cnt.clamp_min(1).unsqueeze(1)
        next_idx = (idx + 1).clamp(max=Nb - 1)
        live = lambda t: t[:, :Nb]  # noqa: E731
        want = ops.read3_decode(
            q, live(write), live(stats)[..., 5], idx, next_idx, idx - qs, valid,
            live(cocktail)[:, Nb - 1:], torch.gather(live(cocktail), 1,
                                                     idx.unsqueeze(-1).expand(-1, -1, 4)),
            torch.gather(live(kb), 1, idx), torch.gather(live(adm), 1, idx), scale, gains)
    assert torch.equal(got, want)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(4, 1, 2048), (3, 5, 24), (7, 3)])
def test_read_mix_and_relu_square_equal_the_tensor_operations(cuda_device, dtype, shape):
    g = torch.Generator().manual_seed(9)
    proj, long, y = (torch.randn(shape, generator=g).to(cuda_device, dtype) for _ in range(3))
    lg = torch.tensor([0.1], device=cuda_device, dtype=dtype)
    rg = torch.tensor([0.01], device=cuda_device, dtype=dtype)
    with torch.no_grad():
        got = ops.read_mix(proj, long, lg, y, rg)
        want = y + rg * (proj + lg * long)
        assert got.dtype == want.dtype and torch.equal(got, want)
        x = torch.randn(shape, generator=g).to(cuda_device, dtype)
        x.view(-1)[0] = float("nan")
        x.view(-1)[1] = -0.0
        got = ops.relu_square(x)
        want = F.relu(x).square()
        assert torch.equal(got.nan_to_num(7.0), want.nan_to_num(7.0))
        assert torch.isnan(got.view(-1)[0])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,H", [(256, 2048), (5, 24), (3, 1000)])
def test_rms_norm_matches_the_module(cuda_device, dtype, rows, H):
    g = torch.Generator().manual_seed(H)
    norm = MLPRMSNorm(H).to(cuda_device, dtype)
    with torch.no_grad():
        norm.weight.copy_(1.0 + 0.3 * torch.randn(H, generator=g))
        x = (3.0 * torch.randn(rows, H, generator=g)).to(cuda_device, dtype)
        got = ops.rms_norm(x, norm.weight, norm.eps)
        want = norm(x)
    assert got.dtype == want.dtype
    if dtype == torch.float32:
        assert rel_err(got.cpu(), want.cpu()) <= 2e-7
    else:
        a, b = got.float().cpu(), want.float().cpu()
        ulp = torch.finfo(torch.bfloat16).eps * torch.maximum(a.abs(), b.abs())
        assert bool(((a - b).abs() <= ulp).all())
        assert float((a != b).float().mean()) <= 0.01


@pytest.mark.parametrize("B,T,H", [(40, 1, 2048), (6, 9, 64), (256, 3, 2048)])
def test_core_scan_carries_a_bf16_state(cuda_device, B, T, H):
    inp = [t.to(cuda_device) for t in core_case(52, B, T, H)]
    inp[0], inp[1] = inp[0].bfloat16(), inp[1].bfloat16()
    states = [s.bfloat16() for s in inp[23:26]]
    with torch.no_grad():
        got = ops.core_scan_batched(*inp[:23], *states)
        want = ops.core_scan_batched(*inp[:23], *[s.float() for s in states])
    for i in range(8):
        assert torch.equal(got[i], want[i]), f"tape {i}"
    for i in range(8, 11):
        assert got[i].dtype == torch.bfloat16
        assert torch.equal(got[i], want[i].bfloat16()), f"final state {i - 8}"
