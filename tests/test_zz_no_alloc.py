"""The allocation-free decode read (dabsn_hip_read3_decode_noalloc), called through the C
ABI, against the workspace entry point it shares its kernels with (dabsn_hip_read3_decode).

The two must agree bit for bit: the same kernels run on the same inputs, only the scratch
differs (the library's per-device array instead of a caller's workspace). Each case makes
two calls in a row on one device, the second with a smaller input, so a result that
depended on what the first call left in the shared array would show. Cases: the one-pass
read (one query row, bf16 and fp32) and the three-pass read (several query rows); a
request larger than the array is refused with DABSN_ERR_ARG and nothing enqueued.
"""

from __future__ import annotations

import pytest
import torch

from dabsn_amd import _lib
from dabsn_amd.kernels import ops

pytestmark = pytest.mark.gpu


def _case(seed, B, T, H, Nb, ld, N, dtype, device):
    g = torch.Generator().manual_seed(seed)
    buf = torch.randn(B, ld, H, generator=g).to(device, dtype)
    bank = buf[:, :Nb]
    norm_w = bank.float().norm(dim=-1)
    idx = torch.stack([torch.randperm(Nb, generator=g)[:N].sort().values for _ in range(B)])
    nxt = (idx + 1).clamp(max=Nb - 1)
    read_idx = idx - (Nb - T)
    valid = torch.rand(B, N, generator=g) < 0.9
    q = torch.nn.functional.normalize(torch.randn(B, T, H, generator=g), dim=-1).to(device, dtype)
    ck = torch.nn.functional.normalize(torch.rand(B, T, 4, generator=g), dim=-1)
    cb = torch.nn.functional.normalize(torch.rand(B, N, 4, generator=g), dim=-1)
    kb = torch.randn(B, N, generator=g) * 0.3
    adm = torch.randn(B, N, generator=g) * 0.3
    d = lambda x: x.to(device)  # noqa: E731
    return dict(q=q, bank=bank, norm_w=d(norm_w), idx=d(idx), nxt=d(nxt), read_idx=d(read_idx),
                valid=d(valid.to(torch.uint8)), ck=d(ck), cb=d(cb), kb=d(kb), adm=d(adm),
                scale=torch.tensor(7.5, device=device),
                gains=[torch.tensor(v, device=device) for v in (1.0, 0.8, 0.2, 1.1)])


def _args(c):
    B, T, H = c["q"].shape
    N = c["idx"].shape[1]
    bank = c["bank"]
    code = 1 if c["q"].dtype == torch.bfloat16 else 0
    gains = _lib.PTR4(*[x.data_ptr() for x in c["gains"]])
    return [code, B, T, N, H, c["q"].data_ptr(), bank.data_ptr(), bank.shape[1],
            bank.stride(0) // H, c["norm_w"].data_ptr(), c["idx"].data_ptr(), c["nxt"].data_ptr(),
            c["read_idx"].data_ptr(), c["valid"].data_ptr(), c["ck"].data_ptr(),
            c["cb"].data_ptr(), c["kb"].data_ptr(), c["adm"].data_ptr(), c["scale"].data_ptr(),
            gains]


def _with_workspace(c):
    lib = _lib.load()
    a = _args(c)
    out = torch.empty_like(c["q"])
    nbytes = lib.dabsn_hip_read3_decode_workspace_bytes(*a[:5])
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=out.device)
    _lib.check(lib.dabsn_hip_read3_decode(*a, out.data_ptr(), ws.data_ptr(), ws.numel(),
                                          ops._stream(out)), "decode read")
    return out


def _without_allocation(c):
    lib = _lib.load()
    out = torch.empty_like(c["q"])
    _lib.check(lib.dabsn_hip_read3_decode_noalloc(*_args(c), out.data_ptr(), ops._stream(out)),
               "decode read without allocation")
    return out


@pytest.mark.parametrize("dtype,T,H", [(torch.bfloat16, 1, 2048), (torch.float32, 1, 256),
                                       (torch.bfloat16, 3, 512)])
def test_noalloc_decode_equals_workspace_decode_twice(cuda_device, dtype, T, H):
    big = _case(1, 6, T, H, Nb=700, ld=900, N=500, dtype=dtype, device=cuda_device)
    small = _case(2, 2, T, H, Nb=90, ld=90, N=40, dtype=dtype, device=cuda_device)
    for c in (big, small):
        want = _with_workspace(c)
        got = _without_allocation(c)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got, want)


def test_noalloc_decode_refuses_a_plan_beyond_its_scratch(cuda_device):
    lib = _lib.load()
    c = _case(3, 1, 1, 64, Nb=80, ld=80, N=40, dtype=torch.float32, device=cuda_device)
    a = _args(c)
    a[1] = 4096          # B
    a[3] = 1 << 20       # N: slot metadata alone exceeds the array
    rc = lib.dabsn_hip_read3_decode_noalloc(*a, c["q"].data_ptr(), ops._stream(c["q"]))
    assert rc == -2
    assert b"more than" in lib.dabsn_hip_last_error()
