"""Carried memory (ingest / forward_with_memory) against one dense pass of the same model.

Reference behaviour: src/dabsn/memory.py and its exactness claim (tests/test_memory_carry.py
of the reference: chunked ingest against a growing bank reproduces one dense pass to
float32 rounding). CPU variants run through the test-only oracle backend
(oracle/torch_backend.py registers the C oracle as the ops' CPU kernels); GPU variants run
the HIP kernels, and every expected value -- the dense pass or the fresh ingest -- is the
CPU oracle run of the same weights. fp32 throughout; tolerance normwise 1e-5 (the chunked
read sums over a bank of a different width, so reductions differ in order).
"""

from __future__ import annotations

import copy

import pytest
import torch

import dabsn_amd
from dabsn_amd import memory as mem
from helpers import rel_err
from oracle import torch_backend


@pytest.fixture(scope="module", autouse=True)
def _oracle_cpu_kernels():
    torch_backend.register()


def _model(device):
    torch.manual_seed(7)
    model = dabsn_amd.DABSNSequenceLM(40, 24, layers="seq:24:24,seq:32:16", residual=True, mlp_ratio=2.0)
    for block in model.blocks:
        block.read.admit_window.data.fill_(0.3)  # a partially admitted bank
    return model.to(device).eval()


def _pair(device):
    """The model on ``device`` and the same weights on the CPU, where the ops run the
    oracle: every expected value below comes from the CPU oracle run."""
    cpu = _model("cpu")
    return copy.deepcopy(cpu).to(device), cpu


def _dense(model, ids):
    with torch.no_grad():
        h = model.embed(ids)
        for block in model.blocks:
            h = block(h)
        return h, model.readout(h)


def _ids(B, T, seed=8):
    return torch.randint(0, 40, (B, T), generator=torch.Generator().manual_seed(seed))


def _chunked_ingest(device):
    model, cpu = _pair(device)
    ids = _ids(2, 45)
    want, _ = _dense(cpu, ids)
    got, memory = mem.forward_with_memory(model, ids.to(device), None, chunk_size=8,
                                          return_hidden=True)
    assert memory.position == 45 and memory.entries == 45
    assert [layer.bank.length for layer in memory.layers] == [45, 45]
    return got.cpu(), want


def _decode(device):
    model, cpu = _pair(device)
    ids = _ids(3, 26, seed=9)
    _, want = _dense(cpu, ids)
    ids = ids.to(device)
    memory = mem.ingest(model, ids[:, :20], chunk_size=6)
    memory.reserve(26)
    logits = []
    for t in range(20, 26):
        step, memory = mem.forward_with_memory(model, ids[:, t:t + 1], memory, extend=True)
        logits.append(step)
    assert memory.position == 26
    return torch.cat(logits, dim=1).cpu(), want[:, 20:]


def test_bank_store_appends_in_place_and_doubles():
    bank = mem.BankStore(2, 3, device="cpu", dtype=torch.float32, capacity=2)
    rows = torch.arange(2 * 5 * 3, dtype=torch.float32).reshape(2, 5, 3)
    stats = torch.arange(2 * 5 * 6, dtype=torch.float32).reshape(2, 5, 6)
    bank.append(rows[:, :2], stats[:, :2])
    storage = bank.write
    bank.append(rows[:, 2:3], stats[:, 2:3])  # full: grows to max(3, 2 * 2) = 4
    assert bank.capacity == 4 and bank.write is not storage
    storage = bank.write
    bank.append(rows[:, 3:4], stats[:, 3:4])  # fits: written in place
    assert bank.write is storage and bank.length == 4
    bank.reserve(16)
    bank.append(rows[:, 4:], stats[:, 4:])
    w, s = bank.live()
    assert bank.capacity == 16 and torch.equal(w, rows) and torch.equal(s, stats)


def test_parameter_edits_through_data_need_parameters_changed():
    """Kept parameter copies and a carried bank's admission key follow a parameter's storage
    and version counter; an in-place edit through ``.data`` moves neither (the contract:
    call ``parameters_changed()`` after it), ``load_state_dict`` does."""
    from dabsn_amd.kernels import ops

    p = torch.nn.Parameter(torch.ones(3))
    twice = lambda x: x * 2  # noqa: E731
    with ops.reuse_parameter_copies():
        a = ops._derived("test_twice", (p,), twice)
        p.data.copy_(torch.full((3,), 5.0))
        assert torch.equal(ops._derived("test_twice", (p,), twice), a)  # kept: stale
        dabsn_amd.kernels.parameters_changed()
        assert torch.equal(ops._derived("test_twice", (p,), twice), torch.full((3,), 10.0))
        with torch.no_grad():
            p.copy_(torch.full((3,), 7.0))  # what load_state_dict does: the version moves
        assert torch.equal(ops._derived("test_twice", (p,), twice), torch.full((3,), 14.0))
    read = dabsn_amd.DABSNRead(8)
    key = mem.BankStore.glue_key(read, torch.float32, 8)
    read.short_read.adm_bias.data.copy_(torch.tensor([0.5]))
    assert mem.BankStore.glue_key(read, torch.float32, 8) == key
    dabsn_amd.kernels.parameters_changed()
    assert mem.BankStore.glue_key(read, torch.float32, 8) != key
    read.load_state_dict(dabsn_amd.DABSNRead(8).state_dict())
    moved = mem.BankStore.glue_key(read, torch.float32, 8)
    assert moved[0] != key[0]


def test_memory_refuses_other_architecture_or_batch():
    model = _model("cpu")
    memory = mem.DABSNMemory(layers=[], position=0, batch_size=2,
                             fingerprint=mem.fingerprint_of(model))
    with pytest.raises(ValueError, match="batch"):
        mem.forward_with_memory(model, _ids(3, 4), memory)
    other = dabsn_amd.DABSNSequenceLM(40, 24, layers="seq:24:24", residual=True, mlp_ratio=2.0)
    with pytest.raises(ValueError, match="different architecture"):
        mem.forward_with_memory(other, _ids(2, 4), memory)


def test_chunked_ingest_equals_dense_pass_cpu():
    got, want = _chunked_ingest("cpu")
    assert rel_err(got, want) <= 1e-5


def test_decode_token_by_token_equals_dense_pass_cpu():
    got, want = _decode("cpu")
    assert rel_err(got, want) <= 1e-5


def test_read_only_query_leaves_memory_unchanged_cpu():
    model = _model("cpu")
    ids = _ids(2, 30)
    memory = mem.ingest(model, ids[:, :24], chunk_size=10)
    a, m1 = mem.forward_with_memory(model, ids[:, 24:], memory)
    b, m2 = mem.forward_with_memory(model, ids[:, 24:], memory)
    assert m1 is memory and m2 is memory and memory.position == 24
    assert [layer.bank.length for layer in memory.layers] == [24, 24]
    assert torch.equal(a, b)
    c, grown = mem.forward_with_memory(model, ids[:, 24:], memory, extend=True)
    assert torch.equal(a, c) and grown.position == 30 and grown.entries == 30


def _branches(device):
    """Two continuations extended from one prefix handle, each against a fresh ingest of
    its own full sequence (the reference rebuilds the bank per call, memory.py:250-254, so
    branching from a shared prefix is valid there)."""
    model, cpu = _pair(device)
    ids = _ids(2, 16, seed=13)
    alt = ids.clone()
    alt[:, 12:] = (alt[:, 12:] + 7) % 40
    fresh_a, _ = mem.forward_with_memory(cpu, ids, None, chunk_size=None)
    fresh_b, _ = mem.forward_with_memory(cpu, alt, None, chunk_size=None)
    ids, alt = ids.to(device), alt.to(device)
    base = mem.ingest(model, ids[:, :12], chunk_size=5)
    out_a, mem_a = mem.forward_with_memory(model, ids[:, 12:], base, extend=True)
    out_b, mem_b = mem.forward_with_memory(model, alt[:, 12:], base, extend=True)
    assert base.position == 12 and [layer.entries for layer in base.layers] == [12, 12]
    assert mem_a.position == mem_b.position == 16
    # The first branch again, after the second one extended the shared prefix.
    again, _ = mem.forward_with_memory(model, ids[:, 12:], base, extend=True)
    return ((out_a.cpu(), fresh_a[:, 12:]), (out_b.cpu(), fresh_b[:, 12:]),
            (again.cpu(), fresh_a[:, 12:]))


def test_branching_from_one_prefix_equals_fresh_ingest_cpu():
    for got, want in _branches("cpu"):
        assert rel_err(got, want) <= 1e-5


@pytest.mark.gpu
def test_branching_from_one_prefix_equals_fresh_oracle_ingest_gpu(cuda_device):
    for got, want in _branches(cuda_device):
        assert rel_err(got, want) <= 1e-5


@pytest.mark.gpu
def test_chunked_ingest_equals_oracle_dense_pass_gpu(cuda_device):
    got, want = _chunked_ingest(cuda_device)
    assert rel_err(got, want) <= 1e-5


@pytest.mark.gpu
def test_decode_token_by_token_equals_oracle_dense_pass_gpu(cuda_device):
    got, want = _decode(cuda_device)
    assert rel_err(got, want) <= 1e-5


def _continue(model, memory, ids):
    out = []
    for t in range(ids.shape[1]):
        step, memory = mem.forward_with_memory(model, ids[:, t:t + 1], memory, extend=True)
        out.append(step)
    return torch.cat(out, dim=1), memory


def test_saved_memory_reloads_and_continues_exactly_cpu(tmp_path):
    """save -> load (weights_only) -> decode equals decoding the memory that was saved."""
    model = _model("cpu")
    ids = _ids(2, 24)
    memory = mem.ingest(model, ids[:, :18], chunk_size=7)
    path = mem.save(memory, tmp_path / "ctx.dmem")
    loaded = mem.load(path, model=model)
    assert loaded.position == 18 and loaded.entries == 18 and loaded.batch_size == 2
    a, _ = _continue(model, memory, ids[:, 18:])
    b, _ = _continue(model, loaded, ids[:, 18:])
    assert torch.equal(a, b)


def test_reference_format_file_loads_cpu(tmp_path):
    """A file in the reference's payload (five bank fields, no statistics rows): the means
    come from the file and the write norms are recomputed, so decoding continues to fp32
    rounding of the norms (1e-5)."""
    model = _model("cpu")
    ids = _ids(2, 24, seed=11)
    memory = mem.ingest(model, ids[:, :18], chunk_size=9)
    payload = mem._to_payload(memory)
    for layer in payload["layers"]:
        del layer["bank"]["stats"]
        for k in mem.MEAN_FIELDS:  # the reference stores the means in the tape dtype
            layer["bank"][f"{k}_mean"] = layer["bank"][f"{k}_mean"].float()
    torch.save(payload, tmp_path / "ref.dmem")
    loaded = mem.load(tmp_path / "ref.dmem", model=model)
    a, _ = _continue(model, memory, ids[:, 18:])
    b, _ = _continue(model, loaded, ids[:, 18:])
    assert rel_err(b, a) <= 1e-5


def test_memory_embeds_in_checkpoint_and_rejects_foreign_payload_cpu(tmp_path):
    model = _model("cpu")
    memory = mem.ingest(model, _ids(2, 10), chunk_size=None)
    ckpt = tmp_path / "model.pt"
    torch.save({"state_dict": model.state_dict()}, ckpt)
    assert mem.extract_from_checkpoint(ckpt) is None
    mem.embed_in_checkpoint(memory, ckpt)
    back = mem.extract_from_checkpoint(ckpt, model=model)
    assert back is not None and back.position == 10
    assert torch.equal(back.layers[0].bank.live()[0], memory.layers[0].bank.live()[0])
    assert "state_dict" in torch.load(ckpt, weights_only=True)
    torch.save({"format": "something_else"}, tmp_path / "bad.dmem")
    with pytest.raises(ValueError, match="not a DABSN memory payload"):
        mem.load(tmp_path / "bad.dmem")


@pytest.mark.gpu
def test_means_glue_matches_the_read_modules_expressions(cuda_device):
    """The fused key bias / admission / cocktail kernel of the inference path against the
    torch expressions the training path uses (read.py key_bias_from_means,
    admission_from_means, _cocktail), on the live prefix of a longer bank buffer and with
    non-default gains: fp32, relative 1e-6 (log1p and the norm may round differently)."""
    from dabsn_amd import read as R
    from dabsn_amd.kernels import ops

    g = torch.Generator().manual_seed(12)
    read = R.DABSNRead(64).to(cuda_device)
    rp = read.short_read
    with torch.no_grad():
        for prm in (rp.p_gain, rp.novelty_gain, rp.null_bias, rp.adm_p_gain, rp.adm_novelty_gain,
                    rp.adm_saturation_gain, rp.adm_energy_gain, rp.adm_bias):
            prm.copy_(torch.randn(prm.shape, generator=g).to(cuda_device))
    buf = torch.rand(3, 50, 6, generator=g).to(cuda_device)
    stats = buf[:, :37]
    prm = (rp.p_gain, rp.novelty_gain, rp.null_bias, rp.adm_p_gain, rp.adm_novelty_gain,
           rp.adm_saturation_gain, rp.adm_energy_gain, rp.adm_bias)
    with torch.no_grad():
        kb, adm, ck = ops.means_glue(stats, 64, prm)
        e, c, n, p = stats.unbind(-1)[:4]
        want = (rp.key_bias_from_means(n, p, 64), rp.admission_from_means(e, c, n, p, 64),
                R._cocktail(e, c, n, p))
    for got, w in zip((kb, adm, ck), want):
        assert rel_err(got.cpu(), w.cpu()) <= 1e-6


@pytest.mark.gpu
@pytest.mark.parametrize("adm_bf16", [False, True])
def test_incremental_admission_equals_bank_select(cuda_device, adm_bf16):
    """Slot lists built position chunk by position chunk (1, 7, 300, 1 ... positions at a
    time) equal bank_select over the whole bank at every length: counts and the member
    prefix of the order, bit for bit (ties and a constant row included)."""
    from dabsn_amd.kernels import ops
    g = torch.Generator().manual_seed(21)
    B, T = 5, 700
    adm = torch.randint(-40, 40, (B, T), generator=g).float() / 8.0
    adm[1] = adm[1, 0]
    if adm_bf16:
        adm = adm.bfloat16().float()
    adm = adm.to(cuda_device)
    window = torch.tensor([1.5], device=cuda_device)
    members = torch.zeros((B, T), device=cuda_device, dtype=torch.int64)
    mcount = torch.full((B,), 99, device=cuda_device, dtype=torch.int64)  # restarts at base 0
    amax = torch.zeros((B,), device=cuda_device, dtype=torch.float32)
    kb = torch.zeros((B, T), device=cuda_device)
    ck = torch.zeros((B, T, 4), device=cuda_device)
    lo = 0
    for n in (1, 7, 300, 1, 1, 90, 300):
        # stats None: membership of the admission values already in `adm`
        ops.admit_step(None, 1, [], torch.float32, window, lo, n, kb, adm, ck, amax, mcount,
                       members, adm_bf16)
        lo += n
        ref = adm[:, :lo].bfloat16() if adm_bf16 else adm[:, :lo]
        order, counts, _ = ops.bank_select(ref, window)
        assert torch.equal(mcount, counts)
        for b in range(B):
            c = int(counts[b])
            assert torch.equal(members[b, :c], order[b, :c]), (lo, b)
            assert not members[b, c:lo].any()


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_incremental_admission_decode_is_bit_identical_to_full_recompute(cuda_device, dtype):
    """Streaming decode with the kept glue and slot lists against the same decode that
    recomputes them over the whole bank every step (the reference's way): identical logits,
    through a prompt, token-by-token steps, a read-only query (rows appended then dropped)
    and a change of a read parameter between steps (the kept glue is rebuilt). One-row
    steps read the slots from the kept lists inside the decode kernel; the recompute builds
    the slot arrays with torch first."""
    model = _model(cuda_device).to(dtype)
    ids = _ids(3, 40, seed=17).to(cuda_device)

    def run():
        out = []
        memory = mem.ingest(model, ids[:, :24], chunk_size=10)
        for t in range(24, 32):
            step, memory = mem.forward_with_memory(model, ids[:, t:t + 1], memory, extend=True)
            out.append(step)
        peek, _ = mem.forward_with_memory(model, ids[:, 32:35], memory)  # read-only
        out.append(peek)
        with torch.no_grad():
            model.blocks[0].read.short_read.adm_bias.add_(0.25)
        for t in range(32, 40):
            step, memory = mem.forward_with_memory(model, ids[:, t:t + 1], memory, extend=True)
            out.append(step)
        with torch.no_grad():
            model.blocks[0].read.short_read.adm_bias.sub_(0.25)
        return torch.cat(out, dim=1)

    assert mem._INCREMENTAL_ADMISSION
    got = run()
    try:
        mem._INCREMENTAL_ADMISSION = False
        want = run()
    finally:
        mem._INCREMENTAL_ADMISSION = True
    assert torch.equal(got, want)
