"""Carried DABSN memory: ingest context once, then query it or extend it token by token.

Reference behaviour: src/dabsn/memory.py (``LayerMemory``, ``DABSNMemory``, ``ingest``,
``forward_with_memory``; the per-block step at memory.py:215-290 and the chunk driver at
293-347), built on the query-bank read (read.py:650-838). Three states carry per block,
all needed for exactness: the bank of past writes, the core's (budget, energy,
saturation) and the long scan's (long, expected, retention).

What differs is how the bank is held:

* The reference keeps ``write`` plus four per-position means and grows them with
  ``torch.cat`` on every chunk (memory.py:250-254), then widens the means back to
  full-width views for the read. Here each bank lives in storage with spare capacity
  (doubling, or reserved up front with ``reserve``) and a chunk is written in place
  after the live prefix, so a decode step copies one token's row, not the bank.
* Per position it keeps the row of ``ops.read_tape_stats`` computed when that position
  was read as a query (means of energy, saturation, novelty, plasticity; query and write
  norms). The read needs the bank's tapes only through those statistics, and the rows are
  the ones a dense pass over the whole sequence computes, so chunked ingest and
  token-by-token decode reproduce one dense pass (up to the summation order of the
  read's reductions over a different bank width).

Only seq read geometry is supported, as in the reference (memory.py:184-196).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from pathlib import Path
from typing import Iterator, Mapping, Sequence

import torch
from torch import Tensor

from .kernels import ops
from .model import DABSNBlock, DABSNSequenceLM

__all__ = ["BankStore", "LayerMemory", "DABSNMemory", "ingest", "forward_with_memory",
           "fingerprint_of", "save", "load", "embed_in_checkpoint", "extract_from_checkpoint",
           "memory_cost"]

#: File format tag and bank field names of the reference's memory files (memory.py:55-87).
FORMAT = "dabsn_memory_v1"
MEAN_FIELDS = ("novelty", "plasticity", "energy", "saturation")
BANK_FIELDS = ("write",) + tuple(f"{name}_mean" for name in MEAN_FIELDS)
# Column of each mean in a read_tape_stats row: (energy, saturation, novelty, plasticity,
# query norm, write norm).
_STATS_COLUMN = {"energy": 0, "saturation": 1, "novelty": 2, "plasticity": 3}


class BankStore:
    """One block's bank: write vectors [B, cap, H] and statistics rows [B, cap, 6] (fp32),
    of which the first ``length`` positions are live.

    For inference on the device it also keeps, per position, the read glue (key bias,
    admission, cocktail) and, per batch row, the admitted-slot list with its count and the
    running admission prefix max (``admission``): in seq geometry a position's floor and
    membership depend only on the positions before it, so each decode step computes them for
    its new positions alone. They are recomputed from the statistics rows whenever the read
    parameters changed (storage or version) since they were computed."""

    def __init__(self, batch: int, hidden: int, *, device, dtype, capacity: int = 0) -> None:
        self.batch, self.hidden = int(batch), int(hidden)
        self.length = 0
        cap = max(int(capacity), 0)
        self.write = torch.empty((batch, cap, hidden), device=device, dtype=dtype)
        self.stats = torch.empty((batch, cap, 6), device=device, dtype=torch.float32)
        self._glue_arrays(cap)
        self.admitted = 0          # positions whose glue and membership are current
        self._glue_key: tuple | None = None

    def _glue_arrays(self, cap: int) -> None:
        dev = self.stats.device
        self.key_bias = torch.empty((self.batch, cap), device=dev, dtype=torch.float32)
        self.adm = torch.empty((self.batch, cap), device=dev, dtype=torch.float32)
        self.cocktail = torch.empty((self.batch, cap, 4), device=dev, dtype=torch.float32)
        # positions past a row's count stay 0: a valid index for the reads, masked by `valid`
        self.members = torch.zeros((self.batch, cap), device=dev, dtype=torch.int64)
        self.mcount = torch.zeros((self.batch,), device=dev, dtype=torch.int64)
        self.amax = torch.zeros((self.batch,), device=dev, dtype=torch.float32)

    @property
    def capacity(self) -> int:
        return int(self.write.shape[1])

    def reserve(self, capacity: int) -> None:
        """Grow the storage to hold at least ``capacity`` positions (keeps the live prefix)."""
        if capacity <= self.capacity:
            return
        write = torch.empty((self.batch, capacity, self.hidden), device=self.write.device,
                            dtype=self.write.dtype)
        stats = torch.empty((self.batch, capacity, 6), device=self.stats.device,
                            dtype=torch.float32)
        if self.length:
            write[:, :self.length].copy_(self.write[:, :self.length])
            stats[:, :self.length].copy_(self.stats[:, :self.length])
        old = (self.key_bias, self.adm, self.cocktail, self.members, self.mcount, self.amax)
        self.write, self.stats = write, stats
        self._glue_arrays(capacity)
        n = self.admitted
        if n:
            self.key_bias[:, :n].copy_(old[0][:, :n])
            self.adm[:, :n].copy_(old[1][:, :n])
            self.cocktail[:, :n].copy_(old[2][:, :n])
            self.members[:, :n].copy_(old[3][:, :n])
            self.mcount.copy_(old[4])
            self.amax.copy_(old[5])

    def admission(self, read, hidden: int, tape_dtype: torch.dtype, length: int):
        """(key_bias [B, L], admission [B, L], cocktail [B, L, 4], (slot list [B, cap],
        counts [B])) of the first ``length`` live positions for ``read`` (a DABSNRead in seq
        geometry), extending the kept glue and admitted-slot lists by the positions appended
        since the last call in one kernel (read.py:58-72, 155-191 for each new position,
        then its membership under the causal floor). Inference on the device only."""
        rp = read.short_read
        prm = (rp.p_gain, rp.novelty_gain, rp.null_bias, rp.adm_p_gain, rp.adm_novelty_gain,
               rp.adm_saturation_gain, rp.adm_energy_gain, rp.adm_bias)
        key = self.glue_key(read, tape_dtype, hidden)
        if key != self._glue_key or self.admitted > length:
            self._glue_key, self.admitted = key, 0
        lo = self.admitted
        if lo < length:
            # The reference's admission is a bf16 tensor when tapes and gains are: its floor
            # is rounded to bf16 too (as in bank_select).
            adm_bf16 = tape_dtype == torch.bfloat16 and rp.adm_bias.dtype == torch.bfloat16
            window = ops._derived("admit_window_f32", (read.admit_window,),
                                  lambda w: torch.nn.functional.softplus(w).float().reshape(()))
            ops.admit_step(self.stats, hidden, prm, tape_dtype, window, lo, length - lo,
                           self.key_bias, self.adm, self.cocktail, self.amax, self.mcount,
                           self.members, adm_bf16)
            self.admitted = length
        return (self.key_bias[:, :length], self.adm[:, :length], self.cocktail[:, :length],
                (self.members, self.mcount))

    @staticmethod
    def glue_key(read, tape_dtype: torch.dtype, hidden: int) -> tuple:
        """What the kept glue and slot lists depend on besides the bank rows: the admission
        parameters (storage, version counter, dtype), the tape dtype, the width and the
        parameter generation. An in-place edit through ``.data`` moves none of the first,
        so it must be followed by ``ops.parameters_changed()`` (which moves the last)."""
        rp = read.short_read
        watched = (rp.p_gain, rp.novelty_gain, rp.null_bias, rp.adm_p_gain, rp.adm_novelty_gain,
                   rp.adm_saturation_gain, rp.adm_energy_gain, rp.adm_bias, read.admit_window)
        return (tuple((p.data_ptr(), p._version, p.dtype) for p in watched), tape_dtype, hidden,
                ops.parameter_generation())

    def append(self, write: Tensor, stats: Tensor) -> None:
        """Write a chunk's rows after the live prefix (doubling the storage when full)."""
        n = int(write.shape[1])
        need = self.length + n
        if need > self.capacity:
            self.reserve(max(need, 2 * self.capacity))
        self.write[:, self.length:need].copy_(write)
        self.stats[:, self.length:need].copy_(stats)
        self.length = need

    def live(self, length: int | None = None) -> tuple[Tensor, Tensor]:
        n = self.length if length is None else int(length)
        return self.write[:, :n], self.stats[:, :n]

    def truncate(self, length: int) -> None:
        """Drop the positions from ``length`` on (a read-only query's rows). Glue and slot
        lists that cover dropped positions are rebuilt on the next ``admission`` call."""
        self.length = int(length)
        if self.admitted > self.length:
            self.admitted, self._glue_key = 0, None

    def fork(self, length: int, extra: int = 0) -> "BankStore":
        """A new store holding a copy of the first ``length`` positions, with room for
        ``extra`` more: used when a handle whose live prefix is shorter than the storage's
        (another handle extended the bank past it) extends or queries again."""
        out = BankStore(self.batch, self.hidden, device=self.write.device,
                        dtype=self.write.dtype, capacity=int(length) + int(extra))
        if length:
            w, st = self.live(length)
            out.append(w, st)
        return out

    def to(self, *, device=None, dtype=None) -> "BankStore":
        out = BankStore(self.batch, self.hidden, device=device or self.write.device,
                        dtype=dtype or self.write.dtype, capacity=self.length)
        if self.length:
            w, s = self.live()
            out.append(w.to(device=out.write.device, dtype=out.write.dtype),
                       s.to(device=out.stats.device))
        return out

    def nbytes(self) -> int:
        w, s = self.live()
        return w.numel() * w.element_size() + s.numel() * s.element_size()


@dataclass
class LayerMemory:
    """One block's carried state (memory.py:90-114)."""

    bank: BankStore
    core: tuple[Tensor, Tensor, Tensor]
    long: tuple[Tensor, Tensor, Tensor]
    #: Live bank positions as seen by this handle. The storage is shared by every handle
    #: derived from one prefix and may hold more rows (written by a later extension).
    length: int = -1

    def __post_init__(self) -> None:
        if self.length < 0:
            self.length = self.bank.length

    @property
    def entries(self) -> int:
        return self.length

    def live(self) -> tuple[Tensor, Tensor]:
        return self.bank.live(self.length)

    def nbytes(self) -> int:
        w, st = self.live()
        return (w.numel() * w.element_size() + st.numel() * st.element_size()
                + sum(t.numel() * t.element_size() for t in (*self.core, *self.long)))

    def to(self, *, device=None, dtype=None) -> "LayerMemory":
        """A copy on ``device``; ``dtype`` applies to the bank's write vectors (the
        statistics and the carried core and long states stay fp32)."""
        bank = self.bank.fork(self.length).to(device=device, dtype=dtype)
        return LayerMemory(bank=bank, core=tuple(t.to(device=device) for t in self.core),
                           long=tuple(t.to(device=device) for t in self.long),
                           length=self.length)


@dataclass
class DABSNMemory:
    """Carried memory for a whole model: one LayerMemory per block (memory.py:117-146)."""

    layers: list[LayerMemory] = field(default_factory=list)
    position: int = 0
    batch_size: int = 0
    fingerprint: dict[str, object] = field(default_factory=dict)

    @property
    def entries(self) -> int:
        """Bank entries in layer 0, i.e. tokens ingested."""
        return self.layers[0].entries if self.layers else 0

    def nbytes(self) -> int:
        return sum(layer.nbytes() for layer in self.layers)

    def to(self, device=None, dtype=None) -> "DABSNMemory":
        return DABSNMemory(layers=[layer.to(device=device, dtype=dtype) for layer in self.layers],
                           position=self.position, batch_size=self.batch_size,
                           fingerprint=dict(self.fingerprint))

    def reserve(self, tokens: int) -> None:
        """Preallocate every bank for ``tokens`` positions in total (no regrowth below it)."""
        for layer in self.layers:
            layer.bank.reserve(int(tokens))

    def __repr__(self) -> str:  # pragma: no cover - display only
        return (f"DABSNMemory(tokens={self.position}, batch={self.batch_size}, "
                f"layers={len(self.layers)}, {self.nbytes() / 2**20:.1f} MiB)")


def fingerprint_of(model: DABSNSequenceLM) -> dict[str, object]:
    """Architecture identity a memory must match: the reference's dictionary, key for key
    (memory.py:149-161), so files cross-load in both directions."""
    return {
        "vocab": int(model.vocab),
        "hidden_dim": int(model.hidden_dim),
        "depth": int(model.depth),
        "layers": [spec.to_metadata() for spec in model.layers],
        "tie_embeddings": bool(model.tie_embeddings),
        "residual": bool(model.residual),
        "mlp_ratio": model.mlp_ratio,
        "mlp_middle_depth": int(model.mlp_middle_depth),
        "mlp_depth_index": int(model.mlp_depth_index),
    }


def _check_fingerprint(memory: DABSNMemory, model: DABSNSequenceLM) -> None:
    """The reference's rule (memory.py:164-181): an empty fingerprint passes; keys that
    predate residual/MLP support default to the disabled architecture; anything else must
    equal the model's fingerprint."""
    if not memory.fingerprint:
        return
    expected = fingerprint_of(model)
    observed = dict(memory.fingerprint)
    observed.setdefault("residual", False)
    observed.setdefault("mlp_ratio", None)
    observed.setdefault("mlp_middle_depth", 0)
    observed.setdefault("mlp_depth_index", 0)
    if observed != expected:
        bad = [f"{k}: memory={observed.get(k)!r} model={v!r}"
               for k, v in expected.items() if observed.get(k) != v]
        raise ValueError("memory was built by a different architecture: " + "; ".join(bad))


def _check(memory: DABSNMemory, model: DABSNSequenceLM, batch: int) -> None:
    _check_fingerprint(memory, model)
    if memory.batch_size != batch:
        raise ValueError(f"memory holds batch {memory.batch_size} but ids are batch {batch}; "
                         "a bank is per-lane and cannot be rebatched")


def _chunks(total: int, size: int | None) -> Iterator[tuple[int, int]]:
    if size is None or size <= 0 or size >= total:
        yield 0, total
        return
    for start in range(0, total, size):
        yield start, min(total, start + size)


#: Extend each bank's glue and admitted-slot lists by the new positions only (the default);
#: False recomputes them over the whole bank every step, as the reference does.
_INCREMENTAL_ADMISSION = True


def _block_step(block: DABSNBlock, inputs: Tensor, layer: LayerMemory | None,
                position: int) -> tuple[Tensor, LayerMemory]:
    """One block over a chunk from carried state, extending its bank (memory.py:215-290):
    core from the carried (b, e, c), the chunk's tape statistics appended to the bank, the
    read of the chunk against the bank ending at the chunk, ``state_to_hidden``, residual
    and MLP as in ``DABSNBlock.forward``."""
    batch = int(inputs.shape[0])
    core_state = (layer.core if layer is not None
                  else block.core.initial_state(batch, device=inputs.device))
    result, final_core = block.core.forward_from_state(
        inputs, initial_state=core_state, return_writes=True, return_cocktail=True,
        return_final_state=True)
    trajectory, novelty, plasticity, expression, write, energy, saturation = result
    y, budget = trajectory.split(block.state_dim, dim=-1)
    stats = ops.direct.read_tape_stats(novelty, plasticity, energy, saturation, expression, write)
    if layer is None:
        bank = BankStore(batch, block.state_dim, device=write.device, dtype=write.dtype,
                         capacity=int(write.shape[1]))
    elif layer.bank.length != layer.length:
        # Another handle extended this storage past our prefix: copy the prefix, so the
        # two continuations never read each other's rows.
        bank = layer.bank.fork(layer.length, int(write.shape[1]))
    else:
        bank = layer.bank
    bank.append(write, stats)
    bank_write, bank_stats = bank.live()
    # Decode-sized steps read at the full bank width (no host sync per layer and token).
    width = bank.length if int(inputs.shape[1]) <= 8 else None
    mixed, final_long = block.read.forward_query_bank_stats(
        y, budget, expression, write, plasticity, query_stats=stats, bank_write=bank_write,
        bank_stats=bank_stats, query_start=position,
        initial_long_state=None if layer is None else layer.long, bank_width=width,
        bank_store=bank if _INCREMENTAL_ADMISSION else None, mix=(y, block.read_gain))
    out = block.finish(inputs, block.state_to_hidden(mixed))
    return block.forward_mlp(out), LayerMemory(bank=bank, core=final_core, long=final_long)


def _run(model: DABSNSequenceLM, ids: Tensor, memory: DABSNMemory | None, *,
         chunk_size: int | None, extend: bool) -> tuple[Tensor, DABSNMemory]:
    if ids.dim() != 2:
        raise ValueError(f"ids must be [B, T]; got {tuple(ids.shape)}")
    blocks = list(model.blocks)
    if any(b.read_geometry != "seq" for b in blocks):
        raise NotImplementedError("carried memory is exact only for seq read geometry")
    batch = int(ids.shape[0])
    if memory is None:
        state: list[LayerMemory | None] = [None] * len(blocks)
        position = 0
    else:
        _check(memory, model, batch)
        state = list(memory.layers)
        position = memory.position
    lengths = [layer.length for layer in memory.layers] if memory is not None else []
    outputs = []
    with torch.no_grad(), ops.reuse_parameter_copies():
        for start, stop in _chunks(int(ids.shape[1]), chunk_size):
            hidden = model.embed(ids[:, start:stop])
            for i, block in enumerate(blocks):
                hidden, state[i] = _block_step(block, hidden, state[i], position)
            outputs.append(hidden)
            position += stop - start
    hidden = outputs[0] if len(outputs) == 1 else torch.cat(outputs, dim=1)
    if memory is not None and not extend:
        # A read-only query (memory.py:340-345): the rows appended past each bank's live
        # prefix are dropped (the storage's length returns to the handle's), and the
        # carried core/long states were never modified.
        for layer, new_state, n in zip(memory.layers, state, lengths):
            if new_state is not None and new_state.bank is layer.bank:
                layer.bank.truncate(n)
        return hidden, memory
    result = DABSNMemory(layers=[s for s in state if s is not None], position=position,
                         batch_size=batch, fingerprint=fingerprint_of(model))
    return hidden, result


def ingest(model: DABSNSequenceLM, ids: Tensor, memory: DABSNMemory | None = None, *,
           chunk_size: int | None = 512) -> DABSNMemory:
    """Read ``ids`` into memory, extending ``memory`` when one is given (memory.py:350-365).
    Any chunk width reproduces one dense pass; the width only bounds the working set."""
    _, result = _run(model, ids, memory, chunk_size=chunk_size, extend=True)
    return result


def forward_with_memory(model: DABSNSequenceLM, ids: Tensor, memory: DABSNMemory | None = None,
                        *, chunk_size: int | None = None, extend: bool = False,
                        return_hidden: bool = False) -> tuple[Tensor, DABSNMemory]:
    """Score ``ids`` against carried ``memory`` and return (logits [B, T, vocab], memory)
    (memory.py:368-386). With ``extend=False`` the memory passed in is returned unchanged,
    so repeated independent queries see the same context; with ``extend=True`` the query
    tokens are appended (streaming decode). Banks are extended in place: a memory that was
    extended should not be used through an older handle afterwards. The ops reuse their
    fp32 copies of the model's parameters, and the banks their admission glue and slot
    lists, across calls while each parameter keeps its storage and version counter
    (``load_state_dict`` moves the counter); a weight edited in place through ``.data``
    between calls needs ``dabsn_amd.kernels.ops.parameters_changed()``."""
    hidden, result = _run(model, ids, memory, chunk_size=chunk_size, extend=extend)
    if return_hidden:
        return hidden, result
    return model.readout(hidden), result


# ---- files ----------------------------------------------------------------------------
def _to_payload(memory: DABSNMemory) -> dict[str, object]:
    """The reference's payload (memory.py:389-403): per layer the five bank fields, core and
    long. The bank also carries ``stats``, the fp32 rows this package reads, so its own
    round trip is exact; the reference's loader takes only its five fields."""
    layers = []
    for layer in memory.layers:
        write, stats = layer.live()
        bank = {"write": write.detach().cpu()}
        for name in MEAN_FIELDS:
            bank[f"{name}_mean"] = stats[..., _STATS_COLUMN[name]].detach().cpu().to(write.dtype)
        bank["stats"] = stats.detach().cpu()
        layers.append({"bank": bank, "core": [t.detach().cpu() for t in layer.core],
                       "long": [t.detach().cpu() for t in layer.long]})
    return {"format": FORMAT, "position": int(memory.position),
            "batch_size": int(memory.batch_size), "fingerprint": dict(memory.fingerprint),
            "layers": layers}


def _from_payload(payload) -> DABSNMemory:
    if not isinstance(payload, Mapping) or payload.get("format") != FORMAT:
        fmt = payload.get("format") if isinstance(payload, Mapping) else type(payload).__name__
        raise ValueError(f"not a DABSN memory payload: its format tag is {fmt!r}, this "
                         f"loader reads {FORMAT!r}")
    raw_layers = payload.get("layers")
    if not isinstance(raw_layers, Sequence):
        raise ValueError("DABSN memory payload: 'layers' holds no list of layer entries")
    layers = []
    for entry in raw_layers:
        bank = entry.get("bank") if isinstance(entry, Mapping) else None
        if not isinstance(bank, Mapping):
            raise ValueError("DABSN memory payload: a layer entry has no 'bank' mapping")
        missing = [k for k in BANK_FIELDS if k not in bank]
        if missing:
            raise ValueError(f"DABSN memory payload: a layer's bank lacks {missing}")
        core, long = entry.get("core"), entry.get("long")
        if not (isinstance(core, Sequence) and len(core) == 3 and isinstance(long, Sequence)
                and len(long) == 3):
            raise ValueError("DABSN memory payload: a layer's 'core' and 'long' entries are "
                             "not three state tensors each")
        write = bank["write"]
        if not isinstance(write, Tensor) or write.dim() != 3:
            raise ValueError("DABSN memory payload: a layer's bank 'write' is not a 3-D "
                             "[B, N, H] tensor")
        stats = bank.get("stats")
        if not isinstance(stats, Tensor):
            # A file written by the reference: the means are stored, the write norms are not.
            stats = torch.zeros(*write.shape[:2], 6, dtype=torch.float32)
            for name in MEAN_FIELDS:
                stats[..., _STATS_COLUMN[name]] = bank[f"{name}_mean"].float()
            stats[..., 5] = torch.linalg.vector_norm(write.float(), dim=-1)
        store = BankStore(write.shape[0], write.shape[2], device=write.device, dtype=write.dtype,
                          capacity=write.shape[1])
        store.append(write, stats.float())
        layers.append(LayerMemory(bank=store, core=tuple(t.float() for t in core),
                                  long=tuple(t.float() for t in long)))
    return DABSNMemory(layers=layers, position=int(payload["position"]),
                       batch_size=int(payload["batch_size"]),
                       fingerprint=dict(payload.get("fingerprint") or {}))


def _check_loaded(memory: DABSNMemory, model: DABSNSequenceLM) -> None:
    """A loaded memory must match the model (memory.py:164-181, 479-486), and each bank's
    width must be its block's state width."""
    _check_fingerprint(memory, model)
    blocks = list(model.blocks)
    if len(memory.layers) != len(blocks) or any(
            layer.bank.hidden != int(block.state_dim) for layer, block in zip(memory.layers, blocks)):
        raise ValueError("memory layers do not match the model's blocks")
    memory.fingerprint = fingerprint_of(model)


def save(memory: DABSNMemory, path) -> Path:
    """Write ``memory`` to its own file (memory.py:461-466)."""
    destination = Path(path)
    destination.parent.mkdir(parents=True, exist_ok=True)
    torch.save(_to_payload(memory), destination)
    return destination


def load(path, *, model: DABSNSequenceLM | None = None, map_location="cpu", device=None,
         dtype=None) -> DABSNMemory:
    """Read a memory file (memory.py:469-491), written by this package or by the reference.
    The file is read with ``weights_only=True``: a payload of tensors, numbers, strings,
    lists and dicts, nothing executed. With ``model`` it is checked against the model and
    moved to its device, the bank's writes cast to its dtype."""
    payload = torch.load(Path(path), map_location=map_location, weights_only=True)
    if isinstance(payload, Mapping) and "dabsn_memory" in payload:
        payload = payload["dabsn_memory"]
    memory = _from_payload(payload)
    if model is not None:
        _check_loaded(memory, model)
        ref = next(model.parameters())
        memory = memory.to(device=device or ref.device, dtype=dtype or ref.dtype)
    elif device is not None or dtype is not None:
        memory = memory.to(device=device, dtype=dtype)
    return memory


def embed_in_checkpoint(memory: DABSNMemory, checkpoint, *, destination=None) -> Path:
    """Attach ``memory`` to a dict checkpoint under ``dabsn_memory`` (memory.py:494-514)."""
    source = Path(checkpoint)
    target = Path(destination) if destination is not None else source
    payload = torch.load(source, map_location="cpu", weights_only=True)
    if not isinstance(payload, dict):
        raise ValueError(f"can only embed memory into a dict checkpoint; {source} holds "
                         f"{type(payload).__name__}")
    payload["dabsn_memory"] = _to_payload(memory)
    torch.save(payload, target)
    return target


def extract_from_checkpoint(checkpoint, *, model: DABSNSequenceLM | None = None,
                            map_location="cpu") -> DABSNMemory | None:
    """The memory embedded in a checkpoint, or None (memory.py:517-532)."""
    payload = torch.load(Path(checkpoint), map_location=map_location, weights_only=True)
    if not isinstance(payload, dict) or "dabsn_memory" not in payload:
        return None
    memory = _from_payload(payload["dabsn_memory"])
    if model is not None:
        _check_loaded(memory, model)
        ref = next(model.parameters())
        memory = memory.to(device=ref.device, dtype=ref.dtype)
    return memory


def memory_cost(model: DABSNSequenceLM, tokens: int, *, batch_size: int = 1,
                bytes_per_element: int = 2) -> dict[str, object]:
    """Bank bytes for ``tokens`` ingested tokens (memory.py:535-549, with this package's
    layout: per layer one write vector in the activation dtype plus a six-float statistics
    row per position)."""
    per_token = sum(int(block.state_dim) * bytes_per_element + 6 * 4 for block in model.blocks)
    total = per_token * tokens * batch_size
    return {"bytes_per_token": per_token * batch_size, "total_bytes": total,
            "total_mib": total / 1024 / 1024}
