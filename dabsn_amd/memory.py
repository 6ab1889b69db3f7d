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
from typing import Iterator

import torch
from torch import Tensor

from .kernels import ops
from .model import DABSNBlock, DABSNSequenceLM

__all__ = ["BankStore", "LayerMemory", "DABSNMemory", "ingest", "forward_with_memory",
           "fingerprint_of"]


class BankStore:
    """One block's bank: write vectors [B, cap, H] and statistics rows [B, cap, 6] (fp32),
    of which the first ``length`` positions are live."""

    def __init__(self, batch: int, hidden: int, *, device, dtype, capacity: int = 0) -> None:
        self.batch, self.hidden = int(batch), int(hidden)
        self.length = 0
        self.write = torch.empty((batch, max(int(capacity), 0), hidden), device=device,
                                 dtype=dtype)
        self.stats = torch.empty((batch, max(int(capacity), 0), 6), device=device,
                                 dtype=torch.float32)

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
        self.write, self.stats = write, stats

    def append(self, write: Tensor, stats: Tensor) -> None:
        """Write a chunk's rows after the live prefix (doubling the storage when full)."""
        n = int(write.shape[1])
        need = self.length + n
        if need > self.capacity:
            self.reserve(max(need, 2 * self.capacity))
        self.write[:, self.length:need].copy_(write)
        self.stats[:, self.length:need].copy_(stats)
        self.length = need

    def live(self) -> tuple[Tensor, Tensor]:
        return self.write[:, :self.length], self.stats[:, :self.length]

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

    @property
    def entries(self) -> int:
        return self.bank.length

    def nbytes(self) -> int:
        return self.bank.nbytes() + sum(t.numel() * t.element_size()
                                        for t in (*self.core, *self.long))


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

    def reserve(self, tokens: int) -> None:
        """Preallocate every bank for ``tokens`` positions in total (no regrowth below it)."""
        for layer in self.layers:
            layer.bank.reserve(int(tokens))

    def __repr__(self) -> str:  # pragma: no cover - display only
        return (f"DABSNMemory(tokens={self.position}, batch={self.batch_size}, "
                f"layers={len(self.layers)}, {self.nbytes() / 2**20:.1f} MiB)")


def fingerprint_of(model: DABSNSequenceLM) -> dict[str, object]:
    """Architecture identity a memory must match (memory.py:149-161)."""
    blocks = list(model.blocks)
    return {
        "vocab": int(model.embed.num_embeddings),
        "hidden_dim": int(model.embed.embedding_dim),
        "depth": len(blocks),
        "layers": [[int(b.hidden_dim), int(b.state_dim), b.read_geometry] for b in blocks],
        "residual": bool(blocks[0].residual) if blocks else False,
        "mlp_ratio": blocks[0].mlp_ratio if blocks else None,
    }


def _check(memory: DABSNMemory, model: DABSNSequenceLM, batch: int) -> None:
    expected = fingerprint_of(model)
    if memory.fingerprint and dict(memory.fingerprint) != expected:
        bad = [f"{k}: memory={memory.fingerprint.get(k)!r} model={v!r}"
               for k, v in expected.items() if memory.fingerprint.get(k) != v]
        raise ValueError("memory was built by a different architecture: " + "; ".join(bad))
    if memory.batch_size != batch:
        raise ValueError(f"memory holds batch {memory.batch_size} but ids are batch {batch}; "
                         "a bank is per-lane and cannot be rebatched")


def _chunks(total: int, size: int | None) -> Iterator[tuple[int, int]]:
    if size is None or size <= 0 or size >= total:
        yield 0, total
        return
    for start in range(0, total, size):
        yield start, min(total, start + size)


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
    stats = ops.read_tape_stats(novelty, plasticity, energy, saturation, expression, write)
    if layer is None:
        bank = BankStore(batch, block.state_dim, device=write.device, dtype=write.dtype,
                         capacity=int(write.shape[1]))
    else:
        bank = layer.bank
    bank.append(write, stats)
    bank_write, bank_stats = bank.live()
    # Decode-sized steps read at the full bank width (no host sync per layer and token).
    width = bank.length if int(inputs.shape[1]) <= 8 else None
    retrieved, final_long = block.read.forward_query_bank_stats(
        y, budget, expression, write, plasticity, query_stats=stats, bank_write=bank_write,
        bank_stats=bank_stats, query_start=position,
        initial_long_state=None if layer is None else layer.long, bank_width=width)
    out = block.finish(inputs, block.state_to_hidden(y + block.read_gain * retrieved))
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
    lengths = [layer.bank.length for layer in memory.layers] if memory is not None else []
    outputs = []
    with torch.no_grad():
        for start, stop in _chunks(int(ids.shape[1]), chunk_size):
            hidden = model.embed(ids[:, start:stop])
            for i, block in enumerate(blocks):
                hidden, state[i] = _block_step(block, hidden, state[i], position)
            outputs.append(hidden)
            position += stop - start
    hidden = outputs[0] if len(outputs) == 1 else torch.cat(outputs, dim=1)
    if memory is not None and not extend:
        # A read-only query (memory.py:340-345): the rows appended past each bank's live
        # prefix are dropped, and the carried core/long states were never modified.
        for layer, n in zip(memory.layers, lengths):
            layer.bank.length = n
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
    extended should not be used through an older handle afterwards."""
    hidden, result = _run(model, ids, memory, chunk_size=chunk_size, extend=extend)
    if return_hidden:
        return hidden, result
    return model.readout(hidden), result
