"""Seq DABSN block with block time-chunking, plus a minimal token harness.

``DABSNBlock`` follows the reference block (src/dabsn/model.py:110-378): core scan
(optionally time-chunked with a carried (b, e, c) state and a per-chunk checkpoint,
model.py:197-307), read, ``state_to_hidden(y + read_gain * read)``, residual and the
optional squared-ReLU MLP. ``DABSNSequenceLM`` is a small token-in/logits-out harness
around a stack of seq blocks, used to drive the hot path in tests and the benchmark;
it is not a port of the reference's backbone/graph machinery.
"""

from __future__ import annotations

import os

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor
from torch.utils.checkpoint import checkpoint

from .core import DABSNCore
from .read import DABSNRead


class MLPRMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.eps = float(eps)
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, inputs: Tensor) -> Tensor:
        scale = torch.rsqrt(inputs.float().pow(2).mean(-1, keepdim=True) + self.eps)
        return (inputs.float() * scale).to(inputs.dtype) * self.weight


class DABSNBlock(nn.Module):
    """One core plus admitted/permanent/induction/long read (seq geometry)."""

    def __init__(self, input_dim: int, hidden_dim: int, state_dim: int, read_geometry: str = "seq",
                 *, residual: bool = False, mlp_ratio: float | None = None,
                 block_chunk_t: int | None = None) -> None:
        super().__init__()
        self.input_dim, self.hidden_dim, self.state_dim = input_dim, hidden_dim, state_dim
        self.read_geometry = read_geometry
        self.core = DABSNCore(input_dim=input_dim, hidden_dim=state_dim)
        self.read = DABSNRead(hidden_dim=state_dim, read_geometry=read_geometry)
        self.read_gain = nn.Parameter(torch.full((1,), 0.01))
        self.state_to_hidden = (nn.Identity() if state_dim == hidden_dim
                                else nn.Linear(state_dim, hidden_dim))
        self.residual = bool(residual)
        self.residual_skip = None
        if self.residual and input_dim != hidden_dim:
            self.residual_skip = nn.Linear(input_dim, hidden_dim, bias=False)
            nn.init.normal_(self.residual_skip.weight, mean=0.0, std=(1.0 / input_dim) ** 0.5)
        self.mlp_ratio = None if mlp_ratio is None else float(mlp_ratio)
        self.mlp_norm = self.mlp_fc1 = self.mlp_fc2 = None
        if self.mlp_ratio is not None:
            inner = int(round(self.mlp_ratio * hidden_dim))
            self.mlp_norm = MLPRMSNorm(hidden_dim)
            self.mlp_fc1 = nn.Linear(hidden_dim, inner, bias=False)
            self.mlp_fc2 = nn.Linear(inner, hidden_dim, bias=False)
            nn.init.normal_(self.mlp_fc1.weight, mean=0.0, std=0.02)
            nn.init.zeros_(self.mlp_fc2.weight)
        self.block_chunk_t = block_chunk_t
        self.last_trace: dict[str, object] = {}

    def _resolve_block_chunk_t(self, inputs: Tensor) -> int:
        """``block_chunk_t`` / ``DABSN_BLOCK_CHUNK_T``: -1 off, >0 explicit width, 0 off
        (model.py:197-272; with 288 GB of HBM the automatic memory-pressure rule never
        engages at the shapes this backend targets, so auto means off)."""
        T = int(inputs.shape[1])
        setting = self.block_chunk_t
        if setting is None:
            raw = os.environ.get("DABSN_BLOCK_CHUNK_T")
            setting = int(raw) if raw not in (None, "") else 0
        if setting <= 0:
            return 0
        return min(setting, T)

    def _chunked_core(self, inputs: Tensor, chunk_t: int):
        """Exact time-chunked core scan with carried state (model.py:274-307)."""
        B, T, _ = inputs.shape
        zeros = torch.zeros(B, self.state_dim, device=inputs.device, dtype=torch.float32)
        carry = (zeros, torch.ones_like(zeros), zeros.clone())
        tapes: list[list[Tensor]] = [[] for _ in range(7)]
        use_ckpt = self.training and torch.is_grad_enabled()
        for t0 in range(0, T, chunk_t):
            chunk = inputs[:, t0:min(T, t0 + chunk_t)]

            def run(chunk_in, b_in, e_in, c_in):
                result, final = self.core.forward_from_state(
                    chunk_in, initial_state=(b_in, e_in, c_in), return_writes=True,
                    return_cocktail=True, return_final_state=True)
                return (*result, *final)

            outs = (checkpoint(run, chunk, *carry, use_reentrant=False) if use_ckpt
                    else run(chunk, *carry))
            for i in range(7):
                tapes[i].append(outs[i])
            carry = (outs[7], outs[8], outs[9])
        return tuple(torch.cat(parts, dim=1) for parts in tapes)

    def core_tapes(self, inputs: Tensor):
        chunk_t = self._resolve_block_chunk_t(inputs)
        if chunk_t and chunk_t < int(inputs.shape[1]):
            if inputs.is_cuda and self.training and torch.is_grad_enabled():
                return self.core.chunked_tapes(inputs, chunk_t)
            return self._chunked_core(inputs, chunk_t)
        return self.core(inputs, return_writes=True, return_cocktail=True)

    def forward_world(self, inputs: Tensor) -> Tensor:
        trajectory, novelty, plasticity, expression, write, energy, saturation = self.core_tapes(inputs)
        y, budget = trajectory.split(self.state_dim, dim=-1)
        read = self.read(y, budget, expression, write, novelty, plasticity, energy, saturation)
        out = self.finish(inputs, self.state_to_hidden(y + self.read_gain * read))
        self.last_trace = {"read_geometry": self.read_geometry,
                           "admitted_n_max": self.read.last_n_max,
                           "read_contract": self.read.last_read_contract}
        return out

    def finish(self, inputs: Tensor, dabsn_output: Tensor) -> Tensor:
        """The block output before the MLP: the DABSN path plus the residual skip, if any."""
        if not self.residual:
            return dabsn_output
        skip = inputs if self.residual_skip is None else self.residual_skip(inputs)
        return skip + dabsn_output

    def forward_mlp(self, hidden: Tensor) -> Tensor:
        if self.mlp_fc2 is None:
            return hidden
        return hidden + self.mlp_fc2(F.relu(self.mlp_fc1(self.mlp_norm(hidden))).square())

    def forward(self, inputs: Tensor) -> Tensor:
        return self.forward_mlp(self.forward_world(inputs))


class DABSNSequenceLM(nn.Module):
    """Token embedding -> seq DABSN blocks -> readout (test/benchmark harness)."""

    def __init__(self, vocab: int, hidden_dim: int, layers: list[tuple[int, int]], *,
                 residual: bool = False, mlp_ratio: float | None = None,
                 block_chunk_t: int | None = None) -> None:
        super().__init__()
        self.embed = nn.Embedding(vocab, hidden_dim)
        blocks = []
        width = hidden_dim
        for hidden, state in layers:
            blocks.append(DABSNBlock(width, hidden, state, "seq", residual=residual,
                                     mlp_ratio=mlp_ratio, block_chunk_t=block_chunk_t))
            width = hidden
        self.blocks = nn.ModuleList(blocks)
        self.readout = nn.Linear(width, vocab)
        nn.init.normal_(self.embed.weight, mean=0.0, std=0.02)
        nn.init.zeros_(self.readout.bias)

    def forward(self, ids: Tensor) -> Tensor:
        h = self.embed(ids)
        for block in self.blocks:
            h = block(h)
        return self.readout(h)
