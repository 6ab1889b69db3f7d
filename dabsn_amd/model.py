"""Seq DABSN block with block time-chunking, plus a minimal token harness.

``DABSNBlock`` follows the reference block (src/dabsn/model.py:110-378): core scan
(optionally time-chunked with a carried (b, e, c) state and a per-chunk checkpoint,
model.py:197-307), read in seq, field or hybrid geometry,
``state_to_hidden(y + read_gain * read)``, residual and the optional squared-ReLU MLP.
``DABSNSequenceLM`` keeps the reference LM's constructor and state-dict layout around a
stack of blocks (model.py:381-436, 804-860); the reference's graph machinery is not part of
this backend.
"""

from __future__ import annotations

import os
from dataclasses import dataclass
from typing import Mapping

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor
from torch.utils.checkpoint import checkpoint

from .core import DABSNCore
from .kernels import ops, pipeline
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
    """One core plus admitted/permanent/induction/long read (seq, field or hybrid
    geometry)."""

    def __init__(self, input_dim: int, hidden_dim: int, state_dim: int, read_geometry: str = "seq",
                 *, residual: bool = False, mlp_ratio: float | None = None,
                 block_chunk_t: int | None = None) -> None:
        super().__init__()
        self.input_dim, self.hidden_dim, self.state_dim = input_dim, hidden_dim, state_dim
        self.read_geometry = read_geometry
        self.core = DABSNCore(input_dim=input_dim, hidden_dim=state_dim)
        self.read = DABSNRead(hidden_dim=state_dim, read_geometry=read_geometry)
        self.read_gain = nn.Parameter(torch.full((1,), 0.01))
        # Present (and unused by the forward) for field blocks, as in the reference
        # (model.py:145-147), so state dicts stay interchangeable.
        self.field_read_gain = (nn.Parameter(torch.full((1,), 1.0)) if read_geometry == "field"
                                else None)
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
        chunk_t = self._resolve_block_chunk_t(inputs)
        scan_dtype = (torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda")
                      else inputs.dtype)
        if self.training and pipeline.enabled() and pipeline.pipeline_applies(
                self.read, inputs, chunk_t, state=self.state_dim, dtype=scan_dtype):
            # Training on the device with block chunking: the read of query chunk k runs
            # beside the scan of chunk k + 1 on the other half of the device.
            Wx, Wgx = self.core.projections(inputs)
            y, _, read = pipeline.pipelined_scan_read(self.read, chunk_t, Wx, Wgx,
                                                      self.core.scan_inputs())
        else:
            trajectory, novelty, plasticity, expression, write, energy, saturation = (
                self.core_tapes(inputs))
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
        if not torch.is_grad_enabled() and ops._same_dtype(hidden, self.mlp_norm.weight):
            # Inference on the device: the norm and the squared ReLU as one kernel each.
            normed = ops.rms_norm(hidden, self.mlp_norm.weight, self.mlp_norm.eps)
            return hidden + self.mlp_fc2(ops.relu_square(self.mlp_fc1(normed)))
        return hidden + self.mlp_fc2(F.relu(self.mlp_fc1(self.mlp_norm(hidden))).square())

    def forward(self, inputs: Tensor) -> Tensor:
        return self.forward_mlp(self.forward_world(inputs))


@dataclass(frozen=True)
class DABSNLayerSpec:
    """Width and read geometry of one block (reference config.py:34-58)."""

    hidden_dim: int
    state_dim: int | None = None
    read_geometry: str = "seq"

    def __post_init__(self) -> None:
        if int(self.hidden_dim) <= 0:
            raise ValueError("hidden_dim must be positive")
        if self.state_dim is not None and int(self.state_dim) <= 0:
            raise ValueError("state_dim must be positive")
        if self.read_geometry not in {"seq", "field", "hybrid"}:
            raise ValueError("read_geometry must be seq, field, or hybrid")

    @property
    def resolved_state_dim(self) -> int:
        return int(self.hidden_dim if self.state_dim is None else self.state_dim)

    def to_metadata(self) -> dict[str, object]:
        return {"hidden_dim": int(self.hidden_dim),
                "state_dim": None if self.state_dim is None else int(self.state_dim),
                "read_geometry": self.read_geometry}


def parse_layer_specs(spec) -> list[DABSNLayerSpec]:
    """Layer specs from the reference's compact form ``geometry:hidden[:state]`` (comma or
    semicolon separated), from mappings with ``hidden_dim``/``state_dim``/``read_geometry``
    (or ``hidden``/``state``/``geometry``), from ``DABSNLayerSpec`` objects, or from
    ``(hidden, state)`` pairs (seq geometry). Mirrors config.py:61-116."""
    if spec is None:
        return []
    if isinstance(spec, str):
        out = []
        for part in (x.strip() for x in spec.replace(";", ",").split(",")):
            if not part:
                continue
            fields = [f.strip() for f in part.split(":")]
            if len(fields) not in (2, 3):
                raise ValueError(f"compact DABSN layer specs must be geometry:hidden[:state], "
                                 f"got {part!r}")
            state = int(fields[2]) if len(fields) == 3 and fields[2] else None
            out.append(DABSNLayerSpec(int(fields[1]), state, fields[0]))
        return out
    out = []
    for item in spec:
        if isinstance(item, DABSNLayerSpec):
            out.append(item)
        elif isinstance(item, Mapping):
            hidden = item.get("hidden", item.get("hidden_dim"))
            if hidden is None:
                raise ValueError(f"DABSN layer spec missing hidden/hidden_dim: {item!r}")
            state = item.get("state", item.get("state_dim"))
            geometry = str(item.get("geometry", item.get("read_geometry", "seq")))
            out.append(DABSNLayerSpec(int(hidden), None if state is None else int(state), geometry))
        elif isinstance(item, (tuple, list)) and len(item) == 2:
            out.append(DABSNLayerSpec(int(item[0]), int(item[1]), "seq"))
        else:
            raise ValueError(f"unsupported DABSN layer spec entry {item!r}")
    return out


class DABSNBackbone(nn.Module):
    """The stack of blocks (reference model.py:381-436 for seq blocks without middle MLPs):
    each block's world view followed by its inline MLP."""

    def __init__(self, input_dim: int, layers, *, residual: bool = False,
                 mlp_ratio: float | None = None, block_chunk_t: int | None = None) -> None:
        super().__init__()
        self.input_dim = int(input_dim)
        self.layer_specs = parse_layer_specs(layers)
        if not self.layer_specs:
            raise ValueError("DABSN needs at least one layer spec")
        blocks = []
        width = self.input_dim
        for spec in self.layer_specs:
            blocks.append(DABSNBlock(width, spec.hidden_dim, spec.resolved_state_dim,
                                     spec.read_geometry, residual=residual, mlp_ratio=mlp_ratio,
                                     block_chunk_t=block_chunk_t))
            width = spec.hidden_dim
        self.blocks = nn.ModuleList(blocks)
        self.output_dim = width

    def forward(self, inputs: Tensor) -> Tensor:
        h = inputs
        for block in self.blocks:
            h = block(h)
        return h


class DABSNSequenceLM(nn.Module):
    """Token embedding -> seq DABSN blocks -> readout.

    Same constructor, attributes and state-dict layout (``embed``, ``backbone.blocks.<k>``,
    ``readout``) as the reference's ``DABSNSequenceLM`` (model.py:804-860), so its weights
    and carried-memory files are interchangeable. ``layers`` takes the reference's layer
    specs (e.g. ``"seq:2048:2048,seq:2048:2048"``); without it, ``depth`` blocks of
    ``hidden_dim`` (state ``state_dim``) are built. Only the seq read geometry is built
    here; the field/hybrid geometries and the middle MLP stack are outside this backend.
    """

    is_dabsn_sequence_lm = True

    def __init__(self, vocab: int, hidden_dim: int, depth: int = 1, layer_geometries=None, *,
                 layers=None, state_dim: int | None = None, tie_embeddings: bool = False,
                 grad_checkpoint: bool = False, residual: bool = False,
                 mlp_ratio: float | None = None, mlp_middle_depth: int = 0,
                 mlp_depth_index: int = 0, block_chunk_t: int | None = None) -> None:
        super().__init__()
        del grad_checkpoint  # block time-chunking (block_chunk_t) is this backend's checkpoint
        if int(mlp_middle_depth) != 0:
            raise NotImplementedError("middle MLP stacks are outside the ROCm scan+read backend")
        self.vocab = int(vocab)
        self.hidden_dim = int(hidden_dim)
        self.state_dim = None if state_dim is None else int(state_dim)
        self.tie_embeddings = bool(tie_embeddings)
        self.residual = bool(residual)
        self.mlp_ratio = None if mlp_ratio is None else float(mlp_ratio)
        self.mlp_middle_depth = int(mlp_middle_depth)
        self.mlp_depth_index = int(mlp_depth_index)
        specs = parse_layer_specs(layers)
        if not specs:
            geoms = layer_geometries or "seq"
            if isinstance(geoms, str):
                geoms = [g for g in geoms.replace(",", " ").split() if g]
            specs = [DABSNLayerSpec(self.hidden_dim, self.state_dim, geoms[i % len(geoms)])
                     for i in range(int(depth))]
        self.layers = specs
        self.depth = len(specs)
        self.layer_geometries = [s.read_geometry for s in specs]
        self.embed = nn.Embedding(self.vocab, self.hidden_dim)
        self.backbone = DABSNBackbone(self.hidden_dim, specs, residual=self.residual,
                                      mlp_ratio=self.mlp_ratio, block_chunk_t=block_chunk_t)
        self.readout = nn.Linear(self.backbone.output_dim, self.vocab)
        if self.tie_embeddings and self.backbone.output_dim == self.hidden_dim:
            self.readout.weight = self.embed.weight
        nn.init.normal_(self.embed.weight, mean=0.0, std=0.02)
        nn.init.zeros_(self.readout.bias)

    @property
    def blocks(self) -> nn.ModuleList:
        return self.backbone.blocks

    def forward_hidden(self, ids: Tensor) -> Tensor:
        return self.backbone(self.embed(ids))

    def forward(self, ids: Tensor) -> Tensor:
        return self.readout(self.forward_hidden(ids))
