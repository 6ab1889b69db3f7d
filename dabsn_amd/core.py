"""DABSN core recurrence module on the ROCm backend.

Parameter names, shapes and initialisation follow the reference module
(src/dabsn/core.py:18-109) so state dicts are interchangeable; the carried-state API
follows ``DABSNCore.forward_from_state`` (core.py:248-342). The scan itself is the
registered ``dabsn::core_scan_batched`` operator (HIP kernels, ``kernels/ops.py``).
"""

from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor

from .kernels import ops


def _parameter(shape: int | tuple[int, ...], value: float) -> nn.Parameter:
    if isinstance(shape, int):
        shape = (shape,)
    return nn.Parameter(torch.full(shape, float(value)))


VECTOR_NAMES = ("k_s", "k_y", "k_b", "k_n", "k_bias", "r_s", "r_y", "r_b", "r_n", "r_bias")


class DABSNCore(nn.Module):
    """Recurrent core with novelty modulation and retained saturation state."""

    _rocm_native_enabled = False

    def __init__(self, input_dim: int, hidden_dim: int, kappa_init: float = -2.25,
                 recover_init: float = -4.60, a_gain: float = 0.5) -> None:
        super().__init__()
        self.hidden_dim = hidden_dim
        self.a_gain = a_gain
        self.W = nn.Linear(input_dim, hidden_dim, bias=False)
        self.A = nn.Linear(hidden_dim, hidden_dim, bias=False)
        self.Wg = nn.Linear(input_dim, hidden_dim, bias=True)
        self.Ug = nn.Linear(hidden_dim, hidden_dim, bias=False)
        self.beta = _parameter(hidden_dim, 0.0)
        self.logit_alpha = _parameter(1, -2.0)
        self.log_lambda = _parameter(1, -1.0)
        self.log_kappa = _parameter(hidden_dim, kappa_init)
        self.logit_recover = _parameter(hidden_dim, recover_init)
        for name in VECTOR_NAMES:
            setattr(self, name, _parameter(hidden_dim, 0.0))
        self.logit_saturation_decay = _parameter(1, 2.2)
        self.k_saturation = _parameter(hidden_dim, 0.0)
        self.r_saturation = _parameter(hidden_dim, 0.0)
        self.logit_saturation_suppress = _parameter(1, -6.0)
        self.reset_parameters()

    def reset_parameters(self) -> None:
        for module in (self.W, self.A, self.Wg, self.Ug):
            nn.init.xavier_uniform_(module.weight)
            if module.bias is not None:
                nn.init.zeros_(module.bias)
        nn.init.orthogonal_(self.A.weight, gain=self.a_gain)
        nn.init.zeros_(self.beta)
        nn.init.constant_(self.Wg.bias, -2.0)

    def initial_state(self, batch_size: int, *, device=None,
                      dtype=None) -> tuple[Tensor, Tensor, Tensor]:
        reference = next(self.parameters())
        device = reference.device if device is None else device
        dtype = reference.dtype if dtype is None else dtype
        budget = torch.zeros(batch_size, self.hidden_dim, dtype=dtype, device=device)
        return budget, torch.ones_like(budget), torch.zeros_like(budget)

    def scan_inputs(self) -> tuple[Tensor, ...]:
        """The 21 parameter inputs of the registered op, in schema order."""
        return (
            self.Ug.weight, self.A.weight, self.beta, self.log_kappa, self.logit_recover,
            self.k_s, self.k_y, self.k_b, self.k_n, self.k_bias, self.r_s, self.r_y, self.r_b,
            self.r_n, self.r_bias, self.logit_saturation_decay.expand(self.hidden_dim),
            self.k_saturation, self.r_saturation, self.logit_alpha.reshape(()),
            self.log_lambda.reshape(()), self.logit_saturation_suppress.reshape(()),
        )

    def projections(self, inputs: Tensor) -> tuple[Tensor, Tensor]:
        """(W x, Wg x + b) (core.py:281-282) as one GEMM over the stacked weight [W; Wg]:
        the [B, T, 2H] result holds Wx and Wgx side by side, and the scan reads the two
        halves in place through its input row stride. Without autograd (inference) the
        stacked weight and bias are built once per parameter version."""
        H = self.hidden_dim

        def stack(w, wg, bg):
            return torch.cat((w, wg), dim=0), torch.cat((bg.new_zeros(H), bg), dim=0)

        params = (self.W.weight, self.Wg.weight, self.Wg.bias)
        if torch.is_grad_enabled():
            weight, bias = stack(*params)
        else:
            weight, bias = ops._derived("proj", params, stack)
        both = F.linear(inputs, weight, bias)
        Wx, Wgx = both.split(H, dim=-1)
        return Wx, Wgx

    def forward_from_state(self, inputs: Tensor, *, initial_state=None, return_writes: bool = False,
                           return_cocktail: bool = False, return_final_state: bool = False):
        if inputs.dim() != 3:
            raise ValueError("DABSNCore inputs must have shape [B,T,input_dim]")
        batch = inputs.shape[0]
        if initial_state is None:
            # The carried state stays fp32 (batched_runtime.py:1681-1694).
            zeros = torch.zeros(batch, self.hidden_dim, device=inputs.device, dtype=torch.float32)
            initial_state = (zeros, torch.ones_like(zeros), zeros.clone())
        else:
            expected = (batch, self.hidden_dim)
            values = tuple(v.to(device=inputs.device) for v in initial_state)
            if any(v.shape != expected for v in values):
                shapes = tuple(tuple(v.shape) for v in values)
                raise ValueError(f"initial_state tensors must have shape {expected}, got {shapes}")
            initial_state = values
        outputs = ops.direct.core_scan_batched(*self.projections(inputs), *self.scan_inputs(),
                                               *initial_state)
        self._last_core_backend = "rocm_native_hip"
        trajectory, novelty, plasticity, expression, write = outputs[:5]
        if return_cocktail:
            result = (trajectory, novelty, plasticity, expression, write, outputs[5], outputs[6])
        elif return_writes:
            result = (trajectory, novelty, plasticity, expression, write)
        else:
            result = (trajectory, novelty, plasticity)
        if return_final_state:
            return result, tuple(outputs[8:11])
        return result

    def chunked_tapes(self, inputs: Tensor, chunk_t: int):
        """Block time-chunked scan from the zero state (model.py:274-307): chunks of
        `chunk_t` steps with the state carried between them. On the device the tapes stay
        resident for the chunks' reverse scans instead of being recomputed per chunk (the
        reference's checkpoint trades that memory for a second forward scan). Returns the
        7 tapes of forward_from_state(..., return_cocktail=True)."""
        from .kernels.chunked import chunked_core_scan

        batch = inputs.shape[0]
        zeros = torch.zeros(batch, self.hidden_dim, device=inputs.device, dtype=torch.float32)
        outputs = chunked_core_scan(chunk_t, *self.projections(inputs), *self.scan_inputs(),
                                    zeros, torch.ones_like(zeros), zeros.clone())
        self._last_core_backend = "rocm_native_hip_chunked"
        return tuple(outputs[:7])

    def forward(self, inputs: Tensor, return_writes: bool = False, return_cocktail: bool = False):
        return self.forward_from_state(inputs, return_writes=return_writes,
                                       return_cocktail=return_cocktail)
