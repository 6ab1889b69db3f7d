"""Chunked readout + cross-entropy loss (reference: src/dabsn/runtime/loss.py).

The readout logits [N, V] of a language-model step are its largest activation. The loss
walks the N rows in chunks of at most ``budget // V`` rows: each chunk's logits come from
one readout GEMM (hipBLASLt through ``F.linear``), and one HIP row kernel
(``ops.ce_rows``) reduces them to the row's logsumexp and masked NLL in fp32, reading the
logits once in their own dtype instead of an fp32 copy plus logsumexp / gather kernels.
The backward recomputes each chunk's logits, forms (softmax - onehot) * scale in one row
kernel (``ops.ce_rows_backward``, reusing the forward's logsumexp), and runs the two
gradient GEMMs in fp32 as the reference does (loss.py:95-137).

Same API, defaults and environment switch as the reference: ``DABSN_LOSS_CHUNK_SCORES``
sets the element budget (default 2**24), ``off`` forces ``F.cross_entropy`` on the full
logits. Inputs must be device tensors (fp32 or bf16); the loss is fp32.
"""

from __future__ import annotations

import os

import torch
import torch.nn.functional as F
from torch import Tensor

from .kernels import ops

_DEFAULT_CHUNK_BUDGET = 1 << 24


def _accum_dtype(dtype: torch.dtype) -> torch.dtype:
    """At least fp32 (loss.py:42-50)."""
    return torch.promote_types(dtype, torch.float32)


def _chunk_rows(num_rows: int, vocab: int, budget: int | None = None) -> int:
    """Rows per chunk so that rows * V stays within the element budget (loss.py:31-39)."""
    if budget is None:
        budget = int(os.environ.get("DABSN_LOSS_CHUNK_SCORES", str(_DEFAULT_CHUNK_BUDGET)))
    if budget <= 0:
        return num_rows
    return min(max(1, budget // max(1, vocab)), num_rows)


def _budget(chunk_budget: int | None) -> tuple[bool, int | None, int]:
    """(forced exact path, explicit budget, effective budget) from the argument and env."""
    env = os.environ.get("DABSN_LOSS_CHUNK_SCORES", "")
    if env.lower() == "off":
        return True, None, 0
    budget = chunk_budget
    if budget is None and env:
        try:
            budget = int(env)
        except ValueError:
            budget = None
    return False, budget, budget if budget is not None else _DEFAULT_CHUNK_BUDGET


def _spans(n: int, rows: int):
    return [(s, min(n, s + rows)) for s in range(0, n, rows)]


def _rows(parts: list[Tensor], like: Tensor) -> Tensor:
    if not parts:  # no rows: an empty fp32 vector
        return like.new_empty((0,), dtype=torch.float32)
    return parts[0] if len(parts) == 1 else torch.cat(parts)


class ChunkedLinearCrossEntropy(torch.autograd.Function):
    """Fused readout + mean cross-entropy that never holds more than [chunk, V] logits.
    Forward saves hidden, weight, bias, targets and the rows' logsumexp (N floats)."""

    @staticmethod
    def forward(ctx, hidden: Tensor, weight: Tensor, bias: Tensor | None, targets: Tensor,
                chunk_rows: int, ignore_index: int) -> Tensor:
        acc = _accum_dtype(hidden.dtype)
        n = int(hidden.shape[0])
        lses, nlls = [], []
        for s, e in _spans(n, chunk_rows):
            logits = F.linear(hidden[s:e], weight, bias)
            lse, nll = ops.ce_rows(logits, targets[s:e], ignore_index)
            lses.append(lse)
            nlls.append(nll)
        lse, nll = _rows(lses, hidden), _rows(nlls, hidden)
        denom = (targets != ignore_index).sum().to(acc).clamp_min(1.0)
        ctx.save_for_backward(hidden, weight, bias, targets, denom, lse)
        ctx.chunk_rows = int(chunk_rows)
        ctx.ignore_index = int(ignore_index)
        ctx.acc = acc
        return nll.to(acc).sum() / denom

    @staticmethod
    def backward(ctx, grad_output):
        hidden, weight, bias, targets, denom, lse = ctx.saved_tensors
        acc = ctx.acc
        scale = (grad_output / denom).to(torch.float32).reshape(1)
        weight_acc = weight.to(acc)
        grad_hidden = torch.empty_like(hidden)
        grad_weight = torch.zeros_like(weight, dtype=acc)
        grad_bias = torch.zeros_like(bias, dtype=acc) if bias is not None else None
        for s, e in _spans(int(hidden.shape[0]), ctx.chunk_rows):
            hid = hidden[s:e]
            logits = F.linear(hid, weight, bias)
            d = ops.ce_rows_backward(logits, targets[s:e], ctx.ignore_index, lse[s:e], scale)
            grad_hidden[s:e] = torch.mm(d, weight_acc).to(hidden.dtype)
            grad_weight.addmm_(d.t(), hid.to(acc))  # accumulated inside the GEMM
            if grad_bias is not None:
                grad_bias += d.sum(dim=0)
        grad_weight = grad_weight.to(weight.dtype)
        if grad_bias is not None:
            grad_bias = grad_bias.to(bias.dtype)
        return grad_hidden, grad_weight, grad_bias, None, None, None


class _CrossEntropyFromLogits(torch.autograd.Function):
    """Mean cross-entropy over materialised logits [N, V], chunked over rows."""

    @staticmethod
    def forward(ctx, logits: Tensor, targets: Tensor, chunk_rows: int, ignore_index: int):
        acc = _accum_dtype(logits.dtype)
        lses, nlls = [], []
        for s, e in _spans(int(logits.shape[0]), chunk_rows):
            lse, nll = ops.ce_rows(logits[s:e], targets[s:e], ignore_index)
            lses.append(lse)
            nlls.append(nll)
        lse, nll = _rows(lses, logits), _rows(nlls, logits)
        denom = (targets != ignore_index).sum().to(acc).clamp_min(1.0)
        ctx.save_for_backward(logits, targets, denom, lse)
        ctx.chunk_rows = int(chunk_rows)
        ctx.ignore_index = int(ignore_index)
        return nll.to(acc).sum() / denom

    @staticmethod
    def backward(ctx, grad_output):
        logits, targets, denom, lse = ctx.saved_tensors
        scale = (grad_output / denom).to(torch.float32).reshape(1)
        grad = torch.empty_like(logits)
        for s, e in _spans(int(logits.shape[0]), ctx.chunk_rows):
            d = ops.ce_rows_backward(logits[s:e], targets[s:e], ctx.ignore_index, lse[s:e], scale)
            grad[s:e] = d.to(logits.dtype)
        return grad, None, None, None


def chunked_linear_cross_entropy(hidden: Tensor, weight: Tensor, bias: Tensor | None,
                                 targets: Tensor, *, ignore_index: int = -100,
                                 chunk_budget: int | None = None) -> Tensor:
    """Mean next-token cross-entropy of ``F.linear(hidden, weight, bias)`` against
    ``targets`` (loss.py:140-183). ``hidden`` is [B, T, H] or [N, H]; ``targets`` matches
    without the H axis. Rows go in chunks of ``budget // V`` (one chunk when the full
    logits fit the budget); ``DABSN_LOSS_CHUNK_SCORES=off`` computes ``F.cross_entropy`` on
    the full logits instead."""
    hidden_flat = hidden.reshape(-1, hidden.shape[-1]) if hidden.dim() == 3 else hidden
    targets_flat = targets.reshape(-1)
    n_rows, vocab = int(hidden_flat.shape[0]), int(weight.shape[0])
    exact, budget, effective = _budget(chunk_budget)
    if exact:
        logits = F.linear(hidden_flat, weight, bias).to(_accum_dtype(hidden_flat.dtype))
        return F.cross_entropy(logits, targets_flat, ignore_index=ignore_index)
    rows = n_rows if n_rows * vocab <= effective else _chunk_rows(n_rows, vocab, budget)
    return ChunkedLinearCrossEntropy.apply(hidden_flat, weight, bias, targets_flat, max(rows, 1),
                                           ignore_index)


def chunked_cross_entropy_from_logits(logits: Tensor, targets: Tensor, *,
                                      ignore_index: int = -100,
                                      chunk_budget: int | None = None) -> Tensor:
    """Mean cross-entropy over already-materialised logits, chunked over rows
    (loss.py:186-231)."""
    logits_flat = logits.reshape(-1, logits.shape[-1])
    targets_flat = targets.reshape(-1)
    n_rows, vocab = (int(d) for d in logits_flat.shape)
    exact, budget, effective = _budget(chunk_budget)
    if exact:
        return F.cross_entropy(logits_flat.to(_accum_dtype(logits_flat.dtype)), targets_flat,
                               ignore_index=ignore_index)
    rows = n_rows if n_rows * vocab <= effective else _chunk_rows(n_rows, vocab, budget)
    return _CrossEntropyFromLogits.apply(logits_flat, targets_flat, max(rows, 1), ignore_index)
