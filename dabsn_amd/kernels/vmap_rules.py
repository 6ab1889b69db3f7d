"""``torch.vmap`` rules for the ``dabsn::`` operators.

The reference registers a vmap rule on every public operator (batched_runtime.py:1639,
compact_flash.py:300, long.py:440, admitted.py:635, permanent.py:435, local_field.py:246),
each a Python loop that calls the operator once per vmapped index and stacks the results
(forward operators only, as there).

Here the common case runs as one launch instead: every one of these operators is already
batched over its leading dimension with per-row independence, and the parameters
(weights, gains, scale, patch tables) are shared. When the vmapped dimension touches only
row-batched arguments, it is folded into that leading dimension ([V, B, ...] ->
[V * B, ...]), the operator runs once on V * B rows -- a wider grid, which is what the
device wants -- and the results are unfolded. Rows are independent in every operator, so
each row's result is the one the per-index loop gives. When a shared argument is itself
vmapped (per-index weights), the rule falls back to the reference's loop.
"""

from __future__ import annotations

from typing import Sequence

import torch

from . import ops


def _pick(value, dim, index):
    if isinstance(value, (list, tuple)):
        dims = dim if isinstance(dim, (list, tuple)) else [dim] * len(value)
        return type(value)(_pick(v, d, index) for v, d in zip(value, dims))
    return value if dim is None else value.movedim(dim, 0)[index]


def _stack(outs):
    first = outs[0]
    if isinstance(first, (list, tuple)):
        stacked = [torch.stack([o[k] for o in outs]) for k in range(len(first))]
        return (type(first)(stacked) if isinstance(first, tuple) else stacked), \
            ([0] * len(first) if isinstance(first, list) else (0,) * len(first))
    return torch.stack(outs), 0


def _loop_rule(op):
    def rule(info, in_dims, *args):
        outs = [op(*(_pick(a, d, i) for a, d in zip(args, in_dims)))
                for i in range(info.batch_size)]
        return _stack(outs)

    return rule


def _fold_rule(op, rows: Sequence[int], out_row_dims: Sequence[int] | None = None):
    """Fold the vmapped dim into the leading (row) dim of the arguments in ``rows``; loop
    when any other argument is vmapped. ``out_row_dims`` gives each output's row dim
    (default 0)."""
    row_set = set(rows)
    loop = _loop_rule(op)

    def rule(info, in_dims, *args):
        if any(d is not None for i, d in enumerate(in_dims) if i not in row_set):
            return loop(info, in_dims, *args)
        V = info.batch_size
        new = list(args)
        lead = None
        for i in rows:
            a, d = args[i], in_dims[i]
            a = a.unsqueeze(0).expand(V, *a.shape) if d is None else a.movedim(d, 0)
            lead = a.shape[1]
            new[i] = a.reshape(V * a.shape[1], *a.shape[2:])
        out = op(*new)

        def unfold(o, r):
            return o.reshape(*o.shape[:r], V, lead, *o.shape[r + 1:])

        if isinstance(out, (tuple, list)):
            dims = tuple(out_row_dims) if out_row_dims else (0,) * len(out)
            return tuple(unfold(o, r) for o, r in zip(out, dims)), dims
        return unfold(out, 0), 0

    return rule


def register() -> None:
    fold = {
        ops.core_scan_batched: (0, 1, 23, 24, 25),
        ops.linear_recurrence: (0, 1, 2),
        ops.permanent_delta_scan: (0, 1, 2),
        ops.local_field_gather: (0,),
        ops.admitted_three_way_read_compact_flash: (0, 1, 2, 3, 4, 5, 6, 7, 9, 10),
        ops.admitted_three_way_read_native: (0, 1, 2, 3, 4, 5, 6, 7, 9, 10, 11, 12),
        ops.admitted_three_way_read: (0, 1, 2, 3, 4, 5, 6, 7, 9, 10, 11, 12),
        ops.long_scan_fused: (0, 1, 6, 7, 8),
    }
    out_rows = {ops.long_scan_fused: (0, 0, 0, 0, 0)}  # the checkpoint is [B, nseg, 3, H]
    for op, rows in fold.items():
        torch.library.register_vmap(op, _fold_rule(op, rows, out_rows.get(op)))


register()
