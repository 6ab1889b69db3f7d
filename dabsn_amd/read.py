"""DABSN read (admitted short memory, permanent associative memory, successor induction,
recurrent long memory) on the ROCm backend.

Parameter names and initial values follow the reference (src/dabsn/read.py:42-113).
``_unified_forward`` follows read.py:139-438 in all three geometries (seq: causal prefix;
field: the whole sequence; hybrid: both, mixed by a learned gate) and
``forward_query_bank`` follows read.py:650-838 (seq only, as there). The heavy pieces run as registered HIP
operators: tape statistics and query normalisation, admitted-slot selection, bank
gather, the three-way read and the fused long-memory scan. The [B,T]-sized glue
(key bias, admission, cocktail, their parameter gradients) stays in torch.
"""

from __future__ import annotations

import contextlib
import os

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor

from . import events
from .kernels import ops


def _parameter(value: float) -> nn.Parameter:
    return nn.Parameter(torch.full((1,), float(value)))


class _AdmittedReadParameters(nn.Module):
    """Parameters shared by the three-way admitted read (read.py:42-72)."""

    def __init__(self, hidden_dim: int) -> None:
        super().__init__()
        self.log_temp = _parameter(0.0)
        self.p_gain = _parameter(1.0)
        self.novelty_gain = _parameter(0.5)
        self.null_bias = _parameter(-2.0)
        self.out = nn.Linear(hidden_dim * 3, hidden_dim)
        self.adm_p_gain = _parameter(1.0)
        self.adm_novelty_gain = _parameter(0.5)
        self.adm_saturation_gain = _parameter(0.5)
        self.adm_energy_gain = _parameter(0.25)
        self.adm_bias = _parameter(-2.0)

    def admission_from_means(self, mean_e, mean_c, mean_n, mean_p, hidden: int) -> Tensor:
        return (self.adm_p_gain * torch.log1p(mean_p * hidden) + self.adm_novelty_gain * mean_n
                + self.adm_saturation_gain * mean_c + self.adm_energy_gain * mean_e + self.adm_bias)

    def project(self, y: Tensor, budget: Tensor, retrieved: Tensor) -> Tensor:
        """out(cat([y, budget, retrieved], -1)) (read.py:435, 821) without materialising the
        [.., 3H] concatenation: each column block of the weight multiplies its own input
        and the products accumulate through addmm."""
        h = y.shape[-1]
        lead = y.shape[:-1]
        w = self.out.weight
        r2 = retrieved.reshape(-1, h)
        if not torch.is_grad_enabled() and _side_by_side(y, budget):
            # Inference on the core's trajectory: y and budget are its two halves, so
            # [y, budget] is one [.., 2H] view and its block of the weight one product.
            yb = torch.as_strided(y, (*lead, 2 * h), y.stride(), y.storage_offset())
            out = F.linear(yb.reshape(-1, 2 * h), w[:, :2 * h], self.out.bias)
            out = torch.addmm(out, r2, w[:, 2 * h:].t())
            return out.reshape(*lead, out.shape[-1])
        y2, b2 = (x.reshape(-1, h) for x in (y, budget))
        out = F.linear(r2, w[:, 2 * h:], self.out.bias)
        out = torch.addmm(out, y2, w[:, :h].t())
        out = torch.addmm(out, b2, w[:, h:2 * h].t())
        return out.reshape(*lead, out.shape[-1])

    def key_bias_from_means(self, mean_n, mean_p, hidden: int) -> Tensor:
        return (self.p_gain * torch.log1p(mean_p * hidden) + self.novelty_gain * mean_n
                + self.null_bias)


def _side_by_side(a: Tensor, b: Tensor) -> bool:
    """b starts right after a's last element along the unit-stride last dim, with a's
    shape and strides: [a, b] is one view of twice the width."""
    return (a.shape == b.shape and a.stride() == b.stride() and a.dim() > 0
            and a.stride(-1) == 1 and a.dtype == b.dtype and a.device == b.device
            and b.data_ptr() == a.data_ptr() + a.shape[-1] * a.element_size())


def _cocktail(mean_e, mean_c, mean_n, mean_p) -> Tensor:
    return F.normalize(torch.stack([mean_e, mean_c, mean_n, mean_p], dim=-1), dim=-1)


def _tape_means(stats: Tensor, energy: Tensor, saturation: Tensor, novelty: Tensor,
                plasticity: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """The four means of a ``read_tape_stats`` row, each in its tape's dtype.

    The reference takes ``x.mean(dim=-1)`` of the tapes (read.py:58-72, 161-183), which
    returns the tape dtype: with bf16 tapes the key bias, admission, cocktail and the
    admission floor are evaluated from bf16-rounded means, in bf16 arithmetic wherever type
    promotion keeps them there. The stats kernel sums in fp32; rounding its means to the
    tape dtype gives the reference's values, so slot selection sees the same admission.
    """
    means = stats.unbind(-1)[:4]
    return tuple(m.to(t.dtype) for m, t in zip(means, (energy, saturation, novelty, plasticity)))


class _ArrayGlue:
    """Read glue held as arrays over the bank positions (key bias, admission, cocktail) plus
    the query cocktails, gathered per admitted slot with torch (read.py:241-256). Used on
    the CPU and by the inference paths that build the arrays in one kernel or keep them per
    bank position."""

    def __init__(self, key_bias: Tensor, admission: Tensor, bank_cocktail: Tensor,
                 query_cocktail: Tensor) -> None:
        self.kb, self.adm, self.cb, self.ck = key_bias, admission, bank_cocktail, query_cocktail

    def admission_for_select(self) -> Tensor:
        return self.adm

    def slots(self, idx: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor]:
        """(bank cocktail [B, N, 4], key bias [B, N], admission [B, N], query cocktail)."""
        return (torch.gather(self.cb, 1, idx.unsqueeze(-1).expand(-1, -1, 4)),
                torch.gather(self.kb, 1, idx), torch.gather(self.adm, 1, idx), self.ck)


class _StatsGlue:
    """Read glue evaluated from statistics rows on the device: the admission of every bank
    position for the selection (``ops.means_glue``, no gradient; the same values as the torch
    expressions, so the same slots), then per admitted slot its key bias, admission and
    cocktail and the query cocktails in one differentiable kernel (``ops.slot_glue``) instead
    of some forty small tensor operations and their backward."""

    def __init__(self, read: "DABSNRead", query_stats: Tensor, bank_stats: Tensor,
                 tape_dtype: torch.dtype, hidden: int) -> None:
        rp = read.short_read
        self.params = (rp.p_gain, rp.novelty_gain, rp.null_bias, rp.adm_p_gain,
                       rp.adm_novelty_gain, rp.adm_saturation_gain, rp.adm_energy_gain,
                       rp.adm_bias)
        self.qs, self.bs, self.dtype, self.hidden = query_stats, bank_stats, tape_dtype, hidden

    def admission_for_select(self) -> Tensor:
        _, adm, _ = ops.means_glue(self.bs.detach(), self.hidden, [p.detach() for p in self.params],
                                   self.dtype)
        if ops.glue_mode(self.dtype, self.params) == 3:
            adm = adm.to(torch.bfloat16)  # the reference's admission is a bf16 tensor here
        return adm

    def slots(self, idx: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor]:
        kb, adm, cb, ck = ops.slot_glue(self.bs, self.qs, idx, self.hidden, self.params,
                                        self.dtype)
        return cb, kb, adm, ck


class DABSNRead(nn.Module):
    """The canonical DABSN memory read: ``seq`` (causal prefix), ``field`` (the whole
    sequence) or ``hybrid`` (both, mixed by ``sigmoid(hybrid_gate)``)."""

    _rocm_native_enabled = False

    def __init__(self, hidden_dim: int, read_geometry: str = "seq") -> None:
        super().__init__()
        if read_geometry not in {"seq", "field", "hybrid"}:
            raise ValueError(f"read_geometry must be seq, field, or hybrid; got {read_geometry}")
        self.hidden_dim = hidden_dim
        self.read_geometry = read_geometry
        self.last_hybrid_gate: float | None = None
        self.last_seq_norm: float | None = None
        self.last_field_norm: float | None = None
        self.last_field_neighbors: float | None = None
        self.collect_traces = os.environ.get("DABSN_COLLECT_TRACES", "0") == "1"
        self.hybrid_gate_override: float | None = None
        self.last_n_max: int | None = None
        self.last_read_contract: dict[str, object] = {}
        self.pad_gain = _parameter(1.0)
        self.short_gain = _parameter(1.0)
        self.induct_gain = _parameter(0.1)
        self.cocktail_gain = _parameter(1.0)
        if read_geometry == "hybrid":
            self.hybrid_gate = _parameter(0.0)
        self.admit_window = _parameter(4.0)
        self.short_read = _AdmittedReadParameters(hidden_dim)
        self.logit_retain = _parameter(2.2)
        self.long_gain = _parameter(0.1)
        self.logit_expect_retain = _parameter(2.2)
        self.logit_retention_decay = _parameter(2.2)
        self.logit_retention_strength = _parameter(1.4)
        # Optional static bank width (read.py:224-231): a capture-safe, sync-free width.
        self._capture_bank_width: int | None = None
        # Work to enqueue while the host waits for the bank width (during_width_read).
        self._width_wait_work = None

    @contextlib.contextmanager
    def during_width_read(self, work):
        """Run ``work()`` (device work on the current stream, enqueued by the host) while the
        next read's host read of the bank width is in flight: the read copies the width into
        pinned memory, calls ``work``, and only then waits, so the device has ``work`` to run
        while the host waits and then enqueues the read's remaining kernels. If no such read
        happens inside the block (a fixed width, or no GPU), ``work`` runs at its end."""
        self._width_wait_work = work
        try:
            yield
        except BaseException:
            self._width_wait_work = None
            raise
        pending, self._width_wait_work = self._width_wait_work, None
        if pending is not None:
            pending()

    def _host_values(self, values: Tensor) -> list:
        """``values.tolist()`` for a small device tensor, running the pending
        ``during_width_read`` work between the copy and the wait."""
        work, self._width_wait_work = self._width_wait_work, None
        if work is None:
            return values.tolist()
        host = torch.empty(values.shape, dtype=values.dtype, pin_memory=True)
        host.copy_(values, non_blocking=True)
        copied = torch.cuda.Event()
        copied.record(torch.cuda.current_stream(values.device))
        work()
        copied.synchronize()
        return host.tolist()

    # ---- selection ------------------------------------------------------------
    def _select(self, admission: Tensor, length: int, width: int | None = None,
                want_fold: bool = False, query_start: int = 0):
        """Slot selection: (n_max, idx, valid, next_idx, rank, fold, read_idx). ``fold`` is
        the successor-fold code array [B, n_max] when ``want_fold`` and every admitted slot's
        next position is a bank row (``ops.bank_fold``), else None; the check rides on the
        host sync of the bank width. ``read_idx`` = idx - query_start. On the device the
        width and fold flag come back in one read and the slot arrays in one launch, so
        little is left to enqueue after the sync."""
        window = F.softplus(self.admit_window)
        # seq: floor from the causal prefix max; field / hybrid: the whole sequence's max
        # (read.py:185-191)
        whole = 0 if self.read_geometry == "seq" else 1
        order, counts, rank = ops.direct.bank_select(admission.detach(), window.detach(), whole)
        fold = None
        fixed = width or self._capture_bank_width
        if order.is_cuda:
            if fixed:
                # A fixed width needs no host sync; slots past a row's admitted count are
                # masked out by `valid`.
                n_max, bad = max(1, min(int(fixed), length)), True
            else:
                # One host read, as read.py:233, that also carries the device's deferred
                # kernel error word.
                width = ops.bank_width(order, counts, want_fold)
                word = ops.pending_error_word(order.device)
                vals = self._host_values(width if word is None else torch.cat((width, word)))
                top, bad = vals[:2]
                if len(vals) > 2:
                    ops.raise_error_word(int(vals[2]), order.device)
                n_max = max(int(top), 1)
            idx, valid, next_idx, read_idx, fold = ops.bank_slots(
                order, counts, n_max, query_start, want_fold and not bad)
            return n_max, idx, valid, next_idx, rank, fold, read_idx
        if fixed:
            # A fixed width needs no host sync; slots past a row's admitted count are
            # masked out by `valid`.
            n_max = max(1, min(int(width or self._capture_bank_width), length))
        elif want_fold:
            unfoldable = ops.bank_fold(order, counts)
            top, bad = torch.stack((counts.max(), unfoldable[0].to(counts.dtype))).tolist()
            n_max = max(int(top), 1)  # one host sync, as read.py:233
            if not bad:
                fold = ops.bank_fold(order, counts, n_max)
        else:
            n_max = max(int(counts.max().item()), 1)  # host sync, as read.py:233
        idx = order[:, :n_max]
        valid = torch.arange(n_max, device=admission.device).unsqueeze(0) < counts.clamp_min(1).unsqueeze(1)
        next_idx = (idx + 1).clamp(max=length - 1)
        read_idx = idx if query_start == 0 else idx - query_start
        return n_max, idx, valid, next_idx, rank, fold, read_idx

    def _bank(self, glue, length: int, query_start: int, width: int | None = None,
              members: tuple[Tensor, Tensor] | None = None) -> dict[str, object]:
        """Slot selection and the per-slot glue for the read (read.py:185-256, 298-303):
        n_max, idx, valid, next_idx, rank, the slots' cocktail, key bias and admission, the
        query cocktails, the read scale and the slot positions relative to the query chunk.
        ``glue``: an _ArrayGlue or _StatsGlue. ``members`` = (slot list [B, cap], counts
        [B]) kept incrementally by a carried bank (inference): the selection is read from it
        instead of rerun over the bank."""
        fold = None
        scale = self._scale()  # ahead of the selection's host sync
        if members is None:
            admission = glue.admission_for_select()
            # The successor fold serves the training read (gather + read under autograd).
            want_fold = torch.is_grad_enabled() and admission.is_cuda
            n_max, idx, valid, next_idx, rank, fold, read_idx = self._select(
                admission, length, width, want_fold, query_start)
        else:
            slots, counts = members
            if width or self._capture_bank_width:
                n_max = max(1, min(int(width or self._capture_bank_width), length))
            else:
                n_max = max(int(counts.max().item()), 1)  # host sync, as read.py:233
            idx = slots[:, :n_max]
            valid = (torch.arange(n_max, device=idx.device).unsqueeze(0)
                     < counts.clamp_min(1).unsqueeze(1))
            next_idx = (idx + 1).clamp(max=length - 1)
            rank = idx.new_empty((0,), dtype=torch.int32)  # the gather's backward only
            read_idx = idx if query_start == 0 else idx - query_start
        cb, kb, adm, ck = glue.slots(idx)
        return {
            "n_max": n_max, "idx": idx, "valid": valid, "next_idx": next_idx, "rank": rank,
            "fold": fold, "cocktail": cb, "key_bias": kb, "admission": adm,
            "query_cocktail": ck, "scale": scale, "read_idx": read_idx,
        }

    def _scale(self, fp32: bool = False) -> Tensor:
        """The read's score scale (softplus(log_temp) + 1) * sqrt(H) (read.py:240), in
        log_temp's dtype (``fp32``: then converted to an fp32 scalar); without autograd, a
        copy kept while log_temp is unchanged."""
        h = self.hidden_dim ** 0.5
        build = lambda t: (F.softplus(t) + 1.0) * h  # noqa: E731
        if torch.is_grad_enabled():
            return build(self.short_read.log_temp)
        if fp32:
            return ops._derived(f"read_scale_f32:{self.hidden_dim}", (self.short_read.log_temp,),
                                lambda t: build(t).float().reshape(()).contiguous())
        return ops._derived(f"read_scale:{self.hidden_dim}", (self.short_read.log_temp,), build)

    def _read_members(self, query: Tensor, store, length: int, width: int,
                      query_start: int) -> Tensor:
        """The one-row decode read with the slots taken from ``store``'s admitted-slot
        lists inside the kernel (``ops.read3_decode_members``): the streaming step's
        selection, glue gathers and read in three launches."""
        n_max = max(1, min(int(width), length))
        self.last_n_max = n_max
        hidden = int(query.shape[-1])
        dtype = "bf16" if query.dtype == torch.bfloat16 else "fp32"
        events.announce("admitted_three_way_read", "rocm_decode_bank_in_place",
                        B=int(query.shape[0]), T=1, H=hidden, dtype=dtype)
        retrieved = ops.read3_decode_members(
            query, store.write, store.stats, length, n_max, store.members, store.mcount,
            int(query_start), store.cocktail, store.key_bias, store.adm, self._scale(True),
            (self.short_gain, self.pad_gain, self.induct_gain, self.cocktail_gain))
        self.last_read_contract = self._contract(True, n_max, length, query, query_start)
        return retrieved

    def _contract(self, decode: bool, n_max: int, length: int, query: Tensor,
                  query_start: int) -> dict[str, object]:
        paths = 2 if self.read_geometry == "hybrid" else 1
        return {
            "read_strategy": "rocm_decode_bank_in_place" if decode else "rocm_compact_admitted_bank",
            "exact": True,
            "max_admitted_bank": int(n_max),
            "bank_growth": "grows_with_T" if n_max >= length else "data_dependent",
            "estimated_read_work": int(query.shape[0]) * int(query.shape[1]) * int(n_max) * 3
            * paths,
            "admission_policy": ("causal_write_prefix_max" if self.read_geometry == "seq"
                                 else "whole_sequence_max"),
            "kernel_backend": "rocm_hip_mfma",
            "query_start": int(query_start),
        }

    def _read_core(self, query, glue, bank_write, norm_w, length: int, query_start: int,
                   width: int | None = None, members: tuple[Tensor, Tensor] | None = None,
                   gather=None):
        """The read of ``query`` rows against the bank (glue: see ``_bank``). ``gather``
        (optional): called as gather(bank_write, norm_w, idx, next_idx, rank, fold) ->
        (K, V, Vn or None) in place of the bank gather op on the training path."""
        bank = self._bank(glue, length, query_start, width, members)
        n_max, idx, valid, next_idx, rank = (bank[k] for k in ("n_max", "idx", "valid",
                                                                "next_idx", "rank"))
        self.last_n_max = n_max
        bank_cocktail, bank_bias, bank_adm = bank["cocktail"], bank["key_bias"], bank["admission"]
        query_cocktail = bank["query_cocktail"]
        scale, read_idx = bank["scale"], bank["read_idx"]
        hidden = int(query.shape[-1])
        rows = int(query.shape[1])
        # A few query rows without autograd (streaming decode): read the bank in place
        # instead of gathering K, V, Vn copies of the admitted slots.
        streaming = (not torch.is_grad_enabled() and query.is_cuda and rows <= 8
                     and self.read_geometry == "seq")
        decode = (streaming and hidden % 8 == 0 and bank_write.stride(-1) == 1
                  and bank_write.stride(1) == hidden and bank_write.stride(0) % hidden == 0)
        dtype = "bf16" if query.dtype == torch.bfloat16 else "fp32"
        if streaming and not decode:
            events.report_fallback(
                "admitted_three_way_read",
                "the bank cannot be read in place (H not a multiple of 8, or its rows are "
                "not contiguous)",
                requested_path="in-place streaming read of the bank",
                selected_path="bank gather + three-way read",
                corrective_action="use a state width that is a multiple of 8 and a bank "
                                  "with contiguous rows",
                H=hidden, dtype=dtype)
        elif decode and (rows != 1 or hidden > 2048):
            events.report_fallback(
                "admitted_three_way_read",
                "the one-pass streaming read takes one query row with H <= 2048",
                requested_path="one-pass streaming read",
                selected_path="three-pass streaming read (scores, softmax rows, products)",
                corrective_action="decode one token per call, or use H <= 2048",
                rows=rows, H=hidden, dtype=dtype)
        if query.is_cuda:
            events.announce("admitted_three_way_read",
                            "rocm_decode_bank_in_place" if decode else "rocm_compact_admitted_bank",
                            B=int(query.shape[0]), T=rows, H=hidden, dtype=dtype)
        if decode:
            retrieved = ops.read3_decode(
                query, bank_write, norm_w, idx, next_idx, read_idx, valid, query_cocktail,
                bank_cocktail, bank_bias, bank_adm, scale,
                (self.short_gain, self.pad_gain, self.induct_gain, self.cocktail_gain))
        else:
            fold = bank["fold"]
            if gather is not None:
                K, V, Vn = gather(bank_write, norm_w, idx, next_idx, rank, fold)
            elif fold is not None:
                # Every admitted slot's successor row is a bank row (Vn[j] = V[j + fold[j]]):
                # the read folds the induction products into V and needs no successor rows.
                K, V = ops.bank_gather_kv(bank_write, norm_w, idx, rank)
                Vn = None
            else:
                K, V, Vn = ops.bank_gather(bank_write, norm_w, idx, next_idx, rank)

            def read(mode: int) -> Tensor:
                # mode 0: causal masks (seq); mode 1: every admitted slot for every query
                # (field), read.py:283-314
                return ops.admitted_three_way_read_train(
                    query, K, V, Vn, query_cocktail, bank_cocktail, bank_bias, bank_adm, scale,
                    read_idx, valid, mode, self.short_gain, self.pad_gain, self.induct_gain,
                    self.cocktail_gain, fold=fold)

            retrieved = self._geometry_mix(read, valid, query)
        self.last_read_contract = self._contract(decode, n_max, length, query, query_start)
        return retrieved

    def _require_seq(self) -> None:
        if self.read_geometry != "seq":
            raise RuntimeError("query-bank read is exact only for seq geometry")

    def _traces_on(self, query: Tensor) -> bool:
        """Host-side trace values (read.py:290-292): on CPU, or with DABSN_COLLECT_TRACES."""
        return not torch.compiler.is_compiling() and (self.collect_traces or not query.is_cuda)

    def _geometry_mix(self, read, valid: Tensor, query: Tensor) -> Tensor:
        """The read of this module's geometry from ``read(mode)`` (read.py:323-420): seq
        reads causally, field reads every admitted slot, hybrid mixes the two with
        ``gate = sigmoid(hybrid_gate)`` (or ``hybrid_gate_override``) as
        ``(1 - gate) * seq + gate * field``."""
        trace = self._traces_on(query)
        self.last_hybrid_gate = None
        self.last_field_neighbors = (float(valid.sum(dim=1).float().mean().cpu())
                                     if trace and self.read_geometry != "seq" else None)
        if self.read_geometry == "seq":
            retrieved = read(0)
            self.last_seq_norm = float(retrieved.detach().norm().cpu()) if trace else None
            self.last_field_norm = None
            return retrieved
        if self.read_geometry == "field":
            retrieved = read(1)
            self.last_seq_norm = None
            self.last_field_norm = float(retrieved.detach().norm().cpu()) if trace else None
            return retrieved
        seq_retrieved, field_retrieved = read(0), read(1)
        if self.hybrid_gate_override is None:
            gate = torch.sigmoid(self.hybrid_gate)
        else:
            gate = torch.as_tensor(float(self.hybrid_gate_override), device=query.device,
                                   dtype=query.dtype)
        self.last_hybrid_gate = float(gate.detach().cpu()) if trace else None
        seq_part = (1.0 - gate) * seq_retrieved
        field_part = gate * field_retrieved
        self.last_seq_norm = float(seq_part.detach().norm().cpu()) if trace else None
        self.last_field_norm = float(field_part.detach().norm().cpu()) if trace else None
        return seq_part + field_part

    # ---- forward ---------------------------------------------------------------
    def forward(self, y, budget, expression, write, novelty, plasticity, energy, saturation,
                field_shape=None) -> Tensor:
        del field_shape
        return self._unified_forward(y, budget, expression, write, novelty, plasticity, energy,
                                     saturation)

    def _glue(self, expression, write, novelty, plasticity, energy, saturation):
        """Per-position glue of the read (read.py:154-183): the tape statistics rows, the
        normalised query and the glue (key bias, admission, cocktail) of every position."""
        hidden = int(expression.shape[-1])
        stats = ops.direct.read_tape_stats(novelty, plasticity, energy, saturation, expression, write)
        query = ops.direct.normalize_rows(expression, stats[..., 4].detach())
        return stats, query, self._glue_from_stats(stats, stats, expression.dtype, hidden)

    def _unified_forward(self, y, budget, expression, write, novelty, plasticity, energy,
                         saturation) -> Tensor:
        rp = self.short_read
        seq_len = int(expression.shape[1])
        stats, query, glue = self._glue(expression, write, novelty, plasticity, energy, saturation)
        retrieved = self._read_core(query, glue, write, stats[..., 5].detach(), seq_len, 0)
        output = rp.project(y, budget, retrieved.to(y.dtype))
        long = self._long_scan(write, plasticity, novelty)
        return ops.direct.read_output(output, long, self.long_gain)

    # ---- long memory -------------------------------------------------------------
    def initial_long_scan_state(self, batch_size: int, hidden_dim: int | None = None, *,
                                device=None, dtype=None):
        hidden = int(hidden_dim or self.hidden_dim)
        device = self.logit_retain.device if device is None else device
        long = torch.zeros(batch_size, hidden, device=device, dtype=torch.float32)
        return long, torch.zeros_like(long), torch.ones_like(long)

    def _long_scan_from_state(self, write, plasticity, novelty, *, initial_state=None,
                              return_final_state: bool = False):
        del novelty  # unused by the long channel (long.py:501)
        batch, _, hidden = write.shape
        if initial_state is None:
            initial_state = self.initial_long_scan_state(batch, hidden, device=write.device)
        else:
            if any(s.shape != (batch, hidden) for s in initial_state):
                raise ValueError(f"initial long-scan state must have shape {(batch, hidden)}")
        if write.is_cuda:
            events.announce("recurrent_long_read", "rocm_chunk_parallel_scan", B=batch,
                            T=int(write.shape[1]), H=hidden,
                            dtype="bf16" if write.dtype == torch.bfloat16 else "fp32")
        long, lf, ef, rf, _ = ops.direct.long_scan_fused(
            write, plasticity, self.logit_expect_retain, self.logit_retention_decay,
            self.logit_retain, self.logit_retention_strength, *initial_state)
        if return_final_state:
            return long, (lf, ef, rf)
        return long

    def _long_scan(self, write, plasticity, novelty) -> Tensor:
        return self._long_scan_from_state(write, plasticity, novelty)

    # ---- external bank ---------------------------------------------------------
    def forward_query_bank(self, y, budget, expression, write, novelty, plasticity, energy,
                           saturation, *, bank_y=None, bank_b=None, bank_ay=None, bank_write,
                           bank_novelty, bank_p, bank_energy, bank_saturation, query_start: int,
                           initial_long_state=None, return_long_state: bool = False):
        """Exact read of a query chunk against an external bank (read.py:650-838)."""
        del bank_y, bank_b, bank_ay
        self._require_seq()
        rp = self.short_read
        _, _, hidden = expression.shape
        bank_len = bank_write.shape[1]
        if bank_len <= 0:
            raise RuntimeError("query-bank read requires a non-empty bank")
        q_stats = ops.direct.read_tape_stats(novelty, plasticity, energy, saturation, expression, write)
        b_stats = ops.direct.read_tape_stats(bank_novelty, bank_p, bank_energy, bank_saturation,
                                      bank_write, bank_write)
        query = ops.direct.normalize_rows(expression, q_stats[..., 4].detach())
        glue = self._glue_from_stats(q_stats, b_stats, bank_write.dtype, hidden)
        retrieved = self._read_core(query, glue, bank_write, b_stats[..., 5].detach(), bank_len,
                                    int(query_start))
        short_output = rp.project(y, budget, retrieved.to(y.dtype))
        result = self._long_scan_from_state(write, plasticity, novelty,
                                            initial_state=initial_long_state,
                                            return_final_state=return_long_state)
        if return_long_state:
            long, final_state = result
            return ops.direct.read_output(short_output, long, self.long_gain), final_state
        return ops.direct.read_output(short_output, result, self.long_gain)

    def forward_query_bank_stats(self, y, budget, expression, write, plasticity, *,
                                 query_stats, bank_write, bank_stats, query_start: int,
                                 initial_long_state=None, bank_width: int | None = None,
                                 bank_store=None, mix: tuple[Tensor, Tensor] | None = None):
        """forward_query_bank with the bank given as its write vectors plus per-position
        statistics instead of full-width tapes.

        The read uses the bank's novelty, plasticity, energy and saturation only through
        their means over H, and its writes through their row norms (read.py:58-72, 161-183).
        A carried bank therefore keeps, per position, the row of ``ops.read_tape_stats``
        computed when that position was a query: means of energy, saturation, novelty and
        plasticity, the query norm and the write norm ([B, N, 6] fp32). Those are the rows
        one dense pass computes for the same positions, so this is the dense read.
        ``query_stats`` are the rows of the query chunk itself (which the caller has
        already appended to the bank, ending at ``query_start + T``). ``bank_width`` fixes
        the slot-list width (no host sync for the admitted count). ``bank_store`` (a
        carried bank, inference on the device) keeps the glue and the admitted-slot list of
        every position it holds and extends them with the new positions only
        (``BankStore.admission``) instead of recomputing them over the bank. ``mix`` =
        (y, read_gain) returns the block's ``y + read_gain * output`` (model.py:336) in
        place of the output (one kernel without autograd).

        Returns (output, final long state)."""
        self._require_seq()
        rp = self.short_read
        _, _, hidden = expression.shape
        bank_len = bank_write.shape[1]
        if bank_len <= 0:
            raise RuntimeError("query-bank read requires a non-empty bank")
        query = ops.direct.normalize_rows(expression, query_stats[..., 4].detach())
        tape_dtype = bank_write.dtype
        members = None
        retrieved = None
        if bank_store is not None and not torch.is_grad_enabled() and bank_stats.is_cuda:
            key_bias, admission, bank_cocktail, members = bank_store.admission(
                self, hidden, tape_dtype, int(bank_len))
            rows = int(expression.shape[1])
            width = bank_width or self._capture_bank_width
            if (rows == 1 and width and hidden % 8 == 0 and hidden <= 2048
                    and query.dtype == bank_store.write.dtype):
                retrieved = self._read_members(query, bank_store, int(bank_len), int(width),
                                               int(query_start))
            glue = _ArrayGlue(key_bias, admission, bank_cocktail,
                              bank_cocktail[:, bank_len - rows:])
        elif not torch.is_grad_enabled() and bank_stats.is_cuda:
            # Inference (streaming decode): the per-position glue of the whole bank in one
            # kernel instead of ~25 small ones per layer and token.
            prm = (rp.p_gain, rp.novelty_gain, rp.null_bias, rp.adm_p_gain,
                   rp.adm_novelty_gain, rp.adm_saturation_gain, rp.adm_energy_gain, rp.adm_bias)
            key_bias, admission, bank_cocktail = ops.means_glue(bank_stats, hidden, prm, tape_dtype)
            if tape_dtype == torch.bfloat16 and rp.adm_bias.dtype == torch.bfloat16:
                # The reference's admission is a bf16 tensor here: its floor is bf16 too.
                admission = admission.to(torch.bfloat16)
            glue = _ArrayGlue(key_bias, admission, bank_cocktail,
                              ops.means_glue(query_stats, hidden, prm, tape_dtype)[2])
        else:
            glue = self._glue_from_stats(query_stats, bank_stats, tape_dtype, hidden)
        if retrieved is None:
            retrieved = self._read_core(query, glue, bank_write, bank_stats[..., 5].detach(),
                                        bank_len, int(query_start), bank_width, members)
        short_output = rp.project(y, budget, retrieved.to(y.dtype))
        long, final_state = self._long_scan_from_state(write, plasticity, None,
                                                       initial_state=initial_long_state,
                                                       return_final_state=True)
        if mix is None:
            return ops.direct.read_output(short_output, long, self.long_gain), final_state
        y_mix, gain = mix
        if not torch.is_grad_enabled() and ops._same_dtype(short_output, long, self.long_gain,
                                                           y_mix, gain):
            return ops.read_mix(short_output, long, self.long_gain, y_mix, gain), final_state
        read = ops.direct.read_output(short_output, long, self.long_gain)
        return y_mix + gain * read, final_state


    def _glue_from_stats(self, query_stats, bank_stats, tape_dtype, hidden: int):
        """The glue (key bias, admission, cocktails; read.py:58-72, 161-183) of the bank rows
        ``bank_stats`` and the query rows ``query_stats``, with the means in the tape dtype:
        evaluated by the device kernels on the GPU (_StatsGlue), by the torch expressions
        elsewhere (_ArrayGlue)."""
        if bank_stats.is_cuda and bank_stats.dtype == torch.float32:
            return _StatsGlue(self, query_stats, bank_stats, tape_dtype, hidden)
        rp = self.short_read
        qe, qc, qn, qp = (m.to(tape_dtype) for m in query_stats.unbind(-1)[:4])
        be, bc, bn, bp = (m.to(tape_dtype) for m in bank_stats.unbind(-1)[:4])
        key_bias = rp.key_bias_from_means(bn, bp, hidden)
        admission = rp.admission_from_means(be, bc, bn, bp, hidden)
        return _ArrayGlue(key_bias, admission, _cocktail(be, bc, bn, bp), _cocktail(qe, qc, qn, qp))

    def query_bank_retrieved(self, expression, *, query_stats, bank_write, bank_norms,
                             bank_stats, query_start: int, gather=None) -> Tensor:
        """The three-way read ``retrieved`` of a seq query chunk against the bank of positions
        [0, bank_stats.shape[1]) (forward_query_bank_stats before its output projection and
        long channel, read.py:650-823). ``bank_write`` [B, >= bank length, H] may be the
        whole write tape with the bank as its prefix; ``bank_norms`` are the write norms of
        its rows ([B, bank_write.shape[1]]). ``gather`` replaces the bank gather (see
        ``_read_core``)."""
        self._require_seq()
        hidden = int(expression.shape[-1])
        query = ops.direct.normalize_rows(expression, query_stats[..., 4].detach())
        glue = self._glue_from_stats(query_stats, bank_stats, bank_write.dtype, hidden)
        return self._read_core(query, glue, bank_write, bank_norms, int(bank_stats.shape[1]),
                               int(query_start), gather=gather)


def collect_traces_enabled() -> bool:
    return os.environ.get("DABSN_COLLECT_TRACES", "0") == "1"
