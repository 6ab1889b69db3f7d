"""Routing and fallback events (reference contract: src/dabsn/events.py:12-86,
runtime/dispatch.py:40-101).

CPU: the event bus itself -- selections announced once per shape, fallback events carry
the four fields, strict mode raises on every occurrence, listeners come and go.
GPU: the product emits them -- a block's forward announces the core scan, the read and
the long scan; a batch too large for one cooperative launch reports the batch-slab
fallback, chunked or not; a streaming read of a bank it
cannot read in place reports the switch to the general read; strict mode turns each of
them into an error.
"""

from __future__ import annotations

import pytest
import torch

import dabsn_amd
from dabsn_amd import events
from dabsn_amd.events import EventCode


@pytest.fixture()
def seen():
    got: list = []
    events.reset_routing_log()
    events.add_event_listener(got.append)
    yield got
    events.remove_event_listener(got.append)
    events.reset_routing_log()


def test_selection_announced_once_per_shape(seen):
    events.announce("core_scan", "rocm", B=2, T=3)
    events.announce("core_scan", "rocm", B=2, T=3)
    events.announce("core_scan", "rocm", B=2, T=4)
    assert [e.code for e in seen] == [EventCode.KERNEL_SELECTION] * 2
    assert seen[0].component_id == "core_scan" and seen[0].fields["selected_path"] == "rocm"
    with pytest.raises(TypeError):
        seen[0].fields["B"] = 5  # read-only mapping


def test_fallback_fields_required_and_strict_raises_every_time(seen):
    with pytest.raises(ValueError, match="reason"):
        events.emit_event(EventCode.PERFORMANCE_FALLBACK, fallback=True, requested_path="a",
                          selected_path="b", corrective_action="c")
    kw = dict(requested_path="fast", selected_path="slow", corrective_action="fix it")
    events.report_fallback("read", "too wide", **kw, H=3)
    events.report_fallback("read", "too wide", **kw, H=3)
    assert len(seen) == 1 and seen[0].fallback
    assert {"reason", "requested_path", "selected_path", "corrective_action"} <= set(seen[0].fields)
    with events.strict_events():
        assert events.strict_mode()
        for _ in range(2):  # already announced, but strict mode still refuses it
            with pytest.raises(events.StrictFallbackError, match="too wide"):
                events.report_fallback("read", "too wide", **kw, H=3)
        with events.strict_events(False):
            events.report_fallback("read", "too wide", **kw, H=3)
    assert not events.strict_mode()
    assert len(seen) == 1


def test_reference_names_and_defaults(seen):
    events.log_routing_once("long", "rocm", T=5)
    events.warn_routing_once("long", "no kernel")
    sel, fb = seen
    assert sel.code is EventCode.KERNEL_SELECTION and fb.code is EventCode.PERFORMANCE_FALLBACK
    assert fb.fields["requested_path"] == "optimized" and fb.fields["selected_path"] == "reference"
    assert fb.fields["corrective_action"]
    assert EventCode("DABSN_PERFORMANCE_FALLBACK") is EventCode.PERFORMANCE_FALLBACK


def test_listener_removed_hears_nothing(seen):
    other: list = []
    events.add_event_listener(other.append)
    events.add_event_listener(other.append)  # registering twice keeps one entry
    events.announce("x", "y")
    events.remove_event_listener(other.append)
    events.announce("x", "z")
    assert len(other) == 1 and len(seen) == 2


@pytest.mark.gpu
def test_block_forward_announces_its_kernels(cuda_device, seen):
    torch.manual_seed(0)
    blk = dabsn_amd.DABSNBlock(16, 24, 24, "seq").to(cuda_device)
    blk(torch.randn(2, 12, 16, device=cuda_device)).sum().backward()
    names = {(e.component_id, e.fields["selected_path"]) for e in seen
             if e.code is EventCode.KERNEL_SELECTION}
    assert ("core_scan", "rocm_cooperative_scan") in names
    assert ("core_scan", "rocm_cooperative_reverse_scan") in names
    assert ("admitted_three_way_read", "rocm_compact_admitted_bank") in names
    assert ("recurrent_long_read", "rocm_chunk_parallel_scan") in names
    assert not any(e.fallback for e in seen)


def _big_batch(cuda_device):
    from helpers import core_case

    from dabsn_amd.kernels.chunked import chunked_core_scan

    B, T, H = 40, 24, 2048
    x = [t.to(cuda_device) for t in core_case(5, B, T, H)]
    x[0], x[1] = x[0].to(torch.bfloat16), x[1].to(torch.bfloat16)
    x[0].requires_grad_(True)
    out = chunked_core_scan(8, *x)
    return out, x


@pytest.mark.gpu
def test_batch_slabs_are_reported(cuda_device, seen):
    """B = 40 at H = 2048 in bf16 needs two cooperative launches (slabs) per chunk, forward
    and reverse (test_gpu_ops covers the values)."""
    out, x = _big_batch(cuda_device)
    out[0].float().sum().backward()
    fb = {e.component_id for e in seen if e.fallback}
    assert "core_scan" in fb
    with events.strict_events():
        with pytest.raises(events.StrictFallbackError, match="cooperative launch"):
            _big_batch(cuda_device)


@pytest.mark.gpu
def test_streaming_read_fallbacks_are_reported(cuda_device, seen):
    """Decode-sized inference reads: a state width that is not a multiple of 8 leaves the
    in-place bank read; two query rows leave the one-pass read."""
    from dabsn_amd import memory as mem

    for width, step in ((20, 1), (24, 2)):
        torch.manual_seed(1)
        model = dabsn_amd.DABSNSequenceLM(30, 16, 1, layers=f"seq:16:{width}").to(cuda_device).eval()
        ids = torch.randint(0, 30, (2, 10), device=cuda_device)
        memory = mem.ingest(model, ids[:, :8])
        mem.forward_with_memory(model, ids[:, 8:8 + step], memory)
        with events.strict_events(), pytest.raises(events.StrictFallbackError):
            mem.forward_with_memory(model, ids[:, 8:8 + step], memory)
    reasons = [e.fields["reason"] for e in seen if e.fallback]
    assert any("in place" in r for r in reasons) and any("one query row" in r for r in reasons)
