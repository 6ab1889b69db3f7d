"""Structured events and strict fallback semantics.

Mirrors the reference's observability contract (src/dabsn/events.py:12-86,
src/dabsn/runtime/dispatch.py:40-101): kernel selections are announced once per
(component, decision, shape); a fallback event must carry reason, requested_path,
selected_path and corrective_action, and raises ``StrictFallbackError`` inside
``strict_events()``.
"""

from __future__ import annotations

import logging
import os
import threading
from contextlib import contextmanager
from dataclasses import dataclass
from enum import Enum
from typing import Callable, Iterator, Mapping


class EventCode(str, Enum):
    KERNEL_SELECTION = "DABSN_KERNEL_SELECTION"
    PERFORMANCE_FALLBACK = "DABSN_PERFORMANCE_FALLBACK"
    DTYPE_CHANGE = "DABSN_DTYPE_CHANGE"


@dataclass(frozen=True)
class StructuredEvent:
    code: EventCode
    component_id: str | None
    fields: Mapping[str, object]
    fallback: bool = False


class StrictFallbackError(RuntimeError):
    pass


_state = threading.local()
_listeners: list[Callable[[StructuredEvent], None]] = []
_LOG = logging.getLogger("dabsn_amd.dispatch")
_SEEN: set = set()
_LOCK = threading.Lock()


def _strict() -> bool:
    return bool(getattr(_state, "strict", False))


def add_event_listener(listener: Callable[[StructuredEvent], None]) -> None:
    if listener not in _listeners:
        _listeners.append(listener)


def remove_event_listener(listener: Callable[[StructuredEvent], None]) -> None:
    if listener in _listeners:
        _listeners.remove(listener)


@contextmanager
def strict_events(enabled: bool = True) -> Iterator[None]:
    previous = _strict()
    _state.strict = bool(enabled)
    try:
        yield
    finally:
        _state.strict = previous


def emit_event(code: EventCode, *, component_id: str | None = None, fallback: bool = False,
               **fields: object) -> StructuredEvent:
    if fallback:
        missing = {"reason", "requested_path", "selected_path", "corrective_action"} - fields.keys()
        if missing:
            raise ValueError(f"fallback event is missing fields {sorted(missing)}")
    event = StructuredEvent(code, component_id, dict(fields), fallback)
    for listener in tuple(_listeners):
        listener(event)
    if fallback and _strict():
        raise StrictFallbackError(
            f"{code.value} strict fallback for {component_id or '<framework>'}: "
            f"{fields['reason']}; corrective action: {fields['corrective_action']}")
    return event


def _once(key: tuple) -> bool:
    with _LOCK:
        if key in _SEEN:
            return False
        _SEEN.add(key)
        return True


def log_routing_once(component: str, decision: str, **fields) -> None:
    """Announce a kernel selection once per (component, decision, shape)."""
    if _once(("route", component, decision, tuple(sorted(fields.items())))):
        emit_event(EventCode.KERNEL_SELECTION, component_id=component, selected_path=decision,
                   **fields)
        if os.environ.get("DABSN_SILENCE_ROUTING", "0") != "1":
            _LOG.info("DABSN routing [%s] -> %s  %s", component, decision,
                      "  ".join(f"{k}={v}" for k, v in fields.items()))


def warn_routing_once(component: str, message: str, **fields) -> None:
    """Announce (once) that a call left the requested fast path."""
    if _once(("warn", component, message, tuple(sorted(fields.items())))):
        f = dict(fields)
        requested = str(f.pop("requested_path", "rocm_native"))
        selected = str(f.pop("selected_path", "none"))
        action = str(f.pop("corrective_action", "select a supported configuration explicitly"))
        emit_event(EventCode.PERFORMANCE_FALLBACK, component_id=component, fallback=True,
                   reason=message, requested_path=requested, selected_path=selected,
                   corrective_action=action, **f)
        if os.environ.get("DABSN_SILENCE_ROUTING", "0") != "1":
            _LOG.warning("DABSN routing WARNING [%s]: %s", component, message)


def reset_routing_log() -> None:
    with _LOCK:
        _SEEN.clear()


__all__ = [
    "EventCode",
    "StrictFallbackError",
    "StructuredEvent",
    "add_event_listener",
    "emit_event",
    "log_routing_once",
    "remove_event_listener",
    "reset_routing_log",
    "strict_events",
    "warn_routing_once",
]
