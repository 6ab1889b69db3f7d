"""Structured events of the ROCm backend: which kernel path a call runs, and every time a
call leaves its fast path.

What callers bind to is the reference's observability contract (src/dabsn/events.py:12-86,
src/dabsn/runtime/dispatch.py:40-101): the event codes and their string values; a fallback
event names ``reason``, ``requested_path``, ``selected_path`` and ``corrective_action``;
inside ``strict_events()`` a fallback raises ``StrictFallbackError``; listeners are
callables that receive each event (with ``code``, ``component_id``, ``fields`` and
``fallback``).

How it is built here:

* events are immutable records; the listener set is a tuple swapped under a lock when it
  changes, so publishing takes no lock;
* the strict flag is a ``contextvars.ContextVar``: it follows the caller's context, so a
  ``strict_events()`` block applies to its own thread or asyncio task only;
* ``announce`` and ``report_fallback`` are the routing helpers the package calls. Listeners
  and the ``dabsn_amd.routing`` logger hear about a given (component, decision, shape) once;
  a fallback still raises on every call under strict mode, not only the first time, since a
  requested fast path must never be left silently.
"""

from __future__ import annotations

import contextvars
import logging
import threading
from contextlib import contextmanager
from dataclasses import dataclass
from enum import Enum
from types import MappingProxyType
from typing import Callable, Iterator, Mapping

__all__ = [
    "EventCode",
    "Event",
    "StructuredEvent",
    "StrictFallbackError",
    "add_event_listener",
    "remove_event_listener",
    "strict_events",
    "strict_mode",
    "emit_event",
    "announce",
    "report_fallback",
    "log_routing_once",
    "warn_routing_once",
    "reset_routing_log",
]


class EventCode(str, Enum):
    """Event codes; the string values are the reference's (events.py:12-23)."""

    PROVIDER_RESOLUTION = "DABSN_PROVIDER_RESOLUTION"
    CONTRACT_VALIDATION = "DABSN_CONTRACT_VALIDATION"
    KERNEL_SELECTION = "DABSN_KERNEL_SELECTION"
    GRAPH_BREAK = "DABSN_GRAPH_BREAK"
    COMPILE_RESULT = "DABSN_COMPILE_RESULT"
    CAPTURE_RESULT = "DABSN_CAPTURE_RESULT"
    DTYPE_CHANGE = "DABSN_DTYPE_CHANGE"
    DISTRIBUTED_PLACEMENT = "DABSN_DISTRIBUTED_PLACEMENT"
    CHECKPOINT_TRANSACTION = "DABSN_CHECKPOINT_TRANSACTION"
    ROUTING_BALANCE = "DABSN_ROUTING_BALANCE"
    PERFORMANCE_FALLBACK = "DABSN_PERFORMANCE_FALLBACK"


FALLBACK_FIELDS = ("reason", "requested_path", "selected_path", "corrective_action")


@dataclass(frozen=True)
class Event:
    """One published event. ``fields`` is a read-only mapping."""

    code: EventCode
    component_id: str | None
    fields: Mapping[str, object]
    fallback: bool = False

    def describe(self) -> str:
        where = self.component_id or "<dabsn_amd>"
        if not self.fallback:
            return f"{self.code.value} [{where}] {dict(self.fields)}"
        f = self.fields
        return (f"{self.code.value} [{where}]: {f['reason']} -- ran {f['selected_path']} "
                f"instead of {f['requested_path']}; to fix: {f['corrective_action']}")


#: The reference's name for the event record.
StructuredEvent = Event


class StrictFallbackError(RuntimeError):
    """A call left its fast path while strict events were on."""


class _Bus:
    def __init__(self) -> None:
        self._lock = threading.Lock()
        self.listeners: tuple[Callable[[Event], None], ...] = ()
        self._seen: set[tuple] = set()

    def subscribe(self, fn: Callable[[Event], None]) -> None:
        with self._lock:
            if fn not in self.listeners:
                self.listeners = self.listeners + (fn,)

    def unsubscribe(self, fn: Callable[[Event], None]) -> None:
        with self._lock:
            # Equality, not identity: each access to a bound method builds a new object.
            self.listeners = tuple(x for x in self.listeners if x != fn)

    def first_time(self, key: tuple) -> bool:
        with self._lock:
            if key in self._seen:
                return False
            self._seen.add(key)
            return True

    def forget(self) -> None:
        with self._lock:
            self._seen.clear()


_BUS = _Bus()
_STRICT: contextvars.ContextVar[bool] = contextvars.ContextVar("dabsn_amd_strict_events",
                                                              default=False)
_LOG = logging.getLogger("dabsn_amd.routing")


def add_event_listener(listener: Callable[[Event], None]) -> None:
    _BUS.subscribe(listener)


def remove_event_listener(listener: Callable[[Event], None]) -> None:
    _BUS.unsubscribe(listener)


def strict_mode() -> bool:
    return _STRICT.get()


@contextmanager
def strict_events(enabled: bool = True) -> Iterator[None]:
    """Inside the block, a fallback raises ``StrictFallbackError``."""
    token = _STRICT.set(bool(enabled))
    try:
        yield
    finally:
        _STRICT.reset(token)


def emit_event(code: EventCode, *, component_id: str | None = None, fallback: bool = False,
               **fields: object) -> Event:
    """Publish one event to the listeners. A fallback event must carry the four fallback
    fields and raises under strict mode after the listeners have seen it."""
    if fallback:
        missing = [k for k in FALLBACK_FIELDS if k not in fields]
        if missing:
            raise ValueError(f"a fallback event needs the fields {missing}")
    event = Event(EventCode(code), component_id, MappingProxyType(dict(fields)), bool(fallback))
    for listener in _BUS.listeners:
        listener(event)
    if fallback and _STRICT.get():
        raise StrictFallbackError(event.describe())
    return event


def _key(kind: str, component: str, decision: str, fields: Mapping[str, object]) -> tuple:
    return (kind, component, decision, tuple(sorted((k, repr(v)) for k, v in fields.items())))


def announce(component: str, path: str, **shape: object) -> None:
    """``KERNEL_SELECTION`` for ``component`` running ``path``, once per distinct shape."""
    if _BUS.first_time(_key("select", component, path, shape)):
        emit_event(EventCode.KERNEL_SELECTION, component_id=component, selected_path=path, **shape)
        _LOG.info("dabsn_amd [%s] -> %s %s", component, path, shape)


def report_fallback(component: str, reason: str, *, requested_path: str, selected_path: str,
                    corrective_action: str, **shape: object) -> None:
    """``PERFORMANCE_FALLBACK``: listeners and the log hear about it once per distinct
    (component, reason, shape); under strict mode every occurrence raises."""
    if _BUS.first_time(_key("fallback", component, reason, shape)):
        _LOG.warning("dabsn_amd [%s]: %s -- ran %s instead of %s; to fix: %s %s", component,
                     reason, selected_path, requested_path, corrective_action, shape)
        emit_event(EventCode.PERFORMANCE_FALLBACK, component_id=component, fallback=True,
                   reason=reason, requested_path=requested_path, selected_path=selected_path,
                   corrective_action=corrective_action, **shape)
    elif _STRICT.get():
        raise StrictFallbackError(
            f"{EventCode.PERFORMANCE_FALLBACK.value} [{component}]: {reason} -- ran "
            f"{selected_path} instead of {requested_path}; to fix: {corrective_action}")


def log_routing_once(component: str, decision: str, **fields: object) -> None:
    """The reference's name (runtime/dispatch.py:40-60) for ``announce``."""
    announce(component, decision, **fields)


def warn_routing_once(component: str, message: str, **fields: object) -> None:
    """The reference's name (runtime/dispatch.py:63-101) for ``report_fallback``; the path
    and action fields default as they do there."""
    requested = str(fields.pop("requested_path", fields.pop("requested_backend", "optimized")))
    selected = str(fields.pop("selected_path", fields.pop("selected_backend", "reference")))
    action = str(fields.pop("corrective_action",
                            "inspect the capability report and select a supported backend "
                            "explicitly"))
    report_fallback(component, message, requested_path=requested, selected_path=selected,
                    corrective_action=action, **fields)


def reset_routing_log() -> None:
    """Forget which decisions were announced (tests)."""
    _BUS.forget()
