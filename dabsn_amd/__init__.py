"""dabsn_amd: MI355X (gfx950) backend for DABSN's recurrent hot path.

The package registers the ``dabsn::`` operators of the core scan, the three-way read,
the long-memory scan and the read glue with hand-written HIP kernels
(``dabsn_amd/csrc``, C ABI in ``include/dabsn_hip.h``), and mirrors the reference's
``DABSNCore`` / ``DABSNRead`` / seq ``DABSNBlock`` on top of them, with the carried
memory (``ingest`` / ``forward_with_memory``) that streams a model over context and decodes
token by token against a bank that grows in place.
"""

from . import kernels
from .core import DABSNCore
from .events import (
    EventCode,
    StrictFallbackError,
    add_event_listener,
    remove_event_listener,
    strict_events,
)
from .loss import chunked_cross_entropy_from_logits, chunked_linear_cross_entropy
from .memory import DABSNMemory, LayerMemory, forward_with_memory, ingest
from .model import DABSNBlock, DABSNSequenceLM
from .read import DABSNRead

__all__ = [
    "DABSNBlock",
    "DABSNCore",
    "DABSNMemory",
    "DABSNRead",
    "DABSNSequenceLM",
    "EventCode",
    "StrictFallbackError",
    "LayerMemory",
    "chunked_cross_entropy_from_logits",
    "chunked_linear_cross_entropy",
    "add_event_listener",
    "forward_with_memory",
    "ingest",
    "kernels",
    "remove_event_listener",
    "strict_events",
]
