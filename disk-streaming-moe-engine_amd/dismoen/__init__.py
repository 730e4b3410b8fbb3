"""dismoen: MI355X (gfx950) MoE FFN block of the disk-streaming MoE engine.

The compute lives in libdismoen_hip.so (C ABI: include/dismoen_hip.h); this
package is the host-side binding that mirrors the reference's layer API.
"""
from ._lib import DismoenError, LIB_PATH, lib  # noqa: F401
from .layers import MoEBlock, RouterConfig, RoutingInfo  # noqa: F401
from . import formats, gguf, synth  # noqa: F401
