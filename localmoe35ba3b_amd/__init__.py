"""MI355X-native quantized MoE-FFN hot path (W8A16 / W8A8 group-128 INT8).

Operators keep the call signatures of the reference operators
(qwen35_deploy/operators and qwen35_deploy/runtime of heliosz616/LocalMoe35Ba3b)
and run hand-written gfx950 HIP kernels through the C ABI declared in
include/localmoe35ba3b.h.
"""
from . import _lib  # noqa: F401

__all__ = ['operators', 'runtime', 'convert', 'router']
__version__ = '0.3.0'
