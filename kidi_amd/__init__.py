"""kidi_amd — MI355X (gfx950) native quantized linear layer for Kidi's PACKED_LINEAR operator.

The compute path is ``lib/libkq_hip.so`` (hand-written HIP kernels behind the C ABI in ``include/kq.h``).
``ops`` mirrors Kidi's ``ops::Context`` packed-linear entry points over that library.
"""

from . import _native
from .ops import Context, DeviceWeight, Failure, PackedWeight

__all__ = ["Context", "DeviceWeight", "Failure", "PackedWeight", "_native"]
