"""hawking_amd -- MI355X (gfx950) quantized decode hot path of hawking-core.

Packed matvec organs (uniform Q4, binary sign planes, mixed <=1.5 BPW), the
device routers and the MoE expert step, as hand-written HIP kernels behind
the C ABI of include/hawking_hip.h.  The Python modules are thin mirrors of
the reference's organ / router / MoE API over that ABI.
"""
from ._lib import HK_BIN, HK_F32, HK_MIXED, HK_Q4, HawkingError  # noqa: F401
from .runtime import Context, DeviceArray, Event  # noqa: F401
