"""zealot_amd — zealot-rl's PPO learning hot path on AMD MI355X (gfx950).

The compute lives in libzealot_hip.so (C ABI, include/zealot_hip.h) and its
hipModuleLoad-ed gfx950 code object of hand-written HIP kernels. This package
is the host-side binding: `device` (context + buffers), `ops` (operator
entry points), `rl` (zealot-rl's Mlp/ActorCritic/update API on the device)
and `synth` (seeded synthetic workloads).
"""

from ._ffi import ZL_SEMANTICS_ACTOR_CRITIC, ZL_SEMANTICS_GPU_TRAINER, load_library  # noqa: F401
from .device import Context, DeviceBuffer, ZealotError  # noqa: F401

__all__ = [
    "Context",
    "DeviceBuffer",
    "ZealotError",
    "load_library",
    "ZL_SEMANTICS_ACTOR_CRITIC",
    "ZL_SEMANTICS_GPU_TRAINER",
]
