"""MI355X (gfx950) per-layer ops of the provider-local GGUF engine.

    cuca_amd.hip       ctypes binding of include/cuca_hip.h (libcuca_hip.so)
    cuca_amd.ops       the reference's op surface over that binding
    cuca_amd.build     builds the code object and libcuca_hip.so in-tree
    cuca_amd.workloads the five workload shapes and their seeded inputs
"""

__all__ = ["hip", "ops", "build", "workloads"]
