"""MI355X (gfx950) kernel backend for the Lancius graph path.

Native libraries (built in-tree by `python -m lancius_amd.build`):
  liblancius_hip.so    C ABI of the HIP kernels and the device executor
                       (include/lancius_hip.h, include/lancius_hip_graph.h)
  liblancius_graph.so  C graph IR / scheduler / planner (include/lancius_graph.h)
                       and the BASIS graph builders (include/lancius_basis.h)

This Python package only loads and wraps them; it computes nothing itself.
"""
from . import abi, prng
from .runtime import (ACT_GELU, ACT_NONE, ACT_RELU, ACT_TANH, DEVICE_GRAPH, DEVICE_KEEP_ALL, DEVICE_NO_CHAIN, DEVICE_NO_FUSION, DEVICE_NO_GROUP, Device,
                      DeviceProgram, HipError, device_count, graph_lib, hip_lib)

__all__ = [
    "abi", "prng", "Device", "DeviceProgram", "HipError", "device_count", "graph_lib", "hip_lib",
    "ACT_NONE", "ACT_RELU", "ACT_GELU", "ACT_TANH", "DEVICE_GRAPH", "DEVICE_NO_CHAIN", "DEVICE_NO_FUSION", "DEVICE_KEEP_ALL", "DEVICE_NO_GROUP",
]
