"""flintnsteel_amd - MI355X (gfx950) native MoE FFN hot path of FlintNSteel.

The compute lives in libfns_hip.so (hand-written HIP in csrc/, C ABI in include/fns_hip.h, C++ API in
include/fns/*.h). This package only loads it and passes torch device memory and streams to it.
"""
from ._lib import FnsError, lib  # noqa: F401

__all__ = ["FnsError", "lib"]
