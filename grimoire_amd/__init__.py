"""grimoire_amd -- MI355X (gfx950) mixture-of-experts layer for GRIMOIRE.

The compute path is libgrimoire_moe.so (hand-written HIP kernels behind the
C ABI of include/grimoire_moe.h).  This package holds its ctypes binding,
the host-side weight descriptors and synthetic workloads, and the Python
mirror of the reference's launchers.
"""
from . import _abi
from ._abi import GrimoireError, lib

__all__ = ["GrimoireError", "lib", "_abi"]
