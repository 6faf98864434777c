"""dotcompute_amd — the MI355X (gfx950) HIP backend of DotCompute.

Layout:
  csrc/   hand-written HIP kernels for gfx950 + the C-ABI library (libdotcompute_hip.so)
  host/   C++ host layer mirroring the reference API (orchestrator, LINQ provider, algorithms)
  hip.py  ctypes binding of the C ABI (tests, bench)
  build.py offline build (hipcc for gfx950, g++ for the host layer)
"""
from . import hip  # noqa: F401

__all__ = ["hip"]
