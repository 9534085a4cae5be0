"""prichs_amd -- MI355X (gfx950) MoE feed-forward hot path of PRICHS.

The computation lives in libprichs_hip.so (prichs_amd/csrc, C ABI in
include/prichs_hip.h).  Python modules:

* ``_lib``  -- ctypes declarations of the C ABI (no torch needed);
* ``ops``   -- stage entry points on torch device tensors;
* ``moe``   -- ``MoEEngine`` and the host-side mirror of the reference's
  ``MoELayer`` / ``Expert`` interface;
* ``synth`` -- the seeded synthetic input generator of the benchmark configs;
* ``build`` -- compiles the library in-tree with hipcc for gfx950.
"""
__version__ = "0.1.0"
