"""MI355X-native QStore quantized-weight hot path (gfx950 HIP kernels behind a C ABI).

Import name: ``mrun_pub_amd`` (the directory name is not a Python identifier; the repo
root's ``__graft_entry__.load_package()`` registers it).  Submodules:

* ``qrow``   -- int8 row-scaled linears: dequant, W8A16 / fp32 GEMV, paired SwiGLU.
* ``_native`` -- ctypes binding of ``libqstore_hip.so``.
"""

from __future__ import annotations

__all__ = ["qrow"]
