"""MI355X-native QStore quantized-weight hot path (gfx950 HIP kernels behind a C ABI).

Import name: ``mrun_pub_amd`` (the directory name is not a Python identifier; the repo
root's ``__graft_entry__.load_package()`` registers it).  Every device operation is one
call into ``libqstore_hip.so``; there is no CPU fallback.  Submodules:

* ``_native``      -- ctypes binding of ``libqstore_hip.so`` (signatures equal to
  ``include/qstore_hip.h``); raises when the library is missing.
* ``build``        -- compiles ``csrc/`` for gfx950 into ``libqstore_hip.so``.
* ``qrow``         -- int8 row-scaled linears: dequant, W8A16 / fp32 GEMV, batched decode,
  paired SwiGLU, multi-linear launches, fused head + top-2 and its fp32 rerank.
* ``store``        -- the QStore v3 on-disk format: reader, writer, layout validation.
* ``provenance``   -- semantic identity and file digests of a sealed store.
* ``dense_store``  -- ``DenseQStore``: compact-page LRU or one fully resident HBM arena.
* ``paged``        -- ``PagedQStore``: pinned host tier (whole store, or bounded staging
  buffers) and the successor-prefetch ring over the ``qs_pager`` slot ring.
* ``lowbit``       -- int3 / int2 pages and ``DeviceLowbitQStore``.
* ``codecs``       -- the offline int8 / int3 / int2 row codecs on the device.
* ``w8a8``         -- W8A8 linear: activation quantizer, outlier protection, int8 GEMM,
  the ``enable_w8a8`` hook.
* ``moe``          -- router, stable route compile, grouped int8 / weight-only GEMMs,
  stable reduce, ``Int8ExpertBackend``.
* ``expert_queue`` -- expert-major packet queues and their committed scatter.
* ``expert_cache`` -- paged int8 experts: page store, pinned host tier, HBM slot cache
  (eviction policies, transient prefill, page trace).
* ``ops``          -- ``torch.library`` custom ops (``torch.ops.qstore_hip.*``) with fake
  kernels.
"""

from __future__ import annotations

__all__ = ["codecs", "dense_store", "expert_cache", "expert_queue", "lowbit", "moe", "ops", "paged",
           "provenance", "qrow", "store", "w8a8"]
