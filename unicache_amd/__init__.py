"""UniCache physical KV-cache engine for AMD Instinct MI355X (gfx950).

``unicache_amd.storage`` and ``unicache_amd.operators`` mirror UniCache's
``unicache.storage`` / ``unicache.operators`` physical-cache API; the tensor
work runs in the HIP kernels of ``libunicache_hip.so`` (C ABI in
``include/unicache_hip.h``), loaded through ``unicache_amd._native``.
"""

__version__ = "0.1.0"
