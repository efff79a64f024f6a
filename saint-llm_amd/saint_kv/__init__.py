"""saint_kv — MI355X (gfx950) heterogeneous KV cache.

A drop-in for the KV-cache classes of saint-llm's ``packages/inference``
(``SWAKVCacheLayer``, ``HCAKVCacheLayer``, ``CSAKVCacheLayer``,
``KVCacheBundle``; kv_cache.py:32-427) backed by paged storage and hand-written
HIP kernels reached through the C ABI in ``include/saintkv.h``.
"""

from saint_kv import ops

__all__ = ["ops"]
__version__ = "0.1.0"
