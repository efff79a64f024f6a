"""saint_kv — MI355X (gfx950) heterogeneous KV cache.

A drop-in for the KV-cache classes of saint-llm's ``packages/inference``
(``SWAKVCacheLayer``, ``HCAKVCacheLayer``, ``CSAKVCacheLayer``,
``KVCacheBundle``; kv_cache.py:32-427) backed by paged storage and hand-written
HIP kernels reached through the C ABI in ``include/saintkv.h``, plus the
ragged serving cache ``DecodeCache`` whose decode step runs as one fused
C-ABI call.
"""

from saint_kv import ops
from saint_kv.attention import cached_attention, decode_attention
from saint_kv.decode import CapturedSteps, DecodeCache, LayerSpec
from saint_kv.kv_cache import CSAKVCacheLayer, HCAKVCacheLayer, KVCacheBundle, SWAKVCacheLayer

__all__ = [
    "CSAKVCacheLayer",
    "CapturedSteps",
    "DecodeCache",
    "HCAKVCacheLayer",
    "KVCacheBundle",
    "LayerSpec",
    "SWAKVCacheLayer",
    "cached_attention",
    "decode_attention",
    "ops",
]
__version__ = "0.1.0"
