"""KV caches with eviction (reference: cab_attention/cache/): the CAB and H2O
caches on one device-resident store and eviction core (``store.py``)."""

from .cab_cache import CABCache, CABCacheConfig
from .h2o_cache import H2OCache
from .prune import gather_into, gather_positions, prune_layers
from .store import EvictingCache, LayeredKV

__all__ = ["CABCache", "CABCacheConfig", "H2OCache", "EvictingCache", "LayeredKV",
           "gather_into", "gather_positions", "prune_layers"]
