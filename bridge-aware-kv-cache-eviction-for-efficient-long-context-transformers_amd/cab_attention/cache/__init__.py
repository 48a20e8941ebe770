"""KV caches with eviction (reference: cab_attention/cache/)."""

from .cab_cache import CABCache, CABCacheConfig
from .h2o_cache import H2OCache
from .prune import gather_positions, prune_layers

__all__ = ["CABCache", "CABCacheConfig", "H2OCache", "gather_positions", "prune_layers"]
