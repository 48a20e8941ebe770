"""KV-cache eviction selection (reference: cab_attention/eviction/)."""

from .h2o import h2o_select_indices
from .policy import EvictionConfig, ThreeComponentEvictionPolicy

__all__ = ["EvictionConfig", "ThreeComponentEvictionPolicy", "h2o_select_indices"]
