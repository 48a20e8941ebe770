"""Importance tracking for KV-cache eviction (reference: cab_attention/scoring/)."""

from .importance import ImportanceTracker

__all__ = ["ImportanceTracker"]
