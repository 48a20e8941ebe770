"""Importance and token-FRC tracking for KV-cache eviction (reference: cab_attention/scoring/)."""

from .frc import FRCTracker
from .importance import ImportanceTracker

__all__ = ["ImportanceTracker", "FRCTracker"]
