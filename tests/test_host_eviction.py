"""Host-side logic of the eviction layer, on the CPU: the counts the Python
layer derives from the budgets alone (it slices the kernel's outputs with
them and never reads the device) must be the counts the selection produces;
the eviction configuration validates its ratios."""

import itertools

import numpy as np
import pytest

from oracle import cab_oracle as O
from cab_attention.eviction import EvictionConfig
from cab_attention.eviction._select import (BRIDGE_MEDIAN, BRIDGE_NONE, BRIDGE_POSITIONAL,
                                            BRIDGE_SCORES, planned_counts)


@pytest.mark.parametrize("mode", [BRIDGE_NONE, BRIDGE_MEDIAN, BRIDGE_SCORES, BRIDGE_POSITIONAL])
def test_planned_counts_match_the_selection(mode):
    rng = np.random.default_rng(mode)
    for n, local, imp, br in itertools.product([1, 2, 7, 30, 100], [0, 1, 5, 30], [0, 3, 40, 200],
                                               [0, 2, 33, 150]):
        if local > n:
            continue
        for scores in (None, rng.standard_normal(n).astype(np.float32),
                       rng.standard_normal(max(1, n // 2)).astype(np.float32)):
            for fallback in (True, False):
                bs = rng.standard_normal(n).astype(np.float32) if mode == BRIDGE_SCORES else None
                want = O.evict_select(scores, n, local, imp, br, fallback, mode, bridge_scores=bs)[1]
                got = planned_counts(n, local, imp, br, scores is not None, fallback, mode)
                assert tuple(got) == tuple(want), (n, local, imp, br, scores is None, fallback)


def test_eviction_config_validates_ratios():
    """EvictionConfig rejects ratios that do not sum to 1 (policy.py:23-27)."""
    EvictionConfig(local_ratio=0.3, bridge_ratio=0.2, importance_ratio=0.5)
    with pytest.raises(ValueError):
        EvictionConfig(local_ratio=0.5, bridge_ratio=0.5, importance_ratio=0.5)
