"""Regenerate the bridge known-answer fixture (run once; output is committed).

The reference's only stored numeric answer for the curvature path is the
"Hidden Bridge" experiment of test.ipynb: a 100-node stochastic block model
(two 50-node communities, intra-probability 0.9, no inter edges, seed 42),
intra edge weights ``clip(N(1, 0.1), 0.1, 2.0)`` drawn with numpy seed 42 in
edge order, and a bridge (0, 99) of weight 0.001 (test.ipynb:64-96). Its
stored output (test.ipynb:19-25) is the bridge curvature -85.71 and the
bridge retrieval flags of the magnitude (H2O) and curvature (CAB) masks at
six sparsities.

This script rebuilds the weighted adjacency with this repository's own code
(networkx 3.4.2, numpy 2.2) and writes:

- ``bridge_sbm_adj.npy``: float32 [100, 100] adjacency (the input vector);
- ``bridge_kat.json``: the reference's stored outputs, transcribed from
  test.ipynb:19-25 (they are data, not recomputed here).
"""

import json
import pathlib

import networkx as nx
import numpy as np

HERE = pathlib.Path(__file__).resolve().parent

# Stored outputs of test.ipynb (cell 0 output, lines 19-25 of the raw JSON).
REFERENCE_OUTPUT = {
    "bridge": [0, 99],
    "bridge_weight": 0.001,
    "bridge_frc_2dp": -85.71,
    "sparsities": [0.5, 0.8, 0.9, 0.95, 0.98, 0.99],
    "h2o_found": [True, False, False, False, False, False],
    "cab_found": [True, True, True, True, True, True],
    "source": "test.ipynb:19-25",
}


def build_adjacency() -> np.ndarray:
    np.random.seed(42)
    graph = nx.stochastic_block_model([50, 50], [[0.9, 0.0], [0.0, 0.9]], seed=42)
    adj = np.zeros((100, 100), dtype=np.float32)
    for u, v in graph.edges():
        w = np.float32(np.clip(np.random.normal(1.0, 0.1), 0.1, 2.0))
        adj[u, v] = w
        adj[v, u] = w
    adj[0, 99] = adj[99, 0] = np.float32(0.001)
    return adj


def main() -> None:
    adj = build_adjacency()
    np.save(HERE / "bridge_sbm_adj.npy", adj)
    (HERE / "bridge_kat.json").write_text(json.dumps(REFERENCE_OUTPUT, indent=1) + "\n")
    print("edges:", int((adj > 0).sum()) // 2)


if __name__ == "__main__":
    main()
