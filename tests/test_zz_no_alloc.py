"""cab_evict_select_noalloc (no workspace argument, built-in device scratch)
against cab_evict_select with a caller workspace, through the C ABI: kept
positions, counts and categories bit-identical, over consecutive calls whose
second input is smaller (the scratch keeps the first call's contents), for
the multi-workgroup path (>= 32768 positions) and the one-workgroup path."""

import numpy as np
import pytest
import torch

from cab_attention import _native as nat

pytestmark = pytest.mark.gpu


def _run(lib, cuda, scores, n, local, imp, bridge, mode, noalloc, bridge_scores=None):
    keep = torch.full((max(n, 1),), -7, dtype=torch.int64, device=cuda)
    counts = torch.full((4,), -7, dtype=torch.int32, device=cuda)
    cat = torch.full((max(n, 1),), 9, dtype=torch.uint8, device=cuda)
    sp = scores.data_ptr() if scores is not None else None
    ns = scores.numel() if scores is not None else 0
    bp = bridge_scores.data_ptr() if bridge_scores is not None else None
    stream = torch.cuda.current_stream(cuda).cuda_stream
    if noalloc:
        st = lib.cab_evict_select_noalloc(sp, ns, bp, n, local, imp, bridge, 1, mode,
                                          keep.data_ptr(), counts.data_ptr(), cat.data_ptr(),
                                          stream)
        nat.check("cab_evict_select_noalloc", st)
    else:
        wb = int(lib.cab_evict_select_workspace_bytes(n))
        ws = torch.empty(max(wb, 256), dtype=torch.uint8, device=cuda)
        st = lib.cab_evict_select(sp, ns, bp, n, local, imp, bridge, 1, mode, keep.data_ptr(),
                                  counts.data_ptr(), cat.data_ptr(), ws.data_ptr(), ws.numel(),
                                  stream)
        nat.check("cab_evict_select", st)
    torch.cuda.synchronize()
    c = counts.cpu().numpy()
    return keep.cpu().numpy()[:c[3]], c, cat.cpu().numpy()[:n]


@pytest.mark.parametrize("sizes", [(300000, 50000), (65536, 40000), (40000, 1000)])
@pytest.mark.parametrize("mode", [1, 2, 3])
def test_noalloc_matches_workspace_entry(cuda, sizes, mode):
    lib = nat.load()
    for n in sizes:
        print(f"noalloc n={n} mode={mode}", flush=True)
        g = torch.Generator(device=cuda).manual_seed(n + mode)
        scores = torch.randn(n, generator=g, device=cuda)
        scores[::7] = 0.5  # ties across segments
        bs = torch.rand(n, generator=g, device=cuda) if mode == 2 else None
        local, imp, br = n // 10, n // 4, n // 6
        want = _run(lib, cuda, scores, n, local, imp, br, mode, False, bs)
        got = _run(lib, cuda, scores, n, local, imp, br, mode, True, bs)
        np.testing.assert_array_equal(got[1], want[1])
        np.testing.assert_array_equal(got[0], want[0])
        np.testing.assert_array_equal(got[2], want[2])
        assert want[1][3] == local + want[1][1] + want[1][2]


def test_noalloc_rejects_caches_beyond_the_scratch(cuda):
    lib = nat.load()
    n = (1 << 20) + 1
    keep = torch.empty(8, dtype=torch.int64, device=cuda)
    counts = torch.empty(4, dtype=torch.int32, device=cuda)
    st = lib.cab_evict_select_noalloc(None, 0, None, n, 0, 0, 0, 1, 0, keep.data_ptr(),
                                      counts.data_ptr(), None,
                                      torch.cuda.current_stream(cuda).cuda_stream)
    assert st == nat.CAB_ESHAPE
    assert b"scratch" in lib.cab_last_error()
