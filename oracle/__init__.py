"""CPU oracle for the CAB-Attention block-sparse hot path.

TEST INFRASTRUCTURE ONLY. This package is a numpy (float64) restatement of
the reference algorithm. It is the checker the parity tests compare the HIP
kernels against, and the CPU baseline that ``bench.py`` times beside the GPU.
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import it. The shipped package never imports it and has no CPU path.

Pinning status of each function is listed in ``cab_oracle.__doc__``.
"""

from .cab_oracle import *  # noqa: F401,F403
