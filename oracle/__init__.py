"""CPU oracle for the compressed-activation path — TEST INFRASTRUCTURE ONLY.

This package is a plain numpy restatement of the reference's PyTorch formulation
of the encode / decode / fused-backward path, plus the new per-group quantiser,
projection, Walsh-Hadamard rotation and outlier-channel split that the build's
compressed format adds.  It is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The product path (the ``triton-kernel-test_amd`` package) never
imports or calls anything here and raises when its HIP library is missing.

Every function cites the reference file:line it restates.  Functions whose
numerics no reference test or golden vector fixes are pinned by closed forms and
invariants in ``tests/test_oracle.py``; see the "pinned by" line of each
docstring.
"""

from .lrq_oracle import *  # noqa: F401,F403
