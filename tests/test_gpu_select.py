"""Column abs-max and top-k channel selection on the GPU against the oracle
(lrq_colmax / lrq_topk; the channel split of config 3).  Ties, k = 1 and k = hidden, and
both column abs-max kernels (16-byte rows and the 4-byte fallback) are covered."""

import numpy as np
import pytest
import torch

import oracle as O
from parity import bits16

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("hidden,k,levels", [
    (4096, 41, 0),       # config 3: distinct values
    (4096, 41, 6),       # heavy ties: six distinct values
    (5000, 1, 3),
    (5000, 5000, 0),     # k = hidden
    (1000, 999, 2),
    (37000, 1024, 50),   # near the LDS limit, many ties
])
def test_topk_matches_oracle(pkg, dev, hidden, k, levels):
    print(f"[topk] hidden={hidden} k={k} levels={levels}", flush=True)
    g = torch.Generator().manual_seed(hidden + k)
    if levels:
        cm = torch.randint(0, levels, (hidden,), generator=g).to(torch.float32) * 0.25
    else:
        cm = torch.rand(hidden, generator=g, dtype=torch.float32) * 3.0
    idx = pkg.topk_channels(cm.to(dev), k)
    torch.cuda.synchronize()
    ref = O.topk_channels(cm.numpy(), k)
    assert np.array_equal(idx.cpu().numpy(), ref)


@pytest.mark.parametrize("rows,hidden", [(129, 2048), (37, 1030), (1000, 4096)])
def test_colmax_matches_oracle(pkg, dev, rows, hidden):
    print(f"[colmax] rows={rows} hidden={hidden}", flush=True)
    x = pkg.inputs.activation(rows, hidden, n_outlier=3, outlier_scale=30.0, seed=rows)
    cm = pkg.column_absmax(x.to(dev))
    torch.cuda.synchronize()
    ref = O.colmax_abs(bits16(x))
    assert np.array_equal(cm.cpu().numpy().view(np.uint32), ref.view(np.uint32))
