"""GPU against the committed golden fixtures (no oracle needed at run time)."""
import glob
import os

import numpy as np
import pytest

from hsdpa import workloads as W
from parity import assert_parity

from gpu_util import run_hsdpa

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "*.npz"))),
                         ids=lambda p: os.path.basename(p)[:-4])
def test_golden_on_gpu(torch_cuda, path):
    z = np.load(path, allow_pickle=False)
    h, kvh, d, rows, past, cap = (int(x) for x in z["geometry"])
    w = W.Workload(os.path.basename(path), h, kvh, d, rows, past, cap, z["q"], z["k"], z["v"], float(z["scale"]))
    print(f"golden {w.name}", flush=True)
    out = run_hsdpa(w)
    assert_parity(out, z["out"], w, w.name)
