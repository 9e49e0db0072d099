"""The fused paths of the verify forward are exact rewrites of the separate
kernels: logits with fusion on (operand built inside the consuming GEMV for
1-2 columns: residual prep, attention combine, SwiGLU rows; residual prep run
by the last workgroup of the o / down GEMVs above 2 columns) equal the logits
of the unfused kernel sequence (SH_FUSE=0) bit for bit."""
import os
import subprocess
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HELPER = os.path.join(os.path.dirname(os.path.abspath(__file__)), "fusion_logits.py")


def _run(tmp_path, fuse):
    out = str(tmp_path / f"fuse{fuse}.npz")
    env = dict(os.environ, SH_FUSE=str(fuse))
    print(f"fusion helper SH_FUSE={fuse}", flush=True)
    r = subprocess.run([sys.executable, HELPER, out], env=env, capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stdout + r.stderr
    return np.load(out)


def test_fused_equals_unfused(tmp_path):
    a, b = _run(tmp_path, 1), _run(tmp_path, 0)
    for k in a.files:
        assert np.array_equal(a[k], b[k]), (k, float(np.abs(a[k] - b[k]).max()))
