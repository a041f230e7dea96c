"""Tuning overrides that change how the kernels move data but not what they
compute give the same bits as the defaults: the down-weight copies of 1 to
3 tokens (TFM_DS_PREFETCH=1), the grouped GEMM's plain and dword-swizzled
scale/bias layouts in LDS (TFM_GGEMM_SB_LAYOUT=0/1), either grouping of
the decode GEMV path (TFM_DECODE_GROUPING=slots/workgroup) and the weight
prefetch depth of 64-row tiles of at most 16 rows (TFM_GGEMM_FEW_ROWS=0/2).
The overrides are read once per process, so each runs in a child process."""
import os
import subprocess
import sys

import numpy as np
import pytest

from tests._knob_cases import outputs
from tests._util import log

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def default_outputs(gpu):
    return outputs()


@pytest.mark.parametrize("env", [{"TFM_DS_PREFETCH": "1"}, {"TFM_GGEMM_SB_LAYOUT": "0"},
                                 {"TFM_GGEMM_SB_LAYOUT": "1"}, {"TFM_DECODE_GROUPING": "slots"},
                                 {"TFM_DECODE_GROUPING": "workgroup"}, {"TFM_GGEMM_FEW_ROWS": "0"},
                                 {"TFM_GGEMM_FEW_ROWS": "2"}],
                         ids=lambda e: ",".join(f"{k}={v}" for k, v in e.items()))
def test_override_gives_default_bits(default_outputs, env, tmp_path):
    log(f"override {env}")
    path = tmp_path / "out.npz"
    res = subprocess.run([sys.executable, "-m", "tests._knob_cases", str(path)], cwd=ROOT,
                         env={**os.environ, **env}, capture_output=True, text=True, timeout=110)
    assert res.returncode == 0, res.stderr[-2000:]
    got = np.load(path)
    for k, ref in default_outputs.items():
        np.testing.assert_array_equal(got[k], ref, err_msg=k)
