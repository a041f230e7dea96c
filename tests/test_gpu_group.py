"""Stable expert grouping on the GPU: order, inverse and offsets bit-exact
against the oracle and against numpy's stable argsort."""
import numpy as np
import pytest
import torch

import oracle
from tests._util import log
from trifuse_amd import _lib
from trifuse_amd import moe as tmoe

pytestmark = pytest.mark.gpu


def _ids(n, E, seed, skew=False):
    rng = np.random.default_rng(seed)
    if skew:
        p = 1.0 / np.arange(1, E + 1) ** 1.1
        return rng.choice(E, size=n, p=p / p.sum()).astype(np.int32)
    return rng.integers(0, E, size=n).astype(np.int32)


@pytest.mark.parametrize("n,E,skew", [(1, 1, False), (8, 64, False), (63, 64, False),
                                      (64, 64, False), (1000, 40, False), (1024, 64, True),
                                      (1025, 2, False), (32768, 64, True), (100003, 64, False),
                                      (16384, 40, True), (5, 64, True)])
def test_group_bitexact(gpu, n, E, skew):
    log(f"group n={n} E={E} skew={skew}")
    ids = _ids(n, E, n * 7 + E, skew)
    order, inverse, offsets = tmoe.group(torch.from_numpy(ids).to(gpu), E)
    torch.cuda.synchronize()
    ro, ri, roff = oracle.group(ids, E)
    np.testing.assert_array_equal(order.cpu().numpy(), ro)
    np.testing.assert_array_equal(inverse.cpu().numpy(), ri)
    np.testing.assert_array_equal(offsets.cpu().numpy(), roff)
    np.testing.assert_array_equal(ro, np.argsort(ids, kind="stable"))


def test_group_empty(gpu):
    log("group n=0")
    order, inverse, offsets = tmoe.group(torch.empty(0, dtype=torch.int32, device=gpu), 8)
    torch.cuda.synchronize()
    assert order.numel() == 0 and inverse.numel() == 0
    np.testing.assert_array_equal(offsets.cpu().numpy(), np.zeros(9, np.int32))


def test_group_bad_ids_flagged(gpu):
    log("group bad ids")
    ids = np.array([3, 9, -1, 3, 0, 8], dtype=np.int32)  # E = 8: 9, -1, 8 are invalid
    E = 8
    t = torch.from_numpy(ids).to(gpu)
    lib = _lib.load()
    n = ids.size
    order = torch.empty(n, dtype=torch.int32, device=gpu)
    inverse = torch.empty(n, dtype=torch.int32, device=gpu)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=gpu)
    wsb = lib.tfm_group_workspace_bytes(n, E)
    ws = torch.empty(wsb, dtype=torch.uint8, device=gpu)
    tmoe.call("tfm_group", t.data_ptr(), n, E, order.data_ptr(), inverse.data_ptr(),
              offsets.data_ptr(), ws.data_ptr(), wsb, tmoe._stream())
    import ctypes
    st = ctypes.c_uint32()
    tmoe.call("tfm_status_word", ws.data_ptr(), tmoe._stream(), ctypes.byref(st))
    assert st.value & _lib.TFM_STATUS_BAD_EXPERT_ID
    off = offsets.cpu().numpy()
    assert off[E] == 3  # valid routes only
    o = order.cpu().numpy()
    np.testing.assert_array_equal(o[:3], [4, 0, 3])  # expert 0 then expert 3 (stable)
    np.testing.assert_array_equal(sorted(o[3:]), [1, 2, 5])
