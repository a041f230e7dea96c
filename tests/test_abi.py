"""The C-ABI library on the host (no GPU): it loads, exports every function
include/trifuse_moe.h declares, and rejects bad arguments before any device
work with the documented status codes."""
import ctypes
import re
from pathlib import Path

import pytest

from trifuse_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "trifuse_moe.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(tfm_[a-z0-9_]+)\s*\(", text)))


def test_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # the ctypes table covers the header exactly
    assert sorted(_lib.SIGNATURES) == names


def test_version_and_stage_names():
    lib = _lib.load()
    assert b"gfx950" in lib.tfm_version()
    assert [lib.tfm_stage_name(i).decode() for i in range(_lib.TFM_STAGE_COUNT)] == \
        ["router", "topk", "group", "gateup", "down", "combine", "norm"]
    assert lib.tfm_stage_name(99) == b""


def _geom(**kw):
    g = dict(hidden_size=2048, intermediate_size=1024, num_experts=64, experts_per_token=8,
             group_size=64, bits=4, dtype=_lib.TFM_DTYPE_BF16, route=_lib.TFM_ROUTE_OLMOE,
             router=_lib.TFM_ROUTER_DENSE, residual_multiplier=1.0)
    g.update(kw)
    return _lib.Geometry(**g)


@pytest.mark.parametrize("kw,code,msg", [
    (dict(hidden_size=2000), _lib.TFM_E_INVALID, "hidden_size"),
    (dict(intermediate_size=0), _lib.TFM_E_INVALID, "intermediate_size"),
    (dict(experts_per_token=65), _lib.TFM_E_INVALID, "experts_per_token"),
    (dict(experts_per_token=0), _lib.TFM_E_INVALID, "experts_per_token"),
    (dict(route=7), _lib.TFM_E_INVALID, "route"),
    (dict(bits=3), _lib.TFM_E_INVALID, "bits"),
    (dict(group_size=48), _lib.TFM_E_INVALID, "group_size"),
    (dict(num_experts=128, experts_per_token=8), _lib.TFM_E_UNSUPPORTED, "num_experts"),
    (dict(dtype=_lib.TFM_DTYPE_F16), _lib.TFM_E_UNSUPPORTED, "affine router"),
    (dict(dtype=7), _lib.TFM_E_INVALID, "dtype"),
    (dict(router=7), _lib.TFM_E_INVALID, "router"),
    (dict(bits=16), _lib.TFM_E_INVALID, "bits"),
    (dict(group_size=128), _lib.TFM_E_UNSUPPORTED, "group_size 64"),
])
def test_plan_create_rejects(kw, code, msg):
    lib = _lib.load()
    g = _geom(**kw)
    h = ctypes.c_void_p()
    st = lib.tfm_plan_create(ctypes.byref(g), ctypes.byref(h))
    assert st == code
    assert msg in lib.tfm_last_error().decode()
    assert not h.value


def test_null_arguments():
    lib = _lib.load()
    assert lib.tfm_plan_create(None, None) == _lib.TFM_E_INVALID
    assert b"geometry" in lib.tfm_last_error()
    assert lib.tfm_workspace_bytes(None, 4) == 0
    assert lib.tfm_group(None, 4, 8, None, None, None, None, 0, None) == _lib.TFM_E_INVALID
    assert lib.tfm_topk(None, 4, 65, 8, 0, 0, None, None) == _lib.TFM_E_UNSUPPORTED
    assert lib.tfm_topk(None, 4, 8, 9, 0, 0, None, None) == _lib.TFM_E_INVALID
    assert lib.tfm_olmoe_softmax(None, 4, 64, 7, None, None) == _lib.TFM_E_INVALID
    assert lib.tfm_olmoe_softmax(None, 4, 64, _lib.TFM_DTYPE_F16, None, None) == _lib.TFM_E_INVALID
    assert b"logits" in lib.tfm_last_error()
    assert lib.tfm_route_affine(None, None, 4, None, 4, None, None, None, None, None, 0, None) == _lib.TFM_E_INVALID
    assert lib.tfm_profiler_stage(None, 0, None, None, None) == _lib.TFM_E_INVALID
    assert lib.tfm_profiler_create(0, ctypes.byref(ctypes.c_void_p())) == _lib.TFM_E_INVALID


def test_group_workspace_checks():
    lib = _lib.load()
    n, E = 100, 8
    need = lib.tfm_group_workspace_bytes(n, E)
    assert need >= 256 + 2 * 4 * n
    buf = ctypes.create_string_buffer(need + 512)
    base = (ctypes.addressof(buf) + 255) // 256 * 256
    ids = ctypes.c_void_p(16)  # never dereferenced: the size check fails first
    st = lib.tfm_group(ids, n, E, ids, ids, ids, ctypes.c_void_p(base), need - 1, None)
    assert st == _lib.TFM_E_WORKSPACE and b"too small" in lib.tfm_last_error()
    st = lib.tfm_group(ids, n, E, ids, ids, ids, ctypes.c_void_p(base + 16), need, None)
    assert st == _lib.TFM_E_WORKSPACE and b"aligned" in lib.tfm_last_error()


def test_gather_qmm_argument_checks():
    lib = _lib.load()
    aff = _lib.Affine(16, 16, 16)
    st = lib.tfm_gather_qmm(None, 4, None, None, 8, ctypes.byref(aff), 4, 128, 256, 64, 4,
                            _lib.TFM_DTYPE_BF16, 0, None, None, 0, None)
    assert st == _lib.TFM_E_INVALID and b"x_row_count" in lib.tfm_last_error()
    # rows to compute but an empty x: refused before any pointer is read
    need = lib.tfm_gather_qmm_workspace_bytes(8, 4, 128, 256)
    buf = ctypes.create_string_buffer(need + 512)
    base = ctypes.c_void_p((ctypes.addressof(buf) + 255) // 256 * 256)
    fake = ctypes.c_void_p(16)  # never dereferenced
    st = lib.tfm_gather_qmm(fake, 0, fake, fake, 8, ctypes.byref(aff), 4, 128, 256, 64, 4,
                            _lib.TFM_DTYPE_BF16, 0, fake, base, need, None)
    assert st == _lib.TFM_E_INVALID and b"no rows" in lib.tfm_last_error()
    st = lib.tfm_gather_qmm(None, 8, None, None, 8, ctypes.byref(aff), 4, 96, 256, 64, 4,
                            _lib.TFM_DTYPE_BF16, 0, None, None, 0, None)
    assert st == _lib.TFM_E_UNSUPPORTED and b"multiple of 64" in lib.tfm_last_error()
    st = lib.tfm_gather_qmm(None, 8, None, None, 8, ctypes.byref(aff), 4, 128, 100, 64, 4,
                            _lib.TFM_DTYPE_BF16, 0, None, None, 0, None)
    assert st == _lib.TFM_E_INVALID and b"group_size" in lib.tfm_last_error()


def test_host_mirror_refuses_cpu_tensors():
    import torch

    from trifuse_amd import moe as tmoe

    q = torch.zeros((2, 64, 16), dtype=torch.int32)
    s = torch.zeros((2, 64, 2), dtype=torch.bfloat16)
    x = torch.zeros((3, 128), dtype=torch.bfloat16)
    idx = torch.zeros(3, dtype=torch.int32)
    with pytest.raises(ValueError, match="GPU tensor"):
        tmoe.native_affine_gather_qmm(x, q, s, s, idx, 64, 4)


def test_validate_affine_mirrors_reference_errors():
    import torch

    from trifuse_amd.moe import validate_affine

    q = torch.zeros((2, 64, 16), dtype=torch.int32)
    s = torch.zeros((2, 64, 2), dtype=torch.bfloat16)
    assert validate_affine(q, s, s, 64, 4, 3) == 128
    with pytest.raises(ValueError, match="bits4/8 and group32/64/128"):
        validate_affine(q, s, s, 64, 5, 3)
    with pytest.raises(ValueError, match="rank2/3 uint32"):
        validate_affine(q.float(), s, s, 64, 4, 3)
    with pytest.raises(ValueError, match="S/B shapes"):
        validate_affine(q, s, s.float(), 64, 4, 3)
    with pytest.raises(ValueError, match="packed/group"):
        validate_affine(q, s[:, :, :1], s[:, :, :1], 64, 4, 3)


@pytest.mark.parametrize("args,code,msg", [
    (dict(rows=-1), _lib.TFM_E_INVALID, "rows"),
    (dict(n_out=0), _lib.TFM_E_INVALID, "n_out"),
    (dict(bits=3), _lib.TFM_E_INVALID, "bits"),
    (dict(group=48), _lib.TFM_E_INVALID, "group_size"),
    (dict(k_in=96), _lib.TFM_E_INVALID, "multiple of group_size"),
    (dict(group=128), _lib.TFM_E_UNSUPPORTED, "group_size 64"),
    (dict(dtype=7), _lib.TFM_E_INVALID, "dtype"),
    (dict(n_out=96), _lib.TFM_E_UNSUPPORTED, "multiple of 64"),
    (dict(x=None), _lib.TFM_E_INVALID, "x"),
    (dict(w=None), _lib.TFM_E_INVALID, "w"),
])
def test_affine_qmm_rejects(args, code, msg):
    """tfm_affine_qmm (native_affine_qmm's entry point) checks its arguments
    before any device work: the messages of native_affine_ops.validate_affine's
    contract and the built limits."""
    lib = _lib.load()
    a = dict(x=16, rows=4, w=True, n_out=128, k_in=256, group=64, bits=4, dtype=_lib.TFM_DTYPE_BF16, out=16)
    a.update(args)
    aff = _lib.Affine(16, 16, 16)
    st = lib.tfm_affine_qmm(a["x"], a["rows"], ctypes.byref(aff) if a["w"] else None, a["n_out"], a["k_in"],
                            a["group"], a["bits"], a["dtype"], a["out"], None)
    assert st == code
    assert msg in lib.tfm_last_error().decode()


def test_affine_qmm_zero_rows_is_a_no_op():
    lib = _lib.load()
    assert lib.tfm_affine_qmm(None, 0, None, 128, 256, 64, 4, _lib.TFM_DTYPE_BF16, None, None) == _lib.TFM_OK
