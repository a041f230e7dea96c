"""The allocation-free entry point (tfm_moe_forward_static) against
tfm_moe_forward: the same kernels on the library's static device scratch
instead of a caller workspace, so outputs, expert ids and gates are
bit-identical. Two calls in a row, the second with fewer tokens (the scratch
keeps the first call's contents), on the decode and the prefill paths, and a
call beyond the static array's size is refused."""
from pathlib import Path

import pytest
import torch

from tests._util import log
from trifuse_amd import _lib
from trifuse_amd import moe as tmoe
from trifuse_amd import workload as wl

pytestmark = pytest.mark.gpu


def _pair(blk, x, wts, res):
    y, idx, gates = blk.forward(x, wts, residual=res, return_routes=True)
    ys, idxs, gates_s = blk.forward_static(x, wts, residual=res, return_routes=True)
    torch.cuda.synchronize()
    assert torch.equal(idxs, idx)
    assert torch.equal(gates_s, gates)
    assert torch.equal(ys, y)


@pytest.mark.parametrize("geom_name,sizes", [("olmoe", (300, 8)), ("olmoe", (8, 1)), ("granite", (600, 32))])
def test_static_matches_workspace_entry_point(gpu, geom_name, sizes):
    geom = wl.OLMOE if geom_name == "olmoe" else wl.GRANITE
    rm = 0.25 if geom_name == "granite" else 1.0
    blk = tmoe.MoEBlock(geom.hidden, geom.intermediate, geom.experts, geom.top_k, route=geom.route,
                        residual_multiplier=rm)
    layer = wl.make_layer(geom, 0, gpu, seed_tag="static")
    wts = tmoe.ExpertWeights.from_layer(layer)
    for T in sizes:
        log(f"static scratch {geom_name} T={T}")
        x = wl.make_x(geom, T, tag=f"static{T}").to(gpu)
        res = wl.make_x(geom, T, tag=f"static_r{T}").to(gpu)
        _pair(blk, x, wts, res)


def test_static_refuses_oversized_call(gpu):
    geom = wl.OLMOE
    blk = tmoe.MoEBlock(geom.hidden, geom.intermediate, geom.experts, geom.top_k, route=geom.route)
    layer = wl.make_layer(geom, 0, gpu, seed_tag="static")
    wts = tmoe.ExpertWeights.from_layer(layer)
    T = 4096
    assert blk.workspace_bytes(T) > _lib.TFM_STATIC_SCRATCH_BYTES
    x = wl.make_x(geom, T, tag="static_big").to(gpu)
    with pytest.raises(_lib.TfmError, match="static array"):
        blk.forward_static(x, wts)


@pytest.mark.parametrize("geom_name,router,limit", [("olmoe", "dense", 776), ("olmoe", "affine", 773),
                                                    ("granite", "dense", 1105), ("granite", "affine", 1103)])
def test_static_token_limit_is_documented_one(gpu, geom_name, router, limit):
    """The token limits include/trifuse_moe.h states are the largest T whose
    workspace fits the static array."""
    geom = wl.OLMOE if geom_name == "olmoe" else wl.GRANITE
    dtype = torch.float16 if router == "affine" else torch.bfloat16
    blk = tmoe.MoEBlock(geom.hidden, geom.intermediate, geom.experts, geom.top_k, route=geom.route,
                        dtype=dtype, router=router)
    assert blk.workspace_bytes(limit) <= _lib.TFM_STATIC_SCRATCH_BYTES < blk.workspace_bytes(limit + 1)
    text = (Path(__file__).resolve().parents[1] / "include" / "trifuse_moe.h").read_text()
    assert f"{limit} " in text.replace("\n", " ")
