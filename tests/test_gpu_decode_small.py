"""Decode at one and two tokens: the three-kernel layer (routing in one
workgroup, down projection fused with the combine) against the oracle, and
bit for bit against the five-kernel layer that larger batches take."""
import numpy as np
import pytest
import torch

from tests._util import log
from tests.test_gpu_moe import _block, _check_layer
from trifuse_amd import moe as tmoe
from trifuse_amd import workload as wl

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("geom_name", ["olmoe", "granite"])
@pytest.mark.parametrize("T", [1, 2])
def test_small_batch_against_oracle(gpu, geom_name, T):
    geom = wl.OLMOE if geom_name == "olmoe" else wl.GRANITE
    log(f"decode small T={T} {geom_name}")
    layer = wl.make_layer(geom, 0, gpu, seed_tag=f"small{geom_name}")
    x = wl.make_x(geom, T, tag=f"small_x{T}")
    residual = wl.make_x(geom, T, tag=f"small_r{T}")
    rm = 0.25 if geom_name == "granite" else 1.0
    _check_layer(geom, _block(geom, rm=rm), x, layer, np.arange(T, dtype=np.int32), residual=residual, rm=rm)


@pytest.mark.parametrize("geom_name", ["olmoe", "granite"])
def test_small_batch_matches_general_path(gpu, geom_name):
    # Tokens 0 and 1 through the small-batch layer (T = 2) and through the
    # general one (T = 3) give identical bits: every route's products and the
    # k-ordered sum are rounded the same way in both.
    geom = wl.OLMOE if geom_name == "olmoe" else wl.GRANITE
    log(f"decode small vs general {geom_name}")
    layer = wl.make_layer(geom, 1, gpu, seed_tag=f"smallgen{geom_name}")
    wts = tmoe.ExpertWeights.from_layer(layer)
    x = wl.make_x(geom, 3, tag="smallgen_x").to(gpu)
    res = wl.make_x(geom, 3, tag="smallgen_r").to(gpu)
    blk = _block(geom, rm=0.5)
    y3 = blk.forward(x, wts, residual=res)
    y2 = blk.forward(x[:2].contiguous(), wts, residual=res[:2].contiguous())
    y1 = blk.forward(x[:1].contiguous(), wts, residual=res[:1].contiguous())
    torch.cuda.synchronize()
    assert torch.equal(y2, y3[:2])
    assert torch.equal(y1, y3[:1])


def test_small_batch_hook_matches_forward(gpu):
    # NativeMoEExpertHook::execute (given routes) takes the same kernels as
    # the whole block at one and two tokens.
    geom = wl.OLMOE
    layer = wl.make_layer(geom, 2, gpu, seed_tag="smallhook")
    wts = tmoe.ExpertWeights.from_layer(layer)
    blk = _block(geom)
    for T in (1, 2):
        log(f"decode small hook T={T}")
        x = wl.make_x(geom, T, tag=f"smallhook{T}").to(gpu)
        y, idx, gates = blk.forward(x, wts, return_routes=True)
        y2 = blk.experts(x, idx, gates, wts)
        torch.cuda.synchronize()
        assert torch.equal(y, y2)


@pytest.mark.parametrize("route,K", [("olmoe", 32), ("olmoe", 17), ("granite", 24)])
@pytest.mark.parametrize("T", [1, 2])
def test_one_token_many_routes(gpu, route, K, T):
    """More routes than the fused down + combine kernel takes (K > 16): one
    token still ranks its routes in the gate/up prologue, but the separate
    down kernel reads h in expert-sorted order, so the gate/up kernel must
    write it that way. Against the oracle, and bit for bit against the
    same tokens inside a three-token batch."""
    geom = wl.Geometry(f"{route}_k{K}", 2048, 1024, 64, K, route)
    log(f"decode one token many routes {route} K={K} T={T}")
    layer = wl.make_layer(geom, 0, gpu, seed_tag=f"manyk{K}")
    x = wl.make_x(geom, 3, tag=f"manyk_x{K}")
    residual = wl.make_x(geom, 3, tag=f"manyk_r{K}")
    blk = _block(geom)
    _check_layer(geom, blk, x[:T].contiguous(), layer, np.arange(T, dtype=np.int32),
                 residual=residual[:T].contiguous())
    wts = tmoe.ExpertWeights.from_layer(layer)
    xg, rg = x.to(gpu), residual.to(gpu)
    y3 = blk.forward(xg, wts, residual=rg)
    yT = blk.forward(xg[:T].contiguous(), wts, residual=rg[:T].contiguous())
    torch.cuda.synchronize()
    assert torch.equal(yT, y3[:T])
