"""Decode at one to three tokens: the three-kernel layer (routing in every
gate/up workgroup, down projection fused with the combine) against the
oracle, and bit for bit against the four-kernel streaming layer that
larger batches take."""
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from tests._util import log
from tests.test_gpu_moe import _block, _check_layer
from trifuse_amd import moe as tmoe
from trifuse_amd import workload as wl

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.parametrize("geom_name", ["olmoe", "granite"])
@pytest.mark.parametrize("T", [1, 2, 3])
def test_small_batch_against_oracle(gpu, geom_name, T):
    geom = wl.OLMOE if geom_name == "olmoe" else wl.GRANITE
    log(f"decode small T={T} {geom_name}")
    layer = wl.make_layer(geom, 0, gpu, seed_tag=f"small{geom_name}")
    x = wl.make_x(geom, T, tag=f"small_x{T}")
    residual = wl.make_x(geom, T, tag=f"small_r{T}")
    rm = 0.25 if geom_name == "granite" else 1.0
    _check_layer(geom, _block(geom, rm=rm), x, layer, np.arange(T, dtype=np.int32), residual=residual, rm=rm)


def _general_case(geom_name, bits, device):
    """Seeded layer, inputs and block of the small-against-general check."""
    geom = wl.OLMOE if geom_name == "olmoe" else wl.GRANITE
    layer = wl.make_layer(geom, 1, device, seed_tag=f"smallgen{geom_name}", bits=bits)
    x = wl.make_x(geom, 4, tag="smallgen_x").to(device)
    res = wl.make_x(geom, 4, tag="smallgen_r").to(device)
    blk = tmoe.MoEBlock(geom.hidden, geom.intermediate, geom.experts, geom.top_k, route=geom.route,
                        residual_multiplier=0.5, bits=bits)
    return geom, tmoe.ExpertWeights.from_layer(layer), x, res, blk


@pytest.mark.parametrize("geom_name", ["olmoe", "granite"])
@pytest.mark.parametrize("bits", [4, 8])
def test_small_batch_matches_general_path(gpu, geom_name, bits, tmp_path):
    # Tokens 0-2 through the small-batch layer (T = 1, 2, 3: down fused with
    # the combine) and through the general streaming layer (T = 4: separate
    # down kernel and combine) give identical bits: every route's products
    # and the k-ordered sum are rounded the same way in both. 8-bit codes
    # stream at four tokens by default; 4-bit ones take the decode GEMV
    # kernels there, so their four-token streaming layer runs in a child
    # process with TFM_DS_MAX_TOKENS=4 (read once per process).
    log(f"decode small vs general {geom_name} {bits}-bit")
    geom, wts, x, res, blk = _general_case(geom_name, bits, gpu)
    if bits == 8:
        y4 = blk.forward(x, wts, residual=res)
        torch.cuda.synchronize()
        y4 = y4.cpu()
    else:
        path = tmp_path / "y4.npy"
        code = ("import sys, numpy as np, torch; from tests.test_gpu_decode_small import _general_case; "
                f"g, w, x, r, b = _general_case({geom_name!r}, 4, 'cuda:0'); "
                "y = b.forward(x, w, residual=r); torch.cuda.synchronize(); "
                "np.save(sys.argv[1], y.cpu().view(torch.int16).numpy())")
        out = subprocess.run([sys.executable, "-c", code, str(path)], cwd=ROOT, capture_output=True, text=True,
                             env={**os.environ, "TFM_DS_MAX_TOKENS": "4"}, timeout=110)
        assert out.returncode == 0, out.stderr[-2000:]
        y4 = torch.from_numpy(np.load(path)).view(torch.bfloat16)
    for T in (3, 2, 1):
        yT = blk.forward(x[:T].contiguous(), wts, residual=res[:T].contiguous())
        torch.cuda.synchronize()
        assert torch.equal(yT.cpu(), y4[:T]), f"T={T}"


def test_small_batch_hook_matches_forward(gpu):
    # NativeMoEExpertHook::execute (given routes) takes the same kernels as
    # the whole block at one to three tokens.
    geom = wl.OLMOE
    layer = wl.make_layer(geom, 2, gpu, seed_tag="smallhook")
    wts = tmoe.ExpertWeights.from_layer(layer)
    blk = _block(geom)
    for T in (1, 2, 3):
        log(f"decode small hook T={T}")
        x = wl.make_x(geom, T, tag=f"smallhook{T}").to(gpu)
        y, idx, gates = blk.forward(x, wts, return_routes=True)
        y2 = blk.experts(x, idx, gates, wts)
        torch.cuda.synchronize()
        assert torch.equal(y, y2)


@pytest.mark.parametrize("route,K", [("olmoe", 32), ("olmoe", 25), ("granite", 24)])
@pytest.mark.parametrize("T", [1, 2])
def test_one_token_many_routes(gpu, route, K, T):
    """Many routes per token. Past the fused down + combine kernel's 24
    routes (K = 25, 32 at one token; every K here at two tokens) one token
    still ranks its routes in the gate/up prologue, but the separate down
    kernel reads h in expert-sorted order, so the gate/up kernel must write
    it that way; K = 24 at one token is the fused kernel's limit (h in route
    order). Against the oracle, and bit for bit against the same tokens
    inside a three-token batch."""
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
