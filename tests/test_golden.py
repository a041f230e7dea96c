"""The committed golden vectors (tests/golden/): the oracle reproduces them
(host), and the HIP path reproduces them bit-exactly for routing and grouping
and within max-rel 1e-2 for the block output (GPU)."""
import os

import numpy as np
import pytest

import oracle
from tests._util import BLOCK_TOL, log, max_rel

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


class Wts:
    def __init__(self, d):
        for k, v in d.items():
            setattr(self, k, v)


def nan_equal(a, b):
    fa, fb = oracle.bf16_to_f32(a), oracle.bf16_to_f32(b)
    return np.array_equal(np.isnan(fa), np.isnan(fb)) and np.array_equal(
        np.where(np.isnan(fa), 0, a), np.where(np.isnan(fb), 0, b))


@pytest.mark.parametrize("E", [64, 40])
def test_oracle_reproduces_routing_golden(E):
    g = load("routing.npz")
    lg = g[f"logits_e{E}"]
    oi, og = oracle.route_olmoe(lg, 8)
    np.testing.assert_array_equal(oi, g[f"olmoe_idx_e{E}"])
    assert nan_equal(og, g[f"olmoe_gates_e{E}"])
    gi, gg = oracle.route_granite(lg, 8)
    np.testing.assert_array_equal(gi, g[f"granite_idx_e{E}"])
    np.testing.assert_array_equal(np.isnan(gg), np.isnan(g[f"granite_gates_e{E}"]))
    assert nan_equal(oracle.olmoe_softmax(lg), g[f"olmoe_probs_e{E}"])
    order, inverse, offsets = oracle.group(oi.reshape(-1), E)
    np.testing.assert_array_equal(order, g[f"order_e{E}"])
    np.testing.assert_array_equal(inverse, g[f"inverse_e{E}"])
    np.testing.assert_array_equal(offsets, g[f"offsets_e{E}"])


def test_oracle_reproduces_block_golden():
    b = load("block.npz")
    w = Wts(b)
    logits = oracle.router_logits(b["x"], b["router"])
    idx, g = oracle.route_olmoe(logits, 2)
    np.testing.assert_array_equal(idx, b["idx"])
    np.testing.assert_array_equal(g, b["gates"])
    y = oracle.moe_reference(b["x"], idx, oracle.bf16_to_f32(g), w)
    np.testing.assert_allclose(y, b["y"], rtol=0, atol=0)


@pytest.mark.gpu
@pytest.mark.parametrize("E", [64, 40])
def test_gpu_routing_golden(gpu, E):
    import torch

    from tests._util import bf16_from_u16, u16
    from trifuse_amd import moe as tmoe

    log(f"golden routing E={E}")
    g = load("routing.npz")
    lg = g[f"logits_e{E}"]
    T = lg.shape[0]
    for route in ("olmoe", "granite"):
        blk = tmoe.MoEBlock(64, 64, E, 8, route=route)
        idx = torch.empty((T, 8), dtype=torch.int32, device=gpu)
        gates = torch.empty((T, 8), dtype=torch.bfloat16 if route == "olmoe" else torch.float32,
                            device=gpu)
        lt = bf16_from_u16(lg).to(gpu)
        tmoe.call("tfm_route_logits", blk._plan, lt.data_ptr(), T, idx.data_ptr(), gates.data_ptr(),
                  tmoe._stream())
        torch.cuda.synchronize()
        np.testing.assert_array_equal(idx.cpu().numpy(), g[f"{route}_idx_e{E}"])
        if route == "olmoe":
            assert nan_equal(u16(gates), g["olmoe_gates_e%d" % E])
    order, inverse, offsets = tmoe.group(torch.from_numpy(g[f"olmoe_idx_e{E}"].reshape(-1)).to(gpu), E)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(order.cpu().numpy(), g[f"order_e{E}"])
    np.testing.assert_array_equal(inverse.cpu().numpy(), g[f"inverse_e{E}"])
    np.testing.assert_array_equal(offsets.cpu().numpy(), g[f"offsets_e{E}"])


@pytest.mark.gpu
@pytest.mark.parametrize("deterministic", [False, True])
def test_gpu_block_golden(gpu, deterministic):
    import torch

    from tests._util import bf16_from_u16
    from trifuse_amd import moe as tmoe

    log(f"golden block deterministic={deterministic}")
    b = load("block.npz")
    dev = {}
    for k in ("gate", "up", "down"):
        dev[k + "_q"] = torch.from_numpy(b[k + "_q"].view(np.int32)).to(gpu)
        dev[k + "_s"] = bf16_from_u16(b[k + "_s"]).to(gpu)
        dev[k + "_b"] = bf16_from_u16(b[k + "_b"]).to(gpu)
    dev["router"] = bf16_from_u16(b["router"]).to(gpu)
    w = tmoe.ExpertWeights(**dev)
    blk = tmoe.MoEBlock(128, 64, 4, 2, route="olmoe")
    y, idx, gates = blk.forward(bf16_from_u16(b["x"]).to(gpu), w, deterministic=deterministic,
                                return_routes=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(idx.cpu().numpy(), b["idx"])
    assert max_rel(y.float().cpu().numpy(), b["y"]) <= BLOCK_TOL
