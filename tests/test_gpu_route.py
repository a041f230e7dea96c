"""Router linear and routing on the GPU against the oracle: bit-exact logits,
expert ids (slot order included), gates and probabilities."""
import numpy as np
import pytest
import torch

import oracle
from tests._util import bf16_from_u16, f32, log, u16
from trifuse_amd import moe as tmoe
from trifuse_amd import workload as wl

pytestmark = pytest.mark.gpu


def assert_bf16_equal(got, ref):
    """Bit equality of bf16 arrays, NaN matching NaN of either sign (a NaN made
    by arithmetic has the host's or the GPU's default sign)."""
    nan_g = np.isnan(oracle.bf16_to_f32(got))
    nan_r = np.isnan(oracle.bf16_to_f32(ref))
    np.testing.assert_array_equal(nan_g, nan_r)
    np.testing.assert_array_equal(np.where(nan_r, 0, got), np.where(nan_r, 0, ref))


def _block(geom):
    return tmoe.MoEBlock(geom.hidden, geom.intermediate, geom.experts, geom.top_k, route=geom.route)


@pytest.mark.parametrize("geom", [wl.OLMOE, wl.GRANITE], ids=lambda g: g.name)
@pytest.mark.parametrize("T", [1, 8, 33, 300])
@pytest.mark.parametrize("bias", [False, True])
def test_route_bitexact(gpu, geom, T, bias):
    log(f"route {geom.name} T={T} bias={bias}")
    x = wl.make_x(geom, T, tag=f"route{T}")
    router = wl.normal_bf16((geom.experts, geom.hidden), 0.02, 1234 + T)
    lb = wl.zipf_bias(geom.experts, 99) if bias else None
    blk = _block(geom)
    idx, gates, logits = blk.route(x.to(gpu), router.to(gpu), None if lb is None else lb.to(gpu))
    torch.cuda.synchronize()
    ref_logits = oracle.router_logits(u16(x), u16(router), None if lb is None else lb.numpy())
    np.testing.assert_array_equal(u16(logits), ref_logits)
    if geom.route == "olmoe":
        ridx, rg = oracle.route_olmoe(ref_logits, geom.top_k)
        np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
        np.testing.assert_array_equal(u16(gates), rg)
    else:
        ridx, rg = oracle.route_granite(ref_logits, geom.top_k)
        np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
        np.testing.assert_array_equal(gates.cpu().numpy().view(np.uint32), rg.view(np.uint32))


def _tie_logits(T, E, seed):
    """Logit rows with planted ties, -inf/+inf, NaN and all-equal rows."""
    rng = np.random.default_rng(seed)
    v = rng.integers(-6, 6, size=(T, E)).astype(np.float32) * 0.25  # many exact ties
    v[0, :] = 0.5                      # all equal
    v[1, 3 % E] = np.nan
    v[2, ::7] = np.nan
    v[3, :] = np.nan                   # all NaN
    v[4, 5 % E] = np.inf
    v[5, 9 % E] = -np.inf
    v[6, :] = -np.inf                  # exp(-inf - (-FLT_MAX)) = 0 everywhere
    return oracle.f32_to_bf16(v)


@pytest.mark.parametrize("E,K,route", [(64, 8, "olmoe"), (40, 8, "granite"), (64, 8, "granite"),
                                       (40, 8, "olmoe"), (7, 3, "olmoe"), (7, 3, "granite"),
                                       (1, 1, "olmoe"), (64, 64, "granite")])
def test_route_logits_ties_nan(gpu, E, K, route):
    log(f"route_logits ties E={E} K={K} {route}")
    T = 64
    lg = _tie_logits(T, E, E * 100 + K)
    blk = tmoe.MoEBlock(64, 64, E, K, route=route)
    lt = bf16_from_u16(lg).to(gpu)
    idx = torch.empty((T, K), dtype=torch.int32, device=gpu)
    gdt = torch.bfloat16 if route == "olmoe" else torch.float32
    gates = torch.empty((T, K), dtype=gdt, device=gpu)
    tmoe.call("tfm_route_logits", blk._plan, lt.data_ptr(), T, idx.data_ptr(), gates.data_ptr(),
              tmoe._stream())
    torch.cuda.synchronize()
    if route == "olmoe":
        ridx, rg = oracle.route_olmoe(lg, K)
        np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
        assert_bf16_equal(u16(gates), rg)
    else:
        ridx, rg = oracle.route_granite(lg, K)
        np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
        g = gates.cpu().numpy()
        np.testing.assert_array_equal(np.isnan(g), np.isnan(rg))
        np.testing.assert_array_equal(np.nan_to_num(g).view(np.uint32), np.nan_to_num(rg).view(np.uint32))


@pytest.mark.parametrize("E", [64, 40, 5])
def test_olmoe_softmax_bitexact(gpu, E):
    log(f"olmoe_softmax E={E}")
    rng = np.random.default_rng(E)
    lg = oracle.f32_to_bf16(rng.standard_normal((129, E)).astype(np.float32) * 3)
    lg[:8] = _tie_logits(8, E, 7)
    p = tmoe.native_olmoe_softmax(bf16_from_u16(lg).to(gpu).reshape(1, 129, E))
    torch.cuda.synchronize()
    ref = oracle.olmoe_softmax(lg)
    assert_bf16_equal(u16(p).reshape(129, E), ref)


@pytest.mark.parametrize("n,k", [(64, 8), (40, 8), (13, 13), (3, 1)])
def test_topk_ops(gpu, n, k):
    log(f"topk ops n={n} k={k}")
    lg = _tie_logits(50, n, n + k)
    x = bf16_from_u16(lg).to(gpu).reshape(1, 50, n)
    got_o = tmoe.native_olmoe_topk_indices(x, k).cpu().numpy().reshape(50, k)
    got_g = tmoe.native_topk_indices(x, k).cpu().numpy().reshape(50, k)
    vals = oracle.bf16_to_f32(lg)
    nan = np.isnan(vals)

    def stable_order(key):  # NaN last, then by key, ties by index (lexsort is stable)
        return np.stack([np.lexsort((np.where(nan[r], 0, key[r]), nan[r])) for r in range(len(key))])

    # OLMoE rule is the reference's torch body argsort(-x, stable)[:k] with NaN last.
    np.testing.assert_array_equal(got_o, stable_order(-vals)[:, :k])
    # Granite rule: stable ascending sort (NaN last), last k slots.
    np.testing.assert_array_equal(got_g, stable_order(vals)[:, n - k:])
    take = tmoe.native_take_along_last(x, tmoe.native_olmoe_topk_indices(x, k))
    np.testing.assert_array_equal(u16(take).reshape(50, k),
                                  np.take_along_axis(lg, got_o.astype(np.int64), axis=-1))


def test_route_large_T(gpu):
    log("route OLMoE T=4096 zipf bias")
    geom = wl.OLMOE
    layer = wl.make_layer(geom, 0, device=gpu, zipf=True, seed_tag="route_big")
    x = wl.make_x(geom, 4096, tag="route_big")
    blk = _block(geom)
    idx, gates, logits = blk.route(x.to(gpu), layer.router, layer.logit_bias)
    torch.cuda.synchronize()
    ref_logits = oracle.router_logits(u16(x), u16(layer.router), f32(layer.logit_bias))
    np.testing.assert_array_equal(u16(logits), ref_logits)
    ridx, rg = oracle.route_olmoe(ref_logits, 8)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_array_equal(u16(gates), rg)
    counts = np.bincount(ridx.reshape(-1), minlength=64)
    top4 = np.sort(counts)[::-1][:4].sum() / counts.sum()
    log(f"  zipf top-4 share {top4:.3f}")
    assert 0.36 <= top4 <= 0.44  # the skew the Zipf(1.1) rank profile is calibrated for
