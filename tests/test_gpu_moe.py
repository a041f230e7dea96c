"""The whole MoE block on the GPU at the benchmark workloads' full sizes:
routing bit-exact against the oracle for every token and layer, block output
within max-rel 1e-2 of the oracle's fp64 reference (exactly dequantised
weights, the oracle's own routes and gates): on every token at the prefill
sizes (the per-expert fp64 matrix-product form of the reference), on sampled
tokens elsewhere."""
import numpy as np
import pytest
import torch

import oracle
from tests._util import BLOCK_TOL, f32, log, max_rel, np_layer, u16
from trifuse_amd import moe as tmoe
from trifuse_amd import workload as wl

pytestmark = pytest.mark.gpu


def _block(geom, rm=1.0):
    return tmoe.MoEBlock(geom.hidden, geom.intermediate, geom.experts, geom.top_k, route=geom.route,
                         residual_multiplier=rm)


def _oracle_routes(geom, x_u16, lay):
    logits = oracle.router_logits(x_u16, lay.router, lay.logit_bias)
    if geom.route == "olmoe":
        idx, g = oracle.route_olmoe(logits, geom.top_k)
        return idx, oracle.bf16_to_f32(g)
    return oracle.route_granite(logits, geom.top_k)


def _check_layer(geom, blk, x, layer, sample, deterministic=False, residual=None, rm=1.0):
    """sample: token indices checked against the sequential reference, or
    None for every token through the per-expert fp64 matrix products."""
    xg = x.to(layer.router.device)
    res_g = None if residual is None else residual.to(xg.device)
    y, idx, gates = blk.forward(xg, tmoe.ExpertWeights.from_layer(layer), residual=res_g,
                                deterministic=deterministic, return_routes=True)
    torch.cuda.synchronize()
    lay = np_layer(layer)
    xu = u16(x)
    ridx, rg = _oracle_routes(geom, xu, lay)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_array_equal(gates.cpu().numpy().view(np.uint32), rg.view(np.uint32))
    res_u = None if residual is None else u16(residual)
    if sample is None:
        ref = oracle.moe_reference_full(xu, ridx, rg, lay, residual=res_u, rm=rm)
        got = oracle.bf16_to_f32(u16(y))
    else:
        ref = oracle.moe_reference(xu, ridx, rg, lay, tokens=sample, residual=res_u, rm=rm)
        got = oracle.bf16_to_f32(u16(y))[sample]
    err = max_rel(got, ref)
    # also the worst single token, relative to that token's own largest value
    tok = float(np.max(np.max(np.abs(got - ref), axis=1) / np.maximum(np.max(np.abs(ref), axis=1), 1e-30)))
    log(f"  max_rel {err:.2e} (worst token {tok:.2e}) over {got.shape[0]} tokens")
    assert err <= BLOCK_TOL
    return y, ridx


def _sample(T, n, ridx=None, seed=0):
    rng = np.random.default_rng(seed)
    s = set(rng.choice(T, size=min(n, T), replace=False).tolist())
    s.update({0, T - 1})
    return np.array(sorted(s), dtype=np.int32)


def test_olmoe_decode_t1(gpu):
    w = wl.WORKLOADS["olmoe_decode_t1"]
    log(f"moe {w.name}")
    layer = wl.workload_layers(w, gpu)[0]
    _check_layer(w.geometry, _block(w.geometry), wl.workload_x(w), layer, np.array([0], np.int32))


def test_olmoe_decode_t8_x16(gpu):
    w = wl.WORKLOADS["olmoe_decode_t8_x16"]
    log(f"moe {w.name}")
    x = wl.workload_x(w)
    blk = _block(w.geometry)
    for l, layer in enumerate(wl.workload_layers(w, gpu)):
        log(f" layer {l}")
        sample = np.arange(8, dtype=np.int32) if l in (0, 15) else np.array([l % 8], np.int32)
        _check_layer(w.geometry, blk, x, layer, sample)
        del layer


@pytest.mark.parametrize("T", [3, 4, 13, 14, 15, 22, 23, 24, 32, 33, 64, 96, 97])
def test_olmoe_batch_sweep(gpu, T):
    """Both sides of the streaming-decode (up to 3 tokens), decode-GEMV (up to
    E + 40 = 104 routes, 13 tokens) and grouped-GEMM path switches, the last
    size whose staged x rows would fit the streaming kernels (14 tokens) and
    the GEMM's 64-row tiles, up to and past 12 routes per expert (96 and 97
    tokens), the limit of the 64-row instance whose tiles of at most 16 rows
    keep their weights two super-steps ahead; every token checked."""
    w = wl.get_workload(f"olmoe_t{T}")
    log(f"moe {w.name}")
    layer = wl.workload_layers(w, gpu)[0]
    _check_layer(w.geometry, _block(w.geometry), wl.workload_x(w), layer, None)


@pytest.mark.parametrize("T", [1, 2, 3, 4, 10, 11, 19, 20, 22, 23, 60, 61])
def test_granite_batch_sweep(gpu, T):
    """Granite (hidden 1536, 40 experts), every token checked: the one- and
    two-token streaming layers, the four-kernel streaming layer (3 tokens),
    the decode GEMV from 4 tokens up to E + 40 = 80 routes (10 tokens) and the
    grouped GEMM's four-wave 64-row tiles beyond (11 tokens; 19 and 20 tokens
    on either side of the streaming kernels' LDS limit; 23 tokens; 60 and 61
    tokens on either side of 12 routes per expert, the limit of the instance
    whose tiles of at most 16 rows keep their weights two super-steps
    ahead)."""
    w = wl.get_workload(f"granite_t{T}")
    log(f"moe {w.name}")
    layer = wl.workload_layers(w, gpu)[0]
    _check_layer(w.geometry, _block(w.geometry), wl.workload_x(w), layer, None)


@pytest.mark.parametrize("name", ["granite_t768", "olmoe_t1792"])
def test_tall_tiles_below_384_routes(gpu, name):
    """256-row grouped-GEMM tiles where experts average fewer than 384 routes:
    Granite 768 tokens (154 per expert; 256-row tiles fit one round of the
    compute units) and OLMoE 1792 tokens (224 per expert), every token
    checked."""
    w = wl.get_workload(name)
    log(f"moe {w.name}")
    layer = wl.workload_layers(w, gpu)[0]
    _check_layer(w.geometry, _block(w.geometry), wl.workload_x(w), layer, None)


@pytest.mark.parametrize("deterministic", [False, True])
def test_olmoe_prefill_t512(gpu, deterministic):
    w = wl.WORKLOADS["olmoe_prefill_t512"]
    log(f"moe {w.name} deterministic={deterministic}")
    layer = wl.workload_layers(w, gpu)[0]
    _check_layer(w.geometry, _block(w.geometry), wl.workload_x(w), layer,
                 None if deterministic else _sample(512, 24), deterministic=deterministic)


def test_olmoe_prefill_t4096_zipf(gpu):
    w = wl.WORKLOADS["olmoe_prefill_t4096_zipf"]
    log(f"moe {w.name}")
    layer = wl.workload_layers(w, gpu)[0]
    x = wl.workload_x(w)
    y, ridx = _check_layer(w.geometry, _block(w.geometry), x, layer, None)
    counts = np.bincount(ridx.reshape(-1), minlength=64)
    top4 = np.sort(counts)[::-1][:4].sum() / counts.sum()
    log(f"  top-4 expert share {top4:.3f}, hottest expert {counts.max()} routes")
    assert 0.36 <= top4 <= 0.44  # the skew the Zipf(1.1) rank profile is calibrated for
    # Every path reduces a token's K routes in k order: a second run, with or
    # without the deterministic flag and on a fresh block, is bit-identical.
    blk = _block(w.geometry)
    wts = tmoe.ExpertWeights.from_layer(layer)
    y1 = blk.forward(x.to(gpu), wts, deterministic=True)
    y2 = blk.forward(x.to(gpu), wts, deterministic=True)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    assert torch.equal(y1, y)


def test_granite_prefill_then_decode(gpu):
    wp = wl.WORKLOADS["granite_prefill_t2048"]
    wd = wl.WORKLOADS["granite_decode_t32"]
    geom = wp.geometry
    layer = wl.workload_layers(wp, gpu)[0]
    blk = _block(geom)
    log(f"moe {wp.name}")
    _check_layer(geom, blk, wl.workload_x(wp), layer, None)
    log(f"moe {wd.name}")
    _check_layer(geom, blk, wl.workload_x(wd), layer, np.arange(32, dtype=np.int32))


def test_residual_and_multiplier(gpu):
    geom = wl.GRANITE
    log("moe residual + residual_multiplier")
    layer = wl.make_layer(geom, 0, gpu, seed_tag="residual")
    x = wl.make_x(geom, 300, tag="res_x")
    residual = wl.make_x(geom, 300, tag="res_r")
    blk = _block(geom, rm=0.25)
    _check_layer(geom, blk, x, layer, _sample(300, 10), residual=residual, rm=0.25)
    x8 = x[:8].contiguous()
    _check_layer(geom, blk, x8, layer, np.arange(8, dtype=np.int32), residual=residual[:8].contiguous(),
                 rm=0.25)


def test_experts_hook_and_routes_callable(gpu):
    geom = wl.OLMOE
    log("hook execute + GPUCallable")
    layer = wl.make_layer(geom, 0, gpu, seed_tag="hook")
    wts = tmoe.ExpertWeights.from_layer(layer)
    blk = _block(geom)
    for T in (4, 300):
        x = wl.make_x(geom, T, tag=f"hook{T}").to(gpu)
        y, idx, gates = blk.forward(x, wts, return_routes=True, deterministic=True)
        y2 = blk.experts(x, idx, gates, wts, deterministic=True)
        torch.cuda.synchronize()
        assert torch.equal(y, y2)
        # GPUCallable: routes in caller order -> expert-sorted rows + inverse.
        N = T * geom.top_k
        tok = torch.arange(N, device=gpu, dtype=torch.int32) // geom.top_k
        out, inv = blk.expert_routes(x, tok, idx.reshape(-1), False, wts)
        torch.cuda.synchronize()
        order = np.argsort(idx.cpu().numpy().reshape(-1), kind="stable")
        np.testing.assert_array_equal(inv.cpu().numpy(), np.argsort(order))
        rows = oracle.bf16_to_f32(u16(out))[inv.cpu().numpy()]          # caller order
        g = gates.cpu().numpy().reshape(-1)
        comb = (rows * g[:, None]).reshape(T, geom.top_k, -1).sum(1)
        assert max_rel(comb, f32(y)) <= BLOCK_TOL
        # experts_sorted: the caller's promise that ids are non-decreasing.
        ids_sorted = idx.reshape(-1)[torch.from_numpy(order).to(gpu)]
        out_s, inv_s = blk.expert_routes(x, tok[torch.from_numpy(order).to(gpu)], ids_sorted, True, wts)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(inv_s.cpu().numpy(), np.arange(N))
        assert torch.equal(out_s, out)
    # N == 0 is allowed.
    out0, inv0 = blk.expert_routes(x, tok[:0], idx.reshape(-1)[:0], False, wts)
    assert out0.shape == (0, geom.hidden) and inv0.numel() == 0


def test_empty_and_bad_routes(gpu):
    geom = wl.OLMOE
    log("moe T=0 and out-of-range expert ids")
    layer = wl.make_layer(geom, 0, gpu, seed_tag="edge")
    wts = tmoe.ExpertWeights.from_layer(layer)
    blk = _block(geom)
    y0 = blk.forward(torch.empty((0, geom.hidden), dtype=torch.bfloat16, device=gpu), wts)
    assert y0.shape == (0, geom.hidden)
    x = wl.make_x(geom, 2, tag="edge").to(gpu)
    y, idx, gates = blk.forward(x, wts, return_routes=True)
    bad = idx.clone()
    bad[0, 3] = 64
    bad[1, 0] = -5
    yb = blk.experts(x, bad, gates, wts)
    torch.cuda.synchronize()
    from trifuse_amd import _lib
    assert blk.status_word() & _lib.TFM_STATUS_BAD_EXPERT_ID
    # The bad routes contribute nothing; the other routes are unchanged.
    g2 = gates.clone()
    g2[0, 3] = 0.0
    g2[1, 0] = 0.0
    ok = idx.clone()
    ok[0, 3] = 0
    ok[1, 0] = 0
    yr = blk.experts(x, ok, g2, wts)
    torch.cuda.synchronize()
    assert max_rel(f32(yb), f32(yr)) <= BLOCK_TOL
    assert blk.status_word() == 0


def test_status_word_is_sticky(gpu):
    """A bad expert id stays reported across later good calls until
    tfm_status_word reads (and clears) the word."""
    from trifuse_amd import _lib

    geom = wl.OLMOE
    log("moe status word: bad call, good calls, then read")
    layer = wl.make_layer(geom, 0, gpu, seed_tag="sticky")
    wts = tmoe.ExpertWeights.from_layer(layer)
    blk = _block(geom)
    for T in (2, 300):  # decode kernels and the prefill grouping
        x = wl.make_x(geom, T, tag=f"sticky{T}").to(gpu)
        _, idx, gates = blk.forward(x, wts, return_routes=True)
        assert blk.status_word() == 0
        bad = idx.clone()
        bad[T - 1, 2] = 99
        blk.experts(x, bad, gates, wts)
        blk.experts(x, idx, gates, wts)      # good call on the same workspace
        blk.forward(x, wts)                  # and a good whole-block call
        torch.cuda.synchronize()
        assert blk.status_word() & _lib.TFM_STATUS_BAD_EXPERT_ID, f"T={T}: bad id lost"
        assert blk.status_word() == 0        # read clears
    # A bad small call, then a larger good call that needs a bigger workspace
    # (the block swaps in a new one), then the read: the bit survives the swap.
    blk = _block(geom)
    x = wl.make_x(geom, 2, tag="sticky_swap").to(gpu)
    _, idx, gates = blk.forward(x, wts, return_routes=True)
    assert blk.status_word() == 0
    small_ws = blk.workspace(2, gpu)
    bad = idx.clone()
    bad[0, 1] = -3
    blk.experts(x, bad, gates, wts)
    xl = wl.make_x(geom, 1024, tag="sticky_swap_big").to(gpu)
    blk.forward(xl, wts)
    assert blk.workspace(1024, gpu).data_ptr() != small_ws.data_ptr()
    torch.cuda.synchronize()
    assert blk.status_word() & _lib.TFM_STATUS_BAD_EXPERT_ID, "bad id lost in the workspace swap"
    assert blk.status_word() == 0


def test_host_mirror_rejects_bad_arguments(gpu):
    """Shape, dtype and device errors raise before any device work."""
    geom = wl.OLMOE
    layer = wl.make_layer(geom, 0, gpu, seed_tag="reject")
    wts = tmoe.ExpertWeights.from_layer(layer)
    blk = _block(geom)
    T, K = 4, geom.top_k
    x = wl.make_x(geom, T, tag="reject").to(gpu)
    _, idx, gates = blk.forward(x, wts, return_routes=True)
    with pytest.raises(ValueError, match="GPU tensor"):
        blk.experts(x, idx.cpu(), gates, wts)
    with pytest.raises(ValueError, match="GPU tensor"):
        blk.experts(x, idx, gates.cpu(), wts)
    with pytest.raises(ValueError, match="gates must be"):
        blk.experts(x, idx, gates[:, :3].contiguous(), wts)
    with pytest.raises(ValueError, match="residual"):
        blk.experts(x, idx, gates, wts, residual=x[:2].contiguous())
    with pytest.raises(ValueError, match="residual"):
        blk.experts(x, idx, gates, wts, residual=x.half())
    with pytest.raises(ValueError, match="router shape"):
        blk.route(x, layer.router[:, :1024].contiguous())
    with pytest.raises(ValueError, match="logit_bias"):
        blk.route(x, layer.router, torch.zeros(geom.experts, device=gpu, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="logit_bias"):
        blk.route(x, layer.router, torch.zeros(geom.experts - 1, device=gpu))
    with pytest.raises(ValueError, match="GPU tensor"):
        blk.expert_routes(x, torch.zeros(8, dtype=torch.int32), idx.reshape(-1)[:8].contiguous(), False, wts)
    with pytest.raises(ValueError, match="GPU tensor"):
        blk.expert_routes(x, torch.zeros(8, dtype=torch.int32, device=gpu), idx.reshape(-1)[:8].cpu(), False,
                          wts)
    # routes but no tokens: the C ABI refuses before reading x
    from trifuse_amd._lib import TfmError
    with pytest.raises(TfmError, match="no tokens"):
        blk.expert_routes(x[:0], torch.zeros(8, dtype=torch.int32, device=gpu),
                          idx.reshape(-1)[:8].contiguous(), False, wts)
