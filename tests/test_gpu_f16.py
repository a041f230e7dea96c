"""IEEE-half storage with the affine-quantised router (the packs TriFuse
ships: F16 scales and biases, export_native_olmoe_target.py:135,160-171,194-202;
export_native_granite_target.py:162-165,231-258) on the GPU: routing bit-exact
against the oracle's half arithmetic, block outputs and gather_qmm within
max-rel 1e-2 of the oracle's fp64 references over exactly dequantised
weights."""
import numpy as np
import pytest
import torch

import oracle
from tests._util import BLOCK_TOL, log, max_rel, np_layer, u16, u32
from tests.test_gpu_moe import _sample
from trifuse_amd import moe as tmoe
from trifuse_amd import workload as wl

pytestmark = pytest.mark.gpu

F16 = torch.float16


def _block(geom, rm=1.0, bits=4, dtype=F16):
    return tmoe.MoEBlock(geom.hidden, geom.intermediate, geom.experts, geom.top_k, route=geom.route,
                         residual_multiplier=rm, bits=bits, dtype=dtype, router="affine")


def _routes(geom, x_u16, lay, dt):
    logits = oracle.router_logits_affine(x_u16, lay.router_q, lay.router_s, lay.router_b,
                                         lay.logit_bias, dtype=dt)
    if geom.route == "olmoe":
        idx, g = oracle.route_olmoe(logits, geom.top_k, dtype=dt)
        return idx, oracle.st_to_f32(g, dt), logits
    idx, g = oracle.route_granite(logits, geom.top_k, dtype=dt)
    return idx, g, logits


def _check(geom, T, bits=4, dtype=F16, rm=1.0, tag="f16", layer_id=0, router_bits=4):
    dt = "f16" if dtype == F16 else "bf16"
    gpu = torch.device("cuda:0")
    layer = wl.make_layer(geom, layer_id, gpu, seed_tag=tag, bits=bits, dtype=dtype, affine_router=True,
                          router_bits=router_bits)
    assert layer.router_bits == router_bits
    x = wl.make_x(geom, T, tag=tag + "_x", dtype=dtype)
    res = wl.make_x(geom, T, tag=tag + "_r", dtype=dtype)
    blk = _block(geom, rm=rm, bits=bits, dtype=dtype)
    y, idx, gates = blk.forward(x.to(gpu), tmoe.ExpertWeights.from_layer(layer), residual=res.to(gpu),
                                return_routes=True)
    torch.cuda.synchronize()
    assert y.dtype == dtype
    lay = np_layer(layer)
    ridx, rg, _ = _routes(geom, u16(x), lay, dt)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_array_equal(gates.cpu().numpy().view(np.uint32), rg.view(np.uint32))
    sample = _sample(T, 24)
    ref = oracle.moe_reference(u16(x), ridx, rg, lay, tokens=sample, residual=u16(res), rm=rm, dtype=dt)
    err = max_rel(oracle.st_to_f32(u16(y), dt)[sample], ref)
    log(f"  max_rel {err:.2e} over {len(sample)} tokens")
    assert err <= BLOCK_TOL
    return blk, layer, x


# 1-3 tokens: streaming kernels; 4 up to E + 40 routes (OLMoE 13 tokens):
# decode GEMV kernels; beyond: grouped GEMM.
@pytest.mark.parametrize("geom_name,T", [("olmoe", 1), ("olmoe", 4), ("olmoe", 8), ("olmoe", 22),
                                         ("olmoe", 23), ("olmoe", 512), ("granite", 1), ("granite", 5),
                                         ("granite", 32), ("granite", 300)])
def test_block_f16_affine_router(gpu, geom_name, T):
    geom = wl.OLMOE if geom_name == "olmoe" else wl.GRANITE
    log(f"moe f16 affine router {geom_name} T={T}")
    _check(geom, T, rm=0.25 if geom_name == "granite" else 1.0)


def test_block_f16_8bit(gpu):
    log("moe f16 8-bit T=64")
    _check(wl.OLMOE, 64, bits=8, tag="f16_8bit")


@pytest.mark.parametrize("dtype", [F16, torch.bfloat16])
@pytest.mark.parametrize("T", [1, 8, 300])
def test_block_8bit_affine_router(gpu, T, dtype):
    """router_bits = 8: four LSB-first byte codes per router word."""
    log(f"moe 8-bit affine router {dtype} T={T}")
    _check(wl.OLMOE, T, dtype=dtype, tag="r8", router_bits=8)


@pytest.mark.parametrize("T", [8, 300])
def test_block_bf16_affine_router(gpu, T):
    log(f"moe bf16 affine router T={T}")
    _check(wl.OLMOE, T, dtype=torch.bfloat16, tag="bf16aff")


def test_f16_hook_and_route_entry_points(gpu):
    geom = wl.OLMOE
    log("f16 hook / route_affine / op mirrors")
    blk, layer, x = _check(geom, 40, tag="f16hook", layer_id=1)
    xg = x.to("cuda:0")
    wts = tmoe.ExpertWeights.from_layer(layer)
    y, idx, gates = blk.forward(xg, wts, return_routes=True)
    y2 = blk.experts(xg, idx, gates, wts)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    # tfm_route_affine: logits bit-equal to the oracle's, routes as the block's
    ridx, rgates, rlogits = blk.route_affine(xg, layer.router_q, layer.router_s, layer.router_b)
    torch.cuda.synchronize()
    lay = np_layer(layer)
    oidx, _, ologits = _routes(geom, u16(x), lay, "f16")
    np.testing.assert_array_equal(u16(rlogits), ologits)
    np.testing.assert_array_equal(ridx.cpu().numpy(), oidx)
    assert rgates.dtype == F16
    # export-time op mirrors on half logits
    probs = tmoe.native_olmoe_softmax(rlogits.unsqueeze(0))
    np.testing.assert_array_equal(u16(probs)[0], oracle.olmoe_softmax(ologits, dtype="f16"))
    top = tmoe.native_olmoe_topk_indices(probs, geom.top_k)
    np.testing.assert_array_equal(top.cpu().numpy()[0], oidx)


def test_gather_qmm_f16(gpu):
    log("gather_qmm f16")
    gpu_dev = torch.device("cuda:0")
    for bits, (E, N, Kin), rows in ((4, (3, 1024, 2048), 300), (8, (2, 512, 1024), 77), (4, (1, 192, 384), 5)):
        per = 32 // bits
        q = wl.packed_nibbles((E, N, Kin // per), 900 + bits, gpu_dev)
        s = wl.uniform_scales((E, N, Kin // 64), 901, gpu_dev, lo=0.005 * 16 / 2 ** bits,
                              hi=0.02 * 16 / 2 ** bits, dtype=F16)
        b = (s.float() * -float(2 ** (bits - 1))).to(F16)
        x = wl.normal_bf16((rows, Kin), 1.0, 902, dtype=F16)
        rhs = np.random.default_rng(rows).integers(0, E, size=rows).astype(np.int32)
        out = tmoe.gather_qmm_rows(x.to(gpu_dev), q, s, b, torch.from_numpy(rhs).to(gpu_dev), bits=bits)
        torch.cuda.synchronize()
        assert out.dtype == F16
        ref = oracle.gather_qmm_f64(u16(x), np.arange(rows), rhs, u32(q), u16(s), u16(b), dtype="f16")
        err = max_rel(oracle.st_to_f32(u16(out), "f16"), ref)
        log(f"  bits={bits} rows={rows} max_rel {err:.2e}")
        assert err <= BLOCK_TOL


def test_forward_rmsnorm_f16(gpu):
    geom = wl.GRANITE
    log("forward_rmsnorm f16")
    gpu_dev = torch.device("cuda:0")
    layer = wl.make_layer(geom, 0, gpu_dev, seed_tag="f16norm", dtype=F16, affine_router=True)
    h = wl.make_x(geom, 48, tag="f16norm_h", dtype=F16)
    nw = wl.normal_bf16((geom.hidden,), 0.1, 77, dtype=F16) + 1.0
    blk = _block(geom, rm=0.25)
    y, idx, gates = blk.forward_rmsnorm(h.to(gpu_dev), tmoe.ExpertWeights.from_layer(layer),
                                        nw.to(gpu_dev), 1e-6, return_routes=True)
    torch.cuda.synchronize()
    post = oracle.rmsnorm(u16(h), u16(nw), 1e-6, dtype="f16")
    lay = np_layer(layer)
    ridx, rg, _ = _routes(geom, post, lay, "f16")
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    sample = _sample(48, 12)
    ref = oracle.moe_reference(post, ridx, rg, lay, tokens=sample, residual=u16(h), rm=0.25, dtype="f16")
    assert max_rel(oracle.st_to_f32(u16(y), "f16")[sample], ref) <= BLOCK_TOL


def test_f16_decode_paths_agree(gpu):
    # Half blocks take the streaming kernels up to three tokens and the decode
    # GEMV kernels from four (as bf16 blocks do): the hook (given routes)
    # matches the whole block bit for bit, one or two tokens (the fused
    # down + combine) match the same tokens inside a three-token batch, and the
    # three-token batch matches the same tokens of an eight-token batch (the
    # other kernel family) within the block tolerance.
    geom = wl.OLMOE
    log("f16 decode hook / small-batch agreement")
    gpu_dev = torch.device("cuda:0")
    layer = wl.make_layer(geom, 3, gpu_dev, seed_tag="f16dec", dtype=F16, affine_router=True)
    wts = tmoe.ExpertWeights.from_layer(layer)
    blk = _block(geom, rm=0.5)
    x = wl.make_x(geom, 8, tag="f16dec_x", dtype=F16).to(gpu_dev)
    res = wl.make_x(geom, 8, tag="f16dec_r", dtype=F16).to(gpu_dev)
    y8, idx, gates = blk.forward(x, wts, residual=res, return_routes=True)
    y8h = blk.experts(x, idx, gates, wts, residual=res)
    y3 = blk.forward(x[:3].contiguous(), wts, residual=res[:3].contiguous())
    y2 = blk.forward(x[:2].contiguous(), wts, residual=res[:2].contiguous())
    y1 = blk.forward(x[:1].contiguous(), wts, residual=res[:1].contiguous())
    torch.cuda.synchronize()
    assert torch.equal(y8, y8h)
    assert torch.equal(y2, y3[:2]) and torch.equal(y1, y3[:1])
    a = oracle.st_to_f32(u16(y3), "f16").astype(np.float64)
    b = oracle.st_to_f32(u16(y8[:3]), "f16").astype(np.float64)
    assert max_rel(a, b) <= BLOCK_TOL


@pytest.mark.parametrize("T", [4, 300])
def test_f16_expert_routes_callable(gpu, T):
    # NativeMoEExpertHook::GPUCallable with half storage: expert-sorted rows
    # whose gate-weighted sum per token is the block's output.
    geom = wl.OLMOE
    log(f"f16 expert_routes T={T}")
    gpu_dev = torch.device("cuda:0")
    layer = wl.make_layer(geom, 4, gpu_dev, seed_tag="f16routes", dtype=F16, affine_router=True)
    wts = tmoe.ExpertWeights.from_layer(layer)
    blk = _block(geom)
    x = wl.make_x(geom, T, tag="f16routes_x", dtype=F16).to(gpu_dev)
    y, idx, gates = blk.forward(x, wts, return_routes=True)
    N = T * geom.top_k
    tok = torch.arange(N, device=gpu_dev, dtype=torch.int32) // geom.top_k
    out, inv = blk.expert_routes(x, tok, idx.reshape(-1), False, wts)
    torch.cuda.synchronize()
    assert out.dtype == F16
    order = np.argsort(idx.cpu().numpy().reshape(-1), kind="stable")
    np.testing.assert_array_equal(inv.cpu().numpy(), np.argsort(order))
    rows = oracle.st_to_f32(u16(out), "f16")[inv.cpu().numpy()]
    comb = (rows * gates.cpu().numpy().reshape(-1)[:, None]).reshape(T, geom.top_k, -1).sum(1)
    assert max_rel(comb, oracle.st_to_f32(u16(y), "f16")) <= BLOCK_TOL
