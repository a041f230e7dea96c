"""The block with the post-attention RMSNorm fused in (tfm_moe_forward_rmsnorm;
reference MLXNativeGraniteMoEPrefill.h:485-487) on the GPU.

The fused call must equal, bit for bit, the plain block run on the oracle's
RMSNorm of h with h as the residual: every kernel of the block is
deterministic, so this holds only if the GPU's normalised input is the
oracle's bit for bit. Routing is also checked against the oracle's routing of
the normalised input, and the output against the fp64 block reference."""
import numpy as np
import pytest
import torch

import oracle
from tests._util import BLOCK_TOL, bf16_from_u16, log, max_rel, np_layer, u16
from trifuse_amd import moe as tmoe
from trifuse_amd import workload as wl

pytestmark = pytest.mark.gpu


def _norm_weight(H, seed):
    rng = np.random.default_rng(seed)
    return bf16_from_u16(oracle.f32_to_bf16(rng.uniform(0.5, 1.5, H).astype(np.float32)))


@pytest.mark.parametrize("geom_name,T", [("olmoe", 8), ("olmoe", 300), ("granite", 16),
                                         ("granite", 97)])
def test_forward_rmsnorm_is_norm_then_block(gpu, geom_name, T):
    geom = wl.OLMOE if geom_name == "olmoe" else wl.GRANITE
    log(f"forward_rmsnorm {geom_name} T={T}")
    layer = wl.make_layer(geom, 0, gpu, seed_tag=f"rms_{geom_name}")
    wts = tmoe.ExpertWeights.from_layer(layer)
    h = wl.make_x(geom, T, tag=f"rms_h{T}") * 3.0  # un-normalised hidden state
    norm_w = _norm_weight(geom.hidden, T)
    eps = 1e-5
    blk = tmoe.MoEBlock(geom.hidden, geom.intermediate, geom.experts, geom.top_k, route=geom.route)
    hg = h.to(gpu)
    y, idx, gates = blk.forward_rmsnorm(hg, wts, norm_w.to(gpu), eps, return_routes=True)
    torch.cuda.synchronize()

    xn = oracle.rmsnorm(u16(h), u16(norm_w), eps)
    y2 = blk.forward(bf16_from_u16(xn).to(gpu), wts, residual=hg)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)

    lay = np_layer(layer)
    logits = oracle.router_logits(xn, lay.router, lay.logit_bias)
    if geom.route == "olmoe":
        ridx, rg = oracle.route_olmoe(logits, geom.top_k)
        rg = oracle.bf16_to_f32(rg)
    else:
        ridx, rg = oracle.route_granite(logits, geom.top_k)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_array_equal(gates.cpu().numpy().view(np.uint32), rg.view(np.uint32))
    sample = np.unique(np.array([0, T // 2, T - 1], dtype=np.int32))
    ref = oracle.moe_reference(xn, ridx, rg, lay, tokens=sample, residual=u16(h), rm=1.0)
    err = max_rel(oracle.bf16_to_f32(u16(y))[sample], ref)
    log(f"  max_rel {err:.2e}")
    assert err <= BLOCK_TOL


def test_forward_rmsnorm_rejects_bad_arguments(gpu):
    geom = wl.GRANITE
    layer = wl.make_layer(geom, 0, gpu, seed_tag="rms_bad")
    wts = tmoe.ExpertWeights.from_layer(layer)
    blk = tmoe.MoEBlock(geom.hidden, geom.intermediate, geom.experts, geom.top_k, route=geom.route)
    h = wl.make_x(geom, 4, tag="rms_bad").to(gpu)
    with pytest.raises(ValueError):
        blk.forward_rmsnorm(h, wts, torch.ones(geom.hidden - 64, dtype=torch.bfloat16, device=gpu), 1e-5)
    from trifuse_amd._lib import TfmError

    with pytest.raises(TfmError):
        blk.forward_rmsnorm(h, wts, torch.ones(geom.hidden, dtype=torch.bfloat16, device=gpu), -1.0)
    y0 = blk.forward_rmsnorm(h[:0], wts, torch.ones(geom.hidden, dtype=torch.bfloat16, device=gpu), 1e-5)
    assert y0.shape == (0, geom.hidden)
