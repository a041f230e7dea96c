"""A synthetic OLMoE checkpoint in the per-expert export layout
(tests/golden/make_checkpoint.py; F16 scales and biases, affine 4-bit router,
full OLMoE geometry) loaded through trifuse_amd.checkpoint onto the GPU: the
loaded tensors are the file's bytes, and the block built from the
checkpoint's config matches the oracle on them (routing bit-exact, outputs
within max-rel 1e-2 of the fp64 reference over the exactly dequantised
weights), at a decode and a prefill batch."""
import numpy as np
import pytest
import torch

import oracle
from tests._util import BLOCK_TOL, log, max_rel, np_layer, u16
from tests.golden.make_checkpoint import write_checkpoint
from tests.test_gpu_f16 import _routes
from tests.test_gpu_moe import _sample
from trifuse_amd import checkpoint as ck
from trifuse_amd import workload as wl

pytestmark = pytest.mark.gpu

F16 = torch.float16
FIELDS = ("gate_q", "gate_s", "gate_b", "up_q", "up_s", "up_b", "down_q", "down_s", "down_b",
          "router_q", "router_s", "router_b")


def _as_np(t: torch.Tensor) -> np.ndarray:
    return t.numpy().view(np.uint32) if t.dtype == torch.int32 else t.numpy()


@pytest.fixture(scope="module")
def loaded(tmp_path_factory):
    geom = wl.OLMOE
    layer = wl.make_layer(geom, 0, "cpu", seed_tag="ckpt", dtype=F16, affine_router=True)
    arrays = {f: _as_np(getattr(layer, f)) for f in FIELDS}
    d = tmp_path_factory.mktemp("ckpt") / "olmoe"
    write_checkpoint(d, [arrays], geom.hidden, geom.intermediate, geom.top_k)
    c = ck.Checkpoint(d)
    w = c.layer(0, "cuda:0")
    yield geom, layer, c, w
    c.close()


def test_loaded_bytes(gpu, loaded):
    _, layer, _, w = loaded
    log("checkpoint: loaded tensors equal the source layer's bytes")
    for f in FIELDS:
        a, b = getattr(layer, f), getattr(w, f)
        assert b.device.type == "cuda" and b.dtype == a.dtype and b.shape == a.shape, f
        assert torch.equal(b.cpu().view(torch.int16) if b.element_size() == 2 else b.cpu(),
                           a.view(torch.int16) if a.element_size() == 2 else a), f
    assert w.router_bits == 4 and w.router is None


@pytest.mark.parametrize("T", [8, 300])
def test_block_on_loaded_weights(gpu, loaded, T):
    geom, layer, c, w = loaded
    log(f"checkpoint: block forward T={T}")
    blk = c.block()
    assert blk.dtype == F16 and blk.router_kind == "affine"
    x = wl.make_x(geom, T, tag="ckpt_x", dtype=F16)
    res = wl.make_x(geom, T, tag="ckpt_r", dtype=F16)
    gpu_dev = torch.device("cuda:0")
    y, idx, gates = blk.forward(x.to(gpu_dev), w, residual=res.to(gpu_dev), return_routes=True)
    torch.cuda.synchronize()
    lay = np_layer(layer)
    ridx, rg, _ = _routes(geom, u16(x), lay, "f16")
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_array_equal(gates.cpu().numpy().view(np.uint32), rg.view(np.uint32))
    sample = _sample(T, 16)
    ref = oracle.moe_reference(u16(x), ridx, rg, lay, tokens=sample, residual=u16(res), rm=1.0, dtype="f16")
    err = max_rel(oracle.st_to_f32(u16(y), "f16")[sample], ref)
    log(f"  max_rel {err:.2e} over {len(sample)} tokens")
    assert err <= BLOCK_TOL
    blk.close()
