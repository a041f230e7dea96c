"""8-bit affine weights (native_affine_ops.py:29-36 with bits = 8: four
LSB-first byte codes per uint32 word) on the GPU: gather_qmm, the dense
quantized matmul and the whole MoE block against the oracle's fp64
references over exactly dequantised weights, routing bit-exact."""
import numpy as np
import pytest
import torch

import oracle
from tests._util import BLOCK_TOL, log, max_rel, np_layer, u16, u32
from tests.test_gpu_moe import _oracle_routes, _sample
from trifuse_amd import moe as tmoe
from trifuse_amd import workload as wl

pytestmark = pytest.mark.gpu


def _weights8(E, N, Kin, key, device):
    q = wl.packed_nibbles((E, N, Kin // 4), key, device)
    s = wl.uniform_scales((E, N, Kin // 64), key + 1, device, lo=0.005 / 16, hi=0.02 / 16)
    b = (s.float() * -128.0).to(torch.bfloat16)
    return q, s, b


@pytest.mark.parametrize("E,N,Kin", [(5, 128, 256), (3, 1024, 2048), (2, 1536, 512), (1, 64, 64)])
@pytest.mark.parametrize("rows", [1, 7, 257, 1500])
def test_gather_qmm_8bit(gpu, E, N, Kin, rows):
    log(f"gather_qmm 8-bit E={E} N={N} Kin={Kin} rows={rows}")
    q, s, b = _weights8(E, N, Kin, E * 1000 + N + Kin, gpu)
    X = max(rows // 2, 1)
    x = wl.normal_bf16((X, Kin), 1.0, rows + Kin)
    rng = np.random.default_rng(rows * 37 + N)
    xrows = rng.integers(0, X, size=rows).astype(np.int32)
    rhs = rng.integers(0, E, size=rows).astype(np.int32)
    out = tmoe.gather_qmm_rows(x.to(gpu), q, s, b, torch.from_numpy(rhs).to(gpu),
                               torch.from_numpy(xrows).to(gpu), bits=8)
    torch.cuda.synchronize()
    ref = oracle.gather_qmm_f64(u16(x), xrows, rhs, u32(q), u16(s), u16(b))
    err = max_rel(oracle.bf16_to_f32(u16(out)), ref)
    log(f"  max_rel {err:.2e}")
    assert err <= BLOCK_TOL
    # Read as 4-bit codes the same words give a different product: the test
    # tells the two layouts apart.
    q4 = u32(q)[:, :, : Kin // 8]
    wrong = oracle.gather_qmm_f64(u16(x), xrows, rhs, q4, u16(s), u16(b))
    assert max_rel(oracle.bf16_to_f32(u16(out)), wrong) > 0.1


def test_native_affine_qmm_8bit(gpu):
    log("native_affine_qmm 8-bit")
    N, Kin = 192, 384
    q, s, b = _weights8(1, N, Kin, 13, gpu)
    x = wl.normal_bf16((3, 7, Kin), 1.0, 13).to(gpu)
    out = tmoe.native_affine_qmm(x, q[0], s[0], b[0], 64, 8)
    assert tuple(out.shape) == (3, 7, N)
    ref = oracle.gather_qmm_f64(u16(x).reshape(21, Kin), np.arange(21), np.zeros(21, np.int32),
                                u32(q), u16(s), u16(b))
    assert max_rel(oracle.bf16_to_f32(u16(out)).reshape(21, N), ref) <= BLOCK_TOL


def _block8(geom, rm=1.0):
    return tmoe.MoEBlock(geom.hidden, geom.intermediate, geom.experts, geom.top_k, route=geom.route,
                         residual_multiplier=rm, bits=8)


@pytest.mark.parametrize("geom_name,T", [("olmoe", 1), ("olmoe", 8), ("olmoe", 512),
                                         ("granite", 5), ("granite", 300)])
def test_block_8bit_against_oracle(gpu, geom_name, T):
    geom = wl.OLMOE if geom_name == "olmoe" else wl.GRANITE
    log(f"moe 8-bit {geom_name} T={T}")
    layer = wl.make_layer(geom, 0, gpu, seed_tag="eightbit", bits=8)
    x = wl.make_x(geom, T, tag="eightbit_x")
    residual = wl.make_x(geom, T, tag="eightbit_r")
    rm = 0.25 if geom_name == "granite" else 1.0
    blk = _block8(geom, rm=rm)
    y, idx, gates = blk.forward(x.to(gpu), tmoe.ExpertWeights.from_layer(layer),
                                residual=residual.to(gpu), return_routes=True)
    torch.cuda.synchronize()
    lay = np_layer(layer)
    ridx, rg = _oracle_routes(geom, u16(x), lay)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_array_equal(gates.cpu().numpy().view(np.uint32), rg.view(np.uint32))
    sample = _sample(T, 24)
    ref = oracle.moe_reference(u16(x), ridx, rg, lay, tokens=sample, residual=u16(residual), rm=rm)
    err = max_rel(oracle.bf16_to_f32(u16(y))[sample], ref)
    log(f"  max_rel {err:.2e} over {len(sample)} tokens")
    assert err <= BLOCK_TOL


def test_block_8bit_hook_and_determinism(gpu):
    # Given routes (NativeMoEExpertHook::execute) take the same kernels as the
    # whole block, and the deterministic flag changes nothing for 8-bit.
    geom = wl.OLMOE
    log("moe 8-bit hook")
    layer = wl.make_layer(geom, 1, gpu, seed_tag="eightbit", bits=8)
    wts = tmoe.ExpertWeights.from_layer(layer)
    blk = _block8(geom)
    x = wl.make_x(geom, 40, tag="eightbit_hook").to(gpu)
    y, idx, gates = blk.forward(x, wts, return_routes=True)
    y2 = blk.experts(x, idx, gates, wts)
    y3 = blk.forward(x, wts, deterministic=True)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    assert torch.equal(y, y3)


def test_block_8bit_rejects_4bit_weights(gpu):
    geom = wl.OLMOE
    layer = wl.make_layer(geom, 0, gpu, seed_tag="eightbit_mismatch")
    x = wl.make_x(geom, 2, tag="eightbit_mismatch").to(gpu)
    with pytest.raises(ValueError, match="shape"):
        _block8(geom).forward(x, tmoe.ExpertWeights.from_layer(layer))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_8bit_decode_paths_agree(gpu, dtype):
    # At decode shapes 8-bit blocks take the streaming kernels (each byte code
    # dotted as its two nibbles): against the oracle at eight tokens, the hook
    # equal to the whole block, and one or two tokens equal to the same tokens
    # of a three-token batch.
    geom = wl.OLMOE
    dt = "f16" if dtype == torch.float16 else "bf16"
    log(f"8-bit decode agreement {dt}")
    layer = wl.make_layer(geom, 2, gpu, seed_tag="eightdec", bits=8, dtype=dtype,
                          affine_router=dtype == torch.float16)
    wts = tmoe.ExpertWeights.from_layer(layer)
    blk = tmoe.MoEBlock(geom.hidden, geom.intermediate, geom.experts, geom.top_k, route=geom.route,
                        residual_multiplier=0.5, bits=8, dtype=dtype,
                        router="affine" if dtype == torch.float16 else "dense")
    x = wl.make_x(geom, 8, tag="eightdec_x", dtype=dtype).to(gpu)
    res = wl.make_x(geom, 8, tag="eightdec_r", dtype=dtype).to(gpu)
    y8, idx, gates = blk.forward(x, wts, residual=res, return_routes=True)
    y8h = blk.experts(x, idx, gates, wts, residual=res)
    y3 = blk.forward(x[:3].contiguous(), wts, residual=res[:3].contiguous())
    y2 = blk.forward(x[:2].contiguous(), wts, residual=res[:2].contiguous())
    y1 = blk.forward(x[:1].contiguous(), wts, residual=res[:1].contiguous())
    torch.cuda.synchronize()
    assert torch.equal(y8, y8h)
    assert torch.equal(y2, y3[:2]) and torch.equal(y1, y3[:1]) and torch.equal(y3, y8[:3])
    lay = np_layer(layer)
    ref = oracle.moe_reference(u16(x), idx.cpu().numpy(), gates.cpu().numpy(), lay, residual=u16(res),
                               rm=0.5, dtype=dt)
    err = max_rel(oracle.st_to_f32(u16(y8), dt), ref)
    log(f"  max_rel {err:.2e}")
    assert err <= BLOCK_TOL
