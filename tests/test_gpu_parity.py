"""Parity margins against both CPU references, per benchmark configuration,
and the hook's GPUCallable checked route by route against the oracle.

1. The whole block at every benchmark configuration against
   * the oracle's fp64 block (exactly dequantised weights, h and the expert
     outputs unrounded; the tolerance reference), and
   * the oracle's MLX-semantics CPU block (orc_moe_block_cpu), which rounds
     where the reference's graph rounds: gate and up to the activation dtype
     before the SwiGLU and h after it (MLXNativeGraniteMoEPrefill.h:685-687),
     each expert output, and the OLMoE combine's products in the activation
     dtype (:690-694; Granite: fp32 products, one rounding, :54-70).
   Routing is identical on all three; both margins are reported and bounded
   by max-rel 1e-2. With TFM_PARITY_OUT set, each margin is appended there as
   one JSON line.
2. NativeMoEExpertHook::GPUCallable (MLXMoEExpertHook.h:23-30;
   MLXNativeGraniteMoEPrefill.h:635-658): every expert-sorted output row
   against the oracle's per-route chain (fp64 gate and up products of the
   route's token row with its expert, SwiGLU, fp64 down product), with
   caller-order and expert-sorted routes, bf16 and half storage, N = 8 (GEMV
   kernels) and N = 2400 (grouped GEMM)."""
import json
import os

import numpy as np
import pytest
import torch

import oracle
from tests._util import BLOCK_TOL, log, max_rel, np_layer, u16
from trifuse_amd import moe as tmoe
from trifuse_amd import workload as wl

pytestmark = pytest.mark.gpu


def _record(**kw):
    path = os.environ.get("TFM_PARITY_OUT")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(kw) + "\n")


def _elem_rel(y, ref):
    """Largest element-wise relative error over the elements whose reference
    magnitude is above 1e-3 of the largest."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    big = np.abs(ref) > 1e-3 * np.max(np.abs(ref))
    return float(np.max(np.abs(y[big] - ref[big]) / np.abs(ref[big])))


# (workload, layers checked)
CONFIGS = [
    ("olmoe_decode_t1", (0,)),
    ("olmoe_decode_t8_x16", (0, 15)),
    ("olmoe_prefill_t512", (0,)),
    ("olmoe_prefill_t4096_zipf", (0,)),
    ("granite_prefill_t2048", (0,)),
    ("granite_decode_t32", (0,)),
    ("olmoe_decode_t8_x16_int8", (0,)),
    ("olmoe_prefill_t512_int8", (0,)),
]


@pytest.mark.parametrize("name,layers", CONFIGS, ids=[c[0] for c in CONFIGS])
def test_block_margins_against_both_references(gpu, name, layers):
    w = wl.WORKLOADS[name]
    geom = w.geometry
    blk = tmoe.MoEBlock(geom.hidden, geom.intermediate, geom.experts, geom.top_k, route=geom.route,
                        bits=w.bits)
    x = wl.workload_x(w)
    xu = u16(x)
    for l in layers:
        log(f"parity margins {name} layer {l}")
        layer = wl.workload_layer(w, l, gpu)
        y, idx, gates = blk.forward(x.to(gpu), tmoe.ExpertWeights.from_layer(layer), return_routes=True)
        torch.cuda.synchronize()
        lay = np_layer(layer)
        del layer
        cy, cidx, cgates, threads = oracle.moe_block_cpu(xu, lay, geom.route, lay.router, lay.logit_bias,
                                                         top_k=geom.top_k)
        # routing: GPU, MLX-semantics CPU block and the oracle's routes agree bit for bit
        np.testing.assert_array_equal(idx.cpu().numpy(), cidx)
        np.testing.assert_array_equal(gates.cpu().numpy().view(np.uint32), cgates.view(np.uint32))
        ref = oracle.moe_reference_full(xu, cidx, cgates, lay)
        got = oracle.bf16_to_f32(u16(y)).astype(np.float64)
        cpu = oracle.bf16_to_f32(cy).astype(np.float64)
        m = dict(workload=name, layer=l, tokens=w.tokens, bits=w.bits,
                 gpu_vs_fp64=max_rel(got, ref), cpu_block_vs_fp64=max_rel(cpu, ref),
                 gpu_vs_cpu_block=max_rel(got, cpu), gpu_vs_fp64_elem=_elem_rel(got, ref),
                 cpu_block_vs_fp64_elem=_elem_rel(cpu, ref), gpu_vs_cpu_block_elem=_elem_rel(got, cpu),
                 routes_identical=True)
        log("  " + " ".join(f"{k}={v:.2e}" for k, v in m.items() if isinstance(v, float)))
        _record(**m)
        assert m["gpu_vs_fp64"] <= BLOCK_TOL
        assert m["gpu_vs_cpu_block"] <= BLOCK_TOL
        assert m["cpu_block_vs_fp64"] <= BLOCK_TOL


def _routes_reference(x64, tok, eid, lay, dtype):
    """fp64 per-route chain: row i = swiglu(x[tok[i]] . Wg[e]^T, x[tok[i]] . Wu[e]^T) . Wd[e]^T,
    e = eid[i], weights dequantised exactly by the oracle."""
    H = x64.shape[1]
    out = np.zeros((tok.size, H), dtype=np.float64)
    for e in np.unique(eid):
        r = np.nonzero(eid == e)[0]
        wg = oracle.dequant_f64(lay.gate_q[e], lay.gate_s[e], lay.gate_b[e], dtype=dtype)
        wu = oracle.dequant_f64(lay.up_q[e], lay.up_s[e], lay.up_b[e], dtype=dtype)
        wd = oracle.dequant_f64(lay.down_q[e], lay.down_s[e], lay.down_b[e], dtype=dtype)
        xe = x64[tok[r]]
        a = xe @ wg.T
        h = a / (1.0 + np.exp(-a)) * (xe @ wu.T)
        out[r] = h @ wd.T
    return out


# N = 8: decode GEMV kernels; 300 (about 5 routes per expert): the grouped
# GEMM's 64-row tiles, with bf16 the few-row instance; 2400: larger tiles.
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("N", [8, 300, 2400])
def test_gpu_callable_rows_against_oracle(gpu, dtype, N):
    geom = wl.OLMOE
    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    blk = tmoe.MoEBlock(geom.hidden, geom.intermediate, geom.experts, geom.top_k, route=geom.route,
                        dtype=tdt, router="affine" if dtype == "f16" else "dense")
    layer = wl.make_layer(geom, 0, gpu, seed_tag="callable", dtype=tdt, affine_router=dtype == "f16")
    wts = tmoe.ExpertWeights.from_layer(layer)
    lay = np_layer(layer)
    T = 300
    x = wl.make_x(geom, T, tag="callable_x", dtype=tdt)
    x64 = oracle.st_to_f32(u16(x), dtype).astype(np.float64)
    rng = np.random.default_rng(N)
    tok = rng.integers(0, T, size=N).astype(np.int32)
    eid = rng.integers(0, geom.experts, size=N).astype(np.int32)
    if N >= geom.experts:
        eid[:geom.experts] = np.arange(geom.experts)  # every expert has a route
    ref = _routes_reference(x64, tok, eid, lay, dtype)
    xg = x.to(gpu)
    for experts_sorted in (False, True):
        log(f"GPUCallable {dtype} N={N} experts_sorted={experts_sorted}")
        if experts_sorted:
            perm = np.argsort(eid, kind="stable")
            t_in, e_in, r_in = tok[perm], eid[perm], ref[perm]
        else:
            t_in, e_in, r_in = tok, eid, ref
        out, inv = blk.expert_routes(xg, torch.from_numpy(t_in).to(gpu), torch.from_numpy(e_in).to(gpu),
                                     experts_sorted, wts)
        torch.cuda.synchronize()
        inv = inv.cpu().numpy()
        # inverse: route i's row sits at the route's stable expert-sorted position
        np.testing.assert_array_equal(inv, np.argsort(np.argsort(e_in, kind="stable"), kind="stable"))
        if experts_sorted:
            np.testing.assert_array_equal(inv, np.arange(N))
        rows = oracle.st_to_f32(u16(out), dtype).astype(np.float64)
        got = rows[inv]  # route order
        err = max_rel(got, r_in)
        per_row = float(np.max(np.max(np.abs(got - r_in), axis=1) / np.max(np.abs(r_in), axis=1)))
        log(f"  max_rel {err:.2e} (worst row {per_row:.2e}) over {N} routes")
        _record(workload=f"gpu_callable_{dtype}_n{N}", experts_sorted=experts_sorted, routes=N,
                gpu_vs_fp64=err, worst_row=per_row)
        assert err <= BLOCK_TOL
        assert per_row <= 2 * BLOCK_TOL
