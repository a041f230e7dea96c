"""Affine 4-bit gather_qmm on the GPU (decode GEMV and prefill grouped-GEMM
paths) against the oracle's fp64 product over exactly dequantised weights."""
import numpy as np
import pytest
import torch

import oracle
from tests._util import BLOCK_TOL, log, max_rel, u16, u32
from trifuse_amd import moe as tmoe
from trifuse_amd import workload as wl

pytestmark = pytest.mark.gpu


def _weights(E, N, Kin, key, device):
    q = wl.packed_nibbles((E, N, Kin // 8), key, device)
    s = wl.uniform_scales((E, N, Kin // 64), key + 1, device)
    b = (s.float() * -8.0).to(torch.bfloat16)
    return q, s, b


# (64, 512, 1024) at 257 rows: about 4 rows per expert past the GEMV limit, so
# the grouped GEMM's 64-row tiles of at most 16 rows (weights two super-steps
# ahead) write rows in flat order.
@pytest.mark.parametrize("E,N,Kin", [(5, 128, 256), (3, 1024, 2048), (4, 2048, 1024),
                                     (2, 512, 1536), (2, 1536, 512), (1, 64, 64), (64, 512, 1024)])
@pytest.mark.parametrize("rows", [1, 7, 100, 257, 1500])
def test_gather_qmm_rows(gpu, E, N, Kin, rows):
    log(f"gather_qmm E={E} N={N} Kin={Kin} rows={rows}")
    q, s, b = _weights(E, N, Kin, E * 1000 + N + Kin, gpu)
    X = max(rows // 2, 1)
    x = wl.normal_bf16((X, Kin), 1.0, rows + Kin)
    rng = np.random.default_rng(rows * 31 + N)
    xrows = rng.integers(0, X, size=rows).astype(np.int32)
    rhs = rng.integers(0, E, size=rows).astype(np.int32)
    out = tmoe.gather_qmm_rows(x.to(gpu), q, s, b, torch.from_numpy(rhs).to(gpu),
                               torch.from_numpy(xrows).to(gpu))
    torch.cuda.synchronize()
    ref = oracle.gather_qmm_f64(u16(x), xrows, rhs, u32(q), u16(s), u16(b))
    err = max_rel(oracle.bf16_to_f32(u16(out)), ref)
    log(f"  max_rel {err:.2e}")
    assert err <= BLOCK_TOL


def test_native_affine_gather_qmm_broadcast(gpu):
    log("native_affine_gather_qmm broadcast shapes")
    E, N, Kin, T, K = 6, 256, 512, 5, 3
    q, s, b = _weights(E, N, Kin, 77, gpu)
    x = wl.normal_bf16((1, T, 1, 1, Kin), 1.0, 5).to(gpu)
    idx = torch.from_numpy(np.random.default_rng(3).integers(0, E, size=(1, T, K)).astype(np.int32)).to(gpu)
    out = tmoe.native_affine_gather_qmm(x, q, s, b, idx, 64, 4, False)
    assert tuple(out.shape) == (1, T, K, 1, N)
    xs = u16(x).reshape(T, Kin)
    ii = idx.cpu().numpy().reshape(T, K)
    ref = oracle.gather_qmm_f64(xs, np.repeat(np.arange(T), K), ii.reshape(-1), u32(q), u16(s), u16(b))
    assert max_rel(oracle.bf16_to_f32(u16(out)).reshape(T * K, N), ref) <= BLOCK_TOL
    # sorted layout: x [T*K, 1, H], idx [T*K]
    flat = ii.reshape(-1)
    order = np.argsort(flat, kind="stable")
    xsorted = torch.from_numpy(xs.view(np.int16)[order // K]).view(torch.bfloat16).reshape(T * K, 1, Kin).to(gpu)
    sel = torch.from_numpy(flat[order].astype(np.int32)).to(gpu)
    out2 = tmoe.native_affine_gather_qmm(xsorted, q, s, b, sel, 64, 4, True)
    assert tuple(out2.shape) == (T * K, 1, N)
    np.testing.assert_array_equal(u16(out2).reshape(T * K, N)[np.argsort(order)],
                                  u16(out).reshape(T * K, N))


def test_native_affine_qmm(gpu):
    log("native_affine_qmm")
    N, Kin = 192, 384
    q, s, b = _weights(1, N, Kin, 11, gpu)
    x = wl.normal_bf16((2, 9, Kin), 1.0, 9).to(gpu)
    out = tmoe.native_affine_qmm(x, q[0], s[0], b[0], 64, 4)
    assert tuple(out.shape) == (2, 9, N)
    ref = oracle.gather_qmm_f64(u16(x).reshape(18, Kin), np.arange(18), np.zeros(18, np.int32),
                                u32(q), u16(s), u16(b))
    assert max_rel(oracle.bf16_to_f32(u16(out)).reshape(18, N), ref) <= BLOCK_TOL


# OLMoE q/k/v/o projections (2048 x 2048), its router (64 x 2048) and the
# Granite k/v projection (512 x 1536) at decode and prefill row counts, across
# the GEMV/GEMM switch (176 rows).
@pytest.mark.parametrize("N,Kin", [(2048, 2048), (64, 2048), (512, 1536)])
@pytest.mark.parametrize("rows", [1, 8, 176, 177, 512])
def test_native_affine_qmm_dense_shapes(gpu, N, Kin, rows):
    """tfm_affine_qmm (no grouping pass) against the oracle's fp64 product and
    bit for bit against the grouped one-expert path of tfm_gather_qmm."""
    log(f"native_affine_qmm N={N} Kin={Kin} rows={rows}")
    q, s, b = _weights(1, N, Kin, 7 * N + Kin, gpu)
    x = wl.normal_bf16((rows, Kin), 1.0, rows + N).to(gpu)
    out = tmoe.native_affine_qmm(x, q[0], s[0], b[0], 64, 4)
    grouped = tmoe.gather_qmm_rows(x, q, s, b, torch.zeros(rows, dtype=torch.int32, device=gpu))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(u16(out), u16(grouped))
    sample = np.unique(np.linspace(0, rows - 1, min(rows, 64)).astype(np.int64))
    ref = oracle.gather_qmm_f64(u16(x)[sample], np.arange(sample.size), np.zeros(sample.size, np.int32),
                                u32(q), u16(s), u16(b))
    err = max_rel(oracle.bf16_to_f32(u16(out)[sample]), ref)
    log(f"  max_rel {err:.2e} over {sample.size} rows")
    assert err <= BLOCK_TOL


@pytest.mark.parametrize("dtype,bits", [("f16", 4), ("bf16", 8), ("f16", 8)])
@pytest.mark.parametrize("rows", [1, 300])
def test_native_affine_qmm_dtypes(gpu, dtype, bits, rows):
    """Half storage and 8-bit codes through tfm_affine_qmm (the grouped GEMM at
    every row count) against the oracle."""
    log(f"native_affine_qmm {dtype} bits={bits} rows={rows}")
    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    N, Kin = 1024, 2048
    q = wl.packed_nibbles((N, Kin * bits // 32), 40 + bits, gpu)
    s = wl.uniform_scales((N, Kin // 64), 41, gpu, lo=0.005 * 16 / 2 ** bits, hi=0.02 * 16 / 2 ** bits,
                          dtype=tdt)
    b = (s.float() * -float(2 ** (bits - 1))).to(tdt)
    x = wl.normal_bf16((rows, Kin), 1.0, 42, dtype=tdt).to(gpu)
    out = tmoe.native_affine_qmm(x, q, s, b, 64, bits)
    torch.cuda.synchronize()
    assert out.dtype == tdt
    ref = oracle.gather_qmm_f64(u16(x), np.arange(rows), np.zeros(rows, np.int32), u32(q)[None], u16(s)[None],
                                u16(b)[None], dtype=dtype)
    err = max_rel(oracle.st_to_f32(u16(out), dtype), ref)
    log(f"  max_rel {err:.2e}")
    assert err <= BLOCK_TOL


def test_affine_validation_errors(gpu):
    q, s, b = _weights(2, 64, 128, 1, gpu)
    x = torch.zeros((3, 128), dtype=torch.bfloat16, device=gpu)
    idx = torch.zeros(3, dtype=torch.int32, device=gpu)
    with pytest.raises(ValueError, match="bits4/8"):
        tmoe.native_affine_gather_qmm(x, q, s, b, idx, 16, 4)
    with pytest.raises(ValueError, match="S/B"):
        tmoe.native_affine_gather_qmm(x, q, s, b[:, :, :1], idx, 64, 4)
    with pytest.raises(ValueError, match="expert input"):
        tmoe.native_affine_gather_qmm(x[:, :64], q, s, b, idx, 64, 4)
