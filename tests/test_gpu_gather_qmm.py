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


@pytest.mark.parametrize("E,N,Kin", [(5, 128, 256), (3, 1024, 2048), (4, 2048, 1024),
                                     (2, 512, 1536), (2, 1536, 512), (1, 64, 64)])
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
