"""Pins the oracle's IEEE-half storage (the f16 packs TriFuse ships,
export_native_olmoe_target.py:135, export_native_granite_target.py:162-165)
and its affine-quantised router on the host, independently of its own code:
half rounding against numpy and torch, the dequantised router weight against
numpy's half arithmetic, softmax and top-k against float64 and the reference's
torch bodies, and planted mistakes that must fail the same checks."""
import numpy as np
import pytest
import torch

import oracle
from tests.test_oracle import stable_topk_desc_nan_last

RNG = np.random.default_rng(20261202)


def h(x):
    """float -> half bits by numpy (round to nearest even)."""
    with np.errstate(over="ignore"):
        return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def fh(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float64)


def test_half_rounding_matches_numpy_and_torch():
    x = np.concatenate([
        RNG.standard_normal(200000).astype(np.float32) * 100,
        RNG.standard_normal(50000).astype(np.float32) * 1e-6,      # half subnormals
        (RNG.random(20000).astype(np.float32) - 0.5) * 1e-7,       # around 2^-24 and below
        np.array([0.0, -0.0, 1.0, 65504.0, 65519.0, 65520.0, -65520.0, 1e6, np.inf, -np.inf,
                  2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 3 * 2.0 ** -26, 2.0 ** -14,
                  1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, 6.1e-5], dtype=np.float32),
    ])
    ours = oracle.f32_to_f16(x)
    np.testing.assert_array_equal(ours, h(x))
    theirs = torch.from_numpy(x).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, theirs)
    assert oracle.f32_to_f16(np.array([1 + 2.0 ** -11], np.float32))[0] == 0x3C00  # tie to even
    assert oracle.f32_to_f16(np.array([65520.0], np.float32))[0] == 0x7C00        # overflow
    assert oracle.f32_to_f16(np.array([2.0 ** -25], np.float32))[0] == 0x0000     # tie to zero
    assert np.isnan(oracle.f16_to_f32(oracle.f32_to_f16(np.array([np.nan], np.float32))))[0]
    # widening is exact for every half value
    allh = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_to_f32(allh)
    ref = allh.view(np.float16).astype(np.float32)
    fin = ~np.isnan(ref)
    np.testing.assert_array_equal(got[fin], ref[fin])
    assert np.all(np.isnan(got[~fin]))


def _router(E, H, bits=4):
    per = 32 // bits
    q = RNG.integers(0, 2 ** 32, size=(E, H // per), dtype=np.uint64).astype(np.uint32)
    s = h(RNG.uniform(0.002, 0.006, size=(E, H // 64)))
    b = h(-(2 ** (bits - 1)) * fh(s))
    return q, s, b


def _np_router_weight(q, s, b, bits=4, msb_first=False):
    """Dequantised router rounded to half (native_affine_ops.py:29-36 with
    half scales): s*q is exact in float32, so one float32 add then one half
    rounding is what fmaf + rounding gives."""
    per = 32 // bits
    shifts = np.arange(per, dtype=np.uint32) * bits
    if msb_first:
        shifts = shifts[::-1]
    codes = ((q[..., None] >> shifts) & ((1 << bits) - 1)).reshape(q.shape[0], -1).astype(np.float32)
    sf = np.repeat(fh(s).astype(np.float32), 64, -1)
    bf_ = np.repeat(fh(b).astype(np.float32), 64, -1)
    return fh(h(sf * codes + bf_))


@pytest.mark.parametrize("bits", [4, 8])
def test_affine_router_one_hot_exact_and_tolerance(bits):
    E, H = 64, 2048
    q, s, b = _router(E, H, bits)
    w = _np_router_weight(q, s, b, bits)
    sel = RNG.choice(H, 9, replace=False)
    x = h(np.eye(H, dtype=np.float32)[sel])
    got = oracle.router_logits_affine(x, q, s, b, dtype="f16")
    np.testing.assert_array_equal(fh(got), w[:, sel].T)  # exactly the rounded weight
    bias = RNG.standard_normal(E).astype(np.float32)
    got_b = oracle.router_logits_affine(x, q, s, b, bias, dtype="f16")
    np.testing.assert_array_equal(got_b, h(w[:, sel].T.astype(np.float32) + bias))
    # general rows: within one half rounding of the float64 product
    xr = h(RNG.standard_normal((16, H)))
    ref = fh(xr) @ w.T
    gotr = fh(oracle.router_logits_affine(xr, q, s, b, dtype="f16"))
    assert np.max(np.abs(gotr - ref) / np.maximum(np.abs(ref), 1e-2)) < 2 ** -9
    # planted mistakes: MSB-first codes, the transposed router, bf16 reading
    wm = _np_router_weight(q, s, b, bits, msb_first=True)
    assert not np.array_equal(fh(got), wm[:, sel].T)
    assert np.max(np.abs(gotr - fh(xr)[:, :E] @ w[:, :E])) > 1e-2
    assert not np.array_equal(oracle.router_logits_affine(xr, q, s, b, dtype="bf16"),
                              oracle.router_logits_affine(xr, q, s, b, dtype="f16"))


def test_affine_router_bf16_matches_dense_router_on_exact_weights():
    # With bf16 storage and weights that dequantise exactly (s a power of two,
    # b = -8 s), the affine router is the dense router on the dequantised
    # matrix, bit for bit: same order, same rounding.
    E, H = 40, 1536
    q = RNG.integers(0, 2 ** 32, size=(E, H // 8), dtype=np.uint64).astype(np.uint32)
    s = oracle.f32_to_bf16(np.full((E, H // 64), 2.0 ** -6, np.float32))
    b = oracle.f32_to_bf16(np.full((E, H // 64), -8 * 2.0 ** -6, np.float32))
    wd = oracle.f32_to_bf16(oracle.dequant_f64(q, s, b).astype(np.float32))
    x = oracle.f32_to_bf16(RNG.standard_normal((12, H)).astype(np.float32))
    np.testing.assert_array_equal(oracle.router_logits_affine(x, q, s, b),
                                  oracle.router_logits(x, wd))


def test_olmoe_softmax_half_close_to_float64():
    lg = h(RNG.standard_normal((500, 64)) * 2)
    p = fh(oracle.olmoe_softmax(lg, dtype="f16"))
    x = fh(lg)
    ref = np.exp(x - x.max(1, keepdims=True))
    ref /= ref.sum(1, keepdims=True)
    # one half rounding, absolute for subnormal probabilities
    assert np.all(np.abs(p - ref) <= np.maximum(ref * 2 ** -11, 2 ** -25) * 1.01)
    # the torch body of native_olmoe_softmax (native_affine_ops.py:131) agrees to one half ulp
    tp = torch.softmax(torch.from_numpy(x.astype(np.float32)), -1).to(torch.float16).double().numpy()
    assert np.all(np.abs(p - tp) <= np.maximum(tp * 2 ** -10, 2 ** -24))


@pytest.mark.parametrize("E,K", [(64, 8), (40, 8), (7, 3)])
def test_routes_on_half_logits(E, K):
    v = RNG.integers(-6, 6, size=(64, E)).astype(np.float32) * 0.25
    v[1, 3 % E] = np.nan
    for lg in (h(v), h(RNG.standard_normal((300, E)))):
        idx, gates = oracle.route_olmoe(lg, K, dtype="f16")
        p = oracle.olmoe_softmax(lg, dtype="f16")
        np.testing.assert_array_equal(idx, stable_topk_desc_nan_last(fh(p), K))
        np.testing.assert_array_equal(gates, np.take_along_axis(p, idx.astype(np.int64), 1))
        gi, gg = oracle.route_granite(lg, K, dtype="f16")
        w = fh(lg)
        order = np.array([np.lexsort((np.where(np.isnan(r), 0, r), np.isnan(r))) for r in w])
        np.testing.assert_array_equal(gi, order[:, E - K:])
        sel = np.take_along_axis(w, gi.astype(np.int64), 1)
        fin = np.all(np.isfinite(sel), 1)
        ref = np.exp(sel[fin] - sel[fin].max(1, keepdims=True))
        ref /= ref.sum(1, keepdims=True)
        np.testing.assert_allclose(gg[fin], ref, rtol=3e-6, atol=1e-7)
    # planted mistake: reading half logits as bf16 changes the routes
    lg = h(RNG.standard_normal((50, E)))
    assert not np.array_equal(oracle.route_olmoe(lg, K, dtype="f16")[0], oracle.route_olmoe(lg, K)[0])


def test_dequant_and_gather_with_half_scales():
    E, N, Kin = 2, 16, 256
    q = RNG.integers(0, 2 ** 32, size=(E, N, Kin // 8), dtype=np.uint64).astype(np.uint32)
    s = h(RNG.uniform(0.005, 0.02, size=(E, N, Kin // 64)))
    b = h(-8 * fh(s))
    codes = ((q[..., None] >> (np.arange(8, dtype=np.uint32) * 4)) & 0xF).reshape(E, N, Kin)
    w = codes * np.repeat(fh(s), 64, -1) + np.repeat(fh(b), 64, -1)
    np.testing.assert_array_equal(oracle.dequant_f64(q[1], s[1], b[1], dtype="f16"), w[1])
    assert not np.array_equal(oracle.dequant_f64(q[1], s[1], b[1]), w[1])  # bf16 reading differs
    x = h(RNG.standard_normal((5, Kin)))
    xrow = np.array([0, 4, 2], np.int32)
    eid = np.array([1, 0, 1], np.int32)
    got = oracle.gather_qmm_f64(x, xrow, eid, q, s, b, dtype="f16")
    for r in range(3):
        np.testing.assert_allclose(got[r], w[eid[r]] @ fh(x[xrow[r]]), rtol=1e-12, atol=1e-12)


def test_rmsnorm_half_exact_cases_and_tolerance():
    H = 2048
    w = h(RNG.uniform(0.5, 1.5, H))
    x = h(RNG.standard_normal((6, H)) * RNG.uniform(0.1, 8.0, (6, 1)))
    got = fh(oracle.rmsnorm(x, w, 1e-5, dtype="f16"))
    xf, wf = fh(x), fh(w)
    ref = xf / np.sqrt((xf ** 2).mean(1, keepdims=True) + 1e-5) * wf
    assert np.max(np.abs(got - ref) / np.abs(ref)) < 2 * 2 ** -10
    xc = h(np.stack([np.full(H, 0.5), np.full(H, -4.0)]))
    out = oracle.rmsnorm(xc, w, 0.0, dtype="f16")
    np.testing.assert_array_equal(out[0], w)
    np.testing.assert_array_equal(out[1], w ^ np.uint16(0x8000))


def test_moe_reference_with_half_storage():
    E, H, I, T, K = 3, 128, 64, 5, 2

    class W:
        pass

    w = W()
    deq = {}
    for proj, (N, Kin) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
        q = RNG.integers(0, 2 ** 32, size=(E, N, Kin // 8), dtype=np.uint64).astype(np.uint32)
        sc = h(RNG.uniform(0.005, 0.02, size=(E, N, Kin // 64)))
        bi = h(-8 * fh(sc))
        setattr(w, proj + "_q", q)
        setattr(w, proj + "_s", sc)
        setattr(w, proj + "_b", bi)
        codes = ((q[..., None] >> (np.arange(8, dtype=np.uint32) * 4)) & 0xF).reshape(E, N, Kin)
        deq[proj] = codes * np.repeat(fh(sc), 64, -1) + np.repeat(fh(bi), 64, -1)
    x = h(RNG.standard_normal((T, H)))
    res = h(RNG.standard_normal((T, H)))
    idx = RNG.integers(0, E, (T, K)).astype(np.int32)
    gates = RNG.random((T, K)).astype(np.float32)
    got = oracle.moe_reference(x, idx, gates, w, residual=res, rm=0.5, dtype="f16")
    ref = np.zeros((T, H))
    for t in range(T):
        for k in range(K):
            e = idx[t, k]
            g = deq["gate"][e] @ fh(x[t])
            u = deq["up"][e] @ fh(x[t])
            ref[t] += gates[t, k] * (deq["down"][e] @ (g / (1 + np.exp(-g)) * u))
    ref = 0.5 * ref + fh(res)
    np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-10)
    assert not np.allclose(oracle.moe_reference(x, idx, gates, w, residual=res, rm=0.5), ref)
