"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and the cpu_baseline
leg of bench.py use it as the checker (or, for the baseline, as the CPU work
being timed). The product library never loads it.

Arrays are numpy: bf16 values travel as uint16 bit patterns, packed weights
as uint32 (int32 arrays are reinterpreted).
"""
from __future__ import annotations

import ctypes
import subprocess
from ctypes import c_float, c_int, c_int64, c_void_p
from pathlib import Path
from typing import Optional

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        lib = ctypes.CDLL(str(LIB))
        lib.orc_bf16_to_f32.restype = c_float
        lib.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        lib.orc_f32_to_bf16.restype = ctypes.c_uint16
        lib.orc_f32_to_bf16.argtypes = [c_float]
        lib.orc_expf.restype = c_float
        lib.orc_expf.argtypes = [c_float]
        lib.orc_moe_block_cpu.restype = c_int
        lib.orc_group.restype = c_int
        _lib = lib
    return _lib


def _p(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(c_void_p)


def _u16(a) -> np.ndarray:
    a = np.asarray(a)
    if a.dtype == np.int16:
        a = a.view(np.uint16)
    assert a.dtype == np.uint16, a.dtype
    return np.ascontiguousarray(a)


def _u32(a) -> np.ndarray:
    a = np.asarray(a)
    if a.dtype == np.int32:
        a = a.view(np.uint32)
    assert a.dtype == np.uint32, a.dtype
    return np.ascontiguousarray(a)


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


def bf16_to_f32(h) -> np.ndarray:
    h = _u16(h)
    return (h.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f) -> np.ndarray:
    f = np.ascontiguousarray(np.asarray(f, dtype=np.float32))
    out = np.empty(f.shape, dtype=np.uint16)
    load().orc_f32_to_bf16_array(_p(f), _p(out), c_int64(f.size))
    return out


_DT = {"bf16": 0, "f16": 1}


def _dt(dtype: str) -> c_int:
    if dtype not in _DT:
        raise ValueError(f"storage dtype must be 'bf16' or 'f16', not {dtype!r}")
    return c_int(_DT[dtype])


def f16_to_f32(h) -> np.ndarray:
    h = _u16(h)
    out = np.empty(h.shape, dtype=np.float32)
    load().orc_f16_to_f32_array(_p(h), _p(out), c_int64(h.size))
    return out


def f32_to_f16(f) -> np.ndarray:
    f = np.ascontiguousarray(np.asarray(f, dtype=np.float32))
    out = np.empty(f.shape, dtype=np.uint16)
    load().orc_f32_to_f16_array(_p(f), _p(out), c_int64(f.size))
    return out


def st_to_f32(h, dtype: str = "bf16") -> np.ndarray:
    """Storage bits (bf16 or f16) to float32."""
    return f16_to_f32(h) if _DT[dtype] else bf16_to_f32(h)


def expf(x) -> np.ndarray:
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    out = np.empty_like(x)
    load().orc_expf_array(_p(x), _p(out), c_int64(x.size))
    return out


def router_logits(x, w, bias=None) -> np.ndarray:
    x, w = _u16(x), _u16(w)
    T, H = x.shape
    E = w.shape[0]
    b = None if bias is None else np.ascontiguousarray(np.asarray(bias, dtype=np.float32))
    out = np.empty((T, E), dtype=np.uint16)
    load().orc_router_logits(_p(x), _p(w), _p(b), c_int(T), c_int(H), c_int(E), _p(out))
    return out


def router_logits_affine(x, q, s, b, bias=None, dtype: str = "bf16") -> np.ndarray:
    """Logits of the affine-quantised router Q [E, H*bits/32], S/B [E, H/64]."""
    x, q, s, b = _u16(x), _u32(q), _u16(s), _u16(b)
    T, H = x.shape
    E = q.shape[0]
    bits = _bits(q.shape[1], H)
    bb = None if bias is None else np.ascontiguousarray(np.asarray(bias, dtype=np.float32))
    out = np.empty((T, E), dtype=np.uint16)
    load().orc_router_logits_affine(_p(x), _p(q), _p(s), _p(b), c_int(bits), _p(bb), c_int(T),
                                    c_int(H), c_int(E), _dt(dtype), _p(out))
    return out


def rmsnorm(x, w, eps: float, dtype: str = "bf16") -> np.ndarray:
    """Post-attention RMSNorm (storage dtype in and out), bit-defined order (oracle.h)."""
    x, w = _u16(x), _u16(w)
    T, H = x.shape
    out = np.empty((T, H), dtype=np.uint16)
    load().orc_rmsnorm(_p(x), _p(w), c_float(eps), c_int(T), c_int(H), _dt(dtype), _p(out))
    return out


def olmoe_softmax(logits, dtype: str = "bf16") -> np.ndarray:
    lg = _u16(logits)
    T, E = lg.shape
    out = np.empty_like(lg)
    load().orc_olmoe_softmax(_p(lg), c_int(T), c_int(E), _dt(dtype), _p(out))
    return out


def route_olmoe(logits, K: int, dtype: str = "bf16"):
    lg = _u16(logits)
    T, E = lg.shape
    idx = np.empty((T, K), dtype=np.int32)
    gates = np.empty((T, K), dtype=np.uint16)
    load().orc_route_olmoe(_p(lg), c_int(T), c_int(E), c_int(K), _dt(dtype), _p(idx), _p(gates))
    return idx, gates


def route_granite(logits, K: int, dtype: str = "bf16"):
    lg = _u16(logits)
    T, E = lg.shape
    idx = np.empty((T, K), dtype=np.int32)
    gates = np.empty((T, K), dtype=np.float32)
    load().orc_route_granite(_p(lg), c_int(T), c_int(E), c_int(K), _dt(dtype), _p(idx), _p(gates))
    return idx, gates


def group(idx, E: int):
    """Stable grouping; raises ValueError on out-of-range ids."""
    ids = _i32(idx).reshape(-1)
    n = ids.size
    order = np.empty(n, dtype=np.int32)
    inverse = np.empty(n, dtype=np.int32)
    offsets = np.empty(E + 1, dtype=np.int32)
    bad = load().orc_group(_p(ids), c_int64(n), c_int(E), _p(order), _p(inverse), _p(offsets))
    if bad:
        raise ValueError(f"{bad} expert ids out of range")
    return order, inverse, offsets


def _bits(words: int, kin: int) -> int:
    """Code width implied by a packed row of `words` uint32 holding `kin` codes."""
    bits = 32 * words // kin
    if bits not in (4, 8) or bits * kin != 32 * words:
        raise ValueError(f"{words} words do not pack {kin} codes at 4 or 8 bits")
    return bits


def dequant_f64(q, s, b, group_size: int = 64, dtype: str = "bf16") -> np.ndarray:
    q, s, b = _u32(q), _u16(s), _u16(b)
    N, W = q.shape
    Kin = s.shape[1] * group_size
    bits = _bits(W, Kin)
    out = np.empty((N, Kin), dtype=np.float64)
    load().orc_dequant_f64(_p(q), _p(s), _p(b), c_int(N), c_int(Kin), c_int(group_size),
                           c_int(bits), _dt(dtype), _p(out))
    return out


def gather_qmm_f64(x, xrow, eid, q, s, b, group_size: int = 64, dtype: str = "bf16") -> np.ndarray:
    x, q, s, b = _u16(x), _u32(q), _u16(s), _u16(b)
    xrow, eid = _i32(xrow).reshape(-1), _i32(eid).reshape(-1)
    E, N, W = q.shape
    Kin = s.shape[2] * group_size
    bits = _bits(W, Kin)
    rows = eid.size
    out = np.empty((rows, N), dtype=np.float64)
    load().orc_gather_qmm_f64(_p(x), _p(xrow), _p(eid), c_int(rows), _p(q), _p(s), _p(b),
                              c_int(N), c_int(Kin), c_int(group_size), c_int(bits), _dt(dtype), _p(out))
    return out


def moe_reference(x, idx, gates, w, tokens=None, residual=None, rm: float = 1.0,
                  dtype: str = "bf16") -> np.ndarray:
    """fp64 block output for `tokens` (default all): residual + rm * sum_k g_k expert_k(x).
    `w` has attributes gate_q/gate_s/gate_b/up_*/down_* as numpy arrays."""
    x = _u16(x)
    T, H = x.shape
    idx = _i32(idx)
    K = idx.shape[1]
    gates = np.ascontiguousarray(np.asarray(gates, dtype=np.float32))
    tok = _i32(np.arange(T) if tokens is None else tokens)
    I = w.gate_q.shape[1]
    out = np.empty((tok.size, H), dtype=np.float64)
    res = None if residual is None else _u16(residual)
    args = []
    for proj in ("gate", "up", "down"):
        args += [_u32(getattr(w, proj + "_q")), _u16(getattr(w, proj + "_s")), _u16(getattr(w, proj + "_b"))]
    bits = _bits(w.gate_q.shape[2], H)
    load().orc_moe_reference(_p(x), _p(res), c_float(rm), _p(tok), c_int(tok.size), c_int(H),
                             c_int(I), c_int(K), _p(idx), _p(gates), c_int(64), c_int(bits), _dt(dtype),
                             *[_p(a) for a in args], _p(out))
    return out


def moe_reference_full(x, idx, gates, w, residual=None, rm: float = 1.0, dtype: str = "bf16") -> np.ndarray:
    """moe_reference for every token, expert by expert with fp64 matrix
    products: the same arithmetic as orc_moe_reference (weights dequantised
    exactly by orc_dequant_f64, h = silu(x.gate) * (x.up) and the expert
    outputs unrounded, then sum_k g_k y_k in k order, times rm, plus the
    residual), with each dot product summed in BLAS order instead of
    sequentially, so it agrees with moe_reference to fp64 rounding."""
    xf = st_to_f32(_u16(x), dtype).astype(np.float64)
    T, H = xf.shape
    idx = _i32(idx)
    K = idx.shape[1]
    g = np.asarray(gates, dtype=np.float32).astype(np.float64).reshape(T, K)
    contrib = np.zeros((T, K, H), dtype=np.float64)
    flat = idx.reshape(-1)
    for e in np.unique(flat):
        routes = np.nonzero(flat == e)[0]
        t, k = routes // K, routes % K
        wg = dequant_f64(w.gate_q[e], w.gate_s[e], w.gate_b[e], dtype=dtype)
        wu = dequant_f64(w.up_q[e], w.up_s[e], w.up_b[e], dtype=dtype)
        wd = dequant_f64(w.down_q[e], w.down_s[e], w.down_b[e], dtype=dtype)
        xe = xf[t]
        a = xe @ wg.T
        h = a / (1.0 + np.exp(-a)) * (xe @ wu.T)
        contrib[t, k] = h @ wd.T
    out = np.zeros((T, H), dtype=np.float64)
    for k in range(K):
        out += g[:, k:k + 1] * contrib[:, k]
    out *= float(np.float32(rm))
    if residual is not None:
        out += st_to_f32(_u16(residual), dtype).astype(np.float64)
    return out


def moe_block_cpu(x, w, route: str, router, router_bias=None, residual=None, rm: float = 1.0,
                  top_k: int = 8, threads: int = 0):
    """The MLX-semantics CPU block (host-core baseline). Returns (y bf16 bits,
    idx, gates fp32, threads used)."""
    x = _u16(x)
    T, H = x.shape
    E = w.gate_q.shape[0]
    I = w.gate_q.shape[1]
    K = top_k
    idx = np.empty((T, K), dtype=np.int32)
    gates = np.empty((T, K), dtype=np.float32)
    y = np.empty((T, H), dtype=np.uint16)
    res = None if residual is None else _u16(residual)
    rb = None if router_bias is None else np.ascontiguousarray(np.asarray(router_bias, dtype=np.float32))
    args = []
    for proj in ("gate", "up", "down"):
        args += [_u32(getattr(w, proj + "_q")), _u16(getattr(w, proj + "_s")), _u16(getattr(w, proj + "_b"))]
    bits = _bits(w.gate_q.shape[2], H)
    used = load().orc_moe_block_cpu(
        _p(x), _p(res), c_float(rm), c_int(T), c_int(H), c_int(E), c_int(K), c_int(I), c_int(64),
        c_int(bits),
        c_int(0 if route == "olmoe" else 1), _p(_u16(router)), _p(rb), *[_p(a) for a in args],
        _p(idx), _p(gates), _p(y), c_int(threads))
    return y, idx, gates, used

