"""Helpers shared by the tests: torch <-> numpy views of bf16/uint32 data and
the block tolerance metric."""
from __future__ import annotations

import sys
import types

import numpy as np
import torch

# Block outputs are bf16 with fp32 accumulation; the bar is max-rel 1e-2 of an
# fp32-dequantised reference: max|y - ref| / max|ref| <= 1e-2.
BLOCK_TOL = 1e-2


def log(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def u16(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def u32(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().numpy().view(np.uint32)


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def bf16_from_u16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


def np_layer(layer) -> types.SimpleNamespace:
    ns = types.SimpleNamespace()
    for proj in ("gate", "up", "down"):
        setattr(ns, proj + "_q", u32(getattr(layer, proj + "_q")))
        setattr(ns, proj + "_s", u16(getattr(layer, proj + "_s")))
        setattr(ns, proj + "_b", u16(getattr(layer, proj + "_b")))
    ns.router = None if layer.router is None else u16(layer.router)
    ns.logit_bias = None if layer.logit_bias is None else f32(layer.logit_bias)
    if getattr(layer, "router_q", None) is not None:
        ns.router_q = u32(layer.router_q)
        ns.router_s = u16(layer.router_s)
        ns.router_b = u16(layer.router_b)
    return ns


def max_rel(y: np.ndarray, ref: np.ndarray) -> float:
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = float(np.max(np.abs(ref)))
    return float(np.max(np.abs(y - ref))) / (den if den > 0 else 1.0)
