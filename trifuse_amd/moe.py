"""Host-side mirror of TriFuse's MoE operator interface over the HIP library.

Two levels, both calling libtrifuse_moe.so through its C ABI (there is no CPU
fallback: every call raises if the library or a GPU is missing):

* Operator functions with the names, argument meaning and validation errors of
  TriFuse's export-time op schema
  (overlays/executorch/backends/mlx/native_affine_ops.py:12-153):
  ``native_affine_gather_qmm``, ``native_affine_qmm``, ``native_olmoe_softmax``,
  ``native_olmoe_topk_indices``, ``native_topk_indices``,
  ``native_take_along_last``, plus ``validate_affine``.
* ``MoEBlock``: the block that NativeGraniteMoEPrefill::moe runs per layer
  (overlays/executorch/backends/mlx/runtime/MLXNativeGraniteMoEPrefill.h:627-702)
  and the NativeMoEExpertHook contract (MLXMoEExpertHook.h:18-51):
  ``forward`` (router -> route -> group -> experts -> combine [+ residual]),
  ``route``, ``experts`` (hook ``execute`` body given routes) and
  ``expert_routes`` (the hook's GPUCallable).

Tensors are torch tensors on the current HIP device; torch only provides
memory and the stream. Activations, scales and biases are bf16; packed
weights are uint32 words stored in int32 (or uint32) tensors.
"""
from __future__ import annotations

import ctypes
import dataclasses
from typing import Dict, Optional, Tuple

import torch

from . import _lib
from ._lib import (TFM_DTYPE_BF16, TFM_DTYPE_F16, TFM_FLAG_DETERMINISTIC, TFM_ROUTE_GRANITE,
                   TFM_ROUTE_OLMOE, TFM_ROUTER_AFFINE, TFM_ROUTER_DENSE, Affine, Geometry,
                   MoeWeights, call)

_ROUTES = {"olmoe": TFM_ROUTE_OLMOE, "granite": TFM_ROUTE_GRANITE}
_PACKED = (torch.int32, torch.uint32)
_INDEX = (torch.int32, torch.int64)


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _dev(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor (the MoE path has no CPU fallback)")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _check_residual(residual: Optional[torch.Tensor], x: torch.Tensor) -> None:
    if residual is None:
        return
    _dev(residual, "residual")
    if residual.shape != x.shape or residual.dtype != x.dtype:
        raise ValueError("residual geometry/dtype differs")


def _check_logit_bias(logit_bias: Optional[torch.Tensor], E: int) -> None:
    if logit_bias is None:
        return
    _dev(logit_bias, "logit_bias")
    if logit_bias.dtype != torch.float32 or logit_bias.numel() != E:
        raise ValueError("logit_bias must be fp32 [E]")


def _index32(t: torch.Tensor) -> torch.Tensor:
    if t.dtype not in (torch.int32, torch.int64, torch.uint32):
        raise ValueError("indices must be integers")
    return t.to(torch.int32).contiguous()


def validate_affine(q: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                    group_size: int, bits: int, rank: int) -> int:
    """Shape/dtype contract of native_affine_ops.validate_affine
    (native_affine_ops.py:12-26) with bf16 scales/biases admitted; returns the
    unpacked input width."""
    if (type(bits) is not int or bits not in (4, 8)
            or type(group_size) is not int or group_size not in (32, 64, 128)):
        raise ValueError("Native affine requires bits4/8 and group32/64/128")
    if q.dtype not in _PACKED or q.ndim != rank or rank not in (2, 3):
        raise ValueError("Native affine Q must be rank2/3 uint32")
    if (scales.dtype not in (torch.bfloat16, torch.float16, torch.float32)
            or biases.dtype != scales.dtype or scales.shape != biases.shape
            or scales.ndim != rank or q.shape[:-1] != scales.shape[:-1]):
        raise ValueError("Native affine S/B shapes or floating dtypes differ")
    width = q.shape[-1] * (32 // bits)
    if (width % group_size or scales.shape[-1] * group_size != width
            or any(int(d) <= 0 for d in q.shape)):
        raise ValueError("Native affine packed/group dimensions differ")
    return width


def _affine(q, s, b) -> Affine:
    for t, n in ((q, "q"), (s, "scales"), (b, "biases")):
        _dev(t, n)
    return Affine(q.data_ptr(), s.data_ptr(), b.data_ptr())


def _workspace(nbytes: int, device) -> torch.Tensor:
    # torch's caching allocator returns blocks aligned to at least 512 bytes.
    # The status word lives in the first 256 bytes and is sticky (kernels only
    # set bits; tfm_status_word clears them), so a fresh workspace starts zeroed.
    ws = torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)
    ws[:256].zero_()
    return ws


_DTYPES = {torch.bfloat16: TFM_DTYPE_BF16, torch.float16: TFM_DTYPE_F16}


def _dtype_code(t: torch.Tensor, name: str) -> int:
    """C-ABI storage dtype of t: bf16 or IEEE half."""
    code = _DTYPES.get(t.dtype)
    if code is None:
        raise NotImplementedError(f"{name}: only bf16 and f16 storage are built (got {t.dtype})")
    return code


def _check_dtype(t: torch.Tensor, dtype: torch.dtype, name: str) -> None:
    if t.dtype != dtype:
        raise ValueError(f"{name}: dtype {t.dtype} differs from the block's {dtype}")


# ---------------------------------------------------------------------------
# Flat-row gather_qmm and grouping
# ---------------------------------------------------------------------------

def gather_qmm_rows(x: torch.Tensor, q: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                    rhs_indices: torch.Tensor, x_rows: Optional[torch.Tensor] = None,
                    sorted_indices: bool = False, group_size: int = 64, bits: int = 4) -> torch.Tensor:
    """out[r] = x[x_rows[r]] . dequant(W[rhs_indices[r]])^T for r in [0, len(rhs_indices)).

    x [X, Kin] bf16 or f16 (scales and biases in the same dtype);
    q [E, N, Kin*bits/32]; x_rows None means identity."""
    kin = validate_affine(q, scales, biases, group_size, bits, 3)
    dt = _dtype_code(x, "x")
    _check_dtype(scales, x.dtype, "scales")
    _dev(x, "x")
    if x.ndim != 2 or x.shape[1] != kin:
        raise ValueError("Native affine expert input differs")
    _dev(rhs_indices, "rhs_indices")
    if x_rows is not None:
        _dev(x_rows, "x_rows")
    rhs = _index32(rhs_indices).reshape(-1)
    rows = rhs.numel()
    xr = None if x_rows is None else _index32(x_rows).reshape(-1)
    if xr is not None and xr.numel() != rows:
        raise ValueError("x_rows and rhs_indices must have the same length")
    E, N = q.shape[0], q.shape[1]
    out = torch.empty((rows, N), dtype=x.dtype, device=x.device)
    lib = _lib.load()
    wsb = lib.tfm_gather_qmm_workspace_bytes(rows, E, N, kin)
    ws = _workspace(wsb, x.device)
    aff = _affine(q, scales, biases)
    call("tfm_gather_qmm", x.data_ptr(), x.shape[0], _ptr(xr), _ptr(rhs), rows, ctypes.byref(aff),
         E, N, kin, group_size, bits, dt, int(bool(sorted_indices)), out.data_ptr(),
         ws.data_ptr(), ws.numel(), _stream())
    return out


def group(expert_ids: torch.Tensor, num_experts: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Stable grouping of flat routes by expert (argsort + inverse of
    MLXNativeGraniteMoEPrefill.h:670-680): returns (order, inverse, offsets[E+1])."""
    ids = _index32(expert_ids).reshape(-1)
    _dev(ids, "expert_ids")
    n = ids.numel()
    order = torch.empty(n, dtype=torch.int32, device=ids.device)
    inverse = torch.empty(n, dtype=torch.int32, device=ids.device)
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=ids.device)
    lib = _lib.load()
    ws = _workspace(lib.tfm_group_workspace_bytes(n, num_experts), ids.device)
    call("tfm_group", ids.data_ptr(), n, num_experts, order.data_ptr(), inverse.data_ptr(),
         offsets.data_ptr(), ws.data_ptr(), ws.numel(), _stream())
    return order, inverse, offsets


# ---------------------------------------------------------------------------
# Operator mirror of native_affine_ops.py
# ---------------------------------------------------------------------------

def native_affine_gather_qmm(x: torch.Tensor, q: torch.Tensor, scales: torch.Tensor,
                             biases: torch.Tensor, indices: torch.Tensor, group_size: int,
                             bits: int, sorted_indices: bool = False) -> torch.Tensor:
    """mlx::native_affine_gather_qmm (native_affine_ops.py:55-74): x [..., M, Kin],
    indices broadcast against x.shape[:-2]; returns [*batch, M, N] in x.dtype."""
    width = validate_affine(q, scales, biases, group_size, bits, 3)
    if (x.ndim < 2 or x.shape[-1] != width or x.dtype != scales.dtype
            or indices.dtype not in _INDEX or type(sorted_indices) is not bool):
        raise ValueError("Native affine expert input differs")
    batch = torch.broadcast_shapes(x.shape[:-2], indices.shape)
    M = x.shape[-2]
    xb = x.reshape(-1, M, width)
    # Row of x feeding each (batch element, m): broadcast the x batch index.
    xbatch = torch.arange(xb.shape[0], device=x.device, dtype=torch.int32).reshape(x.shape[:-2])
    xbatch = torch.broadcast_to(xbatch, batch).reshape(-1)
    experts = torch.broadcast_to(indices, batch).reshape(-1).to(torch.int32)
    m = torch.arange(M, device=x.device, dtype=torch.int32)
    x_rows = (xbatch[:, None] * M + m[None, :]).reshape(-1)
    rhs = experts[:, None].expand(-1, M).reshape(-1)
    out = gather_qmm_rows(xb.reshape(-1, width).contiguous(), q, scales, biases, rhs, x_rows,
                          sorted_indices, group_size, bits)
    return out.reshape(*batch, M, q.shape[-2])


def native_affine_qmm(x: torch.Tensor, q: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                      group_size: int, bits: int) -> torch.Tensor:
    """mlx::native_affine_qmm (native_affine_ops.py:39-52): y = x . dequant(W)^T."""
    width = validate_affine(q, scales, biases, group_size, bits, 2)
    if x.ndim < 1 or x.shape[-1] != width or x.dtype != scales.dtype:
        raise ValueError("Native affine QMM input width/dtype differs")
    _dev(x, "x")
    lead = x.shape[:-1]
    rows = x.reshape(-1, width).contiguous()
    N = q.shape[-2]
    out = torch.empty((rows.shape[0], N), dtype=x.dtype, device=x.device)
    qc, sc, bc = q.contiguous(), scales.contiguous(), biases.contiguous()  # alive through the call
    aff = _affine(qc, sc, bc)
    call("tfm_affine_qmm", rows.data_ptr(), rows.shape[0], ctypes.byref(aff), N, width, group_size, bits,
         _dtype_code(x, "x"), out.data_ptr(), _stream())
    return out.reshape(*lead, N)


def native_olmoe_softmax(x: torch.Tensor) -> torch.Tensor:
    """mlx::native_olmoe_softmax (native_affine_ops.py:128-138): precise fp32
    softmax over the last axis, rounded to the storage dtype. x is [1, T, E],
    FP16 as the reference requires, or BF16."""
    if x.ndim != 3 or x.dtype not in _DTYPES:
        raise ValueError("OLMoE router requires B1/T/E FP16 (or BF16) logits")
    _dev(x, "x")
    E = x.shape[-1]
    rows = x.numel() // E
    out = torch.empty_like(x)
    call("tfm_olmoe_softmax", x.data_ptr(), rows, E, _DTYPES[x.dtype], out.data_ptr(), _stream())
    return out


def _topk(x: torch.Tensor, k: int, rule: int) -> torch.Tensor:
    if type(k) is not int or not 0 < k <= x.shape[-1]:
        raise ValueError("Invalid top-k")
    dt = _dtype_code(x, "x")
    _dev(x, "x")
    n = x.shape[-1]
    rows = x.numel() // n
    out = torch.empty((*x.shape[:-1], k), dtype=torch.int32, device=x.device)
    call("tfm_topk", x.data_ptr(), rows, n, k, rule, dt, out.data_ptr(), _stream())
    return out


def native_olmoe_topk_indices(x: torch.Tensor, k: int) -> torch.Tensor:
    """mlx::native_olmoe_topk_indices (native_affine_ops.py:141-153) as lowered
    (native_affine_lowering.py:93-108): the k largest values in descending
    order, ties to the lower index, NaN last."""
    if x.ndim != 3 or x.dtype not in _DTYPES or type(k) is not int or not 0 < k <= x.shape[-1]:
        raise ValueError("Invalid OLMoE probability/top-k ABI")
    return _topk(x, k, TFM_ROUTE_OLMOE)


def native_topk_indices(x: torch.Tensor, k: int) -> torch.Tensor:
    """mlx::native_topk_indices (native_affine_ops.py:96-112) as lowered
    (argpartition(kth=-k) + slice of the last k, native_affine_lowering.py:61-74):
    slots in ascending order of value, ties resolved by a stable ascending rank."""
    if x.ndim < 1 or type(k) is not int or not 0 < k <= x.shape[-1]:
        raise ValueError("Invalid top-k")
    return _topk(x, k, TFM_ROUTE_GRANITE)


def native_take_along_last(x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
    """mlx::native_take_along_last (native_affine_ops.py:115-125)."""
    if (x.ndim < 1 or x.shape[:-1] != indices.shape[:-1]
            or indices.dtype not in (torch.int32, torch.int64)):
        raise ValueError("Native take requires matching leading dimensions and integer indices")
    return torch.take_along_dim(x, indices.long(), dim=-1)


# ---------------------------------------------------------------------------
# The MoE block
# ---------------------------------------------------------------------------

@dataclasses.dataclass
class ExpertWeights:
    """Stacked switch_mlp weights of one layer (prepare_model.py:67-106 layout):
    gate/up Q [E, I, H*bits/32], S/B [E, I, H/64]; down Q [E, H, I*bits/32],
    S/B [E, H, I/64]; router [E, H] (dense router) or router_q [E, H*router_bits/32],
    router_s/router_b [E, H/64] (affine router); logit_bias optional fp32 [E]."""
    router: Optional[torch.Tensor]
    gate_q: torch.Tensor
    gate_s: torch.Tensor
    gate_b: torch.Tensor
    up_q: torch.Tensor
    up_s: torch.Tensor
    up_b: torch.Tensor
    down_q: torch.Tensor
    down_s: torch.Tensor
    down_b: torch.Tensor
    logit_bias: Optional[torch.Tensor] = None
    router_q: Optional[torch.Tensor] = None
    router_s: Optional[torch.Tensor] = None
    router_b: Optional[torch.Tensor] = None
    router_bits: int = 4

    @classmethod
    def from_layer(cls, layer) -> "ExpertWeights":
        return cls(**{f.name: getattr(layer, f.name) for f in dataclasses.fields(cls)
                      if hasattr(layer, f.name)})


class MoEBlock:
    """One MoE feed-forward block of a fixed geometry (NativeModelConfig,
    resident_prefill.h:18-42; admission MLXNativeGraniteMoEPrefill.h:306-330)."""

    def __init__(self, hidden_size: int, intermediate_size: int, num_experts: int,
                 experts_per_token: int, route: str = "olmoe", residual_multiplier: float = 1.0,
                 group_size: int = 64, bits: int = 4, dtype: torch.dtype = torch.bfloat16,
                 router: str = "dense"):
        if route not in _ROUTES:
            raise ValueError(f"unknown route kind {route!r}")
        if dtype not in _DTYPES:
            raise ValueError(f"unknown storage dtype {dtype}")
        if router not in ("dense", "affine"):
            raise ValueError(f"unknown router kind {router!r}")
        self.dtype = dtype
        self.router_kind = router
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.num_experts = num_experts
        self.experts_per_token = experts_per_token
        self.route_kind = route
        self.residual_multiplier = residual_multiplier
        self.bits = bits
        self.geometry = Geometry(hidden_size, intermediate_size, num_experts, experts_per_token,
                                 group_size, bits, _DTYPES[dtype], _ROUTES[route],
                                 TFM_ROUTER_DENSE if router == "dense" else TFM_ROUTER_AFFINE,
                                 float(residual_multiplier))
        lib = _lib.load()
        handle = ctypes.c_void_p()
        call("tfm_plan_create", ctypes.byref(self.geometry), ctypes.byref(handle))
        self._lib = lib
        self._plan = handle
        self._ws: Optional[torch.Tensor] = None
        self._ws_bytes: Dict[int, int] = {}
        self._wcache: Dict[Tuple[int, bool], tuple] = {}

    def close(self) -> None:
        if getattr(self, "_plan", None):
            self._lib.tfm_plan_destroy(self._plan)
            self._plan = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- workspace ---------------------------------------------------------
    def workspace_bytes(self, tokens: int) -> int:
        n = self._ws_bytes.get(tokens)
        if n is None:
            n = int(self._lib.tfm_workspace_bytes(self._plan, tokens))
            self._ws_bytes[tokens] = n
        return n

    def workspace(self, tokens: int, device) -> torch.Tensor:
        need = self.workspace_bytes(tokens)
        if self._ws is None or self._ws.numel() < need or self._ws.device != torch.device(device):
            fresh = _workspace(need, device)
            if self._ws is not None and self._ws.device == fresh.device:
                # The status bits are sticky until status_word() reads them:
                # carry the old header (first 256 bytes) into the new workspace,
                # in stream order after every call that used the old one.
                fresh[:256].copy_(self._ws[:256])
            self._ws = fresh
        return self._ws

    def status_word(self) -> int:
        """Device status bits (TFM_STATUS_*) of the last calls; clears them."""
        if self._ws is None:
            return 0
        v = ctypes.c_uint32()
        call("tfm_status_word", self._ws.data_ptr(), _stream(), ctypes.byref(v))
        return int(v.value)

    # -- checks --------------------------------------------------------------
    def _check_x(self, x: torch.Tensor) -> int:
        _dev(x, "x")
        _check_dtype(x, self.dtype, "x")
        if x.shape[-1] != self.hidden_size:
            raise ValueError("hidden width differs")
        return x.numel() // self.hidden_size

    _WEIGHT_FIELDS = ("router", "gate_q", "gate_s", "gate_b", "up_q", "up_s", "up_b", "down_q",
                      "down_s", "down_b", "logit_bias", "router_q", "router_s", "router_b")

    def _weights(self, w: ExpertWeights, router: bool) -> MoeWeights:
        """Validated C-ABI weight struct of `w`, cached per weights object while
        its tensors keep their storage (a decode step calls this once per layer)."""
        key = (id(w), router)
        ptrs = tuple(0 if t is None else t.data_ptr() for t in (getattr(w, f) for f in self._WEIGHT_FIELDS))
        hit = self._wcache.get(key)
        if hit is not None and hit[0] is w and hit[1] == ptrs:
            return hit[2]
        mw = self._build_weights(w, router)
        if len(self._wcache) >= 64:
            self._wcache.clear()
        self._wcache[key] = (w, ptrs, mw)
        return mw

    def _build_weights(self, w: ExpertWeights, router: bool) -> MoeWeights:
        H, I, E = self.hidden_size, self.intermediate_size, self.num_experts
        g, per = 64, 32 // self.bits
        shapes = {
            "gate_q": (E, I, H // per), "gate_s": (E, I, H // g), "gate_b": (E, I, H // g),
            "up_q": (E, I, H // per), "up_s": (E, I, H // g), "up_b": (E, I, H // g),
            "down_q": (E, H, I // per), "down_s": (E, H, I // g), "down_b": (E, H, I // g),
        }
        for name, shape in shapes.items():
            t = getattr(w, name)
            if tuple(t.shape) != shape:
                raise ValueError(f"{name} shape {tuple(t.shape)} != {shape}")
        validate_affine(w.gate_q, w.gate_s, w.gate_b, 64, self.bits, 3)
        validate_affine(w.up_q, w.up_s, w.up_b, 64, self.bits, 3)
        validate_affine(w.down_q, w.down_s, w.down_b, 64, self.bits, 3)
        for name in ("gate_s", "up_s", "down_s"):
            _check_dtype(getattr(w, name), self.dtype, name)
        mw = MoeWeights()
        mw.gate = _affine(w.gate_q, w.gate_s, w.gate_b)
        mw.up = _affine(w.up_q, w.up_s, w.up_b)
        mw.down = _affine(w.down_q, w.down_s, w.down_b)
        if router and self.router_kind == "affine":
            rb = w.router_bits
            if w.router_q is None or w.router_s is None or w.router_b is None:
                raise ValueError("affine router needs router_q, router_s and router_b")
            width = validate_affine(w.router_q, w.router_s, w.router_b, 64, rb, 2)
            if width != H or w.router_q.shape[0] != E:
                raise ValueError("router shape differs")
            _check_dtype(w.router_s, self.dtype, "router_s")
            mw.router_affine = _affine(w.router_q, w.router_s, w.router_b)
            mw.router_bits = rb
        elif router:
            if w.router is None:
                raise ValueError("a dense-router block needs weights.router [E, H]")
            _dev(w.router, "router")
            _check_dtype(w.router, self.dtype, "router")
            if tuple(w.router.shape) != (E, H):
                raise ValueError("router shape differs")
            mw.router = w.router.data_ptr()
        if router and w.logit_bias is not None:
            _check_logit_bias(w.logit_bias, E)
            mw.logit_bias = w.logit_bias.data_ptr()
        return mw

    # -- entry points --------------------------------------------------------
    def forward(self, x: torch.Tensor, weights: ExpertWeights, residual: Optional[torch.Tensor] = None,
                deterministic: bool = False, return_routes: bool = False):
        """The whole block: residual + rm * sum_k gate_k * expert_k(x) (y in x's shape).
        With return_routes, also returns (idx [T,K] int32, gates [T,K] fp32)."""
        T = self._check_x(x)
        _check_residual(residual, x)
        mw = self._weights(weights, router=True)
        y = torch.empty_like(x)
        K = self.experts_per_token
        idx = gates = None
        if return_routes:
            idx = torch.empty((T, K), dtype=torch.int32, device=x.device)
            gates = torch.empty((T, K), dtype=torch.float32, device=x.device)
        ws = self.workspace(T, x.device)
        flags = TFM_FLAG_DETERMINISTIC if deterministic else 0
        call("tfm_moe_forward", self._plan, x.data_ptr(), T, _ptr(residual), ctypes.byref(mw),
             y.data_ptr(), _ptr(idx), _ptr(gates), flags, ws.data_ptr(), ws.numel(), _stream())
        return (y, idx, gates) if return_routes else y

    def forward_static(self, x: torch.Tensor, weights: ExpertWeights, residual: Optional[torch.Tensor] = None,
                       return_routes: bool = False):
        """forward() through the allocation-free entry point (tfm_moe_forward_static):
        the library's static device scratch instead of a workspace. Calls on
        one GPU share that scratch and must not overlap."""
        T = self._check_x(x)
        _check_residual(residual, x)
        mw = self._weights(weights, router=True)
        y = torch.empty_like(x)
        K = self.experts_per_token
        idx = gates = None
        if return_routes:
            idx = torch.empty((T, K), dtype=torch.int32, device=x.device)
            gates = torch.empty((T, K), dtype=torch.float32, device=x.device)
        call("tfm_moe_forward_static", self._plan, x.data_ptr(), T, _ptr(residual), ctypes.byref(mw),
             y.data_ptr(), _ptr(idx), _ptr(gates), 0, _stream())
        return (y, idx, gates) if return_routes else y

    def forward_rmsnorm(self, h: torch.Tensor, weights: ExpertWeights, norm_weight: torch.Tensor,
                        eps: float, return_routes: bool = False):
        """The block with the post-attention RMSNorm fused in, as the reference
        layer runs it (MLXNativeGraniteMoEPrefill.h:485-487):
        post = rms_norm(h, norm_weight, eps); y = h + rm * moe(post).
        With return_routes, also returns (idx [T,K] int32, gates [T,K] fp32)."""
        T = self._check_x(h)
        _dev(norm_weight, "norm_weight")
        _check_dtype(norm_weight, self.dtype, "norm_weight")
        if norm_weight.numel() != self.hidden_size or not norm_weight.is_contiguous():
            raise ValueError("norm_weight must be a contiguous [H] tensor")
        mw = self._weights(weights, router=True)
        y = torch.empty_like(h)
        K = self.experts_per_token
        idx = gates = None
        if return_routes:
            idx = torch.empty((T, K), dtype=torch.int32, device=h.device)
            gates = torch.empty((T, K), dtype=torch.float32, device=h.device)
        ws = self.workspace(T, h.device)
        call("tfm_moe_forward_rmsnorm", self._plan, h.data_ptr(), T, norm_weight.data_ptr(), float(eps),
             ctypes.byref(mw), y.data_ptr(), _ptr(idx), _ptr(gates), 0, ws.data_ptr(), ws.numel(),
             _stream())
        return (y, idx, gates) if return_routes else y

    def route(self, x: torch.Tensor, router: torch.Tensor, logit_bias: Optional[torch.Tensor] = None):
        """Router linear + routing: (idx [T,K] int32, gates [T,K], logits [T,E] bf16).
        OLMoE gates are bf16 probabilities; Granite gates are fp32."""
        T = self._check_x(x)
        _dev(router, "router")
        _check_dtype(router, self.dtype, "router")
        K, E = self.experts_per_token, self.num_experts
        if tuple(router.shape) != (E, self.hidden_size):
            raise ValueError("router shape differs")
        _check_logit_bias(logit_bias, E)
        idx = torch.empty((T, K), dtype=torch.int32, device=x.device)
        gdt = self.dtype if self.route_kind == "olmoe" else torch.float32
        gates = torch.empty((T, K), dtype=gdt, device=x.device)
        logits = torch.empty((T, E), dtype=self.dtype, device=x.device)
        ws = self.workspace(T, x.device)
        call("tfm_route", self._plan, x.data_ptr(), T, router.data_ptr(), _ptr(logit_bias),
             logits.data_ptr(), idx.data_ptr(), gates.data_ptr(), ws.data_ptr(), ws.numel(), _stream())
        return idx, gates, logits

    def route_affine(self, x: torch.Tensor, q: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                     bits: int = 4, logit_bias: Optional[torch.Tensor] = None):
        """Affine-quantised router linear + routing (the exports' router
        Affine module, export_native_olmoe_target.py:194-202): (idx [T,K] int32,
        gates [T,K], logits [T,E] in the block's dtype)."""
        T = self._check_x(x)
        K, E = self.experts_per_token, self.num_experts
        width = validate_affine(q, scales, biases, 64, bits, 2)
        if width != self.hidden_size or q.shape[0] != E:
            raise ValueError("router shape differs")
        _check_dtype(scales, self.dtype, "scales")
        idx = torch.empty((T, K), dtype=torch.int32, device=x.device)
        gdt = self.dtype if self.route_kind == "olmoe" else torch.float32
        gates = torch.empty((T, K), dtype=gdt, device=x.device)
        logits = torch.empty((T, E), dtype=self.dtype, device=x.device)
        _check_logit_bias(logit_bias, E)
        aff = _affine(q, scales, biases)
        ws = self.workspace(T, x.device)
        call("tfm_route_affine", self._plan, x.data_ptr(), T, ctypes.byref(aff), bits, _ptr(logit_bias),
             logits.data_ptr(), idx.data_ptr(), gates.data_ptr(), ws.data_ptr(), ws.numel(), _stream())
        return idx, gates, logits

    def experts(self, x: torch.Tensor, idx: torch.Tensor, gates: torch.Tensor, weights: ExpertWeights,
                residual: Optional[torch.Tensor] = None, deterministic: bool = False) -> torch.Tensor:
        """NativeMoEExpertHook::execute body (MLXMoEExpertHook.h:43-51) given routes."""
        T = self._check_x(x)
        K = self.experts_per_token
        _dev(idx, "idx")
        _dev(gates, "gates")
        idx32 = _index32(idx)
        if idx32.numel() != T * K:
            raise ValueError("indices must be [T, K]")
        if gates.numel() != T * K:
            raise ValueError("gates must be [T, K]")
        g32 = gates.to(torch.float32).contiguous()
        _check_residual(residual, x)
        mw = self._weights(weights, router=False)
        y = torch.empty_like(x)
        ws = self.workspace(T, x.device)
        flags = TFM_FLAG_DETERMINISTIC if deterministic else 0
        call("tfm_moe_experts", self._plan, x.data_ptr(), T, _ptr(residual), idx32.data_ptr(),
             g32.data_ptr(), ctypes.byref(mw), y.data_ptr(), flags, ws.data_ptr(), ws.numel(),
             _stream())
        return y

    def expert_routes(self, x: torch.Tensor, token_indices: torch.Tensor, expert_ids: torch.Tensor,
                      experts_sorted: bool, weights: ExpertWeights) -> Tuple[torch.Tensor, torch.Tensor]:
        """NativeMoEExpertHook::GPUCallable (MLXMoEExpertHook.h:23-30):
        returns (expert-sorted out [N, H], inverse [N]) with out[inverse[i]] for route i."""
        T = self._check_x(x)
        _dev(token_indices, "token_indices")
        _dev(expert_ids, "expert_ids")
        tok = _index32(token_indices).reshape(-1)
        eid = _index32(expert_ids).reshape(-1)
        if tok.numel() != eid.numel():
            raise ValueError("expert hook route arrays must be parallel integer vectors")
        N = tok.numel()
        mw = self._weights(weights, router=False)
        out = torch.empty((N, self.hidden_size), dtype=x.dtype, device=x.device)
        inverse = torch.empty(N, dtype=torch.int32, device=x.device)
        wsb = int(self._lib.tfm_expert_routes_workspace_bytes(self._plan, N))
        ws = _workspace(wsb, x.device)
        call("tfm_expert_routes", self._plan, x.data_ptr(), T, _ptr(tok), _ptr(eid), N,
             int(bool(experts_sorted)), ctypes.byref(mw), out.data_ptr(), inverse.data_ptr(),
             ws.data_ptr(), ws.numel(), _stream())
        return out, inverse


class StageProfiler:
    """HIP-event timing of the library's kernel stages (tfm_profiler_*)."""

    STAGES = ("router", "topk", "group", "gateup", "down", "combine", "norm")

    def __init__(self, capacity: int = 4096):
        self._lib = _lib.load()
        h = ctypes.c_void_p()
        call("tfm_profiler_create", capacity, ctypes.byref(h))
        self._h = h

    def __enter__(self):
        call("tfm_profiler_reset", self._h)
        self._lib.tfm_profiler_attach(self._h)
        return self

    def __exit__(self, *exc):
        self._lib.tfm_profiler_attach(None)
        return False

    def stage(self, name: str) -> Tuple[float, int]:
        """(total ms, launches) of one stage since the profiler was entered."""
        ms = ctypes.c_double()
        n = ctypes.c_int32()
        dropped = ctypes.c_int32()
        call("tfm_profiler_stage", self._h, self.STAGES.index(name), ctypes.byref(ms),
             ctypes.byref(n), ctypes.byref(dropped))
        if dropped.value:
            raise RuntimeError(f"profiler capacity exceeded ({dropped.value} stage launches dropped)")
        return ms.value, n.value

    def stage_kernel(self, name: str) -> Tuple[float, int]:
        """(total ms, kernels) of the main kernel of each launch of one stage,
        timed by the kernel dispatch's own start and end (as a kernel trace
        reports it), without the launch gaps that stage() includes."""
        ms = ctypes.c_double()
        n = ctypes.c_int32()
        call("tfm_profiler_stage_kernel", self._h, self.STAGES.index(name), ctypes.byref(ms), ctypes.byref(n))
        return ms.value, n.value

    def close(self):
        if self._h:
            self._lib.tfm_profiler_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
