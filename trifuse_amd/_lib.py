"""ctypes binding of libtrifuse_moe.so (declared in include/trifuse_moe.h).

The library is loaded from trifuse_amd/lib/. If it is missing, every entry
point raises: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import threading
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int32, c_int64, c_size_t, c_uint32, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libtrifuse_moe.so"

TFM_OK = 0
TFM_E_INVALID = 1
TFM_E_UNSUPPORTED = 2
TFM_E_WORKSPACE = 3
TFM_E_HIP = 4
TFM_E_DEVICE = 5

TFM_DTYPE_BF16 = 0
TFM_DTYPE_F16 = 1
TFM_ROUTE_OLMOE = 0
TFM_ROUTE_GRANITE = 1
TFM_ROUTER_DENSE = 0
TFM_ROUTER_AFFINE = 1
TFM_FLAG_DETERMINISTIC = 1
TFM_STATUS_BAD_EXPERT_ID = 1
TFM_STATUS_BAD_ROW_INDEX = 2
TFM_STAGE_ROUTER = 0
TFM_STAGE_TOPK = 1
TFM_STAGE_GROUP = 2
TFM_STAGE_GATEUP = 3
TFM_STAGE_DOWN = 4
TFM_STAGE_COMBINE = 5
TFM_STAGE_NORM = 6
TFM_STATIC_SCRATCH_BYTES = 64 << 20
TFM_STAGE_COUNT = 7

_STATUS_NAMES = {
    TFM_E_INVALID: "invalid argument",
    TFM_E_UNSUPPORTED: "unsupported",
    TFM_E_WORKSPACE: "workspace",
    TFM_E_HIP: "HIP error",
    TFM_E_DEVICE: "device check",
}


class TfmError(RuntimeError):
    """A non-zero status from the C ABI, with the library's message."""

    def __init__(self, status: int, message: str):
        super().__init__(f"trifuse_moe {_STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


class TfmUnsupported(TfmError, NotImplementedError):
    pass


class Geometry(ctypes.Structure):
    _fields_ = [
        ("hidden_size", c_int32),
        ("intermediate_size", c_int32),
        ("num_experts", c_int32),
        ("experts_per_token", c_int32),
        ("group_size", c_int32),
        ("bits", c_int32),
        ("dtype", c_int32),
        ("route", c_int32),
        ("router", c_int32),
        ("residual_multiplier", c_float),
    ]


class Affine(ctypes.Structure):
    _fields_ = [("q", c_void_p), ("scales", c_void_p), ("biases", c_void_p)]


class MoeWeights(ctypes.Structure):
    _fields_ = [
        ("router", c_void_p),
        ("logit_bias", c_void_p),
        ("gate", Affine),
        ("up", Affine),
        ("down", Affine),
        ("router_affine", Affine),
        ("router_bits", c_int32),
    ]


# name -> (restype, argtypes); every function of include/trifuse_moe.h.
SIGNATURES = {
    "tfm_plan_create": (c_int, [POINTER(Geometry), POINTER(c_void_p)]),
    "tfm_plan_destroy": (None, [c_void_p]),
    "tfm_workspace_bytes": (c_size_t, [c_void_p, c_int64]),
    "tfm_route": (c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p,
                          c_void_p, c_void_p, c_size_t, c_void_p]),
    "tfm_route_affine": (c_int, [c_void_p, c_void_p, c_int64, POINTER(Affine), c_int32, c_void_p,
                                 c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "tfm_route_logits": (c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_void_p]),
    "tfm_olmoe_softmax": (c_int, [c_void_p, c_int64, c_int32, c_int32, c_void_p, c_void_p]),
    "tfm_topk": (c_int, [c_void_p, c_int64, c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p]),
    "tfm_group_workspace_bytes": (c_size_t, [c_int64, c_int32]),
    "tfm_group": (c_int, [c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_void_p, c_void_p,
                          c_size_t, c_void_p]),
    "tfm_gather_qmm_workspace_bytes": (c_size_t, [c_int64, c_int32, c_int32, c_int32]),
    "tfm_gather_qmm": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_int64, POINTER(Affine),
                               c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32,
                               c_void_p, c_void_p, c_size_t, c_void_p]),
    "tfm_affine_qmm": (c_int, [c_void_p, c_int64, POINTER(Affine), c_int32, c_int32, c_int32, c_int32,
                               c_int32, c_void_p, c_void_p]),
    "tfm_moe_experts": (c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_void_p,
                                POINTER(MoeWeights), c_void_p, c_uint32, c_void_p, c_size_t,
                                c_void_p]),
    "tfm_moe_forward": (c_int, [c_void_p, c_void_p, c_int64, c_void_p, POINTER(MoeWeights),
                                c_void_p, c_void_p, c_void_p, c_uint32, c_void_p, c_size_t,
                                c_void_p]),
    "tfm_moe_forward_static": (c_int, [c_void_p, c_void_p, c_int64, c_void_p, POINTER(MoeWeights),
                                       c_void_p, c_void_p, c_void_p, c_uint32, c_void_p]),
    "tfm_moe_forward_rmsnorm": (c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_float,
                                        POINTER(MoeWeights), c_void_p, c_void_p, c_void_p, c_uint32,
                                        c_void_p, c_size_t, c_void_p]),
    "tfm_expert_routes_workspace_bytes": (c_size_t, [c_void_p, c_int64]),
    "tfm_expert_routes": (c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_int32,
                                  POINTER(MoeWeights), c_void_p, c_void_p, c_void_p, c_size_t,
                                  c_void_p]),
    "tfm_profiler_create": (c_int, [c_int32, POINTER(c_void_p)]),
    "tfm_profiler_destroy": (None, [c_void_p]),
    "tfm_profiler_attach": (c_int, [c_void_p]),
    "tfm_profiler_reset": (c_int, [c_void_p]),
    "tfm_profiler_stage": (c_int, [c_void_p, c_int32, POINTER(c_double), POINTER(c_int32),
                                   POINTER(c_int32)]),
    "tfm_profiler_stage_kernel": (c_int, [c_void_p, c_int32, POINTER(c_double), POINTER(c_int32)]),
    "tfm_stage_name": (c_char_p, [c_int32]),
    "tfm_status_word": (c_int, [c_void_p, c_void_p, POINTER(c_uint32)]),
    "tfm_last_error": (c_char_p, []),
    "tfm_version": (c_char_p, []),
}

_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Load the library once; raise if it has not been built."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python -m trifuse_amd.build` "
                    "(the MoE path has no CPU fallback)")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Call an int-returning entry point and raise TfmError on failure."""
    lib = load()
    status = getattr(lib, name)(*args)
    if status != TFM_OK:
        msg = lib.tfm_last_error().decode(errors="replace")
        if status == TFM_E_UNSUPPORTED:
            raise TfmUnsupported(status, msg)
        raise TfmError(status, msg)
