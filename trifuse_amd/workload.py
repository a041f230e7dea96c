"""Synthetic MoE-block workloads (OLMoE and Granite-MoE geometry).

Every tensor is a pure function of (seed, workload, layer, tensor name), so
the same bytes can be produced on the host and on the GPU:

* packed 4-bit weights and scales come from a 32-bit integer hash of the
  element index (``lowbias32``, evaluated in int64 torch arithmetic with no
  overflow), so they are bit-identical on any device;
* normal draws (router weight, activations) come from numpy's PCG64 on the
  host and are copied to the device.

Distributions (per tensor):
  router  W_r [E, H] bf16 ~ N(0, 0.02)
  Q       [E, N, Kin/8] uint32 (stored as int32), 8 uniform nibbles per word
          (8-bit layers: [E, N, Kin/4], 4 uniform bytes per word)
  scales  [E, N, Kin/64] bf16 ~ U[0.005, 0.02];  biases = -8 * scales (exact)
          (8-bit layers: U[0.005, 0.02] / 16, biases = -128 * scales)
  x       [T, H] bf16 ~ N(0, 1)
  Zipf router bias (skewed routing): bias_e = 0.875 * (-1.1 * ln r_e) with r
  a seeded permutation of 1..E, added to the fp32 router logits.
"""
from __future__ import annotations

import dataclasses
import hashlib
import re
from typing import Dict, List, Optional

import numpy as np
import torch

SEED = 20261201
GROUP = 64


@dataclasses.dataclass(frozen=True)
class Geometry:
    name: str
    hidden: int
    intermediate: int
    experts: int
    top_k: int
    route: str  # "olmoe" | "granite"

    @property
    def expert_bytes(self) -> int:
        """Packed 4-bit Q + 16-bit scales + biases of one expert (gate, up, down)."""
        return self.expert_bytes_at(4)

    def expert_bytes_at(self, bits: int) -> int:
        """Packed Q at `bits` + 16-bit scales + biases of one expert (gate, up, down)."""
        H, I = self.hidden, self.intermediate
        q = 3 * H * I * bits // 8
        sb = 3 * 2 * (H * I // GROUP) * 2
        return q + sb


OLMOE = Geometry("olmoe", 2048, 1024, 64, 8, "olmoe")
GRANITE = Geometry("granite", 1536, 512, 40, 8, "granite")


@dataclasses.dataclass(frozen=True)
class Workload:
    name: str
    geometry: Geometry
    tokens: int
    layers: int = 1
    zipf: bool = False
    description: str = ""
    bits: int = 4                # expert code width
    dtype: str = "bf16"          # activation / scale storage: "bf16" or "f16"
    router: str = "dense"        # "dense" bf16 router or "affine" 4-bit router

    @property
    def torch_dtype(self):
        return torch.float16 if self.dtype == "f16" else torch.bfloat16


WORKLOADS: Dict[str, Workload] = {
    "olmoe_decode_t1": Workload("olmoe_decode_t1", OLMOE, 1, 1,
                                description="OLMoE MoE block, decode 1 token"),
    "olmoe_decode_t8_x16": Workload("olmoe_decode_t8_x16", OLMOE, 8, 16,
                                    description="OLMoE MoE block, decode batch 8, 16 independent layers"),
    "olmoe_prefill_t512": Workload("olmoe_prefill_t512", OLMOE, 512, 1,
                                   description="OLMoE MoE block, prefill 512 tokens"),
    "olmoe_prefill_t4096_zipf": Workload("olmoe_prefill_t4096_zipf", OLMOE, 4096, 1, zipf=True,
                                         description="OLMoE MoE block, prefill 4096 tokens, Zipf(1.1) router bias"),
    "granite_prefill_t2048": Workload("granite_prefill_t2048", GRANITE, 2048, 1,
                                      description="Granite-3.0-3B-A800M MoE block, prefill 2048 tokens"),
    "granite_decode_t32": Workload("granite_decode_t32", GRANITE, 32, 1,
                                   description="Granite-3.0-3B-A800M MoE block, decode batch 32"),
    "olmoe_decode_t8_x16_int8": Workload("olmoe_decode_t8_x16_int8", OLMOE, 8, 16, bits=8,
                                         description="OLMoE MoE block, decode batch 8, 8-bit experts"),
    "olmoe_prefill_t512_int8": Workload("olmoe_prefill_t512_int8", OLMOE, 512, 1, bits=8,
                                        description="OLMoE MoE block, prefill 512 tokens, 8-bit experts"),
    "olmoe_decode_t8_x16_f16": Workload("olmoe_decode_t8_x16_f16", OLMOE, 8, 16, dtype="f16",
                                        router="affine",
                                        description="OLMoE MoE block, decode batch 8, f16 packs with "
                                                    "the affine 4-bit router"),
    "olmoe_prefill_t512_f16": Workload("olmoe_prefill_t512_f16", OLMOE, 512, 1, dtype="f16",
                                       router="affine",
                                       description="OLMoE MoE block, prefill 512 tokens, f16 packs with "
                                                   "the affine 4-bit router"),
}


_SWEEP = re.compile(r"^(olmoe|granite)_t([1-9][0-9]*)$")


def get_workload(name: str) -> Workload:
    """A named workload, or a batch-size point ``olmoe_t<N>`` / ``granite_t<N>``:
    N tokens of that geometry with uniform routing (the sweep across the
    decode-streaming, decode-GEMV and grouped-GEMM paths)."""
    if name in WORKLOADS:
        return WORKLOADS[name]
    m = _SWEEP.match(name)
    if m is None:
        raise KeyError(f"unknown workload {name!r}")
    geom = OLMOE if m.group(1) == "olmoe" else GRANITE
    T = int(m.group(2))
    return Workload(name, geom, T, 1, description=f"{geom.name} MoE block, {T} tokens (batch-size sweep)")


def _key(*parts) -> int:
    h = hashlib.sha256(repr(parts).encode()).digest()
    return int.from_bytes(h[:4], "little")


def _lowbias32(x: torch.Tensor) -> torch.Tensor:
    """lowbias32 integer hash (x holds values in [0, 2^32) as int64).

    x ^= x >> 16; x *= 0x7feb352d; x ^= x >> 15; x *= 0x846ca68b; x ^= x >> 16,
    all modulo 2^32. Products are split into 16-bit halves of the constant so
    no int64 product overflows.
    """
    M = 0xFFFFFFFF

    def mul(v, c):
        lo, hi = c & 0xFFFF, c >> 16
        return ((v * lo) + (((v * hi) & 0xFFFF) << 16)) & M

    x = x ^ (x >> 16)
    x = mul(x, 0x7FEB352D)
    x = x ^ (x >> 15)
    x = mul(x, 0x846CA68B)
    x = x ^ (x >> 16)
    return x


def hash_u32(n: int, key: int, device) -> torch.Tensor:
    """n hashed 32-bit words (int64 tensor, values in [0, 2^32))."""
    i = torch.arange(n, dtype=torch.int64, device=device) & 0xFFFFFFFF
    return _lowbias32(_lowbias32(i) ^ (key & 0xFFFFFFFF))


def _as_int32(u: torch.Tensor) -> torch.Tensor:
    return torch.where(u >= 2 ** 31, u - 2 ** 32, u).to(torch.int32)


def packed_nibbles(shape, key: int, device) -> torch.Tensor:
    n = int(np.prod(shape))
    return _as_int32(hash_u32(n, key, device)).reshape(shape)


def uniform_scales(shape, key: int, device, lo=0.005, hi=0.02, dtype=torch.bfloat16) -> torch.Tensor:
    n = int(np.prod(shape))
    u = (hash_u32(n, key, device) >> 8).to(torch.float32) * (1.0 / (1 << 24))
    s = torch.tensor(lo, dtype=torch.float32) + torch.tensor(hi - lo, dtype=torch.float32).to(device) * u
    return s.to(dtype).reshape(shape)


def normal_bf16(shape, sigma: float, key: int, dtype=torch.bfloat16) -> torch.Tensor:
    rng = np.random.Generator(np.random.PCG64(np.random.SeedSequence([SEED, key])))
    v = rng.standard_normal(size=int(np.prod(shape)), dtype=np.float64) * sigma
    return torch.from_numpy(v.astype(np.float32)).to(dtype).reshape(shape)


def zipf_bias(experts: int, key: int, s: float = 1.1, alpha: float = 0.875) -> torch.Tensor:
    rng = np.random.Generator(np.random.PCG64(np.random.SeedSequence([SEED, key])))
    r = rng.permutation(experts) + 1
    return torch.from_numpy((alpha * (-s * np.log(r.astype(np.float64)))).astype(np.float32))


@dataclasses.dataclass
class LayerWeights:
    router: Optional[torch.Tensor]  # [E, H] dense router (None with an affine router)
    gate_q: torch.Tensor          # [E, I, H/8] int32 (uint32 bits)
    gate_s: torch.Tensor          # [E, I, H/64] bf16
    gate_b: torch.Tensor
    up_q: torch.Tensor
    up_s: torch.Tensor
    up_b: torch.Tensor
    down_q: torch.Tensor          # [E, H, I/8]
    down_s: torch.Tensor          # [E, H, I/64]
    down_b: torch.Tensor
    logit_bias: Optional[torch.Tensor] = None  # [E] fp32
    router_q: Optional[torch.Tensor] = None    # affine router [E, H*router_bits/32]
    router_s: Optional[torch.Tensor] = None    # [E, H/64]
    router_b: Optional[torch.Tensor] = None
    router_bits: int = 4

    def to(self, device) -> "LayerWeights":
        kw = {f.name: (v.to(device) if isinstance(v, torch.Tensor) else v)
              for f in dataclasses.fields(self) for v in (getattr(self, f.name),)}
        return LayerWeights(**kw)

    def tensors(self) -> List[torch.Tensor]:
        return [v for f in dataclasses.fields(self) for v in (getattr(self, f.name),)
                if isinstance(v, torch.Tensor)]


def make_layer(geom: Geometry, layer: int, device="cpu", zipf: bool = False,
               seed_tag: str = "", bits: int = 4, dtype=torch.bfloat16,
               affine_router: bool = False, router_bits: int = 4) -> LayerWeights:
    """Synthetic layer. Codes are uniform over [0, 2^bits) and the bias is
    -2^(bits-1) * scale, so weights are centred on zero; 8-bit scales are
    1/16 of the 4-bit ones, which keeps the weight range the same. Scales,
    biases and the dense router are in `dtype` (bf16 or f16). With
    affine_router the router is an affine matrix of router_bits-bit codes
    (4-bit scales U[0.002, 0.006], 8-bit scales 1/16 of that, bias
    -2^(router_bits-1) * scale) instead of a dense one."""
    if bits not in (4, 8):
        raise ValueError("bits must be 4 or 8")
    E, H, I = geom.experts, geom.hidden, geom.intermediate
    tag = (geom.name, seed_tag, layer)
    if bits != 4:
        tag = tag + (bits,)
    if dtype != torch.bfloat16:
        tag = tag + (str(dtype),)
    w = {}
    shrink = 16.0 / (1 << bits)
    for proj, (N, Kin) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
        w[f"{proj}_q"] = packed_nibbles((E, N, Kin * bits // 32), _key(*tag, proj, "q"), device)
        s = uniform_scales((E, N, Kin // GROUP), _key(*tag, proj, "s"), device,
                           lo=0.005 * shrink, hi=0.02 * shrink, dtype=dtype)
        w[f"{proj}_s"] = s
        w[f"{proj}_b"] = (s.float() * -float(1 << (bits - 1))).to(dtype)
    if affine_router:
        if router_bits not in (4, 8):
            raise ValueError("router_bits must be 4 or 8")
        rtag = ("router",) if router_bits == 4 else ("router", router_bits)
        rshrink = 16.0 / (1 << router_bits)
        w["router"] = None
        w["router_q"] = packed_nibbles((E, H * router_bits // 32), _key(*tag, *rtag, "q"), device)
        rs = uniform_scales((E, H // GROUP), _key(*tag, *rtag, "s"), device, lo=0.002 * rshrink,
                            hi=0.006 * rshrink, dtype=dtype)
        w["router_s"] = rs
        w["router_b"] = (rs.float() * -float(1 << (router_bits - 1))).to(dtype)
        w["router_bits"] = router_bits
    else:
        w["router"] = normal_bf16((E, H), 0.02, _key(*tag, "router"), dtype).to(device)
    lb = zipf_bias(E, _key(*tag, "zipf")).to(device) if zipf else None
    return LayerWeights(logit_bias=lb, **w)


def make_x(geom: Geometry, tokens: int, tag: str = "x", dtype=torch.bfloat16) -> torch.Tensor:
    return normal_bf16((tokens, geom.hidden), 1.0, _key(geom.name, tag, tokens), dtype)


def workload_layer(wl: Workload, layer: int, device="cpu") -> LayerWeights:
    """Layer `layer` of a workload. The two Granite workloads share weights
    (prefill then decode)."""
    tag = "shared" if wl.geometry is GRANITE else wl.name
    return make_layer(wl.geometry, layer, device, zipf=wl.zipf, seed_tag=tag, bits=wl.bits,
                      dtype=wl.torch_dtype, affine_router=wl.router == "affine")


def workload_layers(wl: Workload, device="cpu", layers: Optional[int] = None) -> List[LayerWeights]:
    """Independently seeded layers of a workload (default: the workload's own
    layer count)."""
    n = wl.layers if layers is None else layers
    return [workload_layer(wl, l, device) for l in range(n)]


# Distinct layers a timing loop rotates through: 16 layers of either geometry
# exceed MI355X's 256 MB last-level cache several times over, so every step
# reads its expert weights from HBM, as a model's layer stack would.
TIMING_LAYERS = 16


def workload_x(wl: Workload) -> torch.Tensor:
    return make_x(wl.geometry, wl.tokens, tag=wl.name, dtype=wl.torch_dtype)


def algorithmic_bytes(geom: Geometry, tokens: int, distinct_experts: int, bits: int = 4,
                      affine_router: bool = False) -> int:
    """HBM bytes one MoE layer must move: routed experts' packed weights,
    the router (dense 16-bit, or 4-bit codes plus 16-bit scales and biases),
    the activations in and the result out."""
    E, H = geom.experts, geom.hidden
    router = E * H // 2 + 2 * (E * H // GROUP) * 2 if affine_router else E * H * 2
    return distinct_experts * geom.expert_bytes_at(bits) + router + 2 * tokens * H * 2


def algorithmic_flops(geom: Geometry, tokens: int) -> int:
    H, I, E, K = geom.hidden, geom.intermediate, geom.experts, geom.top_k
    return 2 * tokens * K * 3 * H * I + 2 * tokens * H * E


def gemm_flops(geom: Geometry, routes: int, which: str) -> int:
    H, I = geom.hidden, geom.intermediate
    return 2 * routes * H * I * (2 if which == "gateup" else 1)


__all__ = [
    "Geometry", "Workload", "OLMOE", "GRANITE", "WORKLOADS", "LayerWeights", "make_layer", "workload_layer",
    "make_x", "get_workload", "workload_layers", "workload_x", "algorithmic_bytes", "algorithmic_flops",
    "gemm_flops", "hash_u32", "SEED", "GROUP", "TIMING_LAYERS",
]
