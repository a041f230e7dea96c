"""Stacked expert checkpoints for the MoE block.

The OLMoE exports keep each layer's experts as one stacked tensor per
projection, `model.layers.{l}.mlp.switch_mlp.{gate,up,down}_proj.{weight,
scales,biases}` with the expert on axis 0 (prepare_model.py:67-106, which
builds them byte for byte from the per-expert tensors
`model.layers.{l}.mlp.experts.{e}.{proj}.{suffix}`). That is exactly the
layout tfm_moe_weights takes: packed codes [E, N, K*bits/32] (uint32, codes
LSB first), scales and biases [E, N, K/64] in the storage dtype. The router is
`model.layers.{l}.mlp.gate`: affine-quantised (weight U32 [E, H*bits/32],
scales/biases [E, H/64]) or dense ([E, H]).

`Checkpoint` reads either layout (stacked, or per-expert, stacked on the fly
from the same bytes), validating the safetensors header the way
prepare_model.py:31-63 does and the expert groups the way :66-93 does
(every expert present, one shape and dtype per group, no mix of stacked and
per-expert tensors). Nothing is converted or requantised: a loaded tensor's
bytes are the file's bytes. `write_stacked` writes the stacked file itself.
"""
import json
import math
import mmap
import re
import struct
from pathlib import Path
from typing import Dict, List, Optional, Tuple, Union

import numpy as np
import torch

from .moe import ExpertWeights, MoEBlock

# Safetensors dtypes the MoE tensors use, with their element sizes.
DTYPES = {"U32": 4, "F16": 2, "BF16": 2, "F32": 4}
_NP = {"U32": np.uint32, "F16": np.float16, "BF16": np.uint16, "F32": np.float32}
EXPERT = re.compile(r"^model\.layers\.(\d+)\.mlp\.experts\.(\d+)\.(gate_proj|up_proj|down_proj)\."
                    r"(weight|scales|biases)$")
STACKED = re.compile(r"^model\.layers\.(\d+)\.mlp\.switch_mlp\.(gate_proj|up_proj|down_proj)\."
                     r"(weight|scales|biases)$")
PROJECTIONS = ("gate_proj", "up_proj", "down_proj")
SUFFIXES = ("weight", "scales", "biases")
MAX_HEADER = 16 * 1024 * 1024


class CheckpointError(ValueError):
    """A checkpoint that does not have the stacked-expert layout's form."""


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise CheckpointError(msg)


def read_header(path: Union[str, Path]) -> Tuple[Dict[str, dict], dict, int]:
    """(tensors, metadata, payload start) of a safetensors file, checked as
    prepare_model.py:31-63 checks it: bounded header length, a JSON object
    with no duplicate keys, known dtypes, positive integer shapes, offsets
    whose span is the tensor's byte count, payloads tiling [0, end) with no
    gap or overlap, and a file exactly as long as header + payload."""
    path = Path(path)
    with path.open("rb") as f:
        head = f.read(8)
        _require(len(head) == 8, "missing safetensors header length")
        (n,) = struct.unpack("<Q", head)
        _require(0 < n <= MAX_HEADER, "invalid safetensors header length")
        raw = f.read(n)
        _require(len(raw) == n, "incomplete safetensors header")

    def no_dups(items):
        out = {}
        for k, v in items:
            _require(k not in out, f"duplicate safetensors key {k!r}")
            out[k] = v
        return out

    try:
        header = json.loads(raw, object_pairs_hook=no_dups)
    except json.JSONDecodeError as e:
        raise CheckpointError(f"safetensors header is not JSON: {e}") from None
    _require(isinstance(header, dict), "safetensors header is not an object")
    meta = header.get("__metadata__", {})
    tensors = {k: v for k, v in header.items() if k != "__metadata__"}
    _require(bool(tensors), "no tensors")
    spans = []
    for name, t in tensors.items():
        _require(isinstance(t, dict), f"{name}: not a tensor entry")
        shape, dtype, off = t.get("shape"), t.get("dtype"), t.get("data_offsets")
        _require(dtype in DTYPES, f"{name}: unexpected dtype {dtype!r}")
        _require(isinstance(shape, list) and all(type(d) is int and d > 0 for d in shape),
                 f"{name}: invalid shape")
        _require(isinstance(off, list) and len(off) == 2 and all(type(o) is int and o >= 0 for o in off),
                 f"{name}: invalid data offsets")
        _require(off[1] - off[0] == math.prod(shape) * DTYPES[dtype], f"{name}: byte count mismatch")
        spans.append((off[0], off[1]))
    end = 0
    for a, b in sorted(spans):
        _require(a == end and b > a, "tensor payloads leave a gap or overlap")
        end = b
    _require(path.stat().st_size == 8 + n + end, "file is not exactly header + payload")
    return tensors, meta, 8 + n


class _Entry:
    """One logical tensor: dtype, shape and the file byte ranges that make it
    (one range, or one per expert in expert order)."""

    def __init__(self, dtype: str, shape: List[int], ranges: List[Tuple[int, int]]):
        self.dtype, self.shape, self.ranges = dtype, shape, ranges

    @property
    def nbytes(self) -> int:
        return sum(b - a for a, b in self.ranges)


def stack_plan(tensors: Dict[str, dict], num_layers: int, num_experts: int) -> Dict[str, _Entry]:
    """Logical tensors of a checkpoint with every per-expert group stacked
    (prepare_model.py:66-106): per-expert tensors of layer l, projection p and
    suffix s become `model.layers.{l}.mlp.switch_mlp.{p}.{s}` of shape
    [E] + the expert shape, their bytes in expert order. Every layer must
    have all 9 groups and every group all experts, with one shape and dtype
    (U32 codes; F16 or BF16 scales and biases). Tensors already stacked pass
    through; a group may not appear in both forms."""
    _require(type(num_layers) is int and num_layers > 0 and type(num_experts) is int and num_experts > 0,
             "invalid layer or expert count")
    groups: Dict[Tuple[int, str, str], Dict[int, Tuple[str, dict]]] = {}
    out: Dict[str, _Entry] = {}
    for name, t in tensors.items():
        m = EXPERT.fullmatch(name)
        if m:
            layer, expert = int(m.group(1)), int(m.group(2))
            _require(layer < num_layers and expert < num_experts, f"{name}: layer or expert out of range")
            groups.setdefault((layer, m.group(3), m.group(4)), {})[expert] = (name, t)
            continue
        m = STACKED.fullmatch(name)
        if m:
            _require(int(m.group(1)) < num_layers, f"{name}: layer out of range")
            _require(len(t["shape"]) == 3 and t["shape"][0] == num_experts,
                     f"{name}: stacked tensor is not [experts, rows, columns]")
        else:
            _require(".mlp.experts." not in name, f"{name}: unrecognised expert tensor")
        off = t["data_offsets"]
        out[name] = _Entry(t["dtype"], list(t["shape"]), [(off[0], off[1])])
    for (layer, proj, suffix), members in groups.items():
        name = f"model.layers.{layer}.mlp.switch_mlp.{proj}.{suffix}"
        _require(name not in out, f"{name}: both stacked and per-expert tensors")
        missing = sorted(set(range(num_experts)) - set(members))
        _require(not missing, f"{name}: missing expert(s) {missing}")
        first = members[0][1]
        want = ("U32",) if suffix == "weight" else ("F16", "BF16")
        _require(len(first["shape"]) == 2 and first["dtype"] in want, f"{name}: invalid expert dtype or rank")
        _require(all(t["dtype"] == first["dtype"] and t["shape"] == first["shape"] for _, t in members.values()),
                 f"{name}: experts differ in shape or dtype")
        out[name] = _Entry(first["dtype"], [num_experts] + list(first["shape"]),
                           [tuple(members[e][1]["data_offsets"]) for e in range(num_experts)])
    for layer in range(num_layers):
        for proj in PROJECTIONS:
            for suffix in SUFFIXES:
                name = f"model.layers.{layer}.mlp.switch_mlp.{proj}.{suffix}"
                _require(name in out, f"{name}: missing (every layer needs all 9 expert groups)")
    return out


class Checkpoint:
    """A checkpoint directory (config.json + model.safetensors) or a
    safetensors file with an explicit config, in the stacked or the
    per-expert layout. Reads through a read-only memory map."""

    def __init__(self, path: Union[str, Path], config: Optional[dict] = None):
        path = Path(path)
        if path.is_dir():
            if config is None:
                config = json.loads((path / "config.json").read_text())
            path = path / "model.safetensors"
        _require(config is not None, "a bare safetensors file needs its config")
        _require(config.get("model_type") == "olmoe", "expected an OLMoE configuration")
        self.config = config
        self.path = path
        tensors, self.metadata, self._start = read_header(path)
        self.num_layers = config.get("num_hidden_layers")
        self.num_experts = config.get("num_experts")
        self.entries = stack_plan(tensors, self.num_layers, self.num_experts)
        q = config.get("quantization") or config.get("quantization_config") or {}
        self.bits = int(q.get("bits", 4))
        self.group_size = int(q.get("group_size", 64))
        _require(self.bits in (4, 8) and self.group_size == 64, "expected 4- or 8-bit affine groups of 64")
        self._file = path.open("rb")
        self._map = mmap.mmap(self._file.fileno(), 0, access=mmap.ACCESS_READ)

    def close(self) -> None:
        if getattr(self, "_map", None) is not None:
            self._map.close()
            self._file.close()
            self._map = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def names(self) -> List[str]:
        return sorted(self.entries)

    def tensor_bytes(self, name: str) -> bytes:
        """The logical tensor's bytes (a stacked group: its experts' bytes in
        expert order)."""
        e = self.entries.get(name)
        _require(e is not None, f"{name}: not in the checkpoint")
        return b"".join(self._map[self._start + a:self._start + b] for a, b in e.ranges)

    def array(self, name: str) -> np.ndarray:
        """The tensor as a numpy array of its stored type (BF16 as uint16 bits)."""
        e = self.entries[name]
        return np.frombuffer(self.tensor_bytes(name), dtype=_NP[e.dtype]).reshape(e.shape)

    def torch_tensor(self, name: str, device="cpu") -> torch.Tensor:
        """The tensor in the type the block takes: codes as int32 (the uint32
        bits), F16 as float16, BF16 as bfloat16, F32 as float32."""
        e = self.entries[name]
        a = np.array(self.array(name))  # writable copy
        if e.dtype == "U32":
            t = torch.from_numpy(a.view(np.int32))
        elif e.dtype == "BF16":
            t = torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)
        else:
            t = torch.from_numpy(a)
        return t.to(device)

    def storage_dtype(self) -> torch.dtype:
        d = self.entries["model.layers.0.mlp.switch_mlp.gate_proj.scales"].dtype
        return torch.float16 if d == "F16" else torch.bfloat16

    def layer(self, layer: int, device="cpu") -> ExpertWeights:
        """Layer `layer`'s stacked expert weights and router as the block takes them."""
        _require(0 <= layer < self.num_layers, f"layer {layer} out of range")
        p = f"model.layers.{layer}.mlp."
        kw = {}
        for short, proj in (("gate", "gate_proj"), ("up", "up_proj"), ("down", "down_proj")):
            kw[f"{short}_q"] = self.torch_tensor(f"{p}switch_mlp.{proj}.weight", device)
            kw[f"{short}_s"] = self.torch_tensor(f"{p}switch_mlp.{proj}.scales", device)
            kw[f"{short}_b"] = self.torch_tensor(f"{p}switch_mlp.{proj}.biases", device)
        H = self.config["hidden_size"]
        E = self.num_experts
        if f"{p}gate.scales" in self.entries:
            rq = self.torch_tensor(f"{p}gate.weight", device)
            _require(rq.dim() == 2 and rq.shape[0] == E and (32 * rq.shape[1]) % H == 0,
                     "affine router weight is not [experts, hidden*bits/32]")
            kw.update(router=None, router_q=rq, router_s=self.torch_tensor(f"{p}gate.scales", device),
                      router_b=self.torch_tensor(f"{p}gate.biases", device),
                      router_bits=32 * rq.shape[1] // H)
        else:
            r = self.torch_tensor(f"{p}gate.weight", device)
            _require(tuple(r.shape) == (E, H), "dense router weight is not [experts, hidden]")
            kw["router"] = r
        return ExpertWeights(**kw)

    def block(self) -> MoEBlock:
        """The MoE block of this checkpoint's geometry and storage dtype
        (OLMoE routing: softmax, top-k, unnormalised gates)."""
        c = self.config
        _require(not c.get("norm_topk_prob", False), "normalised top-k gates are not the OLMoE export's rule")
        router = "affine" if "model.layers.0.mlp.gate.scales" in self.entries else "dense"
        return MoEBlock(c["hidden_size"], c["intermediate_size"], self.num_experts, c["num_experts_per_tok"],
                        route="olmoe", bits=self.bits, dtype=self.storage_dtype(), router=router)


def write_stacked(source: Union[str, Path], dest: Union[str, Path], config: dict) -> Dict[str, str]:
    """Write `source` (per-expert or already stacked) as a stacked safetensors
    file at `dest` (which must not exist): every tensor of stack_plan in name
    order, bytes copied unchanged, the source metadata kept. Returns the
    stacked tensors' names and dtypes."""
    dest = Path(dest)
    _require(not dest.exists(), "destination exists")
    tensors, meta, start = read_header(source)
    plan = stack_plan(tensors, config.get("num_hidden_layers"), config.get("num_experts"))
    header: Dict[str, dict] = {}
    if meta:
        header["__metadata__"] = meta
    cur = 0
    for name in sorted(plan):
        e = plan[name]
        header[name] = {"dtype": e.dtype, "shape": e.shape, "data_offsets": [cur, cur + e.nbytes]}
        cur += e.nbytes
    # The reference writer's encoding (prepare_model.py:128): compact separators,
    # non-ASCII text kept as UTF-8 rather than \u escapes.
    enc = json.dumps(header, separators=(",", ":"), ensure_ascii=False).encode("utf8")
    enc += b" " * ((-len(enc)) % 8)
    with Path(source).open("rb") as src, dest.open("xb") as out:
        out.write(struct.pack("<Q", len(enc)))
        out.write(enc)
        for name in sorted(plan):
            for a, b in plan[name].ranges:
                src.seek(start + a)
                left = b - a
                while left:
                    chunk = src.read(min(left, 1 << 20))
                    _require(bool(chunk), "unexpected end of the source file")
                    out.write(chunk)
                    left -= len(chunk)
    return {n: plan[n].dtype for n in sorted(plan)}
