"""Synthetic OLMoE checkpoints in the per-expert export layout, for the
checkpoint loader's tests: the form of prepare_model.py's self-test
(prepare_model.py:190-227: per-expert gate/up/down weight (U32), scales and
biases (F16) tensors `model.layers.{l}.mlp.experts.{e}.{proj}.{suffix}`, one
non-expert tensor, config.json and tokenizer.json), with the router
`model.layers.{l}.mlp.gate` added (affine: weight U32 + scales + biases, or
dense: weight only).

    python tests/golden/make_checkpoint.py OUT_DIR [--layers 2 --experts 3]

writes a tiny random one; tests call write_checkpoint() with the arrays of a
layer built by trifuse_amd.workload.
"""
import argparse
import json
import struct
from pathlib import Path
from typing import Dict, List, Optional

import numpy as np

_ST = {np.dtype(np.uint32): "U32", np.dtype(np.float16): "F16", np.dtype(np.float32): "F32"}
PROJ = {"gate": "gate_proj", "up": "up_proj", "down": "down_proj"}


def write_safetensors(path: Path, tensors: Dict[str, np.ndarray], metadata: Optional[dict] = None,
                      bf16: frozenset = frozenset()) -> None:
    """Tensors in the given order, payloads back to back. Names in `bf16`
    hold uint16 arrays of bfloat16 bits."""
    header: Dict[str, dict] = {}
    if metadata:
        header["__metadata__"] = metadata
    cur = 0
    for name, a in tensors.items():
        dt = "BF16" if name in bf16 else _ST[a.dtype]
        header[name] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [cur, cur + a.nbytes]}
        cur += a.nbytes
    enc = json.dumps(header).encode()
    enc += b" " * ((-len(enc)) % 8)
    with Path(path).open("wb") as f:
        f.write(struct.pack("<Q", len(enc)))
        f.write(enc)
        for a in tensors.values():
            f.write(np.ascontiguousarray(a).tobytes())


def write_checkpoint(out: Path, layers: List[dict], hidden: int, intermediate: int, top_k: int,
                     bits: int = 4, bf16: bool = False,
                     metadata: Optional[dict] = None) -> Dict[str, np.ndarray]:
    """Per-expert checkpoint directory from `layers`: dicts of numpy arrays
    {gate,up,down}_{q (uint32), s, b (float16, or uint16 bf16 bits)} stacked
    [E, ...], and either router [E, H] or router_q/router_s/router_b.
    `metadata` replaces the default {"format": "mlx"} header metadata.
    Returns the stacked tensors the loader must reproduce (name -> array)."""
    out = Path(out)
    out.mkdir(parents=True, exist_ok=False)
    E = layers[0]["gate_q"].shape[0]
    tensors: Dict[str, np.ndarray] = {}
    stacked: Dict[str, np.ndarray] = {}
    halfs = set()
    for l, lay in enumerate(layers):
        for short, proj in PROJ.items():
            for key, suffix in (("q", "weight"), ("s", "scales"), ("b", "biases")):
                a = lay[f"{short}_{key}"]
                stacked[f"model.layers.{l}.mlp.switch_mlp.{proj}.{suffix}"] = a
                for e in range(E):
                    name = f"model.layers.{l}.mlp.experts.{e}.{proj}.{suffix}"
                    tensors[name] = a[e]
                    if bf16 and key != "q":
                        halfs.add(name)
        if lay.get("router_q") is not None:
            for key, suffix in (("router_q", "weight"), ("router_s", "scales"), ("router_b", "biases")):
                name = f"model.layers.{l}.mlp.gate.{suffix}"
                tensors[name] = stacked[name] = lay[key]
                if bf16 and key != "router_q":
                    halfs.add(name)
        else:
            name = f"model.layers.{l}.mlp.gate.weight"
            tensors[name] = stacked[name] = lay["router"]
            if bf16:
                halfs.add(name)
    norm = np.array([0.25, -2.0] + [1.0] * (hidden - 2), dtype=np.float16)
    tensors["model.norm.weight"] = stacked["model.norm.weight"] = norm
    write_safetensors(out / "model.safetensors", tensors, metadata or {"format": "mlx"}, frozenset(halfs))
    config = {"model_type": "olmoe", "num_hidden_layers": len(layers), "num_experts": E,
              "hidden_size": hidden, "intermediate_size": intermediate, "num_experts_per_tok": top_k,
              "norm_topk_prob": False, "quantization": {"group_size": 64, "bits": bits}}
    (out / "config.json").write_text(json.dumps(config))
    (out / "tokenizer.json").write_text("{}")
    return stacked


def random_layer(rng: np.random.Generator, E: int, H: int, I: int, bits: int = 4, router_bits: int = 4,
                 affine_router: bool = True) -> dict:
    """Random codes, scales and biases of one layer (numbers only, not a model)."""

    def aff(n, k, b=bits):
        q = rng.integers(0, 2 ** 32, size=(E, n, k * b // 32), dtype=np.uint64).astype(np.uint32)
        s = (rng.standard_normal((E, n, k // 64)) * 0.01).astype(np.float16)
        bb = (rng.standard_normal((E, n, k // 64)) * 0.05).astype(np.float16)
        return q, s, bb

    lay = {}
    for short, (n, k) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
        lay[f"{short}_q"], lay[f"{short}_s"], lay[f"{short}_b"] = aff(n, k)
    if affine_router:
        q, s, b = aff(1, H, router_bits)
        lay.update(router_q=q[:, 0], router_s=s[:, 0], router_b=b[:, 0])
    else:
        lay["router"] = (rng.standard_normal((E, H)) * 0.02).astype(np.float16)
    return lay


def main():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("out", type=Path)
    p.add_argument("--layers", type=int, default=2)
    p.add_argument("--experts", type=int, default=3)
    p.add_argument("--hidden", type=int, default=128)
    p.add_argument("--intermediate", type=int, default=128)
    p.add_argument("--top-k", type=int, default=2)
    p.add_argument("--seed", type=int, default=0)
    a = p.parse_args()
    rng = np.random.default_rng(a.seed)
    layers = [random_layer(rng, a.experts, a.hidden, a.intermediate) for _ in range(a.layers)]
    stacked = write_checkpoint(a.out, layers, a.hidden, a.intermediate, a.top_k)
    print(json.dumps({"dir": str(a.out), "stacked_tensors": len(stacked)}))


if __name__ == "__main__":
    main()
