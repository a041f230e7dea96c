"""Stacked-checkpoint loading (trifuse_amd/checkpoint.py) on synthetic
checkpoints in the per-expert export layout (tests/golden/make_checkpoint.py,
the form of prepare_model.py:190-227): the stacked tensors are the
per-expert bytes in expert order, the stacked writer reproduces them, and
malformed checkpoints (a missing expert among them, as prepare_model.py's
self-test checks) are rejected. CPU only."""
import json
import struct

import numpy as np
import pytest
import torch

from tests.golden.make_checkpoint import random_layer, write_checkpoint, write_safetensors
from trifuse_amd import checkpoint as ck


def _tiny(tmp_path, layers=2, experts=3, H=128, I=128, affine_router=True, bf16=False, seed=1):
    rng = np.random.default_rng(seed)
    lays = [random_layer(rng, experts, H, I, affine_router=affine_router) for _ in range(layers)]
    if bf16:  # storage as bf16 bits: reinterpret the half payloads (bytes only matter here)
        for lay in lays:
            for k in list(lay):
                if lay[k].dtype == np.float16:
                    lay[k] = lay[k].view(np.uint16)
    d = tmp_path / "src"
    stacked = write_checkpoint(d, lays, H, I, top_k=2, bf16=bf16)
    return d, lays, stacked


def test_stacked_bytes_are_the_experts_bytes(tmp_path):
    d, lays, stacked = _tiny(tmp_path)
    with ck.Checkpoint(d) as c:
        # prepare_model.py's self-test counts: 2 layers x 9 stacked groups, plus
        # the non-expert tensors (here the norm and the 3 router tensors per layer)
        groups = [n for n in c.names() if ".switch_mlp." in n]
        assert len(groups) == 18
        assert len(c.names()) == 18 + 1 + 2 * 3
        for name, a in stacked.items():
            assert c.tensor_bytes(name) == np.ascontiguousarray(a).tobytes(), name
            assert list(c.entries[name].shape) == list(a.shape)
        # expert e of a stacked group is exactly the per-expert tensor
        a = c.array("model.layers.1.mlp.switch_mlp.down_proj.weight")
        assert a.dtype == np.uint32 and a.shape == lays[1]["down_q"].shape
        np.testing.assert_array_equal(a[2], lays[1]["down_q"][2])


def test_write_stacked_round_trip(tmp_path):
    d, _, stacked = _tiny(tmp_path)
    cfg = json.loads((d / "config.json").read_text())
    out = tmp_path / "stacked.safetensors"
    names = ck.write_stacked(d / "model.safetensors", out, cfg)
    assert sum(".switch_mlp." in n for n in names) == 18
    tensors, meta, _ = ck.read_header(out)
    assert meta == {"format": "mlx"}
    assert not any(".mlp.experts." in n for n in tensors)
    with ck.Checkpoint(out, config=cfg) as c:
        for name, a in stacked.items():
            assert c.tensor_bytes(name) == np.ascontiguousarray(a).tobytes(), name
    # stacking an already stacked file is the identity on the payload
    out2 = tmp_path / "again.safetensors"
    ck.write_stacked(out, out2, cfg)
    assert out2.read_bytes() == out.read_bytes()
    with pytest.raises(ck.CheckpointError, match="exists"):
        ck.write_stacked(d / "model.safetensors", out, cfg)


def test_write_stacked_keeps_utf8_header(tmp_path):
    """Non-ASCII metadata is written as UTF-8 with compact separators, as the
    reference writer encodes its header (prepare_model.py:128), not as \\u escapes."""
    rng = np.random.default_rng(5)
    meta = {"format": "mlx", "note": "Grüße π 模型"}
    d = tmp_path / "utf8"
    write_checkpoint(d, [random_layer(rng, 2, 128, 128)], 128, 128, top_k=2, metadata=meta)
    cfg = json.loads((d / "config.json").read_text())
    out = tmp_path / "stacked_utf8.safetensors"
    ck.write_stacked(d / "model.safetensors", out, cfg)
    raw = out.read_bytes()
    (n,) = struct.unpack("<Q", raw[:8])
    head = raw[8:8 + n]
    assert "Grüße π 模型".encode("utf8") in head
    assert b"\\u" not in head
    tensors, got, _ = ck.read_header(out)
    assert got == meta
    expect = {"__metadata__": meta}
    expect.update({k: {"dtype": v["dtype"], "shape": v["shape"], "data_offsets": v["data_offsets"]}
                   for k, v in tensors.items()})
    enc = json.dumps(expect, separators=(",", ":"), ensure_ascii=False).encode("utf8")
    enc += b" " * ((-len(enc)) % 8)
    assert head == enc


def test_layer_weights(tmp_path):
    d, lays, _ = _tiny(tmp_path)
    with ck.Checkpoint(d) as c:
        assert c.storage_dtype() == torch.float16 and c.bits == 4
        w = c.layer(1)
        assert w.router is None and w.router_bits == 4
        assert w.gate_q.dtype == torch.int32 and tuple(w.gate_q.shape) == lays[1]["gate_q"].shape
        assert w.down_s.dtype == torch.float16
        np.testing.assert_array_equal(w.up_q.numpy().view(np.uint32), lays[1]["up_q"])
        np.testing.assert_array_equal(w.router_s.numpy(), lays[1]["router_s"])
        with pytest.raises(ck.CheckpointError, match="out of range"):
            c.layer(2)


def test_dense_router_and_bf16(tmp_path):
    d, lays, _ = _tiny(tmp_path, layers=1, affine_router=False, bf16=True)
    with ck.Checkpoint(d) as c:
        assert c.storage_dtype() == torch.bfloat16
        w = c.layer(0)
        assert w.router_q is None and w.router.dtype == torch.bfloat16
        np.testing.assert_array_equal(w.router.view(torch.int16).numpy().view(np.uint16), lays[0]["router"])
        np.testing.assert_array_equal(w.gate_b.view(torch.int16).numpy().view(np.uint16), lays[0]["gate_b"])


def test_router_bits_inferred(tmp_path):
    rng = np.random.default_rng(3)
    lay = random_layer(rng, 4, 128, 128, router_bits=8)
    d = tmp_path / "r8"
    write_checkpoint(d, [lay], 128, 128, top_k=2)
    with ck.Checkpoint(d) as c:
        assert c.layer(0).router_bits == 8


def _rewrite(tmp_path, src, edit, name="bad"):
    """A copy of checkpoint dir `src` whose header goes through edit(tensors dict)."""
    tensors, meta, start = ck.read_header(src / "model.safetensors")
    payload = (src / "model.safetensors").read_bytes()[start:]
    edit(tensors)
    header = dict(tensors)
    header["__metadata__"] = meta
    enc = json.dumps(header).encode()
    enc += b" " * ((-len(enc)) % 8)
    d = tmp_path / name
    d.mkdir()
    (d / "config.json").write_text((src / "config.json").read_text())
    (d / "model.safetensors").write_bytes(struct.pack("<Q", len(enc)) + enc + payload)
    return d


def test_missing_expert_rejected(tmp_path):
    d, _, _ = _tiny(tmp_path)

    def drop(t):
        # remove expert 1's tensor and keep the payload tiling: the removed
        # bytes become a renamed non-expert tensor
        t["model.layers.0.extra"] = t.pop("model.layers.0.mlp.experts.1.gate_proj.weight")

    bad = _rewrite(tmp_path, d, drop)
    with pytest.raises(ck.CheckpointError, match=r"missing expert\(s\) \[1\]"):
        ck.Checkpoint(bad)


def test_mixed_layout_rejected(tmp_path):
    d, _, _ = _tiny(tmp_path)

    def mix(t):
        # one group present both stacked and per expert: the router scales
        # (3 x 2 halves) renamed to a stacked [3, 1, 2] up_proj.scales
        e = t.pop("model.layers.0.mlp.gate.scales")
        e["shape"] = [3, 1, 2]
        t["model.layers.0.mlp.switch_mlp.up_proj.scales"] = e

    with pytest.raises(ck.CheckpointError, match="both stacked and per-expert"):
        ck.Checkpoint(_rewrite(tmp_path, d, mix))


def test_mismatched_expert_rejected(tmp_path):
    d, _, _ = _tiny(tmp_path)

    def reshape(t):
        e = t["model.layers.1.mlp.experts.2.down_proj.scales"]
        e["shape"] = [e["shape"][1], e["shape"][0]]  # same byte count, other shape

    with pytest.raises(ck.CheckpointError, match="differ in shape or dtype"):
        ck.Checkpoint(_rewrite(tmp_path, d, reshape))


def test_malformed_files_rejected(tmp_path):
    d, _, _ = _tiny(tmp_path)
    f = d / "model.safetensors"
    data = f.read_bytes()
    cases = {
        "truncated": data[:-2],
        "trailing": data + b"\0",
        "short": data[:5],
    }
    for name, raw in cases.items():
        p = tmp_path / f"{name}.safetensors"
        p.write_bytes(raw)
        with pytest.raises(ck.CheckpointError):
            ck.read_header(p)
    # a payload gap
    p = tmp_path / "gap.safetensors"
    write_safetensors(p, {"a": np.zeros(4, np.float16), "b": np.zeros(4, np.float16)})
    tensors, _, _ = ck.read_header(p)
    (n,) = struct.unpack("<Q", p.read_bytes()[:8])
    hdr = json.loads(p.read_bytes()[8:8 + n])
    hdr["b"]["data_offsets"] = [10, 18]
    enc = json.dumps(hdr).encode()
    enc += b" " * ((-len(enc)) % 8)
    p.write_bytes(struct.pack("<Q", len(enc)) + enc + b"\0" * 18)
    with pytest.raises(ck.CheckpointError, match="gap or overlap"):
        ck.read_header(p)
    # a duplicate key
    raw = b'{"a":{"dtype":"F16","shape":[1],"data_offsets":[0,2]},"a":{"dtype":"F16","shape":[1],"data_offsets":[0,2]}}'
    raw += b" " * ((-len(raw)) % 8)
    p.write_bytes(struct.pack("<Q", len(raw)) + raw + b"\0\0")
    with pytest.raises(ck.CheckpointError, match="duplicate"):
        ck.read_header(p)


def test_non_olmoe_config_rejected(tmp_path):
    d, _, _ = _tiny(tmp_path)
    cfg = json.loads((d / "config.json").read_text())
    cfg["model_type"] = "llama"
    with pytest.raises(ck.CheckpointError, match="OLMoE"):
        ck.Checkpoint(d / "model.safetensors", config=cfg)
