"""Writes the small golden vectors in this folder from the CPU oracle.

    python tests/golden/make_golden.py

routing.npz : tie-rich bf16 logit rows (exact ties, NaN, +-inf, all-equal rows)
              for E in {64, 40} with the OLMoE and Granite routes (ids, gates),
              the OLMoE softmax, and the stable grouping of the OLMoE routes.
block.npz   : a tiny MoE block (E=4, H=128, I=64, K=2): packed weights, x, the
              routes and the fp64 block output.
The oracle itself is pinned by tests/test_oracle.py; these files anchor it
against regressions and give the GPU tests fixed vectors.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle  # noqa: E402


def tie_logits(rng, T, E):
    v = rng.integers(-6, 6, size=(T, E)).astype(np.float32) * 0.25
    v[0] = 0.5
    v[1, 3] = np.nan
    v[2, ::7] = np.nan
    v[3] = np.nan
    v[4, 5] = np.inf
    v[5, 9] = -np.inf
    v[6] = -np.inf
    v[7:16] = rng.standard_normal((9, E)).astype(np.float32) * 3
    return oracle.f32_to_bf16(v)


def main():
    rng = np.random.default_rng(7)
    out = {}
    for E in (64, 40):
        lg = tie_logits(rng, 32, E)
        oi, og = oracle.route_olmoe(lg, 8)
        gi, gg = oracle.route_granite(lg, 8)
        order, inverse, offsets = oracle.group(oi.reshape(-1), E)
        out.update({f"logits_e{E}": lg, f"olmoe_idx_e{E}": oi, f"olmoe_gates_e{E}": og,
                    f"granite_idx_e{E}": gi, f"granite_gates_e{E}": gg,
                    f"olmoe_probs_e{E}": oracle.olmoe_softmax(lg),
                    f"order_e{E}": order, f"inverse_e{E}": inverse, f"offsets_e{E}": offsets})
    np.savez_compressed(os.path.join(HERE, "routing.npz"), **out)

    E, H, I, K, T = 4, 128, 64, 2, 6
    blk = {}
    for proj, (N, Kin) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
        blk[proj + "_q"] = rng.integers(0, 2 ** 32, size=(E, N, Kin // 8), dtype=np.uint64).astype(np.uint32)
        s = oracle.f32_to_bf16(rng.uniform(0.005, 0.02, size=(E, N, Kin // 64)))
        blk[proj + "_s"] = s
        blk[proj + "_b"] = oracle.f32_to_bf16(-8 * oracle.bf16_to_f32(s))
    blk["x"] = oracle.f32_to_bf16(rng.standard_normal((T, H)))
    blk["router"] = oracle.f32_to_bf16(rng.standard_normal((E, H)) * 0.02)
    logits = oracle.router_logits(blk["x"], blk["router"])
    idx, g = oracle.route_olmoe(logits, K)

    class Wts:
        pass

    w = Wts()
    for k, v in blk.items():
        setattr(w, k, v)
    blk["idx"] = idx
    blk["gates"] = g
    blk["y"] = oracle.moe_reference(blk["x"], idx, oracle.bf16_to_f32(g), w)
    np.savez_compressed(os.path.join(HERE, "block.npz"), **blk)
    print("wrote routing.npz, block.npz")


if __name__ == "__main__":
    main()
