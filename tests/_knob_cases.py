"""Block outputs of a few fixed cases, for tests/test_gpu_knobs.py: run once
in the test process and once in a child process whose environment sets a
tuning override, so that the override's code path is checked for the same
bits. As a script: python -m tests._knob_cases OUT.npz"""
import sys

import numpy as np
import torch

from trifuse_amd import moe as tmoe
from trifuse_amd import workload as wl

# (geometry, tokens): one and two tokens take the streaming decode kernels
# (the down-weight copies when TFM_DS_PREFETCH=1); 300 OLMoE tokens and 64
# Granite tokens take the grouped GEMM at 32, 16 and 8 quantisation groups
# per row (the scale/bias layouts of TFM_GGEMM_SB_LAYOUT); 8 tokens take the
# decode GEMV kernels (OLMoE with the published slot table, Granite with the
# grouping in every gate/up workgroup: TFM_DECODE_GROUPING swaps them); 32
# tokens of either take 64-row tiles of at most 16 rows, which keep their
# weights two super-steps ahead (TFM_GGEMM_FEW_ROWS=0 one, as the other
# tiles do; =2 also runs the 300 OLMoE and 64 Granite tokens through that
# instance).
CASES = [("olmoe", 1), ("olmoe", 2), ("granite", 1), ("olmoe", 300), ("granite", 64), ("olmoe", 8),
         ("granite", 8), ("olmoe", 32), ("granite", 32)]


def outputs(device="cuda:0"):
    out = {}
    for name, T in CASES:
        geom = wl.OLMOE if name == "olmoe" else wl.GRANITE
        layer = wl.make_layer(geom, 0, device, seed_tag=f"knob{name}")
        wts = tmoe.ExpertWeights.from_layer(layer)
        blk = tmoe.MoEBlock(geom.hidden, geom.intermediate, geom.experts, geom.top_k, route=geom.route)
        x = wl.make_x(geom, T, tag=f"knob{name}{T}").to(device)
        y = blk.forward(x, wts)
        torch.cuda.synchronize()
        out[f"{name}_{T}"] = y.cpu().view(torch.int16).numpy()
    return out


if __name__ == "__main__":
    np.savez(sys.argv[1], **outputs())
