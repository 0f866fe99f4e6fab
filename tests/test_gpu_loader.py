"""A layer loaded from an EXL3 checkpoint as two tensor-parallel ranks (mi355moe.loader), each rank's slice run
through Exl3MoEMethod.apply: the two partial outputs add up to the full layer's routed output (the all-reduce that
follows the layer in production), checked against the float64 oracle of the unsharded layer, on the decode and the
grouped prefill paths."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe, routing

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("T", [8, 600])
def test_tp2_shards_sum_to_full_layer(cuda, tmp_path, T):
    from mi355moe import Exl3MoEMethod, loader, synthetic
    n, K, NF, topk = 8, 1024, 1024, 8
    print(f"TP=2 loaded shards, T={T}", flush=True)
    full = synthetic.calibrated_layer(n, K, NF, seed=21, device="cpu")
    path = str(tmp_path / "layer.safetensors")
    loader.save_exl3_layer(path, full, layer_idx=3)
    x = synthetic.activations(T, K, seed=22, device=cuda)
    ids = synthetic.random_ids(T, n, topk, seed=23, device=cuda)
    w = synthetic.softmax_weights(T, topk, seed=24, device=cuda)
    parts = []
    for r in range(2):
        layer = torch.nn.Module()
        layer._mi355_experts = loader.load_exl3_layer(path, 3, n, tp_rank=r, tp_size=2, device=cuda)
        parts.append(Exl3MoEMethod(tp_rank=r, tp_size=2).apply(layer, x, w, ids).float())
    got = (parts[0] + parts[1]).cpu().numpy()
    lay = {k: getattr(full, k).numpy() for k in ("w13_trellis", "w13_suh", "w13_svh", "w2_trellis", "w2_suh",
                                                  "w2_svh")}
    local = routing.map_topk_to_local(ids.cpu().numpy(), n)
    tok, exx, w16 = moe.pairs_from_routing(local, w.cpu().numpy(), n, topk)
    mode = "f64" if T * topk < 4096 else "f64_pre"                     # decode path: limit after SiLU; grouped: before
    ref = moe.forward(lay, x.to(torch.float16).cpu().numpy(), tok, exx, w16, 10.0, mode)
    r = _rel(got, ref)
    print(f"  rel_l2 of rank0 + rank1 vs the full layer's float64 output {r:.3e}", flush=True)
    assert r <= 5e-3
