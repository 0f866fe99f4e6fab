"""EXL3 checkpoint loading (mi355moe.loader) on the CPU: a synthetic layer written in the checkpoint's per-expert
naming and read back per tensor-parallel rank must give exactly the column slices (gate/up trellis dim 1, svh) and
row slices (down trellis dim 0, suh) of the full layer (code/fork/docs/prod_exl3_reference.py:644-676); an expert
map selects the local experts; the quant method's per-tensor weight loader produces the same stacked tensors."""
from __future__ import annotations

import pytest
import torch

N_FULL, K, n = 512, 512, 6


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    from mi355moe import loader, synthetic
    full = synthetic.exl3_layer(n, K, N_FULL, seed=3, device="cpu")
    path = str(tmp_path_factory.mktemp("exl3") / "model-00001-of-00001.safetensors")
    loader.save_exl3_layer(path, full, layer_idx=7)
    return path, full


@pytest.mark.parametrize("tp", [1, 2, 4])
def test_tp_slices(ckpt, tp):
    from mi355moe import loader
    path, full = ckpt
    nt = N_FULL // 16 // tp
    for r in range(tp):
        ex = loader.load_exl3_layer(path, 7, n, tp_rank=r, tp_size=tp, device="cpu")
        assert (ex.n, ex.K, ex.N) == (n, K, N_FULL // tp)
        c = slice(r * nt, (r + 1) * nt)
        v = slice(r * nt * 16, (r + 1) * nt * 16)
        assert torch.equal(ex.w13_trellis, full.w13_trellis[:, :, :, c])
        assert torch.equal(ex.w13_svh, full.w13_svh[:, :, v])
        assert torch.equal(ex.w13_suh, full.w13_suh)
        assert torch.equal(ex.w2_trellis, full.w2_trellis[:, c])
        assert torch.equal(ex.w2_suh, full.w2_suh[:, v])
        assert torch.equal(ex.w2_svh, full.w2_svh)
        assert ex.shared_suh == full.shared_suh


def test_expert_map_and_errors(ckpt):
    from mi355moe import loader
    path, full = ckpt
    emap = torch.tensor([-1, 0, -1, 1, 2, -1])
    ex = loader.load_exl3_layer(path, 7, n, tp_rank=1, tp_size=2, expert_map=emap, device="cpu")
    assert ex.n == 3
    assert torch.equal(ex.w13_trellis, full.w13_trellis[[1, 3, 4], :, :, 16:])
    assert torch.equal(ex.w2_svh, full.w2_svh[[1, 3, 4]])
    with pytest.raises(ValueError, match="not divisible"):
        loader.load_exl3_layer(path, 7, n, tp_rank=0, tp_size=3, device="cpu")
    with pytest.raises(KeyError):
        loader.load_exl3_layer(path, 8, n, device="cpu")
    assert loader.suffix_of("experts.w13_trellis") == "trellis" and loader.suffix_of("x.down_proj.svh") == "svh"


def test_quant_method_weight_loader(ckpt):
    """create_weights + the per-tensor weight loader (shard ids w1/w3/w2, global expert ids, expert map) fill the
    stacked parameters exactly as load_exl3_layer does."""
    from safetensors import safe_open

    from mi355moe import Exl3MoEMethod, loader
    path, _ = ckpt
    m = Exl3MoEMethod(tp_rank=1, tp_size=2)
    layer = torch.nn.Module()
    layer.expert_map = torch.tensor([0, -1, 1, 2, -1, 3])
    m.create_weights(layer, 4, K, N_FULL // 2)
    base = "model.language_model.layers.7.mlp.experts"
    with safe_open(path, framework="pt") as f:
        for e in range(n):
            for proj, sid in (("gate_proj", "w1"), ("up_proj", "w3"), ("down_proj", "w2")):
                for suf in ("trellis", "suh", "svh", "mcg"):
                    pname = ("w2_" if sid == "w2" else "w13_") + suf
                    ok = layer.get_parameter(pname).weight_loader(layer.get_parameter(pname),
                                                                  f.get_tensor(f"{base}.{e}.{proj}.{suf}"),
                                                                  f"experts.{pname}", sid, e, return_success=True)
                    assert ok == (int(layer.expert_map[e]) >= 0)
    ref = loader.load_exl3_layer(path, 7, n, 1, 2, expert_map=layer.expert_map, device="cpu")
    for k in ("w13_trellis", "w13_suh", "w13_svh", "w2_trellis", "w2_suh", "w2_svh"):
        assert torch.equal(getattr(layer, k).data, getattr(ref, k)), k
