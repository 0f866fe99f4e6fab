"""EXL3 checkpoint loading into production's stacked expert layout, with tensor-parallel slicing.

A GLM-5.3 EXL3 checkpoint stores every routed expert as separate tensors (safetensors):
  {prefix}.{layer}.mlp.experts.{e}.{gate_proj|up_proj}.trellis   int16 [K/16, N/16, 64]
  {prefix}.{layer}.mlp.experts.{e}.{gate_proj|up_proj}.suh       fp16  [K]
  {prefix}.{layer}.mlp.experts.{e}.{gate_proj|up_proj}.svh       fp16  [N]
  {prefix}.{layer}.mlp.experts.{e}.down_proj.trellis             int16 [N/16, K/16, 64]
  {prefix}.{layer}.mlp.experts.{e}.down_proj.suh                 fp16  [N]
  {prefix}.{layer}.mlp.experts.{e}.down_proj.svh                 fp16  [K]
  {prefix}.{layer}.mlp.experts.{e}.{gate_proj|up_proj|down_proj}.mcg   int32 [1] (0xCBAC1FED)
with N the full intermediate size (code/fork/tests/moee4m3/extract_layer.py:47-68 reads the same names).

Tensor parallelism (code/fork/docs/prod_exl3_reference.py:644-676): gate and up are column-parallel (trellis dim 1,
svh dim 0 sliced), down is row-parallel (trellis dim 0, suh dim 0 sliced); rank r of tp keeps the r-th of tp equal
slices. Each rank's routed output is then a partial sum over its N slice, and the ranks' outputs add up to the full
layer's (the all-reduce that follows the layer). Expert parallelism: an expert map (global id -> local id or -1)
selects the experts this rank loads, as production's loader maps global to local ids (prod:2164-2221).
"""
from __future__ import annotations

import os
from typing import Iterable

import torch

from .layer import MCG_MARKER, Exl3Experts

EXL3_SUFFIXES = ("trellis", "suh", "svh", "mcg")
PROJ = ("gate_proj", "up_proj", "down_proj")


def _slice_tp(t: torch.Tensor, dim: int, tp_rank: int, tp_size: int) -> torch.Tensor:
    """The tp_rank-th of tp_size equal slices of t along dim (t itself when tp_size is 1)."""
    if tp_size <= 1:
        return t
    if not 0 <= tp_rank < tp_size:
        raise ValueError(f"tp_rank {tp_rank} outside [0, {tp_size})")
    size = int(t.shape[dim])
    if size % tp_size:
        raise ValueError(f"cannot cut axis {dim} ({size} entries) into {tp_size} equal tensor-parallel slices: "
                         "not divisible")
    step = size // tp_size
    return t.narrow(dim, step * tp_rank, step).contiguous()


def shard_exl3_col(loaded: torch.Tensor, suffix: str, tp_rank: int, tp_size: int) -> torch.Tensor:
    """Gate / up (column-parallel over N): trellis dim 1 (N tiles) and svh dim 0 are sliced; suh and mcg are whole."""
    if suffix == "trellis":
        return _slice_tp(loaded, 1, tp_rank, tp_size)
    if suffix == "svh":
        return _slice_tp(loaded, 0, tp_rank, tp_size)
    return loaded.contiguous()


def shard_exl3_row(loaded: torch.Tensor, suffix: str, tp_rank: int, tp_size: int) -> torch.Tensor:
    """Down (row-parallel over N): trellis dim 0 (N tiles) and suh dim 0 are sliced; svh and mcg are whole."""
    if suffix in ("trellis", "suh"):
        return _slice_tp(loaded, 0, tp_rank, tp_size)
    return loaded.contiguous()


def suffix_of(name: str) -> str:
    """The EXL3 tensor kind of a checkpoint (or mapped parameter) name: its last component, or the part after the
    last underscore of it (w13_trellis -> trellis)."""
    tail = name.rsplit(".", 1)[-1]
    for s in EXL3_SUFFIXES:
        if tail == s or tail.endswith("_" + s):
            return s
    raise ValueError(f"not an EXL3 tensor name: {name}")


def load_into(layer: torch.nn.Module, loaded: torch.Tensor, weight_name: str, shard_id: str, expert_id: int,
              tp_rank: int = 0, tp_size: int = 1, expert_map: torch.Tensor | None = None) -> bool:
    """Copy one checkpoint tensor of one expert into the layer's stacked parameters (the weight-loader step of
    code/fork/docs/prod_exl3_reference.py:2164-2221): shard_id w1 (gate) / w3 (up) go to w13_*[local, 0 / 1] after
    the column slice, w2 (down) to w2_*[local] after the row slice. expert_id is global; with an expert map, experts
    that are not local are skipped (returns False). Shapes must match exactly."""
    if expert_map is not None:
        local = int(expert_map[int(expert_id)])
        if local < 0:
            return False
        expert_id = local
    suffix = suffix_of(weight_name)
    src = loaded.detach().contiguous()
    if shard_id in ("w1", "w3"):
        part = shard_exl3_col(src, suffix, tp_rank, tp_size)
        dest = getattr(layer, "w13_" + suffix).data[expert_id, 0 if shard_id == "w1" else 1]
    elif shard_id == "w2":
        part = shard_exl3_row(src, suffix, tp_rank, tp_size)
        dest = getattr(layer, "w2_" + suffix).data[expert_id]
    else:
        raise ValueError(f"shard_id must be w1, w2 or w3, got {shard_id!r}")
    if suffix == "mcg":
        part = part.reshape(dest.shape)
    if tuple(dest.shape) != tuple(part.shape):
        raise RuntimeError(f"{weight_name} (shard {shard_id}, expert {expert_id}) has shape {tuple(part.shape)} after "
                           f"tensor-parallel slicing, but the parameter slot holds {tuple(dest.shape)}")
    dest.copy_(part)
    return True


def _open_files(path: str | Iterable[str]) -> list[str]:
    if isinstance(path, (list, tuple)):
        return list(path)
    if os.path.isdir(path):
        return sorted(os.path.join(path, f) for f in os.listdir(path) if f.endswith(".safetensors"))
    return [path]


def load_exl3_layer(path: str | Iterable[str], layer_idx: int, num_experts: int, tp_rank: int = 0, tp_size: int = 1,
                    expert_map: torch.Tensor | None = None, device="cuda",
                    prefix: str = "model.language_model.layers") -> Exl3Experts:
    """Build one MoE layer's Exl3Experts for this rank from an EXL3 checkpoint (a safetensors file, a list of them, or
    a directory): the rank's experts (all, or those an expert map makes local) in production's stacked layout with
    this rank's tensor-parallel slice. Tensors are read with safetensors (no code runs from the file); the mcg marker
    of every matrix is checked."""
    from safetensors import safe_open

    files = _open_files(path)
    index: dict[str, str] = {}
    for f in files:
        with safe_open(f, framework="pt", device="cpu") as h:
            for k in h.keys():
                index[k] = f
    base = f"{prefix}.{layer_idx}.mlp.experts"
    probe = f"{base}.0.gate_proj.trellis"
    if probe not in index:
        raise KeyError(f"{probe} not in the checkpoint")
    local_ids = list(range(num_experts)) if expert_map is None else [
        e for e in range(num_experts) if int(expert_map[e]) >= 0]
    n_local = len(local_ids)
    handles: dict[str, object] = {}

    def get(name: str) -> torch.Tensor:
        f = index.get(name)
        if f is None:
            raise KeyError(f"{name} not in the checkpoint")
        if f not in handles:
            handles[f] = safe_open(f, framework="pt", device="cpu").__enter__()
        return handles[f].get_tensor(name)

    g0 = shard_exl3_col(get(probe), "trellis", tp_rank, tp_size)
    kt, nt, words = g0.shape
    if words != 64:
        raise ValueError(f"only 4-bit trellis tiles (64 int16 words) are supported, got {words}")
    K, N = kt * 16, nt * 16
    dev = torch.device(device)
    layer = torch.nn.Module()
    shapes = {"w13_trellis": ((n_local, 2, kt, nt, 64), torch.int16), "w13_suh": ((n_local, 2, K), torch.float16),
              "w13_svh": ((n_local, 2, N), torch.float16), "w13_mcg": ((n_local, 2, 1), torch.int32),
              "w2_trellis": ((n_local, nt, kt, 64), torch.int16), "w2_suh": ((n_local, N), torch.float16),
              "w2_svh": ((n_local, K), torch.float16), "w2_mcg": ((n_local, 1), torch.int32)}
    for name, (shape, dt) in shapes.items():
        layer.register_parameter(name, torch.nn.Parameter(torch.empty(shape, dtype=dt), requires_grad=False))
    emap = None
    if expert_map is not None:
        emap = torch.full((num_experts,), -1, dtype=torch.int64)
        for i, e in enumerate(local_ids):
            emap[e] = i
    try:
        for e in local_ids:
            for proj, sid in zip(PROJ, ("w1", "w3", "w2")):
                for suffix in EXL3_SUFFIXES:
                    name = f"{base}.{e}.{proj}.{suffix}"
                    load_into(layer, get(name), name, sid, e, tp_rank, tp_size, emap)
    finally:
        for h in handles.values():
            h.__exit__(None, None, None)
    for name in ("w13_mcg", "w2_mcg"):
        if not bool(torch.all(getattr(layer, name) == MCG_MARKER)):
            raise RuntimeError(f"{name}: every entry must be the mcg codebook marker {MCG_MARKER} (0xCBAC1FED as "
                               "int32); this checkpoint uses another trellis codebook")
    return Exl3Experts(*(getattr(layer, k).data.to(dev) for k in
                         ("w13_trellis", "w13_suh", "w13_svh", "w2_trellis", "w2_suh", "w2_svh")))


def save_exl3_layer(path: str, experts: Exl3Experts, layer_idx: int, prefix: str = "model.language_model.layers",
                    first_expert: int = 0) -> None:
    """Write a layer's experts in the checkpoint's per-expert naming (the inverse of load_exl3_layer at tp = 1;
    used to build test checkpoints)."""
    from safetensors.torch import save_file

    out = {}
    base = f"{prefix}.{layer_idx}.mlp.experts"
    cpu = {k: getattr(experts, k).cpu() for k in ("w13_trellis", "w13_suh", "w13_svh", "w2_trellis", "w2_suh",
                                                  "w2_svh")}
    mcg = torch.tensor([MCG_MARKER], dtype=torch.int32)
    for i in range(experts.n):
        e = first_expert + i
        for j, proj in enumerate(("gate_proj", "up_proj")):
            out[f"{base}.{e}.{proj}.trellis"] = cpu["w13_trellis"][i, j].contiguous()
            out[f"{base}.{e}.{proj}.suh"] = cpu["w13_suh"][i, j].contiguous()
            out[f"{base}.{e}.{proj}.svh"] = cpu["w13_svh"][i, j].contiguous()
            out[f"{base}.{e}.{proj}.mcg"] = mcg.clone()
        out[f"{base}.{e}.down_proj.trellis"] = cpu["w2_trellis"][i].contiguous()
        out[f"{base}.{e}.down_proj.suh"] = cpu["w2_suh"][i].contiguous()
        out[f"{base}.{e}.down_proj.svh"] = cpu["w2_svh"][i].contiguous()
        out[f"{base}.{e}.down_proj.mcg"] = mcg.clone()
    save_file(out, path)
