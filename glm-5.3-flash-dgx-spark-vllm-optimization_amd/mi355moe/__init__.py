"""mi355moe: the routed-MoE layer hot path of GLM-style EXL3 models on AMD MI355X (gfx950).

Python host code over libmi355moe.so (hand-written HIP kernels behind the C ABI of include/mi355moe.h):
  ops        torch-level wrappers of every entry point (dequant, router, permutation, rotation, decode forward)
  method     the reference's call contracts: Exl3MoEMethod.apply, apply_exl3_experts, fused_experts, exl3_moe
  layer      production's stacked EXL3 layout and its pointer tables
  fp8        the e4m3 expert variant: block-scaled e4m3 experts, per-token e4m3 activations (fused_experts_fp8)
  e3         the grouped fat-expert tier's stage contract on device row tables (gather / gateup / down, apply)
  e4m3_ext   the e4m3 extension's stage contract (seg_tables / gather2 / fused) and the overlay's run()
  loader     EXL3 checkpoint -> stacked layout with tensor-parallel slicing and expert maps
  synthetic  seeded synthetic layers / routings of the benchmark configurations
  build      in-tree hipcc build of the library
"""
from . import _lib, e3, e4m3_ext, fp8, layer, loader, ops, synthetic  # noqa: F401
from .layer import Exl3Experts  # noqa: F401
from .fp8 import Fp8Experts, fused_experts_fp8  # noqa: F401
from .method import Exl3MoEMethod, apply_exl3_experts, exl3_moe, fused_experts  # noqa: F401

__all__ = ["Exl3Experts", "Exl3MoEMethod", "Fp8Experts", "apply_exl3_experts", "e3", "e4m3_ext", "exl3_moe", "fp8",
           "fused_experts", "fused_experts_fp8", "loader", "ops", "synthetic"]
