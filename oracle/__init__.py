"""CPU oracle for the routed-MoE hot path -- TEST INFRASTRUCTURE ONLY.

This package is the reference the HIP kernels' results are compared with. Only ``tests/``,
``__graft_entry__.smoke()`` and the CPU-baseline leg of ``bench.py`` may import it, and only for that comparison or
as the timed CPU baseline, never as a product code path. The shipped package (``mi355moe``) never imports it and
fails loudly when its HIP library is missing.

Contents (each function cites the reference file:line it restates):
  exl3.py     EXL3 4-bit trellis format: codebook, tile order, states, unpack, Hadamard (numpy)
  routing.py  router (sigmoid + bias top-k), map_topk_to_local, stable permutation, segment tables
  moe.py      routed-MoE forward: float64 reference and the rounding-faithful kernel paths (C, via ctypes)
  e4m3.py     e4m3 quantisation (RN, saturating), per-token activation quant, block-scaled expert FFN
  e4m3_trellis.py  the trellis-sourced e4m3 variant (per-row e4m3 activations, EXL3 weights rounded to e4m3)
  csrc/       the C restatement (oracle.c) behind moe.py, built by oracle/Makefile into oracle/_build/
"""
