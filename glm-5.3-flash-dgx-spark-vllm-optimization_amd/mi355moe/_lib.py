"""ctypes binding of libmi355moe.so (the C ABI declared in include/mi355moe.h).

The library is built in-tree by mi355moe.build (hipcc --offload-arch=gfx950). There is no fallback: if the
library is missing or was built for another ABI version, every operation raises.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
SO_PATH = os.path.join(_HERE, "libmi355moe.so")
ABI_VERSION = 2

F32, F16, BF16, I32, I64 = 0, 1, 2, 3, 4
STAGE_ROUTE, STAGE_GATEUP, STAGE_DOWN, STAGE_COMBINE, STAGE_ALL = 1, 2, 4, 8, 15
PATH_AUTO, PATH_DECODE, PATH_PREFILL = 0, 1, 2
OPT_ACCUMULATE, OPT_BF16_CONTRIB, OPT_E4M3, OPT_PERSISTENT, OPT_DOWN16 = 1, 2, 4, 8, 16
E4M3_DOWN16, E4M3_TOKEN_ROWS, E4M3_LEAN_MAINLOOP = 16, 2048, 8192
LAYER_SHARED_W13_SUH = 1
LAYER_UNIFORM_W13_SUH = 2
PREFILL_MIN_PAIRS = 5120
NOALLOC_SCRATCH_BYTES = 32 << 20
ESCRATCH = 7

_c_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_f = ctypes.c_float
_sz = ctypes.c_size_t


class Exl3LayerDesc(ctypes.Structure):
    """mi355moe_exl3_layer: shape + nine device pointer tables."""
    _fields_ = [("n", _i64), ("hidden", _i64), ("intermediate", _i64),
                ("gate_trellis", _c_p), ("gate_suh", _c_p), ("gate_svh", _c_p),
                ("up_trellis", _c_p), ("up_suh", _c_p), ("up_svh", _c_p),
                ("down_trellis", _c_p), ("down_suh", _c_p), ("down_svh", _c_p), ("flags", _i64)]


class Fp8LayerDesc(ctypes.Structure):
    """mi355moe_fp8_layer: shape + the block-scaled e4m3 weights and their scales (device pointers)."""
    _fields_ = [("n", _i64), ("hidden", _i64), ("intermediate", _i64),
                ("w13", _c_p), ("w13_scale", _c_p), ("w2", _c_p), ("w2_scale", _c_p)]


class MoeError(RuntimeError):
    """A call into libmi355moe.so was rejected (argument check) or failed to launch."""

    def __init__(self, fn: str, code: int):
        self.code = code
        super().__init__(f"{fn}: {strerror(code)} (code {code})")


_LIB = None

# name -> (restype, argtypes)
_SIGS = {
    "mi355moe_abi_version": (_int, []),
    "mi355moe_strerror": (ctypes.c_char_p, [_int]),
    "mi355moe_exl3_dequant": (_int, [_c_p, _i64, _i64, _c_p, _c_p]),
    "mi355moe_sigmoid": (_int, [_c_p, _i64, _int, _c_p, _c_p]),
    "mi355moe_router_logits": (_int, [_c_p, _i64, _i64, _i64, _c_p, _i64, _c_p, _c_p]),
    "mi355moe_router_topk": (_int, [_c_p, _i64, _i64, _c_p, _i64, _f, _int, _c_p, _c_p, _c_p]),
    "mi355moe_route_workspace_bytes": (_i64, [_i64, _i64]),
    "mi355moe_route": (_int, [_c_p, _int, _c_p, _int, _i64, _i64, _c_p, _i64, _i64, _i64, _i64, _c_p, _c_p, _c_p,
                              _c_p, _c_p, _c_p, _c_p, _i64, _c_p, _c_p, _c_p, _sz, _c_p]),
    "mi355moe_route_rows_workspace_bytes": (_i64, [_i64, _i64]),
    "mi355moe_route_rows": (_int, [_c_p, _int, _c_p, _int, _i64, _i64, _c_p, _i64, _i64, _c_p, _c_p, _c_p, _c_p, _c_p,
                                   _c_p, _c_p, _sz, _c_p]),
    "mi355moe_rot_in": (_int, [_c_p, _int, _i64, _i64, _c_p, _c_p, _i64, _c_p, _c_p, _c_p]),
    "mi355moe_moe_workspace_bytes": (_i64, [ctypes.POINTER(Exl3LayerDesc), _i64, _i64]),
    "mi355moe_moe_forward_ids": (_int, [ctypes.POINTER(Exl3LayerDesc), _c_p, _int, _i64, _i64, _c_p, _int, _c_p,
                                        _int, _i64, _c_p, _i64, _f, _c_p, _int, _i64, _c_p, _sz, _c_p]),
    "mi355moe_moe_workspace_bytes_path": (_i64, [ctypes.POINTER(Exl3LayerDesc), _i64, _i64, _int]),
    "mi355moe_moe_forward_ids_ex": (_int, [ctypes.POINTER(Exl3LayerDesc), _c_p, _int, _i64, _i64, _c_p, _int,
                                           _c_p, _int, _i64, _c_p, _i64, _f, _c_p, _int, _i64, _c_p, _sz, _int, _int,
                                           _c_p]),
    "mi355moe_moe_forward_ids_opt": (_int, [ctypes.POINTER(Exl3LayerDesc), _c_p, _int, _i64, _i64, _c_p, _int,
                                            _c_p, _int, _i64, _c_p, _i64, _f, _c_p, _int, _i64, _c_p, _sz, _int,
                                            _int, _int, _c_p]),
    "mi355moe_e4m3_moe_workspace_bytes": (_i64, [ctypes.POINTER(Exl3LayerDesc), _i64, _i64]),
    "mi355moe_e4m3_moe_forward_ids": (_int, [ctypes.POINTER(Exl3LayerDesc), _c_p, _int, _i64, _i64, _c_p, _int,
                                             _c_p, _int, _i64, _c_p, _i64, _f, _c_p, _int, _i64, _c_p, _sz, _int,
                                             _c_p]),
    "mi355moe_exl3_moe_workspace_bytes": (_i64, [ctypes.POINTER(Exl3LayerDesc), _i64]),
    "mi355moe_moe_layer_workspace_bytes": (_i64, [ctypes.POINTER(Exl3LayerDesc), _i64, _i64, _i64]),
    "mi355moe_moe_layer": (_int, [ctypes.POINTER(Exl3LayerDesc), _c_p, _int, _i64, _i64, _c_p, _c_p, _i64, _c_p, _i64,
                                  _f, _int, _f, _c_p, _int, _i64, _c_p, _c_p, _c_p, _sz, _c_p]),
    "mi355moe_moe_layer_noalloc": (_int, [ctypes.POINTER(Exl3LayerDesc), _c_p, _int, _i64, _i64, _c_p, _c_p, _i64,
                                          _c_p, _i64, _f, _int, _f, _c_p, _int, _i64, _c_p, _c_p, _c_p]),
    "mi355moe_moe_split_workspace_bytes": (_i64, [ctypes.POINTER(Exl3LayerDesc), _i64, _i64, _i64]),
    "mi355moe_moe_forward_ids_split": (_int, [ctypes.POINTER(Exl3LayerDesc), _c_p, _int, _i64, _i64, _c_p, _int,
                                              _c_p, _int, _i64, _c_p, _i64, _f, _c_p, _int, _i64, _i64, _c_p, _sz,
                                              _c_p]),
    "mi355moe_e3_tile_rows": (_i64, []),
    "mi355moe_e3_fat_tables": (_int, [_c_p, _i64, _i64, _c_p, _c_p, _i64, _i64, _c_p, _c_p, _c_p, _i64, _c_p, _c_p,
                                      _c_p, _c_p, _c_p, _c_p, _c_p]),
    "mi355moe_e3_gather": (_int, [_c_p, _int, _i64, _i64, _i64, _c_p, _c_p, _i64, _i64, _c_p, _c_p, _c_p, _c_p]),
    "mi355moe_e3_gateup": (_int, [_c_p, _i64, _i64, _i64, _i64, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,
                                  _i64, _c_p, _f, _c_p]),
    "mi355moe_e3_down_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "mi355moe_e3_down": (_int, [_c_p, _i64, _i64, _i64, _i64, _c_p, _c_p, _c_p, _i64, _i64, _c_p, _c_p, _c_p, _c_p,
                                _c_p, _i64, _c_p, _c_p, _sz, _c_p]),
    "mi355moe_e4m3_tile_rows": (_i64, []),
    "mi355moe_e4m3_seg_tables": (_int, [_c_p, _i64, _i64, _i64, _c_p, _c_p, _c_p, _i64, _c_p, _c_p, _c_p]),
    "mi355moe_e4m3_gather2": (_int, [_c_p, _int, _i64, _i64, _i64, _c_p, _c_p, _i64, _i64, _c_p, _c_p, _i64, _c_p,
                                     _c_p, _int, _i64, _c_p]),
    "mi355moe_e4m3_gather_tok": (_int, [_c_p, _int, _i64, _i64, _i64, _c_p, _c_p, _i64, _c_p, _c_p, _int, _i64, _c_p]),
    "mi355moe_e4m3_stage_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "mi355moe_e4m3_gateup": (_int, [_c_p, _c_p, _i64, _i64, _i64, _i64, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,
                                    _i64, _c_p, _f, _i64, _i64, _c_p, _sz, _c_p]),
    "mi355moe_e4m3_actq": (_int, [_c_p, _i64, _i64, _c_p, _i64, _c_p, _c_p, _c_p, _c_p, _c_p, _i64, _c_p, _i64, _i64,
                                  _c_p, _sz, _c_p]),
    "mi355moe_e4m3_down": (_int, [_c_p, _c_p, _i64, _i64, _i64, _i64, _c_p, _c_p, _c_p, _i64, _i64, _c_p, _c_p, _c_p,
                                  _c_p, _c_p, _i64, _c_p, _i64, _i64, _c_p, _sz, _c_p]),
    "mi355moe_e4m3_fused": (_int, [_c_p, _c_p, _i64, _c_p, _c_p, _c_p, _c_p, _int, _i64, _i64, _i64, _i64, _i64, _c_p,
                                   _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _i64, _c_p, _c_p, _c_p, _i64, _c_p,
                                   _f, _int, _c_p, _sz, _c_p]),
    "mi355moe_fp8_quant_rows": (_int, [_c_p, _int, _i64, _i64, _i64, _c_p, _c_p, _c_p]),
    "mi355moe_fp8_moe_workspace_bytes": (_i64, [ctypes.POINTER(Fp8LayerDesc), _i64, _i64]),
    "mi355moe_fp8_moe_forward_ids": (_int, [ctypes.POINTER(Fp8LayerDesc), _c_p, _int, _i64, _i64, _c_p, _int, _c_p,
                                            _int, _i64, _c_p, _i64, _f, _c_p, _int, _i64, _c_p, _sz, _int, _c_p]),
    "mi355moe_sched_item": (_int, [_i64, _i64, _i64, _i64, _i64, ctypes.POINTER(_int), ctypes.POINTER(_int),
                                   ctypes.POINTER(_int)]),
    "mi355moe_exl3_moe": (_int, [ctypes.POINTER(Exl3LayerDesc), _c_p, _i64, _c_p, _c_p, _c_p, _c_p, _i64, _i64,
                                 _int, _int, _int, _int, _int, _int, _int, _int, _int, _int, _f, _c_p, _sz, _c_p]),
}


def exported_symbols() -> list[str]:
    """Every entry point this binding expects the library to export (the declarations of include/mi355moe.h)."""
    return sorted(_SIGS)


def lib() -> ctypes.CDLL:
    """Load libmi355moe.so once; raise ImportError when it is missing or of another ABI version."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(SO_PATH):
            raise ImportError(f"mi355moe: {SO_PATH} is not built; run mi355moe.build.build() "
                              "(or __graft_entry__.build()) first")
        L = ctypes.CDLL(SO_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        v = L.mi355moe_abi_version()
        if v != ABI_VERSION:
            raise ImportError(f"mi355moe: library ABI {v}, binding expects {ABI_VERSION}")
        _LIB = L
    return _LIB


def strerror(code: int) -> str:
    try:
        return lib().mi355moe_strerror(int(code)).decode()
    except ImportError:
        return f"error {code}"


def check(fn: str, rc: int) -> None:
    if rc != 0:
        raise MoeError(fn, rc)
