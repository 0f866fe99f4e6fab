"""The C-ABI library loads and exports every entry point include/mi355moe.h declares; host-side planning entry
points (no device work) answer; the Python layer rejects bad arguments before any device call. No GPU needed."""
from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "mi355moe.h")


def _declared() -> set[str]:
    src = open(HEADER).read()
    return set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(mi355moe_\w+)\s*\(", src, re.M))


def test_header_declarations_match_binding():
    from mi355moe import _lib
    assert _declared() == set(_lib.exported_symbols())


def test_library_exports_every_declared_symbol():
    from mi355moe import _lib
    L = _lib.lib()
    for name in sorted(_declared()):
        assert getattr(L, name) is not None, name
    assert L.mi355moe_abi_version() == _lib.ABI_VERSION
    assert L.mi355moe_strerror(2) == b"unsupported shape"


def _fake_desc(n=288, K=4096, N=1024):
    from mi355moe import _lib
    d = _lib.Exl3LayerDesc()
    d.n, d.hidden, d.intermediate = n, K, N
    for f, t in d._fields_[3:]:
        if t is ctypes.c_void_p:
            setattr(d, f, ctypes.c_void_p(0x1000))  # never dereferenced by the host-side planners
    d.flags = 1
    return d


def test_workspace_planners_answer_without_a_gpu():
    from mi355moe import _lib
    L = _lib.lib()
    d = _fake_desc()
    b8 = L.mi355moe_moe_workspace_bytes(ctypes.byref(d), 8, 8)
    b64 = L.mi355moe_moe_workspace_bytes(ctypes.byref(d), 64, 8)
    assert 0 < b8 < b64 < 1 << 31
    assert L.mi355moe_exl3_moe_workspace_bytes(ctypes.byref(d), 64) > 0
    bad = _fake_desc(K=4000)
    assert L.mi355moe_moe_workspace_bytes(ctypes.byref(bad), 8, 8) == -1
    assert L.mi355moe_route_workspace_bytes(65536, 288) > 0
    # the automatic choice: prefill layout (rotated rows + fp32 accumulator) from 5120 pairs with shared suh
    big = L.mi355moe_moe_workspace_bytes(ctypes.byref(d), 8192, 8)
    assert big >= 8192 * 8 * (4096 + 1024) * 2 + 8192 * 4096 * 4
    assert L.mi355moe_moe_workspace_bytes_path(ctypes.byref(d), 8192, 8, 1) != big      # forced decode layout
    assert L.mi355moe_moe_workspace_bytes_path(ctypes.byref(d), 8, 8, 3) == -1         # bad path


def test_argument_errors_before_any_launch():
    from mi355moe import _lib
    L = _lib.lib()
    null = ctypes.c_void_p(0)
    assert L.mi355moe_exl3_dequant(null, 16, 8, null, null) == 1                     # EINVAL
    assert L.mi355moe_exl3_dequant(ctypes.c_void_p(0x1000), 16, 7, ctypes.c_void_p(0x1000), null) == 2
    assert L.mi355moe_router_topk(ctypes.c_void_p(8), 1, 2000, null, 8, 2.5, 1, ctypes.c_void_p(8),
                                  ctypes.c_void_p(8), null) == 3                       # E > 1024
    d = _fake_desc()
    p = ctypes.c_void_p(0x1000)
    # exl3_moe contract: only SiLU, 4 bits, mcg codebook
    args = [ctypes.byref(d), p, 4, p, p, p, p, 32, 128]
    tail = [0, 0, 0, 0.0, p, 1 << 30, null]
    assert L.mi355moe_exl3_moe(*args, 1, 4, 4, 4, 1, 0, 1, 0, 1, 0, *tail[3:]) == 6   # act_function 1
    assert L.mi355moe_exl3_moe(*args, 0, 3, 4, 4, 1, 0, 1, 0, 1, 0, *tail[3:]) == 6   # 3 bits
    assert L.mi355moe_exl3_moe(*args, 0, 4, 4, 4, 1, 1, 1, 0, 1, 0, *tail[3:]) == 6   # mul1 codebook


def test_forward_options_are_checked_before_any_launch():
    from mi355moe import _lib
    L = _lib.lib()
    d = _fake_desc()
    p = ctypes.c_void_p(0x1000)
    args = [ctypes.byref(d), p, _lib.BF16, 1024, 4, p, _lib.I32, p, _lib.F32, 8, None, 0, 10.0, p, _lib.BF16, 1024,
            p, 1 << 30]
    assert L.mi355moe_moe_forward_ids_opt(*args, _lib.PATH_AUTO, _lib.STAGE_ALL, 16, None) == 1         # unknown bit
    assert L.mi355moe_moe_forward_ids_opt(*args, _lib.PATH_DECODE, _lib.STAGE_ALL, _lib.OPT_E4M3, None) == 1


def test_python_layer_rejects_cpu_tensors_and_bad_shapes():
    from mi355moe import ops
    with pytest.raises(ValueError):
        ops.dequant(torch.zeros(4, 8, 64, dtype=torch.int16))
    with pytest.raises(ValueError):
        ops.router_topk(torch.zeros(2, 8), 2)
    from mi355moe.layer import Exl3Experts
    with pytest.raises(ValueError):
        Exl3Experts(torch.zeros(2, 2, 4, 4, 48, dtype=torch.int16), *[torch.zeros(1)] * 5)


def test_expert_pointer_tables_require_16_byte_alignment():
    from mi355moe.layer import _table
    t = torch.zeros(3, 2, 256, dtype=torch.float16)
    tab = _table(t, (1,))
    assert tab.tolist() == [t.data_ptr() + 512 + 1024 * e for e in range(3)]
    with pytest.raises(ValueError):
        _table(torch.zeros(3 * 256 + 1, dtype=torch.float16)[1:].view(3, 256), ())   # base 2 bytes off
    with pytest.raises(ValueError):
        _table(torch.zeros(3, 260, dtype=torch.float16), ())                          # 520-byte expert stride


def test_workspace_growth_keeps_old_buffer_and_refuses_under_capture(monkeypatch):
    """Host logic of the persistent workspace (on the CPU device): growth retires the old buffer without freeing
    it, and growth while a graph is being captured raises."""
    import torch
    from mi355moe import ops
    dev = torch.device("cpu")
    key = (dev.type, dev.index)
    ops._WS.pop(key, None)
    ops._RETIRED.pop(key, None)
    a = ops.workspace(dev, 100)
    assert a.numel() == 1 << 20 and ops.workspace(dev, 1 << 20) is a
    b = ops.workspace(dev, (1 << 20) + 1)
    assert b is not a and b.numel() == (1 << 20) + 1
    assert ops._RETIRED[key] == [a]
    monkeypatch.setattr(ops, "_capturing", lambda d: True)
    assert ops.workspace(dev, 1000) is b                             # no growth needed: fine under capture
    with pytest.raises(RuntimeError, match="cannot grow during graph capture"):
        ops.workspace(dev, 4 << 20)
    ops._WS.pop(key, None)
    ops._RETIRED.pop(key, None)


def test_reserve_covers_every_call_size(monkeypatch):
    """reserve(experts, max_tokens) asks for at least what every call of 1 .. max_tokens tokens needs (the decode
    plan's split-K partials make the need non-monotone in T), for the per-call and the whole-layer entries."""
    import types
    from mi355moe import ops
    d = _fake_desc()
    ex = types.SimpleNamespace(desc=d, K=4096, shared_suh=True, device="cpu")
    asked = []
    monkeypatch.setattr(ops, "workspace", lambda dev, n: asked.append(n))
    for top in (1, 3, 8, 64):
        for router in (None, 288):
            asked.clear()
            ops.reserve(ex, top, router_experts=router)
            needs = [ops.workspace_bytes(ex, t, 8, router) for t in range(1, top + 1)]
            assert asked == [max(needs)], (top, router)
    sizes = [ops.workspace_bytes(ex, t) for t in range(1, 9)]
    assert any(b > a for a, b in zip(sizes[1:], sizes)), sizes      # the need does fall somewhere: not monotone
