"""GPU parity of the allocation-free whole-layer entry (mi355moe_moe_layer_noalloc, a fixed device array instead of a
workspace argument) against mi355moe_moe_layer through the C ABI: two calls in a row, the second with fewer tokens,
equal bit for bit (routed output and router picks); a shape that needs more than the fixed array is rejected before
any launch."""
from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

K, N, E = 4096, 1024, 288


def _say(*a):
    print(*a, flush=True)


def _noalloc(L, ex, x, w, b, T, out, ids, wts, stream):
    return L.mi355moe_moe_layer_noalloc(
        ctypes.byref(ex.desc), ctypes.c_void_p(x.data_ptr()), 2, x.stride(0), T, ctypes.c_void_p(w.data_ptr()), None,
        E, ctypes.c_void_p(b.data_ptr()), 8, 2.5, 1, 10.0, ctypes.c_void_p(out.data_ptr()), 2, out.stride(0),
        ctypes.c_void_p(ids.data_ptr()), ctypes.c_void_p(wts.data_ptr()), stream)


def test_noalloc_layer_equals_workspace_entry(cuda):
    from mi355moe import _lib, ops, synthetic
    L = _lib.lib()
    ex = synthetic.exl3_layer(E, K, N, seed=61, device=cuda)
    w, b = synthetic.router(E, K, seed=62, device=cuda)
    stream = ctypes.c_void_p(torch.cuda.current_stream(cuda).cuda_stream)
    for T in (64, 8):
        _say(f"moe_layer_noalloc T={T}")
        x = synthetic.activations(T, K, seed=63 + T, device=cuda)
        out = torch.full((T, K), float("nan"), dtype=torch.bfloat16, device=cuda)
        ids = torch.full((T, 8), -7, dtype=torch.int32, device=cuda)
        wts = torch.full((T, 8), float("nan"), dtype=torch.float32, device=cuda)
        rc = _noalloc(L, ex, x, w, b, T, out, ids, wts, stream)
        assert rc == 0, _lib.strerror(rc)
        ref, rid, rw = ops.moe_layer(ex, x, router_w=w, topk=8, bias=b, routed_scale=2.5, limit=10.0,
                                     return_picks=True)
        torch.cuda.synchronize()
        assert torch.equal(ids, rid) and torch.equal(wts, rw)
        assert torch.equal(out, ref)
    # a shape beyond the fixed array: rejected on the host, nothing enqueued, out untouched
    T = 512
    need = L.mi355moe_moe_layer_workspace_bytes(ctypes.byref(ex.desc), T, 8, E)
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    x = synthetic.activations(T, K, seed=70, device=cuda)
    out = torch.zeros(T, K, dtype=torch.bfloat16, device=cuda)
    ids = torch.zeros(T, 8, dtype=torch.int32, device=cuda)
    wts = torch.zeros(T, 8, dtype=torch.float32, device=cuda)
    assert _noalloc(L, ex, x, w, b, T, out, ids, wts, stream) == _lib.ESCRATCH
    torch.cuda.synchronize()
    assert not out.any() and not ids.any()
