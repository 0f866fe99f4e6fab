"""One layer's EXL3 routed experts on the device: production's stacked layout and the pointer tables.

Layout (code/fork/docs/prod_exl3_reference.py:2048-2162, Exl3MoEMethod.create_weights):
  w13_trellis int16 [n, 2, K/16, N/16, 64]   gate (index 0) and up (index 1)
  w13_suh     fp16  [n, 2, K]
  w13_svh     fp16  [n, 2, N]
  w13_mcg     int32 [n, 2, 1]                  the mcg codebook marker (0xCBAC1FED as int32)
  w2_trellis  int16 [n, N/16, K/16, 64]
  w2_suh      fp16  [n, N]
  w2_svh      fp16  [n, K]
  w2_mcg      int32 [n, 1]
The kernels reach expert e's tensors through nine int64 tables of device addresses, as production's
build_exl3_fused_state builds them (prod_exl3_reference.py:1438-1487); here they are computed from the stacked
tensors' strides on the host (one small copy to the device at load time, none per call).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import torch

from . import _lib

MCG_MARKER = -877912083          # int32 view of 0xCBAC1FED (prod_exl3_reference.py:51)


def _table(t: torch.Tensor, per_expert: tuple[int, ...]) -> torch.Tensor:
    """int64 [n] of the addresses of t[e, per_expert...] for every expert e (t contiguous)."""
    if not t.is_contiguous():
        raise ValueError("EXL3 expert tensors must be contiguous")
    n = t.shape[0]
    off = 0
    for d, i in enumerate(per_expert, start=1):
        off += i * t.stride(d)
    base = t.data_ptr() + off * t.element_size()
    step = t.stride(0) * t.element_size()
    if base % 16 or step % 16:
        raise ValueError("EXL3 expert tensors: every expert's trellis, suh and svh must start on a 16-byte boundary "
                         "(the kernels read them with 16-byte loads)")
    return (torch.arange(n, dtype=torch.int64) * step + base).to(t.device)


@dataclass
class Exl3Experts:
    """A layer's routed experts (stacked tensors) plus the pointer tables and the C descriptor."""

    w13_trellis: torch.Tensor
    w13_suh: torch.Tensor
    w13_svh: torch.Tensor
    w2_trellis: torch.Tensor
    w2_suh: torch.Tensor
    w2_svh: torch.Tensor
    tables: dict = field(default_factory=dict)
    desc: _lib.Exl3LayerDesc | None = None

    def __post_init__(self):
        n, two, kt, nt, words = self.w13_trellis.shape
        if two != 2 or words != 64:
            raise ValueError(f"w13_trellis must be int16 [n, 2, K/16, N/16, 64] (4 bits), got "
                             f"{tuple(self.w13_trellis.shape)}")
        K, N = kt * 16, nt * 16
        exp = {"w13_trellis": (n, 2, kt, nt, 64), "w13_suh": (n, 2, K), "w13_svh": (n, 2, N),
               "w2_trellis": (n, nt, kt, 64), "w2_suh": (n, N), "w2_svh": (n, K)}
        for name, shape in exp.items():
            t = getattr(self, name)
            want = torch.int16 if name.endswith("trellis") else torch.float16
            if tuple(t.shape) != shape or t.dtype != want:
                raise ValueError(f"{name}: expected {want} {shape}, got {t.dtype} {tuple(t.shape)}")
            if t.device != self.w13_trellis.device:
                raise ValueError(f"{name} is on {t.device}, w13_trellis on {self.w13_trellis.device}")
        self.n, self.K, self.N = n, K, N
        self.tables = {
            "gate_trellis": _table(self.w13_trellis, (0,)), "gate_suh": _table(self.w13_suh, (0,)),
            "gate_svh": _table(self.w13_svh, (0,)), "up_trellis": _table(self.w13_trellis, (1,)),
            "up_suh": _table(self.w13_suh, (1,)), "up_svh": _table(self.w13_svh, (1,)),
            "down_trellis": _table(self.w2_trellis, ()), "down_suh": _table(self.w2_suh, ()),
            "down_svh": _table(self.w2_svh, ()),
        }
        # gate and up share one input rotation (production's _exl3_shared_w13_suh, prod_exl3_reference.py:2243-2245)
        self.shared_suh = bool(torch.equal(self.w13_suh[:, 0], self.w13_suh[:, 1]))
        # ... and every expert the same one (the reference's TOKGATHER condition, code/fork/docs/OPT_MOE.md:14)
        self.uniform_suh = self.shared_suh and bool(torch.equal(self.w13_suh[:, 0],
                                                                self.w13_suh[:1, 0].expand(n, K)))
        self.desc = self.make_desc(self.tables)

    def make_desc(self, tables: dict) -> _lib.Exl3LayerDesc:
        d = _lib.Exl3LayerDesc()
        d.n, d.hidden, d.intermediate = self.n, self.K, self.N
        for k, v in tables.items():
            setattr(d, k, ctypes.c_void_p(v.data_ptr()))
        d.flags = ((_lib.LAYER_SHARED_W13_SUH if self.shared_suh else 0) |
                   (_lib.LAYER_UNIFORM_W13_SUH if self.uniform_suh else 0))
        return d

    @property
    def device(self) -> torch.device:
        return self.w13_trellis.device

    def expert_bytes(self) -> int:
        """Bytes of one expert's three matrices (trellis + suh/svh)."""
        return (3 * self.K * self.N // 2) + 2 * (3 * self.K + 3 * self.N)

    @staticmethod
    def from_module(layer: torch.nn.Module) -> "Exl3Experts":
        return Exl3Experts(layer.w13_trellis.data, layer.w13_suh.data, layer.w13_svh.data, layer.w2_trellis.data,
                           layer.w2_suh.data, layer.w2_svh.data)


_CHECKED_TABLES: set = set()


def _check_aligned(name: str, t: torch.Tensor, n: int) -> None:
    """Every address in a caller-built pointer table must be 16-byte aligned (the kernels read trellis words and
    scales with 16-byte loads). Checked on the host once per table (address, length, version); the check copies the
    table to the host, so it cannot run during graph capture."""
    key = (t.data_ptr(), n, t._version, str(t.device))
    if key in _CHECKED_TABLES:
        return
    if t.is_cuda and torch.cuda.is_current_stream_capturing():
        raise RuntimeError(f"{name}: pointer table not yet validated; make one eager call with these tables before "
                           "graph capture")
    if bool(((t[:n].cpu() % 16) != 0).any()):
        raise ValueError(f"{name}: every expert's address must be a multiple of 16 bytes")
    _CHECKED_TABLES.add(key)


def tables_desc(n: int, K: int, N: int, tables: dict, shared_suh: bool = False,
                uniform_suh: bool = False) -> _lib.Exl3LayerDesc:
    """Descriptor from caller-built pointer tables (the exl3_moe contract passes them directly); every table entry is
    checked for 16-byte alignment the first time the table is seen. uniform_suh (every expert the same w13 suh)
    implies shared_suh."""
    d = _lib.Exl3LayerDesc()
    d.n, d.hidden, d.intermediate = n, K, N
    d.flags = ((_lib.LAYER_SHARED_W13_SUH if shared_suh or uniform_suh else 0) |
               (_lib.LAYER_UNIFORM_W13_SUH if uniform_suh else 0))
    for k in ("gate_trellis", "gate_suh", "gate_svh", "up_trellis", "up_suh", "up_svh", "down_trellis", "down_suh",
              "down_svh"):
        t = tables[k]
        if t.dtype != torch.int64 or t.dim() != 1 or t.numel() < n or not t.is_contiguous():
            raise ValueError(f"{k}: pointer table must be a contiguous int64 [>= n] tensor")
        _check_aligned(k, t, n)
        setattr(d, k, ctypes.c_void_p(t.data_ptr()))
    return d
