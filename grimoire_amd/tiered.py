"""Tiered NVFP4 experts (include/b70/tiered_moe.hpp, src/tiered_moe.cpp) and
their placement policy (include/b70/expert_heat.hpp), on torch tensors.

A layer is E self-contained expert blocks (`layout(H, I)` bytes each) and a
device table of E block pointers.  A block may be a device tensor or a
pinned host tensor (`torch.empty(..., pin_memory=True)`): the kernels read
both through the table.  `TieredLayer.place` moves an expert between tiers
(block copy + table store, in stream order); `Heat` proposes the moves.
"""
from __future__ import annotations

import ctypes as C
from typing import List, Optional, Sequence

import torch

from . import _abi
from .ops import _dev, _p, _stream, check, lib


def layout(H: int, I: int) -> _abi.NvExpertLayout:
    L = _abi.NvExpertLayout()
    check(lib().grimoire_tmoe_layout(H, I, C.byref(L)), "tmoe_layout")
    return L


class TieredLayer:
    """One layer's routed experts behind a device block table."""

    def __init__(self, H: int, I: int, top_k: int, blocks: Sequence[torch.Tensor], device):
        self.lay = layout(H, I)
        self.H, self.I, self.K, self.E = H, I, top_k, len(blocks)
        for b in blocks:
            if b.dtype != torch.uint8 or b.numel() < self.lay.bytes:
                raise ValueError("expert block smaller than the layout")
        self.blocks: List[torch.Tensor] = list(blocks)
        self.table = torch.tensor([b.data_ptr() for b in blocks], dtype=torch.int64, device=device)

    def view(self) -> _abi.TieredMoeView:
        return _abi.TieredMoeView(self.lay, self.table.data_ptr(), self.E, self.K)

    def gate_up(self, expert, x, h, stream=None):
        """launch_tmoe_gate_up: h[M][K*I]."""
        _dev(x)
        v = self.view()
        check(lib().grimoire_tmoe_gate_up(_stream(stream), C.byref(v), _p(expert), _p(x), _p(h),
                                          x.shape[0]), "tmoe_gate_up")

    def down(self, expert, weight, h, y, stream=None):
        """launch_tmoe_down: y[M][H]."""
        _dev(h)
        v = self.view()
        check(lib().grimoire_tmoe_down(_stream(stream), C.byref(v), _p(expert), _p(weight), _p(h),
                                       _p(y), y.shape[0]), "tmoe_down")

    def place(self, e: int, dst: torch.Tensor, stream=None):
        """Move expert e into `dst` (device or pinned host): copy, then the
        table store; the old block may be reused once the stream passes."""
        src = self.blocks[e]
        check(lib().grimoire_tmoe_place(_stream(stream), self.table.data_ptr(), e, _p(dst), _p(src),
                                        self.lay.bytes), "tmoe_place")
        self.blocks[e] = dst


def _scratch(L, M, device):
    n = int(lib().grimoire_tmoe_scratch_bytes(C.byref(L), M))
    return torch.empty(n, dtype=torch.uint8, device=device)


def expert_gemm(block, L, gate_up, s0, s1, A, out, scratch=None, stream=None):
    """launch_nvfp4_expert_gemm (tiered_moe.hpp:83-93): out fp32 = A (bf16 bits) x W^T."""
    _dev(A)
    M = A.shape[0]
    scratch = _scratch(L, M, A.device) if scratch is None else scratch
    check(lib().grimoire_tmoe_expert_gemm(_stream(stream), _p(block), C.byref(L), int(gate_up),
                                          float(s0), float(s1), _p(A), _p(out), M, _p(scratch),
                                          scratch.numel()), "tmoe_expert_gemm")


def expert_ffn(block, L, sg, su, sd, A, hbuf, out, scratch=None, stream=None):
    """launch_nvfp4_expert_ffn (tiered_moe.hpp:95-107): SwiGLU FFN of one expert."""
    _dev(A)
    M = A.shape[0]
    scratch = _scratch(L, M, A.device) if scratch is None else scratch
    check(lib().grimoire_tmoe_expert_ffn(_stream(stream), _p(block), C.byref(L), float(sg),
                                         float(su), float(sd), _p(A), _p(hbuf), _p(out), M,
                                         _p(scratch), scratch.numel()), "tmoe_expert_ffn")


def _host(t: torch.Tensor, dtype) -> torch.Tensor:
    if t.device.type != "cpu" or t.dtype != dtype or not t.is_contiguous():
        raise ValueError(f"expected a contiguous host {dtype} tensor")
    return t


class CpuExperts:
    """The host expert pool (include/b70/cpu_experts.hpp): NVFP4 blocks in
    host memory computed by `threads` host threads (the caller is worker 0).
    `cpus[t]` pins pool thread t (t >= 1)."""

    def __init__(self, threads: int = 0, cpus: Optional[Sequence[int]] = None):
        c = None if cpus is None else torch.tensor(list(cpus), dtype=torch.int32)
        self._cpus = c
        self._h = lib().grimoire_cpu_experts_create(threads, None if c is None else c.data_ptr(),
                                                    0 if c is None else c.numel())
        if not self._h:
            raise _abi.GrimoireError("grimoire_cpu_experts_create failed")

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            lib().grimoire_cpu_experts_destroy(h)
            self._h = None

    @property
    def threads(self) -> int:
        return int(lib().grimoire_cpu_experts_threads(self._h))

    @property
    def wait_us(self) -> float:
        return float(lib().grimoire_cpu_experts_wait_us(self._h))

    @staticmethod
    def _ptrs(blocks: Sequence[torch.Tensor]):
        arr = (C.c_void_p * max(1, len(blocks)))(*[_host(b, torch.uint8).data_ptr() for b in blocks])
        return arr

    def ffn(self, L: _abi.NvExpertLayout, blocks: Sequence[torch.Tensor], w: torch.Tensor,
            x: torch.Tensor, y: torch.Tensor) -> None:
        """y[H] = sum_j w[j] s_d down_j(silu(s_g gate_j x) * s_u up_j x) (CpuExperts::ffn)."""
        ptrs = self._ptrs(blocks)
        w = _host(w, torch.float32)
        check(lib().grimoire_cpu_experts_ffn(self._h, C.byref(L), C.cast(ptrs, C.c_void_p),
                                             w.data_ptr(), len(blocks), _host(x, torch.float32).data_ptr(),
                                             _host(y, torch.float32).data_ptr()), "cpu_experts_ffn")

    def ffn_rows(self, L: _abi.NvExpertLayout, blocks: Sequence[torch.Tensor], w: torch.Tensor,
                 off: torch.Tensor, x: torch.Tensor, y: torch.Tensor) -> None:
        """ffn for each row r over blocks[off[r]:off[r+1]] (CpuExperts::ffn_rows)."""
        ptrs = self._ptrs(blocks)
        off = _host(off, torch.int32)
        check(lib().grimoire_cpu_experts_ffn_rows(self._h, C.byref(L), off.numel() - 1,
                                                  C.cast(ptrs, C.c_void_p), _host(w, torch.float32).data_ptr(),
                                                  off.data_ptr(), _host(x, torch.float32).data_ptr(),
                                                  _host(y, torch.float32).data_ptr()), "cpu_experts_ffn_rows")


def cpu_nvfp4_dot(pay: torch.Tensor, scl: torch.Tensor, x: torch.Tensor) -> float:
    """One NVFP4 row dotted with x on the host (cpu_nvfp4_dot)."""
    return float(lib().grimoire_cpu_nvfp4_dot(_host(pay, torch.uint8).data_ptr(),
                                              _host(scl, torch.uint8).data_ptr(),
                                              _host(x, torch.float32).data_ptr(), x.numel()))


def cpu_set_isa(isa: int) -> None:
    """Host dot product path: 0 scalar, 1 AVX2, 2 AVX-512, -1 the best."""
    check(lib().grimoire_cpu_set_isa(isa), "cpu_set_isa")


def cpu_pool_cpus(ranks: int, rank: int) -> List[int]:
    """Rank's contiguous share of this process's CPUs."""
    out = torch.empty(1024, dtype=torch.int32)
    n = lib().grimoire_cpu_pool_cpus(ranks, rank, out.data_ptr(), out.numel())
    if n < 0:
        raise _abi.GrimoireError("grimoire_cpu_pool_cpus failed")
    return out[:min(n, 1024)].tolist()


class Heat:
    """grim_heat: decayed routing counts per (layer, expert) and swap proposals."""

    def __init__(self, layers: int, experts: int, params: Optional[_abi.HeatParams] = None):
        if params is None:
            params = _abi.HeatParams()
            lib().grimoire_heat_default_params(C.byref(params))
        self.L, self.E = layers, experts
        self._h = lib().grimoire_heat_create(layers, experts, C.byref(params))
        if not self._h:
            raise _abi.GrimoireError("grimoire_heat_create failed")

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            lib().grimoire_heat_destroy(h)
            self._h = None

    def credit(self, layer: int, ids) -> None:
        ids = torch.as_tensor(ids, dtype=torch.int32).contiguous().cpu()
        lib().grimoire_heat_credit(self._h, layer, ids.data_ptr(), ids.numel())

    def heat(self, layer: int, expert: int) -> float:
        return float(lib().grimoire_heat_get(self._h, layer, expert))

    def propose(self, resident, movable=None, max_out: int = 1 << 16):
        r = torch.as_tensor(resident, dtype=torch.uint8).contiguous().cpu()
        m = None if movable is None else torch.as_tensor(movable, dtype=torch.uint8).contiguous().cpu()
        out = (_abi.ExpertSwap * max_out)()
        n = lib().grimoire_heat_propose(self._h, r.data_ptr(), None if m is None else m.data_ptr(),
                                        out, max_out)
        if n < 0:
            raise _abi.GrimoireError("grimoire_heat_propose failed")
        return [(s.promote_layer, s.promote_expert, s.demote_layer, s.demote_expert)
                for s in out[:n]]
