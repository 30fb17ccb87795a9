"""Packed expert weights and the MoE layer descriptor (host side).

Mirrors b70::QuantWeight / PackedWeight / MoeLayer
(include/b70/weights.hpp:46-151, include/b70/moe.hpp:85-117): flat tensors
in the reference's layouts, expert-major:

    gate_up  [E*2I][H]   rows [e*2I, e*2I+I) gate, [e*2I+I, (e+1)*2I) up
    down     [E*H][I]

Tensors may live on the CPU (for the oracle) or on the GPU (for the
kernels); `struct()` returns the ctypes view the C ABI takes.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import torch

from . import _abi


@dataclass
class Weight:
    """One packed weight [N][K] (b70::QuantWeight fields)."""
    fmt: int
    N: int
    K: int
    payload: torch.Tensor                 # uint8 [N][row_bytes]
    scales: Optional[torch.Tensor] = None  # fp32 [N] | 16-bit [N][rs] | uint8 [N][rs]
    zeros: Optional[torch.Tensor] = None   # uint8 [N][rs]
    row_scales: int = 0

    @property
    def row_bytes(self) -> int:
        return int(self.payload.shape[1])

    def struct(self) -> _abi.QuantWeight:
        return _abi.QuantWeight(
            fmt=self.fmt, N=self.N, K=self.K, row_scales=self.row_scales,
            row_bytes=self.row_bytes, payload=self.payload.data_ptr(),
            scales=self.scales.data_ptr() if self.scales is not None else None,
            zeros=self.zeros.data_ptr() if self.zeros is not None else None)

    def to(self, device) -> "Weight":
        mv = lambda t: None if t is None else t.to(device).contiguous()
        return Weight(self.fmt, self.N, self.K, mv(self.payload), mv(self.scales), mv(self.zeros),
                      self.row_scales)

    def rows(self, r0: int, n: int) -> "Weight":
        """Rows [r0, r0 + n) as a view of the same memory."""
        sl = lambda t: None if t is None else t[r0:r0 + n]
        return Weight(self.fmt, n, self.K, self.payload[r0:r0 + n], sl(self.scales), sl(self.zeros),
                      self.row_scales)

    def pad_mxfp4(self) -> "Weight":
        """This MXFP4 weight with rows padded to mxfp4_padded_k(K) elements
        (zero codes under scale byte 127 past K), on the same device: the
        rows the matrix-core grouped GEMV streams as whole memory lines.
        grimoire_moe_pad_mxfp4_rows does the same on the GPU."""
        assert self.fmt == _abi.FMT_MXFP4
        kp = mxfp4_padded_k(self.K)
        pay = torch.zeros((self.N, kp // 2), dtype=torch.uint8, device=self.payload.device)
        pay[:, :self.K // 2] = self.payload[:, :self.K // 2]
        sc = torch.full((self.N, kp // 32), 127, dtype=torch.uint8, device=self.payload.device)
        sc[:, :self.K // 32] = self.scales[:, :self.K // 32]
        return Weight(self.fmt, self.N, self.K, pay, sc, None, kp // 32)

    def nbytes(self) -> int:
        n = self.payload.numel()
        for t in (self.scales, self.zeros):
            if t is not None:
                n += t.numel() * t.element_size()
        return n

    def row_bytes_total(self) -> float:
        """Bytes one row streams (payload + its scales / zeros)."""
        return self.nbytes() / self.N


def mxfp4_padded_k(K: int) -> int:
    """K rounded up to the matrix-core grouped GEMV's 256-element stages
    (grimoire_moe_mxfp4_padded_k)."""
    return (K + 255) // 256 * 256


def _gen(device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _rand_bytes(shape, g, device):
    return torch.randint(0, 256, shape, dtype=torch.uint8, generator=g, device=device)


def _abs_normal(shape, std, g, device):
    return (torch.randn(shape, generator=g, device=device, dtype=torch.float32) * std).abs()


def make_gptq_int4(N, K, *, group=128, scale_std=0.02, device="cpu", seed=0) -> Weight:
    """GPTQ symmetric int4: codes uniform in [-8, 7] stored offset-binary
    (nibble = v + 8, low nibble = even k), IEEE fp16 scales |N(0, std)| per
    `group` along K.  Format INT4_F16 with zeros = None (zero point 8)."""
    g = _gen(device, seed)
    payload = _rand_bytes((N, K // 2), g, device)   # both nibbles uniform 0..15
    sc = _abs_normal((N, K // group), scale_std, g, device).half().view(torch.int16)
    return Weight(_abi.FMT_INT4_F16, N, K, payload, sc, None, K // group)


def make_mxfp4(N, K, *, exp_lo=-8, exp_hi=-2, device="cpu", seed=0) -> Weight:
    """MXFP4: e2m1 nibbles uniform over the 16 codes, e8m0 scale per 32
    elements uniform over 2^exp_lo .. 2^exp_hi."""
    g = _gen(device, seed)
    payload = _rand_bytes((N, K // 2), g, device)
    sc = torch.randint(127 + exp_lo, 127 + exp_hi + 1, (N, K // 32), dtype=torch.uint8,
                       generator=g, device=device)
    return Weight(_abi.FMT_MXFP4, N, K, payload, sc, None, K // 32)


def make_int8(N, K, *, scale_std=0.02, device="cpu", seed=0) -> Weight:
    """Symmetric int8 per output channel: codes uniform in [-127, 127],
    scales |N(0, std)| rounded to bf16 (held as fp32, exactly)."""
    g = _gen(device, seed)
    q = torch.randint(-127, 128, (N, K), dtype=torch.int8, generator=g, device=device)
    sc = _abs_normal((N,), scale_std, g, device).bfloat16().float()
    return Weight(_abi.FMT_INT8, N, K, q.view(torch.uint8), sc, None, 1)


def make_bf16(N, K, *, std=0.05, device="cpu", seed=0) -> Weight:
    g = _gen(device, seed)
    w = (torch.randn((N, K), generator=g, device=device) * std).bfloat16()
    return Weight(_abi.FMT_BF16, N, K, w.view(torch.uint8).reshape(N, 2 * K), None, None, 0)


MAKERS = {
    "int4": make_gptq_int4,
    "mxfp4": make_mxfp4,
    "int8": make_int8,
    "bf16": make_bf16,
}


@dataclass
class MoeLayer:
    """b70::MoeLayer with its tensors."""
    hidden: int
    inter: int
    num_experts: int
    top_k: int
    gate_up: Weight
    down: Weight
    router: torch.Tensor                       # fp32 [E][H]
    shared_gate_up: Optional[Weight] = None
    shared_down: Optional[Weight] = None
    shared_gate_w: Optional[torch.Tensor] = None   # bf16 bits (int16) [H]
    norm_topk: bool = True
    _keep: list = field(default_factory=list, repr=False)

    @property
    def has_shared(self) -> bool:
        return self.shared_gate_up is not None

    @property
    def shared_inter(self) -> int:
        return self.shared_gate_up.N // 2 if self.has_shared else 0

    def struct(self) -> _abi.MoeLayer:
        L = _abi.MoeLayer()
        L.cfg = _abi.MoeConfig(self.hidden, self.inter, self.num_experts, self.top_k,
                               self.shared_inter, int(self.norm_topk))
        L.gate_up = self.gate_up.struct()
        L.down = self.down.struct()
        L.has_shared = int(self.has_shared)
        if self.has_shared:
            L.shared_gate_up = self.shared_gate_up.struct()
            L.shared_down = self.shared_down.struct()
        L.router = self.router.data_ptr()
        return L

    def to(self, device) -> "MoeLayer":
        mv = lambda w: None if w is None else w.to(device)
        return MoeLayer(self.hidden, self.inter, self.num_experts, self.top_k,
                        self.gate_up.to(device), self.down.to(device),
                        self.router.to(device).contiguous(), mv(self.shared_gate_up),
                        mv(self.shared_down),
                        None if self.shared_gate_w is None else self.shared_gate_w.to(device),
                        self.norm_topk)

    def shard(self, begin: int, count: int, shared: bool = True) -> "MoeLayer":
        """Experts [begin, begin + count) of this layer as views (the router
        stays global: grimoire_moe_forward_shard's layer); the shared expert
        kept when `shared`."""
        return MoeLayer(self.hidden, self.inter, self.num_experts, self.top_k,
                        self.gate_up.rows(begin * 2 * self.inter, count * 2 * self.inter),
                        self.down.rows(begin * self.hidden, count * self.hidden), self.router,
                        self.shared_gate_up if shared else None, self.shared_down if shared else None,
                        self.shared_gate_w if shared else None, self.norm_topk)

    def pad_mxfp4(self) -> "MoeLayer":
        """The layer with every MXFP4 weight's rows padded (Weight.pad_mxfp4):
        the same products, rows of whole memory lines for the grouped GEMV."""
        pw = lambda w: None if w is None else w.pad_mxfp4()
        return MoeLayer(self.hidden, self.inter, self.num_experts, self.top_k,
                        self.gate_up.pad_mxfp4(), self.down.pad_mxfp4(), self.router,
                        pw(self.shared_gate_up), pw(self.shared_down), self.shared_gate_w, self.norm_topk)

    def expert_bytes(self) -> float:
        """Bytes of one routed expert (gate, up and down rows with scales)."""
        gu = self.gate_up.row_bytes_total() * 2 * self.inter
        dn = self.down.row_bytes_total() * self.hidden
        return gu + dn

    def shared_bytes(self) -> float:
        if not self.has_shared:
            return 0.0
        return float(self.shared_gate_up.nbytes() + self.shared_down.nbytes())
