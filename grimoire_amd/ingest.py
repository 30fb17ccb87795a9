"""Expert-weight ingestion: checkpoint tensors -> the stacked expert-major
weights the MoE kernels read (`Weight`, `MoeLayer.gate_up` / `.down`).

Mirrors the per-expert staging of the reference's layer loader
(src/grimoire.cpp:8340-8397): for local expert e, gate rows land at
e*2I, up rows at e*2I + I of gate_up [E*2I][H], and down rows at e*H of
down [E*H][I].  The conversions run on the GPU through
`grimoire_moe_ingest_projection`; the signed-s4 pass through
`grimoire_moe_int4_to_signed`.

Source kinds (one checkpoint projection [out][in] each):
  gptq(qweight, qzeros, scales)      GPTQ / AutoGPTQ 4-bit triple
                                     (include/b70/gptq.hpp:21-55)
  mxfp4_packed(weight_packed, scale) compressed-tensors MXFP4, stored as is
  int4_packed(weight, scale, zp)     compressed-tensors pack-quantized INT4
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional, Sequence, Tuple

import torch

from . import _abi
from .ops import _p, _stream, check, lib
from .weights import Weight


@dataclass
class Projection:
    """One checkpoint projection as stored on disk (grim_expert_src)."""
    kind: int
    in_: int
    out: int
    group: int
    weight: torch.Tensor
    scales: torch.Tensor
    zeros: Optional[torch.Tensor] = None

    def struct(self) -> _abi.ExpertSrc:
        return _abi.ExpertSrc(self.kind, self.in_, self.out, self.group, _p(self.weight),
                              _p(self.zeros), _p(self.scales))


def gptq(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor,
         group: int = 128) -> Projection:
    """qweight int32 [in/8][out], qzeros int32 [in/group][out/8], scales fp16
    [in/group][out].  in/out come from the qweight shape, never a config
    field (down_proj has them reversed)."""
    inn, out = int(qweight.shape[0]) * 8, int(qweight.shape[1])
    if tuple(qzeros.shape) != (inn // group, out // 8) or tuple(scales.shape) != (inn // group, out):
        raise ValueError("GPTQ qzeros/scales shapes do not match qweight")
    return Projection(_abi.SRC_GPTQ, inn, out, group, qweight, scales, qzeros)


def mxfp4_packed(weight_packed: torch.Tensor, weight_scale: torch.Tensor) -> Projection:
    """weight_packed u8 [out][in/2] (e2m1, low nibble = even k), weight_scale
    e8m0 u8 [out][in/32]."""
    out, inn = int(weight_packed.shape[0]), int(weight_packed.shape[1]) * 2
    if tuple(weight_scale.shape) != (out, inn // 32):
        raise ValueError("MXFP4 weight_scale shape does not match weight_packed")
    return Projection(_abi.SRC_MXFP4_PACKED, inn, out, 32, weight_packed, weight_scale)


def int4_packed(weight_packed: torch.Tensor, weight_scale: torch.Tensor,
                weight_zero_point: Optional[torch.Tensor] = None, group: int = 128) -> Projection:
    """weight_packed u8 [out][in/2] (offset binary), weight_scale bf16
    [out][in/group], weight_zero_point int32 [out/8][in/group] or None (8)."""
    out, inn = int(weight_packed.shape[0]), int(weight_packed.shape[1]) * 2
    if tuple(weight_scale.shape) != (out, inn // group):
        raise ValueError("INT4 weight_scale shape does not match weight_packed")
    return Projection(_abi.SRC_INT4_PACKED, inn, out, group, weight_packed, weight_scale,
                      weight_zero_point)


def stacked(fmt: int, N: int, K: int, group: int, device) -> Weight:
    """An empty stacked weight [N][K] of `fmt` (payload, scales, zeros)."""
    if fmt == _abi.FMT_MXFP4:
        return Weight(fmt, N, K, torch.empty((N, K // 2), dtype=torch.uint8, device=device),
                      torch.empty((N, K // 32), dtype=torch.uint8, device=device), None, K // 32)
    if fmt in (_abi.FMT_INT4, _abi.FMT_INT4_F16):
        rs = K // group
        return Weight(fmt, N, K, torch.empty((N, K // 2), dtype=torch.uint8, device=device),
                      torch.empty((N, rs), dtype=torch.int16, device=device),
                      torch.empty((N, rs), dtype=torch.uint8, device=device), rs)
    raise ValueError(f"no ingestion into format {fmt}")


def ingest_projection(src: Projection, dst: Weight, row0: int, stream=None) -> None:
    s, d = src.struct(), dst.struct()
    check(lib().grimoire_moe_ingest_projection(_stream(stream), C.byref(s), C.byref(d), row0),
          "ingest_projection")


def ingest_projections(srcs: Sequence[Projection], dst: Weight, row0: Sequence[int],
                       stream=None) -> None:
    """Projections of one kind and shape into one stacked weight, batched
    (GPTQ: 64 per launch)."""
    n = len(srcs)
    arr = (_abi.ExpertSrc * n)(*[p.struct() for p in srcs])
    rows = (C.c_int32 * n)(*row0)
    d = dst.struct()
    check(lib().grimoire_moe_ingest_projections(_stream(stream), arr, C.cast(rows, C.c_void_p), n,
                                                C.byref(d)), "ingest_projections")


def target_format(kind: int, exact_scales: bool = False) -> int:
    """The reference's target for each source: GPTQ -> INT4 with bf16 scales
    (src/gptq.cpp:65-66), or INT4_F16 keeping the fp16 scales exactly."""
    if kind == _abi.SRC_GPTQ:
        return _abi.FMT_INT4_F16 if exact_scales else _abi.FMT_INT4
    if kind == _abi.SRC_MXFP4_PACKED:
        return _abi.FMT_MXFP4
    return _abi.FMT_INT4


def ingest_experts(experts: Sequence[Tuple[Projection, Projection, Projection]], device,
                   exact_scales: bool = False, stream=None) -> Tuple[Weight, Weight]:
    """(gate, up, down) per local expert -> (gate_up [E*2I][H], down [E*H][I]),
    the staging loop of src/grimoire.cpp:8340-8383.  Source tensors must be
    device-visible for GPTQ and INT4 zero points (copied parts may be host)."""
    g0, _, d0 = experts[0]
    E, I, H = len(experts), g0.out, g0.in_
    fmt = target_format(g0.kind, exact_scales)
    gate_up = stacked(fmt, E * 2 * I, H, g0.group, device)
    down = stacked(fmt, E * H, I, d0.group, device)
    gu_src, gu_rows, dn_src, dn_rows = [], [], [], []
    for e, (g, u, d) in enumerate(experts):
        if {g.kind, u.kind, d.kind} != {g0.kind}:
            raise ValueError("expert source kinds differ within the layer")
        if (g.out, g.in_, u.out, u.in_, d.out, d.in_) != (I, H, I, H, H, I):
            raise ValueError(f"expert {e}: projection shapes differ within the layer")
        gu_src += [g, u]
        gu_rows += [e * 2 * I, e * 2 * I + I]
        dn_src.append(d)
        dn_rows.append(e * H)
    ingest_projections(gu_src, gate_up, gu_rows, stream)
    ingest_projections(dn_src, down, dn_rows, stream)
    return gate_up, down


def to_signed(gate_up: Weight, down: Optional[Weight] = None, stream=None) -> torch.Tensor:
    """The signed-s4 pass over a layer's INT4 experts (src/grimoire.cpp:
    8386-8397).  Returns a device int32 tensor holding 1 if converted."""
    flag = torch.empty(1, dtype=torch.int32, device=gate_up.payload.device)

    def reg(w):
        if w is None:
            return None, 0, None, 0
        return (_p(w.payload), w.payload.numel(), _p(w.zeros),
                0 if w.zeros is None else w.zeros.numel())

    a, b = reg(gate_up), reg(down)
    check(lib().grimoire_moe_int4_to_signed(_stream(stream), *a, *b, _p(flag)), "int4_to_signed")
    return flag
