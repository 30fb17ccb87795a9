"""Seeded synthetic workloads for the five benchmark configurations.

    C1  CPU-reference layer: T=16, H=2048, E=64, top-4 softmax, I=1024,
        GPTQ int4 g128 fp16 scales.
    C2  decode: T=1, H=2048, E=128, top-8 softmax, I=768, GPTQ int4.
    C3  concurrent decode: T=8, H=2880, E=128, top-4 softmax, I=2880,
        MXFP4, Zipf(1.1) expert popularity.
    C4  prefill: T=4096, H=2048, E=512, top-10 softmax, I=512, int8
        per-channel (bf16 scales), shared expert I=512 with sigmoid gate,
        Zipf(1.2) popularity.
    C5  speculative verify: T=32, H=7168, E=256 + shared (I=2048), sigmoid
        scores + bias N(0,1e-3), 8 groups / top-4 groups / top-8, scaling
        2.5, MXFP4.

Router weights fp32 N(0, 0.02); activations bf16 N(0, 1) held as fp32.
Expert popularity skew (C3, C4) is a router logit bias b_e = z(pi(e)), pi a
seeded permutation of the experts and z fitted so that the share of routes
the expert of popularity rank r receives follows Zipf(s): route probability
per token q_r = min(1, lam * (r + 1)^-s) with sum_r q_r = K (an expert
cannot take a token twice, so the head saturates at every token).
"""
from __future__ import annotations

import functools
import math
from dataclasses import dataclass
from typing import Optional

import torch

from . import _abi
from .weights import MAKERS, MoeLayer, Weight


@dataclass
class Config:
    name: str
    T: int
    H: int
    E: int
    K: int
    I: int
    fmt: str
    route: int = _abi.ROUTE_SOFTMAX
    zipf: float = 0.0              # 0 = no popularity skew
    shared: bool = False
    shared_gate: bool = False
    n_group: int = 0
    topk_group: int = 0
    scaling: float = 1.0
    bias_std: float = 0.0          # sigmoid routing selection bias


CONFIGS = {
    "c1": Config("c1", 16, 2048, 64, 4, 1024, "int4"),
    "c2": Config("c2", 1, 2048, 128, 8, 768, "int4"),
    "c3": Config("c3", 8, 2880, 128, 4, 2880, "mxfp4", zipf=1.1),
    "c4": Config("c4", 4096, 2048, 512, 10, 512, "int8", zipf=1.2, shared=True, shared_gate=True),
    "c5": Config("c5", 32, 7168, 256, 8, 2048, "mxfp4", route=_abi.ROUTE_GROUP, shared=True,
                 n_group=8, topk_group=4, scaling=2.5, bias_std=1e-3),
}


def scaled(cfg: Config, **kw) -> Config:
    d = dict(cfg.__dict__)
    d.update(kw)
    return Config(**d)


@dataclass
class Workload:
    cfg: Config
    layer: MoeLayer
    x: torch.Tensor                     # fp32 [T][H] (bf16 values)
    route_bias: Optional[torch.Tensor]  # fp32 [E] or None


def make_layer(cfg: Config, device="cpu", seed=0) -> MoeLayer:
    mk = MAKERS[cfg.fmt]
    gu = mk(cfg.E * 2 * cfg.I, cfg.H, device=device, seed=seed * 1000 + 1)
    dn = mk(cfg.E * cfg.H, cfg.I, device=device, seed=seed * 1000 + 2)
    g = torch.Generator(device=device)
    g.manual_seed(seed * 1000 + 3)
    router = torch.randn((cfg.E, cfg.H), generator=g, device=device) * 0.02
    sgu = sdn = sgw = None
    if cfg.shared:
        sgu = mk(2 * cfg.I, cfg.H, device=device, seed=seed * 1000 + 4)
        sdn = mk(cfg.H, cfg.I, device=device, seed=seed * 1000 + 5)
        if cfg.shared_gate:
            sgw = (torch.randn((cfg.H,), generator=g, device=device) * 0.02).bfloat16().view(torch.int16)
    return MoeLayer(cfg.H, cfg.I, cfg.E, cfg.K, gu, dn, router.contiguous(), sgu, sdn, sgw, True)


def zipf_route_prob(E: int, K: int, s: float) -> torch.Tensor:
    """Target route probability per token of the expert at each popularity
    rank: q_r = min(1, lam * (r + 1)^-s), lam set so that sum q = K."""
    p = (torch.arange(E, dtype=torch.float64) + 1.0) ** -s
    lo, hi = 0.0, float(K) / float(p[-1])
    for _ in range(200):
        lam = 0.5 * (lo + hi)
        if float(torch.clamp(lam * p, max=1.0).sum()) > K:
            hi = lam
        else:
            lo = lam
    return torch.clamp(lo * p, max=1.0)


@functools.lru_cache(maxsize=None)
def zipf_rank_bias(E: int, K: int, s: float, H: int, samples: int = 16384,
                   iters: int = 160) -> torch.Tensor:
    """Logit bias per popularity rank that makes top-K routing over router
    logits N(0, (0.02 * sqrt(H))^2) (router N(0, 0.02) times x N(0, 1))
    follow zipf_route_prob.  Fitted on a fixed seeded sample of logits by
    damped updates of log(target / observed); deterministic."""
    q = zipf_route_prob(E, K, s).float()
    g = torch.Generator().manual_seed(0x5EED + E * 131 + K)
    l = torch.randn((samples, E), generator=g) * (0.02 * math.sqrt(H))
    b = torch.zeros(E)
    eps = 0.5 / samples
    for _ in range(iters):
        idx = torch.topk(l + b, K, dim=1).indices
        f = torch.bincount(idx.flatten(), minlength=E).float() / samples
        b += 0.3 * (torch.log(q + eps) - torch.log(f + eps)).clamp(-1.0, 1.0)
        b -= b.max()
    return b


def make_route_bias(cfg: Config, device="cpu", seed=0) -> Optional[torch.Tensor]:
    g = torch.Generator(device="cpu")
    g.manual_seed(seed * 1000 + 7)
    if cfg.route == _abi.ROUTE_SOFTMAX:
        if cfg.zipf <= 0:
            return None
        pi = torch.randperm(cfg.E, generator=g)
        b = zipf_rank_bias(cfg.E, cfg.K, cfg.zipf, cfg.H)[pi]
        return b.float().contiguous().to(device)
    if cfg.bias_std > 0:
        b = torch.randn((cfg.E,), generator=g) * cfg.bias_std
        if cfg.route == _abi.ROUTE_SIGMOID:
            return b.bfloat16().view(torch.int16).to(device)
        return b.float().to(device)
    return None


def make_x(cfg: Config, device="cpu", seed=0, T=None) -> torch.Tensor:
    g = torch.Generator(device=device)
    g.manual_seed(seed * 1000 + 9)
    T = cfg.T if T is None else T
    return torch.randn((T, cfg.H), generator=g, device=device).bfloat16().float().contiguous()


def make_workload(cfg: Config, device="cpu", seed=0) -> Workload:
    return Workload(cfg, make_layer(cfg, device, seed), make_x(cfg, device, seed),
                    make_route_bias(cfg, device, seed))


def route_params(cfg: Config, bias: Optional[torch.Tensor]) -> _abi.RouteParams:
    return _abi.RouteParams(mode=cfg.route, n_group=cfg.n_group, topk_group=cfg.topk_group,
                            scaling=cfg.scaling,
                            bias=bias.data_ptr() if bias is not None else None)
