"""Comparison metrics and small host-side helpers for the tests."""
from __future__ import annotations

import numpy as np
import torch

# Output tolerance of the layer against the fp32-accumulated oracle:
# max-abs 2e-2 and rel-L2 1e-3.  The max-abs bound is in units of the
# reference output's RMS when that RMS exceeds 1: the C4 distribution
# (int8 codes up to 127, scales |N(0, 0.02)|) gives |y| ~ 1e5, where an
# absolute 2e-2 is a few fp32 ulps of the values themselves.
MAX_ABS = 2e-2
REL_L2 = 1e-3


def rel_l2(got, want) -> float:
    g = torch.as_tensor(got, dtype=torch.float64).cpu()
    w = torch.as_tensor(want, dtype=torch.float64).cpu()
    return float(torch.linalg.norm(g - w) / max(float(torch.linalg.norm(w)), 1e-30))


def max_abs(got, want) -> float:
    g = torch.as_tensor(got, dtype=torch.float64).cpu()
    w = torch.as_tensor(want, dtype=torch.float64).cpu()
    return float((g - w).abs().max()) if g.numel() else 0.0


def rms(t) -> float:
    w = torch.as_tensor(t, dtype=torch.float64).cpu()
    return float(w.pow(2).mean().sqrt()) if w.numel() else 0.0


def assert_close(got, want, max_abs_tol=MAX_ABS, rel_tol=REL_L2, what=""):
    ma, rl = max_abs(got, want), rel_l2(got, want)
    tol = max_abs_tol * max(1.0, rms(want))
    assert ma <= tol and rl <= rel_tol, \
        f"{what}: max-abs {ma:.3e} (bound {tol:.3e}), rel-L2 {rl:.3e}"
    return ma, rl


def dequant(w) -> torch.Tensor:
    """Dense fp32 [N][K] of a grimoire_amd.weights.Weight (on its device)."""
    from grimoire_amd import _abi
    N, K = w.N, w.K
    p = w.payload
    if w.fmt == _abi.FMT_BF16:
        return p.view(torch.int16).reshape(N, K).view(torch.bfloat16).float()
    if w.fmt == _abi.FMT_INT8:
        return p.view(torch.int8)[:, :K].float() * w.scales.view(N, 1)
    lo = (p[:, : K // 2] & 0xF).to(torch.int32)
    hi = (p[:, : K // 2] >> 4).to(torch.int32)
    q = torch.stack([lo, hi], dim=2).reshape(N, K)
    if w.fmt == _abi.FMT_MXFP4:
        mag = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], device=p.device)
        v = mag[q & 7] * torch.where((q & 8) != 0, -1.0, 1.0)
        e = w.scales[:, : K // 32].to(torch.int32)
        s = torch.exp2((e - 127).float())
        return v * s.repeat_interleave(32, dim=1)
    # INT4 / INT4_F16
    G = K // w.row_scales
    raw = w.scales.view(torch.int16)
    if w.fmt == _abi.FMT_INT4:
        s = (raw.to(torch.int32) << 16).view(torch.float32)
    else:
        s = raw.view(torch.float16).float()
    if w.zeros is not None:
        z = w.zeros.to(torch.int32)
    else:
        z = torch.full_like(raw, 8 if w.fmt == _abi.FMT_INT4_F16 else 0, dtype=torch.int32)
    zz = z.repeat_interleave(G, dim=1)
    qs = torch.where(zz == 0xFF, torch.where(q >= 8, q - 16, q), q - zz)
    return qs.float() * s.repeat_interleave(G, dim=1)
