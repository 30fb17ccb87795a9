"""Decode / batched-decode expert products (slot form) on the GPU against
the oracle: h and y within max-abs 2e-2 and rel-L2 1e-3."""
import pytest
import torch

from oracle import oracle as O
from grimoire_amd import configs, ops
from tests.helpers import assert_close

pytestmark = pytest.mark.gpu

CASES = [
    # fmt, H, I, E, K, T, shared
    ("int4", 2048, 768, 16, 8, 1, False),     # C2 shape class, LPR 64 / 32
    ("int4", 256, 128, 8, 3, 3, True),        # LPR 8 / 8
    ("int8", 512, 256, 8, 4, 2, True),
    ("mxfp4", 2880, 2880, 6, 4, 2, False),    # C3 shape class: 90 chunks, tail lanes
    ("bf16", 512, 128, 8, 2, 4, True),
]


def _routes(T, E, K, seed):
    g = torch.Generator().manual_seed(seed)
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).int()
    w = torch.rand(T, K, generator=g) + 0.05
    return ids.contiguous(), (w / w.sum(1, keepdim=True)).contiguous()


@pytest.mark.parametrize("fmt,H,I,E,K,T,shared", CASES)
def test_gate_up_down(gpu, fmt, H, I, E, K, T, shared):
    print(f"gemv {fmt} H={H} I={I} E={E} K={K} T={T} shared={shared}", flush=True)
    cfg = configs.Config("t", T, H, E, K, I, fmt, shared=shared, shared_gate=shared)
    L = configs.make_layer(cfg, "cpu", seed=H + I)
    x = configs.make_x(cfg, "cpu", seed=3)
    ids, w = _routes(T, E, K, H)
    if shared:
        ids[0, 0] = -1 if K > 1 else ids[0, 0]     # a skipped route
    Lg = L.to(gpu)
    KS = K + (1 if shared else 0)
    h = torch.empty(T, KS, I, device=gpu)
    y = torch.empty(T, H, device=gpu)
    gate = torch.empty(T, device=gpu)
    idg, wg, xg = ids.to(gpu), w.to(gpu), x.to(gpu)
    if shared:
        ops.launch_moe_shared_rows(Lg, Lg.shared_gate_w, idg, wg, xg, h, gate, y, T)
    else:
        ops.launch_moe_gate_up_batched(Lg, idg, xg, h, T)
        ops.launch_moe_down_batched(Lg, idg, wg, h, y, T)
    torch.cuda.synchronize()
    # oracle on the same routes
    s = L.struct()
    ho = torch.empty(T, KS, I)
    go = torch.empty(T)
    ids_o = ids.clone()
    ids_o[ids_o < 0] = 0          # gate_up computes a row for every slot
    if shared:
        ws = L.shared_gate_up.struct()
        O.orc().orc_gate_up(O.byref(s), O.byref(ws), O._p(L.shared_gate_w), O._p(ids_o), O._p(x),
                            O._p(ho), O._p(go), T)
    else:
        O.orc().orc_gate_up(O.byref(s), None, None, O._p(ids_o), O._p(x), O._p(ho), None, T)
    if not (shared and K > 1):
        assert_close(h.cpu(), ho, what="h")
    else:
        assert_close(h.cpu()[:, 1:], ho[:, 1:], what="h")
    hc = h.cpu().contiguous()
    yo = torch.empty(T, H)
    if shared:
        assert (gate.cpu() - go).abs().max() < 1e-5
        wds = L.shared_down.struct()
        O.orc().orc_down(O.byref(s), O.byref(wds), O._p(ids), O._p(w), O._p(go), O._p(hc),
                         O._p(yo), T)
    else:
        O.orc().orc_down(O.byref(s), None, O._p(ids), O._p(w), None, O._p(hc), O._p(yo), T)
    assert_close(y.cpu(), yo, what="y (down on the GPU's h)")
    # and the whole layer against the oracle's forward
    yf = O.moe_forward(s, ids, w, go if shared else None, x)
    assert_close(y.cpu(), yf, what="y vs moe_forward")
