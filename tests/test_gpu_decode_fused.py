"""The one-launch decode (router, top-k, gate_up + SwiGLU, down + combine
in one kernel, work-groups exchanging epoch-tagged words): parity with the
oracle and with the three-launch decode on shapes that cover its planner
(grid from the gate_up units or the down rows, several router rows per
work-group, E = 512, K = 1, chunks that leave lanes idle), every routing
mode, the epoch advancing once per call, the error word staying clear, one
workspace shared by layers of different grids, and graph replays."""
import pytest
import torch

from grimoire_amd import _abi, configs, ops
from tests.helpers import assert_close
from tests.test_gpu_forward import _check_routing, _oracle_y

pytestmark = pytest.mark.gpu

EPOCH, ERR = 0, 1    # 32-bit words at the head of the workspace

CASES = {
    "c2": configs.CONFIGS["c2"],
    "int4_small": configs.Config("s1", 1, 512, 16, 4, 256, "int4"),
    "mxfp4": configs.Config("mx", 1, 1024, 64, 4, 512, "mxfp4"),
    "sigmoid": configs.Config("sg", 1, 1024, 40, 6, 256, "int4", route=_abi.ROUTE_SIGMOID,
                              scaling=2.5, bias_std=0.05),
    "group": configs.Config("gr", 1, 2048, 256, 8, 1024, "mxfp4", route=_abi.ROUTE_GROUP,
                            n_group=8, topk_group=4, scaling=2.5, bias_std=1e-3),
    "e512_k1": configs.Config("k1", 1, 256, 512, 1, 64, "mxfp4"),
    "ragged": configs.Config("rg", 1, 1536, 24, 3, 160, "mxfp4"),
}


def _fwd(cfg, dev, seed, regime=7):
    wl = configs.make_workload(cfg, "cpu", seed=seed)
    Lg = wl.layer.to(dev)
    bias = None if wl.route_bias is None else wl.route_bias.to(dev)
    fwd = ops.MoeForward(Lg, 1, configs.route_params(cfg, bias), regime=regime)
    fwd.bias = bias     # the route params hold a raw pointer to it
    return wl, Lg, fwd


def _call(fwd, x, cfg, dev):
    y = torch.empty(1, cfg.H, device=dev)
    oe = torch.empty(1, cfg.K, dtype=torch.int32, device=dev)
    ow = torch.empty(1, cfg.K, device=dev)
    fwd(x, y, oe, ow)
    torch.cuda.synchronize()
    return y.cpu(), oe.cpu(), ow.cpu()


def _flags(fwd):
    return fwd.workspace[:8].view(torch.int32).cpu()


@pytest.mark.parametrize("name", list(CASES))
def test_fused_decode_parity(gpu, name):
    cfg = CASES[name]
    print(f"fused decode {name}: {cfg}", flush=True)
    wl, Lg, fwd = _fwd(cfg, gpu, 11)
    xg = wl.x.to(gpu)
    outs = [_call(fwd, xg, cfg, gpu) for _ in range(3)]
    fl = _flags(fwd)
    assert int(fl[EPOCH]) == 3, "the fused kernel advances the epoch once per call"
    assert int(fl[ERR]) == 0, "a poll ran out of time"
    for i, o in enumerate(outs[1:], 1):
        for what, p, q in zip(("y", "routes", "weights"), o, outs[0]):
            assert torch.equal(p, q), (f"call {i} {what} differs from call 0: {p.flatten()[:8].tolist()} vs "
                                       f"{q.flatten()[:8].tolist()}, max diff {float((p - q).abs().max())}")
    y, oe, ow = outs[0]
    logits = torch.empty(1, cfg.E, device=gpu)
    ops.router_logits(Lg.router, xg, logits)
    torch.cuda.synchronize()
    _check_routing(wl, logits.cpu(), oe, ow)
    assert_close(y, _oracle_y(wl.layer, wl.x, oe, ow, None), what=f"fused {name}")

    # the three-launch decode on the same layer: the same routing bits
    fwd3 = ops.MoeForward(Lg, 1, fwd.route, regime=1)
    y3, oe3, ow3 = _call(fwd3, xg, cfg, gpu)
    assert int(_flags(fwd3)[EPOCH]) == 0, "regime 1 must not run the fused kernel"
    assert torch.equal(oe3, oe) and torch.equal(ow3, ow)
    assert_close(y, y3, what=f"fused vs three-launch {name}")


def test_fused_decode_shared_workspace(gpu):
    """Layers of different grids alternate on one workspace: the epoch
    comes from one word, so tags left by a larger grid never match."""
    print("fused decode: one workspace, two grids", flush=True)
    ca, cb = CASES["c2"], CASES["int4_small"]
    wa, La, fa = _fwd(ca, gpu, 3)
    wb, Lb, fb = _fwd(cb, gpu, 4)
    assert fa.workspace.numel() >= fb.workspace.numel()
    xa, xb = wa.x.to(gpu), wb.x.to(gpu)
    ya0 = _call(fa, xa, ca, gpu)
    yb0 = _call(fb, xb, cb, gpu)
    fb.workspace = fa.workspace
    for _ in range(2):
        yb = _call(fb, xb, cb, gpu)
        ya = _call(fa, xa, ca, gpu)
        assert all(torch.equal(p, q) for p, q in zip(ya, ya0))
        assert all(torch.equal(p, q) for p, q in zip(yb, yb0))
    fl = _flags(fa)
    assert int(fl[EPOCH]) == 5 and int(fl[ERR]) == 0


def test_fused_decode_graph_replays(gpu):
    cfg = CASES["mxfp4"]
    print("fused decode graph replays", flush=True)
    wl, Lg, fwd = _fwd(cfg, gpu, 5)
    xs = [configs.make_x(cfg, "cpu", seed=s).to(gpu) for s in range(3)]
    x = xs[0].clone()
    y = torch.empty(1, cfg.H, device=gpu)
    oe = torch.empty(1, cfg.K, dtype=torch.int32, device=gpu)
    ow = torch.empty(1, cfg.K, device=gpu)
    eager = []
    for xi in xs:
        x.copy_(xi)
        fwd(x, y, oe, ow)
        torch.cuda.synchronize()
        eager.append((y.cpu().clone(), oe.cpu().clone()))
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        fwd(x, y, oe, ow, stream=s)
    for rep in range(3):
        for i, xi in enumerate(xs):
            x.copy_(xi)
            torch.cuda.synchronize()
            with torch.cuda.stream(s):
                g.replay()
            torch.cuda.synchronize()
            assert torch.equal(y.cpu(), eager[i][0]) and torch.equal(oe.cpu(), eager[i][1]), \
                f"replay {rep} input {i}"
    assert int(_flags(fwd)[ERR]) == 0


def test_fused_decode_timeout_is_reported(gpu):
    """A poll that runs out of time (forced from the host: a bound of zero
    ticks makes every poll give up after its first look, and every wave
    still exits) sets the error word; that call and every later one on the
    workspace write NaN outputs and routes -1 until the sync words are
    cleared, and the status entry point reports it.  After a reset, with
    the default bound back, the forward is bit-identical to a fresh one."""
    cfg = CASES["c2"]
    print("fused decode: forced poll time-out", flush=True)
    wl, Lg, fwd = _fwd(cfg, gpu, 13)
    xg = wl.x.to(gpu)
    ref = _call(fwd, xg, cfg, gpu)
    assert fwd.sync_status() == 0
    lib = _abi.lib()
    prev = lib.grimoire_moe_debug_spin_ticks(0)
    try:
        y, oe, ow = _call(fwd, xg, cfg, gpu)
    finally:
        lib.grimoire_moe_debug_spin_ticks(-1)
    assert prev == 2000000
    assert fwd.sync_status() == 1
    # poisoned: the next calls, with the normal bound, write NaN only
    for _ in range(2):
        y, oe, ow = _call(fwd, xg, cfg, gpu)
        assert torch.isnan(y).all() and (oe == -1).all() and torch.isnan(ow).all()
        assert fwd.sync_status() == 1
    fwd.sync_reset()
    assert fwd.sync_status() == 0
    outs = [_call(fwd, xg, cfg, gpu) for _ in range(2)]
    for o in outs:
        assert all(torch.equal(p, q) for p, q in zip(o, ref))
    assert fwd.sync_status() == 0 and int(_flags(fwd)[EPOCH]) == 2
