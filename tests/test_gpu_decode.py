"""The decode forward (router kernel, gate_up kernel running the top-k and
writing h in the staged layout, down kernel): parity with the oracle for
every routing mode and the shared expert, repeated calls on one workspace, and HIP-graph replays checked one by one."""
import pytest
import torch

from oracle import oracle as O
from grimoire_amd import _abi, configs, ops
from tests.helpers import assert_close
from tests.test_gpu_forward import _check_routing, _oracle_y

pytestmark = pytest.mark.gpu

CASES = {
    "c2": configs.CONFIGS["c2"],
    "c3_t4": configs.scaled(configs.CONFIGS["c3"], T=4, E=32),
    "c4_t3": configs.scaled(configs.CONFIGS["c4"], T=3, H=1024, E=64, I=256),
    "c5_t8": configs.scaled(configs.CONFIGS["c5"], T=8, H=1024, E=64, I=256),
    "sigmoid": configs.Config("sg", 2, 512, 40, 6, 128, "int8", route=_abi.ROUTE_SIGMOID,
                              scaling=2.5, bias_std=0.05),
    "bf16_t8": configs.Config("bf", 8, 512, 16, 4, 256, "bf16", shared=True, shared_gate=True),
}


def _setup(cfg, device, seed):
    wl = configs.make_workload(cfg, "cpu", seed=seed)
    Lg = wl.layer.to(device)
    bias = None if wl.route_bias is None else wl.route_bias.to(device)
    fwd = ops.MoeForward(Lg, cfg.T, configs.route_params(cfg, bias), regime=1)
    return wl, Lg, bias, fwd


@pytest.mark.parametrize("name", list(CASES))
def test_decode_parity(gpu, name):
    cfg = CASES[name]
    print(f"decode {name}: {cfg}", flush=True)
    wl, Lg, bias, fwd = _setup(cfg, gpu, 7)
    xg = wl.x.to(gpu)
    y = torch.empty(cfg.T, cfg.H, device=gpu)
    oe = torch.empty(cfg.T, cfg.K, dtype=torch.int32, device=gpu)
    ow = torch.empty(cfg.T, cfg.K, device=gpu)
    outs = []
    for _ in range(3):          # counters must come back to zero every call
        fwd(xg, y, oe, ow)
        torch.cuda.synchronize()
        outs.append((y.cpu().clone(), oe.cpu().clone(), ow.cpu().clone()))
    for y2, e2, w2 in outs[1:]:
        assert torch.equal(y2, outs[0][0]) and torch.equal(e2, outs[0][1]) and torch.equal(w2, outs[0][2])
    yv, oev, owv = outs[0]
    logits = torch.empty(cfg.T, cfg.E, device=gpu)
    ops.router_logits(Lg.router, xg, logits)
    torch.cuda.synchronize()
    _check_routing(wl, logits.cpu(), oev, owv)
    yo = _oracle_y(wl.layer, wl.x, oev, owv, wl.layer.shared_gate_w)
    assert_close(yv, yo, what=f"decode {name}")


def test_decode_graph_replays(gpu):
    cfg = CASES["c2"]
    print("decode graph replays", flush=True)
    wl, Lg, bias, fwd = _setup(cfg, gpu, 9)
    xs = [configs.make_x(cfg, "cpu", seed=s).to(gpu) for s in range(4)]
    x = xs[0].clone()
    y = torch.empty(cfg.T, cfg.H, device=gpu)
    oe = torch.empty(cfg.T, cfg.K, dtype=torch.int32, device=gpu)
    ow = torch.empty(cfg.T, cfg.K, device=gpu)
    eager = []
    for xi in xs:
        x.copy_(xi)
        fwd(x, y, oe, ow)
        torch.cuda.synchronize()
        eager.append(y.cpu().clone())
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
            assert torch.equal(y.cpu(), eager[i]), f"replay {rep} input {i}"
