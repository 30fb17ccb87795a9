"""One GPU's expert shard of the layer (grimoire_moe_forward_shard): the
router and the top-k are global, the layer holds experts [b, b + n) only,
routes to other experts become expert -1 / weight 0 (the reference's remap,
src/grimoire.cpp:15392-15399 and :23231-23240), and y is the shard's
partial sum.

Checks: the remap alone bit-exact against its definition; each shard's y
against the oracle on the sub-layer with the remapped routes; the global
routing written out unchanged (bit-exact against the oracle on the same
logits); and the sum of the partial outputs of every shard equal, within
the layer tolerance, to the unsharded forward (the shared expert given to
shard 0 only).  C5's real shard shape: 32 of 256 experts local."""
import pytest
import torch

from grimoire_amd import _abi, configs, ops
from grimoire_amd.weights import MoeLayer
from oracle import oracle as O
from tests.helpers import assert_close
from tests.test_gpu_forward import _check_routing, _run

pytestmark = pytest.mark.gpu


def test_route_local_remap(gpu):
    print("route_local remap", flush=True)
    g = torch.Generator().manual_seed(4)
    R = 1000
    ids = torch.randint(-1, 256, (R,), generator=g, dtype=torch.int32)
    w = torch.rand(R, generator=g)
    lid = torch.empty(R, dtype=torch.int32, device=gpu)
    lw = torch.empty(R, device=gpu)
    idg, wg = ids.to(gpu), w.to(gpu)
    for b, n in [(0, 32), (96, 32), (250, 6), (0, 256)]:
        assert _abi.lib().grimoire_moe_route_local(None, idg.data_ptr(), wg.data_ptr(), lid.data_ptr(),
                                                   lw.data_ptr(), R, b, n) == 0
        torch.cuda.synchronize()
        own = (ids >= b) & (ids < b + n)
        assert torch.equal(lid.cpu(), torch.where(own, ids - b, torch.full_like(ids, -1)))
        assert torch.equal(lw.cpu(), torch.where(own, w, torch.zeros_like(w)))


def _shard_oracle(layer_cpu, begin, count, x, oe, ow, shared):
    """The shard's y from the oracle: the sub-layer with local routes."""
    sub = layer_cpu.shard(begin, count, shared)
    own = (oe >= begin) & (oe < begin + count)
    le = torch.where(own, oe - begin, torch.full_like(oe, -1)).contiguous()
    lw = torch.where(own, ow, torch.zeros_like(ow)).contiguous()
    gate = None
    if shared and layer_cpu.shared_gate_w is not None:
        gw = (layer_cpu.shared_gate_w.to(torch.int32) << 16).view(torch.float32)
        gate = torch.sigmoid(x.double() @ gw.double()).float().contiguous()
    return O.moe_forward(sub.struct(), le, lw, gate, x)


def _shard_call(cfg, Lsh, bias, x, regime, begin, count, dev):
    fwd = ops.MoeForward(Lsh, cfg.T, configs.route_params(cfg, bias), regime)
    y = torch.full((cfg.T, cfg.H), float("nan"), device=dev)
    oe = torch.empty(cfg.T, cfg.K, dtype=torch.int32, device=dev)
    ow = torch.empty(cfg.T, cfg.K, device=dev)
    fwd.shard(x, y, begin, count, oe, ow)
    torch.cuda.synchronize()
    return y.cpu(), oe.cpu(), ow.cpu()


@pytest.mark.parametrize("name,kw,regime,shards", [
    ("c5", dict(T=32, H=1024, E=64, I=512), 0, 8),    # matrix-core grouped GEMV
    ("c5", dict(T=32, H=1024, E=64, I=256), 2, 4),    # bf16 MFMA grouped GEMM
    ("c4", dict(T=128, H=1024, E=64, I=256), 2, 4),   # INT8 prefill GEMM, Zipf routing
    ("c2", {}, 1, 4),                                 # decode (runs staged)
    ("c3", {}, 0, 2),                                 # MXFP4 T=8, Zipf
])
def test_shards_sum_to_the_layer(gpu, name, kw, regime, shards):
    cfg = configs.scaled(configs.CONFIGS[name], **kw) if kw else configs.CONFIGS[name]
    print(f"shards {name} {kw} regime {regime} x{shards}", flush=True)
    wl = configs.make_workload(cfg, "cpu", seed=41)
    Lg, y_full, oe_full, ow_full, logits = _run(wl, gpu, regime=regime)
    bias = None if wl.route_bias is None else wl.route_bias.to(gpu)
    xg = wl.x.to(gpu)
    n = cfg.E // shards
    total = torch.zeros(cfg.T, cfg.H, dtype=torch.float64)
    for s in range(shards):
        Lsh = Lg.shard(s * n, n, shared=(s == 0))
        y, oe, ow = _shard_call(cfg, Lsh, bias, xg, regime, s * n, n, gpu)
        assert torch.equal(oe, oe_full) and torch.equal(ow, ow_full), "global routing"
        if s == 0:
            _check_routing(wl, logits, oe, ow)
        yo = _shard_oracle(wl.layer, s * n, n, wl.x, oe, ow, s == 0)
        assert_close(y, yo, what=f"{name} shard {s}")
        total += y.double()
    assert_close(total.float(), y_full, what=f"{name} sum of {shards} shards vs the whole layer")


def test_c5_one_shard_of_eight_full_size(gpu):
    """C5's real one-GPU shape under 8-way expert parallelism: H=7168,
    I=2048, MXFP4, 32 tokens, group-limited routing over all 256 experts,
    experts [96, 128) local (0.75 GB), no shared expert on this shard."""
    print("c5 shard 32 of 256 full size", flush=True)
    cfg = configs.CONFIGS["c5"]
    b, n = 96, 32
    loc = configs.make_layer(configs.scaled(cfg, E=n), gpu, seed=8)
    g = torch.Generator(device=gpu).manual_seed(8 * 1000 + 3)
    router = (torch.randn((cfg.E, cfg.H), generator=g, device=gpu) * 0.02).contiguous()
    Lsh = MoeLayer(cfg.H, cfg.I, cfg.E, cfg.K, loc.gate_up, loc.down, router)
    x = configs.make_x(cfg, "cpu", seed=8)
    bias = configs.make_route_bias(cfg, "cpu", seed=8)
    fwd = ops.MoeForward(Lsh, cfg.T, configs.route_params(cfg, bias.to(gpu)), 0)
    fwd.bias = bias.to(gpu)
    fwd.route = configs.route_params(cfg, fwd.bias)
    xg = x.to(gpu)
    y = torch.full((cfg.T, cfg.H), float("nan"), device=gpu)
    oe = torch.empty(cfg.T, cfg.K, dtype=torch.int32, device=gpu)
    ow = torch.empty(cfg.T, cfg.K, device=gpu)
    fwd.shard(xg, y, b, n, oe, ow)
    logits = torch.empty(cfg.T, cfg.E, device=gpu)
    ops.router_logits(router, xg, logits)
    torch.cuda.synchronize()
    wl = configs.Workload(cfg, Lsh, x, bias)
    y, oe, ow = y.cpu(), oe.cpu(), ow.cpu()
    _check_routing(wl, logits.cpu(), oe, ow)
    own = (oe >= b) & (oe < b + n)
    assert int(own.sum()) > 0
    # the oracle on the local experts (copied to the host), all 32 tokens
    sub = MoeLayer(cfg.H, cfg.I, n, cfg.K, loc.gate_up.to("cpu"), loc.down.to("cpu"),
                   router[:n].cpu().contiguous())
    le = torch.where(own, oe - b, torch.full_like(oe, -1)).contiguous()
    lw = torch.where(own, ow, torch.zeros_like(ow)).contiguous()
    yo = O.moe_forward(sub.struct(), le, lw, None, x)
    assert_close(y, yo, what="c5 shard 96..127")
    # tokens with no local route get exact zeros
    none = ~own.any(dim=1)
    if none.any():
        assert (y[none] == 0).all()
