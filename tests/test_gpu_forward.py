"""The whole MoE layer (grimoire_moe_forward) on the GPU against the oracle:
routing bit-exact on the same logits, outputs within max-abs 2e-2 and
rel-L2 1e-3.  Full BASELINE sizes where the oracle finishes in seconds;
sampled tokens and cross-regime agreement where it does not."""
import pytest
import torch

from oracle import oracle as O
from grimoire_amd import _abi, configs, ops
from tests.helpers import assert_close

pytestmark = pytest.mark.gpu


def _run(wl, device, regime=0, T=None):
    cfg = wl.cfg
    Lg = wl.layer if wl.layer.router.is_cuda else wl.layer.to(device)
    x = wl.x[:T] if T else wl.x
    T = x.shape[0]
    xg = x.to(device)
    bias = None if wl.route_bias is None else wl.route_bias.to(device)
    fwd = ops.MoeForward(Lg, T, configs.route_params(cfg, bias), regime)
    y = torch.empty(T, cfg.H, device=device)
    oe = torch.empty(T, cfg.K, dtype=torch.int32, device=device)
    ow = torch.empty(T, cfg.K, dtype=torch.float32, device=device)
    fwd(xg, y, oe, ow)
    # logits through the same router kernel, for the routing check
    lg = torch.empty(T, cfg.E, device=device)
    ops.router_logits(Lg.router, xg, lg)
    torch.cuda.synchronize()
    return Lg, y.cpu(), oe.cpu(), ow.cpu(), lg.cpu()


def _check_routing(wl, logits, oe, ow):
    cfg = wl.cfg
    if cfg.route == _abi.ROUTE_SOFTMAX:
        l = logits if wl.route_bias is None else logits + wl.route_bias.cpu()
        we, ww = O.topk_softmax(l.contiguous(), cfg.K, True)
    elif cfg.route == _abi.ROUTE_GROUP:
        we, ww = O.topk_group(logits, wl.route_bias.cpu().contiguous(), cfg.K, cfg.n_group,
                              cfg.topk_group, True, cfg.scaling)
    else:
        we, ww = O.topk_sigmoid(logits, wl.route_bias.cpu().contiguous(), cfg.K, True, cfg.scaling)
    assert torch.equal(oe, we), "routing indices differ from the oracle"
    assert torch.equal(ow, ww), "routing weights differ from the oracle"


def _oracle_y(wl_cpu_layer, x, oe, ow, gate_w):
    s = wl_cpu_layer.struct()
    gate = None
    if wl_cpu_layer.has_shared and gate_w is not None:
        gw = (gate_w.to(torch.int32) << 16).view(torch.float32)
        gate = torch.sigmoid(x.double() @ gw.double()).float().contiguous()
    return O.moe_forward(s, oe, ow, gate, x)


@pytest.mark.parametrize("name", ["c1", "c2"])
def test_forward_full_size_decode(gpu, name):
    print(f"forward {name} full size", flush=True)
    wl = configs.make_workload(configs.CONFIGS[name], "cpu", seed=1)
    Lg, y, oe, ow, logits = _run(wl, gpu)
    _check_routing(wl, logits, oe, ow)
    yo = _oracle_y(wl.layer, wl.x, oe, ow, None)
    assert_close(y, yo, what=name)


def test_forward_c3_full_size(gpu):
    print("forward c3 full size (mxfp4, zipf)", flush=True)
    wl = configs.make_workload(configs.CONFIGS["c3"], "cpu", seed=2)
    Lg, y, oe, ow, logits = _run(wl, gpu)
    _check_routing(wl, logits, oe, ow)
    yo = _oracle_y(wl.layer, wl.x, oe, ow, None)
    assert_close(y, yo, what="c3")


@pytest.mark.parametrize("regime", [1, 2])
def test_forward_c4_scaled_both_regimes(gpu, regime):
    print(f"forward c4 scaled regime={regime}", flush=True)
    cfg = configs.scaled(configs.CONFIGS["c4"], T=96, H=1024, E=64, I=256)
    wl = configs.make_workload(cfg, "cpu", seed=3)
    Lg, y, oe, ow, logits = _run(wl, gpu, regime=regime)
    _check_routing(wl, logits, oe, ow)
    gate = None
    yo = _oracle_y(wl.layer, wl.x, oe, ow, wl.layer.shared_gate_w)
    assert_close(y, yo, what=f"c4 scaled regime {regime}")


@pytest.mark.parametrize("H", [384, 512, 2048])
def test_forward_int8_gather_edges(gpu, H):
    """The INT8 prefill reads x limbs per token through the route -> token
    map when K = H holds enough K tiles (H >= 512 here), and writes them at
    every permuted row otherwise (H = 384); both against the oracle, with
    the shared expert, on a Zipf-skewed routing that fills both tile kinds."""
    print(f"forward int8 gather edge H={H}", flush=True)
    cfg = configs.scaled(configs.CONFIGS["c4"], T=200, H=H, E=32, I=128)
    wl = configs.make_workload(cfg, "cpu", seed=9)
    Lg, y, oe, ow, logits = _run(wl, gpu, regime=2)
    _check_routing(wl, logits, oe, ow)
    yo = _oracle_y(wl.layer, wl.x, oe, ow, wl.layer.shared_gate_w)
    assert_close(y, yo, what=f"int8 prefill H={H}")


def test_forward_split_router_fp32_x(gpu):
    """T >= 256 takes the split-K router with W's limb planes split once per
    call into the workspace; x not bf16 valued on every other block of 64
    rows (all six limb products there): routing bit-exact against the top-k
    of the standalone router's logits, outputs against the oracle (I = 256:
    the INT8 experts, whose two activation limbs keep fp32 x to ~2^-16 of
    its row's largest value)."""
    print("forward split router, fp32 x", flush=True)
    cfg = configs.scaled(configs.CONFIGS["c4"], T=300, H=512, E=96, I=256)
    wl = configs.make_workload(cfg, "cpu", seed=12)
    x = torch.randn(cfg.T, cfg.H, generator=torch.Generator().manual_seed(12))
    rows = (torch.arange(cfg.T) // 64) % 2 == 0
    x[rows] = x[rows].bfloat16().float()
    wl = configs.Workload(cfg, wl.layer, x.contiguous(), wl.route_bias)
    Lg, y, oe, ow, logits = _run(wl, gpu, regime=2)
    _check_routing(wl, logits, oe, ow)
    yo = _oracle_y(wl.layer, wl.x, oe, ow, wl.layer.shared_gate_w)
    assert_close(y, yo, what="split router, fp32 x")


def test_forward_c5_scaled(gpu):
    print("forward c5 scaled (group-limited sigmoid, mxfp4, shared)", flush=True)
    cfg = configs.scaled(configs.CONFIGS["c5"], T=32, H=1024, E=64, I=256)
    wl = configs.make_workload(cfg, "cpu", seed=4)
    Lg, y, oe, ow, logits = _run(wl, gpu, regime=2)
    _check_routing(wl, logits, oe, ow)
    yo = _oracle_y(wl.layer, wl.x, oe, ow, None)
    assert_close(y, yo, what="c5 scaled")


def test_forward_c4_full_size_sampled(gpu):
    """C4 at full size: routing of all 4096 tokens bit-exact; outputs of a
    seeded sample of tokens against the oracle; the grouped-GEMM regime
    agrees with the independent slot-GEMV regime on a token subset."""
    print("forward c4 full size", flush=True)
    cfg = configs.CONFIGS["c4"]
    wl = configs.make_workload(cfg, "cpu", seed=5)
    Lg, y, oe, ow, logits = _run(wl, gpu, regime=2)
    _check_routing(wl, logits, oe, ow)
    idx = torch.randperm(cfg.T, generator=torch.Generator().manual_seed(0))[:12]
    yo = _oracle_y(wl.layer, wl.x[idx].contiguous(), oe[idx].contiguous(), ow[idx].contiguous(),
                   wl.layer.shared_gate_w)
    assert_close(y[idx], yo, what="c4 sampled tokens")
    Lg2, y2, oe2, ow2, _ = _run(configs.Workload(cfg, Lg, wl.x, wl.route_bias), gpu, regime=1, T=64)
    assert torch.equal(oe2, oe[:64])
    assert_close(y[:64], y2, what="c4 gemm vs gemv regime")


def _slice_experts(w, ids, rows_per_expert):
    """A Weight holding only experts `ids` (rows_per_expert rows each), on the CPU."""
    from grimoire_amd.weights import Weight
    rp = rows_per_expert
    pay = torch.cat([w.payload[e * rp:(e + 1) * rp] for e in ids]).cpu()
    sc = torch.cat([w.scales[e * rp:(e + 1) * rp] for e in ids]).cpu()
    return Weight(w.fmt, len(ids) * rp, w.K, pay, sc, None, w.row_scales)


def test_forward_c5_full_size_sampled(gpu):
    """C5 at full size (T=32, H=7168, 256 routed experts + shared, I=2048,
    MXFP4, group-limited sigmoid top-8 with bias, scaling 2.5; ~6 GB of
    experts): routing of all 32 tokens bit-exact against the oracle on the
    same logits; outputs of a seeded sample of tokens against the oracle,
    which reads only the experts those tokens use (copied to the host)."""
    from grimoire_amd.weights import MoeLayer
    print("forward c5 full size", flush=True)
    cfg = configs.CONFIGS["c5"]
    Lg = configs.make_layer(cfg, gpu, seed=6)
    x = configs.make_x(cfg, "cpu", seed=6)
    bias = configs.make_route_bias(cfg, "cpu", seed=6)
    wl = configs.Workload(cfg, Lg, x, bias)
    _, y, oe, ow, logits = _run(wl, gpu, regime=0)
    _check_routing(wl, logits, oe, ow)
    idx = torch.randperm(cfg.T, generator=torch.Generator().manual_seed(1))[:4]
    ids = sorted(set(oe[idx].flatten().tolist()))
    remap = {e: j for j, e in enumerate(ids)}
    oe_s = torch.tensor([[remap[int(e)] for e in row] for row in oe[idx]], dtype=torch.int32)
    small = MoeLayer(cfg.H, cfg.I, len(ids), cfg.K,
                     _slice_experts(Lg.gate_up, ids, 2 * cfg.I), _slice_experts(Lg.down, ids, cfg.H),
                     Lg.router[:len(ids)].cpu().contiguous(),
                     Lg.shared_gate_up.to("cpu"), Lg.shared_down.to("cpu"), None, True)
    yo = O.moe_forward(small.struct(), oe_s, ow[idx].contiguous(), None, x[idx].contiguous())
    assert_close(y[idx], yo, what="c5 sampled tokens")


@pytest.mark.parametrize("regime", [4, 5])
@pytest.mark.parametrize("name,kw", [
    ("c3", {}),                                           # MXFP4, Zipf routing, T=8 (K % 128 != 0)
    ("c5", dict(T=32, H=1024, E=64, I=256)),              # group-limited, shared expert
    ("c5", dict(T=32, H=1024, E=64, I=512)),              # the same, matrix core: two stages per down item
    ("c5", dict(T=16, H=1280, E=32, I=768)),              # MXFP4, K % 256 == 0, ragged item tail
    ("c5", dict(T=6, H=2112, E=16, I=2240)),              # matrix core, 9 stages, rows across memory lines
    ("c5", dict(T=8, H=1536, E=16, I=1472)),              # matrix core, 6 stages, scale rows 4- / 2-byte aligned
    ("c1", {}),                                           # GPTQ int4, T=16
    ("c2", dict(T=24)),                                   # GPTQ int4, more rows than experts' groups
    # the routing launch's rank top-k: sigmoid + bias over a ragged E, every
    # key slot used (16 tokens x 128, 4 tokens x 512)
    ("c3", dict(T=10, H=1024, E=96, I=256, zipf=0.0, route=_abi.ROUTE_SIGMOID, bias_std=0.05, scaling=2.0)),
    ("c3", dict(T=16, H=512, E=128, K=8, I=256)),
    ("c1", dict(T=4, H=512, E=512, K=10, I=256)),
])
def test_forward_grouped_gemv(gpu, name, kw, regime):
    """The expert-grouped GEMV regimes: each expert's weights streamed once
    per group of up to 4 of its rows -- 4: MXFP4 experts with K % 256 == 0
    on the scaled fp4 x fp8 matrix core (activations as three e4m3 limbs),
    others on the vector ALU; 5: the vector ALU always.  Routing bit-exact,
    outputs within the layer tolerance, on MXFP4 and GPTQ int4 experts."""
    print(f"forward grouped gemv {name} {kw} regime {regime}", flush=True)
    cfg = configs.scaled(configs.CONFIGS[name], **kw) if kw else configs.CONFIGS[name]
    wl = configs.make_workload(cfg, "cpu", seed=9)
    Lg, y, oe, ow, logits = _run(wl, gpu, regime=regime)
    _check_routing(wl, logits, oe, ow)
    yo = _oracle_y(wl.layer, wl.x, oe, ow, wl.layer.shared_gate_w)
    assert_close(y, yo, what=f"grouped gemv {name}")


@pytest.mark.parametrize("regime", [4, 5])
def test_forward_grouped_gemv_fp32_activations(gpu, regime):
    """Activations that are not bf16 values: on the vector ALU the lo halves
    take gate_up's second path; on the matrix core the three limbs carry
    them (12 significant bits)."""
    print(f"forward grouped gemv fp32 x regime {regime}", flush=True)
    cfg = configs.scaled(configs.CONFIGS["c5"], T=12, H=512, E=32, I=256)
    wl = configs.make_workload(cfg, "cpu", seed=10)
    x = torch.randn(cfg.T, cfg.H, generator=torch.Generator().manual_seed(3))
    assert (x != x.bfloat16().float()).any()
    wl = configs.Workload(cfg, wl.layer, x.contiguous(), wl.route_bias)
    Lg, y, oe, ow, logits = _run(wl, gpu, regime=regime)
    _check_routing(wl, logits, oe, ow)
    yo = _oracle_y(wl.layer, wl.x, oe, ow, None)
    assert_close(y, yo, what="grouped gemv fp32 x")


def test_pad_mxfp4_rows_matches_host(gpu):
    """grimoire_moe_pad_mxfp4_rows on the GPU equals the host padding."""
    print("pad mxfp4 rows", flush=True)
    w = configs.MAKERS["mxfp4"](300, 2880, seed=7)
    want = w.pad_mxfp4()
    got = ops.pad_mxfp4(w.to(gpu))
    torch.cuda.synchronize()
    assert got.row_bytes == 1536 and got.row_scales == 96
    assert torch.equal(got.payload.cpu(), want.payload) and torch.equal(got.scales.cpu(), want.scales)


@pytest.mark.parametrize("regime", [0, 1, 2, 4, 5])
@pytest.mark.parametrize("name,kw", [
    ("c3", dict(H=960, I=704, E=32)),                     # K' = 1024 / 768: padded rows of whole lines
    ("c5", dict(T=12, H=1088, E=32, I=320)),              # shared expert, group-limited sigmoid
    # H a whole number of stages already: only down's rows are padded (the
    # grouped GEMV takes the mixed layer: K' = K for gate_up), 16-byte scale rows
    ("c3", dict(H=1536, I=1472, E=32)),
    ("c5", dict(T=12, H=1536, E=32, I=1472)),             # with the shared expert
])
def test_forward_mxfp4_padded_rows(gpu, name, kw, regime):
    """A layer whose MXFP4 rows are padded to grimoire_moe_mxfp4_padded_k(K)
    gives the unpadded layer's routing and outputs bit for bit on every
    regime (the matrix-core grouped GEMV reads the padded rows whole; the
    other kernels stop at K); regime 5, the vector-ALU grouped GEMV, reads
    packed rows only and refuses them."""
    print(f"forward mxfp4 padded rows {name} {kw} regime {regime}", flush=True)
    cfg = configs.scaled(configs.CONFIGS[name], **kw)
    wl = configs.make_workload(cfg, "cpu", seed=13)
    wp = configs.Workload(cfg, wl.layer.pad_mxfp4(), wl.x, wl.route_bias)
    if regime == 5:
        with pytest.raises(_abi.GrimoireError, match="packed MXFP4 rows"):
            _run(wp, gpu, regime=regime)
        return
    Lg, y, oe, ow, logits = _run(wl, gpu, regime=regime)
    _, yp, oep, owp, _ = _run(wp, gpu, regime=regime)
    assert torch.equal(oep, oe) and torch.equal(owp, ow)
    assert torch.equal(yp, y)
    _check_routing(wl, logits, oe, ow)
    yo = _oracle_y(wl.layer, wl.x, oe, ow, wl.layer.shared_gate_w)
    assert_close(y, yo, what=f"padded mxfp4 {name}")


@pytest.mark.parametrize("name,kw,regime", [
    ("c3", {}, 0),                                        # matrix-core grouped GEMV, merged dispatch
    ("c3", dict(pad=True), 0),                            # padded rows (the bench's C3 layer)
    ("c5", dict(T=32, H=1024, E=64, I=512), 0),           # the same, aligned scale loads, shared expert
    ("c4", dict(T=256, H=1024, E=64, I=256), 2),          # INT8 rows mode (128- and 32-row tiles)
])
def test_forward_graph_replays(gpu, name, kw, regime):
    """The forward captured once in a HIP graph and replayed on new inputs,
    three rounds with eager work and synchronisations between replays:
    every replay equals the eager forward on the same input, bit for bit."""
    print(f"forward graph replays {name} {kw} regime {regime}", flush=True)
    kw = dict(kw)
    pad = kw.pop("pad", False)
    cfg = configs.scaled(configs.CONFIGS[name], **kw) if kw else configs.CONFIGS[name]
    wl = configs.make_workload(cfg, "cpu", seed=21)
    Lg = (wl.layer.pad_mxfp4() if pad else wl.layer).to(gpu)
    bias = None if wl.route_bias is None else wl.route_bias.to(gpu)
    fwd = ops.MoeForward(Lg, cfg.T, configs.route_params(cfg, bias), regime)
    xs = [(wl.x * (1.0 + 0.25 * s)).to(gpu) for s in range(3)]
    x = xs[0].clone()
    y = torch.empty(cfg.T, cfg.H, device=gpu)
    oe = torch.empty(cfg.T, cfg.K, dtype=torch.int32, device=gpu)
    ow = torch.empty(cfg.T, cfg.K, dtype=torch.float32, device=gpu)
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
            assert torch.equal(oe.cpu(), eager[i][1]), f"routes, replay {rep} input {i}"
            assert torch.equal(y.cpu(), eager[i][0]), f"output, replay {rep} input {i}"

