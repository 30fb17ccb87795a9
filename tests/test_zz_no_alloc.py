"""grimoire_moe_forward_noalloc (the forward without a workspace argument,
its scratch a fixed device array inside the library) against
grimoire_moe_forward on the same inputs: outputs and routes bit for bit,
on two calls in a row, the second with a smaller input, the one-launch
decode on the array's sync words, and the host-side rejection of a call
whose workspace exceeds the array."""
import ctypes as C

import pytest
import torch

from grimoire_amd import _abi, configs, ops

pytestmark = pytest.mark.gpu


def _both(wl, gpu, regime, T=None):
    cfg = wl.cfg
    T = cfg.T if T is None else T
    Lg = wl.layer.to(gpu)
    bias = None if wl.route_bias is None else wl.route_bias.to(gpu)
    rp = configs.route_params(cfg, bias)
    x = wl.x[:T].to(gpu).contiguous()
    fwd = ops.MoeForward(Lg, T, rp, regime)
    y0 = torch.empty(T, cfg.H, device=gpu)
    e0 = torch.empty(T, cfg.K, dtype=torch.int32, device=gpu)
    w0 = torch.empty(T, cfg.K, dtype=torch.float32, device=gpu)
    fwd(x, y0, e0, w0)
    y1 = torch.full((T, cfg.H), float("nan"), device=gpu)
    e1 = torch.full((T, cfg.K), -7, dtype=torch.int32, device=gpu)
    w1 = torch.full((T, cfg.K), float("nan"), device=gpu)
    st = fwd.struct
    r = _abi.lib().grimoire_moe_forward_noalloc(
        None, C.byref(st), C.byref(rp), ops._p(Lg.shared_gate_w), x.data_ptr(), y1.data_ptr(), T,
        e1.data_ptr(), w1.data_ptr(), regime)
    assert r == 0, _abi.lib().grimoire_moe_last_error().decode()
    torch.cuda.synchronize()
    assert torch.equal(e1, e0)
    assert torch.equal(w1.view(torch.int32), w0.view(torch.int32))
    assert torch.equal(y1.view(torch.int32), y0.view(torch.int32))
    return Lg


def test_noalloc_matches_forward_twice(gpu):
    """C2 at full size (decode), then a smaller input: the GEMM regime on a
    scaled C4 layer (shared expert, gate), then decode of 2 tokens."""
    print("noalloc: c2 full size", flush=True)
    _both(configs.make_workload(configs.CONFIGS["c2"], "cpu", seed=5), gpu, regime=0)
    print("noalloc: c4 scaled, GEMM regime T=64", flush=True)
    cfg = configs.scaled(configs.CONFIGS["c4"], T=64, E=16, H=512, I=256)
    _both(configs.make_workload(cfg, "cpu", seed=6), gpu, regime=2)
    print("noalloc: c4 scaled, decode T=2", flush=True)
    _both(configs.make_workload(cfg, "cpu", seed=7), gpu, regime=1, T=2)


def test_noalloc_one_launch_decode(gpu):
    """The one-launch decode (regime 7) on the library's array: its sync
    words start zero (zero-initialised storage) and stay consistent, so
    repeated calls, a layer of another grid in between, and the same layer
    again all match grimoire_moe_forward bit for bit."""
    c2 = configs.make_workload(configs.CONFIGS["c2"], "cpu", seed=8)
    small = configs.make_workload(configs.Config("s1", 1, 512, 16, 4, 256, "int4"), "cpu", seed=9)
    for wl in (c2, c2, small, c2):
        print(f"noalloc: one-launch decode {wl.cfg.name}", flush=True)
        _both(wl, gpu, regime=7)
    # the array's error word, read and cleared through the status / reset
    # entry points with no workspace
    lib = _abi.lib()
    st = C.c_int(-1)
    assert lib.grimoire_moe_decode_sync_status(None, None, 0, C.byref(st)) == 0 and st.value == 0
    assert lib.grimoire_moe_decode_sync_reset(None, None, 0) == 0
    torch.cuda.synchronize()
    _both(c2, gpu, regime=7)
    assert lib.grimoire_moe_decode_sync_status(None, None, 0, C.byref(st)) == 0 and st.value == 0


def test_noalloc_rejects_beyond_its_scratch(gpu):
    """C4 at full size needs far more than the array: refused on the host."""
    lib = _abi.lib()
    cap = int(lib.grimoire_moe_forward_noalloc_max_bytes())
    assert cap == 8 << 20
    cfg = configs.CONFIGS["c4"]
    # descriptors only: the call is refused before any pointer is used
    L = _abi.MoeLayer()
    L.cfg.hidden, L.cfg.inter, L.cfg.num_experts, L.cfg.top_k = cfg.H, cfg.I, cfg.E, cfg.K
    L.cfg.norm_topk = 1
    L.gate_up.fmt = L.down.fmt = _abi.FMT_INT8
    L.router = 1 << 12
    assert int(lib.grimoire_moe_forward_workspace_bytes(C.byref(L), cfg.T)) > cap
    rp = _abi.RouteParams(mode=_abi.ROUTE_SOFTMAX)
    r = lib.grimoire_moe_forward_noalloc(None, C.byref(L), C.byref(rp), None, 1 << 12, 1 << 12,
                                         cfg.T, None, None, 2)
    assert r == _abi.ERR_WORKSPACE
    assert "scratch limit" in lib.grimoire_moe_last_error().decode()
