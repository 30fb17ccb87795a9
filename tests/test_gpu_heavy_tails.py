"""The layer on heavy-tailed activations (src/moe_ref.cpp:68-105: bf16
activations used exactly, fp32-accumulated products).

The matrix-core paths do not feed the activations to the hardware as
given: the MXFP4 grouped GEMV splits every 32-element block into three
e4m3 limbs under one e8m0 scale (exact within 2^9 of the block's largest
value), and the INT8 prefill GEMM splits every row into two int8 limbs
under one fp32 scale (~16 bits relative to the row's largest value).  N(0,1)
inputs are the easy case for both, so these tests draw x with

  * 32-element blocks holding one element 32-64x the rest,
  * rows with one "massive" element 256-1024x the rest,
  * blocks of tiny values (2^-10 .. 2^-14 of the rest),
  * whole rows scaled down by 2^-8,

rounded to bf16, and hold the output to the layer tolerance (max-abs 2e-2
in units of max(1, rms(y)), rel-L2 1e-3) against the oracle, which uses
the bf16 values exactly.  Routing stays bit-exact on the same logits."""
import pytest
import torch

from grimoire_amd import configs
from tests.helpers import assert_close
from tests.test_gpu_forward import _check_routing, _oracle_y, _run

pytestmark = pytest.mark.gpu


def heavy_x(T, H, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g, dtype=torch.float64)
    nb = H // 32
    blocks = x.view(T, nb, 32)
    # one outlier in every 4th block, 32-64x
    sel = torch.rand(T, nb, generator=g) < 0.25
    pos = torch.randint(0, 32, (T, nb), generator=g)
    amp = 32 + 32 * torch.rand(T, nb, generator=g, dtype=torch.float64)
    sgn = torch.where(torch.rand(T, nb, generator=g) < 0.5, -1.0, 1.0).double()
    for t, b in sel.nonzero().tolist():
        blocks[t, b, pos[t, b]] = sgn[t, b] * amp[t, b]
    # tiny blocks: every 8th block scaled by 2^-10 .. 2^-14
    tiny = torch.rand(T, nb, generator=g) < 0.125
    sc = torch.exp2(-torch.randint(10, 15, (T, nb), generator=g).double())
    blocks.mul_(torch.where(tiny, sc, torch.ones_like(sc)).unsqueeze(-1))
    # massive activations: a third of the rows carry one element 256-1024x
    for t in range(T):
        if t % 3 == 0:
            j = int(torch.randint(0, H, (1,), generator=g))
            x[t, j] = (256.0 + 768.0 * float(torch.rand(1, generator=g, dtype=torch.float64))) * \
                (1 if t % 2 else -1)
    # every 5th row small overall
    x[::5] *= 2.0 ** -8
    return x.float().bfloat16().float().contiguous()


CASES = [
    # (name, config overrides, regime): INT8 row limbs (prefill GEMM), the
    # slot GEMV on the same INT8 layer, MXFP4 e4m3 limbs on the matrix core,
    # the vector-ALU grouped GEMV, and the INT4 decode
    ("c4", dict(T=128, H=1024, E=64, I=256), 2),
    ("c4", dict(T=64, H=2048, E=128, I=512), 2),
    ("c4", dict(T=16, H=1024, E=64, I=256), 1),
    ("c3", {}, 4),
    ("c5", dict(T=32, H=1024, E=64, I=512), 4),
    ("c5", dict(T=32, H=1024, E=64, I=512), 5),
    ("c5", dict(T=32, H=1024, E=64, I=256), 2),
    ("c2", {}, 1),
    ("c1", {}, 0),
]


@pytest.mark.parametrize("name,kw,regime", CASES)
def test_forward_heavy_tailed_x(gpu, name, kw, regime):
    cfg = configs.scaled(configs.CONFIGS[name], **kw) if kw else configs.CONFIGS[name]
    print(f"heavy-tailed x: {name} {kw} regime {regime}", flush=True)
    wl = configs.make_workload(cfg, "cpu", seed=31)
    x = heavy_x(cfg.T, cfg.H, seed=77)
    wl = configs.Workload(cfg, wl.layer, x, wl.route_bias)
    Lg, y, oe, ow, logits = _run(wl, gpu, regime=regime)
    _check_routing(wl, logits, oe, ow)
    yo = _oracle_y(wl.layer, wl.x, oe, ow, wl.layer.shared_gate_w)
    ma, rl = assert_close(y, yo, what=f"heavy tails {name} regime {regime}")
    print(f"  max-abs {ma:.3e} rel-L2 {rl:.3e}", flush=True)
    # per token as well: a small row next to a massive one must not hide
    # behind the global norm
    for t in range(cfg.T):
        assert_close(y[t], yo[t], what=f"heavy tails {name} regime {regime} token {t}")
