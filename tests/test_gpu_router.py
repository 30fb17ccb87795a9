"""Router parity on the GPU: logits to tolerance, top-k bit-exact against
the oracle on the same fp32 logits buffer (indices AND weights)."""
import pytest
import torch

from oracle import oracle as O
from grimoire_amd import ops
from tests.helpers import rel_l2

pytestmark = pytest.mark.gpu


def _ties(T, E, seed, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    l = torch.randn(T, E, generator=g) * scale
    l[:, 5] = l[:, 3]
    l[:, E - 1] = l[:, 0]
    l[::2, 7] = l[::2, 2]
    l[1::3, :] = l[1::3, :].round()          # many exact ties
    return l.contiguous()


# T <= 32 takes the register-resident row kernel for H <= 8192 (2 or 4
# experts x 4 tokens per work-group: ragged expert and token blocks, rows
# not a multiple of 1024, one expert), the one-row kernel above (9000);
# T > 32 the three-limb bf16 MFMA kernel when H % 128 == 0 (33, 300), the
# fp32 MFMA kernel when H % 32 == 0 (2080), else the tiled fp32 kernel (100)
@pytest.mark.parametrize("T,E,H", [(1, 128, 2048), (7, 64, 2048), (32, 256, 7168), (33, 512, 2048),
                                   (300, 96, 512), (70, 64, 2080), (40, 32, 100),
                                   (5, 37, 1028), (13, 3, 64), (32, 130, 8192), (2, 1, 4100),
                                   (4, 9, 9000)])
def test_router_logits(gpu, T, E, H):
    print(f"router_logits T={T} E={E} H={H}", flush=True)
    g = torch.Generator().manual_seed(T + E)
    W = torch.randn(E, H, generator=g) * 0.02
    x = torch.randn(T, H, generator=g).bfloat16().float()
    out = torch.empty(T, E, device=gpu)
    ops.router_logits(W.to(gpu), x.to(gpu), out)
    torch.cuda.synchronize()
    want = O.router_logits(W, x)
    assert (out.cpu() - want).abs().max() < 1e-4
    assert rel_l2(out.cpu(), want) < 1e-5


# T >= 256, H % 64 == 0: the split-K three-limb kernel.  x that is not bf16
# valued takes the six limb products on the tiles that hold it: all rows
# fp32, or every other block of 64 rows, so that clean and full tiles and
# producer waves meet in one launch; ragged token and expert blocks.
@pytest.mark.parametrize("T,E,H,kind", [(1000, 200, 1024, "fp32"), (520, 512, 2048, "mixed"),
                                        (256, 130, 384, "fp32")])
def test_router_logits_split_fp32_x(gpu, T, E, H, kind):
    print(f"router_logits split T={T} E={E} H={H} x={kind}", flush=True)
    g = torch.Generator().manual_seed(T + E + H)
    W = torch.randn(E, H, generator=g) * 0.02
    x = torch.randn(T, H, generator=g)
    if kind == "mixed":
        rows = (torch.arange(T) // 64) % 2 == 0
        x[rows] = x[rows].bfloat16().float()
    out = torch.empty(T, E, device=gpu)
    ops.router_logits(W.to(gpu), x.to(gpu), out)
    torch.cuda.synchronize()
    want = O.router_logits(W, x)
    assert (out.cpu() - want).abs().max() < 1e-4
    assert rel_l2(out.cpu(), want) < 1e-5


@pytest.mark.parametrize("T,E,K", [(1, 128, 8), (1, 256, 8), (5, 64, 4), (40, 512, 10), (3, 20, 16),
                                   (9, 300, 7)])
@pytest.mark.parametrize("normalize", [True, False])
def test_topk_softmax_bit_exact(gpu, T, E, K, normalize):
    print(f"topk softmax T={T} E={E} K={K} norm={normalize}", flush=True)
    l = _ties(T, E, E * K)
    oe = torch.empty(T, K, dtype=torch.int32, device=gpu)
    ow = torch.empty(T, K, dtype=torch.float32, device=gpu)
    if T == 1:
        ops.launch_router_topk(l.to(gpu), E, K, oe, ow, normalize)
        we, ww = O.topk_softmax(l, K, normalize, batched=False)
    else:
        ops.launch_router_topk_batched(l.to(gpu), T, E, K, oe, ow, normalize)
        we, ww = O.topk_softmax(l, K, normalize, batched=True)
    torch.cuda.synchronize()
    assert torch.equal(oe.cpu(), we)
    assert torch.equal(ow.cpu(), ww), (ow.cpu() - ww).abs().max()


@pytest.mark.parametrize("T,E,K", [(1, 128, 8), (40, 512, 10), (9, 300, 7)])
@pytest.mark.parametrize("normalize", [True, False])
def test_topk_bf16_batched_bit_exact(gpu, T, E, K, normalize):
    """launch_router_topk_bf16_batched (src/ops.cpp:1425): the batched
    semantics on bf16 logits (bf16 rounding adds many exact ties)."""
    print(f"topk bf16 T={T} E={E} K={K} norm={normalize}", flush=True)
    lb = _ties(T, E, E * K + 1).bfloat16()
    oe = torch.empty(T, K, dtype=torch.int32, device=gpu)
    ow = torch.empty(T, K, dtype=torch.float32, device=gpu)
    ops.launch_router_topk_bf16_batched(lb.view(torch.int16).to(gpu), T, E, K, oe, ow, normalize)
    torch.cuda.synchronize()
    we, ww = O.topk_softmax(lb.float().contiguous(), K, normalize, batched=True)
    assert torch.equal(oe.cpu(), we)
    assert torch.equal(ow.cpu(), ww)


@pytest.mark.parametrize("T,E,K,scaling", [(1, 128, 8, 1.0), (16, 100, 8, 2.5), (32, 512, 16, 1.0)])
def test_topk_sigmoid_bit_exact(gpu, T, E, K, scaling):
    print(f"topk sigmoid T={T} E={E} K={K}", flush=True)
    l = _ties(T, E, 3 + E)
    bias = (torch.randn(E) * 0.05).bfloat16().view(torch.int16).contiguous()
    oe = torch.empty(T, K, dtype=torch.int32, device=gpu)
    ow = torch.empty(T, K, dtype=torch.float32, device=gpu)
    ops.launch_router_topk_k2(l.to(gpu), bias.to(gpu), T, E, K, oe, ow, True, scaling)
    torch.cuda.synchronize()
    we, ww = O.topk_sigmoid(l, bias, K, True, scaling)
    assert torch.equal(oe.cpu(), we)
    assert torch.equal(ow.cpu(), ww)


# groups of whole lanes (1, 2, 4, 8 or 64 lanes per group: the butterfly
# path) and groups that split lanes (96 experts in 8 groups, 160 in 5: the
# serial path)
@pytest.mark.parametrize("T,E,K,ng,kg", [(32, 256, 8, 8, 4), (5, 64, 6, 8, 3), (4, 512, 8, 16, 4),
                                         (3, 64, 4, 1, 1), (6, 128, 6, 32, 4), (5, 256, 8, 64, 4),
                                         (6, 96, 4, 8, 3), (4, 160, 6, 5, 2)])
def test_topk_group_bit_exact(gpu, T, E, K, ng, kg):
    print(f"topk group T={T} E={E} K={K} groups {kg}/{ng}", flush=True)
    l = _ties(T, E, 17 + E, scale=1.0)
    bias = (torch.randn(E) * 1e-3).contiguous()
    oe = torch.empty(T, K, dtype=torch.int32, device=gpu)
    ow = torch.empty(T, K, dtype=torch.float32, device=gpu)
    ops.launch_router_topk_group(l.to(gpu), bias.to(gpu), T, E, K, ng, kg, oe, ow, True, 2.5)
    torch.cuda.synchronize()
    we, ww = O.topk_group(l, bias, K, ng, kg, True, 2.5)
    assert torch.equal(oe.cpu(), we)
    assert torch.equal(ow.cpu(), ww)
