"""Tiered NVFP4 experts on the GPU (grimoire_tmoe_gate_up / _down /
_place) against the oracle restatement of src/tiered_moe.cpp: blocks in
device memory and in pinned host memory behind one table, slots routed to
no local expert, zero routing weights, and an expert moved between tiers.
Outputs within 1e-5 relative (the device sums each row in another order
and uses its own exp in silu)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from grimoire_amd import tiered
from tests.test_oracle_tiered import make_block

pytestmark = pytest.mark.gpu


def _close(got, want, tol=1e-5):
    scale = max(np.abs(want).max(), 1e-30)
    err = np.abs(got - want).max()
    assert err <= tol * scale, (err, scale)


@pytest.mark.parametrize("H,I,K,E,M,host_every", [(2048, 768, 8, 16, 1, 3), (2048, 768, 8, 16, 4, 0),
                                                  (256, 128, 3, 6, 5, 2), (3072, 640, 4, 8, 2, 4),
                                                  (256, 128, 17, 24, 2, 5), (512, 256, 1, 4, 3, 0)])
def test_tmoe_parity(gpu, H, I, K, E, M, host_every):
    print(f"tmoe H={H} I={I} K={K} E={E} M={M} host_every={host_every}", flush=True)
    lay = O.tmoe_layout(H, I)
    rng = np.random.default_rng(H + M)
    blocks_np = [make_block(lay, rng) for _ in range(E)]
    blocks = []
    for e, b in enumerate(blocks_np):
        t = torch.from_numpy(b)
        if host_every and e % host_every == 0:
            blocks.append(t.pin_memory())              # read over PCIe
        else:
            blocks.append(t.to(gpu))
    layer = tiered.TieredLayer(H, I, K, blocks, gpu)
    ex = np.stack([rng.permutation(E + 2)[:K] - 1 for _ in range(M)]).astype(np.int32)  # -1 and E
    w = rng.random((M, K)).astype(np.float32)
    w[0, K - 1] = 0.0
    x = rng.standard_normal((M, H)).astype(np.float32)
    exd, wd, xd = (torch.from_numpy(a).to(gpu) for a in (ex, w, x))
    h = torch.full((M, K * I), float("nan"), device=gpu)
    y = torch.full((M, H), float("nan"), device=gpu)
    layer.gate_up(exd, xd, h)
    layer.down(exd, wd, h, y)
    torch.cuda.synchronize()
    want_h = O.tmoe_gate_up(blocks_np, H, I, K, ex, x, M)
    _close(h.cpu().numpy(), want_h)
    want_y = O.tmoe_down(blocks_np, H, I, K, ex, w, h.cpu().numpy(), M)
    _close(y.cpu().numpy(), want_y)


def test_tmoe_place_moves_between_tiers(gpu):
    """Expert 1 to pinned host and expert 2 to a new device block: the
    outputs stay the same bit for bit (same bytes, same arithmetic)."""
    print("tmoe place", flush=True)
    H, I, K, E, M = 512, 256, 4, 6, 2
    lay = O.tmoe_layout(H, I)
    rng = np.random.default_rng(8)
    blocks_np = [make_block(lay, rng) for _ in range(E)]
    layer = tiered.TieredLayer(H, I, K, [torch.from_numpy(b).to(gpu) for b in blocks_np], gpu)
    ex = torch.tensor([[1, 2, 0, 5], [2, 1, 3, 4]], dtype=torch.int32, device=gpu)
    w = torch.rand(M, K, device=gpu)
    x = torch.randn(M, H, device=gpu)
    h0 = torch.empty(M, K * I, device=gpu); y0 = torch.empty(M, H, device=gpu)
    layer.gate_up(ex, x, h0); layer.down(ex, w, h0, y0)
    layer.place(1, torch.empty(lay["bytes"], dtype=torch.uint8).pin_memory())
    layer.place(2, torch.empty(lay["bytes"], dtype=torch.uint8, device=gpu))
    h1 = torch.empty_like(h0); y1 = torch.empty_like(y0)
    layer.gate_up(ex, x, h1); layer.down(ex, w, h1, y1)
    torch.cuda.synchronize()
    assert not layer.blocks[1].is_cuda
    assert torch.equal(h0, h1) and torch.equal(y0, y1)
    assert torch.equal(layer.blocks[1], torch.from_numpy(blocks_np[1]))


@pytest.mark.parametrize("H,I,M,host", [(512, 256, 37, False), (2048, 768, 130, True),
                                        (1024, 512, 1, False)])
def test_expert_gemm_and_ffn(gpu, H, I, M, host):
    """launch_nvfp4_expert_gemm / _ffn (tiered_moe.hpp:83-107) against float64
    products of the block dequantised by the reference's nvfp4_dequant_row:
    GEMMs rel-L2 1e-5 (bf16 weights exact, fp32 accumulation); the FFN's
    bf16 h within 2^-7 relative per element (+1e-5 of the largest), its output
    rel-L2 1e-4."""
    from tests.test_oracle_tiered import dequant
    print(f"expert gemm/ffn H={H} I={I} M={M} host={host}", flush=True)
    lay = O.tmoe_layout(H, I)
    rng = np.random.default_rng(M + H)
    b = make_block(lay, rng)
    g3 = b[lay["gsc"]:lay["gsc"] + 16].view(np.float32)
    blk = torch.from_numpy(b)
    blk = blk.pin_memory() if host else blk.to(gpu)
    L = tiered.layout(H, I)
    gu, dn = dequant(b, lay, H, I)            # float64, projection scales applied
    A = torch.randn(M, H, generator=torch.Generator().manual_seed(3)).bfloat16()
    Ad = A.view(torch.int16).to(gpu)
    out = torch.empty(M, 2 * I, device=gpu)
    tiered.expert_gemm(blk, L, True, float(g3[0]), float(g3[1]), Ad, out)
    Ah = torch.randn(M, I, generator=torch.Generator().manual_seed(4)).bfloat16()
    out_d = torch.empty(M, H, device=gpu)
    tiered.expert_gemm(blk, L, False, float(g3[2]), 0.0, Ah.view(torch.int16).to(gpu), out_d)
    hb = torch.empty(M, I, dtype=torch.int16, device=gpu)
    y = torch.empty(M, H, device=gpu)
    tiered.expert_ffn(blk, L, float(g3[0]), float(g3[1]), float(g3[2]), Ad, hb, y)
    torch.cuda.synchronize()

    def rel(a, w):
        return float(np.linalg.norm(a - w) / max(np.linalg.norm(w), 1e-30))
    want = A.double().numpy() @ gu.T
    assert rel(out.cpu().double().numpy(), want) < 1e-5
    want_d = Ah.double().numpy() @ dn.T
    assert rel(out_d.cpu().double().numpy(), want_d) < 1e-5
    g, u = want[:, :I], want[:, I:]
    h64 = g / (1 + np.exp(np.minimum(-g, 700.0))) * u
    hgot = hb.cpu().view(torch.bfloat16).double().numpy()
    # bf16 rounding (2^-8 relative, doubled) plus the fp32 accumulation of
    # g and u, which dominates where they nearly cancel
    assert np.all(np.abs(hgot - h64) <= np.abs(h64) * 2.0 ** -7 + 1e-5 * np.abs(h64).max())
    want_y = hgot @ dn.T
    assert rel(y.cpu().double().numpy(), want_y) < 1e-4
