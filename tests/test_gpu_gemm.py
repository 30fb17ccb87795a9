"""Grouped MFMA GEMM on the GPU against dense products of the dequantised
weights (exact operands, fp32 accumulation: rel-L2 1e-5), over ragged
expert row counts including empty experts and partial tiles."""
import pytest
import torch

from oracle import oracle as O
from grimoire_amd import ops
from grimoire_amd.weights import make_bf16, make_int8, make_mxfp4
from tests.helpers import dequant, rel_l2

pytestmark = pytest.mark.gpu

MAKE = {"int8": make_int8, "mxfp4": make_mxfp4, "bf16": make_bf16}


def _counts(E, seed):
    g = torch.Generator().manual_seed(seed)
    c = torch.randint(0, 300, (E,), generator=g).int()
    c[0] = 0
    c[1] = 128
    c[2] = 1
    return c


def _dense(A, W, counts, offsets, N):
    out = torch.zeros(A.shape[0], N, dtype=torch.float64)
    for e in range(len(counts)):
        r0, n = int(offsets[e]), int(counts[e])
        if n:
            out[r0:r0 + n] = A[r0:r0 + n].double() @ W[e * N:(e + 1) * N].double().T
    return out


@pytest.mark.parametrize("fmt", ["int8", "mxfp4", "bf16"])
@pytest.mark.parametrize("N,K", [(256, 512), (320, 2880)])
def test_grouped_gemm_plain(gpu, fmt, N, K):
    print(f"grouped gemm {fmt} N={N} K={K}", flush=True)
    E = 5
    w = MAKE[fmt](E * N, K, seed=N + K)
    counts = _counts(E, K)
    offsets = (torch.cumsum(counts, 0) - counts).int()
    R = int(counts.sum())
    A = torch.randn(R, K).bfloat16()
    out = torch.full((R, N), float("nan"), device=gpu)
    ops.grouped_gemm(w.to(gpu), N, False, A.view(torch.int16).to(gpu), out, offsets.to(gpu),
                     counts.to(gpu), E, R)
    torch.cuda.synchronize()
    want = _dense(A.float(), dequant(w), counts, offsets, N)
    assert rel_l2(out.cpu(), want) < 1e-5


@pytest.mark.parametrize("fmt", ["int8", "mxfp4"])
def test_grouped_gemm_swiglu_pair_and_down(gpu, fmt):
    print(f"grouped gemm swiglu {fmt}", flush=True)
    E, I, H = 4, 192, 512
    wgu = MAKE[fmt](E * 2 * I, H, seed=1)
    wdn = MAKE[fmt](E * H, I, seed=2)
    counts = _counts(E, 3)
    offsets = (torch.cumsum(counts, 0) - counts).int()
    R = int(counts.sum())
    A = torch.randn(R, H).bfloat16()
    hp = torch.zeros(R, 2, I, dtype=torch.int16, device=gpu)
    ops.grouped_gemm(wgu.to(gpu), 2 * I, True, A.view(torch.int16).to(gpu), hp, offsets.to(gpu),
                     counts.to(gpu), E, R)
    torch.cuda.synchronize()
    gu = _dense(A.float(), dequant(wgu), counts, offsets, 2 * I)
    # per-expert gate/up halves
    g, u = gu[:, :I], gu[:, I:]
    h_want = g / (1 + torch.exp(-g)) * u
    hpc = hp.cpu()
    hi = (hpc[:, 0].to(torch.int32) << 16).view(torch.float32)
    lo = (hpc[:, 1].to(torch.int32) << 16).view(torch.float32)
    h = hi.double() + lo.double()
    assert rel_l2(h, h_want) < 1e-5
    assert rel_l2(hi, h_want) > 1e-4      # the lo half carries real bits
    # down on the pair
    y = torch.empty(R, H, device=gpu)
    ops.grouped_gemm(wdn.to(gpu), H, False, hp, y, offsets.to(gpu), counts.to(gpu), E, R,
                     a_pair=True)
    torch.cuda.synchronize()
    y_want = _dense(h.float(), dequant(wdn), counts, offsets, H)
    assert rel_l2(y.cpu(), y_want) < 1e-5
