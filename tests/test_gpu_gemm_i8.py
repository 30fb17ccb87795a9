"""INT8 grouped GEMM on the int8 MFMA (two activation limbs per row) and its
limb quantiser, on the GPU.

The quantiser is pinned by its definition: a = s * (hi + lo / 254),
s = max|row| / 127, |hi|, |lo| <= 127, reconstruction error <= s / 508 (+ fp32 rounding).
The GEMM is pinned exactly where the limbs are exact (integer rows whose
largest magnitude is 127: s = 1, lo = 0, so the int32 products are the
exact dot products) and otherwise against fp64 products of the dequantised
weights (rel-L2 2e-4: the limb error is ~2^-16 of each row's largest
value), over ragged expert row counts including empty experts, a single
row, a full 128-row tile and partial tiles."""
import pytest
import torch

from grimoire_amd import ops
from grimoire_amd.weights import make_int8
from tests.helpers import dequant, rel_l2

pytestmark = pytest.mark.gpu


def _decode(q, n):
    """limb rows [rows][n/64][2][64] -> hi, lo int tensors [rows][n]"""
    q = q.view(torch.int8).reshape(q.shape[0], n // 64, 2, 64).cpu().to(torch.int32)
    return q[:, :, 0, :].reshape(-1, n), q[:, :, 1, :].reshape(-1, n)


def _limbs(gpu, x):
    rows, n = x.shape
    q = torch.empty(rows, 2 * n, dtype=torch.int8, device=gpu)
    s = torch.empty(rows, device=gpu)
    ops.quant_limbs(x.to(gpu), q, s)
    torch.cuda.synchronize()
    return q, s


def test_quant_limbs_definition(gpu):
    print("quant limbs", flush=True)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(37, 512, generator=g) * torch.logspace(-3, 3, 37).unsqueeze(1)
    x[5] = 0.0
    q, s = _limbs(gpu, x)
    hi, lo = _decode(q, 512)
    s = s.cpu()
    assert hi.abs().max() <= 127 and lo.abs().max() <= 127
    m = x.abs().amax(1)
    assert torch.allclose(s[m > 0], (m / 127)[m > 0], rtol=1e-6)
    assert s[5] == 1.0 and hi[5].abs().sum() == 0 and lo[5].abs().sum() == 0
    rec = s.double().unsqueeze(1) * (hi.double() + lo.double() / 254)
    err = (rec - x.double()).abs()
    # s / 508 from the lo rounding, plus the fp32 evaluation of x * (127 /
    # max) (|y| <= 127: up to 127 * 2^-24 of s)
    assert (err <= s.double().unsqueeze(1) * (1 / 508 + 2e-5) + 1e-30).all()
    assert err.max() > 0                               # the limbs are not exact


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


def test_gemm_i8_exact_on_exact_limbs(gpu):
    print("gemm i8 exact limbs", flush=True)
    E, N, K = 3, 256, 512
    w = make_int8(E * N, K, seed=5)
    counts = torch.tensor([130, 0, 77]).int()
    offsets = (torch.cumsum(counts, 0) - counts).int()
    R = int(counts.sum())
    g = torch.Generator().manual_seed(1)
    A = torch.randint(-127, 128, (R, K), generator=g).float()
    A[:, 0] = 127.0                       # row max exactly 127: s = 1, lo = 0
    q, s = _limbs(gpu, A)
    assert (s.cpu() == 1.0).all()
    out = torch.full((R, N), float("nan"), device=gpu)
    ops.grouped_gemm_i8(w.to(gpu), N, False, q, s, out, offsets.to(gpu), counts.to(gpu), E)
    torch.cuda.synchronize()
    want = _dense(A, dequant(w), counts, offsets, N)
    assert rel_l2(out.cpu(), want) < 1e-6


@pytest.mark.parametrize("N,K", [(256, 512), (320, 2048)])
def test_gemm_i8_plain_ragged(gpu, N, K):
    print(f"gemm i8 plain N={N} K={K}", flush=True)
    E = 5
    w = make_int8(E * N, K, seed=N + K)
    counts = _counts(E, K)
    offsets = (torch.cumsum(counts, 0) - counts).int()
    R = int(counts.sum())
    A = torch.randn(R, K).bfloat16().float()
    q, s = _limbs(gpu, A)
    out = torch.full((R, N), float("nan"), device=gpu)
    ops.grouped_gemm_i8(w.to(gpu), N, False, q, s, out, offsets.to(gpu), counts.to(gpu), E)
    torch.cuda.synchronize()
    want = _dense(A, dequant(w), counts, offsets, N)
    assert not torch.isnan(out).any()
    assert rel_l2(out.cpu(), want) < 2e-4


def test_gemm_i8_swiglu_then_down(gpu):
    print("gemm i8 swiglu + down", flush=True)
    E, I, H = 4, 192, 512
    wgu = make_int8(E * 2 * I, H, seed=1)
    wdn = make_int8(E * H, I, seed=2)
    counts = _counts(E, 3)
    offsets = (torch.cumsum(counts, 0) - counts).int()
    R = int(counts.sum())
    A = torch.randn(R, H).bfloat16().float()
    q, s = _limbs(gpu, A)
    h = torch.full((R, I), float("nan"), device=gpu)
    ops.grouped_gemm_i8(wgu.to(gpu), 2 * I, True, q, s, h, offsets.to(gpu), counts.to(gpu), E)
    torch.cuda.synchronize()
    gu = _dense(A, dequant(wgu), counts, offsets, 2 * I)
    g, u = gu[:, :I], gu[:, I:]
    h_want = g / (1 + torch.exp(-g)) * u
    assert rel_l2(h.cpu(), h_want) < 2e-4
    hq, hs = _limbs(gpu, h)
    y = torch.full((R, H), float("nan"), device=gpu)
    ops.grouped_gemm_i8(wdn.to(gpu), H, False, hq, hs, y, offsets.to(gpu), counts.to(gpu), E)
    torch.cuda.synchronize()
    y_want = _dense(h_want.float(), dequant(wdn), counts, offsets, H)
    assert rel_l2(y.cpu(), y_want) < 5e-4


def _rows_case(E, seed):
    """row counts around both tile sizes (0, 1, 31, 32, 33, 64, 65, 128,
    129, ...) over E experts, most of them empty when E is large"""
    g = torch.Generator().manual_seed(seed)
    edge = torch.tensor([0, 1, 31, 32, 33, 63, 64, 65, 127, 128, 129, 200, 3, 17])
    c = torch.zeros(E, dtype=torch.int32)
    pick = torch.randperm(E, generator=g)[: min(E, 3 * len(edge))]
    c[pick] = edge.repeat(3)[: len(pick)].int()
    return c


@pytest.mark.parametrize("E,split,K", [(14, 64, 512), (37, 1, 512), (37, 32, 256), (37, 100000, 512),
                                       (1000, 64, 640), (1024, 200, 512), (37, 64, 320)])
@pytest.mark.parametrize("swiglu", [False, True])
def test_gemm_i8_rows_mode_matches_tiles(gpu, E, split, K, swiglu):
    """The library's own tile lists (32-row tiles for experts of <= split
    rows, 128-row tiles above) give the tiled call's products bit for bit,
    and the fp64 products within the limb error.  K = 320 is not a whole
    number of the narrow tiles' 128-K stages: all experts then take the
    128-row tiles."""
    print(f"gemm i8 rows mode E={E} split={split} K={K} swiglu={swiglu}", flush=True)
    I = 320
    N = 2 * I if swiglu else 576
    w = make_int8(E * N, K, seed=E + split)
    counts = _rows_case(E, E + 7)
    offsets = (torch.cumsum(counts, 0) - counts).int()
    R = int(counts.sum())
    A = torch.randn(R, K).bfloat16().float()
    q, s = _limbs(gpu, A)
    cols = I if swiglu else N
    ref = torch.full((R, cols), float("nan"), device=gpu)
    out = torch.full((R, cols), float("nan"), device=gpu)
    wg = w.to(gpu)
    ops.grouped_gemm_i8(wg, N, swiglu, q, s, ref, offsets.to(gpu), counts.to(gpu), E)
    ops.grouped_gemm_i8_rows(wg, N, swiglu, q, s, out, offsets.to(gpu), counts.to(gpu), E, split=split)
    torch.cuda.synchronize()
    assert not torch.isnan(out).any()
    assert torch.equal(out.cpu(), ref.cpu())
    want = _dense(A, dequant(w), counts, offsets, N)
    if swiglu:
        g_, u_ = want[:, :I], want[:, I:]
        want = g_ / (1 + torch.exp(-g_)) * u_
    assert rel_l2(out.cpu(), want) < 2e-4


@pytest.mark.parametrize("E,split,K,T", [(37, 64, 512, 300), (14, 1, 640, 97), (1000, 64, 2048, 700),
                                         (37, 100000, 384 + 64, 50)])
@pytest.mark.parametrize("swiglu", [False, True])
def test_gemm_i8_gather_matches_copied_rows(gpu, E, split, K, T, swiglu):
    """Gather mode (routed row r reads token row map[r]) gives the products
    of the call on the rows copied into routed order, bit for bit: the same
    limbs reach the same MFMAs.  K = 512 is the smallest K that runs both
    tile kinds in gather mode (its narrow tiles' row map is read at their
    third K stage), K = 448 one with 128-row tiles only."""
    print(f"gemm i8 gather E={E} split={split} K={K} T={T} swiglu={swiglu}", flush=True)
    I = 320
    N = 2 * I if swiglu else 576
    w = make_int8(E * N, K, seed=E + K)
    counts = _rows_case(E, E + 11)
    offsets = (torch.cumsum(counts, 0) - counts).int()
    R = int(counts.sum())
    g = torch.Generator().manual_seed(K + T)
    X = torch.randn(T, K, generator=g).bfloat16().float()
    qt, st = _limbs(gpu, X)
    row_map = torch.randint(0, T, (R,), generator=g, dtype=torch.int32)
    idx = row_map.long().to(gpu)
    q, s = qt[idx].contiguous(), st[idx].contiguous()
    cols = I if swiglu else N
    ref = torch.full((R, cols), float("nan"), device=gpu)
    out = torch.full((R, cols), float("nan"), device=gpu)
    wg = w.to(gpu)
    ops.grouped_gemm_i8_rows(wg, N, swiglu, q, s, ref, offsets.to(gpu), counts.to(gpu), E, split=split)
    ops.grouped_gemm_i8_rows_gather(wg, N, swiglu, qt, row_map.to(gpu), s, out, offsets.to(gpu),
                                    counts.to(gpu), E, split=split)
    torch.cuda.synchronize()
    assert not torch.isnan(out).any()
    assert torch.equal(out.cpu(), ref.cpu())


def test_gemm_i8_gather_rejects_short_k(gpu):
    """K with too few K tiles for the row map's timing is refused on the host."""
    E, N, K = 4, 256, 256
    w = make_int8(E * N, K, seed=3).to(gpu)
    counts = torch.tensor([10, 0, 5, 1], dtype=torch.int32)
    offsets = (torch.cumsum(counts, 0) - counts).int()
    q = torch.zeros(8, 2 * K, dtype=torch.int8, device=gpu)
    s = torch.ones(16, device=gpu)
    out = torch.empty(16, N, device=gpu)
    with pytest.raises(Exception, match="gather"):
        ops.grouped_gemm_i8_rows_gather(w, N, False, q, torch.zeros(16, dtype=torch.int32, device=gpu), s, out,
                                        offsets.to(gpu), counts.to(gpu), E)
