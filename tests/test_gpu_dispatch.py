"""Dispatch and combine on the GPU: counts, offsets, permutation, token map
and tile table bit-exact against the oracle's stable counting sort; the
permuted bf16 rows exact; the unpermute fma chain bit-exact."""
import pytest
import torch

from oracle import oracle as O
from grimoire_amd import ops

pytestmark = pytest.mark.gpu


def _ids(T, K, E, seed, zipf=0.0, invalid=0):
    g = torch.Generator().manual_seed(seed)
    if zipf > 0:
        p = torch.arange(1, E + 1, dtype=torch.float64) ** -zipf
        ids = torch.stack([torch.multinomial(p, K, replacement=False, generator=g) for _ in range(T)])
    else:
        ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)])
    ids = ids.int()
    if invalid:
        idx = torch.randint(0, T * K, (invalid,), generator=g)
        ids.view(-1)[idx] = -1
    return ids.contiguous()


@pytest.mark.parametrize("T,K,E,mc,zipf,invalid", [
    (1, 8, 128, 128, 0.0, 0),
    (16, 4, 64, 128, 0.0, 0),
    (300, 10, 512, 128, 1.2, 0),       # several count blocks, skewed
    (4096, 10, 512, 128, 1.2, 0),      # C4 size
    (77, 6, 33, 16, 0.0, 5),           # odd sizes, routes not computed here
    (1000, 3, 2000, 64, 0.0, 0),       # more experts than scan threads
])
def test_dispatch_bit_exact(gpu, T, K, E, mc, zipf, invalid):
    print(f"dispatch T={T} K={K} E={E} mc={mc} zipf={zipf} invalid={invalid}", flush=True)
    ids = _ids(T, K, E, T + E, zipf, invalid)
    H = 64
    x = torch.randn(T, H)
    R = T * K
    tmax = E + (R + mc - 1) // mc
    d = gpu
    counts = torch.empty(E, dtype=torch.int32, device=d)
    offsets = torch.empty(E, dtype=torch.int32, device=d)
    inverse = torch.empty(R, dtype=torch.int32, device=d)
    perm = torch.full((R,), -7, dtype=torch.int32, device=d)
    te = torch.empty(tmax, dtype=torch.int32, device=d)
    tm = torch.empty(tmax, dtype=torch.int32, device=d)
    xperm = torch.zeros(R, H, dtype=torch.int16, device=d)
    xrow = torch.empty(T, H, dtype=torch.int16, device=d)
    ops.launch_moe_route_grouped(x.to(d), ids.to(d), xperm, xrow, counts, offsets, inverse, te, tm,
                                 tmax, T, H, E, mc, K, perm_token=perm)
    torch.cuda.synchronize()
    want = O.dispatch(ids, E, mc, tmax)
    assert torch.equal(counts.cpu(), want["counts"])
    assert torch.equal(offsets.cpu(), want["offsets"])
    assert torch.equal(inverse.cpu(), want["inverse"])
    nvalid = int(want["counts"].sum())
    assert torch.equal(perm.cpu()[:nvalid], want["perm_token"][:nvalid])
    assert torch.equal(te.cpu(), want["tile_e"])
    nt = want["n_tiles"]
    assert torch.equal(tm.cpu()[:nt], want["tile_mb"][:nt])
    xb = x.bfloat16().view(torch.int16)
    assert torch.equal(xrow.cpu(), xb)
    inv = want["inverse"]
    for r in range(0, R, max(1, R // 500)):
        if inv[r] >= 0:
            assert torch.equal(xperm.cpu()[inv[r]], xb[r // K])


@pytest.mark.parametrize("T,K,H", [(1, 8, 2048), (33, 10, 2048), (5, 4, 2880)])
def test_unpermute_bit_exact(gpu, T, K, H):
    print(f"unpermute T={T} K={K} H={H}", flush=True)
    R = T * K
    src = torch.randn(R, H)
    inv = torch.randperm(R).int()
    inv[::7] = -1
    rw = torch.rand(R)
    out = torch.empty(T, H, device=gpu)
    ops.launch_moe_unpermute(src.to(gpu), inv.to(gpu), rw.to(gpu), out, T, K, H)
    torch.cuda.synchronize()
    want = O.unpermute(src, inv, rw, T, K, H)
    assert torch.equal(out.cpu(), want)
    # bf16 rows
    sb = src.bfloat16()
    out2 = torch.empty(T, H, device=gpu)
    ops.launch_moe_unpermute(sb.view(torch.int16).to(gpu), inv.to(gpu), rw.to(gpu), out2, T, K, H)
    torch.cuda.synchronize()
    want2 = O.unpermute(sb.float(), inv, rw, T, K, H)
    assert torch.equal(out2.cpu(), want2)


@pytest.mark.parametrize("T,K,H,shared,outs", [(1, 8, 2048, True, "both"), (33, 10, 2048, True, "f32"),
                                               (5, 4, 2880, False, "bf"), (3, 8, 7168, True, "both"),
                                               (2, 2, 9000, True, "both"), (7, 3, 12, False, "both"),
                                               (3, 16, 1024, True, "both"), (4, 1, 256, False, "f32")])
def test_rmsnorm_moe_residual(gpu, T, K, H, shared, outs):
    """launch_rmsnorm_moe_residual_batched (src/prefill.cpp:1004-1045): the residual
    update is bit-exact (same fma order); the normalised output differs only by the
    order of the sum of squares and the device rsqrt (rel 1e-5)."""
    print(f"rmsnorm_moe_residual T={T} K={K} H={H} shared={shared} outs={outs}", flush=True)
    g = torch.Generator().manual_seed(T * 1000 + H)
    R, eps, off = T * K, 1e-6, 1.0 if H != 12 else 0.5
    routed = torch.randn(R, H, generator=g).bfloat16().view(torch.int16)
    inv = torch.randperm(R, generator=g).int()
    inv[::5] = -1
    rw = torch.rand(R, generator=g)
    h = torch.randn(T, H, generator=g) * 2
    sh = torch.randn(T, H, generator=g) if shared else None
    w = (torch.randn(H, generator=g) * 0.2).bfloat16().view(torch.int16)
    hd = h.to(gpu)
    out = torch.full((T, H), float("nan"), device=gpu) if outs in ("both", "f32") else None
    obf = torch.zeros((T, H), dtype=torch.int16, device=gpu) if outs in ("both", "bf") else None
    ops.launch_rmsnorm_moe_residual_batched(hd, routed.to(gpu), inv.to(gpu), rw.to(gpu),
                                            None if sh is None else sh.to(gpu), w.to(gpu), out,
                                            obf, T, K, H, eps, weight_offset=off)
    torch.cuda.synchronize()
    hn, want, want_bf = O.rmsnorm_moe_residual(h, routed, inv, rw, sh, w, off, T, K, H, eps)
    assert torch.equal(hd.cpu(), hn)
    if out is not None:
        err = (out.cpu() - want).abs().max().item()
        assert err <= 1e-5 * want.abs().max().item(), err
    if obf is not None:
        # bf16 of values equal to 1e-5 relative: at most one bf16 ulp apart
        d = (obf.cpu().int() - want_bf.int()).abs()
        assert d.max().item() <= 1, d.max().item()


@pytest.mark.parametrize("T,H,addends", [(1, 2048, 2), (64, 7168, 1), (3, 9000, 0), (17, 2880, 2)])
def test_rmsnorm_residual(gpu, T, H, addends):
    """launch_rmsnorm_residual_batched (src/prefill.cpp:627-700): h bit-exact, out rel 1e-5."""
    print(f"rmsnorm_residual T={T} H={H} addends={addends}", flush=True)
    g = torch.Generator().manual_seed(T + H)
    eps = 1e-6
    h = torch.randn(T, H, generator=g) * 2
    r0 = torch.randn(T, H, generator=g) if addends >= 1 else None
    r1 = torch.randn(T, H, generator=g) if addends >= 2 else None
    w = (torch.randn(H, generator=g) * 0.2).bfloat16().view(torch.int16)
    hd = h.to(gpu)
    out = torch.full((T, H), float("nan"), device=gpu)
    obf = torch.zeros((T, H), dtype=torch.int16, device=gpu)
    ops.launch_rmsnorm_residual_batched(hd, None if r0 is None else r0.to(gpu),
                                        None if r1 is None else r1.to(gpu), w.to(gpu), out, T, H,
                                        eps, out_bf=obf)
    torch.cuda.synchronize()
    hn, want, want_bf = O.rmsnorm_residual(h, r0, r1, w, 1.0, T, H, eps)
    assert torch.equal(hd.cpu(), hn)
    err = (out.cpu() - want).abs().max().item()
    assert err <= 1e-5 * want.abs().max().item(), err
    assert (obf.cpu().int() - want_bf.int()).abs().max().item() <= 1



@pytest.mark.parametrize("T,K,H", [(33, 10, 2048), (5, 4, 2880)])
def test_unpermute_range_bit_exact(gpu, T, K, H):
    """launch_moe_unpermute_range (src/prefill.cpp:2674): two ranges, the
    second accumulating, against the oracle's fma chain; the full range equals
    the plain unpermute bit for bit."""
    print(f"unpermute_range T={T} K={K} H={H}", flush=True)
    R = T * K
    g = torch.Generator().manual_seed(T)
    src = torch.randn(R, H, generator=g)
    inv = torch.randperm(R, generator=g).int()
    inv[::7] = -1
    rw = torch.rand(R, generator=g)
    cut = R // 3
    dst = torch.empty(T, H, device=gpu)
    ops.launch_moe_unpermute_range(src[:cut].to(gpu), inv.to(gpu), rw.to(gpu), dst, T, K, H, 0, cut)
    ops.launch_moe_unpermute_range(src[cut:].to(gpu), inv.to(gpu), rw.to(gpu), dst, T, K, H, cut, R,
                                   accumulate=True)
    torch.cuda.synchronize()
    want = O.unpermute_range(src[:cut], inv, rw, torch.zeros(T, H), T, K, H, 0, cut, False)
    want = O.unpermute_range(src[cut:], inv, rw, want, T, K, H, cut, R, True)
    assert torch.equal(dst.cpu(), want)
    full = torch.empty(T, H, device=gpu)
    ops.launch_moe_unpermute_range(src.to(gpu), inv.to(gpu), rw.to(gpu), full, T, K, H, 0, R)
    torch.cuda.synchronize()
    assert torch.equal(full.cpu(), O.unpermute(src, inv, rw, T, K, H))


@pytest.mark.parametrize("rows,width", [(300, 2048), (7, 130)])
def test_permute_rows_bf16_exact(gpu, rows, width):
    print(f"permute_rows rows={rows} width={width}", flush=True)
    g = torch.Generator().manual_seed(rows)
    src = torch.randn(64, width, generator=g)
    perm = torch.randint(0, 64, (rows,), dtype=torch.int32, generator=g)
    dst = torch.empty(rows, width, dtype=torch.int16, device=gpu)
    ops.launch_permute_rows_bf16(src.to(gpu), perm.to(gpu), dst, rows, width)
    torch.cuda.synchronize()
    assert torch.equal(dst.cpu(), O.permute_rows_bf16(src, perm, width))


def test_swiglu_and_scale_by_sigmoid(gpu):
    """launch_swiglu_bf16 within one bf16 ulp of float64 (plus 1e-6 of the
    largest for cancellation); scale_by_sigmoid{,_batched} within 2e-7
    relative."""
    print("swiglu_bf16 / scale_by_sigmoid", flush=True)
    g = torch.Generator().manual_seed(5)
    T, I, H = 17, 768, 1000
    gu = (torch.randn(T, 2 * I, generator=g) * 3).bfloat16().view(torch.int16)
    out = torch.empty(T, I, dtype=torch.int16, device=gpu)
    ops.launch_swiglu_bf16(gu.to(gpu), out, T, I)
    x = torch.randn(T, H, generator=g)
    gate = torch.randn(T, generator=g) * 4
    xd = x.to(gpu)
    ops.launch_scale_by_sigmoid_batched(xd, gate.to(gpu), T, H)
    x1 = torch.randn(H, generator=g)
    x1d = x1.to(gpu)
    ops.launch_scale_by_sigmoid(x1d, gate[:1].to(gpu), H)
    torch.cuda.synchronize()
    want = O.swiglu_bf16(gu, T, I)
    got = out.cpu().view(torch.bfloat16).double()
    assert ((got - want).abs() <= want.abs() * 2.0 ** -8 + 1e-6 * want.abs().max()).all()
    wx = O.scale_by_sigmoid_batched(x, gate)
    assert ((xd.cpu().double() - wx).abs() <= 2e-7 * wx.abs() + 1e-30).all()
    w1 = x1.double() / (1 + torch.exp(-gate[0].double()))
    assert ((x1d.cpu().double() - w1).abs() <= 2e-7 * w1.abs() + 1e-30).all()


@pytest.mark.parametrize("T,K,E,invalid", [
    (4096, 10, 512, 0),                # C4: 160 rank blocks forming their own offsets
    (700, 6, 2048, 9),                 # the largest E the rank blocks scan; skipped routes
    (300, 4, 3000, 0),                 # beyond it: the single-block scan as with a table
    (5, 3, 7, 0),
])
def test_route_without_tile_table_matches(gpu, T, K, E, invalid):
    """Without a tile table the rank blocks form the expert offsets
    themselves: counts, offsets, rows and token map equal the oracle's
    counting sort (and so the call with a table)."""
    print(f"route without tile table T={T} K={K} E={E}", flush=True)
    ids = _ids(T, K, E, 31 + E, zipf=1.1, invalid=invalid)
    R = T * K
    counts = torch.empty(E, dtype=torch.int32, device=gpu)
    offsets = torch.empty(E, dtype=torch.int32, device=gpu)
    inverse = torch.empty(R, dtype=torch.int32, device=gpu)
    perm = torch.full((R,), -7, dtype=torch.int32, device=gpu)
    ops.launch_moe_route_grouped(None, ids.to(gpu), None, None, counts, offsets, inverse, None, None, 0,
                                 T, 64, E, 0, K, perm_token=perm)
    torch.cuda.synchronize()
    d = O.dispatch(ids, E, 0, 0)
    assert torch.equal(counts.cpu(), d["counts"]) and torch.equal(offsets.cpu(), d["offsets"])
    assert torch.equal(inverse.cpu(), d["inverse"])
    n = int(d["counts"].sum())
    assert torch.equal(perm.cpu()[:n], d["perm_token"][:n])
