"""The three bridge symbols (src/xe2_grouped_bridge.cpp:135,
src/xe2_grouped_bridge.hpp:22, src/xe2_fused_moe_bridge.cpp:32) on the GPU.

Outputs are bf16, so each element is compared with the float64 product of
the exact dequantised weights to one bf16 ulp (2^-8 relative) plus 1e-3 of
the output rms, and the whole to rel-L2 3e-3 (bf16 rounding alone gives up
to ~2.3e-3).  The w4a16 layout and sign convention are pinned by the
reference's own bridge test (src/test_xe2_bridge.cpp:33-77), whose inputs
and closed-form result are restated in test_w4a16_reference_case."""
import pytest
import torch

from grimoire_amd import ops
from grimoire_amd.weights import make_mxfp4
from tests.helpers import dequant, rel_l2

pytestmark = pytest.mark.gpu


def _bf16_close(got, want, what):
    got, want = got.double(), want.double()
    rms = float(want.pow(2).mean().sqrt())
    err = (got - want).abs()
    bound = 2.0 ** -8 * want.abs() + 1e-3 * rms
    bad = int((err > bound).sum())
    rl = rel_l2(got, want)
    assert bad == 0 and rl <= 3e-3, f"{what}: {bad} elements beyond one bf16 ulp, rel-L2 {rl:.3e}"


def _rows(E, seed, hi=200):
    g = torch.Generator().manual_seed(seed)
    r = torch.randint(0, hi, (E,), generator=g).int()
    r[0] = 0
    if E > 2:
        r[2] = 1
    return r


def _dense(a, W, rows, n):
    """out[r] = a[r] . W_e^T for the expert e owning row r (rows in expert order)."""
    out = torch.zeros(a.shape[0], n, dtype=torch.float64)
    r0 = 0
    for e, c in enumerate(rows.tolist()):
        if c:
            out[r0:r0 + c] = a[r0:r0 + c].double() @ W[e * n:(e + 1) * n].double().T
        r0 += c
    return out


def _s4_dense(b, s, E, n, k, gs):
    """Signed-s4 codes [E*n][k/2] (low nibble = even k) x bf16 group scales."""
    lo = (b & 0xF).to(torch.int32)
    hi = (b >> 4).to(torch.int32)
    q = torch.stack([lo, hi], dim=2).reshape(E * n, k)
    q = torch.where(q >= 8, q - 16, q).double()
    sf = s.view(torch.bfloat16).double().reshape(E * n, k // gs).repeat_interleave(gs, dim=1)
    return q * sf


def test_w4a16_reference_case(gpu):
    """src/test_xe2_bridge.cpp:33-77: E=2, M=32, N=K=256, GS=128, rows {13, 19}."""
    E, M, N, K, GS = 2, 32, 256, 256, 128
    m = torch.arange(M).view(M, 1)
    kk = torch.arange(K).view(1, K)
    a = ((((m * 7 + kk * 3) % 19) - 9).float() / 16.0).bfloat16()
    s = torch.zeros(E, N, K // GS)
    for g_ in range(K // GS):
        s[:, :, g_] = 0.03125 * (1 + g_)
    s = s.bfloat16()
    e_ = torch.arange(E).view(E, 1, 1)
    n_ = torch.arange(N).view(1, N, 1)
    kb = torch.arange(K // 2).view(1, 1, K // 2)
    lo = ((e_ * 5 + n_ * 3 + 2 * kb) % 15) - 7
    hi = ((e_ * 7 + n_ + 2 * kb + 1) % 15) - 7
    b = (((hi & 15) << 4) | (lo & 15)).to(torch.uint8)
    rows = torch.tensor([13, 19], dtype=torch.int32)
    # the reference's closed form, in float64
    W = _s4_dense(b.reshape(E * N, K // 2), s.view(torch.int16).reshape(-1), E, N, K, GS)
    want = _dense(a.float(), W.float(), rows, N)
    d = torch.zeros(M, N, dtype=torch.bfloat16, device=gpu)
    ops.xe2_grouped_w4a16(a.to(gpu), b.to(gpu), s.to(gpu), d, N, K, rows.to(gpu), E, GS)
    torch.cuda.synchronize()
    got = d.cpu().float()
    assert float((got.double() - want).abs().max()) < 0.2          # the reference's own bar
    _bf16_close(got, want, "w4a16 reference case")


@pytest.mark.parametrize("gs", [64, 128, 256])
def test_w4a16_ragged(gpu, gs):
    E, n, k = 6, 192, 512
    print(f"xe2 w4a16 gs={gs}", flush=True)
    g = torch.Generator().manual_seed(gs)
    rows = _rows(E, gs)
    R = int(rows.sum())
    a = torch.randn(R, k, generator=g).bfloat16()
    b = torch.randint(0, 256, (E * n, k // 2), generator=g, dtype=torch.int32).to(torch.uint8)
    s = (torch.rand(E * n, k // gs, generator=g) * 0.05 + 0.001).bfloat16()
    want = _dense(a.float(), _s4_dense(b, s.view(torch.int16), E, n, k, gs).float(), rows, n)
    d = torch.full((R, n), float("nan"), dtype=torch.bfloat16, device=gpu)
    ops.xe2_grouped_w4a16(a.to(gpu), b.to(gpu), s.to(gpu), d, n, k, rows.to(gpu), E, gs)
    torch.cuda.synchronize()
    _bf16_close(d.cpu().float(), want, f"w4a16 gs={gs}")


def test_grouped_mxfp4_bridge(gpu):
    E, n, k = 5, 320, 1024
    rows = _rows(E, 3)
    R = int(rows.sum())
    w = make_mxfp4(E * n, k, seed=9)
    a = torch.randn(R, k, generator=torch.Generator().manual_seed(4)).bfloat16()
    want = _dense(a.float(), dequant(w), rows, n)
    d = torch.full((R, n), float("nan"), dtype=torch.bfloat16, device=gpu)
    ops.xe2_grouped_mxfp4_bf16(a.to(gpu), w.payload.to(gpu), w.scales.to(gpu), d, n, k,
                               rows.to(gpu), E)
    torch.cuda.synchronize()
    _bf16_close(d.cpu().float(), want, "grouped mxfp4 bridge")


def test_fused_gate_up_bridge(gpu):
    E, n, k = 4, 256, 768
    rows = _rows(E, 5)
    R = int(rows.sum())
    w = make_mxfp4(E * 2 * n, k, seed=11)
    a = torch.randn(R, k, generator=torch.Generator().manual_seed(6)).bfloat16()
    gu = _dense(a.float(), dequant(w), rows, 2 * n)        # [R][2n]: per expert gate rows then up
    # per expert the 2n outputs are gate[0:n], up[n:2n]
    gate, up = gu[:, :n], gu[:, n:]
    want = gate / (1.0 + torch.exp(-gate)) * up
    d = torch.full((R, n), float("nan"), dtype=torch.bfloat16, device=gpu)
    ops.xe2_fused_moe_gate_up_mxfp4_silu_bf16(a.to(gpu), w.payload.to(gpu), w.scales.to(gpu), d, n,
                                              k, rows.to(gpu), E)
    torch.cuda.synchronize()
    _bf16_close(d.cpu().float(), want, "fused gate_up bridge")


def test_grouped_mxfp4_bridge_variants(gpu):
    """The _full / _m8 / _m16 symbols (src/xe2_grouped_bridge.cpp:149-177)
    give the base bridge's result bit for bit."""
    from grimoire_amd import _abi
    E, n, k = 3, 256, 512
    rows = _rows(E, 7)
    R = int(rows.sum())
    w = make_mxfp4(E * n, k, seed=13)
    a = torch.randn(R, k, generator=torch.Generator().manual_seed(8)).bfloat16().to(gpu)
    pw, ps, rd = w.payload.to(gpu), w.scales.to(gpu), rows.to(gpu)
    base = torch.empty(R, n, dtype=torch.bfloat16, device=gpu)
    ops.xe2_grouped_mxfp4_bf16(a, pw, ps, base, n, k, rd, E)
    for v in ("full", "m8", "m16"):
        d = torch.full((R, n), float("nan"), dtype=torch.bfloat16, device=gpu)
        getattr(_abi.lib(), f"grimoire_xe2_grouped_mxfp4_bf16_{v}")(
            None, a.data_ptr(), pw.data_ptr(), ps.data_ptr(), d.data_ptr(), n, k, rd.data_ptr(),
            None, E, None)
        torch.cuda.synchronize()
        assert torch.equal(d.view(torch.int16), base.view(torch.int16)), v


def test_bridges_on_two_streams(gpu):
    """Bridge calls in flight on two streams at once (the reference runs the
    shared expert on an auxiliary queue, src/grimoire.cpp:22750-22765) with
    different expert layouts: each result matches its own reference, so
    no call's tile order leaks into the other's."""
    E1, n1, k1 = 7, 256, 512
    E2, n2, k2 = 3, 192, 1024
    rows1, rows2 = _rows(E1, 21, hi=300), _rows(E2, 22, hi=90)
    R1, R2 = int(rows1.sum()), int(rows2.sum())
    w1 = make_mxfp4(E1 * n1, k1, seed=31)
    w2 = make_mxfp4(E2 * 2 * n2, k2, seed=32)
    a1 = torch.randn(R1, k1, generator=torch.Generator().manual_seed(33)).bfloat16()
    a2 = torch.randn(R2, k2, generator=torch.Generator().manual_seed(34)).bfloat16()
    want1 = _dense(a1.float(), dequant(w1), rows1, n1)
    gu = _dense(a2.float(), dequant(w2), rows2, 2 * n2)
    want2 = gu[:, :n2] / (1.0 + torch.exp(-gu[:, :n2])) * gu[:, n2:]
    g1 = [t.to(gpu) for t in (a1, w1.payload, w1.scales, rows1)]
    g2 = [t.to(gpu) for t in (a2, w2.payload, w2.scales, rows2)]
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs1 = [torch.full((R1, n1), float("nan"), dtype=torch.bfloat16, device=gpu) for _ in range(6)]
    outs2 = [torch.full((R2, n2), float("nan"), dtype=torch.bfloat16, device=gpu) for _ in range(6)]
    torch.cuda.synchronize()
    for d1, d2 in zip(outs1, outs2):
        ops.xe2_grouped_mxfp4_bf16(g1[0], g1[1], g1[2], d1, n1, k1, g1[3], E1, stream=s1)
        ops.xe2_fused_moe_gate_up_mxfp4_silu_bf16(g2[0], g2[1], g2[2], d2, n2, k2, g2[3], E2,
                                                  stream=s2)
    torch.cuda.synchronize()
    for i, (d1, d2) in enumerate(zip(outs1, outs2)):
        _bf16_close(d1.cpu().float(), want1, f"stream 1 call {i}")
        _bf16_close(d2.cpu().float(), want2, f"stream 2 call {i}")
