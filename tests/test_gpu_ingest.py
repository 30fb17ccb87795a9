"""Expert-weight ingestion on the GPU (grimoire_moe_ingest_projection,
grimoire_moe_int4_to_signed) against the oracle restatements of
src/gptq.cpp:56-83 and src/grimoire.cpp:1396-1434, 8340-8397: byte-exact
payloads, scales and zero points, at row offsets inside stacked weights."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle as O
from grimoire_amd import _abi, ingest, ops
from grimoire_amd.weights import MoeLayer
from tests.test_oracle import _lcg_tensors

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"


def _gptq_src(out, inn, group, seed, dev):
    qw, qz, sc = _lcg_tensors(out, inn, group, seed)
    t = lambda a: torch.from_numpy(a.copy()).to(dev)
    src = ingest.gptq(t(qw).view(inn // 8, out), t(qz).view(inn // group, out // 8),
                      t(sc.view(np.int16)).view(inn // group, out), group)
    return src, (qw, qz, sc)


@pytest.mark.parametrize("out,inn,group,row0,exact", [(512, 2048, 128, 72, False),
                                                      (512, 2048, 128, 0, True),
                                                      (72, 384, 128, 8, False),
                                                      (136, 768, 64, 40, True)])
def test_gptq_ingest_bit_exact(gpu, out, inn, group, row0, exact):
    print(f"gptq ingest out={out} in={inn} g={group} row0={row0} exact={exact}", flush=True)
    src, (qw, qz, sc) = _gptq_src(out, inn, group, 12345, gpu)
    fmt = ingest.target_format(_abi.SRC_GPTQ, exact)
    N = row0 + out + 16
    dst = ingest.stacked(fmt, N, inn, group, gpu)
    dst.payload.fill_(0x5A); dst.scales.fill_(0x1234); dst.zeros.fill_(0xA5)
    ingest.ingest_projection(src, dst, row0)
    torch.cuda.synchronize()
    pay, scl, z = O.gptq_repack(qw, qz, sc, inn, out, group, keep_f16=exact)
    rows = slice(row0, row0 + out)
    assert np.array_equal(dst.payload.cpu().numpy()[rows], pay)
    assert np.array_equal(dst.scales.cpu().numpy()[rows], scl)
    assert np.array_equal(dst.zeros.cpu().numpy()[rows], z)
    # rows outside [row0, row0+out) untouched
    assert (dst.payload.cpu()[:row0] == 0x5A).all() and (dst.payload.cpu()[row0 + out:] == 0x5A).all()
    assert (dst.zeros.cpu()[row0 + out:] == 0xA5).all()
    if out == 512 and exact:
        g = json.loads((GOLD / "gptq_probes.json").read_text())
        w = dst.to("cpu")
        w.N = N
        s = w.struct()
        for o, k, want in zip(g["o"], g["k"], g["w"]):
            got = O.orc().orc_qw_at(O.byref(s), row0 + o, k)
            assert abs(got - want) <= 1e-6 * (1 + abs(want))


def test_mxfp4_packed_copy(gpu):
    print("mxfp4 packed copy", flush=True)
    g = torch.Generator().manual_seed(1)
    out, inn = 96, 2880
    wp = torch.randint(0, 256, (out, inn // 2), dtype=torch.uint8, generator=g)
    ws = torch.randint(119, 126, (out, inn // 32), dtype=torch.uint8, generator=g)
    dst = ingest.stacked(_abi.FMT_MXFP4, 3 * out, inn, 32, gpu)
    ingest.ingest_projection(ingest.mxfp4_packed(wp, ws), dst, out)          # host source
    ingest.ingest_projection(ingest.mxfp4_packed(wp.to(gpu), ws.to(gpu)), dst, 2 * out)
    torch.cuda.synchronize()
    for r0 in (out, 2 * out):
        assert torch.equal(dst.payload.cpu()[r0:r0 + out], wp)
        assert torch.equal(dst.scales.cpu()[r0:r0 + out], ws)


@pytest.mark.parametrize("with_zp", [True, False])
def test_int4_packed_ingest(gpu, with_zp):
    print(f"int4 packed with_zp={with_zp}", flush=True)
    g = torch.Generator().manual_seed(2)
    out, inn, group = 40, 512, 128
    wp = torch.randint(0, 256, (out, inn // 2), dtype=torch.uint8, generator=g)
    ws = (torch.randn(out, inn // group, generator=g) * 0.02).bfloat16().view(torch.int16)
    zp = (torch.randint(0, 2 ** 31 - 1, (out // 8, inn // group), dtype=torch.int32, generator=g)
          if with_zp else None)
    dst = ingest.stacked(_abi.FMT_INT4, out + 8, inn, group, gpu)
    src = ingest.int4_packed(wp.to(gpu), ws.to(gpu), None if zp is None else zp.to(gpu), group)
    ingest.ingest_projection(src, dst, 8)
    torch.cuda.synchronize()
    assert torch.equal(dst.payload.cpu()[8:], wp)
    assert torch.equal(dst.scales.cpu()[8:], ws)
    want = O.int4_zero_unpack(None if zp is None else zp.numpy(), out, inn // group)
    assert np.array_equal(dst.zeros.cpu().numpy()[8:], want)


def _layer(gate_up, down, E, H, I, K, dev):
    g = torch.Generator().manual_seed(9)
    router = (torch.randn(E, H, generator=g) * 0.02).to(dev)
    return MoeLayer(H, I, E, K, gate_up, down, router)


def test_ingest_layer_then_signed(gpu):
    """A GPTQ layer with symmetric zero points (stored 7): staged expert by
    expert, then the signed-s4 pass.  Bytes match the oracle at each step and
    the layer's output is unchanged by the conversion."""
    print("ingest layer + signed", flush=True)
    E, H, I, K, group = 8, 256, 128, 2, 128
    rng = np.random.default_rng(3)
    experts, raw = [], []
    for e in range(E):
        trip = []
        for (out, inn) in ((I, H), (I, H), (H, I)):
            qw = rng.integers(0, 2 ** 32, (inn // 8, out), dtype=np.uint64).astype(np.uint32)
            qz = np.full((inn // group, out // 8), 0x77777777, np.uint32)
            sc = (np.abs(rng.standard_normal((inn // group, out))) * 0.02).astype(np.float16)
            raw.append((qw.view(np.int32), qz.view(np.int32), sc.view(np.uint16), inn, out))
            trip.append(ingest.gptq(torch.from_numpy(qw.view(np.int32)).to(gpu),
                                    torch.from_numpy(qz.view(np.int32)).to(gpu),
                                    torch.from_numpy(sc.view(np.int16)).to(gpu), group))
        experts.append(tuple(trip))
    gu, dn = ingest.ingest_experts(experts, gpu)
    torch.cuda.synchronize()
    want_gu = [O.gptq_repack(*r[:3], r[3], r[4], group) for i, r in enumerate(raw) if i % 3 < 2]
    want_dn = [O.gptq_repack(*r[:3], r[3], r[4], group) for i, r in enumerate(raw) if i % 3 == 2]
    wgp = np.concatenate([w[0] for w in want_gu]); wgz = np.concatenate([w[2] for w in want_gu])
    wdp = np.concatenate([w[0] for w in want_dn]); wdz = np.concatenate([w[2] for w in want_dn])
    assert np.array_equal(gu.payload.cpu().numpy(), wgp)
    assert np.array_equal(gu.scales.cpu().numpy(), np.concatenate([w[1] for w in want_gu]))
    assert np.array_equal(gu.zeros.cpu().numpy(), wgz)
    assert np.array_equal(dn.payload.cpu().numpy(), wdp)
    assert np.array_equal(dn.zeros.cpu().numpy(), wdz)

    T = 16
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(4)).to(gpu)
    L = _layer(gu, dn, E, H, I, K, gpu)
    rp = _abi.RouteParams(_abi.ROUTE_SOFTMAX, 0, 0, 1.0, None)
    y0 = torch.empty(T, H, device=gpu)
    ops.MoeForward(L, T, rp)(x, y0)
    flag = ingest.to_signed(gu, dn)
    torch.cuda.synchronize()
    assert flag.item() == 1
    O.int4_to_signed(wgp, wgz, wdp, wdz)
    assert np.array_equal(gu.payload.cpu().numpy(), wgp)
    assert np.array_equal(gu.zeros.cpu().numpy(), wgz)
    assert np.array_equal(dn.payload.cpu().numpy(), wdp)
    assert np.array_equal(dn.zeros.cpu().numpy(), wdz)
    y1 = torch.empty(T, H, device=gpu)
    ops.MoeForward(L, T, rp)(x, y1)
    torch.cuda.synchronize()
    assert torch.allclose(y0, y1, rtol=1e-5, atol=1e-6), (y0 - y1).abs().max().item()
    # a second pass finds zero points 0xFF, not 8: nothing changes
    flag2 = ingest.to_signed(gu, dn)
    torch.cuda.synchronize()
    assert flag2.item() == 0
    assert np.array_equal(gu.payload.cpu().numpy(), wgp)
