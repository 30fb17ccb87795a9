"""Tiered NVFP4 experts and the heat policy, CPU side: the oracle pinned
against the reference's own e4m3_to_f32, nvfp4_dequant_row and ExpertHeat
(compiled into oracle/_ref), float64 products and closed forms; the
library's layout and heat functions against the oracle (host code, no GPU)."""
import ctypes as C
import math

import numpy as np
import pytest

from oracle import oracle as O
from grimoire_amd import _abi, tiered


def make_block(lay, rng, scale_lo=0x30):
    """Random NVFP4 expert block: payload uniform, E4M3 scales 0x30..0x3F
    (0.5 .. 1.875), projection scales in [0.5, 2)."""
    b = rng.integers(0, 256, lay["bytes"], dtype=np.uint8)
    for off, n in ((lay["gu_s"], lay["dn_p"] - lay["gu_s"]),
                   (lay["dn_s"], lay["gsc"] - lay["dn_s"])):
        b[off:off + n] = scale_lo + rng.integers(0, 16, n, dtype=np.uint8)
    g = np.array([rng.uniform(0.5, 2.0), rng.uniform(0.5, 2.0), rng.uniform(0.5, 2.0), 0.0],
                 dtype=np.float32)
    b[lay["gsc"]:lay["gsc"] + 16] = g.view(np.uint8)
    return b


def dequant(block, lay, H, I):
    """Dense fp64 gate|up [2I][H] and down [H][I] with the projection scales."""
    r = O.ref()
    fn = (r.ref_nvfp4_dequant_row if r is not None else O.orc().orc_nvfp4_dequant_row)
    g3 = block[lay["gsc"]:lay["gsc"] + 16].view(np.float32)
    gu = np.zeros((2 * I, H), np.float32)
    dn = np.zeros((H, I), np.float32)
    for n in range(2 * I):
        p = np.ascontiguousarray(block[lay["gu_p"] + n * (H // 2):][:H // 2])
        s = np.ascontiguousarray(block[lay["gu_s"] + n * (H // 16):][:H // 16])
        fn(p.ctypes.data, s.ctypes.data, 1.0, H, gu[n].ctypes.data, 1)
    for n in range(H):
        p = np.ascontiguousarray(block[lay["dn_p"] + n * (I // 2):][:I // 2])
        s = np.ascontiguousarray(block[lay["dn_s"] + n * (I // 16):][:I // 16])
        fn(p.ctypes.data, s.ctypes.data, 1.0, I, dn[n].ctypes.data, 1)
    gu64 = gu.astype(np.float64)
    gu64[:I] *= g3[0]
    gu64[I:] *= g3[1]
    return gu64, dn.astype(np.float64) * g3[2]


def test_e4m3_all_codes():
    r = O.ref()
    for b in range(256):
        got = O.orc().orc_e4m3_to_f32(b)
        if r is not None:
            want = r.ref_e4m3_to_f32(b)
            assert (math.isnan(got) and math.isnan(want)) or got == want, b
    assert O.orc().orc_e4m3_to_f32(0x38) == 1.0 and O.orc().orc_e4m3_to_f32(0x7E) == 448.0
    assert O.orc().orc_e4m3_to_f32(0x01) == 2.0 ** -9 and O.orc().orc_e4m3_to_f32(0xB8) == -1.0
    assert math.isnan(O.orc().orc_e4m3_to_f32(0x7F))


def test_nvfp4_dequant_row_matches_reference():
    r = O.ref()
    if r is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    rng = np.random.default_rng(1)
    K = 256
    p = rng.integers(0, 256, K // 2, dtype=np.uint8)
    s = rng.integers(0, 256, K // 16, dtype=np.uint8)
    s[s == 0x7F] = 0x38
    s[s == 0xFF] = 0xB8
    for mul, gs in ((1, 1.5), (0, 3.0)):
        a = np.zeros(K, np.float32); b = np.zeros(K, np.float32)
        O.orc().orc_nvfp4_dequant_row(p.ctypes.data, s.ctypes.data, gs, K, a.ctypes.data, mul)
        r.ref_nvfp4_dequant_row(p.ctypes.data, s.ctypes.data, gs, K, b.ctypes.data, mul)
        assert np.array_equal(a, b)


@pytest.mark.parametrize("H,I", [(2048, 768), (256, 128), (7168, 2048)])
def test_layout_library_matches_oracle(H, I):
    want = O.tmoe_layout(H, I)
    got = tiered.layout(H, I)
    assert (got.H, got.I) == (H, I)
    for k, v in want.items():
        assert getattr(got, k) == v, k
    assert want["bytes"] % 4096 == 0 and want["bytes"] >= want["gsc"] + 16
    assert want["gu_s"] - want["gu_p"] == 2 * I * H // 2
    assert want["dn_p"] - want["gu_s"] == 2 * I * H // 16


def test_layout_rejects_unsupported():
    L = _abi.NvExpertLayout()
    assert _abi.lib().grimoire_tmoe_layout(200, 128, C.byref(L)) == _abi.ERR_SHAPE


def test_tmoe_oracle_against_float64():
    H, I, K, E, M = 256, 128, 3, 5, 4
    lay = O.tmoe_layout(H, I)
    rng = np.random.default_rng(2)
    blocks = [make_block(lay, rng) for _ in range(E)]
    ex = np.array([[0, 3, -1], [4, 4, 1], [2, 7, 0], [1, 2, 3]], np.int32)   # 7 >= E: skipped
    w = rng.random((M, K)).astype(np.float32)
    w[3, 1] = 0.0
    x = rng.standard_normal((M, H)).astype(np.float32)
    h = O.tmoe_gate_up(blocks, H, I, K, ex, x, M)
    y = O.tmoe_down(blocks, H, I, K, ex, w, h, M)
    dq = [dequant(b, lay, H, I) for b in blocks]
    for t in range(M):
        yw = np.zeros(H)
        for s in range(K):
            e = ex[t, s]
            hs = h[t, s * I:(s + 1) * I]
            if not 0 <= e < E:
                assert (hs == 0).all()
                continue
            gu, dn = dq[e]
            g = gu[:I] @ x[t].astype(np.float64)
            u = gu[I:] @ x[t].astype(np.float64)
            want = g / (1 + np.exp(-g)) * u
            assert np.abs(hs - want).max() <= 1e-5 * np.abs(want).max()
            if w[t, s] != 0:
                yw += w[t, s] * (dn @ hs.astype(np.float64))
        assert np.abs(y[t] - yw).max() <= 1e-5 * max(1e-30, np.abs(yw).max())


def _heat_sequence(seed, L, E):
    rng = np.random.default_rng(seed)
    seq = []
    for _ in range(30):
        l = int(rng.integers(0, L))
        n = int(rng.choice([1, 8, 40, 700]))
        seq.append((l, rng.integers(-1, E + 1, n).astype(np.int32)))
    return seq


@pytest.mark.parametrize("seed,L,E,moves", [(0, 3, 12, 5), (1, 3, 12, 5), (2, 3, 12, 5),
                                            (3, 6, 40, 32), (4, 2, 100, 64)])
def test_heat_oracle_and_library(seed, L, E, moves):
    """Python restatement == reference ExpertHeat (when built) == library,
    heats exactly and proposals exactly, on random credit sequences with
    over-cap calls and out-of-range ids (budgets below and above the
    candidate counts, many equal heats)."""
    cap = 64.0
    py = O.Heat(L, E, credit_cap=cap, moves=moves)
    p = _abi.HeatParams(0.95, 1.25, 1.5, cap, moves)
    lib_h = tiered.Heat(L, E, p)
    r = O.ref()
    rh = r.ref_heat_create(L, E, 0.95, 1.25, 1.5, cap, moves) if r is not None else None
    rng = np.random.default_rng(seed + 10)
    for l, ids in _heat_sequence(seed, L, E):
        py.credit(l, ids)
        lib_h.credit(l, ids)
        if rh:
            r.ref_heat_credit(rh, l, ids.ctypes.data, ids.size)
        for e in range(E):
            assert lib_h.heat(l, e) == py.h[l, e]
            if rh:
                assert r.ref_heat_get(rh, l, e) == py.h[l, e]
        res = (rng.random((L, E)) < 0.4).astype(np.uint8)
        mov = (rng.random((L, E)) < 0.9).astype(np.uint8)
        want = py.propose(res, mov)
        assert lib_h.propose(res, mov) == want
        if rh:
            out = np.zeros(4 * 64, np.int32)
            n = r.ref_heat_propose(rh, E, res.ctypes.data, mov.ctypes.data, out.ctypes.data, 64)
            assert [tuple(out[4 * i:4 * i + 4]) for i in range(n)] == want
    if rh:
        r.ref_heat_destroy(rh)


def test_heat_closed_form():
    py = O.Heat(1, 8)
    py.credit(0, [3, 3, 5])
    assert py.h[0, 3] == 2.0 and py.h[0, 5] == 1.0
    py.credit(0, [5])
    assert py.h[0, 3] == np.float32(2.0) * np.float32(0.95)
    assert py.h[0, 5] == np.float32(np.float32(0.95) + 1)
    # 1.9 >= 0 * 1.25 + 1.5: expert 3 promoted against the coldest resident (0)
    res = np.zeros((1, 8), np.uint8); res[0, 0] = res[0, 1] = 1
    assert py.propose(res) == [(0, 5, 0, 0), (0, 3, 0, 1)]
    # nothing hot enough: a resident at heat 1 needs 2.75
    py2 = O.Heat(1, 4)
    py2.credit(0, [0, 1, 1])
    r2 = np.array([[1, 0, 0, 0]], np.uint8)
    assert py2.propose(r2) == []
