"""Pins the CPU oracle (oracle/moe_oracle.c) before it is trusted as the
checker: golden vectors of the reference's own tests, the reference's own
CPU code (oracle/_ref, built from its sources), closed forms and brute
force.  CPU only."""
import ctypes as C
import itertools
import json
import math
import struct
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle as O
from grimoire_amd import _abi
from grimoire_amd.weights import Weight, make_bf16, make_gptq_int4, make_int8, make_mxfp4
from tests.helpers import dequant, rel_l2

GOLD = Path(__file__).resolve().parent / "golden"


def orc():
    return O.orc()


def ref_or_skip():
    r = O.ref()
    if r is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    return r


# ------------------------------------------------------------ scalar decodes

def test_f16_exhaustive_closed_form():
    # tests/test_gptq.cpp section 1: every binary16 code against its formula
    for h in range(65536):
        got = orc().orc_f16_to_f32(h)
        e, m = (h >> 10) & 0x1F, h & 0x3FF
        sign = -1.0 if h & 0x8000 else 1.0
        if e == 0x1F:
            assert (math.isnan(got) if m else got == sign * math.inf), hex(h)
            continue
        want = sign * (m / 1024.0) * 2.0 ** -14 if e == 0 else sign * (1 + m / 1024.0) * 2.0 ** (e - 15)
        assert got == np.float32(want), hex(h)


def test_bf16_roundtrip_and_rne():
    for v in [1.0, -2.5, 3.0e38, 1e-40, 0.0, -0.0]:
        b = orc().orc_f32_to_bf16(v)
        assert orc().orc_bf16_to_f32(b) == np.float32(torch.tensor(v).bfloat16().float().item())
    # ties to even: 1 + 2^-8 is halfway between 1 and 1 + 2^-7
    assert orc().orc_bf16_to_f32(orc().orc_f32_to_bf16(1.0 + 2.0 ** -8)) == 1.0
    assert orc().orc_bf16_to_f32(orc().orc_f32_to_bf16(1.0 + 3 * 2.0 ** -8)) == 1.0 + 2.0 ** -6
    assert math.isnan(orc().orc_bf16_to_f32(orc().orc_f32_to_bf16(float("nan"))))


def test_e8m0_table():
    # tests/test_formats.cpp:45-60
    f = orc().orc_e8m0_to_f32
    assert f(127) == 1.0 and f(128) == 2.0 and f(126) == 0.5
    assert f(254) == 2.0 ** 127 and f(1) == 2.0 ** -126 and f(0) == 2.0 ** -127
    assert math.isnan(f(255))
    for x in range(1, 255):
        assert f(x) == 2.0 ** (x - 127)


def test_e2m1_table():
    # tests/test_formats.cpp:62-70
    mags = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    for i, m in enumerate(mags):
        assert orc().orc_e2m1_to_f32(i) == m
        assert orc().orc_e2m1_to_f32(i | 8) == -m


def _read_ggld(name):
    d = (GOLD / name).read_bytes()
    assert d[:4] == b"GGLD"
    typ, n, nb = struct.unpack("<III", d[4:16])
    raw = np.frombuffer(d[16:16 + nb], dtype=np.uint8)
    want = np.frombuffer(d[16 + nb:], dtype=np.float32)
    return typ, n, raw, want


def test_mxfp4_golden_file():
    # reference tests/gguf/data/MXFP4.bin: ggml block = e8m0 + 16 bytes,
    # low nibble element i, high nibble element i + 16
    typ, n, raw, want = _read_ggld("MXFP4.bin")
    assert typ == 39 and n == 256
    got = []
    for b in range(n // 32):
        blk = raw[b * 17:(b + 1) * 17]
        s = orc().orc_e8m0_to_f32(int(blk[0]))
        q = blk[1:]
        vals = [orc().orc_e2m1_to_f32(int(q[i] & 0xF)) * s for i in range(16)] + \
               [orc().orc_e2m1_to_f32(int(q[i] >> 4)) * s for i in range(16)]
        got += vals
    assert np.array_equal(np.array(got, dtype=np.float32), want)


def test_q8_0_golden_file_pins_f16_and_int8():
    typ, n, raw, want = _read_ggld("Q8_0.bin")
    assert typ == 8
    got = []
    for b in range(n // 32):
        blk = raw[b * 34:(b + 1) * 34]
        d = orc().orc_f16_to_f32(int(blk[0]) | (int(blk[1]) << 8))
        got += [np.float32(d) * np.float32(np.int8(v)) for v in blk[2:]]
    assert np.array_equal(np.array(got, dtype=np.float32), want)


def test_expf_against_libm():
    xs = np.concatenate([np.linspace(-103.0, 88.7, 200001, dtype=np.float32),
                         np.array([0.0, -0.0, 1e-30, -1e-30, 88.72, -87.3], dtype=np.float32)])
    got = np.array([orc().orc_expf(float(x)) for x in xs[::7]], dtype=np.float32)
    want = np.exp(xs[::7].astype(np.float64)).astype(np.float32)
    normal = want > 1.2e-38
    ulp = np.abs(got[normal].view(np.int32).astype(np.int64) - want[normal].view(np.int32))
    assert ulp.max() <= 2, ulp.max()
    assert orc().orc_expf(0.0) == 1.0
    assert orc().orc_expf(100.0) == math.inf and orc().orc_expf(-200.0) == 0.0


# ------------------------------------------------------------------- GPTQ

def _lcg_tensors(out, inn, group, seed):
    x = seed
    def nxt():
        nonlocal x
        x = (x * 1664525 + 1013904223) & 0xFFFFFFFF
        return x
    qw = np.array([nxt() for _ in range((inn // 8) * out)], dtype=np.uint32).view(np.int32)
    qz = np.array([nxt() for _ in range((inn // group) * (out // 8))], dtype=np.uint32).view(np.int32)
    sc = np.array([0x2C00 | ((nxt() >> 16) & 0x3FF) for _ in range((inn // group) * out)],
                  dtype=np.uint16)
    return qw, qz, sc


def test_gptq_golden_probes():
    g = json.loads((GOLD / "gptq_probes.json").read_text())
    qw, qz, sc = _lcg_tensors(g["out"], g["in"], g["group"], 12345)
    for o, k, w in zip(g["o"], g["k"], g["w"]):
        got = orc().orc_gptq_at(qw.ctypes.data, qz.ctypes.data, sc.ctypes.data, g["in"], g["out"],
                                g["group"], o, k)
        assert abs(got - w) <= 1e-6 * (1 + abs(w)), (o, k, got, w)
        r = O.ref()
        if r is not None:
            assert got == r.ref_gptq_at(qw.ctypes.data, qz.ctypes.data, sc.ctypes.data, g["in"],
                                        g["out"], g["group"], o, k)


def _gptq_to_int4_f16(qw, qz, sc, out, inn, group):
    """Repack GPTQ (qweight [in/8][out], qzeros [in/g][out/8], fp16 scales)
    into INT4_F16 rows, keeping the fp16 scales and zero+1 exactly."""
    k = np.arange(inn)
    w = qw.view(np.uint32).reshape(inn // 8, out)
    nib = (w[k >> 3, :] >> ((k & 7) * 4)[:, None]) & 0xF          # [in][out]
    nib = nib.T.astype(np.uint8)                                   # [out][in]
    payload = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    z = qz.view(np.uint32).reshape(inn // group, out // 8)
    o = np.arange(out)
    znib = ((z[:, o >> 3] >> ((o & 7) * 4)) & 0xF).T.astype(np.uint8) + 1   # [out][ngrp]
    scales = sc.reshape(inn // group, out).T.copy()
    return (torch.from_numpy(payload.copy()), torch.from_numpy(scales.view(np.int16).copy()),
            torch.from_numpy(znib.copy()))


def test_int4_f16_matches_gptq_exactly():
    out, inn, group = 64, 512, 128
    qw, qz, sc = _lcg_tensors(out, inn, group, 777)
    pay, scl, zer = _gptq_to_int4_f16(qw, qz, sc, out, inn, group)
    w = Weight(_abi.FMT_INT4_F16, out, inn, pay, scl, zer, inn // group)
    s = w.struct()
    for o in range(out):
        for k in range(0, inn, 7):
            a = orc().orc_qw_at(O.byref(s), o, k)
            b = orc().orc_gptq_at(qw.ctypes.data, qz.ctypes.data, sc.ctypes.data, inn, out, group, o, k)
            assert a == b, (o, k)
    # dense dequant used by the GPU tests agrees too
    d = dequant(w)
    for o in range(0, out, 5):
        for k in range(0, inn, 11):
            assert d[o, k].item() == orc().orc_qw_at(O.byref(s), o, k)


@pytest.mark.parametrize("fmt", ["int4_bf16", "int4_s4", "int4_nozero", "int8", "mxfp4", "bf16"])
def test_qw_at_matches_reference(fmt):
    r = ref_or_skip()
    N, K = 24, 256
    if fmt.startswith("int4"):
        g = torch.Generator().manual_seed(3)
        pay = torch.randint(0, 256, (N, K // 2), dtype=torch.uint8, generator=g)
        sc = (torch.randn(N, K // 128, generator=g) * 0.02).bfloat16().view(torch.int16)
        z = None
        if fmt == "int4_bf16":
            z = torch.randint(0, 16, (N, K // 128), dtype=torch.uint8, generator=g)
        elif fmt == "int4_s4":
            z = torch.full((N, K // 128), 0xFF, dtype=torch.uint8)
        w = Weight(_abi.FMT_INT4, N, K, pay, sc, z, K // 128)
    else:
        w = {"int8": make_int8, "mxfp4": make_mxfp4, "bf16": make_bf16}[fmt](N, K, seed=5)
    s = w.struct()
    d = dequant(w)
    for n in range(N):
        for k in range(K):
            a = orc().orc_qw_at(O.byref(s), n, k)
            b = r.ref_qw_at(O.byref(s), n, k)
            assert a == b or (math.isnan(a) and math.isnan(b)), (fmt, n, k, a, b)
            assert d[n, k].item() == a


# ------------------------------------------------------ expert ingestion

def test_gptq_repack_pinned():
    """orc_gptq_repack (src/gptq.cpp:56-83) on the golden LCG tensor: byte for
    byte the reference's own gptq_repack_int4 (when oracle/_ref is built); with
    the fp16 scales kept, every golden probe and every sampled element equals
    gptq_at through the INT4_F16 element decode; with bf16 scales, within the
    bf16 rounding of the scale."""
    g = json.loads((GOLD / "gptq_probes.json").read_text())
    out, inn, group = g["out"], g["in"], g["group"]
    qw, qz, sc = _lcg_tensors(out, inn, group, 12345)
    pay, scb, z = O.gptq_repack(qw, qz, sc, inn, out, group)
    r = O.ref()
    if r is not None:
        rp = np.zeros_like(pay); rs = np.zeros(scb.shape, np.uint16); rz = np.zeros_like(z)
        assert r.ref_gptq_repack_int4(qw.ctypes.data, qz.ctypes.data, sc.ctypes.data, inn, out,
                                      group, rp.ctypes.data, rs.ctypes.data, rz.ctypes.data) == 1
        assert np.array_equal(pay, rp) and np.array_equal(scb.view(np.uint16), rs)
        assert np.array_equal(z, rz)
    pay16, sc16, z16 = O.gptq_repack(qw, qz, sc, inn, out, group, keep_f16=True)
    assert np.array_equal(pay16, pay) and np.array_equal(z16, z)
    w16 = Weight(_abi.FMT_INT4_F16, out, inn, torch.from_numpy(pay16), torch.from_numpy(sc16),
                 torch.from_numpy(z16), inn // group)
    wb = Weight(_abi.FMT_INT4, out, inn, torch.from_numpy(pay), torch.from_numpy(scb),
                torch.from_numpy(z), inn // group)
    s16, sb = w16.struct(), wb.struct()
    for o, k, want in zip(g["o"], g["k"], g["w"]):
        assert abs(orc().orc_qw_at(O.byref(s16), o, k) - want) <= 1e-6 * (1 + abs(want))
    for o in range(0, out, 37):
        for k in range(0, inn, 29):
            ref_v = orc().orc_gptq_at(qw.ctypes.data, qz.ctypes.data, sc.ctypes.data, inn, out,
                                      group, o, k)
            assert orc().orc_qw_at(O.byref(s16), o, k) == ref_v
            assert abs(orc().orc_qw_at(O.byref(sb), o, k) - ref_v) <= abs(ref_v) * 2.0 ** -8


def test_int4_zero_unpack_brute_force():
    rng = np.random.default_rng(4)
    out, groups = 24, 5
    zp = rng.integers(0, 2 ** 32, (out // 8, groups), dtype=np.uint64).astype(np.uint32)
    got = O.int4_zero_unpack(zp.view(np.int32), out, groups)
    for n in range(out):
        for gi in range(groups):
            assert got[n, gi] == (int(zp[n // 8, gi]) >> (4 * (n % 8))) & 0xF
    assert (O.int4_zero_unpack(None, out, groups) == 8).all()


def test_int4_to_signed_keeps_values():
    """src/grimoire.cpp:8386-8397: with every zero point 8 the conversion must
    not change a single dequantised element; one zero point off 8 and nothing
    changes at all."""
    rng = np.random.default_rng(5)
    N, K, G = 16, 256, 128
    gu = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    dn = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    sc = torch.from_numpy((rng.standard_normal((N, K // G)) * 0.02).astype(np.float32)).bfloat16()
    gz = np.full((N, K // G), 8, np.uint8)
    dz = np.full((N, K // G), 8, np.uint8)

    def vals(p, z):
        w = Weight(_abi.FMT_INT4, N, K, torch.from_numpy(p), sc.view(torch.int16),
                   torch.from_numpy(z), K // G)
        s = w.struct()
        return [orc().orc_qw_at(O.byref(s), n, k) for n in range(N) for k in range(0, K, 3)]

    before = vals(gu, gz), vals(dn, dz)
    gu2, gz2, dn2, dz2 = gu.copy(), gz.copy(), dn.copy(), dz.copy()
    assert O.int4_to_signed(gu2, gz2, dn2, dz2) == 1
    assert (gz2 == 0xFF).all() and (dz2 == 0xFF).all() and np.array_equal(gu2, gu ^ 0x88)
    assert (vals(gu2, gz2), vals(dn2, dz2)) == before
    dz3 = dz.copy(); dz3[3, 1] = 7
    gu3, gz3, dn3 = gu.copy(), gz.copy(), dn.copy()
    assert O.int4_to_signed(gu3, gz3, dn3, dz3) == 0
    assert np.array_equal(gu3, gu) and np.array_equal(gz3, gz) and np.array_equal(dn3, dn)
