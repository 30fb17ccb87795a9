"""The host expert pool (include/b70/cpu_experts.hpp, src/cpu_experts.cpp;
the reference's tests/test_cpu_expert_pool.cpp and tools/test_cpu_ffn_rows.cpp
for the properties): NVFP4 dot products and expert FFNs on host threads
against float64 products of blocks dequantised by the reference's own
nvfp4_dequant_row (oracle/_ref, else the oracle pinned to it); outputs
independent of the thread count and of the instruction set; ffn_rows equal
to ffn row by row.  Host code only, no GPU."""
import hashlib

import numpy as np
import pytest
import torch

from grimoire_amd import _abi, tiered
from oracle import oracle as O
from tests.test_oracle_tiered import dequant, make_block


def _isas():
    out = []
    for isa in (0, 1, 2):
        if _abi.lib().grimoire_cpu_set_isa(isa) == 0:
            out.append(isa)
    _abi.lib().grimoire_cpu_set_isa(-1)
    return out


@pytest.fixture(autouse=True)
def _best_isa():
    yield
    _abi.lib().grimoire_cpu_set_isa(-1)


def _row(K, rng, scales=None):
    p = rng.integers(0, 256, K // 2, dtype=np.uint8)
    s = scales if scales is not None else (0x20 + rng.integers(0, 48, K // 16)).astype(np.uint8)
    s[::7] |= 0x80                                     # negative block scales
    s[3] = 0x02                                        # a subnormal one
    return p, s


def _deq_row(p, s, K):
    out = np.zeros(K, np.float32)
    r = O.ref()
    fn = r.ref_nvfp4_dequant_row if r is not None else O.orc().orc_nvfp4_dequant_row
    fn(p.ctypes.data, s.ctypes.data, 1.0, K, out.ctypes.data, 1)
    return out.astype(np.float64)


@pytest.mark.parametrize("K", [64, 128, 2048, 2560])
def test_dot_matches_float64_on_every_isa(K):
    rng = np.random.default_rng(K)
    p, s = _row(K, rng)
    x = rng.standard_normal(K).astype(np.float32)
    wq = _deq_row(p, s, K)
    want = float(wq @ x.astype(np.float64))
    bound = 2.0 ** -21 * float(np.abs(wq * x).sum())
    got = {}
    for isa in _isas():
        tiered.cpu_set_isa(isa)
        got[isa] = tiered.cpu_nvfp4_dot(torch.from_numpy(p), torch.from_numpy(s), torch.from_numpy(x))
        assert abs(got[isa] - want) <= bound, (isa, got[isa], want)
    vals = list(got.values())
    assert all(np.float32(v).tobytes() == np.float32(vals[0]).tobytes() for v in vals), got


def test_dot_closed_forms():
    K = 256
    x = torch.arange(K, dtype=torch.float32) - 100.0
    # every code 2 (e2m1 1.0, both nibbles), every scale 0x38 (1.0): sum(x)
    p = torch.full((K // 2,), 0x22, dtype=torch.uint8)
    s = torch.full((K // 16,), 0x38, dtype=torch.uint8)
    assert tiered.cpu_nvfp4_dot(p, s, x) == float(x.sum())
    # low nibbles 7 (6.0) on even elements, high 0: 6 * sum(x[0::2]) * 2 (scale 0x40)
    p = torch.full((K // 2,), 0x07, dtype=torch.uint8)
    s = torch.full((K // 16,), 0x40, dtype=torch.uint8)
    assert tiered.cpu_nvfp4_dot(p, s, x) == 12.0 * float(x[0::2].sum())
    # one NaN scale poisons the row; K % 64 != 0 is refused (NaN)
    s[5] = 0x7F
    assert np.isnan(tiered.cpu_nvfp4_dot(p, s, x))
    assert np.isnan(_abi.lib().grimoire_cpu_nvfp4_dot(p.data_ptr(), s.data_ptr(), x.data_ptr(), 96))


def _blocks(lay, n, seed):
    rng = np.random.default_rng(seed)
    return [torch.from_numpy(make_block(lay, rng)) for _ in range(n)]


def _ffn64(dq, w, x):
    y = np.zeros(dq[0][1].shape[0])
    I = dq[0][1].shape[1]
    for (gu, dn), wj in zip(dq, w):
        g = gu[:I] @ x
        u = gu[I:] @ x
        y += float(wj) * (dn @ (g / (1 + np.exp(-g)) * u))
    return y


@pytest.mark.parametrize("H,I,n", [(256, 128, 3), (256, 128, 1), (512, 256, 8)])
def test_ffn_matches_float64(H, I, n):
    L = tiered.layout(H, I)
    lay = O.tmoe_layout(H, I)
    blocks = _blocks(lay, n, H + n)
    rng = np.random.default_rng(7)
    w = torch.from_numpy(rng.uniform(0.05, 0.9, n).astype(np.float32))
    x = torch.from_numpy((rng.standard_normal(H) * 0.05).astype(np.float32))
    y = torch.full((H,), float("nan"))
    cx = tiered.CpuExperts(4)
    cx.ffn(L, blocks, w, x, y)
    want = _ffn64([dequant(b.numpy(), lay, H, I) for b in blocks], w.numpy(), x.numpy().astype(np.float64))
    assert np.abs(y.numpy() - want).max() <= 1e-5 * np.abs(want).max()


def test_ffn_no_experts_gives_zeros():
    L = tiered.layout(256, 128)
    y = torch.full((256,), 5.0)
    tiered.CpuExperts(2).ffn(L, [], torch.zeros(1), torch.zeros(256), y)
    assert (y == 0).all()


def _hash(t):
    return hashlib.sha1(t.numpy().tobytes()).hexdigest()


def test_thread_count_and_isa_do_not_change_bits():
    """tests/test_cpu_expert_pool.cpp: the same output bits for 1, 2, 6 and
    14 threads over many calls (a race or an order that depends on the
    split shows as a different hash)."""
    H, I, POOL = 256, 128, 12
    L = tiered.layout(H, I)
    blocks = _blocks(O.tmoe_layout(H, I), POOL, 5)
    rng = np.random.default_rng(9)
    x = torch.from_numpy((rng.standard_normal(H) * 0.05).astype(np.float32))
    w = torch.tensor([0.1, 0.2, 0.3])
    picks = rng.integers(0, POOL, (300, 3))
    y = torch.empty(H)
    hashes = {}
    for isa in _isas():
        tiered.cpu_set_isa(isa)
        for threads in (1, 2, 6, 14):
            cx = tiered.CpuExperts(threads)
            h = hashlib.sha1()
            for row in picks:
                cx.ffn(L, [blocks[int(e)] for e in row], w, x, y)
                h.update(y.numpy().tobytes())
            hashes[(isa, threads)] = h.hexdigest()
            del cx
    assert len(set(hashes.values())) == 1, hashes


def test_ffn_rows_equals_ffn_row_by_row():
    """tools/test_cpu_ffn_rows.cpp: rows sharing experts, a row with none,
    one row, no experts at all, 16 rows of 0-10 of 24 experts; each row
    bit-identical to ffn on it."""
    H, I, E = 512, 256, 24
    L = tiered.layout(H, I)
    blocks = _blocks(O.tmoe_layout(H, I), E, 11)
    rng = np.random.default_rng(1234)
    cases = [[[0, 1, 2, 3], [0, 1, 4, 5], [6, 0, 7], [1, 8]],
             [[3, 9], [], [9, 10, 3], [11]],
             [[5, 6, 7, 8, 9]],
             [[], [], [], []],
             [list(rng.choice(E, int(rng.integers(0, 11)), replace=False)) for _ in range(16)]]
    cx = tiered.CpuExperts(6)
    for routes in cases:
        R = len(routes)
        x = torch.from_numpy(rng.standard_normal((R, H)).astype(np.float32))
        sel, w, off = [], [], [0]
        for r in routes:
            for e in r:
                sel.append(blocks[int(e)])
                w.append(0.05 + 0.1 * float(rng.integers(0, 9)))
            off.append(len(sel))
        wt = torch.tensor(w if w else [0.0], dtype=torch.float32)
        offt = torch.tensor(off, dtype=torch.int32)
        y = torch.full((R, H), -2.0)
        cx.ffn_rows(L, sel, wt, offt, x, y)
        for r in range(R):
            yr = torch.full((H,), -1.0)
            o0, o1 = off[r], off[r + 1]
            cx.ffn(L, sel[o0:o1], wt[o0:o1].contiguous() if o1 > o0 else torch.zeros(1), x[r].contiguous(), yr)
            assert torch.equal(y[r], yr), (routes, r)


def test_errors():
    lib = _abi.lib()
    cx = tiered.CpuExperts(2)
    bad = _abi.NvExpertLayout()
    bad.H, bad.I = 200, 128
    import ctypes as C
    x = torch.zeros(256)
    y = torch.zeros(256)
    assert lib.grimoire_cpu_experts_ffn(cx._h, C.byref(bad), None, None, 0, x.data_ptr(),
                                        y.data_ptr()) == _abi.ERR_SHAPE
    L = tiered.layout(256, 128)
    assert lib.grimoire_cpu_experts_ffn(cx._h, C.byref(L), None, None, 2, x.data_ptr(),
                                        y.data_ptr()) == _abi.ERR_ARG
    off = torch.tensor([1, 1], dtype=torch.int32)
    assert lib.grimoire_cpu_experts_ffn_rows(cx._h, C.byref(L), 1, None, None, off.data_ptr(),
                                             x.data_ptr(), y.data_ptr()) == _abi.ERR_ARG
    assert lib.grimoire_cpu_set_isa(7) == _abi.ERR_ARG


def test_pool_cpus_partition():
    import os
    allowed = sorted(os.sched_getaffinity(0))
    for ranks in (1, 2, 3):
        parts = [tiered.cpu_pool_cpus(ranks, r) for r in range(ranks)]
        assert sorted(c for p in parts for c in p) == allowed
        assert all(len(p) in (len(allowed) // ranks, len(allowed) // ranks + 1) for p in parts)
    cx = tiered.CpuExperts(3, cpus=[-1] + tiered.cpu_pool_cpus(1, 0)[:2])
    assert cx.threads == 3


def test_pool_wakes_after_idle():
    """Idle pool threads go to sleep on the bell; calls spaced out past the
    spin phase must still complete with the same bits as back-to-back ones."""
    import time
    H, I = 256, 128
    L = tiered.layout(H, I)
    blocks = _blocks(O.tmoe_layout(H, I), 4, 21)
    rng = np.random.default_rng(3)
    x = torch.from_numpy((rng.standard_normal(H) * 0.05).astype(np.float32))
    w = torch.tensor([0.4, 0.3, 0.2, 0.1])
    cx = tiered.CpuExperts(5)
    want = torch.empty(H)
    cx.ffn(L, blocks, w, x, want)
    for _ in range(6):
        time.sleep(0.05)
        y = torch.full((H,), float("nan"))
        cx.ffn(L, blocks, w, x, y)
        assert torch.equal(y, want)
