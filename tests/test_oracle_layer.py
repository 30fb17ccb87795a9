"""Pins the oracle's router, dispatch, combine and expert products against
the reference's own CPU oracle (oracle/_ref), brute force and closed forms.
CPU only."""
import itertools
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from grimoire_amd import _abi, configs
from grimoire_amd import weights as weights_mod
from grimoire_amd.weights import MoeLayer, Weight, make_bf16, make_gptq_int4, make_int8, make_mxfp4
from tests.helpers import dequant, rel_l2


def _ties_logits(T, E, seed, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    l = torch.randn(T, E, generator=g) * scale
    # force exact ties, including ties that straddle the k-th place
    l[:, 5] = l[:, 3]
    l[:, E - 1] = l[:, 0]
    l[::2, 7] = l[::2, 2]
    return l.contiguous()


def _brute_topk(scores, K):
    # stable sort on -score: equal scores keep ascending index
    order = np.argsort(-scores, kind="stable")
    return order[:K]


@pytest.mark.parametrize("E,K", [(64, 4), (128, 8), (256, 8), (512, 10), (20, 16)])
def test_topk_softmax_brute_force_and_route_ref(E, K):
    l = _ties_logits(33, E, E + K)
    oe, ow = O.topk_softmax(l, K)
    for t in range(l.shape[0]):
        assert list(oe[t].numpy()) == list(_brute_topk(l[t].numpy(), K))
        assert abs(float(ow[t].double().sum()) - 1.0) < 1e-5
        assert all(ow[t, j] <= ow[t, j - 1] for j in range(1, K))
    # route_ref (src/moe_ref.cpp:30-63) ranks on probabilities: same picks
    # wherever no two probabilities collide, weights within 1e-6
    r = O.ref()
    for t in range(l.shape[0]):
        e_ref = torch.empty(K, dtype=torch.int32)
        w_ref = torch.empty(K, dtype=torch.float32)
        O.orc().orc_route_ref(O._p(l[t].contiguous()), E, K, 1, O._p(e_ref), O._p(w_ref))
        if r is not None:
            e2 = torch.empty(K, dtype=torch.int32)
            w2 = torch.empty(K, dtype=torch.float32)
            r.ref_route_ref(O._p(l[t].contiguous()), E, K, 1, O._p(e2), O._p(w2))
            assert torch.equal(e_ref, e2) and torch.equal(w_ref, w2)
        assert torch.equal(e_ref, oe[t])
        assert (w_ref - ow[t]).abs().max() < 1e-6


def test_topk_softmax_unnormalised_and_batched():
    l = _ties_logits(8, 64, 1)
    oe, ow = O.topk_softmax(l, 6, normalize=False)
    m = l.gather(1, oe.long()).max(dim=1, keepdim=True).values
    want = torch.exp((l.gather(1, oe.long()) - m).double()).float()
    assert (ow - want).abs().max() < 1e-6
    oe2, ow2 = O.topk_softmax(l, 6, normalize=False, batched=True)
    assert torch.equal(oe2, oe)
    assert torch.equal(ow2, l.gather(1, oe.long()))


def test_topk_sigmoid_brute_force():
    T, E, K = 17, 96, 8
    l = _ties_logits(T, E, 9, scale=3.0)
    g = torch.Generator().manual_seed(2)
    bias = (torch.randn(E, generator=g) * 0.1).bfloat16()
    oe, ow = O.topk_sigmoid(l, bias.view(torch.int16).contiguous(), K, normalize=True, scaling=2.5)
    s = torch.tensor([[O.orc().orc_sigmoid(float(v)) for v in row] for row in l])
    sel = s + bias.float()
    for t in range(T):
        assert list(oe[t].numpy()) == list(_brute_topk(sel[t].numpy(), K))
        w = s[t, oe[t].long()]
        want = w / w.sum() * 2.5
        assert (ow[t] - want).abs().max() < 1e-6
    # sigmoid closed form of the oracle's exp
    for v in [-5.0, 0.0, 0.3, 7.0]:
        assert abs(O.orc().orc_sigmoid(v) - 1 / (1 + math.exp(-v))) < 1e-7


def _group_brute(sel, sc, K, n_group, topk_group, scaling):
    E = sel.shape[0]
    gs = E // n_group
    gscore = []
    for gi in range(n_group):
        v = np.sort(sel[gi * gs:(gi + 1) * gs])[::-1]
        gscore.append(np.float32(v[0]) + np.float32(v[1]) if gs > 1 else v[0])
    gscore = np.array(gscore, dtype=np.float32)
    # every subset of topk_group groups: the kept set is the one whose
    # scores dominate (ties: lower group index), found by brute force
    best = None
    for sub in itertools.combinations(range(n_group), topk_group):
        key = sorted([(-gscore[g], g) for g in sub])
        if best is None or key < best[0]:
            best = (key, sub)
    kept = set(best[1])
    cand = np.array([sel[e] if e // gs in kept else -np.inf for e in range(E)], dtype=np.float32)
    picks = _brute_topk(cand, K)
    w = sc[picks].astype(np.float32)
    w = (w / np.float32(w.sum(dtype=np.float32))) * np.float32(scaling)
    return picks, w


@pytest.mark.parametrize("E,K,ng,kg", [(256, 8, 8, 4), (64, 6, 8, 3), (32, 4, 4, 2), (64, 4, 1, 1)])
def test_topk_group_brute_force(E, K, ng, kg):
    T = 12
    l = _ties_logits(T, E, E + ng, scale=1.5)
    g = torch.Generator().manual_seed(4)
    bias = torch.randn(E, generator=g) * 1e-3
    oe, ow = O.topk_group(l, bias.contiguous(), K, ng, kg, normalize=True, scaling=2.5)
    sc = np.array([[O.orc().orc_sigmoid(float(v)) for v in row] for row in l], dtype=np.float32)
    sel = (sc + bias.numpy()).astype(np.float32)
    for t in range(T):
        picks, w = _group_brute(sel[t], sc[t], K, ng, kg, 2.5)
        assert list(oe[t].numpy()) == list(picks), t
        assert np.abs(ow[t].numpy() - w).max() < 1e-6


def test_topk_group_reduces_to_plain_sigmoid():
    # one group kept out of one, or every group kept: plain sigmoid top-k
    T, E, K = 9, 64, 8
    l = _ties_logits(T, E, 11)
    bias = (torch.randn(E) * 0.01).bfloat16()
    e1, w1 = O.topk_sigmoid(l, bias.view(torch.int16).contiguous(), K, True, 1.0)
    e2, w2 = O.topk_group(l, bias.float().contiguous(), K, 8, 8, True, 1.0)
    e3, w3 = O.topk_group(l, bias.float().contiguous(), K, 1, 1, True, 1.0)
    assert torch.equal(e1, e2) and torch.equal(w1, w2)
    assert torch.equal(e1, e3) and torch.equal(w1, w3)


# ----------------------------------------------------------------- dispatch

def test_dispatch_invariants():
    T, K, E, mc = 300, 6, 40, 16
    g = torch.Generator().manual_seed(8)
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).int()
    ids[5, 2] = -1                      # a route not computed here
    tmax = E + T * K // mc + 1
    d = O.dispatch(ids, E, mc, tmax)
    flat = ids.flatten()
    valid = flat >= 0
    assert int(d["counts"].sum()) == int(valid.sum())
    assert torch.equal(d["counts"], torch.bincount(flat[valid].long(), minlength=E).int())
    assert torch.equal(d["offsets"], torch.cumsum(d["counts"], 0).int() - d["counts"])
    inv = d["inverse"]
    assert int(inv[5 * K + 2]) == -1
    p = inv[valid]
    assert torch.equal(torch.sort(p).values, torch.arange(int(valid.sum()), dtype=torch.int32))
    r = torch.arange(T * K)[valid]
    assert torch.equal(d["perm_token"][p.long()], (r // K).int())
    # stable: inside an expert, rows follow ascending route index
    for e in range(E):
        rows = r[flat[valid] == e]
        pos = inv[rows]
        assert torch.equal(pos, torch.arange(int(d["offsets"][e]), int(d["offsets"][e]) + len(rows),
                                             dtype=torch.int32))
    nt = d["n_tiles"]
    assert nt == int(((d["counts"] + mc - 1) // mc).sum())
    te, tm = d["tile_e"], d["tile_mb"]
    assert (te[nt:] == -1).all()
    for i in range(nt):
        assert 0 <= tm[i] * mc < d["counts"][te[i]]


def test_unpermute_closed_form():
    T, K, H = 5, 3, 16
    src = torch.randn(T * K, H)
    inv = torch.randperm(T * K).int()
    rw = torch.zeros(T * K)
    rw[::K] = 1.0                          # one-hot on slot 0
    out = O.unpermute(src, inv, rw, T, K, H)
    assert torch.equal(out, src[inv[::K].long()])
    inv2 = inv.clone()
    inv2[1::K] = -1
    rw2 = torch.rand(T * K)
    out2 = O.unpermute(src, inv2, rw2, T, K, H)
    want = sum(rw2[s::K, None] * torch.where(inv2[s::K, None] >= 0, src[inv2[s::K].clamp(min=0).long()], 0.0)
               for s in range(K))
    assert (out2 - want).abs().max() < 1e-6


def _bf16_bits(x):
    return x.bfloat16().view(torch.int16)


def test_rmsnorm_moe_residual_pinned():
    """launch_rmsnorm_moe_residual_batched (src/prefill.cpp:1004-1045) restated:
    h = 0 without shared reduces the residual update to the pinned unpermute
    bit for bit; all slots skipped leaves exactly h + shared; the normalised
    output matches an independent float64 RMSNorm; out_bf is bf16(out)."""
    g = torch.Generator().manual_seed(7)
    T, K, H, eps = 6, 4, 72, 1e-6
    routed = torch.randn(T * K, H, generator=g)
    rbits = _bf16_bits(routed)
    inv = torch.randperm(T * K, generator=g).int()
    inv[3::5] = -1
    rw = torch.rand(T * K, generator=g)
    w = torch.randn(H, generator=g) * 0.1
    wbits = _bf16_bits(w)
    zero = torch.zeros(T, H)
    hn, _, _ = O.rmsnorm_moe_residual(zero, rbits, inv, rw, None, wbits, 1.0, T, K, H, eps)
    assert torch.equal(hn, O.unpermute(rbits.view(torch.bfloat16).float(), inv, rw, T, K, H))

    h = torch.randn(T, H, generator=g) * 3
    sh = torch.randn(T, H, generator=g)
    hn, out, obf = O.rmsnorm_moe_residual(h, rbits, torch.full_like(inv, -1), rw, sh, wbits, 1.0,
                                          T, K, H, eps)
    assert torch.equal(hn, h + sh)

    for off in (1.0, 0.0):
        hn, out, obf = O.rmsnorm_moe_residual(h, rbits, inv, rw, sh, wbits, off, T, K, H, eps)
        r = rbits.view(torch.bfloat16).double()
        v = h.double() + sh.double()
        for s in range(K):
            p = inv[s::K].long()
            v = v + torch.where(p[:, None] >= 0, rw[s::K, None].double() * r[p.clamp(min=0)], 0.0)
        assert (hn.double() - v).abs().max() < 1e-5
        wd = off + wbits.view(torch.bfloat16).double()
        want = v / torch.sqrt((v * v).mean(1, keepdim=True) + eps) * wd
        assert (out.double() - want).abs().max() < 1e-5 * want.abs().max()
        assert torch.equal(obf, _bf16_bits(out))
    # unit weights, offset 1: every row has RMS sqrt(ms / (ms + eps))
    _, out, _ = O.rmsnorm_moe_residual(h, rbits, inv, rw, sh, _bf16_bits(torch.zeros(H)), 1.0,
                                       T, K, H, 0.0)
    assert (out.double().pow(2).mean(1).sqrt() - 1.0).abs().max() < 1e-6


def test_rmsnorm_residual_pinned():
    """launch_rmsnorm_residual_batched (src/prefill.cpp:627-700) restated: the
    residual is exactly (h + r0) + r1; the output is torch's rms_norm scaled by
    offset + bf16 weight; without addends h is left as it was."""
    g = torch.Generator().manual_seed(11)
    T, H, eps = 5, 96, 1e-5
    h = torch.randn(T, H, generator=g) * 2
    r0 = torch.randn(T, H, generator=g)
    r1 = torch.randn(T, H, generator=g)
    wbits = _bf16_bits(torch.randn(H, generator=g) * 0.1)
    hn, out, obf = O.rmsnorm_residual(h, r0, r1, wbits, 1.0, T, H, eps)
    assert torch.equal(hn, (h + r0) + r1)
    wf = 1.0 + wbits.view(torch.bfloat16).double()
    want = torch.nn.functional.rms_norm(hn.double(), (H,), eps=eps) * wf
    assert (out.double() - want).abs().max() < 1e-5 * want.abs().max()
    assert torch.equal(obf, _bf16_bits(out))
    hn2, out2, _ = O.rmsnorm_residual(h, None, None, wbits, 0.0, T, H, eps)
    assert torch.equal(hn2, h)
    want2 = torch.nn.functional.rms_norm(h.double(), (H,), eps=eps) * wbits.view(torch.bfloat16).double()
    assert (out2.double() - want2).abs().max() < 1e-5 * want2.abs().max()
    hn3, _, _ = O.rmsnorm_residual(h, None, r1, wbits, 1.0, T, H, eps)
    assert torch.equal(hn3, h + r1)


def test_small_launchers_pinned():
    """unpermute_range over the full route range is the pinned unpermute bit
    for bit, an empty range with accumulate leaves dst, and a range reads
    src rows shifted by p0 (brute force); permute_rows is torch's bf16."""
    g = torch.Generator().manual_seed(21)
    T, K, H = 4, 3, 8
    R = T * K
    src = torch.randn(R, H, generator=g)
    inv = torch.randperm(R, generator=g).int()
    inv[2] = -1
    rw = torch.rand(R, generator=g)
    full = O.unpermute_range(src, inv, rw, torch.zeros(T, H), T, K, H, 0, R, False)
    assert torch.equal(full, O.unpermute(src, inv, rw, T, K, H))
    d0 = torch.randn(T, H, generator=g)
    assert torch.equal(O.unpermute_range(src, inv, rw, d0, T, K, H, 5, 5, True), d0)
    part = O.unpermute_range(src[4:9], inv, rw, torch.zeros(T, H), T, K, H, 4, 9, False)
    for t in range(T):
        want = torch.zeros(H)
        for k in range(K):
            p = int(inv[t * K + k])
            if 4 <= p < 9:
                want = want + rw[t * K + k] * src[p]
        assert (part[t] - want).abs().max() < 1e-6
    perm = torch.tensor([3, 0, 0, 2], dtype=torch.int32)
    x = torch.randn(4, 6, generator=g)
    assert torch.equal(O.permute_rows_bf16(x, perm, 6), x[perm.long()].bfloat16().view(torch.int16))


# -------------------------------------------------------------- expert ffn

def _small_layer(fmt, E=8, H=256, I=128, K=3, shared=False, seed=0):
    cfg = configs.Config("t", 4, H, E, K, I, fmt, shared=shared, shared_gate=shared)
    return cfg, configs.make_layer(cfg, "cpu", seed)


def _route(T, E, K, seed):
    g = torch.Generator().manual_seed(seed)
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).int()
    w = torch.rand(T, K, generator=g) + 0.05
    return ids.contiguous(), (w / w.sum(1, keepdim=True)).contiguous()


@pytest.mark.parametrize("fmt", ["bf16", "int8", "mxfp4"])
def test_moe_forward_matches_reference_oracle(fmt):
    r = O.ref()
    if r is None:
        pytest.skip("oracle/_ref not built")
    cfg, L = _small_layer(fmt, shared=True)
    x = configs.make_x(cfg, "cpu", 1, T=4)
    ids, w = _route(4, cfg.E, cfg.K, 2)
    s = L.struct()
    y = O.moe_forward(s, ids, w, None, x)
    yr = torch.empty_like(y)
    r.ref_moe_forward(O.byref(s), O._p(ids), O._p(w), O._p(x), O._p(yr), 4)
    assert torch.equal(y, yr), rel_l2(y, yr)


def test_moe_forward_loose_per_expert():
    # tests/test_moe.cpp:54-196 idea: packed layout vs loose per-expert
    # tensors, including boundary experts 0 and E-1
    cfg, L = _small_layer("int4", E=6, H=256, I=128, K=2)
    x = configs.make_x(cfg, "cpu", 3, T=3)
    ids = torch.tensor([[0, 5], [5, 0], [2, 3]], dtype=torch.int32)
    w = torch.tensor([[0.5, 0.5], [0.7, 0.3], [0.1, 0.9]])
    y = O.moe_forward(L.struct(), ids, w, None, x)
    Wgu, Wdn = dequant(L.gate_up).double(), dequant(L.down).double()
    I, H = cfg.I, cfg.H
    for t in range(3):
        acc = torch.zeros(H, dtype=torch.float64)
        for j in range(2):
            e = int(ids[t, j])
            gate, up = Wgu[e * 2 * I:e * 2 * I + I], Wgu[e * 2 * I + I:(e + 1) * 2 * I]
            g, u = gate @ x[t].double(), up @ x[t].double()
            h = (g / (1 + torch.exp(-g))) * u
            acc += float(w[t, j]) * (Wdn[e * H:(e + 1) * H] @ h)
        assert rel_l2(y[t], acc) < 1e-6


def test_gate_up_down_compose_to_forward():
    cfg, L = _small_layer("mxfp4", shared=True)
    T = 3
    x = configs.make_x(cfg, "cpu", 4, T=T)
    ids, w = _route(T, cfg.E, cfg.K, 5)
    s = L.struct()
    KS = cfg.K + 1
    h = torch.empty(T, KS, cfg.I)
    gate = torch.empty(T)
    ws, wd = L.shared_gate_up.struct(), L.shared_down.struct()
    O.orc().orc_gate_up(O.byref(s), O.byref(ws), O._p(L.shared_gate_w), O._p(ids), O._p(x),
                        O._p(h), O._p(gate), T)
    y = torch.empty(T, cfg.H)
    O.orc().orc_down(O.byref(s), O.byref(wd), O._p(ids), O._p(w), O._p(gate), O._p(h), O._p(y), T)
    y2 = O.moe_forward(s, ids, w, gate, x)
    assert rel_l2(y, y2) < 1e-6
    gw = (L.shared_gate_w.to(torch.int32) << 16).view(torch.float32)
    want = torch.sigmoid((x.double() @ gw.double()))
    assert (gate.double() - want).abs().max() < 1e-6


def test_grouped_gemm_oracle_vs_dense():
    E, N, Kd = 3, 64, 128
    w = make_int8(E * N, Kd, seed=7)
    counts = torch.tensor([5, 0, 9], dtype=torch.int32)
    offsets = torch.tensor([0, 5, 5], dtype=torch.int32)
    A = torch.randn(14, Kd).bfloat16().float()
    out = torch.empty(14, N)
    O.orc().orc_grouped_gemm(O.byref(w.struct()), N, 0, O._p(A), O._p(out), O._p(offsets),
                             O._p(counts), E)
    W = dequant(w).double()
    want = torch.cat([A[0:5].double() @ W[0:N].T, A[5:14].double() @ W[2 * N:3 * N].T])
    assert rel_l2(out, want) < 1e-6
    out2 = torch.empty(14, N // 2)
    O.orc().orc_grouped_gemm(O.byref(w.struct()), N, 1, O._p(A), O._p(out2), O._p(offsets),
                             O._p(counts), E)
    g, u = want[:, : N // 2], want[:, N // 2:]
    assert rel_l2(out2, g / (1 + torch.exp(-g)) * u) < 1e-6


@pytest.mark.parametrize("K", [32, 224, 256, 2880, 3072, 7168])
def test_mxfp4_padded_k_matches_library(K):
    # the Python helper and the C entry agree on K' (K rounded up to 256)
    assert _abi.lib().grimoire_moe_mxfp4_padded_k(K) == weights_mod.mxfp4_padded_k(K)
    assert weights_mod.mxfp4_padded_k(K) % 256 == 0 and 0 <= weights_mod.mxfp4_padded_k(K) - K < 256


def test_mxfp4_padded_layer_same_outputs():
    # padded rows (zero codes under scale byte 127 past K) are exact zeros:
    # the oracle, reading rows through row_bytes / row_scales, gives the
    # unpadded layer's outputs bit for bit; the padding bytes are as stated
    cfg, L = _small_layer("mxfp4", E=6, H=352, I=160, K=2, shared=True, seed=4)
    P = L.pad_mxfp4()
    assert P.gate_up.row_bytes == 512 // 2 and P.gate_up.row_scales == 512 // 32
    assert P.down.row_bytes == 256 // 2 and P.down.row_scales == 256 // 32
    assert (P.gate_up.payload[:, 352 // 2:] == 0).all() and (P.gate_up.scales[:, 352 // 32:] == 127).all()
    assert torch.equal(P.gate_up.payload[:, :352 // 2], L.gate_up.payload)
    x = configs.make_x(cfg, "cpu", 5, T=5)
    ids, w = _route(5, cfg.E, cfg.K, 6)
    y = O.moe_forward(L.struct(), ids, w, None, x)
    yp = O.moe_forward(P.struct(), ids, w, None, x)
    assert torch.equal(y, yp)
