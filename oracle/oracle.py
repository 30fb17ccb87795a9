"""ctypes binding of the CPU oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
this module.  It wraps
  oracle/_build/libmoe_oracle.so  -- this repo's C restatement (moe_oracle.c)
  oracle/_ref/libmoe_ref.so       -- the reference's own src/moe_ref.cpp and
                                     src/gptq.cpp (built only where the
                                     reference tree exists)
Arguments are CPU torch tensors (or numpy arrays) and the ctypes structs of
include/grimoire_moe.h.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "_build" / "libmoe_oracle.so"
REF_SO = HERE / "_ref" / "libmoe_ref.so"

P = C.c_void_p
I32 = C.c_int
F32 = C.c_float

_orc = None
_ref = None


def build(ref: bool = True) -> None:
    """Compile the oracle (and oracle/_ref when the reference is present)."""
    target = "all" if ref else str(ORACLE_SO)
    subprocess.run(["make", "-s", "-C", str(HERE), target], check=True)


def _p(t):
    if t is None:
        return None
    if isinstance(t, np.ndarray):
        assert t.flags["C_CONTIGUOUS"]
        return t.ctypes.data
    # callers must keep `t` referenced until the C call returns
    assert not t.is_cuda and t.is_contiguous()
    return t.data_ptr()


def orc() -> C.CDLL:
    global _orc
    if _orc is None:
        if not ORACLE_SO.exists():
            build(ref=False)
        l = C.CDLL(str(ORACLE_SO))
        sig = {
            "orc_f16_to_f32": (F32, [C.c_uint16]),
            "orc_bf16_to_f32": (F32, [C.c_uint16]),
            "orc_f32_to_bf16": (C.c_uint16, [F32]),
            "orc_e8m0_to_f32": (F32, [C.c_uint8]),
            "orc_e2m1_to_f32": (F32, [C.c_uint8]),
            "orc_expf": (F32, [F32]),
            "orc_sigmoid": (F32, [F32]),
            "orc_qw_at": (F32, [P, I32, I32]),
            "orc_gptq_at": (F32, [P, P, P, I32, I32, I32, I32, I32]),
            "orc_route_ref": (None, [P, I32, I32, I32, P, P]),
            "orc_topk_softmax": (None, [P, I32, I32, I32, I32, I32, P, P]),
            "orc_topk_sigmoid": (None, [P, P, I32, I32, I32, I32, F32, P, P]),
            "orc_topk_group": (None, [P, P, I32, I32, I32, I32, I32, I32, F32, P, P]),
            "orc_router_logits": (None, [P, P, P, I32, I32, I32]),
            "orc_gate_up": (None, [P, P, P, P, P, P, P, I32]),
            "orc_down": (None, [P, P, P, P, P, P, P, I32]),
            "orc_moe_forward": (None, [P, P, P, P, P, P, I32]),
            "orc_dispatch": (I32, [P, I32, I32, I32, I32, P, P, P, P, P, P, I32]),
            "orc_unpermute": (None, [P, P, P, P, I32, I32, I32]),
            "orc_e4m3_to_f32": (F32, [C.c_uint8]),
            "orc_nvfp4_dequant_row": (None, [P, P, F32, I32, P, I32]),
            "orc_tmoe_layout": (None, [I32, I32, P]),
            "orc_tmoe_gate_up": (None, [P, I32, I32, I32, I32, P, P, P, I32]),
            "orc_tmoe_down": (None, [P, I32, I32, I32, I32, P, P, P, P, I32]),
            "orc_gptq_repack": (None, [P, P, P, I32, I32, I32, I32, P, P, P]),
            "orc_int4_zero_unpack": (None, [P, I32, I32, P]),
            "orc_int4_to_signed": (I32, [P, C.c_int64, P, C.c_int64, P, C.c_int64, P, C.c_int64]),
            "orc_rmsnorm_residual": (None, [P, P, P, P, F32, P, P, I32, I32, F32]),
            "orc_rmsnorm_moe_residual": (None, [P, P, P, P, P, P, F32, P, P, I32, I32, I32,
                                                F32]),
            "orc_grouped_gemm": (None, [P, I32, I32, P, P, P, P, I32]),
        }
        for n, (r, a) in sig.items():
            f = getattr(l, n)
            f.restype = r
            f.argtypes = a
        _orc = l
    return _orc


def ref():
    """The reference's own CPU oracle, or None when it was not built."""
    global _ref
    if _ref is None:
        if not REF_SO.exists():
            return None
        l = C.CDLL(str(REF_SO))
        sig = {
            "ref_qw_at": (F32, [P, I32, I32]),
            "ref_gptq_at": (F32, [P, P, P, I32, I32, I32, I32, I32]),
            "ref_gptq_repack_int4": (I32, [P, P, P, I32, I32, I32, P, P, P]),
            "ref_e4m3_to_f32": (F32, [C.c_uint8]),
            "ref_nvfp4_dequant_row": (None, [P, P, F32, I32, P, I32]),
            "ref_heat_create": (P, [I32, I32, F32, F32, F32, F32, I32]),
            "ref_heat_destroy": (None, [P]),
            "ref_heat_credit": (None, [P, I32, P, C.c_size_t]),
            "ref_heat_get": (F32, [P, I32, I32]),
            "ref_heat_propose": (I32, [P, I32, P, P, P, I32]),
            "ref_route_ref": (None, [P, I32, I32, I32, P, P]),
            "ref_moe_forward": (None, [P, P, P, P, P, I32]),
        }
        for n, (r, a) in sig.items():
            f = getattr(l, n)
            f.restype = r
            f.argtypes = a
        _ref = l
    return _ref


def byref(s):
    return C.cast(C.pointer(s), P)


# ------------------------------------------------------------ conveniences

def topk_softmax(logits: torch.Tensor, K: int, normalize=True, batched=False):
    T, E = logits.shape
    oe = torch.empty((T, K), dtype=torch.int32)
    ow = torch.empty((T, K), dtype=torch.float32)
    lc = logits.contiguous()
    orc().orc_topk_softmax(_p(lc), T, E, K, int(normalize), int(batched), _p(oe), _p(ow))
    return oe, ow


def topk_sigmoid(logits, bias_bf16, K, normalize=True, scaling=1.0):
    T, E = logits.shape
    oe = torch.empty((T, K), dtype=torch.int32)
    ow = torch.empty((T, K), dtype=torch.float32)
    lc = logits.contiguous()
    orc().orc_topk_sigmoid(_p(lc), _p(bias_bf16), T, E, K, int(normalize),
                           float(scaling), _p(oe), _p(ow))
    return oe, ow


def topk_group(logits, bias, K, n_group, topk_group, normalize=True, scaling=1.0):
    T, E = logits.shape
    oe = torch.empty((T, K), dtype=torch.int32)
    ow = torch.empty((T, K), dtype=torch.float32)
    lc = logits.contiguous()
    orc().orc_topk_group(_p(lc), _p(bias), T, E, K, n_group, topk_group,
                         int(normalize), float(scaling), _p(oe), _p(ow))
    return oe, ow


def router_logits(router, x):
    T, H = x.shape
    E = router.shape[0]
    out = torch.empty((T, E), dtype=torch.float32)
    rc, xc = router.contiguous(), x.contiguous()
    orc().orc_router_logits(_p(rc), _p(xc), _p(out), T, E, H)
    return out


def dispatch(ids: torch.Tensor, E: int, mc: int, tmax: int):
    T, K = ids.shape
    R = T * K
    counts = torch.empty(E, dtype=torch.int32)
    offsets = torch.empty(E, dtype=torch.int32)
    inverse = torch.empty(R, dtype=torch.int32)
    perm = torch.full((R,), -1, dtype=torch.int32)
    te = torch.empty(max(tmax, 1), dtype=torch.int32)
    tm = torch.empty(max(tmax, 1), dtype=torch.int32)
    ic = ids.contiguous()
    nt = orc().orc_dispatch(_p(ic), T, K, E, mc, _p(counts), _p(offsets),
                            _p(inverse), _p(perm), _p(te), _p(tm), tmax)
    return dict(counts=counts, offsets=offsets, inverse=inverse, perm_token=perm,
                tile_e=te[:tmax], tile_mb=tm[:tmax], n_tiles=nt)


def moe_forward(layer_struct, rex, rwt, gate, x):
    T, H = x.shape
    y = torch.empty((T, H), dtype=torch.float32)
    # keep every contiguous copy alive for the duration of the call
    rc, wc, xc = rex.contiguous(), rwt.contiguous(), x.contiguous()
    gc = None if gate is None else gate.contiguous()
    orc().orc_moe_forward(byref(layer_struct), _p(rc), _p(wc), _p(gc), _p(xc), _p(y), T)
    return y


def unpermute(src, inverse, rw, T, K, H):
    dst = torch.empty((T, H), dtype=torch.float32)
    sc, ic, wc = src.contiguous(), inverse.contiguous(), rw.contiguous()
    orc().orc_unpermute(_p(sc), _p(ic), _p(wc), _p(dst), T, K, H)
    return dst


def rmsnorm_moe_residual(h, routed, inverse, rw, shared, weight, weight_offset, T, K, H, eps):
    """Returns (h_new, out fp32, out_bf as int16 bits); h is not modified."""
    hn = h.contiguous().clone()
    out = torch.empty((T, H), dtype=torch.float32)
    obf = torch.empty((T, H), dtype=torch.int16)
    rc, ic, wc, wt = routed.contiguous(), inverse.contiguous(), rw.contiguous(), weight.contiguous()
    sc = None if shared is None else shared.contiguous()
    orc().orc_rmsnorm_moe_residual(_p(hn), _p(rc), _p(ic), _p(wc), _p(sc), _p(wt),
                                   float(weight_offset), _p(out), _p(obf), T, K, H, float(eps))
    return hn, out, obf


def rmsnorm_residual(h, r0, r1, weight, weight_offset, T, H, eps):
    """Returns (h_new, out fp32, out_bf as int16 bits); h is not modified."""
    hn = h.contiguous().clone()
    out = torch.empty((T, H), dtype=torch.float32)
    obf = torch.empty((T, H), dtype=torch.int16)
    a = None if r0 is None else r0.contiguous()
    b = None if r1 is None else r1.contiguous()
    wt = weight.contiguous()
    orc().orc_rmsnorm_residual(_p(hn), _p(a), _p(b), _p(wt), float(weight_offset), _p(out),
                               _p(obf), T, H, float(eps))
    return hn, out, obf


def gptq_repack(qweight, qzeros, scales, inn, out, group, keep_f16=False):
    """numpy int32/int32/uint16 inputs -> (payload u8 [out][in/2], scales
    int16 bits [out][in/g], zeros u8 [out][in/g])."""
    ng = inn // group
    pay = np.zeros((out, inn // 2), dtype=np.uint8)
    sc = np.zeros((out, ng), dtype=np.uint16)
    z = np.zeros((out, ng), dtype=np.uint8)
    qw, qz, s = (np.ascontiguousarray(a) for a in (qweight, qzeros, scales))
    orc().orc_gptq_repack(_p(qw), _p(qz), _p(s), inn, out, group, int(keep_f16), _p(pay), _p(sc),
                          _p(z))
    return pay, sc.view(np.int16), z


def int4_zero_unpack(zp, out, groups):
    z = np.zeros((out, groups), dtype=np.uint8)
    zc = None if zp is None else np.ascontiguousarray(zp)
    orc().orc_int4_zero_unpack(_p(zc), out, groups, _p(z))
    return z


def int4_to_signed(gu, gz, dn, dz):
    """In place on numpy uint8 arrays; returns 1 when converted."""
    return orc().orc_int4_to_signed(_p(gu), gu.size, _p(gz), gz.size, _p(dn), dn.size, _p(dz),
                                    dz.size)


def tmoe_layout(H, I):
    off = np.zeros(6, dtype=np.int64)
    orc().orc_tmoe_layout(H, I, _p(off))
    return dict(zip(("gu_p", "gu_s", "dn_p", "dn_s", "gsc", "bytes"), (int(v) for v in off)))


def _block_table(blocks):
    bl = [np.ascontiguousarray(b) for b in blocks]
    tab = (C.c_void_p * len(bl))(*[b.ctypes.data for b in bl])
    return bl, tab


def tmoe_gate_up(blocks, H, I, K, expert, x, M):
    """blocks: list of uint8 numpy arrays (one per expert)."""
    keep, tab = _block_table(blocks)
    h = np.zeros((M, K * I), dtype=np.float32)
    ex, xc = np.ascontiguousarray(expert, np.int32), np.ascontiguousarray(x, np.float32)
    orc().orc_tmoe_gate_up(C.cast(tab, C.c_void_p), H, I, K, len(keep), _p(ex), _p(xc), _p(h), M)
    return h


def tmoe_down(blocks, H, I, K, expert, weight, h, M):
    keep, tab = _block_table(blocks)
    y = np.zeros((M, H), dtype=np.float32)
    ex = np.ascontiguousarray(expert, np.int32)
    wc, hc = np.ascontiguousarray(weight, np.float32), np.ascontiguousarray(h, np.float32)
    orc().orc_tmoe_down(C.cast(tab, C.c_void_p), H, I, K, len(keep), _p(ex), _p(wc), _p(hc),
                        _p(y), M)
    return y


class Heat:
    """ExpertHeat (include/b70/expert_heat.hpp) restated in plain Python, in
    float32 arithmetic like the reference: credit() decays the layer's row
    and adds min(1, cap/n) per route; propose() pairs the hottest
    non-resident with the coldest resident while hot >= cold*hyst + gain."""

    def __init__(self, layers, experts, decay=0.95, hysteresis=1.25, min_gain=1.5,
                 credit_cap=512.0, moves=32):
        self.L, self.E = layers, experts
        f = np.float32
        self.decay, self.hyst, self.gain, self.cap = f(decay), f(hysteresis), f(min_gain), f(credit_cap)
        self.moves = moves
        self.h = np.zeros((layers, experts), dtype=np.float32)

    def credit(self, l, ids):
        if not 0 <= l < self.L:
            return
        row = self.h[l]
        row *= self.decay
        n = len(ids)
        w = self.cap / np.float32(n) if np.float32(n) > self.cap else np.float32(1.0)
        for e in ids:
            if 0 <= e < self.E:
                row[e] = np.float32(row[e] + w)

    def propose(self, resident, movable=None):
        hot, cold = [], []
        for l in range(self.L):
            for e in range(self.E):
                if movable is not None and not movable[l][e]:
                    continue
                x = self.h[l, e]
                if resident[l][e]:
                    cold.append((x, l, e))
                elif x > 0:
                    hot.append((x, l, e))
        hot.sort(key=lambda u: (-u[0], u[1], u[2]))
        cold.sort(key=lambda u: (u[0], u[1], u[2]))
        out = []
        for i in range(min(self.moves, len(hot), len(cold))):
            if not (hot[i][0] >= np.float32(cold[i][0] * self.hyst) + self.gain):
                break
            out.append((hot[i][1], hot[i][2], cold[i][1], cold[i][2]))
        return out


# --- small launchers around the path (numpy restatements) -------------------

def permute_rows_bf16(src, perm, width):
    """launch_permute_rows_bf16 (src/prefill.cpp:2644-2652): bf16 bits (int16)."""
    return src[perm.long()].contiguous().bfloat16().view(torch.int16)


def unpermute_range(src, inverse, rw, dst0, T, K, H, p0, p1, accumulate):
    """launch_moe_unpermute_range (src/prefill.cpp:2674-2688), fp32 fma chain
    in slot order (numpy float32; fma emulated in float64 then rounded, exact
    for a single fma)."""
    s = src.numpy().astype(np.float32)
    inv = inverse.numpy().reshape(T, K)
    w = rw.numpy().reshape(T, K).astype(np.float32)
    v = dst0.numpy().astype(np.float32).copy() if accumulate else np.zeros((T, H), np.float32)
    for t in range(T):
        for k in range(K):
            p = int(inv[t, k])
            if p0 <= p < p1:
                v[t] = (np.float64(w[t, k]) * s[p - p0].astype(np.float64) + v[t].astype(np.float64)).astype(np.float32)
    return torch.from_numpy(v)


def swiglu_bf16(gu_bits, T, inter):
    """launch_swiglu_bf16 (src/prefill.cpp:2541-2558) in float64, then bf16."""
    gu = gu_bits.view(torch.bfloat16).double().reshape(T, 2 * inter)
    g, u = gu[:, :inter], gu[:, inter:]
    return (g / (1 + torch.exp(-g)) * u)


def scale_by_sigmoid_batched(x, gate):
    """launch_scale_by_sigmoid_batched (src/prefill.cpp:2610-2622) in float64."""
    return x.double() * (1.0 / (1.0 + torch.exp(-gate.double())))[:, None]
