"""The C ABI library loads, exports every function include/grimoire_moe.h
declares, and rejects bad arguments on the host before any launch.
CPU only: no call here reaches a kernel."""
import ctypes as C
import re
from pathlib import Path

import pytest
import torch

from grimoire_amd import _abi
from grimoire_amd.weights import make_int8

HEADER = Path(__file__).resolve().parents[1] / "include" / "grimoire_moe.h"


def declared():
    txt = HEADER.read_text()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(grimoire_\w+)\s*\(", txt)))


def test_every_declared_symbol_is_exported():
    lib = _abi.lib()
    names = declared()
    assert len(names) >= 25
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_abi.SIGNATURES), set(names) ^ set(_abi.SIGNATURES)


def test_version():
    assert b"gfx950" in _abi.lib().grimoire_moe_version()


def _layer(fmt=_abi.FMT_INT8):
    w = make_int8(8 * 2 * 64, 128)
    d = make_int8(8 * 128, 64)
    L = _abi.MoeLayer()
    L.cfg = _abi.MoeConfig(128, 64, 8, 2, 0, 1)
    L.gate_up = w.struct()
    L.gate_up.fmt = fmt
    L.down = d.struct()
    return L, (w, d)


def test_unknown_format_rejected():
    L, keep = _layer(fmt=99)
    st = _abi.lib().grimoire_moe_gate_up(None, L, 1, 1, 1)
    assert st == _abi.ERR_FORMAT
    assert b"format" in _abi.lib().grimoire_moe_last_error()


def test_shape_rejections():
    lib = _abi.lib()
    L, keep = _layer()
    L.cfg.top_k = 17
    assert lib.grimoire_moe_gate_up(None, L, 1, 1, 1) == _abi.ERR_SHAPE
    L.cfg.top_k = 2
    L.gate_up.K = 100            # K does not match hidden
    assert lib.grimoire_moe_gate_up(None, L, 1, 1, 1) == _abi.ERR_SHAPE
    assert lib.grimoire_moe_router_topk(None, 1, 600, 8, 1, 1, 1) == _abi.ERR_SHAPE
    assert lib.grimoire_moe_router_topk(None, 1, 64, 17, 1, 1, 1) == _abi.ERR_SHAPE
    assert lib.grimoire_moe_router_topk_group(None, 1, None, 1, 256, 8, 7, 4, 1, 1, 1, 1.0) == _abi.ERR_SHAPE
    assert lib.grimoire_moe_router_topk_group(None, 1, None, 1, 256, 40, 8, 1, 1, 1, 1, 1.0) == _abi.ERR_SHAPE
    # the INT8 GEMM's own tile lists cover at most 1024 experts
    w = _abi.QuantWeight()
    w.fmt = _abi.FMT_INT8
    assert lib.grimoire_moe_grouped_gemm_i8_rows(None, w, 64, 0, 1, 1, 1, 1, 1, 1025, 0) == _abi.ERR_SHAPE


def test_null_and_workspace_rejections():
    lib = _abi.lib()
    L, keep = _layer()
    assert lib.grimoire_moe_gate_up(None, L, None, 1, 1) == _abi.ERR_ARG
    assert lib.grimoire_moe_unpermute(None, None, 1, 1, 1, 4, 2, 8) == _abi.ERR_ARG
    assert lib.grimoire_moe_rmsnorm_residual(None, 1, 1, 1, 1, None, None, 1.0, 1, None, 4, 2, 8,
                                             1e-6) == _abi.ERR_ARG
    assert lib.grimoire_moe_rmsnorm_residual(None, 1, 1, 1, 1, None, 1, 1.0, 1, None, 4, 17, 8,
                                             1e-6) == _abi.ERR_SHAPE
    assert lib.grimoire_moe_rmsnorm_residual(None, 1, 1, 1, 1, None, 1, 1.0, 1, None, 4, 8, 6,
                                             1e-6) == _abi.ERR_SHAPE
    ws = lib.grimoire_moe_route_workspace_bytes(100, 8, 64)
    assert ws > 0
    assert lib.grimoire_moe_route_grouped(None, 1, 1, None, None, 1, 1, 1, None, None, 0, 100, 64,
                                          64, 0, 8, None, 1, ws - 1) == _abi.ERR_WORKSPACE
    assert lib.grimoire_moe_forward_workspace_bytes(L, 16) > 0


def test_zero_tokens_is_a_no_op():
    lib = _abi.lib()
    assert lib.grimoire_moe_router_topk_batched(None, None, 0, 64, 8, None, None, 1) == 0
    assert lib.grimoire_moe_unpermute(None, None, None, None, None, 0, 8, 64) == 0
    assert lib.grimoire_moe_rmsnorm_residual(None, None, None, None, None, None, None, 1.0, None,
                                             None, 0, 8, 64, 1e-6) == 0
    assert lib.grimoire_rmsnorm_residual(None, None, None, None, None, 1.0, None, None, 0, 64,
                                         1e-6) == 0
    assert lib.grimoire_rmsnorm_residual(None, 1, None, None, None, 1.0, None, None, 2, 64,
                                         1e-6) == _abi.ERR_ARG
    assert lib.grimoire_rmsnorm_residual(None, 1, None, None, 1, 1.0, None, None, 2, 66,
                                         1e-6) == _abi.ERR_SHAPE


def test_ingest_rejections():
    """grimoire_moe_ingest_projection{,s}: shape, format and alignment checks
    happen on the host, before anything is launched."""
    lib = _abi.lib()
    P = 1 << 12                                     # a fake, aligned address
    dst = _abi.QuantWeight(fmt=_abi.FMT_INT4, N=64, K=256, row_scales=2, row_bytes=128,
                           payload=P, scales=P, zeros=P)
    src = _abi.ExpertSrc(_abi.SRC_GPTQ, 256, 64, 128, P, P, P)
    ing = lambda s, d, r: lib.grimoire_moe_ingest_projection(None, C.byref(s), C.byref(d), r)
    assert ing(src, dst, 8) == _abi.ERR_SHAPE                      # rows past N
    bad = _abi.ExpertSrc(_abi.SRC_GPTQ, 256, 64, 128, P + 2, P, P)
    assert ing(bad, dst, 0) == _abi.ERR_ARG                         # misaligned qweight
    nz = _abi.ExpertSrc(_abi.SRC_GPTQ, 256, 64, 128, P, None, P)
    assert ing(nz, dst, 0) == _abi.ERR_ARG                          # GPTQ without qzeros
    mx = _abi.ExpertSrc(_abi.SRC_MXFP4_PACKED, 256, 64, 32, P, None, P)
    assert ing(mx, dst, 0) == _abi.ERR_FORMAT                       # MXFP4 into INT4
    g64 = _abi.ExpertSrc(_abi.SRC_GPTQ, 256, 64, 64, P, P, P)
    assert ing(g64, dst, 0) == _abi.ERR_SHAPE                       # row_scales != in/group
    two = (_abi.ExpertSrc * 2)(src, _abi.ExpertSrc(_abi.SRC_GPTQ, 256, 32, 128, P, P, P))
    rows = (C.c_int32 * 2)(0, 0)
    assert lib.grimoire_moe_ingest_projections(None, two, C.cast(rows, C.c_void_p), 2,
                                               C.byref(dst)) == _abi.ERR_SHAPE   # shapes differ
    assert lib.grimoire_moe_ingest_projections(None, two, C.cast(rows, C.c_void_p), 0,
                                               C.byref(dst)) == 0                # nothing to do
    assert lib.grimoire_moe_int4_to_signed(None, None, 16, None, 0, None, 0, None, 0,
                                           P) == _abi.ERR_ARG


def test_tiered_rejections():
    lib = _abi.lib()
    L = _abi.NvExpertLayout()
    assert lib.grimoire_tmoe_layout(2048, 768, C.byref(L)) == 0
    v = _abi.TieredMoeView(L, 1 << 12, 16, 8)
    assert lib.grimoire_tmoe_gate_up(None, C.byref(v), None, None, None, 0) == 0   # M = 0
    v.top_k = 33
    assert lib.grimoire_tmoe_gate_up(None, C.byref(v), 1, 1, 1, 1) == _abi.ERR_SHAPE
    v.top_k = 8
    L2 = _abi.NvExpertLayout.from_buffer_copy(L)
    L2.dn_p += 16                                                   # not the library's layout
    v2 = _abi.TieredMoeView(L2, 1 << 12, 16, 8)
    assert lib.grimoire_tmoe_down(None, C.byref(v2), 1, 1, 1, 1, 1) == _abi.ERR_ARG
    need = lib.grimoire_tmoe_scratch_bytes(C.byref(L), 10)
    assert need >= 2 * 2 * 768 * 2048 + 10 * 2 * 768 * 4
    assert lib.grimoire_tmoe_expert_gemm(None, 1, C.byref(L), 1, 1.0, 1.0, 1, 1, 10, 1,
                                         need - 1) == _abi.ERR_WORKSPACE
    assert lib.grimoire_heat_create(0, 8, None) is None
    h = lib.grimoire_heat_create(2, 8, None)
    assert lib.grimoire_heat_propose(h, None, None, None, 0) == _abi.ERR_ARG
    lib.grimoire_heat_destroy(h)


def test_bridge_rejections():
    """Bridge argument errors are caught on the host (nothing launched) and
    reported through grimoire_moe_last_error()."""
    lib = _abi.lib()
    P = 1 << 12
    rows = (C.c_int32 * 2)(3, 4)
    r = C.cast(rows, C.c_void_p)

    def last():
        return lib.grimoire_moe_last_error().decode()

    lib.grimoire_xe2_grouped_mxfp4_bf16(None, P, P, P, P, 128, 96, r, None, 2, None)
    assert "multiple of 64" in last()                    # k % 64
    lib.grimoire_xe2_grouped_mxfp4_bf16(None, P, P, P, P, 128, 128, None, None, 2, None)
    assert "null pointer" in last()                      # rows_per_expert
    lib.grimoire_xe2_grouped_mxfp4_bf16(None, None, P, P, P, 128, 128, r, None, 2, None)
    assert "null pointer" in last()                      # a
    lib.grimoire_xe2_grouped_mxfp4_bf16_m8(None, P, P, P, None, 128, 128, r, None, 2, None)
    assert "null pointer" in last()                      # d, through a variant
    lib.grimoire_xe2_grouped_mxfp4_bf16(None, P, P, P, P, 128, 128, r, None, 2000, None)
    assert "num_experts" in last()                       # beyond the in-LDS tile order
    lib.grimoire_xe2_fused_moe_gate_up_mxfp4_silu_bf16(None, P, P, P, P, 100, 128, r, 2, None)
    assert "n %% 8" in last() or "n % 8" in last()
    lib.grimoire_xe2_fused_moe_gate_up_mxfp4_silu_bf16(None, P, None, P, P, 128, 128, r, 2, None)
    assert "null pointer" in last()
    lib.grimoire_xe2_grouped_w4a16(None, P, P, P, P, 128, 128, r, None, 2, 96, None)
    assert "group" in last()
