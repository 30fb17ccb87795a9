"""ctypes view of include/grimoire_moe.h and the loader of libgrimoire_moe.so.

The library is loaded from this package directory only.  There is no CPU
fallback: if the library is missing, every call raises.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libgrimoire_moe.so"

# enum grim_fmt (include/grimoire_moe.h); codes 0..6 follow the reference's
# Fmt numbering (include/b70/formats.hpp:237-239).
FMT_BF16 = 0
FMT_INT8 = 3
FMT_INT4 = 4
FMT_MXFP4 = 6
FMT_INT4_F16 = 64

ROUTE_SOFTMAX = 0
ROUTE_SIGMOID = 1
ROUTE_GROUP = 2


ERR_FORMAT, ERR_SHAPE, ERR_ARG, ERR_WORKSPACE = -1, -2, -3, -4


class QuantWeight(C.Structure):
    """b70::QuantWeight (include/b70/weights.hpp:46-126)."""
    _fields_ = [
        ("fmt", C.c_int32),
        ("N", C.c_int32),
        ("K", C.c_int32),
        ("row_scales", C.c_int32),
        ("row_bytes", C.c_int64),
        ("payload", C.c_void_p),
        ("scales", C.c_void_p),
        ("zeros", C.c_void_p),
    ]


class MoeConfig(C.Structure):
    """b70::MoeConfig (include/b70/moe.hpp:70-77)."""
    _fields_ = [
        ("hidden", C.c_int32),
        ("inter", C.c_int32),
        ("num_experts", C.c_int32),
        ("top_k", C.c_int32),
        ("shared_inter", C.c_int32),
        ("norm_topk", C.c_int32),
    ]


class MoeLayer(C.Structure):
    """b70::MoeLayer (include/b70/moe.hpp:85-117)."""
    _fields_ = [
        ("cfg", MoeConfig),
        ("gate_up", QuantWeight),
        ("down", QuantWeight),
        ("has_shared", C.c_int32),
        ("_pad", C.c_int32),
        ("shared_gate_up", QuantWeight),
        ("shared_down", QuantWeight),
        ("router", C.c_void_p),
    ]


class RouteParams(C.Structure):
    _fields_ = [
        ("mode", C.c_int32),
        ("n_group", C.c_int32),
        ("topk_group", C.c_int32),
        ("scaling", C.c_float),
        ("bias", C.c_void_p),
    ]


class ExpertSrc(C.Structure):
    """grim_expert_src: one checkpoint projection (weight, zeros, scales)."""
    _fields_ = [
        ("kind", C.c_int32),
        ("in_", C.c_int32),
        ("out", C.c_int32),
        ("group", C.c_int32),
        ("weight", C.c_void_p),
        ("zeros", C.c_void_p),
        ("scales", C.c_void_p),
    ]


SRC_GPTQ, SRC_MXFP4_PACKED, SRC_INT4_PACKED = 1, 2, 3


class NvExpertLayout(C.Structure):
    """grim_nv_expert_layout (b70::NvExpertLayout, include/b70/tiered_moe.hpp:40-60)."""
    _fields_ = [("H", C.c_int32), ("I", C.c_int32), ("gu_p", C.c_int64), ("gu_s", C.c_int64),
                ("dn_p", C.c_int64), ("dn_s", C.c_int64), ("gsc", C.c_int64),
                ("bytes", C.c_int64)]


class TieredMoeView(C.Structure):
    """grim_tiered_moe_view (b70::TieredMoeView)."""
    _fields_ = [("lay", NvExpertLayout), ("eptr", C.c_void_p), ("E", C.c_int32),
                ("top_k", C.c_int32)]


class HeatParams(C.Structure):
    """grim_heat_params (b70::ExpertHeatParams, include/b70/expert_heat.hpp)."""
    _fields_ = [("decay", C.c_float), ("hysteresis", C.c_float), ("min_gain", C.c_float),
                ("credit_cap", C.c_float), ("moves_per_step", C.c_int32)]


class ExpertSwap(C.Structure):
    _fields_ = [("promote_layer", C.c_int32), ("promote_expert", C.c_int32),
                ("demote_layer", C.c_int32), ("demote_expert", C.c_int32)]

P = C.c_void_p
I32 = C.c_int
F32 = C.c_float
SZ = C.c_size_t
QWP = C.POINTER(QuantWeight)
LP = C.POINTER(MoeLayer)
RPP = C.POINTER(RouteParams)

# name -> (restype, argtypes); must match include/grimoire_moe.h
SIGNATURES = {
    "grimoire_moe_last_error": (C.c_char_p, []),
    "grimoire_moe_version": (C.c_char_p, []),
    "grimoire_moe_router_logits": (I32, [P, P, P, P, I32, I32, I32]),
    "grimoire_moe_router_topk": (I32, [P, P, I32, I32, P, P, I32]),
    "grimoire_moe_router_topk_batched": (I32, [P, P, I32, I32, I32, P, P, I32]),
    "grimoire_moe_router_topk_bf16_batched": (I32, [P, P, I32, I32, I32, P, P, I32]),
    "grimoire_moe_router_topk_sigmoid": (I32, [P, P, P, I32, I32, I32, P, P, I32, F32]),
    "grimoire_moe_router_topk_group": (I32, [P, P, P, I32, I32, I32, I32, I32, P, P, I32, F32]),
    "grimoire_moe_gate_up": (I32, [P, LP, P, P, P]),
    "grimoire_moe_down": (I32, [P, LP, P, P, P, P]),
    "grimoire_moe_gate_up_shared": (I32, [P, LP, QWP, P, P, P, P, P]),
    "grimoire_moe_down_shared": (I32, [P, LP, QWP, P, P, P, P, P]),
    "grimoire_moe_gate_up_batched": (I32, [P, LP, P, P, P, I32]),
    "grimoire_moe_down_batched": (I32, [P, LP, P, P, P, P, I32]),
    "grimoire_moe_shared_rows": (I32, [P, LP, QWP, QWP, P, P, P, P, P, P, P, I32]),
    "grimoire_moe_route_workspace_bytes": (SZ, [I32, I32, I32]),
    "grimoire_moe_route_grouped": (I32, [P, P, P, P, P, P, P, P, P, P, I32, I32, I32, I32, I32,
                                         I32, P, P, SZ]),
    "grimoire_moe_remap_bf16": (I32, [P, P, P, P, P, P, P, I32, I32, I32, I32, P, SZ]),
    "grimoire_moe_unpermute": (I32, [P, P, P, P, P, I32, I32, I32]),
    "grimoire_moe_unpermute_bf16": (I32, [P, P, P, P, P, I32, I32, I32]),
    "grimoire_moe_combine": (I32, [P, P, P, P, P, P, P, I32, I32, I32]),
    "grimoire_moe_unpermute_range": (I32, [P, P, P, P, P, I32, I32, I32, I32, I32, I32]),
    "grimoire_moe_permute_rows_bf16": (I32, [P, P, P, P, I32, I32]),
    "grimoire_moe_swiglu_bf16": (I32, [P, P, P, I32, I32]),
    "grimoire_moe_scale_by_sigmoid": (I32, [P, P, P, I32]),
    "grimoire_moe_scale_by_sigmoid_batched": (I32, [P, P, P, I32, I32]),
    "grimoire_moe_rmsnorm_residual": (I32, [P, P, P, P, P, P, P, F32, P, P, I32, I32, I32,
                                            F32]),
    "grimoire_rmsnorm_residual": (I32, [P, P, P, P, P, F32, P, P, I32, I32, F32]),
    "grimoire_moe_ingest_projection": (I32, [P, C.POINTER(ExpertSrc), QWP, I32]),
    "grimoire_moe_ingest_projections": (I32, [P, C.POINTER(ExpertSrc), P, I32, QWP]),
    "grimoire_moe_int4_to_signed": (I32, [P, P, SZ, P, SZ, P, SZ, P, SZ, P]),
    "grimoire_tmoe_layout": (I32, [I32, I32, C.POINTER(NvExpertLayout)]),
    "grimoire_tmoe_gate_up": (I32, [P, C.POINTER(TieredMoeView), P, P, P, I32]),
    "grimoire_tmoe_down": (I32, [P, C.POINTER(TieredMoeView), P, P, P, P, I32]),
    "grimoire_tmoe_place": (I32, [P, P, I32, P, P, SZ]),
    "grimoire_tmoe_scratch_bytes": (SZ, [C.POINTER(NvExpertLayout), I32]),
    "grimoire_tmoe_expert_gemm": (I32, [P, P, C.POINTER(NvExpertLayout), I32, F32, F32, P, P, I32,
                                        P, SZ]),
    "grimoire_tmoe_expert_ffn": (I32, [P, P, C.POINTER(NvExpertLayout), F32, F32, F32, P, P, P,
                                       I32, P, SZ]),
    "grimoire_cpu_experts_create": (P, [I32, P, I32]),
    "grimoire_cpu_experts_destroy": (None, [P]),
    "grimoire_cpu_experts_threads": (I32, [P]),
    "grimoire_cpu_experts_wait_us": (C.c_double, [P]),
    "grimoire_cpu_experts_ffn": (I32, [P, C.POINTER(NvExpertLayout), P, P, I32, P, P]),
    "grimoire_cpu_experts_ffn_rows": (I32, [P, C.POINTER(NvExpertLayout), I32, P, P, P, P, P]),
    "grimoire_cpu_nvfp4_dot": (F32, [P, P, P, I32]),
    "grimoire_cpu_set_isa": (I32, [I32]),
    "grimoire_cpu_pool_cpus": (I32, [I32, I32, P, I32]),
    "grimoire_heat_default_params": (None, [C.POINTER(HeatParams)]),
    "grimoire_heat_create": (P, [I32, I32, C.POINTER(HeatParams)]),
    "grimoire_heat_destroy": (None, [P]),
    "grimoire_heat_credit": (None, [P, I32, P, SZ]),
    "grimoire_heat_get": (F32, [P, I32, I32]),
    "grimoire_heat_propose": (I32, [P, P, P, C.POINTER(ExpertSwap), I32]),
    "grimoire_moe_grouped_gemm": (I32, [P, QWP, I32, I32, P, I32, P, I32, P, P, I32, I32]),
    "grimoire_moe_quant_limbs": (I32, [P, P, I32, I32, P, P]),
    "grimoire_moe_mxfp4_padded_k": (I32, [I32]),
    "grimoire_moe_pad_mxfp4_rows": (I32, [P, QWP, QWP]),
    "grimoire_moe_grouped_gemm_i8": (I32, [P, QWP, I32, I32, P, P, P, P, P, P, P, I32, I32]),
    "grimoire_moe_grouped_gemm_i8_rows": (I32, [P, QWP, I32, I32, P, P, P, P, P, I32, I32]),
    "grimoire_moe_grouped_gemm_i8_rows_gather": (I32, [P, QWP, I32, I32, P, I32, P, P, P, P, P, I32, I32]),
    "grimoire_xe2_grouped_mxfp4_bf16": (None, [P, P, P, P, P, I32, I32, P, P, I32, P]),
    "grimoire_xe2_grouped_mxfp4_bf16_full": (None, [P, P, P, P, P, I32, I32, P, P, I32, P]),
    "grimoire_xe2_grouped_mxfp4_bf16_m8": (None, [P, P, P, P, P, I32, I32, P, P, I32, P]),
    "grimoire_xe2_grouped_mxfp4_bf16_m16": (None, [P, P, P, P, P, I32, I32, P, P, I32, P]),
    "grimoire_xe2_grouped_w4a16": (None, [P, P, P, P, P, I32, I32, P, P, I32, I32, P]),
    "grimoire_xe2_fused_moe_gate_up_mxfp4_silu_bf16": (None, [P, P, P, P, P, I32, I32, P, I32, P]),
    "grimoire_moe_forward_workspace_bytes": (SZ, [LP, I32]),
    "grimoire_moe_forward": (I32, [P, LP, RPP, P, P, P, I32, P, P, I32, P, SZ]),
    "grimoire_moe_forward_noalloc_max_bytes": (SZ, []),
    "grimoire_moe_forward_noalloc": (I32, [P, LP, RPP, P, P, P, I32, P, P, I32]),
    "grimoire_moe_forward_shard": (I32, [P, LP, RPP, P, P, P, I32, P, P, I32, I32, I32, P, SZ]),
    "grimoire_moe_route_local": (I32, [P, P, P, P, P, I32, I32, I32]),
    "grimoire_moe_decode_sync_status": (I32, [P, P, SZ, C.POINTER(C.c_int)]),
    "grimoire_moe_decode_sync_reset": (I32, [P, P, SZ]),
    "grimoire_moe_debug_spin_ticks": (C.c_uint64, [C.c_int64]),
    "grimoire_moe_decode_stage": (I32, [P, LP, RPP, P, P, P, I32, I32, P, SZ]),
}

_lib = None


def lib() -> C.CDLL:
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m grimoire_amd.build` "
                "(there is no CPU fallback)")
        l = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            f = getattr(l, name)
            f.restype = res
            f.argtypes = args
        _lib = l
    return _lib


class GrimoireError(RuntimeError):
    pass


def check(status: int, what: str) -> None:
    if status != 0:
        msg = lib().grimoire_moe_last_error().decode()
        raise GrimoireError(f"{what} failed with status {status}: {msg}")
