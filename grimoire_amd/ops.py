"""Python mirror of the reference's MoE launchers, on torch device tensors.

Same names and argument meaning as the C++ launchers of the reference
(include/b70/moe.hpp:133-173, src/kernels.hpp:500-590, src/prefill.cpp,
src/ops.cpp), with a torch stream in place of the SYCL queue.  Every
function calls libgrimoire_moe.so and raises GrimoireError when the library
rejects the arguments; nothing here computes on the CPU.
"""
from __future__ import annotations

import ctypes as C
from typing import Optional

import torch

from . import _abi
from ._abi import check, lib
from .weights import MoeLayer, Weight


def _p(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _stream(stream=None):
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def _dev(t: torch.Tensor):
    if not t.is_cuda:
        raise _abi.GrimoireError("tensor is not on a GPU: the MoE kernels run on the device only")


# ------------------------------------------------------------------ router

def router_logits(router: torch.Tensor, x: torch.Tensor, logits: torch.Tensor, stream=None):
    """gemv_any(d.router, s.h2, s.rlogits) (src/grimoire.cpp:15364)."""
    _dev(x)
    T, H = x.shape
    E = router.shape[0]
    check(lib().grimoire_moe_router_logits(_stream(stream), _p(router), _p(x), _p(logits), T, E, H),
          "router_logits")


def launch_router_topk(logits, n_experts, top_k, out_expert, out_weight, normalize=True,
                       stream=None):
    """launch_router_topk (src/ops.cpp:1205)."""
    _dev(logits)
    check(lib().grimoire_moe_router_topk(_stream(stream), _p(logits), n_experts, top_k,
                                         _p(out_expert), _p(out_weight), int(normalize)),
          "router_topk")


def launch_router_topk_batched(logits, tokens, n_experts, top_k, out_expert, out_weight,
                               normalize=True, stream=None):
    """launch_router_topk_batched (src/ops.cpp:1347)."""
    _dev(logits)
    check(lib().grimoire_moe_router_topk_batched(_stream(stream), _p(logits), tokens, n_experts,
                                                 top_k, _p(out_expert), _p(out_weight),
                                                 int(normalize)), "router_topk_batched")


def launch_router_topk_bf16_batched(logits_bf16, tokens, n_experts, top_k, out_expert,
                                    out_weight, normalize=True, stream=None):
    """launch_router_topk_bf16_batched (src/ops.cpp:1425): logits as bf16 bits."""
    _dev(logits_bf16)
    check(lib().grimoire_moe_router_topk_bf16_batched(_stream(stream), _p(logits_bf16), tokens,
                                                      n_experts, top_k, _p(out_expert),
                                                      _p(out_weight), int(normalize)),
          "router_topk_bf16_batched")


def launch_router_topk_k2(logits, bias_bf16, tokens, n_experts, top_k, out_expert, out_weight,
                          normalize=True, scaling=1.0, stream=None):
    """launch_router_topk_k2 (src/ops.cpp:2059): sigmoid + selection-only bias."""
    _dev(logits)
    check(lib().grimoire_moe_router_topk_sigmoid(_stream(stream), _p(logits), _p(bias_bf16),
                                                 tokens, n_experts, top_k, _p(out_expert),
                                                 _p(out_weight), int(normalize), float(scaling)),
          "router_topk_sigmoid")


def launch_router_topk_group(logits, bias, tokens, n_experts, top_k, n_group, topk_group,
                             out_expert, out_weight, normalize=True, scaling=1.0, stream=None):
    """Group-limited sigmoid top-k (no reference counterpart)."""
    _dev(logits)
    check(lib().grimoire_moe_router_topk_group(_stream(stream), _p(logits), _p(bias), tokens,
                                               n_experts, top_k, n_group, topk_group,
                                               _p(out_expert), _p(out_weight), int(normalize),
                                               float(scaling)), "router_topk_group")


# ----------------------------------------------------- decode expert products

def launch_moe_gate_up_batched(L: MoeLayer, d_expert, x, h, tokens, stream=None):
    """launch_moe_gate_up(_batched) (src/moe_kernels.cpp:1225, :1372)."""
    _dev(x)
    s = L.struct()
    check(lib().grimoire_moe_gate_up_batched(_stream(stream), s, _p(d_expert), _p(x), _p(h),
                                             tokens), "gate_up")


def launch_moe_down_batched(L: MoeLayer, d_expert, d_weight, h, y, tokens, stream=None):
    """launch_moe_down(_batched) (src/moe_kernels.cpp:1350, :1394)."""
    _dev(h)
    s = L.struct()
    check(lib().grimoire_moe_down_batched(_stream(stream), s, _p(d_expert), _p(d_weight), _p(h),
                                          _p(y), tokens), "down")


def launch_moe_shared_rows(L: MoeLayer, gate_w, rex, rwt, x, h, gate_out, y, M, stream=None):
    """launch_moe_shared_rows (src/moe_kernels.cpp:1316)."""
    _dev(x)
    s = L.struct()
    ws = L.shared_gate_up.struct()
    wd = L.shared_down.struct()
    check(lib().grimoire_moe_shared_rows(_stream(stream), s, ws, wd, _p(gate_w), _p(rex), _p(rwt),
                                         _p(x), _p(h), _p(gate_out), _p(y), M), "shared_rows")


# ---------------------------------------------------------- dispatch/combine

def route_workspace_bytes(tokens, top_k, num_experts) -> int:
    return int(lib().grimoire_moe_route_workspace_bytes(tokens, top_k, num_experts))


def launch_moe_route_grouped(hidden, topk_ids, xperm, xrow, counts, offsets, inverse, tile_e,
                             tile_mb, tmax, tokens, hidden_size, num_experts, mc, top_k,
                             perm_token=None, workspace=None, stream=None):
    """launch_moe_route_grouped (src/prefill.cpp:2726), deterministic order."""
    _dev(topk_ids)
    wsb = route_workspace_bytes(tokens, top_k, num_experts)
    if workspace is None:
        workspace = torch.empty(wsb, dtype=torch.uint8, device=topk_ids.device)
    check(lib().grimoire_moe_route_grouped(_stream(stream), _p(hidden), _p(topk_ids), _p(xperm),
                                           _p(xrow), _p(counts), _p(offsets), _p(inverse),
                                           _p(tile_e), _p(tile_mb), tmax, tokens, hidden_size,
                                           num_experts, mc, top_k, _p(perm_token),
                                           _p(workspace), workspace.numel()), "route_grouped")


def launch_moe_unpermute(src, inverse, route_weight, dst, tokens, top_k, hidden, stream=None):
    """launch_moe_unpermute(_bf16) (src/prefill.cpp:2654, :2690)."""
    _dev(src)
    fn = (lib().grimoire_moe_unpermute_bf16 if src.dtype in (torch.int16, torch.bfloat16)
          else lib().grimoire_moe_unpermute)
    check(fn(_stream(stream), _p(src), _p(inverse), _p(route_weight), _p(dst), tokens, top_k,
             hidden), "unpermute")


def launch_rmsnorm_moe_residual_batched(h, routed, inverse, route_weight, shared, weight, out,
                                        out_bf, tokens, top_k, hidden, eps,
                                        weight_offset=1.0, stream=None):
    """launch_rmsnorm_moe_residual_batched (src/prefill.cpp:1004-1045): h += shared +
    sum_s w_s * routed[inverse]; out = rmsnorm(h) * (weight_offset + weight).  The
    reference reads weight_offset from its global g_norm_weight_offset (1.0 default)."""
    _dev(h)
    check(lib().grimoire_moe_rmsnorm_residual(_stream(stream), _p(h), _p(routed), _p(inverse),
                                              _p(route_weight), _p(shared), _p(weight),
                                              float(weight_offset), _p(out), _p(out_bf), tokens,
                                              top_k, hidden, float(eps)), "rmsnorm_residual")


def launch_rmsnorm_residual_batched(h, r0, r1, weight, out, tokens, hidden, eps, out_bf=None,
                                    weight_offset=1.0, stream=None):
    """launch_rmsnorm_residual_batched (src/prefill.cpp:627-700), ungrouped norms:
    h = (h + r0) + r1 when either is given; out = rmsnorm(h) * (weight_offset + weight)."""
    _dev(h)
    check(lib().grimoire_rmsnorm_residual(_stream(stream), _p(h), _p(r0), _p(r1), _p(weight),
                                          float(weight_offset), _p(out), _p(out_bf), tokens,
                                          hidden, float(eps)), "rmsnorm_residual")


def launch_moe_unpermute_range(src, inverse, route_weight, dst, tokens, top_k, hidden, p0, p1,
                               accumulate=False, stream=None):
    """launch_moe_unpermute_range (src/prefill.cpp:2674)."""
    _dev(src)
    check(lib().grimoire_moe_unpermute_range(_stream(stream), _p(src), _p(inverse),
                                             _p(route_weight), _p(dst), tokens, top_k, hidden, p0,
                                             p1, int(accumulate)), "unpermute_range")


def launch_permute_rows_bf16(src, perm_token, dst, rows, width, stream=None):
    """launch_permute_rows_bf16 (src/prefill.cpp:2644)."""
    _dev(src)
    check(lib().grimoire_moe_permute_rows_bf16(_stream(stream), _p(src), _p(perm_token), _p(dst),
                                               rows, width), "permute_rows_bf16")


def launch_swiglu_bf16(gu, out, tokens, inter, stream=None):
    """launch_swiglu_bf16 (src/prefill.cpp:2541)."""
    _dev(gu)
    check(lib().grimoire_moe_swiglu_bf16(_stream(stream), _p(gu), _p(out), tokens, inter),
          "swiglu_bf16")


def launch_scale_by_sigmoid_batched(x, gate, tokens, hidden, stream=None):
    """launch_scale_by_sigmoid_batched (src/prefill.cpp:2610)."""
    _dev(x)
    check(lib().grimoire_moe_scale_by_sigmoid_batched(_stream(stream), _p(x), _p(gate), tokens,
                                                      hidden), "scale_by_sigmoid_batched")


def launch_scale_by_sigmoid(x, g, n, stream=None):
    """launch_scale_by_sigmoid (src/ops.cpp:1491)."""
    _dev(x)
    check(lib().grimoire_moe_scale_by_sigmoid(_stream(stream), _p(x), _p(g), n),
          "scale_by_sigmoid")


def grouped_gemm(w: Weight, N, swiglu, A, out, offsets, counts, num_experts, total_rows,
                 a_pair=False, out_bf16=False, stream=None):
    """launch_moe_mxfp4_grouped (src/gemm_fast.cpp:2343) for int8/mxfp4/bf16."""
    _dev(A)
    check(lib().grimoire_moe_grouped_gemm(_stream(stream), w.struct(), N, int(swiglu), _p(A),
                                          int(a_pair), _p(out), int(out_bf16), _p(offsets),
                                          _p(counts), num_experts, total_rows), "grouped_gemm")


def pad_mxfp4(w, stream=None):
    """grimoire_moe_pad_mxfp4_rows: a GPU copy of MXFP4 weight w with rows
    padded to grimoire_moe_mxfp4_padded_k(K) elements (zero codes under
    scale byte 127 past K)."""
    _dev(w.payload)
    kp = lib().grimoire_moe_mxfp4_padded_k(w.K)
    if kp <= 0:
        raise ValueError(f"K={w.K}: a multiple of 32")
    dst = Weight(w.fmt, w.N, w.K, torch.empty((w.N, kp // 2), dtype=torch.uint8, device=w.payload.device),
                 torch.empty((w.N, kp // 32), dtype=torch.uint8, device=w.payload.device), None, kp // 32)
    s, d = w.struct(), dst.struct()
    check(lib().grimoire_moe_pad_mxfp4_rows(_stream(stream), C.byref(s), C.byref(d)), "pad_mxfp4_rows")
    return dst


def quant_limbs(src, dst, scale, stream=None):
    """Activation rows fp32 [rows][n] -> two int8 limbs per element (row layout
    [n/64][2][64]) and one fp32 scale per row: a = s * (hi + lo / 254)."""
    _dev(src)
    rows, n = src.shape
    check(lib().grimoire_moe_quant_limbs(_stream(stream), _p(src), rows, n, _p(dst), _p(scale)),
          "quant_limbs")


def tile_table(counts, mc: int = 128, tmax: int = None):
    """The (expert, m-block) tile table of the dispatch (src/grimoire.cpp:
    20743 layout: tile_e / tile_mb, -1 padded to tmax) from per-expert row
    counts, formed on the host."""
    c = [max(0, int(v)) for v in torch.as_tensor(counts).cpu().tolist()]
    te, tm = [], []
    for e, n in enumerate(c):
        for mb in range((n + mc - 1) // mc):
            te.append(e)
            tm.append(mb)
    if tmax is None:
        tmax = max(1, len(te))
    te += [-1] * (tmax - len(te))
    tm += [0] * (tmax - len(tm))
    dev = torch.as_tensor(counts).device
    return (torch.tensor(te[:tmax], dtype=torch.int32, device=dev),
            torch.tensor(tm[:tmax], dtype=torch.int32, device=dev))


def grouped_gemm_i8_rows(w: Weight, N, swiglu, A, a_scale, out, offsets, counts, num_experts,
                         split=0, stream=None):
    """grouped_gemm_i8 with the library's own tile lists formed from counts:
    experts of more than `split` rows (0: the default) on 128-row tiles,
    the others on 32-row tiles."""
    _dev(A)
    check(lib().grimoire_moe_grouped_gemm_i8_rows(_stream(stream), w.struct(), N, int(swiglu), _p(A),
                                                  _p(a_scale), _p(out), _p(offsets), _p(counts),
                                                  num_experts, int(split)), "grouped_gemm_i8_rows")


def grouped_gemm_i8_rows_gather(w: Weight, N, swiglu, A, row_map, a_scale, out, offsets, counts,
                                num_experts, split=0, stream=None):
    """grouped_gemm_i8_rows with routed row r read from A[row_map[r]]
    (A: limb rows of e.g. the tokens; a_scale per routed row)."""
    _dev(A)
    check(lib().grimoire_moe_grouped_gemm_i8_rows_gather(_stream(stream), w.struct(), N, int(swiglu), _p(A),
                                                         A.shape[0], _p(row_map), _p(a_scale), _p(out),
                                                         _p(offsets), _p(counts), num_experts, int(split)),
          "grouped_gemm_i8_rows_gather")


def grouped_gemm_i8(w: Weight, N, swiglu, A, a_scale, out, offsets, counts, num_experts,
                    tile_e=None, tile_mb=None, stream=None):
    """INT8 experts on the int8 MFMA (limb rows from quant_limbs), fp32 out,
    walked through the tile table (tile_table(counts) when not given)."""
    _dev(A)
    if tile_e is None:
        tile_e, tile_mb = tile_table(counts)
    check(lib().grimoire_moe_grouped_gemm_i8(_stream(stream), w.struct(), N, int(swiglu), _p(A),
                                             _p(a_scale), _p(out), _p(offsets), _p(counts),
                                             _p(tile_e), _p(tile_mb), int(tile_e.numel()),
                                             num_experts), "grouped_gemm_i8")


# ------------------------------------------------------------------- layer

class MoeForward:
    """One layer's whole MoE block with a preallocated workspace."""

    def __init__(self, L: MoeLayer, max_tokens: int, route: _abi.RouteParams,
                 regime: int = 0):
        self.L = L
        self.struct = L.struct()
        self.route = route
        self.regime = regime
        nbytes = int(lib().grimoire_moe_forward_workspace_bytes(self.struct, max_tokens))
        # zeroed once: its head holds the one-launch decode's sync words
        self.workspace = torch.zeros(nbytes, dtype=torch.uint8, device=L.router.device)
        self.max_tokens = max_tokens

    def __call__(self, x, y, out_expert=None, out_weight=None, stream=None):
        _dev(x)
        T = x.shape[0]
        if T > self.max_tokens:
            raise _abi.GrimoireError("more tokens than the workspace was sized for")
        check(lib().grimoire_moe_forward(_stream(stream), self.struct, self.route,
                                         _p(self.L.shared_gate_w), _p(x), _p(y), T,
                                         _p(out_expert), _p(out_weight), self.regime,
                                         _p(self.workspace), self.workspace.numel()),
              "moe_forward")


    def shard(self, x, y, begin, count, out_expert=None, out_weight=None, stream=None):
        """grimoire_moe_forward_shard: this layer holds experts [begin,
        begin + count) of a layer whose router is global."""
        _dev(x)
        T = x.shape[0]
        if T > self.max_tokens:
            raise _abi.GrimoireError("more tokens than the workspace was sized for")
        check(lib().grimoire_moe_forward_shard(_stream(stream), self.struct, self.route,
                                               _p(self.L.shared_gate_w), _p(x), _p(y), T,
                                               _p(out_expert), _p(out_weight), self.regime, begin, count,
                                               _p(self.workspace), self.workspace.numel()),
              "moe_forward_shard")

    def sync_status(self, stream=None) -> int:
        """1 when a one-launch decode call on this workspace timed out (the
        workspace is poisoned until sync_reset), else 0; waits for the stream."""
        out = C.c_int(-1)
        check(lib().grimoire_moe_decode_sync_status(_stream(stream), _p(self.workspace),
                                                    self.workspace.numel(), C.byref(out)),
              "decode_sync_status")
        return int(out.value)

    def sync_reset(self, stream=None):
        """Clears the one-launch decode's sync words (stream order)."""
        check(lib().grimoire_moe_decode_sync_reset(_stream(stream), _p(self.workspace),
                                                   self.workspace.numel()), "decode_sync_reset")

    STAGE_ROUTER, STAGE_GATE_UP, STAGE_DOWN = 1, 2, 4

    def stage(self, which, x, y, stream=None):
        """One launch of the decode path (grimoire_moe_decode_stage), on what
        earlier stages or forward calls left in this workspace."""
        _dev(x)
        check(lib().grimoire_moe_decode_stage(_stream(stream), self.struct, self.route,
                                              _p(self.L.shared_gate_w), _p(x), _p(y), x.shape[0],
                                              which, _p(self.workspace), self.workspace.numel()),
              "decode_stage")


# ------------------------------------------------------------------ bridges
# Same symbols and argument order as the reference's dlopen'd bridges, with
# a stream in place of the SYCL queue.  They return nothing (as the
# reference's); a rejected call leaves its reason in
# grimoire_moe_last_error() and writes no output.

def xe2_grouped_mxfp4_bf16(a, b, scales, d, n, k, rows_per_expert, num_experts, stream=None):
    """grimoire_xe2_grouped_mxfp4_bf16 (src/xe2_grouped_bridge.cpp:135)."""
    _dev(a)
    lib().grimoire_xe2_grouped_mxfp4_bf16(_stream(stream), _p(a), _p(b), _p(scales), _p(d), n, k,
                                          _p(rows_per_expert), None, num_experts, None)


def xe2_grouped_w4a16(a, b, scales, d, n, k, rows_per_expert, num_experts, group_size,
                      stream=None):
    """grimoire_xe2_grouped_w4a16 (src/xe2_grouped_bridge.hpp:22)."""
    _dev(a)
    lib().grimoire_xe2_grouped_w4a16(_stream(stream), _p(a), _p(b), _p(scales), _p(d), n, k,
                                     _p(rows_per_expert), None, num_experts, group_size, None)


def xe2_fused_moe_gate_up_mxfp4_silu_bf16(a, b, scales, d, n, k, rows_per_expert, num_experts,
                                          stream=None):
    """grimoire_xe2_fused_moe_gate_up_mxfp4_silu_bf16 (src/xe2_fused_moe_bridge.cpp:32)."""
    _dev(a)
    lib().grimoire_xe2_fused_moe_gate_up_mxfp4_silu_bf16(_stream(stream), _p(a), _p(b),
                                                         _p(scales), _p(d), n, k,
                                                         _p(rows_per_expert), num_experts, None)
