"""Benchmark of the MI355X MoE layer.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-prefill] [--no-cpu]

Workload ("C2"): single-token decode through 48
distinct MoE layers back to back (T=1, H=2048, E=128, top-8 softmax, SwiGLU
I=768, GPTQ int4 g128 fp16 scales, random weights generated on the GPU).
One step = one token through all 48 layers (router GEMV, top-k, gate_up,
down), so the 48 x 20.5 MB of touched weights (985 MB) exceed the 256 MB
MALL.  `value` is HBM GB/s over the algorithmic bytes of the step: the
distinct experts each layer touches (payload + scales), the fp32 router,
x and y.  Inputs are resident in HBM before timing starts.

The JSON line also carries:
  roofline      gate_up decode kernel (the dominant one), timed with HIP
                events on its stream, against 8 TB/s;
  cpu_baseline  the CPU path on all host threads (this build's C restatement
                of src/moe_ref.cpp, OpenMP over tokens) on a bounded sample
                of the same layer, with the host's core count; beside it
                the reference's own moe_ref.cpp (oracle/_ref), one thread;
  prefill       C4 (T=4096, E=512, top-10 Zipf(1.2), int8, shared expert):
                layer time and grouped-GEMM TFLOPS against the bf16 MFMA
                peak;
  c3, c5        C3 (T=8 MXFP4 decode, Zipf(1.1)) and C5 (T=32 verify, 6 GB
                of MXFP4 experts, group-limited routing): layer time, GB/s
                and the HBM fraction;
  edges         the fused combine + residual + RMSNorm and the residual
                RMSNorm (C4 shapes) against 8 TB/s, and the GPTQ ingestion
                of one C2 layer's experts, and the tiered NVFP4 experts.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from grimoire_amd import _abi, configs, ops  # noqa: E402

HBM_PEAK_GBS = 8000.0
BF16_MFMA_PEAK_TFLOPS = 2500.0
LAYERS = 48


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Timer:
    """HIP events recorded on the given stream."""

    def __init__(self, stream):
        self.s = stream
        self.a = torch.cuda.Event(enable_timing=True)
        self.b = torch.cuda.Event(enable_timing=True)

    def __enter__(self):
        self.a.record(self.s)
        return self

    def __exit__(self, *exc):
        self.b.record(self.s)

    def ms(self):
        self.b.synchronize()
        return self.a.elapsed_time(self.b)


def _graph(fn, stream):
    """Capture fn() (kernel launches on `stream`) into a HIP graph."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        fn()
    return g


def _replay(g, stream, n=1):
    """Replay on `stream` (a graph launches on the current stream)."""
    with torch.cuda.stream(stream):
        for _ in range(n):
            g.replay()


def decode_bench(steps, warmup, dev, stream, regime=1):
    cfg = configs.CONFIGS["c2"]
    layers = [configs.make_layer(cfg, dev, seed=100 + i) for i in range(LAYERS)]
    x = configs.make_x(cfg, dev, seed=7)
    fwds = [ops.MoeForward(L, 1, configs.route_params(cfg, None), regime=regime)
            for L in layers]
    ys = [torch.empty(1, cfg.H, device=dev) for _ in layers]
    oes = [torch.empty(1, cfg.K, dtype=torch.int32, device=dev) for _ in layers]
    ows = [torch.empty(1, cfg.K, dtype=torch.float32, device=dev) for _ in layers]

    def step():
        for f, y, oe, ow in zip(fwds, ys, oes, ows):
            f(x, y, oe, ow, stream=stream)

    # eager once (routing for the byte count), then the step as one graph
    with torch.cuda.stream(stream):
        step()
    torch.cuda.synchronize()
    g_step = _graph(step, stream)
    ebytes = layers[0].expert_bytes()
    step_bytes = 0.0
    for oe in oes:
        distinct = len(set(oe.flatten().tolist()))
        step_bytes += distinct * ebytes + cfg.E * cfg.H * 4 + 2 * cfg.H * 4
    _replay(g_step, stream, warmup)
    torch.cuda.synchronize()
    with Timer(stream) as tm:
        _replay(g_step, stream, steps)
    ms = tm.ms() / steps

    # one layer replayed on its own (its 20.5 MB stay in the 256 MB MALL)
    g_one = _graph(lambda: fwds[0](x, ys[0], oes[0], ows[0], stream=stream), stream)
    _replay(g_one, stream, 20)
    reps1 = 200
    with Timer(stream) as t1:
        _replay(g_one, stream, reps1)
    one_us = t1.ms() * 1e3 / reps1

    # dominant kernel: the forward's gate_up launch (top-k + gate_up +
    # SwiGLU, decode stage 2), 48 layers' launches captured alone, each on
    # the logits and activations its layer's forward left in its workspace
    gu_bytes = cfg.K * layers[0].gate_up.row_bytes_total() * 2 * cfg.I + cfg.H * 4 + cfg.K * cfg.I * 4

    def gu_only():
        for f, y in zip(fwds, ys):
            f.stage(ops.MoeForward.STAGE_GATE_UP, x, y, stream=stream)

    g_gu = _graph(gu_only, stream)
    _replay(g_gu, stream)
    torch.cuda.synchronize()
    reps = max(steps, 10)
    with Timer(stream) as tg:
        _replay(g_gu, stream, reps)
    gu_us = tg.ms() * 1e3 / (reps * LAYERS)

    gbs = step_bytes / (ms * 1e-3) / 1e9
    return dict(cfg=cfg, ms=ms, step_bytes=step_bytes, gbs=gbs, gu_us=gu_us, gu_bytes=gu_bytes,
                one_us=one_us, layers=layers, x=x, oes=oes, ows=ows)


def decode_one_launch(d, dev, stream, steps):
    """The same 48 layers through the one-launch decode (regime 7): µs per
    layer in one graph, for comparison with the default three launches."""
    cfg = d["cfg"]
    fwds = [ops.MoeForward(L, 1, configs.route_params(cfg, None), regime=7) for L in d["layers"]]
    ys = [torch.empty(1, cfg.H, device=dev) for _ in fwds]

    def step():
        for f, y in zip(fwds, ys):
            f(d["x"], y, stream=stream)

    with torch.cuda.stream(stream):
        step()
    torch.cuda.synchronize()
    g = _graph(step, stream)
    _replay(g, stream, 3)
    torch.cuda.synchronize()
    with Timer(stream) as tm:
        _replay(g, stream, steps)
    us = tm.ms() * 1e3 / (steps * LAYERS)
    return {"kernel": "grim::moe_decode_fused_kernel (router, top-k, gate_up, down in one launch)",
            "us_per_layer": round(us, 2), "GB/s": round(d["step_bytes"] / LAYERS / (us * 1e-6) / 1e9, 1)}


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, each scaled by the copy-kernel
    calibration recorded beside it), or None when there is none."""
    f = ROOT / "profiles" / "traffic.json"
    try:
        t = json.loads(f.read_text())
        return t["kernels"][kernel]["hbm_bytes_per_launch"]
    except Exception:
        return None


def prefill_bench(dev, stream, reps=20, warm=10):
    cfg = configs.CONFIGS["c4"]
    wl = configs.make_workload(cfg, dev, seed=11)
    L = wl.layer
    fwd = ops.MoeForward(L, cfg.T, configs.route_params(cfg, wl.route_bias), regime=2)
    y = torch.empty(cfg.T, cfg.H, device=dev)
    oe = torch.empty(cfg.T, cfg.K, dtype=torch.int32, device=dev)
    ow = torch.empty(cfg.T, cfg.K, dtype=torch.float32, device=dev)
    with torch.cuda.stream(stream):
        # untimed calls first: the clocks settle over the first few ms of
        # this much matrix-core work
        for _ in range(warm):
            fwd(wl.x, y, oe, ow, stream=stream)
        torch.cuda.synchronize()
        with Timer(stream) as tm:
            for _ in range(reps):
                fwd(wl.x, y, oe, ow, stream=stream)
        layer_ms = tm.ms() / reps
        # the routed grouped GEMMs alone, on the same routing: the INT8
        # experts' path of the forward (activation limbs -> int8 MFMA)
        R = cfg.T * cfg.K
        tmax = cfg.E + (R + 127) // 128
        counts = torch.empty(cfg.E, dtype=torch.int32, device=dev)
        offsets = torch.empty(cfg.E, dtype=torch.int32, device=dev)
        inverse = torch.empty(R, dtype=torch.int32, device=dev)
        te = torch.empty(tmax, dtype=torch.int32, device=dev)
        tmb = torch.empty(tmax, dtype=torch.int32, device=dev)
        ops.launch_moe_route_grouped(wl.x, oe, None, None, counts, offsets, inverse, te, tmb, tmax,
                                     cfg.T, cfg.H, cfg.E, 128, cfg.K, stream=stream)
        # as in the forward: x limbs once per token, gathered by the GEMM
        # through the routed row -> token map
        xq = torch.empty(cfg.T, 2 * cfg.H, dtype=torch.int8, device=dev)
        xs_tok = torch.empty(cfg.T, device=dev)
        ops.quant_limbs(wl.x, xq, xs_tok, stream=stream)
        row_map = torch.empty(R, dtype=torch.int32, device=dev)
        row_map[inverse.long()] = torch.arange(R, device=dev, dtype=torch.int32) // cfg.K
        xs = xs_tok[row_map.long()].contiguous()
        h = torch.empty(R, cfg.I, device=dev)
        hq = torch.empty(R, 2 * cfg.I, dtype=torch.int8, device=dev)
        hs = torch.empty(R, device=dev)
        yp = torch.empty(R, cfg.H, device=dev)
        # the forward's own call: tile lists formed from the row counts
        # (experts of few rows on 32-row tiles)
        def gate_up():
            ops.grouped_gemm_i8_rows_gather(L.gate_up, 2 * cfg.I, True, xq, row_map, xs, h, offsets, counts,
                                            cfg.E, stream=stream)

        def down():
            ops.grouped_gemm_i8_rows(L.down, cfg.H, False, hq, hs, yp, offsets, counts, cfg.E,
                                     stream=stream)

        gate_up()
        ops.quant_limbs(h, hq, hs, stream=stream)
        for _ in range(3):
            gate_up()
            down()
        torch.cuda.synchronize()
        # each GEMM timed in the layer's order (gate_up, h limbs, down), as
        # the forward runs them: back-to-back repeats of one GEMM alone run
        # the matrix core hotter than a layer does
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
               torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
        for a, b, c, d in ev:
            a.record(stream)
            gate_up()
            b.record(stream)
            ops.quant_limbs(h, hq, hs, stream=stream)
            c.record(stream)
            down()
            d.record(stream)
        torch.cuda.synchronize()
        gu_ms = sum(a.elapsed_time(b) for a, b, c, d in ev) / reps
        dn_ms = sum(c.elapsed_time(d) for a, b, c, d in ev) / reps
        cnt = counts.cpu()
    touched = int((cnt > 0).sum())
    routed_flops = 6.0 * R * cfg.H * cfg.I
    shared_flops = 6.0 * cfg.T * cfg.H * cfg.I
    gu_flops, dn_flops = 4.0 * R * cfg.H * cfg.I, 2.0 * R * cfg.H * cfg.I
    ebytes = L.expert_bytes()
    layer_bytes = touched * ebytes + L.shared_bytes() + cfg.E * cfg.H * 4 + 2 * cfg.T * cfg.H * 4
    # algorithmic bytes of each GEMM: the touched experts' int8 rows with
    # their bf16 row scales, the two int8 activation limbs of every input
    # row (gate_up: the tokens' rows, gathered per route; down: the routed
    # h rows), the fp32 output rows; its roofline time is the larger of the
    # FLOP time at the bf16 peak and the byte time at the HBM peak
    gu_bytes = touched * 2 * cfg.I * (cfg.H + 2) + cfg.T * 2 * cfg.H + R * cfg.I * 4
    dn_bytes = touched * cfg.H * (cfg.I + 2) + R * 2 * cfg.I + R * cfg.H * 4

    def roof(flops, nbytes, ms):
        floor_s = max(flops / (BF16_MFMA_PEAK_TFLOPS * 1e12), nbytes / (HBM_PEAK_GBS * 1e9))
        return round(floor_s / (ms * 1e-3), 4)

    return {
        "workload": "c4: T=4096 H=2048 E=512 top-10 softmax (Zipf 1.2) I=512 int8 + shared I=512",
        "layer_us": round(layer_ms * 1e3, 1),
        "layer_tflops": round((routed_flops + shared_flops) / (layer_ms * 1e-3) / 1e12, 2),
        "experts_touched": touched,
        "layer_hbm_gbs": round(layer_bytes / (layer_ms * 1e-3) / 1e9, 1),
        "gate_up_gemm_us": round(gu_ms * 1e3, 1),
        "gate_up_gemm_tflops": round(gu_flops / (gu_ms * 1e-3) / 1e12, 2),
        "down_gemm_us": round(dn_ms * 1e3, 1),
        "down_gemm_tflops": round(dn_flops / (dn_ms * 1e-3) / 1e12, 2),
        "gemm_arithmetic": "int8 MFMA on two int8 activation limbs per row (2 passes, the cost of one bf16 pass); FLOP/s algorithmic, against the bf16 dense peak",
        "mfma_peak_tflops": BF16_MFMA_PEAK_TFLOPS,
        "gate_up_mfma_frac": round(gu_flops / (gu_ms * 1e-3) / 1e12 / BF16_MFMA_PEAK_TFLOPS, 4),
        "down_mfma_frac": round(dn_flops / (dn_ms * 1e-3) / 1e12 / BF16_MFMA_PEAK_TFLOPS, 4),
        "gate_up_gemm_bytes": int(gu_bytes),
        "gate_up_gemm_hbm_frac": round(gu_bytes / (gu_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "down_gemm_bytes": int(dn_bytes),
        "down_gemm_hbm_frac": round(dn_bytes / (dn_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "gate_up_roofline_frac": roof(gu_flops, gu_bytes, gu_ms),
        "down_roofline_frac": roof(dn_flops, dn_bytes, dn_ms),
        "roofline_note": "every one of the 512 experts is touched under Zipf(1.2) routing, so the GEMMs "
                         "stream 1.07 GB (gate_up) and 0.54 GB (down) of int8 weights: the roofline "
                         "time is max(FLOP time at 2.5 PF, byte time at 8 TB/s), and the byte time "
                         "is the larger one",
    }


def edges_bench(dev, stream, reps=20):
    """The steps either side of the path, on C4 / C2 shapes: the fused
    combine + residual + RMSNorm after it, the residual RMSNorm that feeds
    the router, and the ingestion of one C2 layer's GPTQ experts."""
    from grimoire_amd import ingest
    cfg = configs.CONFIGS["c4"]
    T, K, H = cfg.T, cfg.K, cfg.H
    R = T * K
    g = torch.Generator(device=dev).manual_seed(5)
    routed = torch.randn(R, H, device=dev, generator=g).bfloat16().view(torch.int16)
    inverse = torch.randperm(R, device=dev, generator=g).int()
    rw = torch.rand(R, device=dev, generator=g)
    h = torch.randn(T, H, device=dev, generator=g)
    shared = torch.randn(T, H, device=dev, generator=g)
    r1 = torch.randn(T, H, device=dev, generator=g)
    w = torch.randn(H, device=dev, generator=g).bfloat16().view(torch.int16)
    out = torch.empty(T, H, device=dev)
    out_bf = torch.empty(T, H, dtype=torch.int16, device=dev)
    res = {}
    with torch.cuda.stream(stream):
        def timed(fn):
            fn()
            torch.cuda.synchronize()
            with Timer(stream) as t:
                for _ in range(reps):
                    fn()
            return t.ms() / reps
        ms = timed(lambda: ops.launch_rmsnorm_moe_residual_batched(
            h, routed, inverse, rw, shared, w, out, out_bf, T, K, H, 1e-6, stream=stream))
        nbytes = R * H * 2 + R * 8 + 4 * T * H * 4 + T * H * 2 + H * 2
        res["combine_rmsnorm_residual"] = {
            "shape": f"T={T} K={K} H={H}, bf16 routed rows, fp32 shared, fp32 + bf16 out",
            "us": round(ms * 1e3, 1), "bytes": nbytes,
            "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        ms = timed(lambda: ops.launch_rmsnorm_residual_batched(
            h, shared, r1, w, out, T, H, 1e-6, out_bf=out_bf, stream=stream))
        nbytes = 5 * T * H * 4 + T * H * 2 + H * 2
        res["rmsnorm_residual"] = {
            "shape": f"T={T} H={H}, two fp32 residuals, fp32 + bf16 out",
            "us": round(ms * 1e3, 1), "bytes": nbytes,
            "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        c2 = configs.CONFIGS["c2"]
        E, H2, I, grp = c2.E, c2.H, c2.I, 128

        def proj(out_f, in_f):
            return ingest.gptq(
                torch.randint(-2 ** 31, 2 ** 31 - 1, (in_f // 8, out_f), dtype=torch.int32,
                              device=dev, generator=g),
                torch.full((in_f // grp, out_f // 8), 0x77777777, dtype=torch.int32, device=dev),
                (torch.rand(in_f // grp, out_f, device=dev, generator=g) * 0.02).half()
                .view(torch.int16), grp)
        experts = [(proj(I, H2), proj(I, H2), proj(H2, I)) for _ in range(E)]
        gu, dn = ingest.ingest_experts(experts, dev, stream=stream)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        with Timer(stream) as t:
            for _ in range(3):
                ingest.ingest_experts(experts, dev, stream=stream)
        ms = t.ms() / 3
        host_ms = (time.perf_counter() - t0) * 1e3 / 3
        src_bytes = sum(p.weight.numel() * 4 + p.zeros.numel() * 4 + p.scales.numel() * 2
                        for tr in experts for p in tr)
        dst_bytes = gu.nbytes() + dn.nbytes()
        res["ingest_gptq_layer"] = {
            "shape": f"c2 layer: {E} experts x (gate, up [{I}x{H2}], down [{H2}x{I}]) GPTQ g{grp} "
                     "-> INT4 bf16 scales, device-resident sources",
            "ms": round(ms, 3), "host_ms": round(host_ms, 3), "bytes": src_bytes + dst_bytes,
            "gbs": round((src_bytes + dst_bytes) / (ms * 1e-3) / 1e9, 1),
            "note": "two batched calls (gate+up, down), 64 GPTQ projections per launch"}
        res["tiered_nvfp4"] = _tiered_bench(dev, stream, timed)
    return res


def _tiered_bench(dev, stream, timed):
    """Tiered NVFP4 experts at C2 shapes (H=2048, I=768, top-8 of 128): one
    token's gate_up and down with every block in device memory, then with
    every block in pinned host memory (read over PCIe)."""
    from grimoire_amd import tiered
    H, I, K, E = 2048, 768, 8, 128
    lay = tiered.layout(H, I)
    g = torch.Generator(device=dev).manual_seed(9)
    blocks = [torch.randint(0, 256, (lay.bytes,), dtype=torch.uint8, device=dev, generator=g)
              for _ in range(E)]
    for b in blocks:   # E4M3 scales 0x30..0x3F, projection scales 1
        b[lay.gu_s:lay.gsc].copy_(0x30 + (b[lay.gu_s:lay.gsc] & 15))
        b[lay.gsc:lay.gsc + 16].copy_(torch.tensor([1.0, 1.0, 1.0, 0.0]).view(torch.uint8))
    ex = torch.tensor([[3, 17, 40, 55, 77, 90, 101, 127]], dtype=torch.int32, device=dev)
    w = torch.full((1, K), 1.0 / K, device=dev)
    x = torch.randn(1, H, device=dev, generator=g)
    h = torch.empty(1, K * I, device=dev)
    y = torch.empty(1, H, device=dev)
    gu_bytes = K * 2 * I * (H // 2 + H // 16)
    dn_bytes = K * H * (I // 2 + I // 16)
    out = {"shape": f"T=1 H={H} I={I} top-{K} of {E}, NVFP4 blocks of {lay.bytes} B"}
    for tier in ("vram", "pinned_host"):
        bl = blocks if tier == "vram" else [b.cpu().pin_memory() for b in blocks]
        L = tiered.TieredLayer(H, I, K, bl, dev)
        gu_ms = timed(lambda: L.gate_up(ex, x, h, stream=stream))
        dn_ms = timed(lambda: L.down(ex, w, h, y, stream=stream))
        out[tier] = {"gate_up_us": round(gu_ms * 1e3, 1),
                     "gate_up_gbs": round(gu_bytes / (gu_ms * 1e-3) / 1e9, 1),
                     "down_us": round(dn_ms * 1e3, 1),
                     "down_gbs": round(dn_bytes / (dn_ms * 1e-3) / 1e9, 1)}
    # the host pool on the same token with the blocks in host memory: the
    # whole FFN (gate_up + SwiGLU + down + weighted sum) on the host cores
    # (each call routes to the next 8 of the 128 blocks, 340 MB in all, so
    # the blocks come from DRAM, not from the last-level cache)
    hb = [b.cpu() for b in blocks]
    wh, xh, yh = w[0].cpu().contiguous(), x[0].cpu().contiguous(), torch.empty(H)
    threads = min(16, len(os.sched_getaffinity(0)))
    cx = tiered.CpuExperts(threads)
    sels = [[hb[(8 * c + j) % E] for j in range(K)] for c in range(E // K)]
    for c in range(E // K):
        cx.ffn(lay, sels[c], wh, xh, yh)
    n, t0 = 0, time.perf_counter()
    while n < 400 and time.perf_counter() - t0 < 2.0:
        cx.ffn(lay, sels[n % len(sels)], wh, xh, yh)
        n += 1
    ffn_us = (time.perf_counter() - t0) / n * 1e6
    out["cpu_pool"] = {"threads": threads, "ffn_us": round(ffn_us, 1),
                       "gbs": round((gu_bytes + dn_bytes) / (ffn_us * 1e-6) / 1e9, 1),
                       "note": "grimoire_cpu_experts_ffn, blocks in host memory (rotating over all 128), host threads"}
    return out


def _host_info():
    info = {"os_cpu_count": os.cpu_count()}
    try:
        info["affinity_cpus"] = len(os.sched_getaffinity(0))
    except Exception:  # pragma: no cover
        pass
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                info["model"] = line.split(":", 1)[1].strip()
                break
    except Exception:  # pragma: no cover
        pass
    return info


def _omp_threads():
    n = os.environ.get("OMP_NUM_THREADS")
    if n and n.isdigit():
        return int(n)
    try:
        return len(os.sched_getaffinity(0))
    except Exception:  # pragma: no cover
        return os.cpu_count() or 1


def cpu_baseline(d, budget_s=12.0):
    """The CPU path on the host cores: this build's C restatement of
    src/moe_ref.cpp (oracle/moe_oracle.c, OpenMP over tokens) on all the
    threads OpenMP is given, one C2 token per thread (the layer's own
    routing), as whole-host GB/s of the decode metric; beside it the
    reference's own moe_ref.cpp (oracle/_ref), single thread."""
    try:
        from oracle import oracle as O
    except Exception as e:  # pragma: no cover
        return {"error": f"oracle unavailable: {e}"}
    cfg = d["cfg"]
    x = d["x"].cpu()
    L0 = d["layers"][0]
    Lc = L0.to("cpu")                         # host copy of the layer: not timed
    s = Lc.struct()
    e1, w1 = d["oes"][0].cpu().contiguous(), d["ows"][0].cpu().contiguous()
    one_bytes = (len(set(e1.flatten().tolist())) * L0.expert_bytes() + cfg.E * cfg.H * 4
                 + 2 * cfg.H * 4)
    nt = _omp_threads()
    xs = x.repeat(nt, 1).contiguous()
    es, ws = e1.repeat(nt, 1).contiguous(), w1.repeat(nt, 1).contiguous()
    ys = torch.empty(nt, cfg.H)
    O.orc().orc_moe_forward(O.byref(s), O._p(es), O._p(ws), None, O._p(xs), O._p(ys), nt)
    calls, dt = 0, 0.0
    while dt < budget_s and calls < 200:
        t0 = time.perf_counter()
        O.orc().orc_moe_forward(O.byref(s), O._p(es), O._p(ws), None, O._p(xs), O._p(ys), nt)
        dt += time.perf_counter() - t0
        calls += 1
    out = {"value": round(nt * calls * one_bytes / dt / 1e9, 4), "unit": "GB/s", "cores": nt,
           "kind": "port",
           "sample": f"layer 0 of the C2 step, {nt} copies of its token (one per OpenMP "
                     f"thread), {calls} calls ({dt:.1f} s); value = tokens x the one-token "
                     f"layer's algorithmic bytes / time",
           "us_per_token_layer": round(dt / (calls * nt) * 1e6, 1),
           "host": _host_info()}
    r = O.ref()
    if r is not None:
        y = torch.empty(1, cfg.H)
        done, dt1 = 0, 0.0
        while dt1 < budget_s / 2 and done < 100:
            t0 = time.perf_counter()
            r.ref_moe_forward(O.byref(s), O._p(e1), O._p(w1), O._p(x), O._p(y), 1)
            dt1 += time.perf_counter() - t0
            done += 1
        out["reference_single_thread"] = {
            "value": round(done * one_bytes / dt1 / 1e9, 4), "unit": "GB/s", "cores": 1,
            "kind": "reference", "us_per_layer": round(dt1 / done * 1e6, 1),
            "sample": f"src/moe_ref.cpp built into oracle/_ref, layer 0, {done} calls"}
    return out


def _touched_bytes(L, oe):
    return len(set(oe.flatten().tolist())) * L.expert_bytes() + L.shared_bytes()


def c3_bench(dev, stream, n_layers=4, reps=10, regime=0, padded=True):
    """C3 (T=8 users, H=2880, E=128, top-4 softmax with Zipf(1.1)
    popularity, I=2880, MXFP4): the forward of n_layers distinct layers in
    one graph (their touched experts exceed the 256 MB MALL).  regime 0 is
    what the forward picks (the matrix-core expert-grouped GEMV); regime 1,
    the per-route decode kernels, is reported beside it.  padded: the
    experts' MXFP4 rows padded once at load to 3072 elements
    (MoeLayer.pad_mxfp4 / grimoire_moe_pad_mxfp4_rows: whole memory lines
    per streamed piece, the same outputs bit for bit); bytes and GB/s are
    the unpadded rows' either way."""
    cfg = configs.CONFIGS["c3"]
    base = [configs.make_layer(cfg, dev, seed=300 + i) for i in range(n_layers)]
    layers = [L.pad_mxfp4() for L in base] if padded else base
    bias = configs.make_route_bias(cfg, dev, seed=3)
    x = configs.make_x(cfg, dev, seed=3)
    fwds = [ops.MoeForward(L, cfg.T, configs.route_params(cfg, bias), regime=regime) for L in layers]
    ys = [torch.empty(cfg.T, cfg.H, device=dev) for _ in layers]
    oes = [torch.empty(cfg.T, cfg.K, dtype=torch.int32, device=dev) for _ in layers]
    ows = [torch.empty(cfg.T, cfg.K, dtype=torch.float32, device=dev) for _ in layers]

    def step():
        for f, y, oe, ow in zip(fwds, ys, oes, ows):
            f(x, y, oe, ow, stream=stream)

    with torch.cuda.stream(stream):
        step()
    torch.cuda.synchronize()
    g = _graph(step, stream)
    _replay(g, stream, 3)
    torch.cuda.synchronize()
    with Timer(stream) as t:
        _replay(g, stream, reps)
    us = t.ms() * 1e3 / (reps * n_layers)
    nbytes = sum(_touched_bytes(L, oe.cpu()) for L, oe in zip(base, oes)) / n_layers
    nbytes += cfg.E * cfg.H * 4 + 2 * cfg.T * cfg.H * 4
    touched = sum(len(set(oe.cpu().flatten().tolist())) for oe in oes) / n_layers
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"workload": "c3: T=8 H=2880 E=128 top-4 softmax (Zipf 1.1) I=2880 MXFP4, "
                        f"{n_layers} distinct layers in one graph",
            "regime": ["chosen by the forward (expert-grouped GEMV, matrix core)", "per-route decode kernels"][
                min(regime, 1)],
            "weight_rows": "padded to 3072 elements at load" if padded else "packed (the reference's layout)",
            "us_per_layer": round(us, 2), "experts_touched": touched,
            "bytes_per_layer": int(nbytes), "gbs": round(gbs, 1),
            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "tflops": round(6.0 * cfg.T * cfg.K * cfg.H * cfg.I / (us * 1e-6) / 1e12, 3)}


def c5_bench(dev, stream, reps=5):
    """C5 (T=32, H=7168, 256 routed + 1 shared expert, I=2048, MXFP4,
    group-limited sigmoid top-8, scaling 2.5): the whole layer forward as
    the forward picks it (the matrix-core expert-grouped GEMV), launched
    eagerly (a captured graph of it replays slower: 788 vs 763 us)."""
    cfg = configs.CONFIGS["c5"]
    L = configs.make_layer(cfg, dev, seed=500)
    bias = configs.make_route_bias(cfg, dev, seed=5)
    x = configs.make_x(cfg, dev, seed=5)
    fwd = ops.MoeForward(L, cfg.T, configs.route_params(cfg, bias), regime=0)
    y = torch.empty(cfg.T, cfg.H, device=dev)
    oe = torch.empty(cfg.T, cfg.K, dtype=torch.int32, device=dev)
    ow = torch.empty(cfg.T, cfg.K, dtype=torch.float32, device=dev)
    with torch.cuda.stream(stream):
        fwd(x, y, oe, ow, stream=stream)
        torch.cuda.synchronize()
        with Timer(stream) as t:
            for _ in range(reps):
                fwd(x, y, oe, ow, stream=stream)
    us = t.ms() * 1e3 / reps
    nbytes = _touched_bytes(L, oe.cpu()) + cfg.E * cfg.H * 4 + 2 * cfg.T * cfg.H * 4
    flops = 6.0 * cfg.T * (cfg.K + 1) * cfg.H * cfg.I
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"workload": "c5: T=32 H=7168 E=256+1 shared, group-limited sigmoid top-8 "
                        "(8 groups, top-4 groups, bias, scaling 2.5) I=2048 MXFP4",
            "us_per_layer": round(us, 1), "experts_touched": len(set(oe.cpu().flatten().tolist())),
            "bytes_per_layer": int(nbytes), "gbs": round(gbs, 1),
            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "tflops": round(flops / (us * 1e-6) / 1e12, 2),
            "bound": "hbm (intensity ~6.6 FLOP/B, far below the ~315 FLOP/B bf16 ridge)"}


def c5_shard_bench(dev, stream, reps=10, begin=96, count=32):
    """One GPU's share of C5 under 8-way expert parallelism
    (grimoire_moe_forward_shard): the global router and group-limited top-k
    over all 256 experts, experts [96, 128) local, routes to others masked;
    no shared expert on this shard.  Bytes = the local experts the routing
    touches + the global router + x + y."""
    from grimoire_amd.weights import MoeLayer
    cfg = configs.CONFIGS["c5"]
    loc = configs.make_layer(configs.scaled(cfg, E=count), dev, seed=510)
    g = torch.Generator(device=dev).manual_seed(510)
    router = (torch.randn((cfg.E, cfg.H), generator=g, device=dev) * 0.02).contiguous()
    L = MoeLayer(cfg.H, cfg.I, cfg.E, cfg.K, loc.gate_up, loc.down, router)
    bias = configs.make_route_bias(cfg, dev, seed=5)
    x = configs.make_x(cfg, dev, seed=5)
    fwd = ops.MoeForward(L, cfg.T, configs.route_params(cfg, bias), regime=0)
    y = torch.empty(cfg.T, cfg.H, device=dev)
    oe = torch.empty(cfg.T, cfg.K, dtype=torch.int32, device=dev)
    ow = torch.empty(cfg.T, cfg.K, dtype=torch.float32, device=dev)
    with torch.cuda.stream(stream):
        fwd.shard(x, y, begin, count, oe, ow, stream=stream)
        torch.cuda.synchronize()
        with Timer(stream) as t:
            for _ in range(reps):
                fwd.shard(x, y, begin, count, oe, ow, stream=stream)
    us = t.ms() * 1e3 / reps
    e = oe.cpu().flatten()
    local = sorted(set(int(v) for v in e.tolist() if begin <= v < begin + count))
    nbytes = len(local) * loc.expert_bytes() + cfg.E * cfg.H * 4 + 2 * cfg.T * cfg.H * 4
    routes = int(((e >= begin) & (e < begin + count)).sum())
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"workload": f"c5 shard: experts [{begin}, {begin + count}) of 256 local (8-way expert "
                        "parallelism, one GPU's share), T=32 H=7168 I=2048 MXFP4, global group-limited "
                        "routing, no shared expert",
            "us_per_layer": round(us, 1), "local_routes": routes, "local_experts_touched": len(local),
            "bytes_per_layer": int(nbytes), "gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run a 64 MiB device copy 5 times (HBM counter calibration)")
    ap.add_argument("--only", choices=("c3", "c4", "c5", "c5_shard", "edges"),
                    help="run only this workload's section and print it alone (for profiling runs)")
    ap.add_argument("--decode-regime", type=int, default=1, choices=(1, 3, 7),
                    help="1: router logits, gate_up (with the top-k), down; "
                         "3: router logits, top-k, gate_up, down as four launches; "
                         "7: the whole layer in one launch")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(expert parallelism is a design note, not code).", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    _abi.lib()
    stream = torch.cuda.Stream()
    if a.copy_probe:
        src = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
    if a.only:
        run = {"c3": lambda: c3_bench(dev, stream), "c4": lambda: prefill_bench(dev, stream),
               "c5": lambda: c5_bench(dev, stream), "c5_shard": lambda: c5_shard_bench(dev, stream),
               "edges": lambda: edges_bench(dev, stream)}[a.only]
        print(json.dumps({"only": a.only, a.only: run()}), flush=True)
        return
    log("decode bench (C2, 48 layers)...")
    d = decode_bench(a.steps, a.warmup, dev, stream, a.decode_regime)
    out = {
        "metric": "MoE decode layer HBM GB/s (T=1, C2, 48 layers back to back)",
        "value": round(d["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(d["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights (fp16 group scales), fp32 accumulate",
        "data": "synthetic (seeded random weights and activations of the C2 shapes)",
        "config": {"workload": "c2: T=1 H=2048 E=128 top-8 softmax I=768 GPTQ int4 g128, "
                               "48 distinct layers", "layers": LAYERS},
        "us_per_layer": round(d["ms"] * 1e3 / LAYERS, 2),
        "us_per_layer_standalone_mall_hot": round(d["one_us"], 2),
        "hbm_frac": round(d["gbs"] / HBM_PEAK_GBS, 4),
        "roofline": {
            "bound": "hbm",
            "kernel": "grim::moe_gate_up_wave_kernel<64, 6, 1, false> (decode stage 2: top-k + "
                      "gate_up + SwiGLU, GPTQ int4 fp16 scales; 6 row pairs per wave), 48 layers "
                      "in one graph",
            "achieved": round(d["gu_bytes"] / (d["gu_us"] * 1e-6) / 1e9, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(d["gu_bytes"] / (d["gu_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic("moe_gate_up_wave_kernel"),
            "launch_us": round(d["gu_us"], 3),
            "bytes_per_launch": int(d["gu_bytes"]),
        },
    }
    if a.decode_regime == 1:
        log("one-launch decode (regime 7) on the same layers...")
        out["c2_one_launch"] = decode_one_launch(d, dev, stream, a.steps)
    if not a.no_prefill:
        log("prefill bench (C4)...")
        out["prefill"] = prefill_bench(dev, stream)
    if not a.no_prefill:
        log("C3 (T=8 MXFP4 decode) and C5 (T=32 verify, 6 GB of experts)...")
        out["c3"] = c3_bench(dev, stream)
        out["c3_packed_rows"] = c3_bench(dev, stream, padded=False)
        out["c3_decode_kernels"] = c3_bench(dev, stream, regime=1)
        out["c5"] = c5_bench(dev, stream)
        out["c5_shard"] = c5_shard_bench(dev, stream)
        log("edges (fused norms, ingestion)...")
        out["edges"] = edges_bench(dev, stream)
    if not a.no_cpu:
        log("cpu baseline...")
        out["cpu_baseline"] = cpu_baseline(d)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
