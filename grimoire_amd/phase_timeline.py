"""Phase timelines from the GRIM_TIMING build: the decode layer (C2: T = 1,
top-8 of 128 GPTQ int4 experts, I = 768; the default) and the waves of the
matrix-core grouped GEMV on C3 (--c3).

    python -m grimoire_amd.build --timing
    python -m grimoire_amd.phase_timeline [--layers 8] [--reps 5]
    python -m grimoire_amd.phase_timeline --c3 [--layers 4] [--reps 5]

The three-launch forward (router; gate_up with the top-k; down with the
combine) runs on distinct layers, one token each.  Thread 0 of every
work-group stamps the real-time counter (100 MHz, 10 ns) at the phase
boundaries of its kernel; the table gives, per phase, the earliest /
median / latest work-group's stamp in µs from the first router
work-group's start, as the median over the timed layer calls.  Phases:

    router   start, end (its row of logits stored)
    gate_up  start; routing done (logits read, top-k ranks formed, the
             slot's expert known); weights issued (every payload, scale
             and zero-point load of the work-group's rows requested);
             dots done; end (h stored)
    down     start; h and routes in; weights issued; dots done; end
             (slot-order combine stored)

The stamps cost a store each and sit on the timing build only.

--c3: C3 (T = 8, top-4 of 128 MXFP4 experts, H = I = 2880, rows padded to
3072) through the forward's grouped GEMV, distinct layers in turn.  Lane 0
of every wave of the two launches (gate_up, down; 1024 waves each) stamps
its start, its first stage's arrival and the end of each of its items;
per stamp the earliest / 10th percentile / median / 90th percentile /
latest wave in µs from gate_up's first wave, median over the calls, and
how many waves had one, two, ... items.
"""
from __future__ import annotations

import argparse
import ctypes as C
from pathlib import Path

import numpy as np
import torch

from . import _abi, configs, ops

TIMING_LIB = Path(__file__).resolve().parent / "_timing" / "libgrimoire_moe.so"

PHASES = [
    (0, "router", [(0, "start"), (1, "end")], 128),
    (1, "gate_up", [(0, "start"), (1, "routing done"), (2, "weights issued"), (3, "dots done"), (4, "end")], 256),
    (2, "down", [(0, "start"), (1, "h and routes in"), (2, "weights issued"), (3, "dots done"), (4, "end")], 256),
]


def c3_waves(lib, dev, n_layers, reps):
    """The grouped GEMV's wave stamps on C3 (gemv_mx.hip's GVM_TS: 16 per
    wave, gate_up at [0, 1024 * 16), down from 4096 * 16)."""
    ts = torch.zeros(2 * 4096 * 16, dtype=torch.int64, device=dev)
    lib.grim_timing_set(ts.data_ptr())
    cfg = configs.CONFIGS["c3"]
    calls = []
    for i in range(n_layers):
        wl = configs.make_workload(cfg, dev, seed=11 + i)
        bias = wl.route_bias
        fw = ops.MoeForward(wl.layer.pad_mxfp4(), cfg.T, configs.route_params(cfg, bias), regime=0)
        calls.append((fw, wl.x, bias))
    y = torch.empty(cfg.T, cfg.H, device=dev)
    rows, hist = {}, {}
    labels = [(0, "start"), (1, "first stage in"), (2, "item 0 end"), (3, "item 1 end"), (15, "exit")]
    for rep in range(reps + 1):
        for fw, x, _bias in calls:
            ts.zero_()
            torch.cuda.synchronize()
            fw(x, y)
            torch.cuda.synchronize()
            if rep == 0:
                continue                      # warm-up pass over the layers
            t = ts.view(2, 4096, 16)[:, :1024].cpu().numpy().astype(np.int64)
            base = t[0, :, 0][t[0, :, 0] > 0].min()
            for role, name in ((0, "gate_up"), (1, "down")):
                tt = t[role][t[role][:, 0] > 0]
                for i, label in labels:
                    v = tt[:, i]
                    v = (v[v > 0] - base) * 10 / 1e3
                    if len(v):
                        rows.setdefault((name, label), []).append(
                            [v.min(), np.percentile(v, 10), np.median(v), np.percentile(v, 90), v.max()])
                n_items = (tt[:, 2:15] > 0).sum(1)
                hist.setdefault(name, []).append(np.bincount(n_items, minlength=4)[:4])
    print(f"C3 grouped GEMV waves, {n_layers} distinct layers x {reps} calls; µs from gate_up's first wave "
          "(median over calls)")
    print("| launch | stamp | earliest | 10% | median | 90% | latest |")
    print("|---|---|---:|---:|---:|---:|---:|")
    for (name, label), v in rows.items():
        r = np.median(np.array(v), axis=0)
        print(f"| {name} | {label} | " + " | ".join(f"{x:.2f}" for x in r) + " |")
    for name, h in hist.items():
        m = np.median(np.array(h), axis=0).astype(int)
        print(f"{name}: waves with 0 / 1 / 2 / 3 items: {' / '.join(str(x) for x in m)}")


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--layers", type=int, default=None)
    ap.add_argument("--reps", type=int, default=5)
    ap.add_argument("--c3", action="store_true", help="the C3 grouped GEMV's waves instead of the C2 decode")
    a = ap.parse_args(argv)
    if not TIMING_LIB.exists():
        raise SystemExit(f"{TIMING_LIB} is missing: python -m grimoire_amd.build --timing")
    _abi._lib = None
    _abi.LIB_PATH = TIMING_LIB
    lib = _abi.lib()
    dev = torch.device("cuda:0")
    lib.grim_timing_set.argtypes = [C.c_void_p]
    if a.c3:
        c3_waves(lib, dev, a.layers or 4, a.reps)
        return
    a.layers = a.layers or 8
    # stamp buffer: 3 roles x 2048 work-groups x 8 stamps (the GEMM regimes'
    # stamps, further on, are not used here)
    ts = torch.zeros(3 * 2048 * 8 + 4096 * 16 * 2, dtype=torch.int64, device=dev)
    lib.grim_timing_set.argtypes = [C.c_void_p]
    lib.grim_timing_set(ts.data_ptr())
    cfg = configs.CONFIGS["c2"]
    layers = [configs.make_layer(cfg, dev, seed=100 + i) for i in range(a.layers)]
    x = configs.make_x(cfg, dev, seed=7)
    fw = [ops.MoeForward(L, 1, configs.route_params(cfg, None), regime=1) for L in layers]
    y = torch.empty(1, cfg.H, device=dev)
    rows = {}
    for rep in range(a.reps + 1):
        for f in fw:
            ts.zero_()
            f(x, y)
            torch.cuda.synchronize()
            if rep == 0:
                continue                      # warm-up pass over the layers
            t = ts[:3 * 2048 * 8].view(3, 2048, 8).cpu().numpy().astype(np.int64)
            base = t[0, :128, 0].min()
            for role, name, stamps, nwg in PHASES:
                for i, label in stamps:
                    v = (t[role, :nwg, i] - base) * 10      # ns
                    v = v[t[role, :nwg, i] > 0]
                    rows.setdefault((name, label), []).append((v.min(), np.median(v), v.max()))
    print(f"C2 decode layer, {a.layers} distinct layers x {a.reps} calls, three launches; "
          "µs from the first router work-group's start (median over calls)")
    print("| kernel | phase | earliest | median | latest |")
    print("|---|---|---:|---:|---:|")
    for role, name, stamps, nwg in PHASES:
        for i, label in stamps:
            r = np.median(np.array(rows[(name, label)]), axis=0) / 1e3
            print(f"| {name} | {label} | {r[0]:.2f} | {r[1]:.2f} | {r[2]:.2f} |")


if __name__ == "__main__":
    main()
