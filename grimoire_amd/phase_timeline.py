"""Phase timeline of the decode layer (C2: T = 1, top-8 of 128 GPTQ int4
experts, I = 768) from the GRIM_TIMING build.

    python -m grimoire_amd.build --timing
    python -m grimoire_amd.phase_timeline [--layers 8] [--reps 5]

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


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--reps", type=int, default=5)
    a = ap.parse_args(argv)
    if not TIMING_LIB.exists():
        raise SystemExit(f"{TIMING_LIB} is missing: python -m grimoire_amd.build --timing")
    _abi._lib = None
    _abi.LIB_PATH = TIMING_LIB
    lib = _abi.lib()
    dev = torch.device("cuda:0")
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
