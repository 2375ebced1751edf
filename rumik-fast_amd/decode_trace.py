#!/usr/bin/env python3
"""Phase trace of the one-launch decode step (config 4, the full-width 36-layer synthetic model).

    python rumik-fast_amd/decode_trace.py build              # CPU: lib/librumik_decode_trace.so (-DRK_DECODE_TRACE)
    python rumik-fast_amd/decode_trace.py run [CTX ...]      # GPU: a markdown table per context (default 256 1024 2048)

The traced library is decode_persistent.hip built with RK_DECODE_TRACE: the same kernel with wall-clock stamps per
(block, layer, event) kept in LDS and copied out at the end of the step (the product library compiles them out).
`run` drives it with the engine's own parameters (decode.PersistentDecode) for a few steps per context and reports,
per event, the median and 90th percentile over blocks and layers 2 .. L-2 of the time since the previous layer's
last x publication (the moment the slowest block published: every block's next layer needs all of x), and the
median over layers of the slowest block. The layer period is the spacing of those last x publications.
"""
import ctypes
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB = PKG / "lib" / "librumik_decode_trace.so"
EVENTS = ["x polled (row wave 0)", "LayerNorm done (row wave 0)", "h staged (row wave 0)",
          "tile 0 part done (row wave 0)", "q/k/v published (last row wave)", "q polled (attention wave 0)",
          "attention computed (attention wave 0)", "split partial published (attention wave 0)",
          "combine part done (attention wave 0)", "combine merged (attention wave 0)",
          "o partials published (attention wave 0)", "pass 2 start (tile wave W4)", "act ready (last tile wave)",
          "down partials published (down wave W12)", "gather polled (row wave 0)", "x rows published (last row wave)",
          "x polled (row wave 4)", "gather polled (row wave 4)"]


def build():
    sys.path.insert(0, str(PKG))
    import build as B
    LIB.parent.mkdir(exist_ok=True)
    cmd = [B.HIPCC, *B.FLAGS, "-DRK_DECODE_TRACE", "-shared", str(B.CSRC / "decode_persistent.hip"), "-o", str(LIB)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise SystemExit(r.stderr)
    print(f"[decode_trace] built {LIB}", flush=True)


def run(ctxs, steps=4):
    import numpy as np
    sys.path.insert(0, str(PKG / "kernels"))
    sys.path.insert(0, str(PKG / "engine"))
    import torch
    import decode
    lib = ctypes.CDLL(str(LIB))
    lib.rk_decode_trace_set.argtypes = [ctypes.c_void_p]
    lib.rk_decode_step_persistent.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    ne = lib.rk_decode_trace_events()
    assert ne == len(EVENTS), (ne, len(EVENTS))
    dev = torch.device("cuda:0")
    cfg = decode.Config()
    eng = decode.PersistentDecode(cfg, decode.random_weights(cfg, 4, device=dev), device=dev)
    eng.fill_cache(cfg.S, seed=5)
    buf = torch.zeros(eng.nblocks * 64 * ne, dtype=torch.int64, device=dev)
    assert lib.rk_decode_trace_set(ctypes.c_void_p(buf.data_ptr())) == 0
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    L = cfg.L
    print(f"Config 4 (H 2048, 36 layers, GQA 16/4, int4 g128, fp16), {eng.nblocks} blocks; times in us.\n")
    for ctx in ctxs:
        eng.set_state(7, ctx - 1)
        times = []
        for it in range(steps + 2):
            buf.zero_()
            eng.pos.fill_(ctx - 1)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            assert lib.rk_decode_step_persistent(ctypes.byref(eng.params), eng.nblocks, st) == 0
            e1.record()
            torch.cuda.synchronize()
            if eng.status_word() != 0:
                raise SystemExit(f"status {eng.status_word()}")
            times.append(e0.elapsed_time(e1) * 1e3)
        t = buf.view(eng.nblocks, 64, ne).cpu().numpy().astype(np.float64) / 100.0  # the last step's stamps, us
        T0 = [t[:, l, EVENTS.index("x rows published (last row wave)")].max() for l in range(L)]
        per = np.diff(T0[1:L - 1])
        print(f"### ctx {ctx}: step {np.median(times[2:]):.1f} us (traced), layer period median {np.median(per):.2f} "
              f"(min {per.min():.2f}, max {per.max():.2f})\n")
        print("| event | median | p90 | slowest block (median over layers) |\n|---|---|---|---|")
        order = [0, 16, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 17, 14, 15]
        for e in order:
            rel = np.stack([t[:, l, e] - T0[l - 1] for l in range(2, L - 1)])
            valid = np.stack([t[:, l, e] > 0 for l in range(2, L - 1)])
            if not valid.any():
                continue
            vals = rel[valid]
            slow = np.median([rel[i][valid[i]].max() for i in range(rel.shape[0]) if valid[i].any()])
            print(f"| {EVENTS[e]} | {np.median(vals):.2f} | {np.percentile(vals, 90):.2f} | {slow:.2f} |")
        print()


if __name__ == "__main__":
    if len(sys.argv) >= 2 and sys.argv[1] == "build":
        build()
    elif len(sys.argv) >= 2 and sys.argv[1] == "run":
        run([int(c) for c in sys.argv[2:]] or [256, 1024, 2048])
    else:
        raise SystemExit(__doc__)
