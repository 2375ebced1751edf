#!/usr/bin/env python3
"""Phase trace of the small-M stream kernel of the int4 prefill product (mm_int4_stream_kernel, M <= 48).

    python rumik-fast_amd/mm_stream_trace.py build        # CPU: lib/librumik_stream_trace.so (-DRK_STREAM_TRACE)
    python rumik-fast_amd/mm_stream_trace.py run          # GPU: a markdown table per shape

The traced library is mm_int4.hip built with RK_STREAM_TRACE: the same kernel with wall-clock stamps (100 MHz) per
(block, wave, event) kept in scalar registers and stored at the end of the launch (the product library compiles
them out). `run` launches rk_mm_int4_g128_ws eagerly over 8 rotated weight copies per shape, three rounds, and
reports per event the median and 90th percentile over blocks and waves of the last 8 launches (us since the
launch's first block started), the median over launches of the latest stamp, and the launch's HIP-event time.
"""
import ctypes
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB = PKG / "lib" / "librumik_stream_trace.so"
EVENTS = ["start", "prologue loads issued", "X fragments and row sums", "tables in LDS (barrier)",
          "tile 0 computed", "tile 0 reduced (barrier)", "tile 1 computed", "tile 1 reduced (barrier)",
          "last tile computed", "last tile reduced (barrier)", "loop done", "stores issued", "stores complete"]
SHAPES = ((34, 22016, 2048), (16, 22016, 2048), (48, 22016, 2048), (34, 25088, 2048), (34, 3072, 2048))


def build():
    sys.path.insert(0, str(PKG))
    import build as B
    LIB.parent.mkdir(exist_ok=True)
    cmd = [B.HIPCC, *B.FLAGS, "-DRK_STREAM_TRACE", "-shared", str(B.CSRC / "mm_int4.hip"), "-o", str(LIB)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise SystemExit(r.stderr)
    print(f"[stream_trace] built {LIB}", flush=True)


def run(copies=8, rounds=3):
    import numpy as np
    sys.path.insert(0, str(PKG / "kernels"))
    import torch
    import synth
    import _hiplib as H
    lib = ctypes.CDLL(str(LIB))
    _p, _i = ctypes.c_void_p, ctypes.c_int
    lib.rk_stream_trace_set.argtypes = [_p]
    lib.rk_mm_int4_workspace_bytes.argtypes = [_i, _i, _i]
    lib.rk_mm_int4_workspace_bytes.restype = ctypes.c_size_t
    lib.rk_mm_int4_g128_ws.argtypes = [_p, _i, _i, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p, ctypes.c_size_t, _p]
    dev = torch.device("cuda:0")
    st = H.stream(dev)
    stream = torch.cuda.current_stream(dev)
    for M, N, K in SHAPES:
        assert H.mm_plan(M, N, K)[0] == H.MM_STREAM, (M, N, K)
        gen = synth.generator(1, "cuda")
        mats = [synth.int4_weights(N, K, gen, device=dev) for _ in range(copies)]
        X = torch.randn(M, K, device=dev, generator=gen).half()
        Y = torch.empty(M, N, device=dev, dtype=torch.float16)
        nws = lib.rk_mm_int4_workspace_bytes(M, N, K)
        ws = torch.empty(max(nws, 16), device=dev, dtype=torch.uint8)
        nb = 512  # at least the grid (<= 256 blocks per K chunk layout, one block per CU)
        bufs = [torch.zeros(nb * 8 * 16, dtype=torch.int64, device=dev) for _ in range(copies)]
        ev = []
        for _ in range(rounds):
            for (q, s, m), buf in zip(mats, bufs):
                assert lib.rk_stream_trace_set(buf.data_ptr()) == 0
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                r = lib.rk_mm_int4_g128_ws(H.ptr(X), H.F16, K, H.ptr(q), H.ptr(s), H.ptr(m), H.ptr(Y), H.F16, N, M, N,
                                           K, H.ptr(ws), nws, st)
                e1.record(stream)
                assert r == 0, r
                ev.append((e0, e1))
        torch.cuda.synchronize()
        us = sorted(a.elapsed_time(b) * 1e3 for a, b in ev[-copies:])
        launches = []
        for buf in bufs:
            t = buf.view(nb, 8, 16).cpu().numpy().astype(np.float64)
            used = t[:, 0, 0] > 0
            t = t[used]
            launches.append(np.where(t == 0, np.nan, (t - t[:, :, 0].min()) / 100.0))
        A = np.stack(launches)  # [launch, block, wave, event]
        print(f"\n### M={M} N={N} K={K}: {A.shape[1]} blocks, HIP-event time per launch {us[len(us) // 2]:.2f} us "
              f"(median of the last {copies})\n")
        print("| event | median | p90 | latest (median over launches) |\n|---|---|---|---|")
        for e, name in enumerate(EVENTS):
            v = A[:, :, :, e]
            if np.all(np.isnan(v)):
                continue
            print(f"| {name} | {np.nanmedian(v):.2f} | {np.nanpercentile(v, 90):.2f} | "
                  f"{np.nanmedian(np.nanmax(v, axis=(1, 2))):.2f} |", flush=True)
        del mats, bufs
        torch.cuda.empty_cache()


if __name__ == "__main__":
    if len(sys.argv) >= 2 and sys.argv[1] == "build":
        build()
    elif len(sys.argv) >= 2 and sys.argv[1] == "run":
        run()
    else:
        raise SystemExit(__doc__)
