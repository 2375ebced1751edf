#!/usr/bin/env python3
"""Phase trace of the one-launch layer projections (rk_gemv_int4_g128_layer, config 1's four projections).

    python rumik-fast_amd/layer_trace.py build        # CPU: lib/librumik_layer_trace.so (-DRK_LAYER_TRACE)
    python rumik-fast_amd/layer_trace.py run          # GPU: a markdown table of the phases

The traced library is gemv_layer.hip built with RK_LAYER_TRACE: the same kernel with wall-clock stamps per (block,
wave, event) kept in registers and stored at the end of the launch (the product library compiles them out). `run`
launches it eagerly over 16 rotated weight copies of the config-1 layer (so no launch is served from the Infinity
Cache), three rounds, and reports per event and wave role the median and 90th percentile over blocks, waves and the
last 12 launches of the time since the launch's first block started, and the median over launches of the latest
stamp.
"""
import ctypes
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB = PKG / "lib" / "librumik_layer_trace.so"
EVENTS = ["start", "x and tables in LDS", "gate / up done, act published", "streams done (phase 1)",
          "phase 2 start (down waves)", "act chunk in registers (down waves)", "down rows done (down waves)", "end"]
ROLES = (("down waves (2..7)", slice(2, 8)), ("q/o waves (0, 1)", slice(0, 2)))


def build():
    sys.path.insert(0, str(PKG))
    import build as B
    LIB.parent.mkdir(exist_ok=True)
    cmd = [B.HIPCC, *B.FLAGS, "-DRK_LAYER_TRACE", "-shared", str(B.CSRC / "gemv_layer.hip"), "-o", str(LIB)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise SystemExit(r.stderr)
    print(f"[layer_trace] built {LIB}", flush=True)


def run(copies=16, rounds=3):
    import numpy as np
    sys.path.insert(0, str(PKG / "kernels"))
    import torch
    import synth
    import _hiplib as H
    lib = ctypes.CDLL(str(LIB))
    _p, _i = ctypes.c_void_p, ctypes.c_int
    lib.rk_layer_trace_set.argtypes = [_p]
    lib.rk_gemv_int4_g128_layer_ws_bytes.argtypes = [_i]
    lib.rk_gemv_int4_g128_layer_ws_bytes.restype = ctypes.c_size_t
    lib.rk_gemv_int4_g128_layer.argtypes = [_p, _p, _i] + [_p] * 13 + [_i, _i, _i, _i, _p, ctypes.c_size_t, _p]
    dev = torch.device("cuda:0")
    nq, inter, hid = 3072, 11008, 2048
    gen = synth.generator(1, "cuda")
    layers = [(synth.int4_weights(nq + 2 * inter, hid, gen, device=dev), synth.int4_weights(hid, hid, gen, device=dev),
               synth.int4_weights(hid, inter, gen, device=dev)) for _ in range(copies)]
    x = torch.randn(hid, device=dev, generator=gen).half()
    ob = torch.randn(hid, device=dev, generator=gen).half()
    outs = [torch.empty(n, device=dev, dtype=torch.float16) for n in (nq, inter, hid, hid)]
    ws = torch.zeros(lib.rk_gemv_int4_g128_layer_ws_bytes(inter) // 4, device=dev, dtype=torch.int32)
    nb = torch.cuda.get_device_properties(dev).multi_processor_count
    bufs = [torch.zeros(nb * 8 * 8, dtype=torch.int64, device=dev) for _ in range(copies)]
    st = H.stream(dev)
    for _ in range(rounds):
        for (w_in, w_o, w_d), buf in zip(layers, bufs):
            assert lib.rk_layer_trace_set(buf.data_ptr()) == 0
            r = lib.rk_gemv_int4_g128_layer(H.ptr(x), H.ptr(ob), H.F16, *(H.ptr(t) for t in w_in + w_o + w_d),
                                            *(H.ptr(t) for t in outs), H.F16, nq, inter, hid, H.ptr(ws),
                                            ws.numel() * 4, st)
            assert r == 0, r
    torch.cuda.synchronize()
    assert int(ws[0].item()) == 0, "an exchange wait ran out"
    launches = []
    for buf in bufs[copies - 12:]:
        t = buf.view(nb, 8, 8).cpu().numpy().astype(np.int64)
        launches.append(np.where(t == 0, np.nan, (t - t[:, :, 0].min()) / 100.0))  # us since the first block
    A = np.stack(launches)  # [launch, block, wave, event]
    print(f"Config 1 layer (q/k/v 3072, gate/up 2 x 11008, o 2048, down 2048 x 11008; fp16), {nb} blocks, eager "
          f"launches over {copies} weight copies; us since the launch's first block started.\n")
    print("| event | role | median | p90 | latest (median over launches) |\n|---|---|---|---|---|")
    for e, name in enumerate(EVENTS):
        for role, ws_ in ROLES:
            v = A[:, :, ws_, e]
            if np.all(np.isnan(v)):
                continue
            print(f"| {name} | {role} | {np.nanmedian(v):.2f} | {np.nanpercentile(v, 90):.2f} | "
                  f"{np.nanmedian(np.nanmax(v, axis=(1, 2))):.2f} |")


if __name__ == "__main__":
    if len(sys.argv) >= 2 and sys.argv[1] == "build":
        build()
    elif len(sys.argv) >= 2 and sys.argv[1] == "run":
        run()
    else:
        raise SystemExit(__doc__)
