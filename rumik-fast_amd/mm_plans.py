"""Time the int4 prefill product's two plans on the benchmark shapes (config 3 and the reference's w_in prompts).

    python rumik-fast_amd/mm_plans.py [--reps 20]

For each shape: rk_mm_int4_g128 (the tile kernels, no workspace) and rk_mm_int4_g128_ws (split-K or the prepared-X
kernel, as rk_mm_int4_plan reports), fp16 X and Y, synthetic seeded inputs, best of 5 bursts of `reps` launches
timed with HIP events on the launching stream. Prints one line per shape and, at the end, one JSON line.
"""
import argparse
import json
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "rumik-fast_amd" / "kernels", ROOT / "rumik-fast_amd" / "engine", ROOT):
    sys.path.insert(0, str(p))

import torch  # noqa: E402

import _hiplib as H  # noqa: E402
import synth  # noqa: E402

SHAPES = ((16, 22016, 2048), (48, 22016, 2048), (34, 25088, 2048), (34, 3072, 2048), (34, 22016, 2048), (34, 2048, 11008), (128, 3072, 2048), (128, 22016, 2048),
          (128, 2048, 11008), (512, 3072, 2048), (512, 22016, 2048), (512, 2048, 11008), (69, 25088, 2048),
          (201, 25088, 2048), (512, 25088, 2048))
NAMES = {H.MM_REGS: "regs", H.MM_TILE128: "tile128", H.MM_TILE64: "tile64", H.MM_PREP128: "prep128",
         H.MM_PREP64: "prep64", H.MM_PREP48: "prep48", H.MM_STREAM: "stream"}


def _best_us(fn, reps, stream):
    fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    best = float("inf")
    for _ in range(5):
        e0.record(stream)
        for _ in range(reps):
            fn()
        e1.record(stream)
        e1.synchronize()
        best = min(best, e0.elapsed_time(e1) * 1e3 / reps)
    return best


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--reps", type=int, default=20)
    args = ap.parse_args()
    dev = torch.device("cuda:0")
    L = H.lib()
    stream = torch.cuda.current_stream(dev)
    rows = []
    for M, N, K in SHAPES:
        X, q, s, m = (t.to(dev) for t in synth.prefill_case(M, N, K, 1))
        Y = torch.empty(M, N, device=dev, dtype=torch.float16)
        nws = L.rk_mm_int4_workspace_bytes(M, N, K)
        ws = torch.empty(max(nws, 16), device=dev, dtype=torch.uint8)
        a = [H.ptr(X), H.F16, K, H.ptr(q), H.ptr(s), H.ptr(m), H.ptr(Y), H.F16, N, M, N, K]
        st = H.stream(dev)
        H.check(L.rk_mm_int4_g128(*a, st))
        H.check(L.rk_mm_int4_g128_ws(*a, H.ptr(ws), nws, st))
        t_plain = _best_us(lambda: L.rk_mm_int4_g128(*a, st), args.reps, stream)
        t_ws = _best_us(lambda: L.rk_mm_int4_g128_ws(*a, H.ptr(ws), nws, st), args.reps, stream)
        kp, sp = H.mm_plan(M, N, K, use_workspace=False)
        kw, sw = H.mm_plan(M, N, K, use_workspace=True)
        flop = 2.0 * M * N * K
        row = {"M": M, "N": N, "K": K, "plain_us": round(t_plain, 2), "plain_kernel": NAMES[kp],
               "ws_us": round(t_ws, 2), "ws_kernel": NAMES[kw], "ws_splits": sw,
               "ws_TFLOP_s": round(flop / t_ws / 1e6, 1)}
        rows.append(row)
        print(f"M={M:4d} N={N:6d} K={K:6d}: plain {t_plain:8.2f} us ({NAMES[kp]}) | workspace {t_ws:8.2f} us "
              f"({NAMES[kw]}, splits {sw}) {row['ws_TFLOP_s']} TFLOP/s", flush=True)
    print(json.dumps({"mm_plans": rows}))


if __name__ == "__main__":
    main()
