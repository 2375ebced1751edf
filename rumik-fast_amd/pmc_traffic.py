#!/usr/bin/env python3
"""HBM traffic per launch from rocprofv3 hardware counters: the one-launch layer projections (rk_gemv_int4_g128_layer,
the dominant kernel of bench.py's step and the source of its roofline.traffic), the fused w_in int4 GEMV + SiLU*up
(rows [qkv 3072 | gate 11008 | up 11008], K=2048) and the one-launch 36-layer decode step.

Two steps for the fused w_in GEMV:

    run        launches a plain elementwise copy of known size (torch.neg over 256 MiB fp16: reads and writes
               268,435,456 B each) and then the fused w_in GEMV over 16 rotated weight copies, eagerly, one dispatch
               each. Run it under `rocprofv3 --pmc FETCH_SIZE` and again under `rocprofv3 --pmc WRITE_SIZE`.
    summarize  reads the two counter-collection CSVs, scales each counter by what it reads for the copy kernel
               (counter KiB * 1024 / known bytes), and writes profiles/traffic.json (read by bench.py) plus a
               markdown summary on stdout.

    cd /tmp && export TMPDIR=/tmp
    timeout -s KILL 60 rocprofv3 --pmc FETCH_SIZE --kernel-trace -d OUT/fetch -o fetch --output-format csv \
        -- python3 rumik-fast_amd/pmc_traffic.py run
    timeout -s KILL 60 rocprofv3 --pmc WRITE_SIZE --kernel-trace -d OUT/write -o write --output-format csv \
        -- python3 rumik-fast_amd/pmc_traffic.py run
    python3 rumik-fast_amd/pmc_traffic.py summarize OUT/fetch OUT/write

The same two steps for the one-launch layer projections (bench.py's step: w_in + SiLU*up, o and down in one
launch of rk_gemv_int4_g128_layer): `run-layer` and `summarize-layer` (key gemv_layer_config1 of
profiles/traffic.json).

The same two steps for the one-launch 36-layer decode step (config 4): `run-decode [roles|persistent]` launches the
copy kernel, then DECODE_STEPS eager steps at each of ctx 256, 1024 and 2048 (one dispatch each) of the role-split
step (decode.RoleDecode, the default) or the every-block-every-role one (decode.PersistentDecode);
`summarize-decode DIR DIR [roles|persistent]` gives the HBM bytes per token against the algorithmic bytes (every
weight once plus the K/V slots read) and writes that engine's entry of profiles/decode_step_traffic.json.
"""
import csv
import glob
import json
import os
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
COPY_BYTES = 256 << 20
N_PLAIN, INTER, K = 3072, 11008, 2048
N = N_PLAIN + 2 * INTER
GEMV_BYTES = N * K // 2 + 4 * N * (K // 128) + 2 * K + 2 * (N_PLAIN + INTER)  # outputs: y [3072] and act [11008]
N_COPIES = 16
KEY = "gemv_int4_w_in_silu_25088x2048"


def run():
    sys.path.insert(0, str(ROOT / "rumik-fast_amd" / "kernels"))
    import torch
    import cuda_gemv
    import synth
    dev = torch.device("cuda:0")
    src = torch.ones(COPY_BYTES // 2, dtype=torch.float16, device=dev)
    dst = torch.empty_like(src)
    gen = synth.generator(1, "cuda")
    mats = [synth.int4_weights(N, K, gen, device=dev) for _ in range(N_COPIES)]
    x = torch.randn(K, device=dev, generator=gen).half()
    y = torch.empty(N_PLAIN, device=dev, dtype=torch.float16)
    act = torch.empty(INTER, device=dev, dtype=torch.float16)
    torch.cuda.synchronize()
    for _ in range(4):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    for _ in range(2):
        for w in mats:
            cuda_gemv.gemv_int4_silu_cuda(x, *w, N_PLAIN, out=y, act=act)
    torch.cuda.synchronize()
    print("pmc_traffic: run done", flush=True)


def _rows(d):
    files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {d}")
    with open(files[0]) as f:
        return list(csv.DictReader(f))


def _per_dispatch(rows, counter, pred):
    """mean over matching dispatches of the counter value (summed over the rows of one dispatch)"""
    per = {}
    for r in rows:
        if r.get("Counter_Name") != counter or not pred(r.get("Kernel_Name", "")):
            continue
        key = r.get("Dispatch_Id") or r.get("Correlation_Id")
        per[key] = per.get(key, 0.0) + float(r["Counter_Value"])
    if not per:
        raise SystemExit(f"no {counter} rows for the kernel")
    vals = list(per.values())
    return sum(vals) / len(vals), len(vals)


def summarize(fetch_dir, write_dir):
    is_copy = lambda n: "neg" in n.lower()  # noqa: E731
    is_gemv = lambda n: "gemv_int4" in n  # noqa: E731
    fr, wr = _rows(fetch_dir), _rows(write_dir)
    f_copy, nfc = _per_dispatch(fr, "FETCH_SIZE", is_copy)
    w_copy, nwc = _per_dispatch(wr, "WRITE_SIZE", is_copy)
    f_gemv, nfg = _per_dispatch(fr, "FETCH_SIZE", is_gemv)
    w_gemv, nwg = _per_dispatch(wr, "WRITE_SIZE", is_gemv)
    kf = f_copy * 1024 / COPY_BYTES  # counter KiB*1024 per true byte
    kw = w_copy * 1024 / COPY_BYTES
    fetch_b = f_gemv * 1024 / kf
    write_b = w_gemv * 1024 / kw
    rec = {KEY: {
        "traffic_bytes": round(fetch_b + write_b), "fetch_bytes": round(fetch_b), "write_bytes": round(write_b),
        "algorithmic_bytes": GEMV_BYTES, "fetch_scale": round(kf, 4), "write_scale": round(kw, 4),
        "dispatches": {"copy_fetch": nfc, "copy_write": nwc, "gemv_fetch": nfg, "gemv_write": nwg}}}
    _merge_traffic(rec)
    r = rec[KEY]
    print("| quantity | value |\n|---|---|")
    print(f"| copy kernel (torch.neg, 256 MiB fp16) FETCH_SIZE / dispatch | {f_copy:.0f} KiB (scale {kf:.4f}) |")
    print(f"| copy kernel WRITE_SIZE / dispatch | {w_copy:.0f} KiB (scale {kw:.4f}) |")
    print(f"| w_in GEMV + SiLU FETCH_SIZE / dispatch | {f_gemv:.0f} KiB -> {fetch_b:,.0f} B |")
    print(f"| w_in GEMV + SiLU WRITE_SIZE / dispatch | {w_gemv:.0f} KiB -> {write_b:,.0f} B |")
    print(f"| traffic / launch (scaled) | {r['traffic_bytes']:,} B |")
    print(f"| algorithmic bytes / launch | {GEMV_BYTES:,} B (traffic / algorithmic = "
          f"{r['traffic_bytes'] / GEMV_BYTES:.3f}) |")


def _merge_traffic(rec):
    f = ROOT / "profiles" / "traffic.json"
    d = json.loads(f.read_text()) if f.exists() else {}
    d.update(rec)
    f.write_text(json.dumps(d, indent=1) + "\n")


H_O, LAYER_KEY = 2048, "gemv_layer_config1"


def _int4_bytes(n, k):
    return n * k // 2 + 4 * n * (k // 128) + 2 * k + 2 * n


LAYER_BYTES = sum(_int4_bytes(n, k) for n, k in ((N_PLAIN, K), (H_O, K), (2 * INTER, K), (H_O, INTER)))


def run_layer():
    sys.path.insert(0, str(ROOT / "rumik-fast_amd" / "kernels"))
    import torch
    import cuda_gemv
    import synth
    dev = torch.device("cuda:0")
    src = torch.ones(COPY_BYTES // 2, dtype=torch.float16, device=dev)
    dst = torch.empty_like(src)
    gen = synth.generator(1, "cuda")
    layers = [(synth.int4_weights(N, K, gen, device=dev), synth.int4_weights(H_O, K, gen, device=dev),
               synth.int4_weights(H_O, INTER, gen, device=dev)) for _ in range(N_COPIES)]
    x = torch.randn(K, device=dev, generator=gen).half()
    ob = torch.randn(K, device=dev, generator=gen).half()
    outs = [torch.empty(n, device=dev, dtype=torch.float16) for n in (N_PLAIN, INTER, H_O, H_O)]
    lp = cuda_gemv.LayerProjections(N_PLAIN, INTER, dev)
    torch.cuda.synchronize()
    for _ in range(4):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    for _ in range(2):
        for w_in, w_o, w_d in layers:
            lp(x, w_in, ob, w_o, w_d, *outs)
    torch.cuda.synchronize()
    if lp.status() != 0:
        raise SystemExit(f"layer launch status {lp.status()}")
    print("pmc_traffic: layer run done", flush=True)


def summarize_layer(fetch_dir, write_dir):
    is_copy = lambda n: "neg" in n.lower()  # noqa: E731
    is_layer = lambda n: "gemv_layer_kernel" in n  # noqa: E731
    fr, wr = _rows(fetch_dir), _rows(write_dir)
    f_copy, nfc = _per_dispatch(fr, "FETCH_SIZE", is_copy)
    w_copy, nwc = _per_dispatch(wr, "WRITE_SIZE", is_copy)
    f_l, nfl = _per_dispatch(fr, "FETCH_SIZE", is_layer)
    w_l, nwl = _per_dispatch(wr, "WRITE_SIZE", is_layer)
    kf, kw = f_copy * 1024 / COPY_BYTES, w_copy * 1024 / COPY_BYTES
    fetch_b, write_b = f_l * 1024 / kf, w_l * 1024 / kw
    rec = {LAYER_KEY: {
        "traffic_bytes": round(fetch_b + write_b), "fetch_bytes": round(fetch_b), "write_bytes": round(write_b),
        "algorithmic_bytes": LAYER_BYTES, "fetch_scale": round(kf, 4), "write_scale": round(kw, 4),
        "dispatches": {"copy_fetch": nfc, "copy_write": nwc, "layer_fetch": nfl, "layer_write": nwl}}}
    _merge_traffic(rec)
    r = rec[LAYER_KEY]
    print("| quantity | value |\n|---|---|")
    print(f"| copy kernel (torch.neg, 256 MiB fp16) FETCH_SIZE / dispatch | {f_copy:.0f} KiB (scale {kf:.4f}) |")
    print(f"| copy kernel WRITE_SIZE / dispatch | {w_copy:.0f} KiB (scale {kw:.4f}) |")
    print(f"| layer launch FETCH_SIZE / dispatch | {f_l:.0f} KiB -> {fetch_b:,.0f} B |")
    print(f"| layer launch WRITE_SIZE / dispatch | {w_l:.0f} KiB -> {write_b:,.0f} B |")
    print(f"| traffic / launch (scaled) | {r['traffic_bytes']:,} B |")
    print(f"| algorithmic bytes / launch | {LAYER_BYTES:,} B (traffic / algorithmic = "
          f"{r['traffic_bytes'] / LAYER_BYTES:.3f}) |")


DECODE_STEPS = 4
DECODE_CTX = (256, 1024, 2048)


DECODE_KERNEL = {"roles": "decode_roles_kernel", "persistent": "decode_step_kernel"}


def run_decode(engine="roles"):
    sys.path.insert(0, str(ROOT / "rumik-fast_amd" / "kernels"))
    sys.path.insert(0, str(ROOT / "rumik-fast_amd" / "engine"))
    import torch
    import decode
    dev = torch.device("cuda:0")
    src = torch.ones(COPY_BYTES // 2, dtype=torch.float16, device=dev)
    dst = torch.empty_like(src)
    cfg = decode.Config()
    cls = {"roles": decode.RoleDecode, "persistent": decode.PersistentDecode}[engine]
    eng = cls(cfg, decode.random_weights(cfg, 4, device=dev), device=dev)
    eng.fill_cache(cfg.S, seed=5)
    eng.set_state(7, 0)
    torch.cuda.synchronize()
    for _ in range(4):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    for ctx in DECODE_CTX:
        for _ in range(DECODE_STEPS):
            eng.pos.fill_(ctx - 1)
            eng.step()
    torch.cuda.synchronize()
    if eng.status_word() != 0:
        raise SystemExit(f"decode step status {eng.status_word()}")
    print("pmc_traffic: decode run done", flush=True)


def _per_dispatch_list(rows, counter, pred):
    """[(dispatch id, counter value summed over the dispatch's rows)] in dispatch order"""
    per = {}
    for r in rows:
        if r.get("Counter_Name") != counter or not pred(r.get("Kernel_Name", "")):
            continue
        key = int(r.get("Dispatch_Id") or r.get("Correlation_Id"))
        per[key] = per.get(key, 0.0) + float(r["Counter_Value"])
    return [per[k] for k in sorted(per)]


def summarize_decode(fetch_dir, write_dir, engine="roles"):
    sys.path.insert(0, str(ROOT / "rumik-fast_amd" / "engine"))
    import decode
    cfg = decode.Config()
    is_copy = lambda n: "neg" in n.lower()  # noqa: E731
    is_dec = lambda n: DECODE_KERNEL[engine] in n  # noqa: E731
    fr, wr = _rows(fetch_dir), _rows(write_dir)
    f_copy, _ = _per_dispatch(fr, "FETCH_SIZE", is_copy)
    w_copy, _ = _per_dispatch(wr, "WRITE_SIZE", is_copy)
    kf, kw = f_copy * 1024 / COPY_BYTES, w_copy * 1024 / COPY_BYTES
    fd, wd = _per_dispatch_list(fr, "FETCH_SIZE", is_dec), _per_dispatch_list(wr, "WRITE_SIZE", is_dec)
    n = DECODE_STEPS
    if len(fd) != n * len(DECODE_CTX) or len(wd) != n * len(DECODE_CTX):
        raise SystemExit(f"expected {n * len(DECODE_CTX)} decode dispatches, got {len(fd)} / {len(wd)}")
    rec = {"kernel": DECODE_KERNEL[engine], "fetch_scale": round(kf, 4), "write_scale": round(kw, 4),
           "steps_per_ctx": n}
    print("| ctx | FETCH_SIZE / step | WRITE_SIZE / step | HBM bytes / token (scaled) | algorithmic bytes / token "
          "| traffic / algorithmic |\n|---|---|---|---|---|---|")
    for i, ctx in enumerate(DECODE_CTX):
        f = sum(fd[i * n:(i + 1) * n]) / n
        w = sum(wd[i * n:(i + 1) * n]) / n
        fb, wb = f * 1024 / kf, w * 1024 / kw
        alg = cfg.weight_bytes() + cfg.kv_bytes(ctx)
        rec[f"ctx{ctx}"] = {"fetch_bytes": round(fb), "write_bytes": round(wb), "traffic_bytes": round(fb + wb),
                            "algorithmic_bytes": alg, "ratio": round((fb + wb) / alg, 4)}
        print(f"| {ctx} | {f:,.0f} KiB | {w:,.0f} KiB | {fb + wb:,.0f} B | {alg:,} B | {(fb + wb) / alg:.3f} |")
    path = ROOT / "profiles" / "decode_step_traffic.json"
    allrec = json.loads(path.read_text()) if path.exists() else {}
    if "ctx256" in allrec:  # the single-engine layout: that record is the every-block-every-role kernel's
        allrec = {"persistent": allrec}
    allrec[engine] = rec
    path.write_text(json.dumps(allrec, indent=1) + "\n")


if __name__ == "__main__":
    if len(sys.argv) >= 2 and sys.argv[1] == "run":
        run()
    elif len(sys.argv) >= 2 and sys.argv[1] == "run-layer":
        run_layer()
    elif len(sys.argv) == 4 and sys.argv[1] == "summarize-layer":
        summarize_layer(sys.argv[2], sys.argv[3])
    elif len(sys.argv) in (2, 3) and sys.argv[1] == "run-decode":
        run_decode(*sys.argv[2:])
    elif len(sys.argv) == 4 and sys.argv[1] == "summarize":
        summarize(sys.argv[2], sys.argv[3])
    elif len(sys.argv) in (4, 5) and sys.argv[1] == "summarize-decode":
        summarize_decode(*sys.argv[2:])
    else:
        raise SystemExit(__doc__)
