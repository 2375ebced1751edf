#!/usr/bin/env python3
"""Benchmark of the MI355X int4 decode hot path (one JSON line on stdout).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--cpu-seconds S] [--no-cpu]

Workload (one "step"): config 1 of the benchmark definition — one decoder layer's decode projections at batch 1,
int4 g128, x fp16 ~N(0,1): fused QKV (2048 -> 3072), O (2048 -> 2048), fused gate+up (2048 -> 2*11008) followed by
SiLU(gate)*up, down (11008 -> 2048). QKV and gate+up are the reference engine's one input projection over the rows
[q k v | gate | up] (w_in, 25088 rows; engine/rumik_fused.py:100, engine/rumik_int4.py:97) with SiLU(gate)*up (the
MLP part of the reference's post); O takes a given attention output and down takes that act. The step is ONE launch
of rk_gemv_int4_g128_layer (all four projections; the grid meets once, when act is complete); the two-launch form
(w_in + SiLU, then O + down) is timed beside it. Each step uses the weights of the next of 16 distinct synthetic
layers (665 MB in all), so no step is served from the 256 MB Infinity Cache. 16 steps are one hipGraph replay;
weights and inputs are resident in HBM before timing.

value = algorithmic bytes per step (sum over the four projections of N*K/2 + 4*N*K/128 + 2K + 2N) / wall time.
roofline: the dominant kernel (the layer launch: the step's bytes in one launch), its average launch duration
measured with HIP events on its stream over back-to-back launches with rotated weights. The layer launch is a
bench-only projection-throughput kernel: o's input is given at launch time, so no engine path can call it (in the
decode step o's input is this layer's attention output, which needs the q / k / v the same launch produces); the
drop-in GEMVs and the realisable two-launch schedule are reported beside it (`gemv_gate_up`, `two_launch`).
roofline.read_ceiling_us: the best time of a read-only kernel over the same number of bytes in the same setting
(the reference's kernels/roofline.py method: one grid-stride pass, swept over threads per block, blocks and loads
in flight); roofline.read_ceilings: that ceiling at each projection's exact byte count, next to the kernel's time;
and a dense bf16 GEMV's read rate.
parity: the layer launch's outputs on copy 0 (q/k/v rows and down) and the w_in projection against the float64
oracle (max_rel and max_rel_strict).
decode_tok_s: the 36-layer step's tokens per second at ctx 256 / 1024 / 2048 (config 4), as the role-split one-launch
kernel (decode.RoleDecode) replayed as the generate loop replays it: graphs of 8 consecutive steps (one Mimi frame)
ending at slot ctx - 1; the one-step replay figure is beside it (`single_step_replays`);
decode.persistent_engine times the every-block-every-role kernel on the same weights.
cpu_baseline: the reference's CPU path for the same step, dequantize then matmul in torch fp32
(kernels/int4_gemv.py:27-30 as kernels/bench_gemv.py:43 runs it) on CPU tensors with every thread torch is given,
with a matmul-only time, and the numpy oracle's single-threaded dequantization and configs 2 / 3 / a config-4 layer
beside it.
Extra fields: the per-projection kernel times, the int8 audio head (config 2), the int4 prefill (config 3), the
sampling tail, and the 36-layer decode step (config 4) with and without sampling inside the graph.
"""
import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (ROOT / "rumik-fast_amd" / "kernels", ROOT / "rumik-fast_amd" / "engine"):
    sys.path.insert(0, str(p))

PEAK_HBM_GBS = 8000.0        # MI355X HBM3E, published
PEAK_FP16_TFLOPS = 2500.0    # MI355X dense fp16 MFMA, published
H, INTER, NQKV = 2048, 11008, 2048 + 512 + 512
SHAPES = {"qkv": (NQKV, H), "o": (H, H), "gate_up": (2 * INTER, H), "down": (H, INTER)}
N_WIN = NQKV + 2 * INTER
WIN_BYTES = N_WIN * H // 2 + 4 * N_WIN * (H // 128) + 2 * H + 2 * (NQKV + INTER)  # fused w_in + SiLU launch
N_COPIES = 16


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def int4_bytes(N, K):
    return N * K // 2 + 4 * N * (K // 128) + 2 * K + 2 * N


def int8_bytes(N, K):
    return N * K + 2 * N + 2 * K + 4 * N


def graph_of(fns):
    import torch
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for f in fns:
            f()
    torch.cuda.synchronize()
    return g


def time_graph_us(g, launches_per_replay, reps=20, trials=5):
    """best-of-trials average per launch (HIP events on the replay stream)"""
    import torch
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    best = math.inf
    for _ in range(trials):
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        e1.synchronize()
        best = min(best, e0.elapsed_time(e1) * 1e3 / reps / launches_per_replay)
    return best


def load_traffic():
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 --pmc summary, if present."""
    f = ROOT / "profiles" / "traffic.json"
    if not f.exists():
        return None
    try:
        d = json.loads(f.read_text())
        return d.get("gemv_layer_config1", {}).get("traffic_bytes")
    except Exception:
        return None


def _cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def _timed(fn, budget_s):
    """repetitions of fn() in about budget_s seconds (one warm call first): (reps, seconds)"""
    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        if time.perf_counter() - t0 >= budget_s:
            return n, time.perf_counter() - t0


def cpu_baseline(budget_s):
    """The CPU oracle on this host, bounded to about budget_s seconds in all:
    - config 1 (the bench's workload, the value): one decoder layer's four projections, numpy fp32
      dequantize-then-matmul (the reference's own CPU check, kernels/int4_gemv.py:27-30), and the same products
      with the weights dequantized once beforehand (matmul only);
    - config 2: the int8 audio head 16385 x 2048, both ways;
    - config 3: the prefill product at M = 34 over the three layer shapes, both ways;
    - a config-4 layer: the oracle's whole decode step for one full-width layer at ctx 256 (embedding, LayerNorm,
      w_in, RoPE, attention, o, down, residual, a 16-row head), both ways.
    The value is the torch path (the reference's dequantize then @, with every thread torch has: `cores`); the
    numpy oracle's figures (single-threaded dequantization, BLAS-threaded matmuls) are reported beside it."""
    import numpy as np
    import synth
    import decode
    from oracle import glue as OG
    from oracle import int4 as O
    try:
        from threadpoolctl import threadpool_info
        cores = max([i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"] or [1])
    except Exception:
        cores = 1
    share = budget_s / 10.0
    g = synth.generator(1)
    mats = {k: tuple(t.numpy() for t in synth.int4_weights(N, K, g)) for k, (N, K) in SHAPES.items()}
    deq = {k: O.dequantize(*w) for k, w in mats.items()}
    x = synth.activations(H, g).numpy()
    ob = synth.activations(H, g).numpy()
    f32 = lambda v: np.asarray(v, np.float32)  # noqa: E731

    def step(dequant):
        mv = (lambda k, v: O.gemv_int4(v, *mats[k])) if dequant else (lambda k, v: deq[k] @ f32(v))
        mv("qkv", x)
        mv("o", ob)
        gu = mv("gate_up", x)
        gate, up = gu[:INTER], gu[INTER:]
        act = (gate / (1 + np.exp(-gate)) * up).astype(np.float16)
        mv("down", act)

    nbytes = sum(int4_bytes(N, K) for N, K in SHAPES.values())
    # the reference's own CPU path in torch: dequantize (the format's definition, kernels/int4_gemv.py:27-30, the
    # drop-in module's torch function on CPU tensors) then @ x.float(), every projection of the step, with all the
    # threads torch is given (OMP_NUM_THREADS: the box's CPU share)
    import torch
    import int4_gemv
    threads = torch.get_num_threads()
    tm = {k: tuple(torch.from_numpy(np.ascontiguousarray(a)) for a in w) for k, w in mats.items()}
    tdeq = {k: int4_gemv.dequantize(*w) for k, w in tm.items()}
    tx, tob = torch.from_numpy(x).float(), torch.from_numpy(ob).float()

    def tstep(dequant):
        mv = (lambda k, v: int4_gemv.dequantize(*tm[k]) @ v) if dequant else (lambda k, v: tdeq[k] @ v)
        mv("qkv", tx)
        mv("o", tob)
        gu = mv("gate_up", tx)
        act = (torch.nn.functional.silu(gu[:INTER]) * gu[INTER:]).half().float()
        mv("down", act)

    with torch.inference_mode():
        n0, t0 = _timed(lambda: tstep(True), 2 * share)
        n0m, t0m = _timed(lambda: tstep(False), share)
    del tdeq
    n1, t1 = _timed(lambda: step(True), share)
    n1m, t1m = _timed(lambda: step(False), share / 2)
    res = {"value": round(nbytes * n0 / t0 / 1e9, 3), "unit": "GB/s", "cores": int(threads), "kind": "port",
           "sample": f"{n0} config-1 steps (one weight copy): torch fp32 dequantize-then-matmul on CPU tensors, "
                     f"{threads} threads, {t0:.1f} s",
           "host_cpus": os.cpu_count(), "cpu_model": _cpu_model(),
           "config1_us_per_step": {"dequant_matmul": round(t0 / n0 * 1e6, 1),
                                   "matmul_only": round(t0m / n0m * 1e6, 1)},
           "config1_matmul_only_GB_s": round(nbytes * n0m / t0m / 1e9, 3),
           "numpy_oracle": {"config1_us_per_step": {"dequant_matmul": round(t1 / n1 * 1e6, 1),
                                                    "matmul_only": round(t1m / n1m * 1e6, 1)},
                            "dequant_threads": 1, "blas_threads": int(cores)}}
    del deq
    # config 2: int8 head
    q8, s8 = synth.int8_weights(16385, H, g)
    q8, s8 = q8.numpy(), s8.numpy()
    w8 = O.int8_codes(q8, "s8").astype(np.float32) * s8.astype(np.float32)[:, None]
    n2, t2 = _timed(lambda: O.gemv_int8_rows(x, q8, s8, "s8"), share / 2)
    n2m, t2m = _timed(lambda: w8 @ f32(x), share / 2)
    res["config2_us"] = {"dequant_matmul": round(t2 / n2 * 1e6, 1), "matmul_only": round(t2m / n2m * 1e6, 1)}
    del w8
    # config 3: prefill product at M = 34 over the three shapes
    X = np.stack([synth.activations(H, g).numpy() for _ in range(34)])
    Xd = np.stack([synth.activations(INTER, g).numpy() for _ in range(34)])
    shapes3 = {"qkv": X, "gate_up": X, "down": Xd}
    deq3 = {k: O.dequantize(*mats[k]) for k in shapes3}
    n3, t3 = _timed(lambda: [O.mm_int4(v, *mats[k]) for k, v in shapes3.items()], share)
    n3m, t3m = _timed(lambda: [f32(v) @ deq3[k].T for k, v in shapes3.items()], share / 2)
    res["config3_M34_us"] = {"dequant_matmul": round(t3 / n3 * 1e6, 1), "matmul_only": round(t3m / n3m * 1e6, 1),
                             "shapes": ["3072x2048", "22016x2048", "2048x11008"]}
    del deq3
    # a config-4 layer: the oracle's decode step of a one-layer full-width model at ctx 256
    cfg = decode.Config(L=1, vocab=64, n_audio=16)
    w = decode.random_weights(cfg, 5, device="cpu", gen_device="cpu")
    nf = lambda t: t.numpy()  # noqa: E731
    cos, sin = OG.rope_tables(cfg.S, cfg.HD, cfg.rope_theta)

    def model(cache):
        return OG.DecodeModel(cache_weights=cache, L=1, H=cfg.H, NH=cfg.NH, NKV=cfg.NKV, HD=cfg.HD, inter=cfg.inter,
                              eps=cfg.eps, w_in=[tuple(map(nf, w["w_in"][0]))], w_o=[tuple(map(nf, w["w_o"][0]))],
                              w_down=[tuple(map(nf, w["w_down"][0]))], ln=[nf(w["ln"][0])], norm=nf(w["norm"]),
                              emb=(nf(w["emb"][0]), nf(w["emb"][1])), head=(nf(w["head"][0]), nf(w["head"][1])),
                              rope=(OG.round_to(cos, np.float16), OG.round_to(sin, np.float16)), sliding=cfg.sliding)
    rng = np.random.default_rng(6)
    kc = rng.standard_normal((1, cfg.NKV, cfg.S, cfg.HD)).astype(np.float16)
    vc = rng.standard_normal((1, cfg.NKV, cfg.S, cfg.HD)).astype(np.float16)
    md, mdc = model(False), model(True)
    n4, t4 = _timed(lambda: OG.decode_step(md, 7, 255, kc, vc), share)
    n4m, t4m = _timed(lambda: OG.decode_step(mdc, 7, 255, kc, vc), share / 2)
    res["config4_layer_ctx256_us"] = {"dequant_matmul": round(t4 / n4 * 1e6, 1),
                                      "matmul_only": round(t4m / n4m * 1e6, 1)}
    return res


FRAME = 8  # tokens per generate-loop frame (num_quantizers: one Mimi frame), one hipGraph replay


def _time_steps(eng, cfg, steps, ctxs):
    """us per token of eng's step at each context, HIP events on the engine's stream, two ways:
    - frames (the reported figure): graphs of FRAME consecutive steps (capture_frame, as the generate loop replays
      them), each frame started at pos = ctx - FRAME so its steps write slots ctx - 8 .. ctx - 1 (attention over
      ctx - 7 .. ctx slots); one tiny fill kernel per frame resets pos;
    - single: one-step graph replays with pos reset to ctx - 1 before every replay (one fill kernel per step)."""
    import torch
    res = {}
    eng.capture()
    eng.capture_frame(FRAME)
    nfr = max(1, steps // FRAME)

    def timed(fn, n):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / 1e3

    for ctx in ctxs:
        def one():
            eng.pos.fill_(ctx - 1)
            eng.replay()

        def frame():
            eng.pos.fill_(ctx - FRAME)
            eng.replay_frame(FRAME)
        dt1 = timed(one, steps)
        dt = timed(frame, nfr)
        if eng.status_word() != 0:
            raise RuntimeError(f"one-launch decode step reported status {eng.status_word()}")
        n = nfr * FRAME
        nbytes = cfg.weight_bytes() + cfg.kv_bytes(ctx)
        res[f"ctx{ctx}"] = {"us_per_token": round(dt * 1e6 / n, 1), "tok_s": round(n / dt, 1),
                            "GB_s": round(nbytes * n / dt / 1e9, 1), "bytes_per_token": nbytes,
                            "timing": f"graphs of {FRAME} steps (slots ctx-{FRAME}..ctx-1), {n} tokens",
                            "single_step_replays": {"us_per_token": round(dt1 * 1e6 / steps, 1),
                                                    "tok_s": round(steps / dt1, 1)}}
    return res


def run_decode(dev, steps):
    """Config 4: tok/s of the 36-layer step as the role-split one-launch kernel (decode.RoleDecode), captured in a
    hipGraph (random-init int4 weights, int8 head, fp16 KV cache ~N(0,1) filled to ctx - 1 slots; each step writes
    slot ctx - 1 and attends over ctx slots); the every-block-every-role one-launch kernel (PersistentDecode) is
    timed beside it on the same weights."""
    import torch
    import decode
    import synth
    cfg = decode.Config()
    w = decode.random_weights(cfg, 4, device=dev)
    w["head"][0][-1].zero_()  # </audio>'s row: its logit 0 is never sampled, so the generate run below is full length
    ctxs = (256, 1024, 2048)
    old = decode.PersistentDecode(cfg, w, device=dev, keep_layer_weights=True)
    old.fill_cache(cfg.S, seed=5)
    old.set_state(7, 0)
    persistent = _time_steps(old, cfg, steps, ctxs)
    log(f"[bench] decode, every-block-every-role step: {persistent}")
    del old
    torch.cuda.empty_cache()
    eng = decode.RoleDecode(cfg, w, device=dev, keep_layer_weights=True)  # the prefill reads the int4 layout
    out = {"engine": "role-split one-launch step (hipGraph)", "weights_bytes_per_token": cfg.weight_bytes(),
           "layers": cfg.L, "blocks": eng.nblocks, "latency_groups_in_l2": eng.local_xcd,
           "persistent_engine": persistent}
    eng.fill_cache(cfg.S, seed=5)
    eng.set_state(7, 0)
    out.update(_time_steps(eng, cfg, steps, ctxs))
    for ctx in ctxs:
        log(f"[bench] decode ctx {ctx}: {out[f'ctx{ctx}']}")
    # the same step with the sampling tail inside the graph (a full token: decode, head, stop predictor, top-30,
    # Gumbel-max pick; the sampled token is the next step's input), ctx 256
    g = synth.generator(11, "cuda")
    stop = {"0.weight": torch.ones(cfg.H, device=dev), "0.bias": torch.zeros(cfg.H, device=dev),
            "1.weight": (torch.randn(512, cfg.H, device=dev, generator=g) / cfg.H ** 0.5).bfloat16(),
            "1.bias": torch.zeros(512, device=dev),
            "3.weight": torch.randn(1, 512, device=dev, generator=g) / 512 ** 0.5 * 0.01,
            "3.bias": torch.tensor([-50.0], device=dev)}  # the stop predictor never fires (full-length generation)
    ids = torch.arange(cfg.n_audio, dtype=torch.int64) % (cfg.vocab - 1)
    ids[-1] = cfg.vocab - 1
    eng.attach_sampler(stop, ids, end_id=cfg.vocab - 1)
    ctx = 256
    eng.pos.fill_(ctx - 1)  # the capture's warm-up step needs a cache slot (the last loop left pos at S)
    eng.capture()
    eng.capture_frame(FRAME)
    nfr = max(1, steps // FRAME)
    for _ in range(3):
        eng.pos.fill_(ctx - FRAME); eng.step_i.fill_(9); eng.replay_frame(FRAME)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(nfr):
        eng.pos.fill_(ctx - FRAME); eng.step_i.fill_(9); eng.replay_frame(FRAME)
    e1.record()
    torch.cuda.synchronize()
    dt = e0.elapsed_time(e1) / 1e3
    if eng.status_word() != 0:
        raise RuntimeError(f"one-launch decode step reported status {eng.status_word()}")
    n = nfr * FRAME
    out["sampled_ctx256"] = {"us_per_token": round(dt * 1e6 / n, 1), "tok_s": round(n / dt, 1),
                             "timing": f"graphs of {FRAME} steps with the sampling tail (slots 248..255)"}
    log(f"[bench] decode + sampling ctx 256: {out['sampled_ctx256']}")
    # the host generate loop (frames of 8 replays, pinned read-back, one frame queued ahead): a 4-token prompt, then
    # 256 generated tokens from position 4
    import generate
    gen = generate.Generator(eng, Q=8, max_new=256)
    gen.generate([1, 2, 3, 4], seed=0)  # warm
    toks, st = gen.generate([1, 2, 3, 4], seed=0)
    out["generate"] = {k: st[k] for k in ("prompt_tokens", "tokens", "prefill_ms", "first_frame_ms", "decode_tok_s")}
    log(f"[bench] generate: {out['generate']}")
    # time to first frame with the batched prefill: a 34-token prompt (the reference's README quotes 50 ms for its
    # whole 34-token prefill) through Prefill's graph replay, the head and the sampling tail, then 64 tokens
    import prefill as PF
    pfq = PF.Prefill(cfg, w, eng.kc, eng.vc, eng.cos, eng.sin, max_T=64, graphs=True)
    genp = generate.Generator(eng, Q=8, max_new=64, prefill=pfq)
    prompt = [(5 * i + 3) % cfg.vocab for i in range(34)]
    genp.generate(prompt, seed=0)  # warm (captures the 48-row prefill graph)
    toks, st = genp.generate(prompt, seed=0)
    out["generate_prefilled"] = {k: st[k] for k in ("prompt_tokens", "tokens", "prefill_ms", "first_frame_ms",
                                                    "decode_tok_s")}
    log(f"[bench] generate with the batched prefill: {out['generate_prefilled']}")
    del genp, pfq
    # batched prompt prefill (36 layers: mm_int4, the matrix-core causal attention, row glue), best of 3: eager
    # launches from the host (`ms`) and, as a serving loop would replay it, the hipGraph of the prompt's 16-row
    # length bucket (`graph_ms`; T = 34 and 69 run as 48 and 80 rows)
    pf = PF.Prefill(cfg, w, eng.kc, eng.vc, eng.cos, eng.sin, max_T=512)
    pfg = PF.Prefill(cfg, w, eng.kc, eng.vc, eng.cos, eng.sin, max_T=512, graphs=True)
    res = {}
    for T in (34, 69, 512):
        ids = [(7 * i) % cfg.vocab for i in range(T)]
        row = {}
        for key, p in (("ms", pf), ("graph_ms", pfg)):
            p.run(ids)
            best = math.inf
            for _ in range(3):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                p.run(ids)
                torch.cuda.synchronize()
                best = min(best, time.perf_counter() - t0)
            row[key] = round(best * 1e3, 2)
        row["tok_s"] = round(T / row["ms"] * 1e3, 1)
        res[f"T{T}"] = row
    g = graph_of([lambda: PF.prefill_attn(pf.q, eng.kc[0], eng.vc[0], pf.o, 512, 0, cfg.NH, cfg.NKV, cfg.HD, cfg.S,
                                          cfg.HD ** -0.5)] * 10)
    us = time_graph_us(g, 10)
    fl = 4.0 * cfg.NH * cfg.HD * (512 * 513 / 2)  # QK^T and PV over the causal half
    res["attn_T512_us"] = round(us, 2)
    res["attn_T512_mfma_frac"] = round(fl / us / 1e6 / PEAK_FP16_TFLOPS, 4)
    del g
    out["prefill"] = res
    log(f"[bench] prefill (36 layers): {res}")
    del eng, w
    torch.cuda.empty_cache()
    return out


def run_sampler(dev):
    """The sampling tail alone (reference engine/sample.py at the model's sizes: hidden 2048, stop predictor 512 x 2048
    bf16, 16385 audio logits fp32, top-30): the one-launch FusedSampler call (with its torch.rand) and the
    reference's three-kernel sequence, each as hipGraph replays."""
    import types
    import torch
    import sample
    import synth
    g = synth.generator(12, "cuda")
    n, H, NZ = 16385, 2048, 512
    stop = {"0.weight": torch.ones(H, device=dev), "0.bias": torch.zeros(H, device=dev),
            "1.weight": (torch.randn(NZ, H, device=dev, generator=g) / H ** 0.5).bfloat16(),
            "1.bias": torch.zeros(NZ, device=dev), "3.weight": torch.randn(1, NZ, device=dev, generator=g) / NZ ** 0.5,
            "3.bias": torch.tensor([-5.0], device=dev)}
    e = types.SimpleNamespace(dev=dev, H=H, hn=torch.randn(H, device=dev, generator=g).bfloat16(), stop=stop,
                              audio_ids=torch.arange(n, dtype=torch.int64, device=dev), end_id=n - 1, top_k=30,
                              min_new=8, temperature=0.8, step_i=torch.zeros(1, dtype=torch.int64, device=dev),
                              pos=torch.zeros(1, dtype=torch.int64, device=dev),
                              tok=torch.zeros(1, dtype=torch.int64, device=dev),
                              out=torch.zeros(4096, dtype=torch.int64, device=dev))
    logits = torch.randn(n, device=dev, generator=g) * 3
    smp = sample.FusedSampler(e, lambda: logits)

    def three():
        torch.rand(32, device=dev, out=smp.u)
        sample.stop_hidden(e.hn, smp.lnw, smp.lnb, smp.w1, smp.b1, smp.z1, 1e-5)
        sample.topk_partial(logits, e.step_i, smp.keys, smp.nv, smp.end_idx, e.min_new)
        sample.pick(smp.keys, smp.scratch, smp.u, smp.z1, smp.w2, smp.b2, e.audio_ids, e.step_i, e.pos, e.tok, e.out,
                    1.0 / e.temperature, e.end_id, e.min_new, smp.nch, NC=smp.nc, TOPK=e.top_k)

    res = {"nv": n, "nz": NZ, "H": H, "top_k": 30}
    for name, fn in (("fused_us", smp), ("three_kernel_us", three)):
        reps = 20
        e.step_i.fill_(0)
        gr = graph_of([fn] * reps)
        e.step_i.fill_(0)
        res[name] = round(time_graph_us(gr, reps, reps=5, trials=5), 2)
        e.step_i.fill_(0)
        del gr
    # algorithmic bytes of the fused call: W1 (bf16) + logits + hn + the stop predictor's fp32 vectors
    nbytes = NZ * H * 2 + n * 4 + H * 2 + (2 * H + 2 * NZ + 1) * 4
    res["bytes"] = nbytes
    res["GB_s"] = round(nbytes / res["fused_us"] / 1e3, 1)
    log(f"[bench] sampler: {res}")
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--decode-steps", type=int, default=100, help="timed decode steps per context length (0: skip)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: --gpus {args.gpus} requested, but this build measures one GPU only: the int4 decode path "
              "is a single-GPU batch-1 workload here (no collectives are built); run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import cuda_gemv
    import mm_int4
    import synth
    import _hiplib as HL

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log(f"[bench] {torch.cuda.get_device_name(dev)}, {torch.cuda.get_device_properties(dev).multi_processor_count} CUs")

    # ---- weights: 16 distinct layers (GPU-side RNG: values are irrelevant to timing); w_in = [qkv | gate+up] rows,
    # with the separate projections as row slices of it (contiguous views, no copy)
    gen = synth.generator(1, "cuda")
    layers = []
    for _ in range(N_COPIES):
        L = {k: synth.int4_weights(N, K, gen, device=dev) for k, (N, K) in SHAPES.items() if k in ("o", "down")}
        L["w_in"] = synth.int4_weights(N_WIN, H, gen, device=dev)
        L["qkv"] = tuple(t[:NQKV] for t in L["w_in"])
        L["gate_up"] = tuple(t[NQKV:] for t in L["w_in"])
        layers.append(L)
    x = torch.randn(H, device=dev, generator=gen).half()
    ob = torch.randn(H, device=dev, generator=gen).half()
    y_qkv = torch.empty(NQKV, device=dev, dtype=torch.float16)
    y_o = torch.empty(H, device=dev, dtype=torch.float16)
    y_gu = torch.empty(2 * INTER, device=dev, dtype=torch.float16)
    act = torch.empty(INTER, device=dev, dtype=torch.float16)
    y_d = torch.empty(H, device=dev, dtype=torch.float16)

    lp = cuda_gemv.LayerProjections(NQKV, INTER, dev)

    def step_fns(L):
        # the four projections in one launch (w_in with SiLU*up, o over ob, down over this launch's act)
        return [lambda: lp(x, L["w_in"], ob, L["o"], L["down"], y_qkv, act, y_o, y_d)]

    def two_launch_fns(L):
        # the same step as two launches: w_in with SiLU*up fused, then o and down in one launch
        return [lambda: cuda_gemv.gemv_int4_silu_cuda(x, *L["w_in"], NQKV, out=y_qkv, act=act),
                lambda: cuda_gemv.gemv_int4_pair_cuda(ob, L["o"], act, L["down"], out1=y_o, out2=y_d)]

    # one hipGraph holds N_COPIES consecutive steps (one per weight copy, as consecutive layers sit in the decode
    # step's graph); a second one the remaining steps, so a run replays exactly K steps
    def run_steps(n):
        full, rest = divmod(n, N_COPIES)
        if full:
            g16 = graph_of([f for L in layers for f in step_fns(L)])
        if rest:
            gr = graph_of([f for L in layers[:rest] for f in step_fns(L)])
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(full):
            g16.replay()
        if rest:
            gr.replay()
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    step_bytes = sum(int4_bytes(N, K) for N, K in SHAPES.values())

    # ---- warm-up, then the timed region: exactly K steps, synchronized on both sides
    run_steps(args.warmup)
    elapsed = run_steps(args.steps)
    ms_per_step = elapsed * 1e3 / args.steps
    value = step_bytes * args.steps / elapsed / 1e9
    log(f"[bench] config 1: {ms_per_step * 1e3:.2f} us/step, {value:.0f} GB/s")
    if lp.status() != 0:
        raise RuntimeError("layer launch: an exchange wait ran out during the timed steps")

    # ---- the dominant kernel: the layer launch alone (16 rotated copies back to back in one graph), and the
    # two-launch form of the same step
    g = graph_of([f for L in layers for f in step_fns(L)])
    layer_us = time_graph_us(g, N_COPIES)
    del g
    if lp.status() != 0:
        raise RuntimeError("layer launch: an exchange wait ran out while timing the launch")
    g = graph_of([f for L in layers for f in two_launch_fns(L)])
    two_us = time_graph_us(g, N_COPIES)
    del g
    log(f"[bench] layer launch {layer_us:.2f} us, two-launch step {two_us:.2f} us")

    # ---- per-projection kernel times (back-to-back launches over the 16 copies)
    proj = {}
    for k, (N, K) in SHAPES.items():
        out = {"qkv": y_qkv, "o": y_o, "gate_up": y_gu, "down": y_d}[k]
        inp = {"o": ob, "down": act}.get(k, x)
        g = graph_of([lambda L=L: cuda_gemv.gemv_int4_cuda(inp, *L[k], out=out) for L in layers])
        us = time_graph_us(g, N_COPIES)
        proj[k] = {"N": N, "K": K, "us": round(us, 2), "GB_s": round(int4_bytes(N, K) / us / 1e3, 1)}
        del g
    g = graph_of([lambda L=L: cuda_gemv.gemv_int4_silu_cuda(x, *L["w_in"], NQKV, out=y_qkv, act=act)
                  for L in layers])
    win_us = time_graph_us(g, N_COPIES)
    del g
    proj["w_in_silu"] = {"N": N_WIN, "K": H, "us": round(win_us, 2), "GB_s": round(WIN_BYTES / win_us / 1e3, 1)}
    g = graph_of([lambda L=L: cuda_gemv.gemv_int4_pair_cuda(ob, L["o"], act, L["down"], out1=y_o, out2=y_d)
                  for L in layers])
    pair_us = time_graph_us(g, N_COPIES)
    del g
    pair_bytes = int4_bytes(*SHAPES["o"]) + int4_bytes(*SHAPES["down"])
    proj["o_down_pair"] = {"us": round(pair_us, 2), "GB_s": round(pair_bytes / pair_us / 1e3, 1)}
    log(f"[bench] projections: {proj}")
    achieved = step_bytes / layer_us / 1e3
    # the read ceiling of that launch: rk_read_only over buffers of the same sizes as one copy's codes, scales and
    # mins (all four projections), 16 rotated copies back to back in one graph, best over launch shapes (the
    # reference's kernels/roofline.py method); and a dense bf16 GEMV (torch.mm, 4x the weight bytes) as the vendor
    # library's practical read rate
    import roofline as RF
    mats0 = [layers[0][k] for k in ("w_in", "o", "down")]
    sizes = [sum(m[i].numel() * m[i].element_size() for m in mats0) for i in range(3)]
    ro_mats = [tuple(torch.empty(n, device=dev, dtype=torch.uint8) for n in sizes) for _ in range(N_COPIES)]
    ro_us, ro_shape, ro_all = RF.ceiling_us(ro_mats)
    ro_bytes = sum(sizes)
    del ro_mats
    log(f"[bench] read ceiling: {ro_us:.2f} us for {ro_bytes} B ({ro_bytes / ro_us / 1e3:.0f} GB/s), {ro_shape}")
    # the same ceiling at each projection's exact algorithmic byte count (one contiguous buffer per copy): the full
    # sweep for gate+up (the GEMV the >= 70 % target names), the 8 best shapes of it for the others
    ceil = {}
    gu_bytes = int4_bytes(*SHAPES["gate_up"])
    us, sh, allr = RF.ceiling_at(gu_bytes, dev)
    ceil["gate_up"] = (gu_bytes, us, sh)
    best8 = [s for _, s in allr[:8]]
    for name, nb in (("w_in_silu", WIN_BYTES), ("down", int4_bytes(*SHAPES["down"])),
                     ("qkv", int4_bytes(*SHAPES["qkv"])), ("o", int4_bytes(*SHAPES["o"])),
                     ("int8_head", int8_bytes(16385, H))):
        us, sh, _ = RF.ceiling_at(nb, dev, copies=16 if nb > 8e6 else 64, candidates=best8)
        ceil[name] = (nb, us, sh)
    kern_us = {k: proj[k]["us"] for k in ("gate_up", "down", "qkv", "o", "w_in_silu")}
    read_ceilings = {k: {"bytes": nb, "ceiling_us": round(us, 2), "ceiling_GB_s": round(nb / us / 1e3, 1),
                         "ceiling_frac_of_peak": round(nb / us / 1e3 / PEAK_HBM_GBS, 4), "shape": sh,
                         **({"kernel_us": kern_us[k], "kernel_frac_of_ceiling": round(us / kern_us[k], 4)}
                            if k in kern_us else {})}
                     for k, (nb, us, sh) in ceil.items()}
    log(f"[bench] read ceilings: {read_ceilings}")
    # parity on copy 0 against the float64 oracle (max_rel with the per-output conditioning floor, max_rel_strict
    # with the fp16 floor alone): the layer launch's q/k/v rows (over x) and down rows (over the act it wrote), and
    # the w_in projection alone
    from oracle import int4 as O

    def rep(y, xv, w, label):
        a = (xv.float().cpu().numpy(), *(t.cpu().numpy() for t in w))
        r = O.parity_report(y.float().cpu().numpy(), O.gemv_int4_f64(*a), O.cond_floor(O.gemv_int4_abs(*a)))
        return {"check": label, **{k: (round(v, 8) if isinstance(v, float) else v) for k, v in r.items()}}
    L0 = layers[0]
    y_l, act_l, yo_l, yd_l = lp(x, L0["w_in"], ob, L0["o"], L0["down"])
    torch.cuda.synchronize()
    y_chk = cuda_gemv.gemv_int4_cuda(x, *L0["w_in"], out=torch.empty(N_WIN, device=dev, dtype=torch.float32))
    parity = rep(y_chk, x, L0["w_in"], "gemv int4 w_in 25088x2048 (copy 0) vs float64 oracle")
    parity["layer"] = [rep(y_l, x, tuple(t[:NQKV] for t in L0["w_in"]), "layer launch q/k/v rows"),
                       rep(yo_l, ob, L0["o"], "layer launch o rows"),
                       rep(yd_l, act_l, L0["down"], "layer launch down rows (over the act it wrote)")]
    log(f"[bench] parity: {parity}")
    del layers, y_chk, y_l, act_l, yo_l, yd_l
    torch.cuda.empty_cache()
    wb = [torch.randn(H, N_WIN, device=dev, generator=gen).bfloat16() for _ in range(4)]  # 4 x 103 MB: past the cache
    xb, yb = x.bfloat16().view(1, H), torch.empty(1, N_WIN, device=dev, dtype=torch.bfloat16)
    for w in wb:  # hipBLASLt picks its algorithm and workspace on a first call, which a capture does not allow
        torch.mm(xb, w, out=yb)
    g = graph_of([lambda w=w: torch.mm(xb, w, out=yb) for w in wb])
    bf_us = time_graph_us(g, len(wb))
    del g, wb
    torch.cuda.empty_cache()
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": load_traffic(),
                "kernel": "gemv_layer_kernel: w_in [qkv | gate | up] 25088x2048 + SiLU*up, o 2048x2048, down "
                          "2048x11008 in one launch (bench-only projection throughput: o's input is given at "
                          "launch; no engine path calls it, the decode step runs each layer inside "
                          "decode_step_kernel)",
                "us_per_launch": round(layer_us, 2), "bytes_per_launch": step_bytes,
                "two_launch_us_per_step": round(two_us, 2),
                "read_ceiling_us": round(ro_us, 2), "read_ceiling_GB_s": round(ro_bytes / ro_us / 1e3, 1),
                "read_ceiling_shape": ro_shape, "frac_of_read_ceiling": round(ro_us / layer_us, 4),
                "read_ceilings": read_ceilings,
                "dense_bf16_gemv_us": round(bf_us, 2),
                "dense_bf16_gemv_GB_s": round(2 * N_WIN * H / bf_us / 1e3, 1)}

    # ---- config 2: int8 audio head (16385 x 2048, fp16 row scale, fp32 logits), 20 rotated copies
    heads = [synth.int8_weights(16385, H, gen, device=dev) for _ in range(20)]
    hx = torch.randn(H, device=dev, generator=gen).half()
    logits = torch.empty(16385, device=dev, dtype=torch.float32)
    g = graph_of([lambda w=w: cuda_gemv.gemv_int8_cuda(hx, w[0], w[1], out=logits) for w in heads])
    us = time_graph_us(g, len(heads))
    head = {"N": 16385, "K": H, "us": round(us, 2), "GB_s": round(int8_bytes(16385, H) / us / 1e3, 1)}
    log(f"[bench] int8 head: {head}")
    del g, heads
    torch.cuda.empty_cache()

    # ---- config 3: int4 prefill matmul (M in {34, 128, 512}), 8 rotated copies per shape
    prefill = {}
    for (N, K) in ((NQKV, H), (2 * INTER, H), (H, INTER)):
        mats = [synth.int4_weights(N, K, gen, device=dev) for _ in range(8)]
        for M in (34, 128, 512):
            X = torch.randn(M, K, device=dev, generator=gen).half()
            Y = torch.empty(M, N, device=dev, dtype=torch.float16)
            try:
                g = graph_of([lambda w=w: mm_int4.mm_int4(X, *w, out=Y) for w in mats])
            except Exception as e:  # prefill kernel not available in this build
                prefill = {"error": str(e)[:200]}
                break
            us = time_graph_us(g, len(mats), reps=10, trials=3)
            fl = 2.0 * M * N * K
            prefill[f"M{M}_{N}x{K}"] = {"us": round(us, 2), "TFLOP_s": round(fl / us / 1e6, 1),
                                        "mfma_frac": round(fl / us / 1e6 / PEAK_FP16_TFLOPS, 4)}
            del g
        if "error" in prefill:
            break
        del mats
        torch.cuda.empty_cache()
    log(f"[bench] prefill: {prefill}")

    # ---- the sampling tail (stop predictor + top-30 + Gumbel-max pick + counters)
    sampler_res = run_sampler(dev)

    # ---- config 4: the full 36-layer decode step, hipGraph replays at ctx 256 / 1024 / 2048
    decode_res = run_decode(dev, args.decode_steps) if args.decode_steps > 0 else None

    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)
    if cpu:
        log(f"[bench] cpu baseline: {cpu}")

    rec = {
        "metric": "int4 GEMV HBM GB/s (% of peak); batch-1 decode tok/s, 36-layer 3B synthetic",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights x fp16 activations, fp32 accumulate",
        "data": "synthetic (seeded int4 g128 codes / fp16 scale+min, x ~ N(0,1)); 16 distinct weight copies",
        "config": {"workload": "config 1: one decoder layer's decode projections (qkv 3072x2048, o 2048x2048, "
                               "gate+up 22016x2048 + SiLU*up, down 2048x11008), batch 1; qkv and gate+up run as "
                               "the reference engine's one w_in projection with SiLU*up fused; all four in one "
                               "bench-only launch per step (o's input given), 16 steps (16 weight copies) per "
                               "hipGraph replay",
                   "bytes_per_step": step_bytes, "pct_of_peak": round(100 * value / PEAK_HBM_GBS, 2)},
        "decode_tok_s": ({k: decode_res[k]["tok_s"] for k in ("ctx256", "ctx1024", "ctx2048")}
                         if decode_res else None),
        "roofline": roofline,
        "gemv_gate_up": {"kernel": "drop-in gemv_int4_cuda, 22016x2048 (the GEMV the >= 70% target names)",
                         "us": proj["gate_up"]["us"], "GB_s": proj["gate_up"]["GB_s"],
                         "frac_of_peak": round(proj["gate_up"]["GB_s"] / PEAK_HBM_GBS, 4),
                         "frac_of_read_ceiling": read_ceilings["gate_up"]["kernel_frac_of_ceiling"]},
        "two_launch": {"kernel": "realisable schedule: w_in + SiLU*up, then o + down (drop-in GEMVs)",
                       "us_per_step": round(two_us, 2), "GB_s": round(step_bytes / two_us / 1e3, 1)},
        "parity": parity,
        "cpu_baseline": cpu,
        "projections": proj,
        "int8_head": head,
        "prefill": prefill,
        "sampler": sampler_res,
        "decode": decode_res,
    }
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
