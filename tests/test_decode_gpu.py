"""The whole decode step (config 4) on the GPU vs the CPU oracle's decode_step (oracle/glue.py), from identical
seeded weights, KV cache and token, over several consecutive steps (pos advances on the device), eagerly and as a
replayed hipGraph. State is compared after every step (the reference's state-cloning check pattern,
engine/check_fused.py:20-34).

Tolerances: every activation is stored in fp16 and the step chains ~8 kernels per layer, so results are compared by
norm-relative error / cosine: hidden state and logits within 1e-2 / 0.9999 per step on the small model, on the
full-width model, at the benchmarked contexts (1023 / 1030 slots: 32 / 33 attention splits of 32 slots; 2040 / 2046:
all 64 splits) and for one whole 36-layer step at the last cache slot. The one-launch step's int8 head is also held
to the GEMV bar on every logit: the head recomputed by the oracle over the kernel's own exported final hidden state
`hn`, max relative error <= 1e-2 per output with the per-output conditioning floor (oracle.int4.cond_floor).
"""
import numpy as np
import pytest
import torch

import decode
from oracle import glue as OG
from oracle import int4 as O

pytestmark = pytest.mark.gpu

# the one-launch engines: every block doing every role (csrc/decode_persistent.hip) and the grid split into
# latency and stream blocks (csrc/decode_roles.hip), the latter with its latency groups' exchanges kept in their
# XCD's L2 (local_xcd, the default where the placement probe confirms the round-robin XCD placement) and through
# memory, and with q/k/v computed where its default picks by position (latency blocks below pos 384), always on the
# stream blocks ("roles_sq") or always on the latency blocks ("roles_lq")
ONE_LAUNCH = ["persistent", "roles", "roles_mem", "roles_sq", "roles_lq"]


def _one_launch(engine, cfg, w, dev):
    if engine == "persistent":
        return decode.PersistentDecode(cfg, w, device=dev)
    sqf = {"roles_sq": 0, "roles_lq": 1 << 40}.get(engine)
    eng = decode.RoleDecode(cfg, w, device=dev, local_xcd=False if engine == "roles_mem" else None,
                            stream_qkv_from=sqf)
    assert eng.local_xcd == (engine != "roles_mem"), "blocks with equal b % 8 did not share an XCD"
    return eng


def _np(t):
    return t.detach().float().cpu().numpy()


def _oracle_model(cfg, w, dt=np.float16):
    n = lambda t: t.cpu().float().numpy() if t.dtype == torch.bfloat16 else t.cpu().numpy()  # noqa: E731
    cos, sin = OG.rope_tables(cfg.S, cfg.HD, cfg.rope_theta)
    return OG.DecodeModel(cache_weights=True,
        L=cfg.L, H=cfg.H, NH=cfg.NH, NKV=cfg.NKV, HD=cfg.HD, inter=cfg.inter, eps=cfg.eps,
        w_in=[tuple(map(n, t)) for t in w["w_in"]], w_o=[tuple(map(n, t)) for t in w["w_o"]],
        w_down=[tuple(map(n, t)) for t in w["w_down"]], ln=[n(t) for t in w["ln"]], norm=n(w["norm"]),
        emb=(n(w["emb"][0]), n(w["emb"][1])), head=(n(w["head"][0]), n(w["head"][1])),
        rope=(OG.round_to(cos, dt), OG.round_to(sin, dt)), sliding=cfg.sliding)


def _run(cfg, dev, ctx, steps, use_graph, seed=4, tol=1e-2, engine="graph", dtype=torch.float16):
    """dtype: the activation / KV-cache dtype of the graph engine (the persistent engine is fp16); for bf16 the
    LayerNorm weights are bf16 too (as the reference engine's are) and the oracle rounds at bf16."""
    w = decode.random_weights(cfg, seed, device="cpu", gen_device="cpu")
    if dtype == torch.bfloat16:
        w["ln"] = [t.bfloat16() for t in w["ln"]]
        w["norm"] = w["norm"].bfloat16()
    wd = {k: ([tuple(t.to(dev) for t in v) if isinstance(v, tuple) else v.to(dev) for v in vv]
              if isinstance(vv, list) else (tuple(t.to(dev) for t in vv) if isinstance(vv, tuple) else vv.to(dev)))
          for k, vv in w.items()}
    eng = (decode.DecodeStep(cfg, wd, device=dev, dtype=dtype) if engine == "graph"
           else _one_launch(engine, cfg, wd, dev))
    g = torch.Generator().manual_seed(seed + 1)
    kc = torch.zeros(cfg.L, cfg.NKV, cfg.S, cfg.HD, dtype=dtype)
    kc[:, :, :ctx] = torch.randn(cfg.L, cfg.NKV, ctx, cfg.HD, generator=g).to(dtype)
    vc = torch.zeros_like(kc)
    vc[:, :, :ctx] = torch.randn(cfg.L, cfg.NKV, ctx, cfg.HD, generator=g).to(dtype)
    eng.kc.copy_(kc.to(dev))
    eng.vc.copy_(vc.to(dev))
    tok = 7
    eng.set_state(tok, ctx)
    if use_graph:
        eng.capture()
    odt = "bf16" if dtype == torch.bfloat16 else np.float16
    md = _oracle_model(cfg, w, odt)
    okc, ovc = kc.float().numpy().copy(), vc.float().numpy().copy()
    reps = []
    for s in range(steps):
        pos = ctx + s
        eng.replay() if use_graph else eng.step()
        torch.cuda.synchronize()
        logits, h, x = OG.decode_step(md, tok, pos, okc, ovc, dt=odt)
        assert int(eng.pos.item()) == pos + 1
        if engine != "graph":
            assert eng.status_word() == 0, "a grid barrier timed out"
        rx = O.parity_report(_np(eng.x), x)
        rl = O.parity_report(_np(eng.logits), logits)
        if engine != "graph":  # the exported final hidden state (the sampler's input)
            rh = O.parity_report(_np(eng.hn), h)
            assert rh["norm_rel"] < tol and rh["cosine"] > 0.9999, (s, rh)
            _head_per_output(eng, w["head"])
        reps.append((rx, rl))
        assert rx["norm_rel"] < tol and rx["cosine"] > 0.9999, (s, rx)
        assert rl["norm_rel"] < tol and rl["cosine"] > 0.9999, (s, rl)
        # this step's K/V were written at slot pos of every layer
        np.testing.assert_allclose(_np(eng.vc[:, :, pos]), ovc[:, :, pos].astype(np.float32), rtol=1e-2, atol=1e-2)
        # continue from the oracle's own state for the next step, so errors do not compound across steps
        eng.x.copy_(torch.tensor(x).to(eng.x.dtype).to(dev))
        eng.kc[:, :, pos].copy_(torch.tensor(okc[:, :, pos]).to(dtype).to(dev))
        eng.vc[:, :, pos].copy_(torch.tensor(ovc[:, :, pos]).to(dtype).to(dev))
    return reps


def _head_per_output(eng, head):
    """the one-launch step's int8 head against the oracle's over the kernel's own hn, on every logit: max relative
    error <= 1e-2 with the per-output conditioning floor (the GEMV bar; reference kernels/cuda_gemv.py:245-249)"""
    hq, hs = (t.cpu().numpy() for t in head)
    hn = _np(eng.hn)
    ref = O.gemv_int8_rows_f64(hn, hq, hs, "s8")
    rep = O.parity_report(_np(eng.logits), ref, O.cond_floor(O.gemv_int8_abs(hn, hq, hs, "s8")))
    assert rep["max_rel"] <= 1e-2 and rep["n"] == hq.shape[0], rep
    return rep


SMALL = dict(L=3, H=256, NH=4, NKV=2, HD=128, inter=384, S=64, n_audio=100, vocab=50, nsplit=8)


@pytest.mark.parametrize("use_graph", [False, True])
def test_small_model_steps(use_graph, dev):
    cfg = decode.Config(**SMALL)
    reps = _run(cfg, dev, ctx=5, steps=4, use_graph=use_graph)
    print(reps[-1])


@pytest.mark.parametrize("use_graph", [False, True])
def test_small_model_steps_bf16(use_graph, dev):
    """The graph engine as the reference engine allocates it (engine/rumik_fused.py:40-52): bf16 x / h / q / o / act,
    bf16 KV cache, bf16 cos / sin and LayerNorm weights; the oracle rounds at bf16 at the same points."""
    cfg = decode.Config(**SMALL)
    reps = _run(cfg, dev, ctx=5, steps=4, use_graph=use_graph, dtype=torch.bfloat16)
    print(reps[-1])


def test_full_width_two_layers_bf16(dev):
    cfg = decode.Config(L=2, vocab=64, sliding=[True, False])
    reps = _run(cfg, dev, ctx=700, steps=2, use_graph=True, dtype=torch.bfloat16)
    print(reps[-1])


def test_full_width_four_layers(dev):
    cfg = decode.Config(L=4, vocab=64)
    reps = _run(cfg, dev, ctx=300, steps=2, use_graph=True)
    print(reps[-1])


@pytest.mark.parametrize("engine", ONE_LAUNCH)
@pytest.mark.parametrize("use_graph", [False, True])
def test_persistent_full_width(use_graph, engine, dev):
    # the one-launch step: hidden 2048, 16 / 4 heads, MLP 11008, 3 layers (one of them NoPE), ctx 300
    cfg = decode.Config(L=3, vocab=64, sliding=[True, False, True])
    reps = _run(cfg, dev, ctx=300, steps=3, use_graph=use_graph, engine=engine)
    print(reps[-1])


@pytest.mark.parametrize("engine", ["roles", "roles_mem", "roles_sq"])
def test_roles_eight_kv_heads(engine, dev):
    # 16 q / 8 kv heads: latency groups of 8 blocks (4 q/k/v tiles each, 8 splits per KV head of at most 128
    # slots, so a 1024-slot cache), ctx 300
    cfg = decode.Config(L=2, NKV=8, S=1024, vocab=64, sliding=[True, False])
    reps = _run(cfg, dev, ctx=300, steps=2, use_graph=False, engine=engine)
    print(reps[-1])


def test_roles_qkv_placements_identical(dev):
    """q/k/v on the latency blocks and on the stream blocks compute the same tiles with the same K-split sums, so two
    steps of each, from the same state (ctx 383: the default engine switches placement at pos 384, on its second
    step), give bit-identical logits, final hidden state, residual stream and new K / V cache slots."""
    cfg = decode.Config(L=3, vocab=64, S=1024, sliding=[True, False, True])
    w = decode.random_weights(cfg, 9, device=dev, gen_device="cuda")
    g = torch.Generator(device=dev).manual_seed(3)
    kc = torch.randn(cfg.L, cfg.NKV, cfg.S, cfg.HD, device=dev, generator=g).half()
    vc = torch.randn(cfg.L, cfg.NKV, cfg.S, cfg.HD, device=dev, generator=g).half()
    outs = []
    for sqf in (1 << 40, 0, None):
        eng = decode.RoleDecode(cfg, w, device=dev, stream_qkv_from=sqf, keep_layer_weights=True)
        eng.kc.copy_(kc)
        eng.vc.copy_(vc)
        eng.set_state(7, 383)
        res = []
        for _ in range(2):
            eng.step()
            torch.cuda.synchronize()
            assert eng.status_word() == 0
            res.append((eng.logits.clone(), eng.hn.clone(), eng.x.clone()))
        outs.append((res, eng.kc[:, :, 383:385].clone(), eng.vc[:, :, 383:385].clone()))
        del eng
    for other in outs[1:]:
        for (la, ha, xa), (lb, hb, xb) in zip(outs[0][0], other[0]):
            assert torch.equal(la, lb) and torch.equal(ha, hb) and torch.equal(xa, xb)
        assert torch.equal(outs[0][1], other[1]) and torch.equal(outs[0][2], other[2])


@pytest.mark.parametrize("engine", ["roles", "persistent"])
def test_frame_graph_equals_single_replays(engine, dev):
    """capture_frame(n): n consecutive steps (decode + sampling tail) in ONE graph, as the generate loop and the
    bench replay them, do exactly what n replays of the one-step graph do: from the same state and seed the sampled
    tokens, the new K / V slots, logits, hidden state, pos and step counter are bit-identical (ctx 377 .. 381
    crosses the role-split step's q/k/v placement switch at pos 384 on the second frame)."""
    cfg = decode.Config(L=2, vocab=64, n_audio=700, S=512)
    w = decode.random_weights(cfg, 12, device=dev, gen_device="cuda")
    eng = _one_launch(engine, cfg, w, dev)
    g = torch.Generator().manual_seed(13)
    stop = {"0.weight": torch.ones(cfg.H), "0.bias": torch.zeros(cfg.H),
            "1.weight": (torch.randn(512, cfg.H, generator=g) / cfg.H ** 0.5).bfloat16(),
            "1.bias": torch.zeros(512), "3.weight": torch.randn(1, 512, generator=g) / 512 ** 0.5,
            "3.bias": torch.tensor([-5.0])}
    ids = torch.arange(cfg.n_audio, dtype=torch.int64) % (cfg.vocab - 1)
    ids[-1] = cfg.vocab - 1
    eng.attach_sampler(stop, ids, end_id=cfg.vocab - 1)
    gk = torch.Generator(device=dev).manual_seed(14)
    eng.kc.normal_(generator=gk)
    eng.vc.normal_(generator=gk)
    kc0, vc0 = eng.kc.clone(), eng.vc.clone()
    n, pos0 = 5, 377
    eng.set_state(3, pos0)
    eng.capture()
    eng.capture_frame(n)
    res = []
    for use_frame in (False, True):
        eng.kc.copy_(kc0); eng.vc.copy_(vc0); eng.set_state(3, pos0)
        eng.step_i.zero_(); eng.out.zero_()
        torch.manual_seed(21)
        for _ in range(2):  # two frames: the second starts from the state the first left
            if use_frame:
                eng.replay_frame(n)
            else:
                for _ in range(n):
                    eng.replay()
        torch.cuda.synchronize()
        assert eng.status_word() == 0
        res.append((eng.out[:2 * n].clone(), eng.kc[:, :, pos0:pos0 + 2 * n].clone(),
                    eng.vc[:, :, pos0:pos0 + 2 * n].clone(), eng.logits.clone(), eng.hn.clone(), eng.pos.clone(),
                    eng.step_i.clone(), eng.tok.clone()))
    assert int(res[0][5].item()) == pos0 + 2 * n and int(res[0][6].item()) == 2 * n
    for a, b in zip(*res):
        assert torch.equal(a, b)


@pytest.mark.parametrize("engine", ONE_LAUNCH)
def test_persistent_small_mlp_and_ctx_edges(engine, dev):
    # inter 2048, contexts at the edges: first slot and the last slot of the cache (the role-split step: 128 MLP
    # slices over 192 stream blocks, so 64 of them hold none)
    cfg = decode.Config(L=2, inter=2048, S=256, vocab=32, n_audio=1000)
    _run(cfg, dev, ctx=0, steps=2, use_graph=True, engine=engine)
    _run(cfg, dev, ctx=254, steps=2, use_graph=False, engine=engine)


@pytest.mark.parametrize("engine", ONE_LAUNCH)
def test_persistent_step_with_sampler_token_loop(engine, dev):
    """Decode step + sampling tail in one captured graph (reference engine/rumik_fused.py:92-94): each replay's
    sampled token is the next replay's input. Per replay: the token is the sampling oracle's pick on the step's own
    logits / hidden state and uniforms (oracle/sample.py), and the step itself matches the decode oracle run on the
    sampled token stream (oracle/glue.py)."""
    import sample
    from oracle import sample as OS
    cfg = decode.Config(L=2, vocab=64, n_audio=700)
    w = decode.random_weights(cfg, 8, device="cpu", gen_device="cpu")
    wd = {k: ([tuple(t.to(dev) for t in v) if isinstance(v, tuple) else v.to(dev) for v in vv]
              if isinstance(vv, list) else (tuple(t.to(dev) for t in vv) if isinstance(vv, tuple) else vv.to(dev)))
          for k, vv in w.items()}
    eng = _one_launch(engine, cfg, wd, dev)
    g = torch.Generator().manual_seed(9)
    stop = {"0.weight": torch.ones(cfg.H), "0.bias": torch.zeros(cfg.H),
            "1.weight": (torch.randn(512, cfg.H, generator=g) / cfg.H ** 0.5).bfloat16(),
            "1.bias": torch.zeros(512), "3.weight": torch.randn(1, 512, generator=g) / 512 ** 0.5,
            "3.bias": torch.tensor([-5.0])}
    ids = torch.arange(cfg.n_audio, dtype=torch.int64) % (cfg.vocab - 1)  # head row -> next input token (< vocab)
    ids[-1] = cfg.vocab - 1
    eng.attach_sampler(stop, ids, end_id=cfg.vocab - 1, top_k=30, min_new=8, temperature=0.8)
    ctx = 40
    kc = torch.zeros(cfg.L, cfg.NKV, cfg.S, cfg.HD, dtype=torch.float16)
    kc[:, :, :ctx] = torch.randn(cfg.L, cfg.NKV, ctx, cfg.HD, generator=g).half()
    vc = torch.zeros_like(kc)
    vc[:, :, :ctx] = torch.randn(cfg.L, cfg.NKV, ctx, cfg.HD, generator=g).half()
    eng.kc.copy_(kc.to(dev))
    eng.vc.copy_(vc.to(dev))
    eng.set_state(5, ctx)
    eng.capture()
    md = _oracle_model(cfg, w)
    okc, ovc = kc.numpy().copy(), vc.numpy().copy()
    st = {k: v.float().numpy() for k, v in stop.items()}
    tok = 5
    for s in range(4):
        eng.replay()
        torch.cuda.synchronize()
        assert eng.status_word() == 0
        logits, h, x = OG.decode_step(md, tok, ctx + s, okc, ovc)
        rl = O.parity_report(_np(eng.logits), logits)
        assert rl["norm_rel"] < 1e-2 and rl["cosine"] > 0.9999, (s, rl)
        # the sampler's pick on the step's own outputs
        lg, hn, u = _np(eng.logits), _np(eng.hn), _np(eng.sampler.u)
        z1 = OS.stop_hidden(hn, st["0.weight"], st["0.bias"], st["1.weight"], st["1.bias"])
        sl = OS.stop_logit(z1, st["3.weight"].reshape(-1), st["3.bias"])
        sc, idx = OS.scores(lg, u, s, cfg.n_audio - 1, 8, 30, 0.8)
        new = int(eng.tok.item())
        order = np.argsort(-sc, kind="stable")
        near = [int(ids[idx[j]]) for j in order if sc[order[0]] - sc[j] <= 1e-4]
        assert new in near and sl < 0, (new, near, sl)
        assert int(eng.step_i.item()) == s + 1 and int(eng.out[s].item()) == new
        assert int(eng.pos.item()) == ctx + s + 1
        tok = new  # the oracle continues on the GPU's token stream
        eng.kc[:, :, ctx + s].copy_(torch.tensor(okc[:, :, ctx + s]).to(dev))
        eng.vc[:, :, ctx + s].copy_(torch.tensor(ovc[:, :, ctx + s]).to(dev))


@pytest.mark.parametrize("engine", ONE_LAUNCH)
def test_persistent_fp16_overflow_sets_status(engine, dev):
    """The one-launch step is fp16 end to end (the reference engine is bf16): a residual sum beyond 65504 becomes
    inf. Forced from the host: the token's embedding scale is set so that the embedding row itself overflows. The
    step must still finish normally (no wait times out, pos advances) and report status bit 3 (value 8); a finite
    step on a normal token reports 0."""
    cfg = decode.Config(L=2, vocab=16, n_audio=64, S=64)
    w = decode.random_weights(cfg, 3, device=dev, gen_device="cuda")
    w["emb"][1][5] = 60000.0  # fp16 scale: 127 * 60000 is far beyond the fp16 range
    eng = _one_launch(engine, cfg, w, dev)
    eng.set_state(4, 3)
    eng.step()
    torch.cuda.synchronize()
    assert eng.status_word() == 0 and int(eng.pos.item()) == 4
    eng.set_state(5, 4)
    eng.step()
    torch.cuda.synchronize()
    st = eng.status_word()
    assert st & 8 and not st & 3, st
    assert int(eng.pos.item()) == 5
    eng.reset()
    eng.set_state(4, 3)  # slots 0..3 only: slot 4 now holds the overflowed step's K / V
    eng.step()
    torch.cuda.synchronize()
    assert eng.status_word() == 0


@pytest.mark.parametrize("engine", ONE_LAUNCH)
@pytest.mark.parametrize("n_audio", [16321, 16384, 257])
def test_persistent_head_ragged_tail(n_audio, engine, dev):
    """The one-launch step's int8 head splits its rows over the blocks in runs of ceil(n_audio / blocks): 16321 leaves
    the last block one row, 16384 fills every block exactly (64 rows), 257 gives 128 blocks two rows, one block a
    single row and the rest none. Every logit is checked against the head over the kernel's own hn."""
    cfg = decode.Config(L=1, vocab=32, n_audio=n_audio, S=64)
    _run(cfg, dev, ctx=10, steps=1, use_graph=False, engine=engine, seed=50 + n_audio % 11)


@pytest.mark.parametrize("engine", ONE_LAUNCH)
@pytest.mark.parametrize("ctx", [1023, 1030, 2040, 2046])
def test_persistent_long_contexts(ctx, engine, dev):
    """The contexts the benchmark times, on the full 2048-slot cache (at most 64 splits per KV head, at least 32
    slots per split): ctx 1023 / 1030 (the first step attends over 1024 / 1031 slots) use 32 / 33 splits of 32 slots,
    2040 / 2046 all 64 splits of 32 (every prefetched K / V slot of a split is used, and the 64-split combine runs in
    every head's blocks). Two steps each, both checked."""
    cfg = decode.Config(L=2, vocab=64, sliding=[True, False])
    reps = _run(cfg, dev, ctx=ctx, steps=2, use_graph=True, engine=engine, seed=40 + ctx % 7)
    print(ctx, reps[-1])


def _cpu(w):
    return {k: ([tuple(t.cpu() for t in v) if isinstance(v, tuple) else v.cpu() for v in vv]
                if isinstance(vv, list) else (tuple(t.cpu() for t in vv) if isinstance(vv, tuple) else vv.cpu()))
            for k, vv in w.items()}


@pytest.mark.timeout(900)
@pytest.mark.parametrize("engine", ONE_LAUNCH)
def test_persistent_36_layers_at_last_slot(engine, dev):
    """Config 4's whole step: 36 full-width layers (RoPE on 3 of every 4), the int8 head over 16385 rows, the
    2048-slot cache filled to 2047 slots, one step at pos 2047 (the benchmark's ctx 2048). x, the final hidden state,
    the logits and the new K / V slot of every layer against the decode oracle."""
    cfg = decode.Config(vocab=64)
    w = decode.random_weights(cfg, 6, device=dev, gen_device="cuda")
    wc = _cpu(w)
    eng = _one_launch(engine, cfg, w, dev)
    pos = cfg.S - 1
    g = torch.Generator(device=dev).manual_seed(7)
    eng.kc[:, :, :pos].normal_(generator=g)
    eng.vc[:, :, :pos].normal_(generator=g)
    okc, ovc = eng.kc.cpu().numpy(), eng.vc.cpu().numpy()
    eng.set_state(9, pos)
    eng.capture()
    eng.replay()
    torch.cuda.synchronize()
    assert eng.status_word() == 0 and int(eng.pos.item()) == pos + 1
    md = _oracle_model(cfg, wc)
    logits, h, x = OG.decode_step(md, 9, pos, okc, ovc)
    for name, got, ref in (("x", eng.x, x), ("hn", eng.hn, h), ("logits", eng.logits, logits),
                           ("k", eng.kc[:, :, pos], okc[:, :, pos]), ("v", eng.vc[:, :, pos], ovc[:, :, pos])):
        rep = O.parity_report(_np(got).ravel(), np.asarray(ref, np.float32).ravel())
        print(name, rep)
        assert rep["norm_rel"] < 1e-2 and rep["cosine"] > 0.9999, (name, rep)
    print("head per output", _head_per_output(eng, wc["head"]))
