"""The whole decode step (config 4) on the GPU vs the CPU oracle's decode_step (oracle/glue.py), from identical
seeded weights, KV cache and token, over several consecutive steps (pos advances on the device), eagerly and as a
replayed hipGraph. State is compared after every step (the reference's state-cloning check pattern,
engine/check_fused.py:20-34).

Tolerances: every activation is stored in fp16 and the step chains ~8 kernels per layer, so results are compared by
norm-relative error / cosine: hidden state and logits within 1e-2 / 0.9999 per step on the small model and on the
full-width model (4 layers of the 36-layer shape; each layer is the same computation).
"""
import numpy as np
import pytest
import torch

import decode
from oracle import glue as OG
from oracle import int4 as O

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().float().cpu().numpy()


def _oracle_model(cfg, w):
    n = lambda t: t.cpu().numpy()  # noqa: E731
    cos, sin = OG.rope_tables(cfg.S, cfg.HD, cfg.rope_theta)
    return OG.DecodeModel(
        L=cfg.L, H=cfg.H, NH=cfg.NH, NKV=cfg.NKV, HD=cfg.HD, inter=cfg.inter, eps=cfg.eps,
        w_in=[tuple(map(n, t)) for t in w["w_in"]], w_o=[tuple(map(n, t)) for t in w["w_o"]],
        w_down=[tuple(map(n, t)) for t in w["w_down"]], ln=[n(t) for t in w["ln"]], norm=n(w["norm"]),
        emb=(n(w["emb"][0]), n(w["emb"][1])), head=(n(w["head"][0]), n(w["head"][1])),
        rope=(cos.astype(np.float16).astype(np.float32), sin.astype(np.float16).astype(np.float32)),
        sliding=cfg.sliding)


def _run(cfg, dev, ctx, steps, use_graph, seed=4, tol=1e-2, engine="graph"):
    w = decode.random_weights(cfg, seed, device="cpu", gen_device="cpu")
    wd = {k: ([tuple(t.to(dev) for t in v) if isinstance(v, tuple) else v.to(dev) for v in vv]
              if isinstance(vv, list) else (tuple(t.to(dev) for t in vv) if isinstance(vv, tuple) else vv.to(dev)))
          for k, vv in w.items()}
    eng = decode.DecodeStep(cfg, wd, device=dev) if engine == "graph" else decode.PersistentDecode(cfg, wd, device=dev)
    g = torch.Generator().manual_seed(seed + 1)
    kc = torch.zeros(cfg.L, cfg.NKV, cfg.S, cfg.HD, dtype=torch.float16)
    kc[:, :, :ctx] = torch.randn(cfg.L, cfg.NKV, ctx, cfg.HD, generator=g).half()
    vc = torch.zeros_like(kc)
    vc[:, :, :ctx] = torch.randn(cfg.L, cfg.NKV, ctx, cfg.HD, generator=g).half()
    eng.kc.copy_(kc.to(dev))
    eng.vc.copy_(vc.to(dev))
    tok = 7
    eng.set_state(tok, ctx)
    if use_graph:
        eng.capture()
    md = _oracle_model(cfg, w)
    okc, ovc = kc.numpy().copy(), vc.numpy().copy()
    reps = []
    for s in range(steps):
        pos = ctx + s
        eng.replay() if use_graph else eng.step()
        torch.cuda.synchronize()
        logits, h, x = OG.decode_step(md, tok, pos, okc, ovc)
        assert int(eng.pos.item()) == pos + 1
        if engine == "persistent":
            assert eng.status_word() == 0, "a grid barrier timed out"
        rx = O.parity_report(_np(eng.x), x)
        rl = O.parity_report(_np(eng.logits), logits)
        if engine == "persistent":  # the exported final hidden state (the sampler's input)
            rh = O.parity_report(_np(eng.hn), h)
            assert rh["norm_rel"] < tol and rh["cosine"] > 0.9999, (s, rh)
        reps.append((rx, rl))
        assert rx["norm_rel"] < tol and rx["cosine"] > 0.9999, (s, rx)
        assert rl["norm_rel"] < tol and rl["cosine"] > 0.9999, (s, rl)
        # this step's K/V were written at slot pos of every layer
        np.testing.assert_allclose(_np(eng.vc[:, :, pos]), ovc[:, :, pos].astype(np.float32), rtol=1e-2, atol=1e-2)
        # continue from the oracle's own state for the next step, so errors do not compound across steps
        eng.x.copy_(torch.tensor(x).half().to(dev))
        eng.kc[:, :, pos].copy_(torch.tensor(okc[:, :, pos]).to(dev))
        eng.vc[:, :, pos].copy_(torch.tensor(ovc[:, :, pos]).to(dev))
    return reps


SMALL = dict(L=3, H=256, NH=4, NKV=2, HD=128, inter=384, S=64, n_audio=100, vocab=50, nsplit=8)


@pytest.mark.parametrize("use_graph", [False, True])
def test_small_model_steps(use_graph, dev):
    cfg = decode.Config(**SMALL)
    reps = _run(cfg, dev, ctx=5, steps=4, use_graph=use_graph)
    print(reps[-1])


def test_full_width_four_layers(dev):
    cfg = decode.Config(L=4, vocab=64)
    reps = _run(cfg, dev, ctx=300, steps=2, use_graph=True)
    print(reps[-1])


@pytest.mark.parametrize("use_graph", [False, True])
def test_persistent_full_width(use_graph, dev):
    # the one-launch step: hidden 2048, 16 / 4 heads, MLP 11008, 3 layers (one of them NoPE), ctx 300
    cfg = decode.Config(L=3, vocab=64, sliding=[True, False, True])
    reps = _run(cfg, dev, ctx=300, steps=3, use_graph=use_graph, engine="persistent")
    print(reps[-1])


def test_persistent_small_mlp_and_ctx_edges(dev):
    # inter 2048, contexts at the edges: first slot and the last slot of the cache
    cfg = decode.Config(L=2, inter=2048, S=256, vocab=32, n_audio=1000)
    _run(cfg, dev, ctx=0, steps=2, use_graph=True, engine="persistent")
    _run(cfg, dev, ctx=254, steps=2, use_graph=False, engine="persistent")


def test_persistent_step_with_sampler_token_loop(dev):
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
    eng = decode.PersistentDecode(cfg, wd, device=dev)
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
