"""Prompt prefill on the GPU (rumik-fast_amd/engine/prefill.py: rk_embed_ln_rows, mm_int4, rk_post_rows,
rk_prefill_attn, rk_add_ln_rows; the reference's RumikFused.prefill, engine/rumik_fused.py:54-78):

- the matrix-core causal attention against the oracle's causal_attend (engine/rumik_int4.py:163-171, fp32) for
  prompts of 1, 16, 37 and 130 tokens and for a prompt that continues a filled cache (p0 > 0): norm-relative
  error <= 1e-2 and cosine >= 0.9999 per query row and head (P is fp16, as the reference's tensor-core PV);
- the whole prefill of a 12-token prompt on a full-width 2-layer model against the decode oracle stepped over the
  prompt one position at a time (the same maths, causal): every K / V cache slot and the final hidden state;
- the generate loop started from the batched prefill: the first token's logits are the head of the oracle's final
  hidden state, and the frames that follow are valid audio tokens."""
import numpy as np
import pytest
import torch

import decode
import prefill as PF
from generate import Generator
from oracle import glue as OG
from oracle import int4 as O

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize("T,p0", [(1, 0), (16, 0), (37, 0), (130, 0), (20, 50)])
def test_prefill_attention_matches_oracle(dev, T, p0):
    NH, NKV, HD, S = 16, 4, 128, 256
    g = torch.Generator().manual_seed(T + 7 * p0)
    q = torch.randn(T, NH * HD, generator=g).half()
    kc = torch.zeros(NKV, S, HD, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    kc[:, :p0 + T] = torch.randn(NKV, p0 + T, HD, generator=g).half()
    vc[:, :p0 + T] = torch.randn(NKV, p0 + T, HD, generator=g).half()
    o = torch.empty(T, NH * HD, dtype=torch.float16, device=dev)
    PF.prefill_attn(q.to(dev), kc.to(dev), vc.to(dev), o, T, p0, NH, NKV, HD, S, HD ** -0.5)
    torch.cuda.synchronize()
    ref = OG.causal_attend(q.float().numpy().reshape(T, NH, HD), kc.numpy(), vc.numpy(), p0)
    got = _np(o).reshape(T, NH, HD)
    for t in range(T):
        for h in range(NH):
            rep = O.parity_report(got[t, h], ref[t, h])
            assert rep["norm_rel"] < 1e-2 and rep["cosine"] > 0.9999, (t, h, rep)


def _model(dev, seed=21):
    cfg = decode.Config(L=2, vocab=300, n_audio=500, S=256, sliding=[True, False])
    w = decode.random_weights(cfg, seed, device="cpu", gen_device="cpu")
    wd = {k: ([tuple(t.to(dev) for t in v) if isinstance(v, tuple) else v.to(dev) for v in vv]
              if isinstance(vv, list) else (tuple(t.to(dev) for t in vv) if isinstance(vv, tuple) else vv.to(dev)))
          for k, vv in w.items()}
    n = lambda t: t.numpy()  # noqa: E731
    cos, sin = OG.rope_tables(cfg.S, cfg.HD, cfg.rope_theta)
    md = OG.DecodeModel(
        L=cfg.L, H=cfg.H, NH=cfg.NH, NKV=cfg.NKV, HD=cfg.HD, inter=cfg.inter, eps=cfg.eps,
        w_in=[tuple(map(n, t)) for t in w["w_in"]], w_o=[tuple(map(n, t)) for t in w["w_o"]],
        w_down=[tuple(map(n, t)) for t in w["w_down"]], ln=[n(t) for t in w["ln"]], norm=n(w["norm"]),
        emb=(n(w["emb"][0]), n(w["emb"][1])), head=(n(w["head"][0]), n(w["head"][1])),
        rope=(cos.astype(np.float16).astype(np.float32), sin.astype(np.float16).astype(np.float32)),
        sliding=cfg.sliding)
    return cfg, wd, md


def test_prefill_matches_stepwise_oracle(dev):
    cfg, wd, md = _model(dev)
    eng = decode.PersistentDecode(cfg, wd, device=dev, keep_layer_weights=True)
    pf = PF.Prefill(cfg, wd, eng.kc, eng.vc, eng.cos, eng.sin, max_T=64)
    ids = [int(v) for v in torch.randint(0, cfg.vocab, (12,), generator=torch.Generator().manual_seed(4))]
    hn = pf.run(ids, hn=eng.hn)
    torch.cuda.synchronize()
    okc = np.zeros((cfg.L, cfg.NKV, cfg.S, cfg.HD), np.float16)
    ovc = np.zeros_like(okc)
    for t, tok in enumerate(ids):
        _, h, x = OG.decode_step(md, tok, t, okc, ovc)
    for got, ref in ((eng.kc[:, :, :12], okc[:, :, :12]), (eng.vc[:, :, :12], ovc[:, :, :12]), (hn, h)):
        rep = O.parity_report(_np(got).reshape(-1), ref.astype(np.float32).reshape(-1))
        assert rep["norm_rel"] < 1e-2 and rep["cosine"] > 0.9999, rep
    # each layer's cache rows, slot by slot
    for i in range(cfg.L):
        for t in (0, 5, 11):
            rep = O.parity_report(_np(eng.kc[i, :, t]).reshape(-1), okc[i, :, t].astype(np.float32).reshape(-1))
            assert rep["norm_rel"] < 1e-2, (i, t, rep)


def test_generate_from_batched_prefill(dev):
    cfg, wd, md = _model(dev, seed=22)
    eng = decode.PersistentDecode(cfg, wd, device=dev, keep_layer_weights=True)
    g = torch.Generator().manual_seed(5)
    stop = {"0.weight": torch.ones(cfg.H), "0.bias": torch.zeros(cfg.H),
            "1.weight": (torch.randn(512, cfg.H, generator=g) / cfg.H ** 0.5).bfloat16(),
            "1.bias": torch.zeros(512), "3.weight": torch.randn(1, 512, generator=g) / 512 ** 0.5 * 0.01,
            "3.bias": torch.tensor([-50.0])}
    ids_head = torch.arange(cfg.n_audio, dtype=torch.int64) % (cfg.vocab - 1)
    ids_head[-1] = cfg.vocab - 1
    eng.attach_sampler(stop, ids_head, end_id=cfg.vocab - 1, max_new=40)
    pf = PF.Prefill(cfg, wd, eng.kc, eng.vc, eng.cos, eng.sin, max_T=64)
    gen = Generator(eng, Q=8, max_new=32, prefill=pf)
    prompt = [3, 50, 7, 99, 120, 5, 8]
    first = int(gen.prefill(prompt))
    torch.cuda.synchronize()
    okc = np.zeros((cfg.L, cfg.NKV, cfg.S, cfg.HD), np.float16)
    ovc = np.zeros_like(okc)
    for t, tok in enumerate(prompt):
        logits, h, x = OG.decode_step(md, tok, t, okc, ovc)
    rep = O.parity_report(_np(eng.logits), logits)
    assert rep["norm_rel"] < 1e-2 and rep["cosine"] > 0.9999, rep
    assert int(eng.pos.item()) == len(prompt) and int(eng.out[0].item()) == first
    toks, st = gen.generate(prompt, seed=1)
    print(st)
    assert len(toks) == 33 and all(0 <= t < cfg.vocab - 1 for t in toks)
