"""A checkpoint in the reference's int4 format, loaded and run: a full-width synthetic model (hidden 2048, 16 / 4
heads of 128, MLP 11008, 2 layers, one of them NoPE; 1200-token vocabulary, 1000 audio rows) is written by the
exporter mapping, loaded by rumik-fast_amd/engine/weights.py onto the GPU, and stepped by the one-launch engine with
the sampling tail in its graph. Each step's hidden state and logits are compared with the decode oracle run on the
loaded tensors (oracle/glue.py, norm-relative error <= 1e-2 and cosine >= 0.9999, as tests/test_decode_gpu.py), and
each sampled token is a token id of the head (audio_ids) that the next step embeds."""
import time

import numpy as np
import pytest
import torch

import decode
import weights as W
from oracle import glue as OG
from oracle import int4 as O

pytestmark = pytest.mark.gpu

CFG = {"num_hidden_layers": 2, "hidden_size": 2048, "num_attention_heads": 16, "num_key_value_heads": 4,
       "head_dim": 128, "intermediate_size": 11008, "layer_norm_eps": 1e-5, "rope_theta": 10000.0,
       "layer_types": ["sliding_attention", "full_attention"], "audio_end_token_id": 299}


def _np(t):
    return t.detach().float().cpu().numpy()


def test_loaded_checkpoint_decodes_like_the_oracle(dev, tmp_path):
    st = W.synthetic_float_model(CFG, vocab=1200, n_audio=1000, seed=5)
    path = tmp_path / "rumik-int4.safetensors"
    W.save(path, W.export_int4(st), CFG)
    nbytes = path.stat().st_size
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    cfg, w, extras = W.load(path, tmp_path / "config.json", device=dev, S=512)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    print(f"\n[load] {nbytes / 1e6:.1f} MB in {dt:.2f} s ({nbytes / dt / 1e9:.2f} GB/s)", flush=True)
    wc = {k: ([tuple(t.cpu() for t in v) if isinstance(v, tuple) else v.cpu() for v in vv]
              if isinstance(vv, list) else (tuple(t.cpu() for t in vv) if isinstance(vv, tuple) else vv.cpu()))
          for k, vv in w.items()}
    n = lambda t: t.numpy()  # noqa: E731
    cos, sin = OG.rope_tables(cfg.S, cfg.HD, cfg.rope_theta)
    md = OG.DecodeModel(
        L=cfg.L, H=cfg.H, NH=cfg.NH, NKV=cfg.NKV, HD=cfg.HD, inter=cfg.inter, eps=cfg.eps,
        w_in=[tuple(map(n, t)) for t in wc["w_in"]], w_o=[tuple(map(n, t)) for t in wc["w_o"]],
        w_down=[tuple(map(n, t)) for t in wc["w_down"]], ln=[n(t) for t in wc["ln"]], norm=n(wc["norm"]),
        emb=(n(wc["emb"][0]), n(wc["emb"][1])), head=(n(wc["head"][0]), n(wc["head"][1])),
        rope=(cos.astype(np.float16).astype(np.float32), sin.astype(np.float16).astype(np.float32)),
        sliding=cfg.sliding)
    eng = decode.PersistentDecode(cfg, w, device=dev)
    eng.attach_sampler(extras["stop"], extras["audio_ids"], extras["end_id"])
    g = torch.Generator().manual_seed(6)
    ctx = 20
    kc = torch.zeros(cfg.L, cfg.NKV, cfg.S, cfg.HD, dtype=torch.float16)
    kc[:, :, :ctx] = torch.randn(cfg.L, cfg.NKV, ctx, cfg.HD, generator=g).half()
    vc = torch.zeros_like(kc)
    vc[:, :, :ctx] = torch.randn(cfg.L, cfg.NKV, ctx, cfg.HD, generator=g).half()
    eng.kc.copy_(kc.to(dev))
    eng.vc.copy_(vc.to(dev))
    tok = int(extras["audio_ids"][3])
    eng.set_state(tok, ctx)
    eng.capture()
    okc, ovc = kc.numpy().copy(), vc.numpy().copy()
    ids = set(extras["audio_ids"].tolist())
    for s in range(3):
        eng.replay()
        torch.cuda.synchronize()
        assert eng.status_word() == 0
        logits, h, x = OG.decode_step(md, tok, ctx + s, okc, ovc)
        for got, ref in ((eng.x, x), (eng.hn, h), (eng.logits, logits)):
            rep = O.parity_report(_np(got), ref)
            assert rep["norm_rel"] < 1e-2 and rep["cosine"] > 0.9999, (s, rep)
        new = int(eng.tok.item())
        assert new in ids and int(eng.out[s].item()) == new
        tok = new
        eng.kc[:, :, ctx + s].copy_(torch.tensor(okc[:, :, ctx + s]).to(dev))
        eng.vc[:, :, ctx + s].copy_(torch.tensor(ovc[:, :, ctx + s]).to(dev))
