"""Prompt prefill on the GPU (rumik-fast_amd/engine/prefill.py: rk_embed_ln_rows, mm_int4, rk_post_rows,
rk_prefill_attn, rk_add_ln_rows; the reference's RumikFused.prefill, engine/rumik_fused.py:54-78):

- the matrix-core causal attention against the oracle's causal_attend (engine/rumik_int4.py:163-171, fp32) for
  prompts of 1, 16, 37, 130 and 512 tokens (512: the benchmarked prompt) and for prompts that continue a filled
  cache (p0 > 0): norm-relative error <= 1e-2 and cosine >= 0.9999 per query row and head (P is fp16, as the
  reference's tensor-core PV);
- the whole prefill of 12-, 69- and 512-token prompts on a full-width 2-layer model against the decode oracle
  stepped over the prompt one position at a time (the same maths, causal): every K / V cache slot and the final
  hidden state;
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


def _rows_close(got, ref, tol=1e-2):
    """per (query row, head): norm-relative error < tol and cosine > 0.9999 (got / ref [T, NH, HD])"""
    g = got.astype(np.float64)
    r = ref.astype(np.float64)
    nr = np.linalg.norm(g - r, axis=-1) / np.linalg.norm(r, axis=-1)
    cos = (g * r).sum(-1) / (np.linalg.norm(g, axis=-1) * np.linalg.norm(r, axis=-1))
    t, h = np.unravel_index(int(np.argmax(nr - cos)), nr.shape)
    assert (nr < tol).all() and (cos > 0.9999).all(), (int(t), int(h), float(nr[t, h]), float(cos[t, h]))


@pytest.mark.parametrize("T,p0,NKV,qs,ramp", [(1, 0, 4, 1, 0), (16, 0, 4, 1, 0), (37, 0, 4, 1, 0), (130, 0, 4, 1, 0),
                                              (20, 50, 4, 1, 0), (512, 0, 4, 1, 0), (512, 50, 4, 1, 0),
                                              (130, 0, 8, 1, 0), (130, 0, 2, 1, 0), (384, 0, 4, 1, 0),
                                              (385, 0, 4, 1, 0), (300, 100, 4, 1, 0), (512, 0, 4, 6, 1),
                                              (200, 0, 4, 6, 1), (96, 0, 4, 4, 2)])
def test_prefill_attention_matches_oracle(dev, T, p0, NKV, qs, ramp):
    """T = 512 is the benchmarked prompt (16 key blocks of 32 per query tile at the last tile); NKV 8 / 2 give 2 / 8
    query heads per KV head (other wave layouts of the block); p0 + T = 384 / 385 sit on either side of the switch
    to four key groups per block. qs scales q (score ranges of tens), and ramp grows the keys' norm along the
    sequence (1: slot 0 x0.2 .. last slot x3, so a row's running max keeps moving in later key blocks and the lazy
    rescale fires mid-loop; 2: the reverse, the max set by the first blocks)."""
    NH, HD = 16, 128
    S = 256 if p0 + T <= 256 else 640
    g = torch.Generator().manual_seed(T + 7 * p0 + 13 * ramp)
    q = (torch.randn(T, NH * HD, generator=g) * qs).half()
    kc = torch.zeros(NKV, S, HD, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    kr = torch.randn(NKV, p0 + T, HD, generator=g)
    if ramp:
        gain = torch.linspace(0.2, 3.0, p0 + T) if ramp == 1 else torch.linspace(3.0, 0.2, p0 + T)
        kr = kr * gain[None, :, None]
    kc[:, :p0 + T] = kr.half()
    vc[:, :p0 + T] = torch.randn(NKV, p0 + T, HD, generator=g).half()
    o = torch.empty(T, NH * HD, dtype=torch.float16, device=dev)
    PF.prefill_attn(q.to(dev), kc.to(dev), vc.to(dev), o, T, p0, NH, NKV, HD, S, HD ** -0.5)
    torch.cuda.synchronize()
    ref = OG.causal_attend(q.float().numpy().reshape(T, NH, HD), kc.numpy(), vc.numpy(), p0)
    _rows_close(_np(o).reshape(T, NH, HD), ref)


def _model(dev, seed=21, S=256):
    cfg = decode.Config(L=2, vocab=300, n_audio=500, S=S, sliding=[True, False])
    w = decode.random_weights(cfg, seed, device="cpu", gen_device="cpu")
    wd = {k: ([tuple(t.to(dev) for t in v) if isinstance(v, tuple) else v.to(dev) for v in vv]
              if isinstance(vv, list) else (tuple(t.to(dev) for t in vv) if isinstance(vv, tuple) else vv.to(dev)))
          for k, vv in w.items()}
    n = lambda t: t.numpy()  # noqa: E731
    cos, sin = OG.rope_tables(cfg.S, cfg.HD, cfg.rope_theta)
    md = OG.DecodeModel(cache_weights=True,
        L=cfg.L, H=cfg.H, NH=cfg.NH, NKV=cfg.NKV, HD=cfg.HD, inter=cfg.inter, eps=cfg.eps,
        w_in=[tuple(map(n, t)) for t in w["w_in"]], w_o=[tuple(map(n, t)) for t in w["w_o"]],
        w_down=[tuple(map(n, t)) for t in w["w_down"]], ln=[n(t) for t in w["ln"]], norm=n(w["norm"]),
        emb=(n(w["emb"][0]), n(w["emb"][1])), head=(n(w["head"][0]), n(w["head"][1])),
        rope=(cos.astype(np.float16).astype(np.float32), sin.astype(np.float16).astype(np.float32)),
        sliding=cfg.sliding)
    return cfg, wd, md


@pytest.mark.timeout(600)
@pytest.mark.parametrize("T", [12, 69, 512])
def test_prefill_matches_stepwise_oracle(dev, T):
    """The whole batched prefill against the decode oracle stepped over the prompt (the reference's decode-vs-prefill
    consistency check, engine/check.py:46-56); T = 69 and T = 512 are the benchmarked prompt lengths (at 512 the
    w_in product takes the prepared-X plan and the attention walks 16 key blocks)."""
    cfg, wd, md = _model(dev, S=256 if T < 256 else 640)
    eng = decode.PersistentDecode(cfg, wd, device=dev, keep_layer_weights=True)
    pf = PF.Prefill(cfg, wd, eng.kc, eng.vc, eng.cos, eng.sin, max_T=max(128, T))
    ids = [int(v) for v in torch.randint(0, cfg.vocab, (T,), generator=torch.Generator().manual_seed(4))]
    hn = pf.run(ids, hn=eng.hn)
    torch.cuda.synchronize()
    okc = np.zeros((cfg.L, cfg.NKV, cfg.S, cfg.HD), np.float16)
    ovc = np.zeros_like(okc)
    for t, tok in enumerate(ids):
        _, h, x = OG.decode_step(md, tok, t, okc, ovc)
    for got, ref in ((eng.kc[:, :, :T], okc[:, :, :T]), (eng.vc[:, :, :T], ovc[:, :, :T]), (hn, h)):
        rep = O.parity_report(_np(got).reshape(-1), ref.astype(np.float32).reshape(-1))
        assert rep["norm_rel"] < 1e-2 and rep["cosine"] > 0.9999, rep
    # each layer's cache rows, slot by slot
    for i in range(cfg.L):
        for t in (0, T // 2, T - 1):
            rep = O.parity_report(_np(eng.kc[i, :, t]).reshape(-1), okc[i, :, t].astype(np.float32).reshape(-1))
            assert rep["norm_rel"] < 1e-2, (i, t, rep)


def test_prefill_graph_buckets_match_eager(dev):
    """Prefill(graphs=True): each prompt replays the hipGraph of its length rounded up to 16 (the rows past the
    prompt run on token 0). Against the eager prefill of the same prompt: the final hidden state and cache slots
    0..T-1 of every layer (the padded rows change none of the prompt's rows; the products' plans may differ with the
    padded row count, so the bar is the parity tolerance, not bit equality). Prompts of 37 and 45 tokens share the
    48-row graph (captured once, replayed with new ids), 69 tokens takes the 80-row one."""
    cfg, wd, md = _model(dev, S=256)
    eng = decode.PersistentDecode(cfg, wd, device=dev, keep_layer_weights=True)
    eager = PF.Prefill(cfg, wd, eng.kc, eng.vc, eng.cos, eng.sin, max_T=128)
    graph = PF.Prefill(cfg, wd, eng.kc, eng.vc, eng.cos, eng.sin, max_T=128, graphs=True)
    g = torch.Generator().manual_seed(8)
    for T in (37, 45, 69):
        ids = [int(v) for v in torch.randint(0, cfg.vocab, (T,), generator=g)]
        h_e = eager.run(ids).clone()
        kc_e, vc_e = eng.kc[:, :, :T].clone(), eng.vc[:, :, :T].clone()
        eng.kc.zero_(); eng.vc.zero_()
        h_g = graph.run(ids).clone()
        torch.cuda.synchronize()
        for name, got, ref in (("hn", h_g, h_e), ("k", eng.kc[:, :, :T], kc_e), ("v", eng.vc[:, :, :T], vc_e)):
            rep = O.parity_report(_np(got).reshape(-1), _np(ref).reshape(-1))
            assert rep["norm_rel"] < 1e-3 and rep["cosine"] > 0.99999, (T, name, rep)
    assert sorted(graph.graphs) == [48, 80]


@pytest.mark.parametrize("T", [37, 300])
def test_prefill_overlap_is_bit_identical(dev, T):
    """The down product's branch on a second stream (overlap=True) runs the same kernels on the same inputs as the
    serial order, so the final hidden state and every K / V slot written are bit-identical; both eagerly and, for
    T = 37, as a graph replay (graphs=True; 48 rows)."""
    cfg, wd, md = _model(dev, S=512)
    eng = decode.PersistentDecode(cfg, wd, device=dev, keep_layer_weights=True)
    ids = [int(v) for v in torch.randint(0, cfg.vocab, (T,), generator=torch.Generator().manual_seed(T))]
    outs = []
    for kw in (dict(overlap=False), dict(overlap=True), dict(overlap=True, graphs=True)):
        if kw.get("graphs") and T > 64:
            continue
        eng.kc.zero_(); eng.vc.zero_()
        pf = PF.Prefill(cfg, wd, eng.kc, eng.vc, eng.cos, eng.sin, max_T=max(64, T), **kw)
        h = pf.run(ids).clone()
        torch.cuda.synchronize()
        outs.append((h, eng.kc[:, :, :T].clone(), eng.vc[:, :, :T].clone()))
    for other in outs[1:]:
        for a, b in zip(outs[0], other):
            assert torch.equal(a, b)


@pytest.mark.parametrize("kind", ["roles", "persistent"])
def test_generate_from_batched_prefill(dev, kind):
    cfg, wd, md = _model(dev, seed=22)
    eng = (decode.RoleDecode if kind == "roles" else decode.PersistentDecode)(cfg, wd, device=dev,
                                                                              keep_layer_weights=True)
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


# ---- the row kernels on their own (vector path: H % 8 == 0 and 16-byte aligned rows; scalar path otherwise)
@pytest.mark.parametrize("dtype,H,T,offset", [(torch.float16, 2048, 37, 0), (torch.bfloat16, 2048, 5, 0),
                                              (torch.float16, 200, 9, 0), (torch.float16, 196, 9, 0),
                                              (torch.float16, 2048, 3, 1), (torch.float16, 4096, 6, 0),
                                              (torch.bfloat16, 8192, 3, 0)])
def test_add_ln_rows(dev, dtype, H, T, offset):
    """x[t] = dt(x[t] + a[t] + b[t]) exactly; h[t] = LayerNorm(x[t]) * w against the oracle's fp32 LayerNorm.
    H = 200 takes the vector kernel with a partial last pass, H = 4096 / 8192 with two / four passes, H = 196 (rows
    not 16-byte aligned) and offset = 1 (every buffer shifted by one element) the scalar one."""
    g = torch.Generator().manual_seed(H + T)
    x, a, b = (torch.randn(T * H + offset, generator=g).to(dtype) for _ in range(3))
    w = (torch.rand(H + offset, generator=g) + 0.5).to(dtype)
    xd, ad, bd, wd = (t.to(dev) for t in (x, a, b, w))
    hd = torch.empty(T * H + offset, dtype=dtype, device=dev)
    PF.add_ln_rows(xd[offset:], ad[offset:], bd[offset:], wd[offset:], hd[offset:], T, 1e-5)
    torch.cuda.synchronize()
    xs = (x[offset:].float() + a[offset:].float() + b[offset:].float()).to(dtype)
    assert torch.equal(xd[offset:].cpu(), xs)
    tol = 2e-3 if dtype == torch.float16 else 1.6e-2
    wf = w[offset:].float().numpy()
    for t in range(T):
        ref = OG.cohere_ln(xs[t * H:(t + 1) * H].float().numpy(), wf)
        np.testing.assert_allclose(_np(hd[offset + t * H:offset + (t + 1) * H]), ref, rtol=tol, atol=tol)


@pytest.mark.parametrize("dtype,H", [(torch.float16, 2048), (torch.bfloat16, 2048), (torch.float16, 200),
                                     (torch.float16, 196)])
def test_embed_ln_rows(dev, dtype, H):
    g = torch.Generator().manual_seed(H)
    eq = torch.randint(-127, 128, (40, H), generator=g, dtype=torch.int8)
    es = (torch.rand(40, generator=g) * 0.01 + 1e-3).half()
    w = (torch.rand(H, generator=g) + 0.5).to(dtype)
    ids = torch.tensor([3, 17, 39, 0, 17], dtype=torch.int64)
    x = torch.empty(len(ids), H, dtype=dtype, device=dev)
    h = torch.empty_like(x)
    PF.embed_ln_rows(ids.to(dev), eq.to(dev), es.to(dev), w.to(dev), x, h, 1e-5)
    torch.cuda.synchronize()
    tol = 2e-3 if dtype == torch.float16 else 1.6e-2
    for t, i in enumerate(ids.tolist()):
        xr = (eq[i].float() * es[i].float()).to(dtype)
        assert torch.equal(x[t].cpu(), xr)
        np.testing.assert_allclose(_np(h[t]), OG.cohere_ln(xr.float().numpy(), w.float().numpy()), rtol=tol, atol=tol)


@pytest.mark.parametrize("dtype,p0,T,rope,act_offset", [(torch.float16, 0, 7, True, 0), (torch.float16, 100, 33, True, 0),
                                                        (torch.bfloat16, 5, 4, True, 0), (torch.float16, 9, 6, False, 0),
                                                        (torch.float16, 3, 5, True, 1)])
def test_post_rows(dev, dtype, p0, T, rope, act_offset):
    """per row t at position p0 + t: q / k with the interleaved RoPE (oracle.rope), K / V into the cache slot, v
    copied exactly, act = silu(gate) * up (oracle.silu); act_offset = 1 misaligns act (the scalar kernel)."""
    NH, NKV, HD, inter, S = 16, 4, 128, 11008, 256
    n_in = (NH + 2 * NKV) * HD + 2 * inter
    g = torch.Generator().manual_seed(p0 + T)
    y = torch.randn(T, n_in, generator=g).to(dtype)
    cos, sin = (torch.tensor(t).to(dtype) for t in OG.rope_tables(S, HD))
    kc = torch.zeros(NKV, S, HD, dtype=dtype, device=dev)
    vc = torch.zeros_like(kc)
    qo = torch.empty(T, NH * HD, dtype=dtype, device=dev)
    actb = torch.empty(T * inter + act_offset, dtype=dtype, device=dev)
    PF.post_rows(y.to(dev), p0, cos.to(dev), sin.to(dev), kc, vc, qo, actb[act_offset:], T, NH, NKV, HD, S, inter,
                 rope)
    torch.cuda.synchronize()
    act = actb[act_offset:].view(T, inter)
    tol = 2e-3 if dtype == torch.float16 else 1.6e-2
    for t in range(T):
        yf = y[t].float().numpy()
        q = yf[:NH * HD].reshape(NH, HD)
        k = yf[NH * HD:(NH + NKV) * HD].reshape(NKV, HD)
        v = yf[(NH + NKV) * HD:(NH + 2 * NKV) * HD].reshape(NKV, HD)
        gt, up = yf[(NH + 2 * NKV) * HD:][:inter], yf[(NH + 2 * NKV) * HD:][inter:]
        pos = p0 + t
        if rope:
            q = OG.rope(q, cos[pos].float().numpy(), sin[pos].float().numpy())
            k = OG.rope(k, cos[pos].float().numpy(), sin[pos].float().numpy())
        else:
            assert np.array_equal(_np(qo[t]).reshape(NH, HD), q)
        np.testing.assert_allclose(_np(qo[t]).reshape(NH, HD), q, rtol=tol, atol=tol)
        np.testing.assert_allclose(_np(kc[:, pos]), k, rtol=tol, atol=tol)
        assert np.array_equal(_np(vc[:, pos]), v)
        np.testing.assert_allclose(_np(act[t]), OG.silu(gt) * up, rtol=tol, atol=tol)
    untouched = torch.ones(S, dtype=torch.bool)
    untouched[p0:p0 + T] = False
    assert torch.count_nonzero(kc[:, untouched]) == 0 and torch.count_nonzero(vc[:, untouched]) == 0
