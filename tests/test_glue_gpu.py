"""Decode-step glue kernels on the GPU vs the CPU oracle (oracle/glue.py).

Closed-form checks: LayerNorm of a constant vector is 0; RoPE at position 0 and on NoPE layers is the identity and
preserves pair norms; attention at pos 0 returns v[0]; with q = 0 it returns the mean of V[0..pos]; the split
combine equals the unsplit softmax. The attention positions are the reference's own (engine/test_attn.py:47).
Tolerances: activations are stored in fp16, so element errors are bounded by fp16 rounding of the outputs
(relative 2^-11) plus fp32 math differences; attention is held to a norm-relative 2e-3 (the reference reports
0.17% / 0.21% for its Triton kernels, engine/README.md:80).
"""
import math

import numpy as np
import pytest
import torch

import fused
from oracle import glue as OG
from oracle import int4 as O

pytestmark = pytest.mark.gpu
F16 = torch.float16


def _np(t):
    return t.detach().float().cpu().numpy()


def test_add_ln_matches_oracle(dev):
    g = torch.Generator().manual_seed(0)
    x, a, b = (torch.randn(2048, generator=g).half() for _ in range(3))
    w = (torch.rand(2048, generator=g) + 0.5).half()
    xd, hd = x.to(dev), torch.empty(2048, dtype=F16, device=dev)
    fused.add_ln(xd, a.to(dev), b.to(dev), w.to(dev), hd, 1e-5)
    xs = (x.float() + a.float() + b.float()).half()
    assert torch.equal(xd.cpu(), xs)  # the residual sum is rounded once, exactly as the oracle does
    ref = OG.cohere_ln(xs.float().numpy(), w.float().numpy()).astype(np.float16).astype(np.float32)
    np.testing.assert_allclose(_np(hd), ref, rtol=2e-3, atol=2e-3)


def test_layernorm_of_constant_is_zero(dev):
    x = torch.full((2048,), 3.0, dtype=F16, device=dev)
    h = torch.empty_like(x)
    fused.add_ln(x, torch.zeros_like(x), None, torch.ones_like(x), h, 1e-5)
    assert torch.count_nonzero(h) == 0


def test_embed_ln(dev):
    g = torch.Generator().manual_seed(1)
    eq = torch.randint(-127, 128, (50, 2048), generator=g, dtype=torch.int8)
    es = (torch.rand(50, generator=g) * 0.01 + 1e-3).half()
    w = (torch.rand(2048, generator=g) + 0.5).half()
    tok = torch.tensor([17], dtype=torch.int64, device=dev)
    x, h = torch.empty(2048, dtype=F16, device=dev), torch.empty(2048, dtype=F16, device=dev)
    fused.embed_ln(tok, eq.to(dev), es.to(dev), w.to(dev), x, h, 1e-5)
    xr = (eq[17].float() * es[17].float()).half()
    assert torch.equal(x.cpu(), xr)
    ref = OG.cohere_ln(xr.float().numpy(), w.float().numpy())
    np.testing.assert_allclose(_np(h), ref, rtol=2e-3, atol=2e-3)


def _post_case(pos, rope, dev, NH=16, NKV=4, HD=128, inter=11008, S=2048):
    g = torch.Generator().manual_seed(2 + pos)
    y = torch.randn((NH + 2 * NKV) * HD + 2 * inter, generator=g).half()
    cos, sin = (torch.tensor(t).half() for t in OG.rope_tables(S, HD))
    kc = torch.zeros(NKV, S, HD, dtype=F16, device=dev)
    vc = torch.zeros_like(kc)
    qo = torch.empty(NH * HD, dtype=F16, device=dev)
    act = torch.empty(inter, dtype=F16, device=dev)
    fused.post[(1,)](y.to(dev), torch.tensor([pos], device=dev), cos.to(dev), sin.to(dev), kc, vc, qo, act, S, inter,
                     NH=NH, NKV=NKV, HD=HD, ROPE=rope, BLOCK=512, num_warps=4)
    return y, cos, sin, kc, vc, qo, act


@pytest.mark.parametrize("pos,rope", [(0, True), (5, True), (1777, True), (300, False)])
def test_post(pos, rope, dev):
    NH, NKV, HD, inter = 16, 4, 128, 11008
    y, cos, sin, kc, vc, qo, act = _post_case(pos, rope, dev)
    yf = y.float().numpy()
    q = yf[:NH * HD].reshape(NH, HD)
    k = yf[NH * HD:(NH + NKV) * HD].reshape(NKV, HD)
    v = yf[(NH + NKV) * HD:(NH + 2 * NKV) * HD].reshape(NKV, HD)
    gt, up = yf[(NH + 2 * NKV) * HD:][:inter], yf[(NH + 2 * NKV) * HD:][inter:]
    if rope:
        q = OG.rope(q, cos[pos].float().numpy(), sin[pos].float().numpy())
        k = OG.rope(k, cos[pos].float().numpy(), sin[pos].float().numpy())
    if pos == 0 or not rope:  # identity rotation: bit-exact copies
        assert np.array_equal(_np(qo).reshape(NH, HD), q)
    np.testing.assert_allclose(_np(qo).reshape(NH, HD), q, rtol=2e-3, atol=2e-3)
    np.testing.assert_allclose(_np(kc[:, pos]), k, rtol=2e-3, atol=2e-3)
    assert np.array_equal(_np(vc[:, pos]), v)
    assert torch.count_nonzero(kc[:, pos + 1:]) == 0 and torch.count_nonzero(kc[:, :pos]) == 0
    np.testing.assert_allclose(_np(act), OG.silu(gt) * up, rtol=2e-3, atol=2e-3)
    # rotation preserves the norm of every pair
    qp = _np(qo).reshape(NH, HD // 2, 2)
    y0 = yf[:NH * HD].reshape(NH, HD // 2, 2)
    np.testing.assert_allclose(np.hypot(qp[..., 0], qp[..., 1]), np.hypot(y0[..., 0], y0[..., 1]), rtol=3e-3, atol=3e-3)


def _attn(q, kc, vc, pos, dev, nsplit=64, NH=16, NKV=4, HD=128):
    po = torch.empty(NH, nsplit, HD, device=dev)
    pm = torch.empty(NH, nsplit, device=dev)
    pl = torch.empty(NH, nsplit, device=dev)
    out = torch.empty(NH * HD, dtype=F16, device=dev)
    p = torch.tensor([pos], device=dev)
    fused.attn_split[(NKV, nsplit)](q, kc, vc, p, po, pm, pl, kc.shape[1], HD ** -0.5, REP=NH // NKV, HD=HD, NSPLIT=nsplit)
    fused.attn_combine[(NH,)](po, pm, pl, p, out, HD=HD, NSPLIT=nsplit)
    torch.cuda.synchronize()
    return out, po, pm, pl


@pytest.mark.parametrize("pos", [0, 31, 100, 300, 777, 1500, 2047])
@pytest.mark.parametrize("nsplit", [16, 64])
def test_attention_vs_oracle(pos, nsplit, dev):
    NH, NKV, HD, S = 16, 4, 128, 2048
    g = torch.Generator().manual_seed(pos)
    kc = torch.randn(NKV, S, HD, generator=g).half()
    vc = torch.randn(NKV, S, HD, generator=g).half()
    q = torch.randn(NH * HD, generator=g).half()
    out, _, pm, pl = _attn(q.to(dev), kc.to(dev), vc.to(dev), pos, dev, nsplit)
    ref = OG.attend(q.float().numpy().reshape(NH, HD), kc[:, :pos + 1].float().numpy(), vc[:, :pos + 1].float().numpy())
    rep = O.parity_report(_np(out), ref.ravel())
    assert rep["norm_rel"] < 2e-3 and rep["cosine"] > 0.99999, rep
    # the split bookkeeping: splits holding no slot carry m = -inf and l = 0
    ch = ((pos + 1 + nsplit - 1) // nsplit + 7) // 8 * 8
    used = np.arange(nsplit) * ch < pos + 1
    assert np.all(np.isinf(_np(pm)[:, ~used])) and np.all(_np(pl)[:, ~used] == 0)
    assert np.all(np.isfinite(_np(pm)[:, used]))
    # same partials as the oracle's split (m and l per split)
    _, om, ol = OG.attend_split(q.float().numpy().reshape(NH, HD), kc[:, :pos + 1].float().numpy(),
                                vc[:, :pos + 1].float().numpy(), nsplit, ch)
    np.testing.assert_allclose(_np(pm)[:, used], om[:, used], rtol=1e-3, atol=1e-3)
    np.testing.assert_allclose(_np(pl)[:, used], ol[:, used], rtol=2e-3, atol=1e-3)


def test_attention_closed_forms(dev):
    NH, NKV, HD, S = 16, 4, 128, 2048
    g = torch.Generator().manual_seed(9)
    kc = torch.randn(NKV, S, HD, generator=g).half().to(dev)
    vc = torch.randn(NKV, S, HD, generator=g).half().to(dev)
    q = torch.randn(NH * HD, generator=g).half().to(dev)
    out, *_ = _attn(q, kc, vc, 0, dev)  # a single slot: softmax weight 1
    expect = vc[:, 0].repeat_interleave(NH // NKV, 0).reshape(-1)
    assert torch.equal(out, expect)
    out, *_ = _attn(torch.zeros_like(q), kc, vc, 999, dev)  # q = 0: uniform weights -> mean of V rows 0..pos
    mean = vc[:, :1000].float().mean(1).repeat_interleave(NH // NKV, 0).reshape(-1)
    np.testing.assert_allclose(_np(out), mean.cpu().numpy(), rtol=2e-3, atol=2e-4)


def test_graph_replay_reads_pos_on_device(dev):
    # one captured split+combine serves every position: pos is read on the GPU
    NH, NKV, HD, S, nsplit = 16, 4, 128, 2048, 64
    g = torch.Generator().manual_seed(3)
    kc = torch.randn(NKV, S, HD, generator=g).half().to(dev)
    vc = torch.randn(NKV, S, HD, generator=g).half().to(dev)
    q = torch.randn(NH * HD, generator=g).half().to(dev)
    pos = torch.tensor([10], device=dev)
    po = torch.empty(NH, nsplit, HD, device=dev)
    pm = torch.empty(NH, nsplit, device=dev)
    pl = torch.empty(NH, nsplit, device=dev)
    out = torch.empty(NH * HD, dtype=F16, device=dev)
    fused.attn_split[(NKV, nsplit)](q, kc, vc, pos, po, pm, pl, kc.shape[1], HD ** -0.5, REP=NH // NKV, HD=HD, NSPLIT=nsplit)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        fused.attn_split[(NKV, nsplit)](q, kc, vc, pos, po, pm, pl, kc.shape[1], HD ** -0.5, REP=NH // NKV, HD=HD, NSPLIT=nsplit)
        fused.attn_combine[(NH,)](po, pm, pl, pos, out, HD=HD, NSPLIT=nsplit)
    for p in (10, 511, 2047, 64):
        pos.fill_(p)
        gr.replay()
        torch.cuda.synchronize()
        ref = OG.attend(_np(q).reshape(NH, HD), _np(kc[:, :p + 1]), _np(vc[:, :p + 1]))
        rep = O.parity_report(_np(out), ref.ravel())
        assert rep["norm_rel"] < 2e-3, (p, rep)


def test_unsplit_attn_matches_split(dev):
    """fused.attn (the reference's unsplit kernel, engine/fused.py:92-125) equals the split + combine result."""
    NH, NKV, HD, S = 16, 4, 128, 256
    g = torch.Generator().manual_seed(9)
    q = torch.randn(NH * HD, generator=g).half().to(dev)
    kc = torch.randn(NKV, S, HD, generator=g).half().to(dev)
    vc = torch.randn(NKV, S, HD, generator=g).half().to(dev)
    pos = torch.tensor([200], device=dev)
    o1 = torch.empty(NH * HD, dtype=F16, device=dev)
    fused.attn[(NH,)](q, kc, vc, pos, o1, S, HD ** -0.5, REP=NH // NKV, HD=HD, BT=64, num_warps=4)
    o2 = _attn(q, kc, vc, 200, dev, nsplit=8)[0]
    torch.cuda.synchronize()
    ref = OG.attend(_np(q).reshape(NH, HD), _np(kc)[:, :201], _np(vc)[:, :201])
    np.testing.assert_allclose(_np(o1).reshape(NH, HD), ref, rtol=1e-2, atol=2e-3)
    np.testing.assert_allclose(_np(o1), _np(o2), rtol=1e-2, atol=2e-3)


# ---- bf16: the reference engine's activation dtype (engine/rumik_fused.py:40-52); the oracle rounds at bf16
BF16 = torch.bfloat16


def _bf(v):
    return OG.round_bf16(np.asarray(v, np.float32))


def test_add_ln_bf16(dev):
    g = torch.Generator().manual_seed(10)
    x, a, b = (torch.randn(2048, generator=g).bfloat16() for _ in range(3))
    w = (torch.rand(2048, generator=g) + 0.5).bfloat16()
    xd, hd = x.to(dev), torch.empty(2048, dtype=BF16, device=dev)
    fused.add_ln(xd, a.to(dev), b.to(dev), w.to(dev), hd, 1e-5)
    xs = _bf(x.float().numpy() + a.float().numpy() + b.float().numpy())
    np.testing.assert_array_equal(_np(xd), xs)  # one rounding of the fp32 sum, bit-exact
    ref = _bf(OG.cohere_ln(xs, w.float().numpy()))
    np.testing.assert_allclose(_np(hd), ref, rtol=8e-3, atol=8e-3)  # bf16 output: 2^-8 relative per value


def test_embed_ln_bf16(dev):
    g = torch.Generator().manual_seed(11)
    eq = torch.randint(-127, 128, (50, 2048), generator=g, dtype=torch.int8)
    es = (torch.rand(50, generator=g) * 0.01 + 1e-3).half()
    w = (torch.rand(2048, generator=g) + 0.5).bfloat16()
    tok = torch.tensor([33], dtype=torch.int64, device=dev)
    x, h = torch.empty(2048, dtype=BF16, device=dev), torch.empty(2048, dtype=BF16, device=dev)
    fused.embed_ln(tok, eq.to(dev), es.to(dev), w.to(dev), x, h, 1e-5)
    xr = _bf(eq[33].float().numpy() * np.float32(es[33].float()))
    np.testing.assert_array_equal(_np(x), xr)
    np.testing.assert_allclose(_np(h), _bf(OG.cohere_ln(xr, w.float().numpy())), rtol=8e-3, atol=8e-3)


@pytest.mark.parametrize("pos,rope", [(0, True), (1777, True), (300, False)])
def test_post_bf16(pos, rope, dev):
    NH, NKV, HD, inter, S = 16, 4, 128, 11008, 2048
    g = torch.Generator().manual_seed(12 + pos)
    y = torch.randn((NH + 2 * NKV) * HD + 2 * inter, generator=g).bfloat16()
    cos, sin = (torch.tensor(t).bfloat16() for t in OG.rope_tables(S, HD))
    kc = torch.zeros(NKV, S, HD, dtype=BF16, device=dev)
    vc = torch.zeros_like(kc)
    qo = torch.empty(NH * HD, dtype=BF16, device=dev)
    act = torch.empty(inter, dtype=BF16, device=dev)
    fused.post[(1,)](y.to(dev), torch.tensor([pos], device=dev), cos.to(dev), sin.to(dev), kc, vc, qo, act, S, inter,
                     NH=NH, NKV=NKV, HD=HD, ROPE=rope)
    torch.cuda.synchronize()
    yf = y.float().numpy()
    q = yf[:NH * HD].reshape(NH, HD)
    k = yf[NH * HD:(NH + NKV) * HD].reshape(NKV, HD)
    v = yf[(NH + NKV) * HD:(NH + 2 * NKV) * HD].reshape(NKV, HD)
    gt, up = yf[(NH + 2 * NKV) * HD:][:inter], yf[(NH + 2 * NKV) * HD:][inter:]
    if rope:
        c, s_ = cos[pos].float().numpy(), sin[pos].float().numpy()
        q, k = OG.rope(q, c, s_), OG.rope(k, c, s_)
    np.testing.assert_allclose(_np(qo).reshape(NH, HD), _bf(q), rtol=8e-3, atol=8e-3)
    np.testing.assert_allclose(_np(kc[:, pos]), _bf(k), rtol=8e-3, atol=8e-3)
    np.testing.assert_array_equal(_np(vc[:, pos]), v)
    np.testing.assert_allclose(_np(act), _bf(OG.silu(gt) * up), rtol=8e-3, atol=8e-3)


def _attn_dt(q, kc, vc, pos, dev, nsplit=64, NH=16, NKV=4, HD=128, dt=BF16):
    po = torch.empty(NH, nsplit, HD, device=dev)
    pm = torch.empty(NH, nsplit, device=dev)
    pl = torch.empty(NH, nsplit, device=dev)
    out = torch.empty(NH * HD, dtype=dt, device=dev)
    p = torch.tensor([pos], device=dev)
    fused.attn_split[(NKV, nsplit)](q, kc, vc, p, po, pm, pl, kc.shape[1], HD ** -0.5, REP=NH // NKV, HD=HD,
                                    NSPLIT=nsplit)
    fused.attn_combine[(NH,)](po, pm, pl, p, out, HD=HD, NSPLIT=nsplit)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("pos", [0, 300, 2047])
def test_attention_bf16(pos, dev):
    NH, NKV, HD, S = 16, 4, 128, 2048
    g = torch.Generator().manual_seed(100 + pos)
    kc = torch.randn(NKV, S, HD, generator=g).bfloat16()
    vc = torch.randn(NKV, S, HD, generator=g).bfloat16()
    q = torch.randn(NH * HD, generator=g).bfloat16()
    out = _attn_dt(q.to(dev), kc.to(dev), vc.to(dev), pos, dev)
    ref = OG.attend(q.float().numpy().reshape(NH, HD), kc[:, :pos + 1].float().numpy(), vc[:, :pos + 1].float().numpy())
    rep = O.parity_report(_np(out), _bf(ref).ravel())
    assert rep["norm_rel"] < 4e-3 and rep["cosine"] > 0.99999, rep


def test_attention_bf16_beyond_fp16_range(dev):
    """bf16 keys and queries far outside fp16's range (|k| up to 3e5, |q| down to 1e-6) keep their values: the
    q . k products are formed in fp32, so scores stay finite and the result matches the fp32 oracle."""
    NH, NKV, HD, S, pos = 16, 4, 128, 256, 99
    g = torch.Generator().manual_seed(7)
    kc = (torch.randn(NKV, S, HD, generator=g) * 1e5).bfloat16()       # |k| ~ 1e5 > 65504
    vc = torch.randn(NKV, S, HD, generator=g).bfloat16()
    q = (torch.randn(NH * HD, generator=g) * 3e-6).bfloat16()          # scores q.k / sqrt(128) = O(1)
    assert float(kc.float().abs().max()) > 65504 and float(q.float().abs().min()) < 6e-5
    out = _attn_dt(q.to(dev), kc.to(dev), vc.to(dev), pos, dev, nsplit=16)
    assert torch.isfinite(out.float()).all()
    ref = OG.attend(q.float().numpy().reshape(NH, HD), kc[:, :pos + 1].float().numpy(), vc[:, :pos + 1].float().numpy())
    rep = O.parity_report(_np(out), _bf(ref).ravel())
    assert rep["norm_rel"] < 1e-2 and rep["cosine"] > 0.9999, rep
