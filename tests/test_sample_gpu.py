"""The sampling tail on the GPU (rumik-fast_amd/engine/sample.py -> rk_stop_hidden / rk_topk_partial / rk_pick and
the one-launch rk_sample_tail) vs the CPU oracle (oracle/sample.py) on identical seeded inputs: a 2048-wide bf16
hidden state, a 512 x 2048 bf16 stop-predictor W1, 16385 audio logits (the last chunk holds one logit) in fp32 or
bf16 (bf16 makes ties common), top-30, temperature 0.8, min_new 8, </audio> = the last head row.

What must match (the reference's own sampler check, engine/check_sample.py:19-58, made exact where it can be):
- keys: every 512-logit chunk's packed keys sorted descending, and scratch[:32]: the global top 32 in order, are
  bit-exact (integer work: the key order is total, ties go to the larger index; scratch[:32] is what the
  reference's pick and check read of the candidate list);
- the top-30 (scratch[:30]) is exactly the oracle's top-30 in key order;
- z1 (stop predictor hidden layer, fp32 vs the oracle's float64): |diff| <= 1e-4 * (1 + |z1|);
- the stop decision, whenever the oracle's stop logit is not within 1e-3 of zero;
- the token, whenever the oracle's best Gumbel score beats the runner-up by more than 1e-4 (otherwise it must be
  one of the near-tied candidates); then out[step] = token, tok = token, step += 1.
"""
import types

import numpy as np
import pytest
import torch

import sample
from oracle import sample as OS

pytestmark = pytest.mark.gpu

H, NZ, NV = 2048, 512, 16385


def _engine(dev, seed, b2=0.0):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g)  # noqa: E731
    stop = {"0.weight": 1 + 0.1 * r(H), "0.bias": 0.1 * r(H), "1.weight": (r(NZ, H) / H ** 0.5).bfloat16(),
            "1.bias": 0.1 * r(NZ), "3.weight": r(1, NZ) / NZ ** 0.5, "3.bias": torch.tensor([float(b2)])}
    ids = torch.arange(NV, dtype=torch.int64) + 1000
    return types.SimpleNamespace(
        dev=dev, H=H, hn=r(H).bfloat16().to(dev), stop={k: v.to(dev) for k, v in stop.items()},
        audio_ids=ids.to(dev), end_id=int(ids[-1]), top_k=30, min_new=8, temperature=0.8,
        step_i=torch.zeros(1, dtype=torch.int64, device=dev), pos=torch.zeros(1, dtype=torch.int64, device=dev),
        tok=torch.zeros(1, dtype=torch.int64, device=dev), out=torch.zeros(64, dtype=torch.int64, device=dev))


def _logits(dev, seed, dtype):
    g = torch.Generator().manual_seed(seed + 100)
    return (3 * torch.randn(NV, generator=g)).to(dtype).to(dev)


def _np(t):
    return t.detach().cpu().numpy()


def _oracle(eng, logits, u, step):
    st = {k: _np(v.float()) for k, v in eng.stop.items()}
    z1 = OS.stop_hidden(_np(eng.hn.float()), st["0.weight"], st["0.bias"], st["1.weight"], st["1.bias"])
    s = OS.stop_logit(z1, st["3.weight"].reshape(-1), st["3.bias"])
    lg = _np(logits.float())
    sc, idx = OS.scores(lg, u, step, NV - 1, eng.min_new, eng.top_k, eng.temperature)
    return z1, s, lg, sc, idx


def _check_token(eng, tok, lg, sc, idx, s, step, u):
    ids = _np(eng.audio_ids)
    if s > 1e-3 and step >= eng.min_new:
        assert tok == eng.end_id, (tok, s)
        return
    order = np.argsort(-sc, kind="stable")
    near = [int(ids[idx[j]]) for j in order if sc[order[0]] - sc[j] <= 1e-4]
    if abs(s) <= 1e-3 and step >= eng.min_new:
        near.append(eng.end_id)
    if len(near) == 1:
        assert tok == near[0], (tok, near)
    else:
        assert tok in near, (tok, near)


def _check_buffers(eng, smp, lg, step, z1_ref):
    # keys: chunk c sorted descending (the oracle's keys, chunk by chunk; padding = -inf at indices >= NV)
    masked = OS.masked_logits(lg, step, NV - 1, eng.min_new)
    nch = smp.nch
    pad = np.full(nch * sample.CH, -np.inf, np.float32)
    pad[:NV] = masked
    keys = OS.make_keys(pad, np.arange(pad.size)).reshape(nch, sample.CH)
    ref_keys = np.sort(keys, axis=1)[:, ::-1]
    assert np.array_equal(_np(smp.keys).reshape(nch, sample.CH), ref_keys)
    cand = np.sort(ref_keys[:, :sample.KEEP].reshape(-1))[::-1]
    assert np.array_equal(_np(smp.scratch)[:sample.KEEP], cand[:sample.KEEP])
    assert np.array_equal(_np(smp.scratch)[:eng.top_k], OS.sorted_keys(lg, step, NV - 1, eng.min_new)[:eng.top_k])
    z1 = _np(smp.z1)
    assert np.all(np.abs(z1 - z1_ref) <= 1e-4 * (1 + np.abs(z1_ref))), np.abs(z1 - z1_ref).max()


@pytest.mark.parametrize("ldt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("step", [3, 20])
def test_three_kernels_match_oracle(dev, ldt, step):
    eng = _engine(dev, 1)
    smp = sample.FusedSampler(eng, None)
    logits = _logits(dev, 1, ldt)
    u = torch.rand(32, generator=torch.Generator().manual_seed(7)).to(dev)
    eng.step_i.fill_(step)
    sample.stop_hidden[(smp.nz // 16,)](eng.hn, smp.lnw, smp.lnb, smp.w1, smp.b1, smp.z1, 1e-5, H=H, ROWS=16)
    sample.topk_partial[(smp.nch,)](logits, eng.step_i, smp.keys, smp.nv, smp.end_idx, eng.min_new, CH=sample.CH)
    sample.pick[(1,)](smp.keys, smp.scratch, u, smp.z1, smp.w2, smp.b2, eng.audio_ids, eng.step_i, eng.pos, eng.tok,
                      eng.out, 1.0 / eng.temperature, eng.end_id, eng.min_new, smp.nch, CH=sample.CH,
                      KEEP=sample.KEEP, NC=smp.nc, TOPK=eng.top_k, NZ=smp.nz)
    torch.cuda.synchronize()
    z1_ref, s, lg, sc, idx = _oracle(eng, logits, _np(u), step)
    _check_buffers(eng, smp, lg, step, z1_ref)
    tok = int(eng.tok.item())
    _check_token(eng, tok, lg, sc, idx, s, step, _np(u))
    assert int(eng.step_i.item()) == step + 1 and int(eng.out[step].item()) == tok
    zl = float((smp.z1 * smp.w2).sum() + smp.b2)
    if abs(s) > 1e-3:
        assert (zl > 0) == (s > 0)


@pytest.mark.parametrize("ldt", [torch.float32, torch.bfloat16])
def test_fused_tail_matches_three_kernels(dev, ldt):
    eng = _engine(dev, 2)
    logits = _logits(dev, 2, ldt)
    smp = sample.FusedSampler(eng, lambda: logits)
    for step in (5, 9, 31):
        eng.step_i.fill_(step)
        smp()
        torch.cuda.synchronize()
        u = _np(smp.u)
        z1_ref, s, lg, sc, idx = _oracle(eng, logits, u, step)
        _check_buffers(eng, smp, lg, step, z1_ref)
        tok = int(eng.tok.item())
        _check_token(eng, tok, lg, sc, idx, s, step, u)
        assert int(eng.step_i.item()) == step + 1 and int(eng.out[step].item()) == tok
        assert int(smp.counter.item()) == 0
        # the three kernels on the same uniforms give the same buffers and token
        keys, scratch, z1 = smp.keys.clone(), smp.scratch.clone(), smp.z1.clone()
        eng.step_i.fill_(step)
        sample.stop_hidden(eng.hn, smp.lnw, smp.lnb, smp.w1, smp.b1, smp.z1, 1e-5)
        sample.topk_partial(logits, eng.step_i, smp.keys, smp.nv, smp.end_idx, eng.min_new)
        sample.pick(smp.keys, smp.scratch, smp.u, smp.z1, smp.w2, smp.b2, eng.audio_ids, eng.step_i, eng.pos,
                    eng.tok, eng.out, 1.0 / eng.temperature, eng.end_id, eng.min_new, smp.nch, NC=smp.nc,
                    TOPK=eng.top_k)
        torch.cuda.synchronize()
        assert torch.equal(keys, smp.keys) and torch.equal(scratch[:32], smp.scratch[:32]) and torch.equal(z1, smp.z1)
        assert int(eng.tok.item()) == tok


def test_graph_replays_follow_the_oracle(dev):
    eng = _engine(dev, 3)
    logits = _logits(dev, 3, torch.bfloat16)
    smp = sample.FusedSampler(eng, lambda: logits)
    smp()  # warm up outside the graph
    torch.cuda.synchronize()
    eng.step_i.fill_(0)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        smp()
    torch.cuda.synchronize()
    eng.step_i.fill_(0)
    toks = []
    for r in range(12):
        logits.copy_(_logits(dev, 10 + r, torch.bfloat16))  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        u = _np(smp.u)
        z1_ref, s, lg, sc, idx = _oracle(eng, logits, u, r)
        _check_buffers(eng, smp, lg, r, z1_ref)
        tok = int(eng.tok.item())
        _check_token(eng, tok, lg, sc, idx, s, r, u)
        assert int(eng.step_i.item()) == r + 1 and int(eng.out[r].item()) == tok
        assert int(smp.counter.item()) == 0
        toks.append(tok)
    assert _np(eng.out)[:12].tolist() == toks


def test_end_masking_and_stop_rule(dev):
    eng = _engine(dev, 4, b2=-50.0)  # stop logit far below zero
    logits = _logits(dev, 4, torch.float32)
    logits[NV - 1] = 100.0  # </audio> is the largest logit by far
    smp = sample.FusedSampler(eng, lambda: logits)
    eng.step_i.fill_(3)
    smp()
    torch.cuda.synchronize()
    top = (_np(smp.scratch)[:eng.top_k] & 0xFFFFFFFF).tolist()
    assert NV - 1 not in top and int(eng.tok.item()) != eng.end_id  # masked before min_new
    eng.step_i.fill_(8)
    smp()
    torch.cuda.synchronize()
    assert (_np(smp.scratch)[0] & 0xFFFFFFFF) == NV - 1 and int(eng.tok.item()) == eng.end_id  # sampled, not stopped
    eng2 = _engine(dev, 4, b2=50.0)  # stop logit far above zero
    logits2 = _logits(dev, 5, torch.float32)
    smp2 = sample.FusedSampler(eng2, lambda: logits2)
    eng2.step_i.fill_(7)
    smp2()
    torch.cuda.synchronize()
    assert int(eng2.tok.item()) != eng2.end_id  # the stop rule waits for min_new
    smp2()
    torch.cuda.synchronize()
    assert int(eng2.tok.item()) == eng2.end_id and int(eng2.out[8].item()) == eng2.end_id


def test_small_vocab_and_top_k(dev):
    # 700 logits (two chunks, the second partial), top-5, fp16 logits and fp16 hidden state / W1
    eng = _engine(dev, 6)
    eng.hn = eng.hn.half()
    eng.stop["1.weight"] = eng.stop["1.weight"].half()
    eng.audio_ids = eng.audio_ids[:700].clone()
    eng.end_id = int(eng.audio_ids[-1])
    eng.top_k = 5
    logits = _logits(dev, 6, torch.float16)[:700].clone()
    smp = sample.FusedSampler(eng, lambda: logits)
    assert smp.nch == 2 and smp.nc == 64
    eng.step_i.fill_(12)
    smp()
    torch.cuda.synchronize()
    u = _np(smp.u)
    st = {k: _np(v.float()) for k, v in eng.stop.items()}
    z1 = OS.stop_hidden(_np(eng.hn.float()), st["0.weight"], st["0.bias"], st["1.weight"], st["1.bias"])
    s = OS.stop_logit(z1, st["3.weight"].reshape(-1), st["3.bias"])
    lg = _np(logits.float())
    assert np.array_equal(_np(smp.scratch)[:5], OS.sorted_keys(lg, 12, 699, eng.min_new)[:5])
    sc, idx = OS.scores(lg, u, 12, 699, eng.min_new, 5, eng.temperature)
    _check_token(eng, int(eng.tok.item()), lg, sc, idx, s, 12, u)
