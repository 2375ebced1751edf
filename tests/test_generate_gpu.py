"""The generate loop (rumik-fast_amd/engine/generate.py, the reference's RumikInt4.generate, engine/rumik_int4.py:251-307)
on a full-width 2-layer synthetic model with the sampling tail in the captured step:
- the double-buffered frame loop returns exactly the token stream that stepping one replay at a time (reading every
  token back) gives for the same seed: queueing frames ahead changes nothing but the timing;
- every token is a head token id, generation ends at </audio> (not included) once the stop predictor fires after
  min_new tokens, and at max_new tokens otherwise;
- to_codes turns a round-robin stream into whole frames."""
import pytest
import torch

import decode
from generate import Generator, to_codes

pytestmark = pytest.mark.gpu

FIRST, Q = 100, 8


@pytest.fixture(params=["roles", "persistent"])
def kind(request):
    """the one-launch engine under the loop: the role-split step (the default) or the every-block-every-role one"""
    return request.param


def _engine(dev, b2, kind, seed=3):
    cfg = decode.Config(L=2, vocab=1024, n_audio=700, S=512)
    w = decode.random_weights(cfg, seed, device=dev)
    w["head"][0][-1].zero_()  # </audio>'s logit is 0: never among the top 30 of 700 (~N(0, 18)) logits by chance
    eng = (decode.RoleDecode if kind == "roles" else decode.PersistentDecode)(cfg, w, device=dev)
    g = torch.Generator().manual_seed(seed)
    stop = {"0.weight": torch.ones(cfg.H), "0.bias": torch.zeros(cfg.H),
            "1.weight": (torch.randn(512, cfg.H, generator=g) / cfg.H ** 0.5).bfloat16(),
            "1.bias": torch.zeros(512), "3.weight": torch.randn(1, 512, generator=g) / 512 ** 0.5 * 0.01,
            "3.bias": torch.tensor([float(b2)])}
    ids = FIRST + torch.arange(cfg.n_audio, dtype=torch.int64)  # audio token ids (the last one is </audio>)
    eng.attach_sampler(stop, ids, end_id=int(ids[-1]), max_new=96)
    return eng, ids


def _stepwise(eng, prompt, seed, n):
    """one replay at a time, every token read back (no queued frames)"""
    torch.manual_seed(seed)
    gen = Generator(eng, Q=Q)
    toks = [int(gen.prefill(prompt))]
    for _ in range(n - 1):
        eng.replay()
        torch.cuda.synchronize()
        toks.append(int(eng.tok.item()))
    return toks


def test_frames_match_stepwise_decoding(dev, kind):
    eng, ids = _engine(dev, b2=-50.0, kind=kind)
    gen = Generator(eng, Q=Q, first_unit_id=FIRST, last_unit_id=FIRST + 698, max_new=64)
    prompt = [5, 17, 300, 41]
    toks, stats = gen.generate(prompt, seed=11)
    print(stats)
    assert len(toks) == 65  # the first token, then frames of 8 while n < max_new
    ref = _stepwise(eng, prompt, 11, len(toks))
    assert toks == ref
    assert all(t in set(ids.tolist()) and t != eng.end_id for t in toks)
    codes = gen.to_codes(toks)
    assert codes.shape[0] == 1 and codes.shape[1] == Q
    assert torch.equal(codes, to_codes(toks, FIRST, FIRST + 698, Q))


def test_stop_after_min_new(dev, kind):
    eng, ids = _engine(dev, b2=50.0, kind=kind)  # the stop logit is far above zero: </audio> from step min_new on
    gen = Generator(eng, Q=Q, max_new=64)
    toks, stats = gen.generate([3, 9], seed=2)
    assert len(toks) == eng.min_new and eng.end_id not in toks
    assert int(eng.out[eng.min_new].item()) == eng.end_id


def test_nonzero_status_stops_generation(dev, kind):
    """A step whose status word is nonzero ends generation with DecodeError instead of emitting tokens sampled from
    invalid logits. The condition is forced from the host: after the first frame the device position is moved past
    the cache, so the next step's blocks all leave at entry (status bit 2); no wait times out."""
    from generate import DecodeError
    eng, ids = _engine(dev, b2=-50.0, kind=kind)
    gen = Generator(eng, Q=Q, max_new=64)
    seen = []

    def on_frame(toks):
        seen.append(len(toks))
        if len(seen) == 1:
            eng.pos.fill_(eng.cfg.S + 3)  # ordered after the frame already queued, before the next one
    with pytest.raises(DecodeError, match="status 4"):
        gen.generate([5, 17], seed=1, on_frame=on_frame)
    assert seen and eng.status_word() == 0  # the engine was reset before the error was raised
    toks, _ = gen.generate([5, 17], seed=1)  # and still generates afterwards
    assert len(toks) == 65
