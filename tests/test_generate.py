"""to_codes (rumik-fast_amd/engine/generate.py), the audio-token -> Mimi-code regrouping of the reference
(engine/rumik_int4.py:310-324), on hand-built token streams whose frames follow from the rule itself: token t in
[first, last] is code (t - first) // Q of codebook (t - first) % Q; frames are Q tokens in codebook order; an
out-of-order token restarts the frame at itself when it is codebook 0 and drops it otherwise; a non-audio token
drops the partial frame; a trailing partial frame is not returned."""
import torch

from generate import to_codes

FIRST, Q = 1000, 8


def tok(code, q):
    return FIRST + code * Q + q


def test_whole_frames_in_order():
    toks = [tok(c, q) for c, q in [(5, 0), (6, 1), (7, 2), (8, 3), (9, 4), (10, 5), (11, 6), (12, 7)]]
    toks += [tok(100 + q, q) for q in range(Q)]
    codes = to_codes(toks, FIRST, FIRST + 2048 * Q - 1, Q)
    assert codes.shape == (1, Q, 2)
    assert codes[0, :, 0].tolist() == [5, 6, 7, 8, 9, 10, 11, 12]
    assert codes[0, :, 1].tolist() == [100 + q for q in range(Q)]


def test_broken_round_robin_resyncs():
    last = FIRST + 2048 * Q - 1
    # codebooks 0,1,2 then a codebook-0 token: the frame restarts at it
    toks = [tok(1, 0), tok(2, 1), tok(3, 2), tok(4, 0)] + [tok(10 + q, q) for q in range(1, Q)]
    assert to_codes(toks, FIRST, last, Q)[0, :, 0].tolist() == [4] + [10 + q for q in range(1, Q)]
    # codebooks 0,1 then codebook 3: the partial frame is dropped, and so is everything until a codebook 0
    toks = [tok(1, 0), tok(2, 1), tok(3, 3), tok(4, 4)] + [tok(20 + q, q) for q in range(Q)]
    assert to_codes(toks, FIRST, last, Q)[0, :, 0].tolist() == [20 + q for q in range(Q)]


def test_non_audio_tokens_and_partial_tail():
    last = FIRST + 2048 * Q - 1
    toks = [tok(1, 0), tok(2, 1), 7, tok(3, 2)] + [tok(30 + q, q) for q in range(Q)] + [tok(40, 0), tok(41, 1)]
    codes = to_codes(toks, FIRST, last, Q)
    assert codes.shape == (1, Q, 1) and codes[0, :, 0].tolist() == [30 + q for q in range(Q)]
    assert to_codes([last + 1, FIRST - 1], FIRST, last, Q).shape == (1, Q, 0)
    assert to_codes([], FIRST, last, Q).dtype == torch.long
