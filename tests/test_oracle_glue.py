"""Pins of the glue oracle (oracle/glue.py) by what the mathematics fixes, so that a dropped term, a wrong sign or
index, or a transposed operand fails one of them:
  LayerNorm  constant input -> 0; output has zero mean and unit mean square (w = 1, eps = 0); invariant to
             x -> a x + b (a > 0); w scales elementwise                      (engine/rumik_int4.py:38-43)
  RoPE       pos 0 -> identity; pair norms kept; angle of pair j at pos p is p * theta^(-2j/HD); rotating by p then
             q equals rotating by p + q; only the pair partner mixes in       (engine/rumik_int4.py:46-52,110-112)
  attention  one slot -> v[0]; q = 0 -> mean of V; a dominant score selects its row; GQA head h reads KV head
             h // REP; the split combine equals the unsplit softmax, with empty splits  (engine/fused.py:120-187)
  SiLU       g * sigmoid(g) against scipy's logistic                           (engine/fused.py:84)
  step       zero O / down weights leave x unchanged (the residual of the parallel block, rumik_int4.py:9-10)
"""
import numpy as np
import pytest
from scipy.special import expit

from oracle import glue as OG
from oracle import int4 as O


def test_layernorm_invariants():
    r = np.random.default_rng(0)
    x = r.standard_normal(2048).astype(np.float32) * 3 + 1
    one = np.ones(2048, np.float32)
    h = OG.cohere_ln(x, one, eps=0.0)
    assert abs(h.mean()) < 1e-5 and abs((h * h).mean() - 1) < 1e-5
    np.testing.assert_allclose(OG.cohere_ln(2.5 * x - 7, one, eps=0.0), h, atol=1e-4)
    w = r.uniform(0.5, 2, 2048).astype(np.float32)
    np.testing.assert_allclose(OG.cohere_ln(x, w, eps=0.0), h * w, rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(OG.cohere_ln(np.full(2048, 3.0, np.float32), one), np.zeros(2048, np.float32))


def test_rope_tables_angles():
    cos, sin = OG.rope_tables(16, 128, 10000.0)
    for p, j in ((1, 0), (5, 3), (15, 63), (7, 31)):
        ang = p * 10000.0 ** (-2 * j / 128)
        for col in (2 * j, 2 * j + 1):  # both elements of pair j share its angle
            assert abs(cos[p, col] - np.cos(ang)) < 1e-5 and abs(sin[p, col] - np.sin(ang)) < 1e-5
    np.testing.assert_array_equal(cos[0], np.ones(128, np.float32))
    np.testing.assert_array_equal(sin[0], np.zeros(128, np.float32))


def test_rope_rotation_properties():
    r = np.random.default_rng(1)
    cos, sin = OG.rope_tables(64, 128, 10000.0)
    v = r.standard_normal(128).astype(np.float32)
    np.testing.assert_array_equal(OG.rope(v, cos[0], sin[0]), v)
    for p in (1, 9, 63):
        w = OG.rope(v, cos[p], sin[p])
        np.testing.assert_allclose(w[0::2] ** 2 + w[1::2] ** 2, v[0::2] ** 2 + v[1::2] ** 2, rtol=1e-5)
    np.testing.assert_allclose(OG.rope(OG.rope(v, cos[20], sin[20]), cos[13], sin[13]),
                               OG.rope(v, cos[33], sin[33]), atol=1e-5)
    # interleaved pairs: a one-hot at element 2j only reaches elements 2j, 2j+1, with (cos, +sin)
    e = np.zeros(128, np.float32)
    e[10] = 1
    w = OG.rope(e, cos[3], sin[3])
    assert np.count_nonzero(w) == 2 and w[10] == cos[3, 10] and w[11] == sin[3, 10]


def test_attention_closed_forms():
    r = np.random.default_rng(2)
    NH, NKV, HD = 8, 2, 128
    q = r.standard_normal((NH, HD)).astype(np.float32)
    K = r.standard_normal((NKV, 9, HD)).astype(np.float32)
    V = r.standard_normal((NKV, 9, HD)).astype(np.float32)
    one = OG.attend(q, K[:, :1], V[:, :1])
    for h in range(NH):
        np.testing.assert_allclose(one[h], V[h // 4, 0], rtol=1e-6)
    zero = OG.attend(np.zeros_like(q), K, V)
    for h in range(NH):
        np.testing.assert_allclose(zero[h], V[h // 4].mean(0), rtol=1e-5, atol=1e-6)
    # a dominant score picks its slot, and the query head reads KV head h // REP (not h % NKV)
    K2 = np.zeros((NKV, 9, HD), np.float32)
    K2[0, 3, 0] = 100.0
    K2[1, 6, 0] = 100.0
    q2 = np.zeros((NH, HD), np.float32)
    q2[:, 0] = 1.0
    out = OG.attend(q2, K2, V, scale=1.0)
    for h in range(NH):
        np.testing.assert_allclose(out[h], V[h // 4, 3 if h < 4 else 6], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("n,nsplit,chunk", [(37, 5, 8), (37, 8, 8), (5, 16, 8), (64, 4, 16), (1, 4, 8)])
def test_split_combine_equals_softmax(n, nsplit, chunk):
    r = np.random.default_rng(n + nsplit)
    q = r.standard_normal((8, 128)).astype(np.float32)
    K = r.standard_normal((2, n, 128)).astype(np.float32)
    V = r.standard_normal((2, n, 128)).astype(np.float32)
    out, m, l = OG.attend_split(q, K, V, nsplit, chunk)
    np.testing.assert_allclose(out, OG.attend(q, K, V), rtol=1e-5, atol=1e-6)
    empty = [sp for sp in range(nsplit) if sp * chunk >= n]
    assert np.all(np.isneginf(m[:, empty])) and np.all(l[:, empty] == 0)


def test_silu_closed_form():
    g = np.linspace(-20, 20, 401).astype(np.float32)
    np.testing.assert_allclose(OG.silu(g), g * expit(g), rtol=1e-6, atol=1e-7)
    assert OG.silu(np.float32(0.0)) == 0


def test_decode_step_residual_identity():
    """With zero O and down projections the layer adds nothing: x after the layer equals the embedding."""
    r = np.random.default_rng(3)
    H, NH, NKV, HD, inter, S, L = 256, 2, 1, 128, 128, 8, 1

    def mat(N, K, zero=False):
        codes = np.zeros((N, K), np.uint8) if zero else r.integers(0, 16, (N, K)).astype(np.uint8)
        s = np.full((N, K // 128), 0.01, np.float16)
        m = np.zeros((N, K // 128), np.float16) if zero else (-7.5 * s).astype(np.float16)
        return O.pack_int4(codes), s, m

    emb = (r.integers(-127, 128, (4, H)).astype(np.int8), np.full(4, 0.02, np.float16))
    md = OG.DecodeModel(L=L, H=H, NH=NH, NKV=NKV, HD=HD, inter=inter, eps=1e-5,
                        w_in=[mat((NH + 2 * NKV) * HD + 2 * inter, H)], w_o=[mat(H, NH * HD, zero=True)],
                        w_down=[mat(H, inter, zero=True)], ln=[np.ones(H, np.float16)], norm=np.ones(H, np.float16),
                        emb=emb, head=(r.integers(-127, 128, (5, H)).astype(np.int8), np.full(5, 0.01, np.float16)),
                        rope=OG.rope_tables(S, HD), sliding=[True])
    kc = np.zeros((L, NKV, S, HD), np.float16)
    vc = np.zeros_like(kc)
    _, _, x = OG.decode_step(md, 2, 3, kc, vc)
    x0 = (emb[0][2].astype(np.float32) * np.float32(emb[1][2])).astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(x, x0)
    assert np.any(kc[0, :, 3] != 0) and np.all(kc[0, :, :3] == 0)  # K written at pos only


def test_causal_attend_rows_are_decode_attention():
    """row t of the prefill attention is the decode attention of query t over slots 0..p0+t (the pinned `attend`),
    and the first row of a fresh prompt is v[0] exactly (one slot)"""
    rng = np.random.default_rng(12)
    T, NH, NKV, HD, p0 = 9, 4, 2, 16, 3
    q = rng.standard_normal((T, NH, HD)).astype(np.float32)
    K = rng.standard_normal((NKV, p0 + T, HD)).astype(np.float32)
    V = rng.standard_normal((NKV, p0 + T, HD)).astype(np.float32)
    out = OG.causal_attend(q, K, V, p0)
    for t in range(T):
        np.testing.assert_allclose(out[t], OG.attend(q[t], K[:, :p0 + t + 1], V[:, :p0 + t + 1]), rtol=1e-5, atol=1e-6)
    first = OG.causal_attend(q[:1], K, V, 0)
    np.testing.assert_array_equal(first[0], V[np.arange(NH) // 2, 0])
