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


def test_round_bf16_matches_torch():
    """The oracle's bf16 rounding is torch's float32 -> bfloat16 conversion (round to nearest, ties to even)."""
    import torch
    rng = np.random.default_rng(5)
    a = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 20000),
                        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 3.3895314e38, 3.40e38, -3.40e38, np.inf,
                                  -np.inf, 1e-40, -1e-40, 9.1835e-41], np.float32)]).astype(np.float32)
    # exact ties: the low 16 bits are 0x8000, odd and even upper halves
    ties = (np.arange(1000, dtype=np.uint32) * 0x00010000 + 0x3F808000).view(np.float32)
    a = np.concatenate([a, ties])
    got = OG.round_bf16(a)
    ref = torch.from_numpy(a).bfloat16().float().numpy()
    np.testing.assert_array_equal(got, ref)


def _one_hot_rows(n_rows, K, cols, scale=1.0):
    """int4 rows w[r] = e_{cols[r]} * scale (cols[r] < 0: an all-zero row), exact in the g128 format:
    code 1 at the column, 0 elsewhere, group scale `scale`, min 0."""
    codes = np.zeros((n_rows, K), np.uint8)
    for r, c in enumerate(cols):
        if c >= 0:
            codes[r, c] = 1
    s = np.full((n_rows, K // 128), scale, np.float16)
    m = np.zeros((n_rows, K // 128), np.float16)
    return O.pack_int4(codes), s, m


def test_decode_step_closed_form():
    """The wiring of the whole step (reference engine/rumik_fused.py:97-121) on a 2-layer model whose projections
    are one-hot rows, so every intermediate follows by hand:
      - q rows zero: all scores 0, so attention = the mean of V over slots 0..pos (both query heads, GQA);
      - k / v rows pick channels of h: k at pos = rope(h[ck]) on layer 0 (RoPE) and h[ck] on layer 1 (NoPE),
        v at pos = h[cv];
      - gate / up rows pick channels cg / cu: act = silu(h[cg]) * h[cu];
      - w_o row r picks attention channel co[r], w_down row r picks act channel cd[r] (other rows zero);
      - x += o + d; every layer has its own LayerNorm weights, the final norm differs from both;
      - head row j picks channel ch[j] of the final-norm output, times its scale.
    A slice swap (q | k | v | gate | up), a LayerNorm index error, RoPE on the wrong layer or the head read before
    the final norm each changes a checked value by O(1)."""
    rng = np.random.default_rng(17)
    H, NH, NKV, HD, inter, S, L, pos = 256, 2, 1, 128, 128, 8, 2, 5
    f16 = lambda v: np.asarray(v, np.float32).astype(np.float16).astype(np.float32)  # noqa: E731
    ck = rng.permutation(H)[:HD]
    cv = rng.permutation(H)[:HD]
    cg = rng.permutation(H)[:inter]
    cu = rng.permutation(H)[:inter]
    co = [int(c) if r % 3 else -1 for r, c in enumerate(rng.integers(0, NH * HD, H))]
    cd = [int(c) if r % 4 else -1 for r, c in enumerate(rng.integers(0, inter, H))]
    w_in = _one_hot_rows(NH * HD + 2 * NKV * HD + 2 * inter, H,
                         [-1] * (NH * HD) + list(ck) + list(cv) + list(cg) + list(cu))
    ln = [(rng.random(H) + 0.5).astype(np.float16) for _ in range(L)]
    norm = (rng.random(H) + 0.5).astype(np.float16)
    ch = rng.integers(0, H, 6)
    head_q = np.zeros((6, H), np.int8)
    head_q[np.arange(6), ch] = 1
    head_s = np.array([1.0, 0.5, 2.0, 0.25, 1.5, 3.0], np.float16)
    emb_q = rng.integers(-127, 128, (4, H)).astype(np.int8)
    emb_s = np.full(4, 0.02, np.float16)
    cos, sin = OG.rope_tables(S, HD)
    md = OG.DecodeModel(L=L, H=H, NH=NH, NKV=NKV, HD=HD, inter=inter, eps=1e-5,
                        w_in=[w_in, w_in], w_o=[_one_hot_rows(H, NH * HD, co)] * L,
                        w_down=[_one_hot_rows(H, inter, cd)] * L, ln=ln, norm=norm, emb=(emb_q, emb_s),
                        head=(head_q, head_s), rope=(cos, sin), sliding=[True, False])
    kc = np.zeros((L, NKV, S, HD), np.float16)
    vc = np.zeros_like(kc)
    kc[:, :, :pos] = rng.standard_normal((L, NKV, pos, HD)).astype(np.float16)
    vc[:, :, :pos] = rng.standard_normal((L, NKV, pos, HD)).astype(np.float16)
    v_prefix = vc[:, 0, :pos].astype(np.float32).copy()
    logits, hn, x_out = OG.decode_step(md, 3, pos, kc, vc)

    # by hand
    x = f16(emb_q[3].astype(np.float32) * np.float32(emb_s[3]))
    for i in range(L):
        h = f16(OG.cohere_ln(x, ln[i]))
        k = h[ck].reshape(1, HD)
        if i == 0:  # RoPE on layer 0 only: pair (2j, 2j+1) rotated by pos * theta_j
            ang = pos * 10000.0 ** (-np.arange(0, HD, 2) / HD)
            ke, ko = k[0, 0::2].astype(np.float64), k[0, 1::2].astype(np.float64)
            k = np.empty((1, HD))
            k[0, 0::2], k[0, 1::2] = ke * np.cos(ang) - ko * np.sin(ang), ko * np.cos(ang) + ke * np.sin(ang)
        np.testing.assert_allclose(kc[i, 0, pos].astype(np.float32), f16(k[0]), rtol=2e-3, atol=2e-3)
        np.testing.assert_array_equal(vc[i, 0, pos].astype(np.float32), h[cv])
        v_mean = (v_prefix[i].sum(0) + h[cv]) / (pos + 1)
        o = f16(np.tile(v_mean, NH))  # q = 0: uniform weights; both query heads read KV head 0
        act = f16(h[cg] / (1 + np.exp(-h[cg].astype(np.float64))) * h[cu])
        a = np.array([o[c] if c >= 0 else 0.0 for c in co], np.float32)
        d = np.array([act[c] if c >= 0 else 0.0 for c in cd], np.float32)
        x = f16(x + a + d)
    hf = f16(OG.cohere_ln(x, norm))
    np.testing.assert_allclose(x_out, x, rtol=2e-3, atol=2e-3)
    np.testing.assert_allclose(hn, hf, rtol=2e-3, atol=2e-3)
    np.testing.assert_allclose(logits, hf[ch] * head_s.astype(np.float32), rtol=2e-3, atol=2e-3)
    # the checked values are far from what the plausible wiring errors give
    assert np.abs(hf - f16(OG.cohere_ln(x, ln[1]))).max() > 0.05       # final norm vs the last layer's LN weights
    assert np.abs(x - f16(emb_q[3] * np.float32(emb_s[3]))).max() > 0.05  # the layers change x


def test_decode_step_weight_cache_is_transparent():
    """cache_weights=True (dequantize once) gives the same step as dequantizing at every call."""
    rng = np.random.default_rng(2)
    H, NH, NKV, HD, inter, S, L = 256, 2, 1, 128, 128, 8, 2

    def mat(N, K):
        s = (rng.random((N, K // 128)) * 0.02 + 0.001).astype(np.float16)
        return O.pack_int4(rng.integers(0, 16, (N, K)).astype(np.uint8)), s, (-7.5 * s).astype(np.float16)

    kw = dict(L=L, H=H, NH=NH, NKV=NKV, HD=HD, inter=inter, eps=1e-5,
              w_in=[mat((NH + 2 * NKV) * HD + 2 * inter, H) for _ in range(L)], w_o=[mat(H, H) for _ in range(L)],
              w_down=[mat(H, inter) for _ in range(L)], ln=[np.ones(H, np.float16)] * L, norm=np.ones(H, np.float16),
              emb=(rng.integers(-127, 128, (4, H)).astype(np.int8), np.full(4, 0.02, np.float16)),
              head=(rng.integers(-127, 128, (5, H)).astype(np.int8), np.full(5, 0.01, np.float16)),
              rope=OG.rope_tables(S, HD), sliding=[True, False])
    outs = []
    for cache in (False, True):
        md = OG.DecodeModel(cache_weights=cache, **kw)
        kc = np.zeros((L, NKV, S, HD), np.float16)
        vc = np.zeros_like(kc)
        for p in range(3):
            res = OG.decode_step(md, p + 1, p, kc, vc)
        outs.append((res, kc.copy()))
    for a, b in zip(outs[0][0], outs[1][0]):
        np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(outs[0][1], outs[1][1])
