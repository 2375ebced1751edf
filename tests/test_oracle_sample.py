"""Pins of the sampling-tail oracle (oracle/sample.py) on the CPU, against what the mathematics fixes rather than a
retyped copy of the oracle:

- sortable keys: integer order == float order over special values and 100k random bit patterns; exact inverse;
  ties broken by the larger index (reference engine/sample.py:7-11);
- top-k: brute force (argsort); </audio> masked only while step < min_new (engine/rumik_int4.py:183-184);
- Gumbel-max: the empirical distribution of the sampled candidate over 40k uniforms equals softmax(top_v / T)
  (chi-square), i.e. the sign and nesting of -log(-log(u)) are right (engine/rumik_int4.py:186-189);
- GELU: closed forms (gelu(0) = 0, gelu(1) = Phi(1), tails) and scipy's erf;
- stop predictor: an input whose LayerNorm is itself (mean 0, variance 1) with W1 = unit rows gives gelu(+-1);
- stop rule: the stop logit's sign decides only from min_new on (engine/rumik_int4.py:191).
"""
import math

import numpy as np
import pytest
from scipy import special, stats

from oracle import sample as OS


def test_sortable_key_order_special_values():
    f = np.float32
    vals = np.array([-np.inf, -np.finfo(f).max, -1.5, -np.finfo(f).tiny, -np.finfo(f).smallest_subnormal, -0.0, 0.0,
                     np.finfo(f).smallest_subnormal, np.finfo(f).tiny, 1.0, 1.5, np.finfo(f).max, np.inf], dtype=f)
    k = OS.sortable(vals)
    assert np.all(np.diff(k.astype(np.int64)) > 0)


def test_sortable_key_order_random_bits():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 32, size=100_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    k = OS.sortable(x).astype(np.int64)
    # brute-force pairwise check on neighbours of the value order (+0 / -0 aside, equal values have equal keys)
    o = np.argsort(x, kind="stable")
    xs, ks = x[o], k[o]
    same = xs[1:] == xs[:-1]
    assert np.all(ks[1:][~same] > ks[:-1][~same])
    assert np.array_equal(OS.unsortable(OS.sortable(x)).view(np.uint32), x.view(np.uint32))


def test_keys_break_ties_by_larger_index():
    keys = OS.sorted_keys(np.array([1.0, 3.0, 1.0, 3.0, 1.0], np.float32), step=100, end_idx=0, min_new=8)
    idx = (keys & 0xFFFFFFFF).tolist()
    assert idx == [3, 1, 4, 2, 0]


def test_topk_matches_argsort_and_masks_end_early():
    rng = np.random.default_rng(1)
    lg = rng.standard_normal(16385).astype(np.float32)
    end = 16384
    lg[end] = 50.0  # the largest logit is </audio>
    v, i = OS.topk(lg, step=3, end_idx=end, min_new=8, k=30)
    assert end not in i.tolist()
    ref = np.argsort(-np.where(np.arange(lg.size) == end, -np.inf, lg), kind="stable")[:30]
    assert i.tolist() == ref.tolist() and np.array_equal(v, lg[ref])
    v2, i2 = OS.topk(lg, step=8, end_idx=end, min_new=8, k=30)
    assert i2[0] == end and v2[0] == 50.0


def test_gumbel_max_samples_softmax_of_topk():
    rng = np.random.default_rng(2)
    lg = np.array([2.0, 1.5, 1.0, 0.2, -0.5, -3.0], dtype=np.float32)
    T, k, n = 0.8, 5, 40_000
    ids = np.arange(lg.size) + 100
    counts = np.zeros(lg.size)
    for _ in range(n):
        t = OS.pick(lg, rng.random(32, dtype=np.float32), ids, step=20, end_idx=5, min_new=8, end_id=-1, top_k=k,
                    temperature=T, stop_s=-1.0)
        counts[t - 100] += 1
    assert counts[5] == 0  # outside the top-k
    p = np.exp(lg[:k] / T) / np.exp(lg[:k] / T).sum()
    chi2 = ((counts[:k] - n * p) ** 2 / (n * p)).sum()
    assert chi2 < stats.chi2.ppf(0.999, k - 1), (counts, n * p)


def test_gelu_closed_forms():
    assert OS.gelu(np.array([0.0]))[0] == 0.0
    assert OS.gelu(np.array([1.0]))[0] == pytest.approx(0.5 * (1 + math.erf(1 / math.sqrt(2))), rel=1e-15)
    assert OS.gelu(np.array([1.0]))[0] == pytest.approx(stats.norm.cdf(1.0), rel=1e-12)
    assert OS.gelu(np.array([10.0]))[0] == pytest.approx(10.0, rel=1e-12)
    assert abs(OS.gelu(np.array([-10.0]))[0]) < 1e-20
    y = np.linspace(-6, 6, 101)
    np.testing.assert_allclose(OS.gelu(y), 0.5 * y * (1 + special.erf(y / np.sqrt(2))), rtol=1e-13, atol=1e-300)


def test_stop_hidden_on_a_self_normalized_input():
    H, nz = 256, 8
    h = np.where(np.arange(H) % 2 == 0, 1.0, -1.0)  # mean 0, variance 1: LayerNorm(h) = h (eps aside)
    w1 = np.zeros((nz, H))
    w1[np.arange(nz), np.arange(nz)] = 1.0          # row r picks h[r]
    z1 = OS.stop_hidden(h, np.ones(H), np.zeros(H), w1, np.zeros(nz), eps=0.0)
    expect = [stats.norm.cdf(1.0) if r % 2 == 0 else -stats.norm.cdf(-1.0) for r in range(nz)]
    np.testing.assert_allclose(z1, expect, rtol=1e-12)
    # LayerNorm bias and weight enter as affine terms: lnb = 2 on every column adds 2 before the GELU
    z2 = OS.stop_hidden(h, np.ones(H), 2 * np.ones(H), w1, np.zeros(nz), eps=0.0)
    np.testing.assert_allclose(z2[0], 3 * stats.norm.cdf(3.0), rtol=1e-12)


def test_stop_rule_applies_from_min_new():
    lg = np.array([1.0, 0.0, -1.0], np.float32)
    u = np.full(32, 0.5, np.float32)
    ids = np.array([10, 11, 12])
    kw = dict(end_idx=2, min_new=8, end_id=99, top_k=2, temperature=1.0)
    assert OS.pick(lg, u, ids, step=7, stop_s=5.0, **kw) == 10
    assert OS.pick(lg, u, ids, step=8, stop_s=5.0, **kw) == 99
    assert OS.pick(lg, u, ids, step=8, stop_s=-5.0, **kw) == 10
