"""Pins the CPU oracle (oracle/int4.py) with closed forms, brute force and invariants — never with a retyped copy
of the oracle's own formula. Each check is chosen so a plausible mistake fails it:

  nibble order        one-hot codes at even and odd columns -> packed byte value from the format spec
                      (low nibble = even column); pack/unpack bijection over all 256 byte values
  affine / min term   codes 0, min 1, x = 1 -> y = K exactly (the reference's historical 4x-min bug,
                      engine/README.md:102); codes 15, min 0 -> 15 * 128 * sum_g scale_g
  GEMV                one-hot x picks one dequantized column; factored identity (scale * sum(code*x) +
                      min * sum(x), kernels/int4_gemv.py:3) computed with Python loops on a tiny case equals
                      dequantize-then-matmul; fp32 vs an independent float64 product
  quantize            grid-exact weights give back their codes; round-trip error <= scale/2 (+ fp16 rounding);
                      constant group -> clamped scale, code 0; ties round half to even
  int8                all-+127 / all--127 rows -> +-127*K*scale; the two code layouts agree; quantize round trip
  prefill             row m of the product = the GEMV of X[m]
"""

import numpy as np
import pytest

from oracle import int4 as O


def rng(seed=0):
    return np.random.default_rng(seed)


# ------------------------------------------------------------------ nibble order / packing
def test_onehot_code_position_matches_spec():
    # spec: byte j of a row = (column 2j in the low nibble, column 2j+1 in the high nibble)
    K = 16
    for k in range(K):
        for c in (1, 7, 15):
            codes = np.zeros((1, K), np.uint8)
            codes[0, k] = c
            q = O.pack_int4(codes)
            expect = np.zeros(K // 2, np.uint8)
            expect[k // 2] = c if k % 2 == 0 else c * 16
            assert np.array_equal(q[0], expect), (k, c)


def test_pack_unpack_bijection_all_bytes():
    q = np.arange(256, dtype=np.uint8).reshape(1, 256)
    codes = O.unpack_int4(q)
    assert codes.shape == (1, 512)
    assert codes.max() <= 15
    # every (low, high) pair appears exactly once
    pairs = set(zip(codes[0, 0::2].tolist(), codes[0, 1::2].tolist()))
    assert len(pairs) == 256
    assert np.array_equal(O.pack_int4(codes), q)
    # byte 0x21 holds columns (1, 2)
    assert O.unpack_int4(np.array([[0x21]], np.uint8)).tolist() == [[1, 2]]


def test_pack_rejects_out_of_range():
    with pytest.raises(ValueError):
        O.pack_int4(np.full((1, 2), 16, np.uint8))


# ------------------------------------------------------------------ dequantize / GEMV known answers
@pytest.mark.parametrize("K", [128, 256, 2048])
def test_min_term_known_answer(K):
    N = 5
    q = np.zeros((N, K // 2), np.uint8)
    s = rng(1).uniform(1e-3, 2e-2, (N, K // 128)).astype(np.float16)
    m = np.ones((N, K // 128), np.float16)
    y = O.gemv_int4(np.ones(K, np.float16), q, s, m)
    assert np.array_equal(y, np.full(N, float(K), np.float32))


def test_all_fifteen_known_answer():
    N, K = 3, 512
    q = np.full((N, K // 2), 0xFF, np.uint8)
    s = rng(2).uniform(1e-3, 2e-2, (N, K // 128)).astype(np.float16)
    m = np.zeros_like(s)
    y = O.gemv_int4(np.ones(K, np.float16), q, s, m)
    expect = 15 * 128 * s.astype(np.float64).sum(axis=1)
    np.testing.assert_allclose(y, expect, rtol=1e-6)


def test_onehot_x_selects_column():
    N, K = 4, 256
    r = rng(3)
    codes = r.integers(0, 16, (N, K), dtype=np.uint8)
    q = O.pack_int4(codes)
    s = r.uniform(1e-3, 2e-2, (N, K // 128)).astype(np.float16)
    m = (-7.5 * s.astype(np.float32)).astype(np.float16)
    for k in (0, 1, 127, 128, 255):
        x = np.zeros(K, np.float16)
        x[k] = 1
        y = O.gemv_int4(x, q, s, m)
        g = k // 128
        expect = codes[:, k].astype(np.float64) * s[:, g].astype(np.float64) + m[:, g].astype(np.float64)
        np.testing.assert_allclose(y, expect, rtol=1e-6, atol=1e-9)


def test_factored_identity_bruteforce():
    # y[n] = sum_g ( scale[n,g] * sum_{k in g} code*x + min[n,g] * sum_{k in g} x ), with plain Python loops
    N, K = 3, 256
    r = rng(4)
    codes = r.integers(0, 16, (N, K))
    q = O.pack_int4(codes.astype(np.uint8))
    s = r.uniform(1e-3, 2e-2, (N, K // 128)).astype(np.float16)
    m = r.normal(0, 0.05, (N, K // 128)).astype(np.float16)
    x = r.normal(0, 1, K).astype(np.float16)
    ys = []
    for n in range(N):
        tot = 0.0
        for g in range(K // 128):
            dot = sum(int(codes[n, k]) * float(x[k]) for k in range(g * 128, (g + 1) * 128))
            xs = sum(float(x[k]) for k in range(g * 128, (g + 1) * 128))
            tot += float(s[n, g]) * dot + float(m[n, g]) * xs
        ys.append(tot)
    np.testing.assert_allclose(O.gemv_int4(x, q, s, m), ys, rtol=2e-5, atol=1e-6)
    np.testing.assert_allclose(O.gemv_int4_f64(x, q, s, m), ys, rtol=1e-12, atol=1e-12)


def test_fp32_oracle_close_to_float64():
    N, K = 256, 2048
    r = rng(5)
    q = O.pack_int4(r.integers(0, 16, (N, K), dtype=np.uint8))
    s = r.uniform(1e-3, 2e-2, (N, K // 128)).astype(np.float16)
    m = (-7.5 * s.astype(np.float32) + r.normal(0, 1, s.shape) * s.astype(np.float32)).astype(np.float16)
    x = r.normal(0, 1, K).astype(np.float16)
    y32 = O.gemv_int4(x, q, s, m)
    y64 = O.gemv_int4_f64(x, q, s, m)
    rep = O.parity_report(y32, y64)
    assert rep["cosine"] > 1 - 1e-10 and rep["norm_rel"] < 1e-6


# ------------------------------------------------------------------ quantize
def test_quantize_grid_exact_roundtrip():
    N, K = 4, 256
    r = rng(6)
    codes = r.integers(0, 16, (N, K), dtype=np.uint8)
    codes[:, ::128] = 0   # every group spans the full 0..15 range, so min/max fix the grid exactly
    codes[:, 1::128] = 15
    lo = -np.float32(0.25)
    step = np.float32(2.0 ** -6)  # (max - min) / 15 is then exactly step
    w = codes.astype(np.float32) * step + lo
    q, s, m = O.quantize(w)
    assert np.array_equal(O.unpack_int4(q), codes)
    assert np.all(s == np.float16(step)) and np.all(m == np.float16(lo))


def test_quantize_roundtrip_error_bound():
    N, K = 8, 512
    w = rng(7).normal(0, 0.02, (N, K)).astype(np.float32)
    q, s, m = O.quantize(w)
    wd = O.dequantize(q, s, m)
    s32 = np.repeat(s.astype(np.float32), 128, axis=1)
    # half a step of rounding + the fp16 rounding of scale (x15) and min
    bound = 0.5 * s32 + 16 * np.abs(s32) * 2.0 ** -11 + np.repeat(np.abs(m.astype(np.float32)), 128, 1) * 2.0 ** -11
    assert np.all(np.abs(wd - w) <= bound + 1e-9)


def test_quantize_constant_group_and_ties():
    w = np.full((1, 128), 0.5, np.float32)
    q, s, m = O.quantize(w)
    assert np.all(O.unpack_int4(q) == 0) and s[0, 0] == np.float16(1e-8) and m[0, 0] == np.float16(0.5)
    # ties: (w - min) / scale = 0.5 and 2.5 must round to 0 and 2 (half to even)
    w = np.zeros((1, 128), np.float32)
    w[0, 1] = 15.0            # max: scale = 1
    w[0, 2] = 0.5
    w[0, 3] = 2.5
    w[0, 4] = 3.5
    codes = O.unpack_int4(O.quantize(w)[0])
    assert codes[0, 2] == 0 and codes[0, 3] == 2 and codes[0, 4] == 4


# ------------------------------------------------------------------ int8 per-row head
def test_int8_extreme_rows():
    K = 2048
    q = np.stack([np.full(K, 127, np.int8), np.full(K, -127, np.int8), np.zeros(K, np.int8)])
    s = np.array([1e-3, 7e-3, 5e-3], np.float16)
    y = O.gemv_int8_rows(np.ones(K, np.float16), q, s, "s8")
    np.testing.assert_allclose(y, [127 * K * float(s[0]), -127 * K * float(s[1]), 0.0], rtol=2e-5)  # fp32 sums of K terms


def test_int8_layouts_agree():
    r = rng(8)
    q = r.integers(-127, 128, (16, 256)).astype(np.int8)
    s = r.uniform(1e-3, 1e-2, 16).astype(np.float16)
    x = r.normal(0, 1, 256).astype(np.float16)
    u = (q.astype(np.int16) + 128).astype(np.uint8)
    assert np.array_equal(O.gemv_int8_rows(x, q, s, "s8"), O.gemv_int8_rows(x, u, s, "u8"))


def test_quantize_int8_rows_roundtrip_and_padding():
    w = rng(9).normal(0, 0.02, (21, 64)).astype(np.float32)
    q, s = O.quantize_int8_rows(w, pad_to=16)
    assert q.shape == (32, 64) and s.shape == (32,)
    codes = O.int8_codes(q, "u8")
    assert codes.min() >= -127 and codes.max() <= 127
    assert np.all(codes[21:] == 0) and np.all(s[21:] == np.float32(1e-8))
    # the largest |w| of every row maps to +-127
    assert np.all(np.abs(codes[:21]).max(axis=1) == 127)
    assert np.all(np.abs(codes[:21] * s[:21, None] - w) <= 0.5 * s[:21, None] * (1 + 1e-6))


# ------------------------------------------------------------------ prefill
@pytest.mark.parametrize("M", [1, 3, 34])
def test_prefill_rows_are_gemvs(M):
    N, K = 48, 384
    r = rng(10 + M)
    q = O.pack_int4(r.integers(0, 16, (N, K), dtype=np.uint8))
    s = r.uniform(1e-3, 2e-2, (N, K // 128)).astype(np.float16)
    m = (-7.5 * s.astype(np.float32)).astype(np.float16)
    X = r.normal(0, 1, (M, K)).astype(np.float16)
    Y = O.mm_int4(X, q, s, m)
    for i in range(M):
        np.testing.assert_allclose(Y[i], O.gemv_int4_f64(X[i], q, s, m), rtol=1e-5, atol=1e-6)


def test_parity_metrics():
    ref = np.array([1.0, -2.0, 1e-6, 0.0])
    y = np.array([1.001, -2.0, 2e-6, 0.0])
    rep = O.parity_report(y, ref)
    # 1e-6 sits below the fp16 floor: its error is measured against 2^-14
    assert rep["max_rel"] == pytest.approx(max(1e-3, 1e-6 / 2.0 ** -14))
    assert 0.9999 < rep["cosine"] <= 1.0


def test_fp32_reference_within_conditioning_floor():
    # the premise of cond_floor: the fp32 dequantize-then-matmul itself stays within the bar against float64
    # (|err| <= 1e-2 * max(|ref|, 256 u32 sum|w x|)) on a config-sized problem
    N, K = 4096, 2048
    r = rng(13)
    q = O.pack_int4(r.integers(0, 16, (N, K), dtype=np.uint8))
    s = r.uniform(1e-3, 2e-2, (N, K // 128)).astype(np.float16)
    m = (-7.5 * s.astype(np.float32) + r.normal(0, 1, s.shape) * s.astype(np.float32)).astype(np.float16)
    x = r.normal(0, 1, K).astype(np.float16)
    ref64 = O.gemv_int4_f64(x, q, s, m)
    floor = O.cond_floor(O.gemv_int4_abs(x, q, s, m))
    rep = O.parity_report(O.gemv_int4(x, q, s, m), ref64, floor)
    assert rep["max_rel"] <= 1e-2 / 4, rep
    assert np.all(floor >= O.FP16_TINY) and np.all(floor < 0.01)
