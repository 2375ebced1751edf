#!/usr/bin/env python3
"""Writes the small golden fixtures of this directory (inputs + float64 expected outputs), from seeded CPU
generators. Run from the repository root:  python tests/golden/make_golden.py

The expected outputs are computed here in float64 straight from the definitions of the formats (not through the
oracle package), so the fixtures also check the oracle:
  int4 GEMV   y[n] = sum_k (code[n,k] * scale[n,k/128] + min[n,k/128]) * x[k]; code k = low nibble of byte k/2
              when k is even, high nibble when odd (reference kernels/int4_gemv.py:3,23,29-30)
  int8 head   y[n] = s[n] * sum_k c[n,k] x[k], c int8 in [-127, 127] (kernels/cuda_gemv.py:236,246 with c = q - 128)
  prefill     Y[m] = the int4 GEMV of X[m] (kernels/mm_int4.py:37-46)
  LayerNorm   (x - mean) / sqrt(mean((x - mean)^2) + eps) * w (engine/rumik_int4.py:38-43)
  RoPE        pairs (2j, 2j+1) rotated by pos * theta^(-2j/128) (engine/rumik_int4.py:46-52,110-112)
  attention   softmax(K q * 128^-0.5) V per query head, KV head h // (NH/NKV) (engine/rumik_int4.py:163-171)
"""
import math
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def rng(seed):
    return np.random.default_rng(seed)


def int4_case(r, N, K):
    codes = r.integers(0, 16, size=(N, K), dtype=np.uint8)
    q = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    s = r.uniform(1e-3, 2e-2, size=(N, K // 128)).astype(np.float16)
    m = (-7.5 * s.astype(np.float32) + r.standard_normal((N, K // 128)).astype(np.float32) * s).astype(np.float16)
    return codes, q, s, m


def dequant64(codes, s, m):
    s64 = np.repeat(s.astype(np.float64), 128, axis=1)
    m64 = np.repeat(m.astype(np.float64), 128, axis=1)
    return codes.astype(np.float64) * s64 + m64


def main():
    # int4 GEMV: ragged N, three groups
    r = rng(100)
    codes, q, s, m = int4_case(r, 96, 384)
    x = r.standard_normal(384).astype(np.float16)
    y = dequant64(codes, s, m) @ x.astype(np.float64)
    np.savez_compressed(HERE / "gemv_int4_96x384.npz", x=x, q=q, s=s, m=m, y=y)

    # int8 per-row head GEMV
    r = rng(101)
    c = r.integers(-127, 128, size=(80, 256), dtype=np.int8)
    sc = r.uniform(1e-3, 1e-2, size=80).astype(np.float16)
    x = r.standard_normal(256).astype(np.float16)
    y = sc.astype(np.float64) * (c.astype(np.float64) @ x.astype(np.float64))
    np.savez_compressed(HERE / "gemv_int8_80x256.npz", x=x, codes=c, s=sc, y=y)

    # prefill matmul
    r = rng(102)
    codes, q, s, m = int4_case(r, 64, 256)
    X = r.standard_normal((5, 256)).astype(np.float16)
    Y = X.astype(np.float64) @ dequant64(codes, s, m).T
    np.savez_compressed(HERE / "mm_int4_5x64x256.npz", X=X, q=q, s=s, m=m, Y=Y)

    # LayerNorm of a hidden vector
    r = rng(103)
    x = (r.standard_normal(2048) * 3 + 0.5).astype(np.float16)
    w = r.uniform(0.5, 1.5, 2048).astype(np.float16)
    x64 = x.astype(np.float64)
    d = x64 - x64.mean()
    h = d / math.sqrt((d * d).mean() + 1e-5) * w.astype(np.float64)
    np.savez_compressed(HERE / "layernorm_2048.npz", x=x, w=w, eps=np.float64(1e-5), h=h)

    # RoPE tables (theta 10000, head dim 128) and one rotated head
    S, HD, theta = 64, 128, 10000.0
    inv = theta ** (-np.arange(0, HD, 2, dtype=np.float64) / HD)
    ang = np.repeat(np.outer(np.arange(S, dtype=np.float64), inv), 2, axis=1)
    r = rng(104)
    v = r.standard_normal(HD).astype(np.float16)
    pos = 37
    v64 = v.astype(np.float64)
    c, sn = np.cos(ang[pos, 0::2]), np.sin(ang[pos, 0::2])
    rot = np.empty(HD)
    rot[0::2] = v64[0::2] * c - v64[1::2] * sn
    rot[1::2] = v64[1::2] * c + v64[0::2] * sn
    np.savez_compressed(HERE / "rope_64x128.npz", cos=np.cos(ang), sin=np.sin(ang), v=v, pos=np.int64(pos), rot=rot)

    # GQA decode attention, 8 query heads over 2 KV heads, 37 slots
    r = rng(105)
    NH, NKV, n = 8, 2, 37
    qh = r.standard_normal((NH, HD)).astype(np.float16)
    Kc = r.standard_normal((NKV, n, HD)).astype(np.float16)
    Vc = r.standard_normal((NKV, n, HD)).astype(np.float16)
    out = np.empty((NH, HD))
    for hh in range(NH):
        k, vv = Kc[hh // (NH // NKV)].astype(np.float64), Vc[hh // (NH // NKV)].astype(np.float64)
        sc = k @ qh[hh].astype(np.float64) / math.sqrt(HD)
        p = np.exp(sc - sc.max())
        out[hh] = p @ vv / p.sum()
    np.savez_compressed(HERE / "attention_8x2x37.npz", q=qh, K=Kc, V=Vc, out=out)
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
