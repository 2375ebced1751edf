"""numpy restatement of the decode-step glue and of one whole decode step (test infrastructure only).

References (neoandmatrix/rumik-fast):
  cohere_ln        engine/rumik_int4.py:38-43 (centre, rsqrt(mean(d^2) + eps), scale by w, no bias; fp32)
  rope tables      engine/rumik_int4.py:110-112 (inv = theta^(-arange(0, HD, 2)/HD); angles repeated twice)
  rope             engine/rumik_int4.py:46-52 / engine/fused.py:57-65 (interleaved pairs (2j, 2j+1))
  decode attention engine/rumik_int4.py:163-171, engine/test_attn.py:25-30 (GQA, fp32 softmax, scale HD^-0.5)
  flash-decoding   engine/fused.py:120-187 (partials (m, l, acc) per split; combine with w_i = exp(m_i - max m))
  post / add_ln    engine/fused.py:30-84 (where the fused step rounds to the activation dtype)
  step             engine/rumik_fused.py:97-121 (embed_ln; per layer gemv(w_in), post, attention, gemv(w_o),
                   gemv(w_down), add_ln; pos += 1; then the audio head)
Activations are rounded to `dt` (np.float16, or "bf16" as the reference engine stores them) exactly where the fused
step stores them: the projection outputs, q after RoPE, the K/V cache, act, the attention output, x after the residual
add, and h after each LayerNorm.
"""
import numpy as np

from . import int4 as I4


def round_bf16(v):
    """float32 -> the nearest bfloat16 (ties to even), returned as float32: bits + 0x7FFF + lsb, then the low 16 bits
    cleared (the usual round-to-nearest-even on the truncated half); inf / nan pass through."""
    a = np.asarray(v, np.float32)
    b = a.view(np.uint32).astype(np.uint64)
    r = (((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16).astype(np.uint32).view(np.float32)
    return np.where(np.isfinite(a), r, a).astype(np.float32)


def round_to(v, dt):
    """v rounded to the activation dtype dt (np.float16, "bf16" or np.float32), as float32."""
    if isinstance(dt, str) and dt == "bf16":
        return round_bf16(v)
    return np.asarray(v, np.float32).astype(dt).astype(np.float32)


def cohere_ln(x, w, eps=1e-5):
    xf = np.asarray(x, dtype=np.float32)
    d = xf - xf.mean(dtype=np.float32)
    return d / np.sqrt((d * d).mean(dtype=np.float32) + np.float32(eps)) * np.asarray(w, dtype=np.float32)


def rope_tables(S, HD, theta=10000.0):
    """cos, sin [S, HD] fp32, each angle repeated for the two elements of its pair."""
    inv = 1.0 / (np.float32(theta) ** (np.arange(0, HD, 2, dtype=np.float32) / np.float32(HD)))
    ang = np.outer(np.arange(S, dtype=np.float32), inv.astype(np.float32)).astype(np.float32)
    ang = np.repeat(ang, 2, axis=1)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def rope(x, cos_row, sin_row):
    """interleaved rotation of pairs (2j, 2j+1): (xe c - xo s, xo c + xe s); x [..., HD]."""
    xf = np.asarray(x, dtype=np.float32)
    xe, xo = xf[..., 0::2], xf[..., 1::2]
    c, s = np.asarray(cos_row, np.float32)[0::2], np.asarray(sin_row, np.float32)[0::2]
    out = np.empty_like(xf)
    out[..., 0::2] = xe * c - xo * s
    out[..., 1::2] = xo * c + xe * s
    return out


def attend(q, K, V, scale=None):
    """q [NH, HD], K / V [NKV, n, HD] -> [NH, HD] fp32; query head h reads KV head h // (NH / NKV)."""
    q = np.asarray(q, np.float32)
    NH, HD = q.shape
    NKV = K.shape[0]
    rep = NH // NKV
    scale = HD ** -0.5 if scale is None else scale
    out = np.empty((NH, HD), np.float32)
    for h in range(NH):
        k = np.asarray(K[h // rep], np.float32)
        v = np.asarray(V[h // rep], np.float32)
        s = (k @ q[h]) * np.float32(scale)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ v
    return out


def causal_attend(q, K, V, p0=0, scale=None):
    """Prefill attention (engine/rumik_int4.py:163-171: fp32 scores, causal bias, GQA): q [T, NH, HD] of positions
    p0 .. p0 + T - 1, K / V [NKV, >= p0 + T, HD] -> [T, NH, HD] fp32; query t reads slots 0 .. p0 + t."""
    q = np.asarray(q, np.float32)
    T, NH, HD = q.shape
    NKV = K.shape[0]
    rep = NH // NKV
    scale = HD ** -0.5 if scale is None else scale
    n = p0 + T
    k = np.asarray(K[:, :n], np.float32)
    v = np.asarray(V[:, :n], np.float32)
    bias = np.where(np.arange(n)[None, :] <= (p0 + np.arange(T))[:, None], 0.0, -np.inf).astype(np.float32)
    out = np.empty((T, NH, HD), np.float32)
    for h in range(NH):
        s = (q[:, h] @ k[h // rep].T) * np.float32(scale) + bias
        p = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, h] = (p / p.sum(axis=1, keepdims=True)) @ v[h // rep]
    return out


def attend_split(q, K, V, nsplit, chunk, scale=None):
    """Flash-decoding as the reference splits it: per split the partial (m, l, acc) over its slots, then the
    combine. Returns (out [NH, HD], m [NH, nsplit], l [NH, nsplit]); empty splits have m = -inf, l = 0."""
    q = np.asarray(q, np.float32)
    NH, HD = q.shape
    NKV, n = K.shape[0], K.shape[1]
    rep = NH // NKV
    scale = HD ** -0.5 if scale is None else scale
    m = np.full((NH, nsplit), -np.inf, np.float32)
    l = np.zeros((NH, nsplit), np.float32)
    acc = np.zeros((NH, nsplit, HD), np.float32)
    for h in range(NH):
        k = np.asarray(K[h // rep], np.float32)
        v = np.asarray(V[h // rep], np.float32)
        for sp in range(nsplit):
            a, b = sp * chunk, min(n, (sp + 1) * chunk)
            if a >= b:
                continue
            s = (k[a:b] @ q[h]) * np.float32(scale)
            m[h, sp] = s.max()
            p = np.exp(s - m[h, sp])
            l[h, sp] = p.sum()
            acc[h, sp] = p @ v[a:b]
    M = m.max(axis=1, keepdims=True)
    w = np.where(np.isfinite(m), np.exp(m - M), 0.0).astype(np.float32)
    out = (w[..., None] * acc).sum(1) / (w * l).sum(1)[:, None]
    return out, m, l


def silu(g):
    g = np.asarray(g, np.float32)
    return g / (1 + np.exp(-g))


class DecodeModel:
    """The synthetic decoder of config 4 (all arrays numpy, weights in the int4 / int8 formats).

    Fields: L, H, NH, NKV, HD, inter, eps; per layer w_in (q|k|v|gate|up rows), w_o, w_down as (q, s, m) and ln [H];
    norm [H]; emb (int8 [V, H], fp16 scale [V]); head (int8 codes [NV, H], fp16 scale [NV]); rope (cos, sin) [S, HD];
    sliding[L] (RoPE on / off per layer). cache_weights=True keeps each dequantized matrix after its first use (the
    same fp32 dequantize-then-matmul, computed once: for runs of many steps)."""

    def __init__(self, cache_weights=False, **kw):
        self.__dict__.update(kw)
        self.cache = {} if cache_weights else None


def _gemv(md, w, x):
    """dequantize(w) @ x in fp32 (oracle int4.gemv_int4), the dequantized matrix cached when the model asks for it."""
    if md.cache is None:
        return I4.gemv_int4(x, *w)
    key = id(w[0])
    if key not in md.cache:
        md.cache[key] = I4.dequantize(*w)
    return md.cache[key] @ np.asarray(x, np.float32)


def decode_step(md: DecodeModel, tok, pos, kc, vc, dt=np.float16):
    """One decode step at position `pos` for token `tok`; kc / vc [L, NKV, S, HD] are updated in place at `pos`
    (float16 arrays, or float32 arrays holding bf16 values when dt = "bf16"). Returns (logits fp32 [NV], hn [H],
    x [H]) as float32 holding dt values. Follows engine/rumik_fused.py:97-121 with the rounding points of
    engine/fused.py."""
    H, NH, NKV, HD, inter = md.H, md.NH, md.NKV, md.HD, md.inter
    r = lambda v: round_to(v, dt)  # noqa: E731 — round to the act dtype
    x = r(md.emb[0][tok].astype(np.float32) * np.float32(md.emb[1][tok]))                 # fused.py:20-22
    h = r(cohere_ln(x, md.ln[0], md.eps))
    cos, sin = md.rope
    for i in range(md.L):
        y = r(_gemv(md, md.w_in[i], h))                                                      # rumik_fused.py:102
        q = y[:NH * HD].reshape(NH, HD)
        k = y[NH * HD:(NH + NKV) * HD].reshape(NKV, HD)
        v = y[(NH + NKV) * HD:(NH + 2 * NKV) * HD].reshape(NKV, HD)
        g, u = y[(NH + 2 * NKV) * HD:(NH + 2 * NKV) * HD + inter], y[(NH + 2 * NKV) * HD + inter:]
        if md.sliding[i]:                                                                    # fused.py:57-65
            q, k = rope(q, cos[pos], sin[pos]), rope(k, cos[pos], sin[pos])
        q, k = r(q), r(k)
        kc[i, :, pos] = k
        vc[i, :, pos] = v
        act = r(silu(g) * u)                                                                 # fused.py:84
        o = r(attend(q, kc[i, :, :pos + 1].astype(np.float32), vc[i, :, :pos + 1].astype(np.float32)))
        a = r(_gemv(md, md.w_o[i], o.reshape(-1)))
        d = r(_gemv(md, md.w_down[i], act))
        x = r(x + a + d)                                                                     # fused.py:33-35
        h = r(cohere_ln(x, md.norm if i == md.L - 1 else md.ln[i + 1], md.eps))
    logits = I4.gemv_int8_rows(h, md.head[0], md.head[1], "s8")
    return logits, h, x
