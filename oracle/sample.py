"""numpy restatement of the decode step's sampling tail (test infrastructure only).

References (neoandmatrix/rumik-fast):
  stop predictor  engine/rumik_int4.py:174-180 (logits_and_stop: LayerNorm with weight and bias, eps 1e-5; linear;
                  exact GELU; linear; sigmoid > 0.5) and engine/sample.py:34-49, 84-87 (the fused kernels: W1 in
                  bf16, everything else fp32; sigmoid(s) > 0.5 tested as s > 0)
  sortable keys   engine/sample.py:7-11, 23-31 (key32 = b ^ ((b >> 31) & 0x7FFFFFFF); key = key32 << 32 | index)
  top-k + sample  engine/rumik_int4.py:182-191 (_pick: </audio> masked for the first min_new steps, top-k, Gumbel
                  noise -log(-log(clamp(u, 1e-10, 1))), argmax of top_v / T + g, ids lookup, stop -> end_id once
                  step >= min_new) and engine/sample.py:53-93 (stage 1 / stage 2 on packed keys, first maximum)
  counters        engine/rumik_int4.py:193-198 (out[step] = token, tok = token, step += 1)
"""
import math

import numpy as np


def sortable(x):
    """float32 values -> int32 keys whose integer order is the value order (-inf included)."""
    b = np.asarray(x, dtype=np.float32).view(np.int32)
    return b ^ ((b >> 31) & np.int32(0x7FFFFFFF))


def unsortable(k):
    k = np.asarray(k, dtype=np.int32)
    return (k ^ ((k >> 31) & np.int32(0x7FFFFFFF))).view(np.float32)


def make_keys(x, idx):
    """int64 key = key32 << 32 | index (key32 sign-extended first, as the Triton code does)."""
    return (sortable(x).astype(np.int64) << 32) | np.asarray(idx, dtype=np.int64)


def masked_logits(logits, step, end_idx, min_new):
    """fp32 logits with </audio> (index end_idx) at -inf while step < min_new."""
    lg = np.asarray(logits, dtype=np.float32).copy()
    if step < min_new:
        lg[end_idx] = -np.inf
    return lg


def sorted_keys(logits, step, end_idx, min_new):
    """every logit's key, sorted descending (value first, then the larger index)."""
    lg = masked_logits(logits, step, end_idx, min_new)
    return np.sort(make_keys(lg, np.arange(lg.size)))[::-1]


def topk(logits, step, end_idx, min_new, k):
    """(values, indices) of the top k in key order."""
    keys = sorted_keys(logits, step, end_idx, min_new)[:k]
    return unsortable((keys >> 32).astype(np.int32)), (keys & 0xFFFFFFFF).astype(np.int64)


def gelu(y):
    """exact GELU (F.gelu default): 0.5 y (1 + erf(y / sqrt 2))."""
    y = np.asarray(y, dtype=np.float64)
    return 0.5 * y * (1.0 + np.vectorize(math.erf)(y / math.sqrt(2.0)))


def stop_hidden(h, lnw, lnb, w1, b1, eps=1e-5):
    """z1 = gelu(W1 . LayerNorm(h) + b1), float64 arithmetic on the given (fp32 / bf16-valued) inputs."""
    x = np.asarray(h, dtype=np.float64)
    d = x - x.mean()
    z = d / np.sqrt((d * d).mean() + eps) * np.asarray(lnw, np.float64) + np.asarray(lnb, np.float64)
    return gelu(np.asarray(w1, np.float64) @ z + np.asarray(b1, np.float64))


def stop_logit(z1, w2, b2):
    return float(np.asarray(z1, np.float64) @ np.asarray(w2, np.float64) + float(np.asarray(b2).reshape(-1)[0]))


def gumbel(u):
    """-log(-log(clamp(u, 1e-10, 1))) in fp32."""
    uu = np.clip(np.asarray(u, dtype=np.float32), np.float32(1e-10), np.float32(1.0))
    return (-np.log(-np.log(uu))).astype(np.float32)


def scores(logits, u, step, end_idx, min_new, top_k, temperature):
    """fp32 Gumbel scores of the top-k candidates (key order) and their indices."""
    v, i = topk(logits, step, end_idx, min_new, top_k)
    return (v * np.float32(1.0 / temperature) + gumbel(np.asarray(u)[:top_k])).astype(np.float32), i


def pick(logits, u, ids, step, end_idx, min_new, end_id, top_k, temperature, stop_s):
    """the next token: the first maximum of the scores (candidates in key order), then the stop rule."""
    sc, i = scores(logits, u, step, end_idx, min_new, top_k, temperature)
    nxt = int(np.asarray(ids)[i[int(np.argmax(sc))]])
    if stop_s > 0 and step >= min_new:
        nxt = int(end_id)
    return nxt
