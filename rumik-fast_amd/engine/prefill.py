"""Prompt prefill on MI355X: all T prompt rows of a layer at once, weights staying int4 (the reference's
RumikFused.prefill, engine/rumik_fused.py:54-78).

    x = embed(ids); h = LN(x)                                      rk_embed_ln_rows
    per layer:  y   = h @ w_in^T                                   mm_int4 (rk_mm_int4_g128_ws, matrix cores)
                q, K/V cache slots 0..T-1, act = silu(g) * u        rk_post_rows (RoPE on sliding layers)
                o   = causal GQA attention(q, K, V)                rk_prefill_attn (matrix cores, replaces the
                                                                   reference's torch fp32 _attend, rumik_int4.py:163-171)
                x  += o @ w_o^T + act @ w_down^T; h = LN(x)        mm_int4, mm_int4, rk_add_ln_rows
    hn = h[T-1] (the final LayerNorm), pos = T

The engine's K / V cache and activation dtype are used (fp16); `hn` then feeds the audio head and the sampling tail
(PersistentDecode.first_token). No CPU path: every kernel is in librumik_hip.so.
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "kernels"))
import _hiplib as HL  # noqa: E402
import mm_int4 as MM  # noqa: E402


def _s(t):
    return HL.stream(t.device)


def embed_ln_rows(ids, emb_q, emb_s, ln_w, x, h, eps):
    T, H = ids.numel(), ln_w.numel()
    HL.check(HL.lib().rk_embed_ln_rows(HL.ptr(ids), HL.ptr(emb_q), HL.ptr(emb_s), HL.ptr(ln_w), HL.ptr(x), HL.ptr(h),
                                       HL.dt(x), T, H, float(eps), _s(x)), "embed_ln_rows")


def add_ln_rows(x, a, b, ln_w, h, T, eps):
    HL.check(HL.lib().rk_add_ln_rows(HL.ptr(x), HL.ptr(a), HL.ptr(b), HL.ptr(ln_w), HL.ptr(h), HL.dt(x), T,
                                     ln_w.numel(), float(eps), _s(x)), "add_ln_rows")


def post_rows(y, p0, cos, sin, kc, vc, q_out, act, T, NH, NKV, HD, S, inter, rope):
    HL.check(HL.lib().rk_post_rows(HL.ptr(y), y.stride(0), int(p0), HL.ptr(cos), HL.ptr(sin), HL.ptr(kc), HL.ptr(vc),
                                   HL.ptr(q_out), HL.ptr(act), HL.dt(y), T, NH, NKV, HD, S, inter, int(bool(rope)),
                                   _s(y)), "post_rows")


def prefill_attn(q, kc, vc, o, T, p0, NH, NKV, HD, S, scale):
    """o[t] = softmax(q[t] K[0..p0+t]^T * scale) V[0..p0+t] per query head (GQA: heads h of KV head h // (NH / NKV));
    q, o [T, NH * HD] fp16; kc, vc [NKV, S, HD] fp16 (one layer's cache)."""
    HL.require_gpu(q, kc, vc, o)
    HL.check(HL.lib().rk_prefill_attn(HL.ptr(q), HL.ptr(kc), HL.ptr(vc), HL.ptr(o), HL.dt(q), T, int(p0), NH, NKV,
                                      HD, S, float(scale), _s(q)), "prefill_attn")


class Prefill:
    """Buffers for prompts of up to max_T tokens. `w`: the per-layer int4 weights in the reference layout (the dict
    decode.random_weights / weights.load return; keep it: PersistentDecode re-lays out its own copy), `kc` / `vc`:
    the engine's cache [L, NKV, S, HD], `cos` / `sin`: its RoPE tables."""

    def __init__(self, cfg, w, kc, vc, cos, sin, max_T=512, graphs=False, bucket=16, overlap=None):
        """graphs: run each prompt as a replay of a hipGraph holding all of its ~220 launches, one graph per prompt
        length rounded up to a multiple of `bucket` (captured on the first prompt of that bucket). The rows past the
        prompt run on token id 0: they change none of the prompt's rows (every kernel is row-wise or causal), and
        their K / V go to cache slots the decode step overwrites (slot pos) before any step attends to them."""
        self.cfg, self.w, self.kc, self.vc, self.cos, self.sin = cfg, w, kc, vc, cos, sin
        self.graphs = {} if graphs else None
        self.bucket = int(bucket)
        # overlap: the down product's branch (its X pre-pass, product and split-K sum) runs on a second stream,
        # beside the attention and the o product (both read only what post_rows wrote and meet again at
        # add_ln_rows); default priority, like every stream here. None: on for graph replays and for prompts of at
        # least 256 rows (eagerly, the two extra stream switches per layer cost more host time than a short prompt's
        # kernels take).
        self.overlap = overlap
        self.side = torch.cuda.Stream(device=kc.device)
        self.ev_fork = [torch.cuda.Event() for _ in range(cfg.L)]
        self.ev_join = [torch.cuda.Event() for _ in range(cfg.L)]
        c, d, dt = cfg, kc.device, kc.dtype
        if dt != torch.float16:
            raise RuntimeError("the prefill attention runs on fp16 K / V")
        for key in ("w_in", "w_o", "w_down"):
            if len(w[key]) != c.L:
                raise RuntimeError(f"weights[{key!r}] holds {len(w[key])} layers, expected {c.L} (build the engine "
                                   "with keep_layer_weights=True)")
        self.max_T = int(min(max_T, c.S))
        z = lambda *s: torch.zeros(*s, dtype=dt, device=d)  # noqa: E731
        T = self.max_T
        self.x, self.h = z(T, c.H), z(T, c.H)
        self.y = z(T, c.n_in)
        self.q, self.o = z(T, c.NH * c.HD), z(T, c.NH * c.HD)
        self.act = z(T, c.inter)
        self.a, self.d = z(T, c.H), z(T, c.H)
        self.ids = torch.zeros(T, dtype=torch.int64, device=d)

    def run(self, ids, hn=None):
        """Fill cache slots 0..T-1 for the prompt `ids` and return hn (= LN_final(x[T-1]), written to `hn` too)."""
        c, w = self.cfg, self.w
        T = len(ids)
        if not 1 <= T <= self.max_T:
            raise ValueError(f"prompt of {T} tokens (1..{self.max_T})")
        if self.graphs is None:
            self.ids[:T].copy_(torch.as_tensor(list(ids), dtype=torch.int64))
            self._enqueue(T)
        else:
            Tb = min(self.max_T, -(-T // self.bucket) * self.bucket)
            self.ids[:Tb].copy_(torch.as_tensor(list(ids) + [0] * (Tb - T), dtype=torch.int64))
            g = self.graphs.get(Tb)
            if g is None:
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    self._enqueue(Tb)
                self.graphs[Tb] = g
            g.replay()
        if hn is not None:
            hn.copy_(self.h[T - 1])
        return self.h[T - 1]

    def _enqueue(self, T):
        """Every kernel of the prefill of rows 0..T-1 (the prompt ids already in self.ids), on the current stream."""
        c, w = self.cfg, self.w
        embed_ln_rows(self.ids[:T], w["emb"][0], w["emb"][1], w["ln"][0], self.x, self.h, c.eps)
        scale = c.HD ** -0.5
        main = torch.cuda.current_stream(self.kc.device)
        ov = self.overlap if self.overlap is not None else (self.graphs is not None or T >= 256)
        for i in range(c.L):
            MM.mm_int4(self.h[:T], *w["w_in"][i], out=self.y[:T])
            post_rows(self.y, 0, self.cos, self.sin, self.kc[i], self.vc[i], self.q, self.act, T, c.NH, c.NKV, c.HD,
                      c.S, c.inter, c.sliding[i])
            if ov:
                self.ev_fork[i].record(main)  # act is written
                self.side.wait_event(self.ev_fork[i])
                with torch.cuda.stream(self.side):
                    MM.mm_int4(self.act[:T], *w["w_down"][i], out=self.d[:T])
                self.ev_join[i].record(self.side)
            prefill_attn(self.q, self.kc[i], self.vc[i], self.o, T, 0, c.NH, c.NKV, c.HD, c.S, scale)
            MM.mm_int4(self.o[:T], *w["w_o"][i], out=self.a[:T])
            if ov:
                main.wait_event(self.ev_join[i])  # d is written (and act may be rewritten by the next layer)
            else:
                MM.mm_int4(self.act[:T], *w["w_down"][i], out=self.d[:T])
            add_ln_rows(self.x, self.a, self.d, w["norm"] if i == c.L - 1 else w["ln"][i + 1], self.h, T, c.eps)
