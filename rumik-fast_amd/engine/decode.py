"""The batch-1 decode step of the synthetic Rumik decoder on MI355X (config 4 of the benchmark definition).

Mirrors RumikFused._step (reference engine/rumik_fused.py:97-121) with this build's kernels:

    embed_ln(tok) -> 36 x [ gemv(w_in) -> post -> attn_split -> attn_combine -> gemv(w_o) -> gemv(w_down)
                             -> add_ln (next layer's LayerNorm; the final norm after the last layer) ]
    -> pos += 1 -> int8 audio head (fp32 logits)

Weights are in the reference's formats: per layer w_in = [q 2048 | k 512 | v 512 | gate 11008 | up 11008] rows
(the engine concatenates them at load time, engine/rumik_int4.py:95-98), w_o, w_down, all int4 g128; the audio head
is int8 with a per-row scale; the token embedding is int8 with a per-row fp16 scale. All buffers are static and
`pos` / `tok` live on the GPU, so one captured hipGraph replays the step at every position
(reference engine/rumik_int4.py:225-248). The sampler after the head is outside this path.
"""
import math
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "kernels"))
import cuda_gemv  # noqa: E402
import synth  # noqa: E402
import fused  # noqa: E402


class Config:
    """Model shape. Defaults: the 36-layer 3B decoder (hidden 2048, 16 q / 4 kv heads of 128, MLP 11008)."""

    def __init__(self, L=36, H=2048, NH=16, NKV=4, HD=128, inter=11008, S=2048, n_audio=16385, vocab=4096,
                 eps=1e-5, rope_theta=10000.0, nsplit=64, sliding=None):
        self.L, self.H, self.NH, self.NKV, self.HD, self.inter = L, H, NH, NKV, HD, inter
        self.S, self.n_audio, self.vocab, self.eps, self.rope_theta, self.nsplit = S, n_audio, vocab, eps, rope_theta, nsplit
        # RoPE on 3 of every 4 layers ("sliding" layers), none on every 4th (reference engine/rumik_int4.py:10-11)
        self.sliding = list(sliding) if sliding is not None else [i % 4 != 3 for i in range(L)]

    @property
    def n_in(self):
        return (self.NH + 2 * self.NKV) * self.HD + 2 * self.inter

    def weight_bytes(self):
        def i4(N, K):
            return N * K // 2 + 4 * N * (K // 128)
        per_layer = i4(self.n_in, self.H) + i4(self.H, self.NH * self.HD) + i4(self.H, self.inter)
        return self.L * per_layer + self.n_audio * self.H + 2 * self.n_audio

    def kv_bytes(self, ctx):
        return self.L * 2 * self.NKV * ctx * self.HD * 2


def rope_tables(S, HD, theta, dtype, device):
    """cos / sin [S, HD], each angle repeated for its pair (reference engine/rumik_int4.py:110-112)."""
    inv = 1.0 / (theta ** (torch.arange(0, HD, 2, dtype=torch.float32) / HD))
    ang = torch.outer(torch.arange(S, dtype=torch.float32), inv).repeat_interleave(2, -1)
    return ang.cos().to(dtype).to(device).contiguous(), ang.sin().to(dtype).to(device).contiguous()


def random_weights(cfg: Config, seed: int, device, gen_device="cuda"):
    """Random-init weights of the config's architecture in the reference formats (values irrelevant to speed)."""
    g = synth.generator(seed, gen_device)
    w = {"w_in": [], "w_o": [], "w_down": [], "ln": []}
    for _ in range(cfg.L):
        w["w_in"].append(synth.int4_weights(cfg.n_in, cfg.H, g, device=device))
        w["w_o"].append(synth.int4_weights(cfg.H, cfg.NH * cfg.HD, g, device=device))
        w["w_down"].append(synth.int4_weights(cfg.H, cfg.inter, g, device=device))
        w["ln"].append(torch.ones(cfg.H, dtype=torch.float16, device=device))
    w["norm"] = torch.ones(cfg.H, dtype=torch.float16, device=device)
    w["emb"] = synth.int8_weights(cfg.vocab, cfg.H, g, device=device)
    w["head"] = synth.int8_weights(cfg.n_audio, cfg.H, g, device=device)
    return w


class DecodeStep:
    """Static buffers + the step. `weights` is a dict as from random_weights (tensors already on `device`)."""

    def __init__(self, cfg: Config, weights, device="cuda", dtype=torch.float16):
        self.cfg, self.w, self.dev, self.dt = cfg, weights, torch.device(device), dtype
        c, d = cfg, self.dev
        self.x = torch.zeros(c.H, dtype=dtype, device=d)
        self.h = torch.zeros(c.H, dtype=dtype, device=d)
        self.buf_in = torch.zeros(c.n_in, dtype=dtype, device=d)
        self.qb = torch.zeros(c.NH * c.HD, dtype=dtype, device=d)
        self.ob = torch.zeros(c.NH * c.HD, dtype=dtype, device=d)
        self.act = torch.zeros(c.inter, dtype=dtype, device=d)
        self.buf_o = torch.zeros(c.H, dtype=dtype, device=d)
        self.buf_d = torch.zeros(c.H, dtype=dtype, device=d)
        self.logits = torch.zeros(c.n_audio, dtype=torch.float32, device=d)
        self.po = torch.zeros(c.NH, c.nsplit, c.HD, dtype=torch.float32, device=d)
        self.pm = torch.zeros(c.NH, c.nsplit, dtype=torch.float32, device=d)
        self.pl = torch.zeros(c.NH, c.nsplit, dtype=torch.float32, device=d)
        self.kc = torch.zeros(c.L, c.NKV, c.S, c.HD, dtype=dtype, device=d)
        self.vc = torch.zeros_like(self.kc)
        self.tok = torch.zeros(1, dtype=torch.int64, device=d)
        self.pos = torch.zeros(1, dtype=torch.int64, device=d)
        self.cos, self.sin = rope_tables(c.S, c.HD, c.rope_theta, dtype, d)
        self.graph = None

    def set_state(self, tok: int, pos: int):
        self.tok.fill_(tok)
        self.pos.fill_(pos)

    def fill_cache(self, ctx: int, seed: int = 0):
        """KV cache slots [0, ctx) ~ N(0, 1) (the config-4 synthetic context)."""
        g = torch.Generator(device=self.dev).manual_seed(seed)
        self.kc[:, :, :ctx].normal_(generator=g)
        self.vc[:, :, :ctx].normal_(generator=g)

    def step(self):
        """Enqueue one decode step on the current stream (engine/rumik_fused.py:97-121)."""
        c, w = self.cfg, self.w
        scale = c.HD ** -0.5
        fused.embed_ln(self.tok, w["emb"][0], w["emb"][1], w["ln"][0], self.x, self.h, c.eps)
        for i in range(c.L):
            cuda_gemv.gemv_int4_cuda(self.h, *w["w_in"][i], out=self.buf_in)
            fused.post(self.buf_in, self.pos, self.cos, self.sin, self.kc[i], self.vc[i], self.qb, self.act,
                       c.NH, c.NKV, c.HD, c.inter, c.sliding[i])
            fused.attn_split(self.qb, self.kc[i], self.vc[i], self.pos, self.po, self.pm, self.pl, c.NH, c.NKV, c.HD,
                             c.nsplit, scale)
            fused.attn_combine(self.po, self.pm, self.pl, self.pos, self.ob, c.NH, c.HD, c.nsplit)
            cuda_gemv.gemv_int4_cuda(self.ob, *w["w_o"][i], out=self.buf_o)
            cuda_gemv.gemv_int4_cuda(self.act, *w["w_down"][i], out=self.buf_d)
            fused.add_ln(self.x, self.buf_o, self.buf_d, w["norm"] if i == c.L - 1 else w["ln"][i + 1], self.h, c.eps)
        fused.pos_advance(self.pos)
        cuda_gemv.gemv_int8_cuda(self.h, *w["head"], out=self.logits)

    def capture(self):
        """Record one step in a hipGraph (warm-up on a side stream first, as engine/rumik_int4.py:225-248).
        Device state (x, KV cache, pos) is saved and restored around the warm-up and the capture."""
        saved = (self.x.clone(), self.kc.clone(), self.vc.clone(), self.pos.clone())
        s = torch.cuda.Stream(device=self.dev)
        s.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(s):
            self.step()
        torch.cuda.current_stream(self.dev).wait_stream(s)
        torch.cuda.synchronize(self.dev)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.step()
        torch.cuda.synchronize(self.dev)
        self.x.copy_(saved[0]); self.kc.copy_(saved[1]); self.vc.copy_(saved[2]); self.pos.copy_(saved[3])
        torch.cuda.synchronize(self.dev)
        self.graph = g
        return g

    def replay(self):
        self.graph.replay()
