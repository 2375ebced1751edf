"""The batch-1 decode step of the synthetic Rumik decoder on MI355X (config 4 of the benchmark definition).

Mirrors RumikFused._step (reference engine/rumik_fused.py:97-121) with this build's kernels:

    embed_ln(tok) -> 36 x [ gemv(w_in) -> post -> attn_split -> attn_combine -> gemv(w_o) + gemv(w_down) (one launch)
                             -> add_ln (next layer's LayerNorm; the final norm after the last layer) ]
    -> pos += 1 -> int8 audio head (fp32 logits)

Weights are in the reference's formats: per layer w_in = [q 2048 | k 512 | v 512 | gate 11008 | up 11008] rows
(the engine concatenates them at load time, engine/rumik_int4.py:95-98), w_o, w_down, all int4 g128; the audio head
is int8 with a per-row scale; the token embedding is int8 with a per-row fp16 scale. All buffers are static and
`pos` / `tok` live on the GPU, so one captured hipGraph replays the step at every position
(reference engine/rumik_int4.py:225-248). The sampler after the head is outside this path.
"""
import ctypes
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "kernels"))
import cuda_gemv  # noqa: E402
import synth  # noqa: E402
import _hiplib as HL  # noqa: E402
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
    """Random-init weights of the config's architecture in the reference formats (values irrelevant to speed).
    LayerNorm weights are drawn per layer (not 1), so a wrong layer index changes the results."""
    g = synth.generator(seed, gen_device)
    w = {"w_in": [], "w_o": [], "w_down": [], "ln": []}
    for _ in range(cfg.L):
        w["w_in"].append(synth.int4_weights(cfg.n_in, cfg.H, g, device=device))
        w["w_o"].append(synth.int4_weights(cfg.H, cfg.NH * cfg.HD, g, device=device))
        w["w_down"].append(synth.int4_weights(cfg.H, cfg.inter, g, device=device))
        w["ln"].append(synth.ln_weights(cfg.H, g, device=device))
    w["norm"] = synth.ln_weights(cfg.H, g, device=device)
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
        fused.embed_ln[(1,)](self.tok, w["emb"][0], w["emb"][1], w["ln"][0], self.x, self.h, c.eps, H=c.H)
        for i in range(c.L):
            cuda_gemv.gemv_int4_cuda(self.h, *w["w_in"][i], out=self.buf_in)
            fused.post[(1,)](self.buf_in, self.pos, self.cos, self.sin, self.kc[i], self.vc[i], self.qb, self.act,
                             c.S, c.inter, NH=c.NH, NKV=c.NKV, HD=c.HD, ROPE=c.sliding[i])
            fused.attn_split[(c.NKV, c.nsplit)](self.qb, self.kc[i], self.vc[i], self.pos, self.po, self.pm, self.pl,
                                                c.S, scale, REP=c.NH // c.NKV, HD=c.HD, NSPLIT=c.nsplit)
            fused.attn_combine[(c.NH,)](self.po, self.pm, self.pl, self.pos, self.ob, HD=c.HD, NSPLIT=c.nsplit)
            cuda_gemv.gemv_int4_pair_cuda(self.ob, w["w_o"][i], self.act, w["w_down"][i], out1=self.buf_o,
                                          out2=self.buf_d)
            fused.add_ln[(1,)](self.x, self.buf_o, self.buf_d, w["norm"] if i == c.L - 1 else w["ln"][i + 1], self.h,
                               c.eps, H=c.H)
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


# ---------------------------------------------------------------------------------------------- one-launch step
class RkDecodeParams(ctypes.Structure):
    """ctypes mirror of rk_decode_params (include/rumik_hip.h); its size is checked against the library."""
    _fields_ = [(n, ctypes.c_int) for n in ("L", "NH", "NKV", "inter", "S", "n_audio", "nsp")] + [
        ("eps", ctypes.c_float), ("scale", ctypes.c_float), ("sliding", ctypes.c_ulonglong)] + [
        (n, ctypes.c_void_p) for n in (
            "tok", "pos", "emb_q", "emb_s", "win_t", "win_sm", "wo_q", "wo_sm", "wd_t", "wd_sm", "ln_w", "norm_w",
            "cos_t", "sin_t", "kc", "vc", "head_q", "head_s", "logits", "work", "tx", "tq", "tkv", "top", "tdp",
            "tpo", "tml", "ctr", "status", "hn")]


class RkDecodeLimits(ctypes.Structure):
    """ctypes mirror of rk_decode_limits (include/rumik_hip.h): the persistent kernel's compiled limits."""
    _fields_ = [(n, ctypes.c_int) for n in ("max_tiles", "first_pass", "max_slices", "work_stride", "slice_begin_col",
                                            "slice_end_col", "x_copies", "max_splits", "max_slots_per_split")]


def decode_limits() -> RkDecodeLimits:
    """The limits the library was compiled with (a host-only query: no GPU needed)."""
    lim = RkDecodeLimits()
    HL.check(HL.lib().rk_decode_get_limits(ctypes.byref(lim)), "decode_get_limits")
    return lim


def interleave_gate_up(t, cfg):
    """Reorder w_in rows (or their scale / min rows) [q | k | v | gate | up] -> [q | k | v | (gate 8, up 8) ...]:
    the persistent kernel computes silu(gate) * up in the epilogue of a 16-row tile holding both."""
    a = (cfg.NH + 2 * cfg.NKV) * cfg.HD
    g, u = t[a:a + cfg.inter], t[a + cfg.inter:]
    gu = torch.stack([g.reshape(cfg.inter // 8, 8, -1), u.reshape(cfg.inter // 8, 8, -1)], 1)
    return torch.cat([t[:a], gu.reshape(2 * cfg.inter, -1)]).contiguous()


def pack_scale_min(s, m):
    """fp16 scale, min [..] -> int32 scale | min << 16 (the kernel's per-(row, group) word)."""
    lo = s.contiguous().view(torch.int16).to(torch.int32) & 0xFFFF
    hi = m.contiguous().view(torch.int16).to(torch.int32) << 16
    return (lo | hi).contiguous()


def wave_scale_min(sm):
    """per-(row, group) scale | min words [n_in, 16] -> per (tile, wave, row) the two words of the wave's groups:
    waves 1..7 hold groups 2(w - 1), 2(w - 1) + 1, wave 0 groups 14, 15. Returns int32 [n_in / 16, 8, 16, 2]."""
    nt = sm.shape[0] // 16
    per_group = sm.reshape(nt, 16, 8, 2)            # [tile, row, group pair, 2]
    order = torch.tensor([7, 0, 1, 2, 3, 4, 5, 6])  # wave w -> group pair (w + 7) % 8
    return per_group[:, :, order].permute(0, 2, 1, 3).contiguous()


def tile_layout(q):
    """w_in codes [n_in, 1024] -> per (tile, 128-column group) the 16 rows x 64 bytes in lane order: lane j + 16s
    holds row j's bytes [16s, 16s + 16) of the group. Returns [n_in / 16, 16, 64, 16] uint8."""
    nt = q.shape[0] // 16
    return q.reshape(nt, 16, 16, 4, 16).permute(0, 2, 3, 1, 4).contiguous().reshape(nt, 16, 64, 16)


def down_layout(q):
    """w_down codes [2048, inter / 2] -> per 16-column slice the 2048 rows x 8 bytes: [inter / 16, 2048, 8]."""
    return q.reshape(q.shape[0], -1, 8).permute(1, 0, 2).contiguous()


def o_layout(q, nh):
    """w_o codes [2048, nh * 64] -> per (head h, row group r of 128 rows) 512 items of 16 bytes, item i = row
    128r + i / 4, the codes of columns 128h + 32(i % 4) .. + 32: [nh, 16, 512, 16]."""
    rows = q.shape[0]
    return q.reshape(rows // 128, 128, nh, 4, 16).permute(2, 0, 1, 3, 4).reshape(nh, rows // 128, 512, 16).contiguous()


def work_table(cfg, nblocks, nsp, lim=None):
    """Per block: its w_in tiles (q / k / v tiles first, then the gate / up tiles of its MLP channels) and its
    w_down slices [sb, se) (16 channels each; a block owns both gate / up tiles of each of its slices).
    Returns int16 [nblocks, lim.work_stride]; unused entries are -1."""
    lim = lim or decode_limits()
    qkv_tiles = (cfg.NH + 2 * cfg.NKV) * cfg.HD // 16
    nsl = cfg.inter // 16
    tiles = [[] for _ in range(nblocks)]
    ranges = []
    for b in range(nblocks):
        sb, se = b * nsl // nblocks, (b + 1) * nsl // nblocks
        if se - sb > lim.max_slices:
            raise ValueError("too many MLP channels per block")
        ranges.append((sb, se))
        for k in range(sb, se):
            tiles[b] += [qkv_tiles + 2 * k, qkv_tiles + 2 * k + 1]
    qkv = [[] for _ in range(nblocks)]
    for t in range(qkv_tiles):  # each q / k / v tile to the block with the fewest tiles so far (first pass at most)
        b = min((i for i in range(nblocks) if len(qkv[i]) < lim.first_pass),
                key=lambda i: (len(tiles[i]) + len(qkv[i]), len(qkv[i]), i), default=None)
        if b is None:
            raise ValueError("too many q/k/v tiles for the blocks' first passes")
        qkv[b].append(t)
    table = torch.full((nblocks, lim.work_stride), -1, dtype=torch.int16)
    for b in range(nblocks):
        tl = qkv[b] + tiles[b]
        if len(tl) > lim.max_tiles:
            raise ValueError(f"block {b} would hold {len(tl)} tiles (at most {lim.max_tiles})")
        if tl:
            table[b, :len(tl)] = torch.tensor(tl, dtype=torch.int16)
        table[b, lim.slice_begin_col], table[b, lim.slice_end_col] = ranges[b]
    validate_work_table(table, cfg, lim)
    return table


def validate_work_table(table, cfg, lim=None):
    """Raise ValueError unless `table` is a work table the persistent kernel can run without a circular wait:
    every w_in tile listed exactly once, at most max_tiles per block with no gap before the last one, every q / k / v
    tile in its block's first pass (positions [0, first_pass): a later one is published after the block's own q
    poll, which may be waiting for it), the down slices a contiguous partition of the MLP channels with at most
    max_slices per block, and each block's gate / up tiles exactly those of its slices (the kernel keeps
    SiLU(gate) * up only for the block's own channels)."""
    lim = lim or decode_limits()
    t = torch.as_tensor(table)
    if t.dim() != 2 or t.shape[1] != lim.work_stride:
        raise ValueError(f"work table must be [nblocks, {lim.work_stride}]")
    qkv_tiles = (cfg.NH + 2 * cfg.NKV) * cfg.HD // 16
    n_tiles = qkv_tiles + 2 * cfg.inter // 16
    nsl = cfg.inter // 16
    seen = []
    prev_end = 0
    for b in range(t.shape[0]):
        row = [int(v) for v in t[b, :lim.max_tiles]]
        n = sum(v >= 0 for v in row)
        if any(v < 0 for v in row[:n]) or any(v >= 0 for v in row[n:]):
            raise ValueError(f"block {b}: tiles must fill positions 0 .. n-1")
        if any(v >= n_tiles for v in row[:n]):
            raise ValueError(f"block {b}: tile index out of range")
        if any(v < qkv_tiles for v in row[lim.first_pass:n]):
            raise ValueError(f"block {b}: a q/k/v tile outside the first {lim.first_pass} positions")
        seen += row[:n]
        sb, se = int(t[b, lim.slice_begin_col]), int(t[b, lim.slice_end_col])
        if sb != prev_end or se < sb or se - sb > lim.max_slices:
            raise ValueError(f"block {b}: down slices [{sb}, {se}) break the contiguous partition")
        prev_end = se
        own = {v for v in row[:n] if v >= qkv_tiles}
        if own != {qkv_tiles + 2 * k + h for k in range(sb, se) for h in (0, 1)}:
            raise ValueError(f"block {b}: gate/up tiles differ from those of its slices")
    if prev_end != nsl:
        raise ValueError("down slices do not cover every MLP channel")
    if sorted(seen) != list(range(n_tiles)):
        raise ValueError("every w_in tile must be listed exactly once")


class _OneLaunch:
    """What the one-launch engines share: state, cache filling, the sampling tail in the captured step, capture /
    replay and the status word. Subclasses set kc, vc, tok, pos, logits, hn, status, the exchange buffers
    (`_exchange`) and `_launch()`."""

    def reset(self):
        """Zero the exchange buffers, step counters and status (needed after a nonzero status)."""
        for t in self._exchange:
            t.zero_()

    def set_state(self, tok: int, pos: int):
        self.tok.fill_(tok)
        self.pos.fill_(pos)

    def fill_cache(self, ctx: int, seed: int = 0):
        g = torch.Generator(device=self.dev).manual_seed(seed)
        self.kc[:, :, :ctx].normal_(generator=g)
        self.vc[:, :, :ctx].normal_(generator=g)

    def attach_sampler(self, stop, audio_ids, end_id, top_k=30, min_new=8, temperature=0.8, max_new=1800):
        """Sample the next token inside the step (reference engine/rumik_fused.py:92-94, engine/sample.py): after
        the int8 head, the fused sampling tail reads `logits` and `hn`, writes out[step_i] and `tok` (the next
        step's input token) and advances step_i, so replaying the captured step generates tokens autoregressively
        on the device. `stop`: the stop predictor's state dict (0.weight, 0.bias, 1.weight, 1.bias, 3.weight,
        3.bias); `audio_ids` [n_audio] int64 maps head rows to token ids."""
        import sample
        self.H = self.cfg.H
        self.stop = {k: v.to(self.dev) for k, v in stop.items()}
        self.audio_ids = audio_ids.to(self.dev, torch.int64).contiguous()
        self.end_id, self.top_k, self.min_new, self.temperature = int(end_id), int(top_k), int(min_new), float(temperature)
        self.step_i = torch.zeros(1, dtype=torch.int64, device=self.dev)
        self.out = torch.zeros(max_new + 8, dtype=torch.int64, device=self.dev)
        self.sampler = sample.FusedSampler(self, lambda: self.logits)
        self.graph, self.frames = None, {}  # graphs captured before hold the step without the tail
        return self.sampler

    def step(self):
        self._launch()
        if self.sampler is not None:
            self.sampler()

    def _capture(self, steps):
        saved = [self.kc.clone(), self.vc.clone(), self.pos.clone(), self.tok.clone()]
        if self.sampler is not None:
            saved += [self.step_i.clone(), self.out.clone()]
        self.step()
        torch.cuda.synchronize(self.dev)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(steps):
                self.step()
        torch.cuda.synchronize(self.dev)
        self.kc.copy_(saved[0]); self.vc.copy_(saved[1]); self.pos.copy_(saved[2]); self.tok.copy_(saved[3])
        if self.sampler is not None:
            self.step_i.copy_(saved[4]); self.out.copy_(saved[5])
        torch.cuda.synchronize(self.dev)
        return g

    def capture(self):
        """One step (decode, and the sampling tail when attached) as a hipGraph; replay() runs it."""
        self.graph = self._capture(1)
        self.frames = {}
        return self.graph

    def capture_frame(self, n: int):
        """n consecutive steps as ONE hipGraph (replay_frame(n) runs them). The kernel advances pos and the
        sampling tail advances tok / step_i on the device, so one replay of it does exactly what n replays of the
        one-step graph do (same tokens for the same seed), without the per-replay launch gap between the steps
        (~9-13 us per token on MI355X against ~0 between the kernels of one graph)."""
        n = int(n)
        if n < 1:
            raise ValueError("a frame holds at least one step")
        if not hasattr(self, "frames"):
            self.frames = {}
        if n not in self.frames:
            self.frames[n] = self._capture(n)
        return self.frames[n]

    def replay(self):
        self.graph.replay()

    def replay_frame(self, n: int):
        self.frames[int(n)].replay()

    def status_word(self) -> int:
        """0 when every wait of every step so far completed in time."""
        return int(self.status.item())


class PersistentDecode(_OneLaunch):
    """The decode step as one persistent kernel launch (csrc/decode_persistent.hip). Same weights, state and
    outputs as DecodeStep; needs hidden 2048 and head dim 128 and one block per 8 rows of the hidden state
    (256 blocks, one per CU on MI355X). `weights` as from random_weights; they are re-laid out once (stacked over
    layers, gate / up interleaved, tile / slice layouts) and the per-layer copies can then be dropped."""

    def __init__(self, cfg: Config, weights, device="cuda", nsp=None, keep_layer_weights=False):
        if cfg.H != 2048 or cfg.HD != 128 or cfg.NH * cfg.HD != 2048:
            raise ValueError("the persistent step is built for hidden 2048 / head dim 128")
        self.cfg, self.dev = cfg, torch.device(device)
        d = self.dev
        self.nblocks = 2048 // 8
        self.nsp = nsp or min(64, self.nblocks // cfg.NKV)
        lib = HL.lib()
        if lib.rk_decode_params_size() != ctypes.sizeof(RkDecodeParams):
            raise RuntimeError("rk_decode_params layout mismatch between the library and decode.py")
        w, c = weights, cfg
        stack = lambda f, key: torch.stack([f(t) for t in w[key]]).contiguous()  # noqa: E731
        self.win_t = stack(lambda t: tile_layout(interleave_gate_up(t[0], c)), "w_in")
        self.win_sm = stack(lambda t: wave_scale_min(pack_scale_min(interleave_gate_up(t[1], c),
                                                                     interleave_gate_up(t[2], c))), "w_in")
        self.wo_q = stack(lambda t: o_layout(t[0], c.NH), "w_o")
        self.wo_sm = stack(lambda t: pack_scale_min(t[1], t[2]), "w_o")
        self.wd_t = stack(lambda t: down_layout(t[0]), "w_down")
        self.wd_sm = stack(lambda t: pack_scale_min(t[1], t[2]).t().contiguous(), "w_down")
        self.ln = torch.stack(w["ln"]).contiguous()
        self.norm, self.emb, self.head = w["norm"], w["emb"], w["head"]
        if not keep_layer_weights:
            for k in ("w_in", "w_o", "w_down"):
                w[k].clear()
        self.limits = decode_limits()
        if self.nsp > self.limits.max_splits or -(-c.S // self.nsp) > self.limits.max_slots_per_split:
            raise ValueError("cache length / attention splits beyond the kernel's limits")
        self.work = work_table(c, self.nblocks, self.nsp, self.limits).to(d)
        f16, f32, i32 = torch.float16, torch.float32, torch.int32
        nb = self.nblocks
        self.tx = torch.zeros(self.limits.x_copies * 2048, dtype=i32, device=d)
        self.tq = torch.zeros(c.NH * c.HD, dtype=i32, device=d)
        self.tkv = torch.zeros(2 * c.NKV * c.HD, dtype=i32, device=d)
        self.top = torch.zeros(nb * c.NH * 8, dtype=i32, device=d)
        self.tdp = torch.zeros(nb * 2048, dtype=i32, device=d)
        self.tpo = torch.zeros(c.NH * self.nsp * c.HD, dtype=i32, device=d)
        self.tml = torch.zeros(c.NH * self.nsp * 2, dtype=torch.int64, device=d)
        self.ctr = torch.zeros(nb, dtype=i32, device=d)
        self.status = torch.zeros(1, dtype=i32, device=d)
        self.logits = torch.zeros(c.n_audio, dtype=f32, device=d)
        self.hn = torch.zeros(c.H, dtype=f16, device=d)  # final LayerNorm output (the sampler's stop predictor input)
        self.kc = torch.zeros(c.L, c.NKV, c.S, c.HD, dtype=f16, device=d)
        self.vc = torch.zeros_like(self.kc)
        self.tok = torch.zeros(1, dtype=torch.int64, device=d)
        self.pos = torch.zeros(1, dtype=torch.int64, device=d)
        self.cos, self.sin = rope_tables(c.S, c.HD, c.rope_theta, f16, d)
        sliding = sum(1 << i for i, on in enumerate(c.sliding) if on)
        P = RkDecodeParams(L=c.L, NH=c.NH, NKV=c.NKV, inter=c.inter, S=c.S, n_audio=c.n_audio, nsp=self.nsp,
                           eps=c.eps, scale=c.HD ** -0.5, sliding=sliding)
        for name, t in (("tok", self.tok), ("pos", self.pos), ("emb_q", self.emb[0]), ("emb_s", self.emb[1]),
                        ("win_t", self.win_t), ("win_sm", self.win_sm), ("wo_q", self.wo_q), ("wo_sm", self.wo_sm),
                        ("wd_t", self.wd_t), ("wd_sm", self.wd_sm), ("ln_w", self.ln), ("norm_w", self.norm),
                        ("cos_t", self.cos), ("sin_t", self.sin), ("kc", self.kc), ("vc", self.vc),
                        ("head_q", self.head[0]), ("head_s", self.head[1]), ("logits", self.logits),
                        ("work", self.work), ("tx", self.tx), ("tq", self.tq), ("tkv", self.tkv), ("top", self.top),
                        ("tdp", self.tdp), ("tpo", self.tpo), ("tml", self.tml), ("ctr", self.ctr),
                        ("status", self.status), ("hn", self.hn)):
            if not t.is_contiguous() or t.device != d:
                raise RuntimeError(f"{name} must be a contiguous tensor on {d}")
            setattr(P, name, t.data_ptr())
        self.params = P
        self.graph = None
        self.sampler = None

    @property
    def x(self):
        """the residual stream after the last layer of the last step (fp16, decoded from the tagged words)"""
        return self.tx[:2048].view(torch.float16)[0::2]

    @property
    def _exchange(self):
        return (self.tx, self.tq, self.tkv, self.top, self.tdp, self.tpo, self.tml, self.ctr, self.status)

    def _launch(self):
        HL.check(HL.lib().rk_decode_step_persistent(ctypes.byref(self.params), self.nblocks, HL.stream(self.dev)),
                 "decode_step_persistent")


# ---------------------------------------------------------------------------------------------- role-split step
class RkDecodeRolesParams(ctypes.Structure):
    """ctypes mirror of rk_decode_roles_params (include/rumik_hip.h); its size is checked against the library."""
    _fields_ = [(n, ctypes.c_int) for n in ("L", "NH", "NKV", "inter", "S", "n_audio", "nsp", "min_chunk")] + [
        ("eps", ctypes.c_float), ("scale", ctypes.c_float), ("sliding", ctypes.c_ulonglong)] + [
        (n, ctypes.c_void_p) for n in (
            "tok", "pos", "emb_q", "emb_s", "win_t", "win_sm", "wo_q", "wo_sm", "wd_t", "wd_sm", "ln_w", "norm_w",
            "cos_t", "sin_t", "kc", "vc", "head_q", "head_s", "logits", "role", "tx", "tq", "tkv", "tpo", "tml",
            "top", "tdp", "ctr", "status", "hn")] + [("local_xcd", ctypes.c_int), ("stream_qkv_from", ctypes.c_longlong)]


class RkDecodeRolesLimits(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("blocks", "latency_blocks", "max_slices", "x_copies", "max_splits",
                                            "slots_per_wave", "waves")]


def roles_limits() -> RkDecodeRolesLimits:
    """The role-split kernel's compiled limits (a host-only query: no GPU needed)."""
    lim = RkDecodeRolesLimits()
    HL.check(HL.lib().rk_decode_roles_get_limits(ctypes.byref(lim)), "decode_roles_get_limits")
    return lim


def group_scale_min(sm):
    """per-(row, group) scale | min words [n_in, 16] -> per (tile, group, row): int32 [n_in / 16, 16, 16]."""
    return sm.reshape(sm.shape[0] // 16, 16, -1).permute(0, 2, 1).contiguous()


def latency_xcd(cfg):
    """b % 8 of latency group g's blocks (its 64 / NKV blocks, those of KV head g): 2g for 4 groups, g for 8."""
    return [g * (8 // cfg.NKV) for g in range(cfg.NKV)]


def role_table(cfg, lim=None):
    """Block -> role for the role-split step: int16 [blocks, 4] = (kind, index, slice begin, slice end).
    A launch deals block b to XCD (b + c) % 8 (the dispatcher's round robin, confirmed by placement_ok), so the
    blocks with equal b % 8 share an XCD.
    Latency blocks (kind 0): group g (indices j = g * 64 / NKV .. + 64 / NKV - 1: KV head g's attention splits,
    combines and q / k / v tiles, which exchange words only inside the group) on one XCD, latency_xcd(cfg)[g],
    taking that XCD's lowest blocks. Stream blocks (kind 1): the others, numbered XCD by XCD, so stream blocks with
    neighbouring MLP slices, which share w_down scale rows, sit on one XCD and its L2; stream block i takes slices
    [i * n / 192, (i + 1) * n / 192) of the n = inter / 16."""
    lim = lim or roles_limits()
    nb, nl = lim.blocks, lim.latency_blocks
    ns = nb - nl
    nsl = cfg.inter // 16
    if -(-nsl // ns) > lim.max_slices:
        raise ValueError("too many MLP slices per stream block")
    if nl % cfg.NKV or nb % 8 or nl // cfg.NKV > nb // 8:
        raise ValueError("latency groups do not fit the XCDs")
    table = torch.zeros(nb, 4, dtype=torch.int16)
    per = nl // cfg.NKV
    lat = [x + 8 * k for x in latency_xcd(cfg) for k in range(per)]
    for j, b in enumerate(lat):
        table[b] = torch.tensor([0, j, 0, 0], dtype=torch.int16)
    taken = set(lat)
    stream = sorted((b for b in range(nb) if b not in taken), key=lambda b: (b % 8, b))
    for i, b in enumerate(stream):
        table[b] = torch.tensor([1, i, i * nsl // ns, (i + 1) * nsl // ns], dtype=torch.int16)
    return table


def placement_ok(device) -> bool:
    """Are a launch's blocks dealt to the XCDs round robin on this device (block b on XCD (b + c) % 8, so blocks
    with equal b % 8 share an XCD: the placement the latency groups' L2-local exchanges rely on)? One tiny launch,
    synchronized."""
    d = torch.device(device)
    xcc = torch.full((roles_limits().blocks,), -1, dtype=torch.int32, device=d)
    HL.check(HL.lib().rk_decode_roles_placement(xcc.data_ptr(), HL.stream(d)), "decode_roles_placement")
    got = xcc.cpu()
    if (got < 0).any() or (got >= 8).any():
        return False
    return bool(((got - torch.arange(got.numel(), dtype=torch.int32)) % 8 == (got[0] % 8)).all())


class RoleDecode(_OneLaunch):
    """The decode step as one persistent launch with the grid split by role (csrc/decode_roles.hip): 64 latency
    blocks run the step's chain (attention, combine, o, the residual rows; at short contexts also x, LayerNorm and
    q/k/v), 192 stream blocks the MLP (gate / up, SiLU, down), the int8 head and, at long contexts, q/k/v. Same weights, state and outputs as DecodeStep and
    PersistentDecode; hidden 2048, head dim 128, 16 query heads with 4 or 8 KV heads, 256 CUs.
    nsp: attention splits per KV head (default min(16, 64 / NKV)); min_chunk: the fewest cache slots per split.
    stream_qkv_from: steps at pos >= this compute q/k/v on the stream blocks (the latency blocks then skip x, the
    LayerNorm and the q/k/v tiles), earlier ones on the latency blocks; both give the same results, and the default
    switches where the second became faster in the step's timing (0: always the stream blocks)."""

    STREAM_QKV_FROM = 384

    def __init__(self, cfg: Config, weights, device="cuda", nsp=None, min_chunk=32, keep_layer_weights=False,
                 local_xcd=None, stream_qkv_from=None):
        if cfg.H != 2048 or cfg.HD != 128 or cfg.NH * cfg.HD != 2048 or cfg.NKV not in (4, 8):
            raise ValueError("the role-split step is built for hidden 2048 / head dim 128 / 16 q and 4 or 8 kv heads")
        self.cfg, self.dev = cfg, torch.device(device)
        d = self.dev
        lib = HL.lib()
        if lib.rk_decode_roles_params_size() != ctypes.sizeof(RkDecodeRolesParams):
            raise RuntimeError("rk_decode_roles_params layout mismatch between the library and decode.py")
        self.limits = roles_limits()
        nl, ns = self.limits.latency_blocks, self.limits.blocks - self.limits.latency_blocks
        self.nblocks = self.limits.blocks
        self.nsp = nsp or min(self.limits.max_splits, nl // cfg.NKV)
        if self.nsp > min(self.limits.max_splits, nl // cfg.NKV) or -(-cfg.S // self.nsp) > \
                self.limits.waves * self.limits.slots_per_wave:
            raise ValueError("cache length / attention splits beyond the kernel's limits")
        w, c = weights, cfg
        stack = lambda f, key: torch.stack([f(t) for t in w[key]]).contiguous()  # noqa: E731
        self.win_t = stack(lambda t: tile_layout(interleave_gate_up(t[0], c)), "w_in")
        self.win_sm = stack(lambda t: group_scale_min(pack_scale_min(interleave_gate_up(t[1], c),
                                                                     interleave_gate_up(t[2], c))), "w_in")
        self.wo_q = stack(lambda t: o_layout(t[0], c.NH), "w_o")
        self.wo_sm = stack(lambda t: pack_scale_min(t[1], t[2]).t().contiguous(), "w_o")
        self.wd_t = stack(lambda t: down_layout(t[0]), "w_down")
        self.wd_sm = stack(lambda t: pack_scale_min(t[1], t[2]).t().contiguous(), "w_down")
        self.ln = torch.stack(w["ln"]).contiguous()
        self.norm, self.emb, self.head = w["norm"], w["emb"], w["head"]
        if not keep_layer_weights:
            for k in ("w_in", "w_o", "w_down"):
                w[k].clear()
        self.role = role_table(c, self.limits).to(d)
        i32 = torch.int32
        xr = self.limits.x_copies
        self.tx = torch.zeros(2, xr, 2048, dtype=i32, device=d)
        self.tq = torch.zeros(2, c.NH * c.HD, dtype=i32, device=d)
        self.tkv = torch.zeros(2, 2, c.NKV * c.HD, dtype=i32, device=d)
        self.tpo = torch.zeros(2, c.NH, self.nsp, c.HD, dtype=i32, device=d)
        self.tml = torch.zeros(2, c.NH, self.nsp, 2, dtype=torch.int64, device=d)
        self.top = torch.zeros(2, nl, c.NH, 32, dtype=i32, device=d)
        self.tdp = torch.zeros(2, nl, ns, 32, dtype=i32, device=d)
        self.ctr = torch.zeros(self.nblocks, dtype=i32, device=d)
        self.status = torch.zeros(1, dtype=i32, device=d)
        self.logits = torch.zeros(c.n_audio, dtype=torch.float32, device=d)
        self.hn = torch.zeros(c.H, dtype=torch.float16, device=d)
        self.kc = torch.zeros(c.L, c.NKV, c.S, c.HD, dtype=torch.float16, device=d)
        self.vc = torch.zeros_like(self.kc)
        self.tok = torch.zeros(1, dtype=torch.int64, device=d)
        self.pos = torch.zeros(1, dtype=torch.int64, device=d)
        self.cos, self.sin = rope_tables(c.S, c.HD, c.rope_theta, torch.float16, d)
        sliding = sum(1 << i for i, on in enumerate(c.sliding) if on)
        if local_xcd is None:
            local_xcd = placement_ok(d)
        self.local_xcd = bool(local_xcd)
        P = RkDecodeRolesParams(L=c.L, NH=c.NH, NKV=c.NKV, inter=c.inter, S=c.S, n_audio=c.n_audio, nsp=self.nsp,
                                min_chunk=int(min_chunk), eps=c.eps, scale=c.HD ** -0.5, sliding=sliding,
                                local_xcd=int(self.local_xcd),
                                stream_qkv_from=int(self.STREAM_QKV_FROM if stream_qkv_from is None
                                                    else stream_qkv_from))
        for name, t in (("tok", self.tok), ("pos", self.pos), ("emb_q", self.emb[0]), ("emb_s", self.emb[1]),
                        ("win_t", self.win_t), ("win_sm", self.win_sm), ("wo_q", self.wo_q), ("wo_sm", self.wo_sm),
                        ("wd_t", self.wd_t), ("wd_sm", self.wd_sm), ("ln_w", self.ln), ("norm_w", self.norm),
                        ("cos_t", self.cos), ("sin_t", self.sin), ("kc", self.kc), ("vc", self.vc),
                        ("head_q", self.head[0]), ("head_s", self.head[1]), ("logits", self.logits),
                        ("role", self.role), ("tx", self.tx), ("tq", self.tq), ("tkv", self.tkv), ("tpo", self.tpo),
                        ("tml", self.tml), ("top", self.top), ("tdp", self.tdp), ("ctr", self.ctr),
                        ("status", self.status), ("hn", self.hn)):
            if not t.is_contiguous() or t.device != d:
                raise RuntimeError(f"{name} must be a contiguous tensor on {d}")
            setattr(P, name, t.data_ptr())
        self.params = P
        self.graph = None
        self.sampler = None

    @property
    def x(self):
        """the residual stream after the last layer of the last step (fp16, decoded from the tagged words)"""
        return self.tx[self.cfg.L & 1, 0].view(torch.float16)[0::2]

    @property
    def _exchange(self):
        return (self.tx, self.tq, self.tkv, self.tpo, self.tml, self.top, self.tdp, self.ctr, self.status)

    def _launch(self):
        HL.check(HL.lib().rk_decode_step_roles(ctypes.byref(self.params), HL.stream(self.dev)), "decode_step_roles")
