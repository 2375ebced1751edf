"""The host side of generation on MI355X: prompt, then captured decode steps read back a frame at a time.

Mirrors RumikInt4.generate / to_codes (reference engine/rumik_int4.py:251-324) over a one-launch decode engine
(RoleDecode or PersistentDecode) with the sampling tail attached (one hipGraph = decode step + sample; the sampled
token is the next replay's input):
- frames of Q tokens (Q = num_quantizers, one Mimi frame): one replay of a graph holding Q consecutive steps (no
  launch gap between them; the same tokens as Q one-step replays), then an asynchronous copy of the frame's tokens to
  pinned host memory and an event; the next frame is queued before waiting for the current one (double
  buffering: the GPU never idles while the host handles a frame), and waiting on the event waits only for the work
  before it;
- generation stops at </audio> (tokens after it in the same frame are dropped, a frame queued after it is ignored),
  at max_new tokens or when the cache is full;
- the one-launch step's status word is copied back with every frame (same event): a nonzero status (a wait that
  timed out, so the step drained with garbage, a position outside the cache, or a residual sum beyond the fp16
  range) raises DecodeError after the engine's exchange buffers are reset, instead of emitting tokens sampled from
  invalid logits;
- to_codes: audio token ids -> [1, Q, frames] Mimi codes, whole frames only, resynchronising on a broken codebook
  round robin (rumik_int4.py:310-324).
The prompt: with a prefill.Prefill (all prompt rows of a layer at once: mm_int4 and the matrix-core causal
attention), then the audio head and the sampling tail; without one, prefill() runs the one-launch decode step once
per prompt token (teacher forcing: each replay's input is the prompt's next token, its sampled token is discarded
except after the last prompt token, which is the first generated token).
"""
import time

import torch


class DecodeError(RuntimeError):
    """The one-launch decode step reported a nonzero status (see _OneLaunch.status_word in decode.py)."""


class Generator:
    """`eng`: a one-launch decode engine (decode.RoleDecode, the fastest, or decode.PersistentDecode) with
    attach_sampler() done. first_unit_id / last_unit_id bound the audio
    token ids (config.json first_unit_id / last_unit_id); Q = num_quantizers."""

    def __init__(self, eng, Q=8, first_unit_id=None, last_unit_id=None, max_new=None, prefill=None):
        if eng.sampler is None:
            raise RuntimeError("attach_sampler() first: the captured step must sample its next token")
        self.eng, self.Q, self.pf = eng, int(Q), prefill
        self.first, self.last = first_unit_id, last_unit_id
        self.max_new = int(max_new) if max_new is not None else eng.out.shape[0] - 8
        if self.max_new + self.Q > eng.out.shape[0]:
            raise ValueError("max_new + Q exceeds the sampler's output buffer")
        self.max_seq = eng.cfg.S
        self.host = torch.empty(eng.out.shape[0], dtype=torch.long, pin_memory=True)
        self.host_status = torch.zeros(eng.out.shape[0], dtype=torch.int32, pin_memory=True)
        if eng.graph is None:
            eng.capture()
        eng.capture_frame(self.Q)  # a frame's Q steps as one graph: no launch gap between its tokens

    def _fail(self, status, where):
        self.eng.reset()
        raise DecodeError(f"decode step status {status} ({where}): bit 1 = a cross-block wait timed out, bit 2 = "
                          "position outside the cache, bit 3 = a residual sum left the fp16 range; the engine's "
                          "exchange buffers were reset")

    @torch.inference_mode()
    def prefill(self, ids):
        """Process the prompt; returns the first generated token (a device scalar, also in eng.tok / eng.out[0]).
        With a prefill.Prefill: all prompt rows per layer at once on the matrix cores, then the audio head and the
        sampling tail on hn (rumik_fused.py:54-78); otherwise the decode step once per prompt token."""
        e = self.eng
        T = len(ids)
        if T < 1 or T + 1 >= self.max_seq:
            raise ValueError(f"prompt of {T} tokens for a {self.max_seq}-slot cache")
        if self.pf is not None:
            import cuda_gemv
            self.pf.run(ids, hn=e.hn)
            e.pos.fill_(T)
            cuda_gemv.gemv_int8_cuda(e.hn, *e.head, out=e.logits)
            e.step_i.zero_()
            e.sampler()  # out[0] = the first token, tok = it, step_i = 1
            return e.tok[0]
        ids_t = torch.tensor(list(ids), dtype=torch.long).to(e.dev)
        e.pos.fill_(0)
        for i in range(T):
            e.tok.copy_(ids_t[i:i + 1])
            e.step_i.zero_()  # every prompt replay samples into out[0]; the last one's is generated token 0
            e.replay()
        return e.tok[0]

    @torch.inference_mode()
    def generate(self, ids, seed=0, on_frame=None):
        """(tokens, stats) as the reference's generate: the first token from the prompt, then frames of Q."""
        e = self.eng
        torch.manual_seed(seed)
        torch.cuda.synchronize(e.dev)
        t0 = time.perf_counter()
        first = int(self.prefill(ids))
        torch.cuda.synchronize(e.dev)
        if e.status_word() != 0:
            self._fail(e.status_word(), "prompt")
        t_prefill = time.perf_counter() - t0
        pos, n, toks, t_frame0 = len(ids), 1, [first], None
        done = first == e.end_id
        host, queued = self.host, []

        def launch():
            nonlocal pos, n
            e.replay_frame(self.Q)
            pos += self.Q
            host[n:n + self.Q].copy_(e.out[n:n + self.Q], non_blocking=True)
            self.host_status[n:n + 1].copy_(e.status, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record()
            queued.append((n, ev))
            n += self.Q

        def can_launch():
            return n < self.max_new and pos + self.Q < self.max_seq

        if not done and can_launch():
            launch()
        while queued:
            if not done and can_launch():
                launch()                                         # keep one frame ahead
            k, ev = queued.pop(0)
            ev.synchronize()
            if int(self.host_status[k]) != 0:
                queued.clear()
                torch.cuda.synchronize(e.dev)
                self._fail(int(self.host_status[k]), f"frame at token {k}")
            new = host[k:k + self.Q].tolist()
            if t_frame0 is None:
                t_frame0 = time.perf_counter() - t0
            if e.end_id in new:
                new = new[:new.index(e.end_id)]
                done = True
            toks += new
            if on_frame:
                on_frame(toks)
            if done:
                queued.clear()                                   # the frame after </audio> is ignored
        torch.cuda.synchronize(e.dev)
        total = time.perf_counter() - t0
        n_dec = max(len(toks) - 1, 1)
        return toks, {"prompt_tokens": len(ids), "tokens": len(toks), "prefill_ms": round(t_prefill * 1e3, 1),
                      "first_frame_ms": round((t_frame0 or total) * 1e3, 1),
                      "decode_tok_s": round(n_dec / max(total - t_prefill, 1e-9), 1),
                      "audio_s": round(len(toks) / 100, 2), "total_s": round(total, 2)}

    def to_codes(self, toks):
        return to_codes(toks, self.first, self.last, self.Q)


def to_codes(toks, first, last, Q=8):
    """audio token ids -> [1, Q, frames] Mimi codes: token t in [first, last] is code (t - first) // Q of codebook
    (t - first) % Q; a frame is Q tokens with codebooks 0..Q-1 in order; a token out of order restarts the frame
    (at itself when it is codebook 0), a non-audio token drops the partial frame."""
    frames, fr = [], []
    for t in toks:
        if not first <= t <= last:
            fr = []
            continue
        code, q = divmod(t - first, Q)
        if q == len(fr):
            fr.append(code)
            if len(fr) == Q:
                frames.append(fr)
                fr = []
        else:
            fr = [code] if q == 0 else []
    return torch.tensor(frames, dtype=torch.long).reshape(-1, Q).T.unsqueeze(0)
