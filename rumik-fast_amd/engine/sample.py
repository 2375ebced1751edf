"""The tail of a decode step on MI355X: stop predictor + top-k + Gumbel-max sampling + token counters.

Drop-in for the reference's engine/sample.py (imported by engine/rumik_fused.py:12,38 as `FusedSampler`): the same
module constants (CH, KEEP), the same three kernels with the same argument order and `kernel[grid](...)` launch
form (the grid and the Triton tuning keywords ROWS / num_warps are accepted and ignored: each HIP wrapper picks its
own launch shape), the same buffers (`keys`: every 512-logit chunk's packed keys sorted descending; `scratch[:32]`:
the global top 32 in order, so `scratch[:top_k]` is the top-k -- what the reference's pick and its sampler check
read of the candidate list; its other slots are not written; `z1`: the stop predictor's hidden layer), and
`FusedSampler(eng, logits_fn)()`, which samples the next token from `eng.hn` and
updates `eng.out[step]`, `eng.tok` and `eng.step_i` in place. FusedSampler runs the whole tail as ONE launch
(rk_sample_tail) instead of three; the uniforms come from torch.rand on the device, as in the reference
(sample.py:113), so the call stays capturable.

Maths (reference engine/rumik_int4.py:174-191, engine/sample.py:1-11):
  stop   = sigmoid(w2 . gelu(W1 . LayerNorm(h) + b1) + b2) > 0.5, applied from step min_new on
  logits = the audio head's output with </audio> masked to -inf for the first min_new steps
  token  = ids[argmax over the top-k logits of (logit / T + Gumbel(u))]
There is no CPU path: every call goes to librumik_hip.so and raises if it is missing or the tensors are not on a GPU.
"""
import ctypes
import functools
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "kernels"))
import _hiplib as HL  # noqa: E402

CH = 512          # logits per stage-1 chunk
KEEP = 32         # survivors per chunk (>= top_k)
MAX_NC = 4096     # candidate slots of the pick (128 chunks)


class _Kernel:
    """`kernel[grid](...)` as in the reference's Triton launches, or a plain call."""

    def __init__(self, fn):
        self._fn = fn
        functools.update_wrapper(self, fn)

    def __getitem__(self, grid):
        return self._fn

    def __call__(self, *args, **kwargs):
        return self._fn(*args, **kwargs)


def _f32(*ts):
    for t in ts:
        if t.dtype != torch.float32:
            raise RuntimeError("the stop predictor's LayerNorm weight / bias, b1, w2, b2 and the uniforms are fp32 "
                               "(the reference converts them with .float())")


def _i64(*ts):
    for t in ts:
        if t.dtype != torch.int64:
            raise RuntimeError("ids, step, pos, tok, out, keys and scratch are int64")


def next_power_of_2(n: int) -> int:
    return 1 << max(0, (int(n) - 1).bit_length())


@_Kernel
def stop_hidden(h_ptr, lnw_ptr, lnb_ptr, w1_ptr, b1_ptr, z1_ptr, eps, H=None, ROWS=None, num_warps=None):
    """z1 = gelu(W1 . LayerNorm(h; lnw, lnb, eps) + b1), exact GELU (reference sample.py:34-49). W1 [nz, H]."""
    HL.require_gpu(h_ptr, lnw_ptr, lnb_ptr, w1_ptr, b1_ptr, z1_ptr)
    _f32(lnw_ptr, lnb_ptr, b1_ptr, z1_ptr)
    nz, Hs = w1_ptr.shape
    if H is not None and H != Hs:
        raise AssertionError(f"H={H} does not match W1's {Hs} columns")
    HL.check(HL.lib().rk_stop_hidden(HL.ptr(h_ptr), HL.dt(h_ptr), HL.ptr(lnw_ptr), HL.ptr(lnb_ptr), HL.ptr(w1_ptr),
                                     HL.dt(w1_ptr), HL.ptr(b1_ptr), HL.ptr(z1_ptr), float(eps), Hs, nz,
                                     HL.stream(h_ptr.device)), "stop_hidden")


@_Kernel
def topk_partial(logits_ptr, step_ptr, keys_ptr, NV, END_IDX, MIN_NEW, CH=CH, num_warps=None):
    """keys[c*512 : (c+1)*512] = chunk c's packed keys sorted descending; </audio> masked while step < MIN_NEW
    (reference sample.py:53-61)."""
    if CH != globals()["CH"]:
        raise AssertionError(f"chunks are {globals()['CH']} logits")
    HL.require_gpu(logits_ptr, step_ptr, keys_ptr)
    _i64(step_ptr, keys_ptr)
    if keys_ptr.numel() < -(-int(NV) // CH) * CH:
        raise RuntimeError("shape")
    HL.check(HL.lib().rk_topk_partial(HL.ptr(logits_ptr), HL.dt(logits_ptr), HL.ptr(step_ptr), HL.ptr(keys_ptr),
                                      int(NV), int(END_IDX), int(MIN_NEW), HL.stream(logits_ptr.device)),
             "topk_partial")


@_Kernel
def pick(keys_ptr, scratch_ptr, u_ptr, z1_ptr, w2_ptr, b2_ptr, ids_ptr, step_ptr, pos_ptr, tok_ptr, out_ptr,
         inv_temp, END_ID, MIN_NEW, NCH, CH=CH, KEEP=KEEP, NC=None, TOPK=30, NZ=None, num_warps=None):
    """Merge the chunks' top KEEP, sample from the top TOPK with Gumbel-max, apply the stop rule, write
    out[step] and tok, step += 1 (reference sample.py:65-93). pos is accepted and unused, as in the reference."""
    if CH != globals()["CH"] or KEEP != globals()["KEEP"]:
        raise AssertionError("chunks are 512 logits with 32 survivors each")
    HL.require_gpu(keys_ptr, scratch_ptr, u_ptr, z1_ptr, w2_ptr, b2_ptr, ids_ptr, step_ptr, tok_ptr, out_ptr)
    _f32(u_ptr, z1_ptr, w2_ptr, b2_ptr)
    _i64(keys_ptr, scratch_ptr, ids_ptr, step_ptr, tok_ptr, out_ptr)
    nc = NC if NC is not None else next_power_of_2(NCH * KEEP)
    nz = NZ if NZ is not None else z1_ptr.numel()
    if scratch_ptr.numel() < nc:
        raise RuntimeError("shape")
    HL.check(HL.lib().rk_pick(HL.ptr(keys_ptr), HL.ptr(scratch_ptr), HL.ptr(u_ptr), HL.ptr(z1_ptr), HL.ptr(w2_ptr),
                              HL.ptr(b2_ptr), HL.ptr(ids_ptr), HL.ptr(step_ptr), HL.ptr(tok_ptr), HL.ptr(out_ptr),
                              float(inv_temp), int(END_ID), int(MIN_NEW), int(NCH), int(nc), int(TOPK), int(nz),
                              HL.stream(keys_ptr.device)), "pick")


class FusedSampler:
    """Holds the buffers; `__call__` samples the next token from eng.hn and updates eng.out / tok / step_i in place
    (reference engine/sample.py:96-127). `eng` provides dev, H, hn, stop (the stop predictor's state dict: 0.weight,
    0.bias, 1.weight, 1.bias, 3.weight, 3.bias), audio_ids, end_id, top_k, min_new, temperature, step_i, pos, tok,
    out; `logits_fn()` returns the audio logits ([>= nv], fp32 / bf16 / fp16)."""

    def __init__(self, eng, logits_fn):
        d = eng.dev
        self.eng, self.logits_fn = eng, logits_fn
        st = eng.stop
        self.lnw, self.lnb = st["0.weight"].float().contiguous(), st["0.bias"].float().contiguous()
        self.w1, self.b1 = st["1.weight"].contiguous(), st["1.bias"].float().contiguous()     # bf16 W1 (exact)
        self.w2, self.b2 = st["3.weight"].reshape(-1).float().contiguous(), st["3.bias"].float().contiguous()
        self.nz = self.w1.shape[0]
        self.nv = eng.audio_ids.numel()
        ends = (eng.audio_ids == eng.end_id).nonzero().flatten().tolist()
        assert len(ends) == 1
        self.end_idx = ends[0]
        self.nch = -(-self.nv // CH)
        self.nc = next_power_of_2(self.nch * KEEP)
        if self.nc > MAX_NC:
            raise RuntimeError("shape")
        self.keys = torch.empty(self.nch * CH, dtype=torch.int64, device=d)
        self.scratch = torch.empty(self.nc, dtype=torch.int64, device=d)
        self.z1 = torch.empty(self.nz, dtype=torch.float32, device=d)
        self.u = torch.empty(32, dtype=torch.float32, device=d)
        self.counter = torch.zeros(1, dtype=torch.int32, device=d)  # rk_sample_tail's completion count (self-reset)
        assert eng.top_k <= 32

    def __call__(self):
        e = self.eng
        logits = self.logits_fn()
        torch.rand(32, device=e.dev, out=self.u)                         # graph-safe RNG (Philox offsets)
        HL.require_gpu(e.hn, logits, e.step_i, e.tok, e.out)
        _i64(e.step_i, e.tok, e.out, e.audio_ids)
        HL.check(HL.lib().rk_sample_tail(
            HL.ptr(e.hn), HL.dt(e.hn), HL.ptr(self.lnw), HL.ptr(self.lnb), HL.ptr(self.w1), HL.dt(self.w1),
            HL.ptr(self.b1), HL.ptr(self.w2), HL.ptr(self.b2), 1e-5, int(e.H), self.nz, HL.ptr(logits), HL.dt(logits),
            self.nv, self.end_idx, HL.ptr(self.u), HL.ptr(e.audio_ids), HL.ptr(e.step_i), HL.ptr(e.tok),
            HL.ptr(e.out), 1.0 / e.temperature, int(e.end_id), int(e.min_new), int(e.top_k), HL.ptr(self.keys),
            HL.ptr(self.scratch), self.nc, HL.ptr(self.z1), HL.ptr(self.counter), HL.stream(e.dev)), "sample_tail")
