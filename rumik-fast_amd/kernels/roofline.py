"""Read-only ceiling of an int4 weight stream (the counterpart of the reference's kernels/roofline.py, which times a
`read_only` kernel doing the int4 GEMV's loads with almost no maths, and a dense bf16 GEMV, against the real kernel).

read_only(q, s, m, ...) runs rk_read_only_ex over the matrix's three buffers (the bytes one int4 GEMV launch reads
from HBM) as one range in a single grid-stride pass and returns the per-block sink; sink_total() is the wrapping sum
of every 32-bit word of the buffers, which word_sum() computes on the host for the check. ceiling_us() sweeps the
launch shape (threads per block, blocks, loads in flight per thread) over rotated copies (so no launch is served
from the Infinity Cache) and returns the best time per launch; ceiling_at() does that for a given byte count.
"""
import math

import numpy as np
import torch

import _hiplib as H

THREADS = (256, 512, 1024)
BLOCKS = (256, 512, 1024, 2048)   # one to eight blocks per CU
UNROLLS = (1, 2, 4, 8)


def read_only(q, s, m, blocks=1024, unroll=4, sink=None, threads=256):
    """One read of q, s, m (any contiguous device tensors whose sizes are multiples of 16 bytes)."""
    for t in (q, s, m):
        assert t.is_cuda and t.is_contiguous(), "device tensors, contiguous"
    if sink is None:
        sink = torch.empty(blocks, dtype=torch.int32, device=q.device)
    assert sink.numel() >= blocks and sink.dtype == torch.int32
    H.check(H.lib().rk_read_only_ex(H.ptr(q), q.numel() * q.element_size(), H.ptr(s), s.numel() * s.element_size(),
                                    H.ptr(m), m.numel() * m.element_size(), threads, blocks, unroll, H.ptr(sink),
                                    H.stream(q.device)), "read_only")
    return sink


def sink_total(sink, blocks):
    return int(sink[:blocks].cpu().numpy().view(np.uint32).astype(np.uint64).sum() % (1 << 32))


def word_sum(*tensors):
    """wrapping sum of the 32-bit words of the tensors' bytes (host)"""
    tot = 0
    for t in tensors:
        w = t.detach().cpu().contiguous().view(torch.uint8).numpy().view(np.uint32)
        tot += int(w.astype(np.uint64).sum())
    return tot % (1 << 32)


def shapes():
    """every (threads, blocks, unroll) of the sweep"""
    return [(t, b, u) for t in THREADS for b in BLOCKS for u in UNROLLS]


def _time_shape(mats, shape, sink, reps, trials):
    threads, blocks, unroll = shape
    fns = [lambda w=w: read_only(*w, blocks=blocks, unroll=unroll, sink=sink, threads=threads) for w in mats]
    for f in fns:
        f()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for f in fns:
            f()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    best = math.inf
    for _ in range(trials):
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        e1.synchronize()
        best = min(best, e0.elapsed_time(e1) * 1e3 / reps / len(mats))
    del g
    return best


def ceiling_us(mats, reps=10, trials=3, candidates=None):
    """best time per launch (us) of read_only over the rotated copies `mats` [(q, s, m), ...], over the launch shapes
    (`candidates`, default every shape of the sweep), each timed as hipGraph replays of back-to-back launches (HIP
    events on the replay stream). Returns (us, {"threads", "blocks", "unroll"}, [(us, shape) sorted])."""
    dev = mats[0][0].device
    sink = torch.empty(max(BLOCKS), dtype=torch.int32, device=dev)
    res = sorted((_time_shape(mats, sh, sink, reps, trials), sh) for sh in (candidates or shapes()))
    us, (t, b, u) = res[0]
    return us, {"threads": t, "blocks": b, "unroll": u}, res


def ceiling_at(nbytes, device, copies=16, reps=10, trials=3, candidates=None):
    """the read ceiling of one launch reading `nbytes` (rounded up to 16): one contiguous buffer per copy, `copies`
    rotated copies (past the 256 MB Infinity Cache for the sizes of these projections)."""
    n = -(-int(nbytes) // 16) * 16
    empty = torch.empty(0, dtype=torch.uint8, device=device)
    mats = [(torch.empty(n, dtype=torch.uint8, device=device), empty, empty) for _ in range(copies)]
    try:
        return ceiling_us(mats, reps, trials, candidates)
    finally:
        del mats
