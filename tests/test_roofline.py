"""The read-only ceiling kernel (rk_read_only / rk_read_only_ex, counterpart of the reference's
kernels/roofline.py:20-33): it must read every byte it is given, exactly once: the sink's total equals the wrapping
sum of every 32-bit word of the three buffers (one range, one grid-stride pass), for every launch shape the ceiling
sweep uses (GPU). Argument checks run before any device work (CPU)."""
import ctypes

import numpy as np
import pytest
import torch

import _hiplib as H
import roofline
import synth


def _addr(a):
    return ctypes.c_void_p(a.ctypes.data)


def test_read_only_validates_before_any_device_work():
    L = H.lib()
    buf = np.zeros(64, np.uint8)
    base = buf.ctypes.data + (-buf.ctypes.data) % 16
    al, mis = ctypes.c_void_p(base), ctypes.c_void_p(base + 4)
    sink = _addr(np.zeros(8, np.uint32))
    assert L.rk_read_only(al, 16, al, 16, al, 16, 8, 4, None, None) == H.ERR_NULL
    assert L.rk_read_only(None, 16, al, 16, al, 16, 8, 4, sink, None) == H.ERR_NULL
    assert L.rk_read_only(al, 24, al, 16, al, 16, 8, 4, sink, None) == H.ERR_SHAPE
    assert L.rk_read_only(mis, 16, al, 16, al, 16, 8, 4, sink, None) == H.ERR_ALIGN
    assert L.rk_read_only(al, 16, al, 16, al, 16, 0, 4, sink, None) == H.ERR_BLOCK
    assert L.rk_read_only(al, 16, al, 16, al, 16, 8, 3, sink, None) == H.ERR_BLOCK
    assert L.rk_read_only_ex(al, 16, al, 16, al, 16, 128, 8, 4, sink, None) == H.ERR_BLOCK
    assert L.rk_read_only_ex(al, 16, al, 16, al, 16, 2048, 8, 4, sink, None) == H.ERR_BLOCK
    assert L.rk_read_only_ex(al, 24, al, 16, al, 16, 512, 8, 4, sink, None) == H.ERR_SHAPE


@pytest.mark.gpu
@pytest.mark.parametrize("N,K", [(256, 2048), (2048, 11008), (25088, 2048)])
def test_read_only_reads_every_word_once(N, K, dev):
    q, s, m = synth.int4_weights(N, K, synth.generator(N + K, "cuda"), device=dev)
    ref = roofline.word_sum(q, s, m)
    for threads, blocks, unroll in roofline.shapes():
        sink = roofline.read_only(q, s, m, blocks=blocks, unroll=unroll, threads=threads)
        torch.cuda.synchronize()
        assert roofline.sink_total(sink, blocks) == ref, (threads, blocks, unroll)


@pytest.mark.gpu
def test_read_only_ragged_sizes(dev):
    # buffers of different, non-power-of-two sizes (multiples of 16 bytes), including an empty one
    g = torch.Generator(device="cpu").manual_seed(3)
    a = torch.randint(0, 256, (16 * 12345,), dtype=torch.uint8, generator=g).to(dev)
    b = torch.randint(0, 256, (16 * 7,), dtype=torch.uint8, generator=g).to(dev)
    c = torch.empty(0, dtype=torch.uint8, device=dev)
    for threads, blocks, unroll in ((256, 1, 1), (256, 3, 8), (256, 1000, 2), (512, 7, 4), (1024, 1, 8),
                                    (1024, 300, 1)):
        for bufs in ((a, b, c), (b, c, a), (c, a, b)):  # the empty range first, last and in the middle
            sink = roofline.read_only(*bufs, blocks=blocks, unroll=unroll, threads=threads)
            torch.cuda.synchronize()
            assert roofline.sink_total(sink, blocks) == roofline.word_sum(a, b, c), (threads, blocks, unroll)
