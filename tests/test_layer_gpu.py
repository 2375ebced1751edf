"""One-launch layer projections (rk_gemv_int4_g128_layer) against the CPU oracle on identical seeded inputs.

Each output is held to the bar of its own GEMV: y_plain and y_o against the oracle's fp32 dequantize-then-matmul
(max relative error 1e-2 with the per-output conditioning floor, cosine 0.9999); act against silu(gate) * up
evaluated in float64 on the oracle's gate / up with a first-order error bound; y_down against the oracle's down
projection of the act this same launch wrote (the kernel's own act is down's input, as in the reference's layer).
The launch counters in the workspace make every launch's exchange distinct: repeated launches and hipGraph replays
with new inputs between them are each checked, and the status word must stay 0.
"""
import numpy as np
import pytest
import torch

import cuda_gemv
import synth
import _hiplib as H
from oracle import int4 as O

pytestmark = pytest.mark.gpu

MAX_REL, MIN_COS = 1e-2, 0.9999
HID = 2048


def _np(t):
    return t.detach().float().cpu().numpy()


def _parity(y, x, q, s, m, label):
    a = (_np(x), q.cpu().numpy(), s.cpu().numpy(), m.cpu().numpy())
    rep = O.parity_report(_np(y), O.gemv_int4(*a), O.cond_floor(O.gemv_int4_abs(*a)))
    assert rep["max_rel"] <= MAX_REL and rep["cosine"] >= MIN_COS, f"{label} {rep}"


def _act_bound(act, x, q, s, m, n_plain, inter, ydt, label):
    """act against silu(gate) * up from the oracle's gate / up (first-order bound, as the fused w_in test)."""
    a = (_np(x), q.cpu().numpy(), s.cpu().numpy(), m.cpu().numpy())
    ref, floor = O.gemv_int4(*a), O.cond_floor(O.gemv_int4_abs(*a))
    g = torch.tensor(ref[n_plain:n_plain + inter], dtype=torch.float64)
    u = torch.tensor(ref[n_plain + inter:n_plain + 2 * inter], dtype=torch.float64)
    sg = torch.sigmoid(g)
    want = g * sg * u
    eps = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}[ydt]
    eg = 2 * eps * g.abs() + torch.tensor(floor[n_plain:n_plain + inter])
    eu = 2 * eps * u.abs() + torch.tensor(floor[n_plain + inter:n_plain + 2 * inter])
    tol = 1.1 * u.abs() * eg + (g * sg).abs() * eu + 2 * eps * want.abs()
    got = act[:inter].double().cpu()
    assert torch.all((got - want).abs() <= tol), f"{label}: {float(((got - want).abs() - tol).max())}"


def _case(n_plain, inter, seed, dev, xdt=torch.float16):
    g = synth.generator(seed)
    w_in = synth.int4_weights(n_plain + 2 * inter, HID, g)
    w_o = synth.int4_weights(HID, HID, g)
    w_d = synth.int4_weights(HID, inter, g)
    x = synth.activations(HID, g, dtype=xdt)
    ob = synth.activations(HID, g, dtype=xdt)
    d = lambda w: tuple(t.to(dev) for t in w)  # noqa: E731
    return x.to(dev), ob.to(dev), d(w_in), d(w_o), d(w_d)


def _check_all(outs, x, ob, w_in, w_o, w_d, n_plain, inter, ydt, label):
    y, act, yo, yd = outs
    torch.cuda.synchronize()
    if n_plain:
        _parity(y[:n_plain], x, *(t[:n_plain] for t in w_in), f"{label} q/k/v")
    _act_bound(act, x, *w_in, n_plain, inter, ydt, f"{label} act")
    _parity(yo, ob, *w_o, f"{label} o")
    _parity(yd, act[:inter], *w_d, f"{label} down")


def test_layer_config1_against_oracle_and_two_launches(dev):
    """The benchmark's layer (q/k/v 3072, gate / up 2 x 11008, o 2048 x 2048, down 2048 x 11008), fp16: every
    output against the oracle; y_plain / y_o against the two-launch path within the same bar, and act equal to the
    fused w_in kernel's wherever both round gate and up the same way (they sum in different orders)."""
    n_plain, inter = 3072, 11008
    x, ob, w_in, w_o, w_d = _case(n_plain, inter, 41, dev)
    lp = cuda_gemv.LayerProjections(n_plain, inter, dev)
    outs = lp(x, w_in, ob, w_o, w_d)
    _check_all(outs, x, ob, w_in, w_o, w_d, n_plain, inter, torch.float16, "config 1")
    assert lp.status() == 0
    y2, act2 = cuda_gemv.gemv_int4_silu_cuda(x, *w_in, n_plain)
    yo2, yd2 = cuda_gemv.gemv_int4_pair_cuda(ob, w_o, act2, w_d)
    torch.cuda.synchronize()
    same = (outs[1] == act2).float().mean().item()
    assert same > 0.95, same
    for a, b in ((outs[0], y2), (outs[2], yo2)):
        assert torch.allclose(a.float(), b.float(), rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("n_plain,inter,xdt,ydt", [(3072, 11008, torch.bfloat16, torch.bfloat16),
                                                   (100, 1280, torch.float16, torch.bfloat16),
                                                   (0, 128, torch.bfloat16, torch.float16),
                                                   (3072, 12288, torch.float16, torch.float16),
                                                   (5, 11136, torch.bfloat16, torch.float16)])
def test_layer_shapes_and_dtypes(n_plain, inter, xdt, ydt, dev):
    """Ragged and extreme part sizes for the 256-block grid (1 pair per block at inter = 128, all 6 pair slots of
    every wave at 12288, plain rows on a few blocks only, none at all) in every dtype pairing; guard values past
    each output."""
    x, ob, w_in, w_o, w_d = _case(n_plain, inter, 42 + inter % 7, dev, xdt)
    lp = cuda_gemv.LayerProjections(n_plain, inter, dev)
    y = torch.full((n_plain + 3,), 5.0, device=dev, dtype=ydt)
    act = torch.full((inter + 3,), 5.0, device=dev, dtype=ydt)
    yo = torch.full((HID + 3,), 5.0, device=dev, dtype=ydt)
    yd = torch.full((HID + 3,), 5.0, device=dev, dtype=ydt)
    L = H.lib()
    st = L.rk_gemv_int4_g128_layer(H.ptr(x), H.ptr(ob), H.dt(x), *(H.ptr(t) for t in w_in + w_o + w_d), H.ptr(y),
                                   H.ptr(act), H.ptr(yo), H.ptr(yd), H.dt(act), n_plain, inter, HID, H.ptr(lp.ws),
                                   lp.ws.numel() * 4, H.stream(dev))
    H.check(st)
    _check_all((y, act, yo[:HID], yd[:HID]), x, ob, w_in, w_o, w_d, n_plain, inter, ydt, f"{n_plain}/{inter}")
    for t, n in ((y, n_plain), (act, inter), (yo, HID), (yd, HID)):
        assert torch.all(t[n:] == 5.0)
    assert lp.status() == 0


def test_layer_repeated_launches_and_graph_replays(dev):
    """Eager launches back to back with new inputs, then a graph of two captured launches (two layers' weights)
    replayed with new inputs written by eager work between replays: every launch checked, status stays 0."""
    n_plain, inter = 3072, 11008
    x, ob, w_in, w_o, w_d = _case(n_plain, inter, 43, dev)
    _, _, w_in2, w_o2, w_d2 = _case(n_plain, inter, 44, dev)
    lp = cuda_gemv.LayerProjections(n_plain, inter, dev)
    outs = [torch.empty(n, device=dev, dtype=torch.float16) for n in (n_plain, inter, HID, HID)]
    gen = synth.generator(45)
    for i in range(3):
        x.copy_(synth.activations(HID, gen).to(dev))
        ob.copy_(synth.activations(HID, gen).to(dev))
        lp(x, w_in, ob, w_o, w_d, *outs)
        _check_all(outs, x, ob, w_in, w_o, w_d, n_plain, inter, torch.float16, f"eager {i}")
    outs2 = [torch.empty_like(t) for t in outs]
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        lp(x, w_in, ob, w_o, w_d, *outs)
        lp(x, w_in2, ob, w_o2, w_d2, *outs2)
    for i in range(3):
        x.copy_(synth.activations(HID, gen).to(dev))
        ob.copy_(synth.activations(HID, gen).to(dev))
        for t in outs + outs2:
            t.fill_(0.0)
        g.replay()
        torch.cuda.synchronize()
        _check_all(outs, x, ob, w_in, w_o, w_d, n_plain, inter, torch.float16, f"replay {i} layer 0")
        _check_all(outs2, x, ob, w_in2, w_o2, w_d2, n_plain, inter, torch.float16, f"replay {i} layer 1")
    assert lp.status() == 0


def test_layer_rejects_bad_arguments(dev):
    n_plain, inter = 3072, 11008
    x, ob, w_in, w_o, w_d = _case(n_plain, inter, 46, dev)
    lp = cuda_gemv.LayerProjections(n_plain, inter, dev)
    y, act, yo, yd = (torch.empty(n, device=dev, dtype=torch.float16) for n in (n_plain, inter, HID, HID))
    L = H.lib()
    nws = lp.ws.numel() * 4

    def call(xdt=H.F16, ydt=H.F16, np_=n_plain, it=inter, hid=HID, ws=nws, yp=H.ptr(y)):
        return L.rk_gemv_int4_g128_layer(H.ptr(x), H.ptr(ob), xdt, *(H.ptr(t) for t in w_in + w_o + w_d), yp,
                                         H.ptr(act), H.ptr(yo), H.ptr(yd), ydt, np_, it, hid, H.ptr(lp.ws), ws,
                                         H.stream(dev))
    assert call(hid=4096) == -1                 # hidden size other than 2048
    assert call(it=11008 + 64) == -1            # inter not a multiple of 128
    assert call(it=12288 + 128) == -1           # inter past 64 * 6 * 32
    assert call(np_=3073) == -1                 # more than 12 plain rows per block
    assert call(ws=nws - 4) == -1               # workspace too small
    assert call(xdt=H.F32) == -3 and call(ydt=H.F32) == -3
    assert call(yp=None) == -4                  # y_plain missing while n_plain > 0
    assert call(np_=0, yp=None, it=128) == 0    # no plain rows: y_plain may be NULL
    torch.cuda.synchronize()
    assert lp.status() == 0
    with pytest.raises(RuntimeError):
        lp(x, w_in, ob, w_o, (w_d[0][:, :1024], w_d[1], w_d[2]))
