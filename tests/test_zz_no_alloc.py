"""rk_mm_int4_g128_noalloc: the split-K prefill product with its partial sums in the library's fixed scratch array
instead of a caller-provided workspace. Through the C ABI, two calls in a row (the second on a smaller input, so
the scratch holds the first call's larger contents), each against rk_mm_int4_g128_ws with a fresh workspace on the
same inputs: the same plan and kernels, so the outputs are bit-identical; both are also held to the oracle bar.
Shapes without a split (no scratch used) take the same path."""
import numpy as np
import pytest
import torch

import synth
import _hiplib as H
from oracle import int4 as O

pytestmark = pytest.mark.gpu


def _call(fn_name, X, q, s, m, Y, ws=None):
    L = H.lib()
    M, K = X.shape
    N = q.shape[0]
    args = [H.ptr(X), H.dt(X), K, H.ptr(q), H.ptr(s), H.ptr(m), H.ptr(Y), H.dt(Y), N, M, N, K]
    if fn_name == "rk_mm_int4_g128_ws":
        args += [H.ptr(ws), ws.numel() if ws is not None else 0]
    H.check(getattr(L, fn_name)(*args, H.stream(X.device)), fn_name)


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
def test_noalloc_matches_workspace_entry(xdt, dev):
    L = H.lib()
    for M, N, K, seed in ((34, 2048, 11008, 51), (5, 200, 4096, 52), (40, 256, 2048, 53)):
        nws = L.rk_mm_int4_workspace_bytes(M, N, K)
        assert 0 <= nws <= H.MM_SCRATCH_BYTES
        X, q, s, m = synth.prefill_case(M, N, K, seed)
        X = X.to(xdt)
        Xd, qd, sd, md = X.to(dev), q.to(dev), s.to(dev), m.to(dev)
        ws = torch.full((max(nws, 16),), 0xFF, device=dev, dtype=torch.uint8)
        Yw = torch.full((M, N), 5.0, device=dev, dtype=torch.float32)
        Yn = torch.full((M, N), -5.0, device=dev, dtype=torch.float32)
        _call("rk_mm_int4_g128_ws", Xd, qd, sd, md, Yw, ws)
        _call("rk_mm_int4_g128_noalloc", Xd, qd, sd, md, Yn)
        torch.cuda.synchronize()
        assert torch.equal(Yn, Yw), (M, N, K)  # same plan, same kernels, same summation order
        a = (X.float().numpy(), q.numpy(), s.numpy(), m.numpy())
        rep = O.parity_report(Yn.cpu().numpy(), O.mm_int4(*a), O.cond_floor(O.mm_int4_abs(*a)))
        assert rep["max_rel"] <= 1e-2 and rep["cosine"] >= 0.9999, (M, N, K, rep)
        print(M, N, K, nws, rep)


def test_noalloc_in_a_graph_replay(dev):
    """Captured in a hipGraph (no allocation happens at capture or replay), replayed with new inputs in between."""
    M, N, K = 34, 2048, 11008  # split over K: the partial sums in the scratch
    assert H.mm_plan(M, N, K) == (H.MM_TILE64, 8)
    assert H.lib().rk_mm_int4_workspace_bytes(M, N, K) > 0
    X, q, s, m = (t.to(dev) for t in synth.prefill_case(M, N, K, 60))
    Y = torch.empty(M, N, device=dev, dtype=torch.float16)
    _call("rk_mm_int4_g128_noalloc", X, q, s, m, Y)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _call("rk_mm_int4_g128_noalloc", X, q, s, m, Y)
    for i in range(3):
        X.copy_(synth.prefill_case(M, N, K, 61 + i)[0].to(dev))
        Y.zero_()
        g.replay()
        torch.cuda.synchronize()
        ref = torch.empty_like(Y)
        ws = torch.empty(H.lib().rk_mm_int4_workspace_bytes(M, N, K), device=dev, dtype=torch.uint8)
        _call("rk_mm_int4_g128_ws", X, q, s, m, ref, ws)
        torch.cuda.synchronize()
        assert torch.equal(Y, ref), i
