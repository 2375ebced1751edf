"""int8 per-row (audio head) GEMV on the GPU vs the CPU oracle ((q - 128) * s) @ x in fp32 (reference
kernels/cuda_gemv.py:234-249). Config 2: K=2048, N=16385 (ragged), int8 codes, fp16 row scale, fp32 logits.
Same bar as the int4 GEMV: max relative error <= 1e-2 with the per-output floor max(2^-14, 256 u32 sum|w x|),
cosine >= 0.9999."""
import numpy as np
import pytest
import torch

import cuda_gemv
import synth
import _hiplib as H
from oracle import int4 as O

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().float().cpu().numpy()


def _ref(x, q, s, kind):
    a = (x.float().numpy(), q.numpy(), s.numpy(), kind)
    return O.gemv_int8_rows(*a), O.cond_floor(O.gemv_int8_abs(*a))


def _check(y, ref, label=""):
    rep = O.parity_report(_np(y), *ref)
    assert rep["max_rel"] <= 1e-2 and rep["cosine"] >= 0.9999, f"{label} {rep}"
    return rep


def test_config2_head(dev):
    x, q, s = synth.int8_case(16385, 2048, 2)
    y = torch.empty(16385, device=dev, dtype=torch.float32)
    cuda_gemv.gemv_int8_cuda(x.to(dev), q.to(dev), s.to(dev), out=y)
    rep = _check(y, _ref(x, q, s, "s8"))
    print(rep)


def test_reference_layout_u8_fp32_scale_bf16(dev):
    # the reference's own layout: uint8 = int8 + 128, fp32 scale, bf16 x and y, rows padded to 16
    g = torch.Generator().manual_seed(5)
    w = torch.randn(16385, 2048, generator=g) * 0.02
    q, s = cuda_gemv.quantize_int8_rows(w)
    assert q.shape == (16400, 2048) and q.dtype == torch.uint8 and s.dtype == torch.float32
    qo, so = O.quantize_int8_rows(w.numpy())
    assert np.array_equal(q.numpy(), qo) and np.array_equal(s.numpy(), so)
    x = torch.randn(2048, generator=g).bfloat16()
    y = cuda_gemv.gemv_int8_cuda(x.to(dev), q.to(dev), s.to(dev))
    assert y.dtype == torch.bfloat16 and y.shape == (16400,)
    ref = _ref(x, q, s, "u8")
    rep = O.parity_report(_np(y), *ref)
    assert rep["cosine"] >= 0.9999 and rep["norm_rel"] < 5e-3, rep
    assert torch.all(y[16385:].float() == 0)
    y32 = torch.empty(16400, device=dev, dtype=torch.float32)
    cuda_gemv.gemv_int8_cuda(x.to(dev), q.to(dev), s.to(dev), out=y32)
    _check(y32, ref)


@pytest.mark.parametrize("N,K", [(1, 16), (3, 48), (17, 512), (100, 2048), (33, 4096), (5, 11008)])
def test_ragged_and_small(N, K, dev):
    x, q, s = synth.int8_case(N, K, 8)
    y = torch.empty(N, device=dev, dtype=torch.float32)
    cuda_gemv.gemv_int8_cuda(x.to(dev), q.to(dev), s.to(dev), out=y)
    _check(y, _ref(x, q, s, "s8"), f"N={N} K={K}")


@pytest.mark.parametrize("waves,rows", [(1, 1), (2, 2), (4, 1), (4, 2), (4, 4), (8, 1), (8, 2), (16, 1), (4, 8)])
def test_block_shapes(waves, rows, dev):
    x, q, s = synth.int8_case(4099, 2048, 9)
    xd, qd, sd = x.to(dev), q.to(dev), s.to(dev)
    y = torch.empty(4099, device=dev, dtype=torch.float32)
    H.check(H.lib().rk_gemv_int8_rows_ex(H.ptr(xd), H.F16, H.ptr(qd), H.Q_S8, H.ptr(sd), H.F16, H.ptr(y), H.F32,
                                         4099, 2048, waves, rows, H.stream(dev)))
    torch.cuda.synchronize()
    _check(y, _ref(x, q, s, "s8"), f"{waves}x{rows}")


def test_extreme_codes_known_answer(dev):
    K = 2048
    q = torch.stack([torch.full((K,), 127, dtype=torch.int8), torch.full((K,), -127, dtype=torch.int8),
                     torch.zeros(K, dtype=torch.int8)]).to(dev)
    s = torch.tensor([1e-3, 7e-3, 5e-3], dtype=torch.float16, device=dev)
    y = torch.empty(3, device=dev, dtype=torch.float32)
    cuda_gemv.gemv_int8_cuda(torch.ones(K, dtype=torch.float16, device=dev), q, s, out=y)
    expect = torch.tensor([127 * K * float(s[0]), -127 * K * float(s[1]), 0.0])
    torch.testing.assert_close(y.cpu(), expect, rtol=1e-6, atol=0)


def test_onehot_bit_exact(dev):
    # row n: code c_n in [-127, 127] at column k_n, scale 1 -> y[n] = c_n * x[k_n] exactly; both layouts
    N, K = 256, 2048
    g = torch.Generator().manual_seed(12)
    ks = torch.randint(0, K, (N,), generator=g)
    cs = torch.randint(-127, 128, (N,), generator=g)
    codes = torch.zeros(N, K, dtype=torch.int16)
    codes[torch.arange(N), ks] = cs.to(torch.int16)
    x = torch.randn(K, generator=g).half()
    expect = cs.float() * x.float()[ks]
    for q in (codes.to(torch.int8), (codes + 128).to(torch.uint8)):
        y = torch.empty(N, device=dev, dtype=torch.float32)
        cuda_gemv.gemv_int8_cuda(x.to(dev), q.contiguous().to(dev), torch.ones(N, device=dev), out=y)
        assert torch.equal(y.cpu(), expect)
