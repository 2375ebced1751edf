"""The committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py with float64
expected outputs computed from the format definitions): the CPU oracle and the engine's host-side tables must
reproduce them (CPU tests), and the HIP kernels must meet the parity bar against them (GPU tests: max relative
error 1e-2 with the per-output conditioning floor, cosine >= 0.9999)."""
import numpy as np
import pytest

from conftest import GOLDEN
from oracle import glue as OG
from oracle import int4 as O


def load(name):
    with np.load(GOLDEN / name, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def _close_to_f64(y, ref, abs_sum, ulps=8):
    # fp32 accumulation: error bounded by a few unit roundoffs of the absolute sum
    assert np.all(np.abs(np.asarray(y, np.float64) - ref) <= ulps * 2.0 ** -24 * abs_sum + 1e-12)


# ---------------------------------------------------------------------------------------------- CPU: the oracle
def test_oracle_gemv_int4_fixture():
    d = load("gemv_int4_96x384.npz")
    np.testing.assert_allclose(O.gemv_int4_f64(d["x"], d["q"], d["s"], d["m"]), d["y"], rtol=1e-12, atol=1e-12)
    _close_to_f64(O.gemv_int4(d["x"], d["q"], d["s"], d["m"]), d["y"],
                  O.gemv_int4_abs(d["x"], d["q"], d["s"], d["m"]))


def test_oracle_gemv_int8_fixture():
    d = load("gemv_int8_80x256.npz")
    np.testing.assert_allclose(O.gemv_int8_rows_f64(d["x"], d["codes"], d["s"], "s8"), d["y"], rtol=1e-12,
                               atol=1e-12)
    y = O.gemv_int8_rows(d["x"], d["codes"], d["s"], "s8")
    _close_to_f64(y, d["y"], O.gemv_int8_abs(d["x"], d["codes"], d["s"], "s8"))
    # the reference's uint8 + 128 layout gives the same result
    np.testing.assert_array_equal(O.gemv_int8_rows(d["x"], (d["codes"].astype(np.int16) + 128).astype(np.uint8),
                                                   d["s"], "u8"), y)


def test_oracle_mm_int4_fixture():
    d = load("mm_int4_5x64x256.npz")
    np.testing.assert_allclose(O.mm_int4_f64(d["X"], d["q"], d["s"], d["m"]), d["Y"], rtol=1e-12, atol=1e-12)
    _close_to_f64(O.mm_int4(d["X"], d["q"], d["s"], d["m"]), d["Y"], O.mm_int4_abs(d["X"], d["q"], d["s"], d["m"]))


def test_oracle_layernorm_fixture():
    d = load("layernorm_2048.npz")
    np.testing.assert_allclose(OG.cohere_ln(d["x"], d["w"], float(d["eps"])), d["h"], rtol=1e-5, atol=1e-5)


def test_oracle_rope_fixture():
    d = load("rope_64x128.npz")
    cos, sin = OG.rope_tables(64, 128, 10000.0)
    np.testing.assert_allclose(cos, d["cos"], atol=2e-5)
    np.testing.assert_allclose(sin, d["sin"], atol=2e-5)
    p = int(d["pos"])
    np.testing.assert_allclose(OG.rope(d["v"], cos[p], sin[p]), d["rot"], rtol=1e-5, atol=1e-5)


def test_engine_rope_tables_fixture():
    import torch
    import decode
    cos, sin = decode.rope_tables(64, 128, 10000.0, torch.float16, "cpu")
    d = load("rope_64x128.npz")
    np.testing.assert_allclose(cos.float().numpy(), d["cos"], atol=1e-3)  # fp16 tables
    np.testing.assert_allclose(sin.float().numpy(), d["sin"], atol=1e-3)


def test_oracle_attention_fixture():
    d = load("attention_8x2x37.npz")
    np.testing.assert_allclose(OG.attend(d["q"], d["K"], d["V"]), d["out"], rtol=1e-5, atol=1e-5)
    out, _, _ = OG.attend_split(d["q"], d["K"], d["V"], nsplit=5, chunk=8)
    np.testing.assert_allclose(out, d["out"], rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------------------------------------- GPU: HIP kernels
MAX_REL, MIN_COS = 1e-2, 0.9999


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _bar(y, ref, floor):
    rep = O.parity_report(y, ref, floor)
    assert rep["max_rel"] <= MAX_REL and rep["cosine"] >= MIN_COS, rep


@pytest.mark.gpu
@pytest.mark.parametrize("path", ["default", "valu", "mfma"])
def test_gpu_gemv_int4_fixture(dev, path):
    import torch
    import cuda_gemv
    import _hiplib as HL
    d = load("gemv_int4_96x384.npz")
    x, q, s, m = (_t(d[k], dev) for k in ("x", "q", "s", "m"))
    y = torch.empty(96, dtype=torch.float16, device=dev)
    if path == "default":
        cuda_gemv.gemv_int4_cuda(x, q, s, m, out=y)
    else:
        fn = {"valu": HL.lib().rk_gemv_int4_g128_valu, "mfma": HL.lib().rk_gemv_int4_g128_mfma}[path]
        HL.check(fn(HL.ptr(x), HL.dt(x), HL.ptr(q), HL.ptr(s), HL.ptr(m), HL.ptr(y), HL.dt(y), 96, 384, 0, 0,
                    HL.stream(dev)))
    torch.cuda.synchronize()
    _bar(y.float().cpu().numpy(), d["y"], O.cond_floor(O.gemv_int4_abs(d["x"], d["q"], d["s"], d["m"])))


@pytest.mark.gpu
def test_gpu_gemv_int8_fixture(dev):
    import torch
    import cuda_gemv
    d = load("gemv_int8_80x256.npz")
    y = torch.empty(80, dtype=torch.float32, device=dev)
    cuda_gemv.gemv_int8_cuda(_t(d["x"], dev), _t(d["codes"], dev), _t(d["s"], dev), out=y)
    torch.cuda.synchronize()
    _bar(y.cpu().numpy(), d["y"], O.cond_floor(O.gemv_int8_abs(d["x"], d["codes"], d["s"], "s8")))


@pytest.mark.gpu
def test_gpu_mm_int4_fixture(dev):
    import torch
    import mm_int4
    d = load("mm_int4_5x64x256.npz")
    Y = mm_int4.mm_int4(_t(d["X"], dev), _t(d["q"], dev), _t(d["s"], dev), _t(d["m"], dev))
    torch.cuda.synchronize()
    _bar(Y.float().cpu().numpy(), d["Y"], O.cond_floor(O.mm_int4_abs(d["X"], d["q"], d["s"], d["m"])))


@pytest.mark.gpu
def test_gpu_layernorm_fixture(dev):
    import torch
    import fused
    d = load("layernorm_2048.npz")
    x = _t(d["x"], dev)
    zero = torch.zeros_like(x)
    h = torch.empty_like(x)
    fused.add_ln(x, zero, None, _t(d["w"], dev), h, float(d["eps"]))
    torch.cuda.synchronize()
    np.testing.assert_allclose(h.float().cpu().numpy(), d["h"], rtol=1e-2, atol=2e-3)  # fp16 output


@pytest.mark.gpu
@pytest.mark.parametrize("nsplit", [1, 4, 16])
def test_gpu_attention_fixture(dev, nsplit):
    import torch
    import fused
    d = load("attention_8x2x37.npz")
    NH, NKV, n, HD, S = 8, 2, 37, 128, 48
    kc = torch.zeros(NKV, S, HD, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    kc[:, :n] = torch.from_numpy(d["K"])
    vc[:, :n] = torch.from_numpy(d["V"])
    kc, vc = kc.to(dev), vc.to(dev)
    q = _t(d["q"].reshape(-1), dev)
    pos = torch.tensor([n - 1], dtype=torch.int64, device=dev)
    po = torch.empty(NH, nsplit, HD, dtype=torch.float32, device=dev)
    pm = torch.empty(NH, nsplit, dtype=torch.float32, device=dev)
    pl = torch.empty_like(pm)
    out = torch.empty(NH * HD, dtype=torch.float16, device=dev)
    fused.attn_split[(NKV, nsplit)](q, kc, vc, pos, po, pm, pl, kc.shape[1], HD ** -0.5, REP=NH // NKV, HD=HD, NSPLIT=nsplit)
    fused.attn_combine[(NH,)](po, pm, pl, pos, out, HD=HD, NSPLIT=nsplit)
    torch.cuda.synchronize()
    np.testing.assert_allclose(out.float().cpu().numpy().reshape(NH, HD), d["out"], rtol=1e-2, atol=2e-3)
