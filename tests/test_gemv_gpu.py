"""int4 g128 GEMV on the GPU vs the CPU oracle (dequantize-then-matmul in fp32) on identical seeded inputs.

Bar (benchmark definition): max relative error <= 1e-2 per output and cosine >= 0.9999, against the fp32
dequantize-then-matmul. Relative error is |y - ref| / max(|ref|, F_n) with the per-output floor
F_n = max(2^-14, 256 * 2^-24 * sum_k |w_nk x_k|) (oracle.int4.cond_floor): below it the fp32 reference's own
rounding (up to ~1 unit roundoff of sum|w x|) or the fp16 output grid decides the relative error, so there the bar
is absolute. The report also carries the plain fixed-floor figure (max_rel_strict). Integer unpacking is checked
bit-exactly with one-hot codes (scale 1, min 0: y = code * x[k] exactly).
"""
import numpy as np
import pytest
import torch

import cuda_gemv
import int4_gemv
import synth
import _hiplib as H
from oracle import int4 as O

pytestmark = pytest.mark.gpu

MAX_REL, MIN_COS = 1e-2, 0.9999


def _np(t):
    return t.detach().float().cpu().numpy()


def _oracle(x, q, s, m):
    """(fp32 reference, per-output floor)"""
    a = (_np(x), q.cpu().numpy(), s.cpu().numpy(), m.cpu().numpy())
    return O.gemv_int4(*a), O.cond_floor(O.gemv_int4_abs(*a))


def _assert_parity(y, ref, label=""):
    ref, floor = ref
    rep = O.parity_report(_np(y), ref, floor)
    assert rep["max_rel"] <= MAX_REL and rep["cosine"] >= MIN_COS, f"{label} {rep}"
    return rep


def _run(N, K, seed, dev, xdt=torch.float16, ydt=None, warps=None, rows=None, path="default"):
    """path: "default" (the drop-in wrapper) or one of the C ABI variants "mfma", "valu"."""
    x, q, s, m = synth.gemv_case(N, K, seed)
    x = x.to(xdt)
    xd, qd, sd, md = (t.to(dev) for t in (x, q, s, m))
    y = torch.empty(N, device=dev, dtype=ydt or xdt)
    if path == "default":
        cuda_gemv.gemv_int4_cuda(xd, qd, sd, md, out=y, warps=warps, rows=rows)
    else:
        fn = {"mfma": H.lib().rk_gemv_int4_g128_mfma, "valu": H.lib().rk_gemv_int4_g128_valu}[path]
        H.check(fn(H.ptr(xd), H.dt(xd), H.ptr(qd), H.ptr(sd), H.ptr(md), H.ptr(y), H.dt(y), N, K, warps or 0,
                   rows or 0, H.stream(dev)))
    torch.cuda.synchronize()
    return y, _oracle(x, q, s, m)


# ---- the benchmark's shapes: config 0 (seed 0) and the config-1 projections (seed 1), plus the engine's fused w_in
@pytest.mark.parametrize("path", ["default", "mfma", "valu"])
@pytest.mark.parametrize("N,K,seed", [(2048, 2048, 0), (3072, 2048, 1), (2048, 2048, 1), (22016, 2048, 1),
                                      (2048, 11008, 1), (25088, 2048, 1), (2048, 13056, 1)])
def test_config_shapes(N, K, seed, path, dev):
    y, ref = _run(N, K, seed, dev, path=path)
    rep = _assert_parity(y, ref, f"{path} N={N} K={K}")
    print(f"{path} N={N} K={K}: {rep}")


@pytest.mark.parametrize("N,K,seed", [(32768, 2048, 21), (8192, 3072, 22), (16384, 1024, 23), (8200, 4096, 24)])
def test_large_n_split_plans(N, K, seed, dev):
    """Large-N shapes of the matrix-core path, one per split of K over a tile's waves (2 waves at K = 2048, 4 at
    3072 / 4096, 1 at 1024; N = 8200 also leaves a partial last tile), through the default entry."""
    y, ref = _run(N, K, seed, dev)
    _assert_parity(y, ref, f"N={N} K={K}")


@pytest.mark.parametrize("path", ["default", "mfma", "valu"])
@pytest.mark.parametrize("N,K", [(1, 128), (3, 256), (17, 384), (1001, 2048), (63, 4096), (5, 11008), (7, 32768),
                                 (40, 1152), (33, 65536)])
def test_ragged_and_small(N, K, path, dev):
    y, ref = _run(N, K, 7, dev, path=path)
    _assert_parity(y, ref, f"N={N} K={K}")


@pytest.mark.parametrize("path", ["default", "mfma", "valu"])
@pytest.mark.parametrize("warps,rows", [(8, 2), (8, 1), (8, 4), (4, 1), (4, 2), (4, 4), (16, 1), (16, 2), (1, 8), (2, 8)])
@pytest.mark.parametrize("N,K", [(2048, 2048), (2048, 11008), (100, 2048)])
def test_reference_block_shapes(warps, rows, N, K, path, dev):
    y, ref = _run(N, K, 3, dev, warps=warps, rows=rows, path=path)
    _assert_parity(y, ref, f"{warps}x{rows} N={N} K={K}")


@pytest.mark.parametrize("xdt,ydt", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float32),
                                     (torch.bfloat16, torch.float32), (torch.float16, torch.bfloat16)])
def test_dtypes(xdt, ydt, dev):
    y, ref = _run(3072, 2048, 4, dev, xdt=xdt, ydt=ydt)
    _assert_parity(y, ref, f"{xdt}->{ydt}")  # bf16 output rounding alone is <= 2^-8 relative, inside the bar


# ---- known answers
@pytest.mark.parametrize("K", [128, 2048, 11008])
def test_min_term_known_answer(K, dev):
    N = 96
    q = torch.zeros(N, K // 2, dtype=torch.uint8, device=dev)
    s = torch.rand(N, K // 128, device=dev).half() * 0.02 + 0.001
    m = torch.ones(N, K // 128, dtype=torch.float16, device=dev)
    y = torch.empty(N, device=dev, dtype=torch.float32)
    cuda_gemv.gemv_int4_cuda(torch.ones(K, dtype=torch.float16, device=dev), q, s, m, out=y)
    assert torch.equal(y.cpu(), torch.full((N,), float(K)))


def test_all_fifteen_known_answer(dev):
    N, K = 64, 2048
    q = torch.full((N, K // 2), 0xFF, dtype=torch.uint8, device=dev)
    s = (torch.rand(N, K // 128, device=dev) * 0.02 + 0.001).half()
    m = torch.zeros_like(s)
    y = torch.empty(N, device=dev, dtype=torch.float32)
    cuda_gemv.gemv_int4_cuda(torch.ones(K, dtype=torch.float16, device=dev), q, s, m, out=y)
    expect = 15 * 128 * s.double().sum(1)
    torch.testing.assert_close(y.double().cpu(), expect.cpu(), rtol=1e-6, atol=0)


@pytest.mark.parametrize("K", [256, 2048, 11008])
def test_onehot_unpack_bit_exact(K, dev):
    # row n has a single code c_n = 1 + n % 15 at column k_n; scale 1, min 0 -> y[n] = c_n * x[k_n] exactly
    N = 512
    g = torch.Generator().manual_seed(11)
    ks = torch.randint(0, K, (N,), generator=g)
    cs = 1 + torch.arange(N) % 15
    codes = torch.zeros(N, K, dtype=torch.uint8)
    codes[torch.arange(N), ks] = cs.to(torch.uint8)
    q = (codes[:, 0::2] | (codes[:, 1::2] << 4)).contiguous()
    s = torch.ones(N, K // 128, dtype=torch.float16)
    m = torch.zeros_like(s)
    x = (torch.randn(K, generator=g) * 4).half()
    y = torch.empty(N, device=dev, dtype=torch.float32)
    cuda_gemv.gemv_int4_cuda(x.to(dev), q.to(dev), s.to(dev), m.to(dev), out=y)
    expect = cs.float() * x.float()[ks]
    assert torch.equal(y.cpu(), expect)
    assert np.array_equal(O.gemv_int4(x.numpy(), q.numpy(), s.numpy(), m.numpy()), expect.numpy())


# ---- drop-in API behaviour
def test_default_output_dtype_and_fallback_alias(dev):
    x, q, s, m = (t.to(dev) for t in synth.gemv_case(256, 512, 2))
    y = cuda_gemv.gemv_int4_cuda(x.bfloat16(), q, s, m)
    assert y.dtype == torch.bfloat16 and y.shape == (256,)
    y2 = int4_gemv.gemv_int4(x, q, s, m)
    assert y2.dtype == torch.float16


def test_shape_errors(dev):
    x, q, s, m = (t.to(dev) for t in synth.gemv_case(64, 256, 2))
    with pytest.raises(RuntimeError, match="shape"):
        cuda_gemv.gemv_int4_cuda(x[:128], q, s, m)
    with pytest.raises(RuntimeError, match="unsupported block shape"):
        cuda_gemv.gemv_int4_cuda(x, q, s, m, warps=3, rows=2)
    xb = torch.empty(257, dtype=torch.float16, device=dev)[1:]  # 2-byte offset: not 16-byte aligned
    xb.copy_(x)
    with pytest.raises(RuntimeError, match="aligned"):
        cuda_gemv.gemv_int4_cuda(xb, q, s, m)
    with pytest.raises(RuntimeError, match="GPU"):
        cuda_gemv.gemv_int4_cuda(x.cpu(), q, s, m)


def test_graph_capture_replays(dev):
    N, K = 3072, 2048
    x, q, s, m = (t.to(dev) for t in synth.gemv_case(N, K, 9))
    y = torch.empty(N, device=dev, dtype=torch.float16)
    cuda_gemv.gemv_int4_cuda(x, q, s, m, out=y)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        cuda_gemv.gemv_int4_cuda(x, q, s, m, out=y)
    for i in range(4):
        if i:  # new input between replays, written by ordinary eager work
            x.copy_(synth.gemv_case(N, K, 9 + i)[0].to(dev))
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        _assert_parity(y, _oracle(x.cpu(), q.cpu(), s.cpu(), m.cpu()), f"replay {i}")


def test_silu_fused_w_in_equals_gemv_then_silu(dev):
    """The engine's w_in shape ([q k v | gate | up] = 3072 + 2 x 11008 rows): one launch of the fused kernel gives
    bit-for-bit the GEMV followed by the SiLU·up kernel (same tile plan, same rounding of gate and up)."""
    n_plain, inter, K = 3072, 11008, 2048
    x, q, s, m = (t.to(dev) for t in synth.gemv_case(n_plain + 2 * inter, K, 12))
    y_all = cuda_gemv.gemv_int4_cuda(x, q, s, m, out=torch.empty(n_plain + 2 * inter, device=dev,
                                                                    dtype=torch.float16))
    act_ref = torch.empty(inter, device=dev, dtype=torch.float16)
    H.check(H.lib().rk_silu_mul(H.ptr(y_all[n_plain:]), H.ptr(act_ref), H.F16, inter, H.stream(dev)))
    y, act = cuda_gemv.gemv_int4_silu_cuda(x, q, s, m, n_plain)
    torch.cuda.synchronize()
    assert torch.equal(y, y_all[:n_plain])
    assert torch.equal(act, act_ref)
    _assert_parity(y, _oracle(x, q[:n_plain], s[:n_plain], m[:n_plain]), "w_in plain rows")


@pytest.mark.parametrize("n_plain,inter,K,xdt,ydt", [(40, 100, 256, torch.bfloat16, torch.float32),
                                                       (0, 8, 128, torch.float16, torch.float16),
                                                       (16, 1, 2048, torch.float16, torch.bfloat16),
                                                       (3, 37, 1152, torch.bfloat16, torch.bfloat16)])
def test_silu_fused_ragged(n_plain, inter, K, xdt, ydt, dev):
    """Ragged part sizes (plain rows not a multiple of 16, channels not a multiple of 8) and every dtype: y against
    the oracle's bar, act against silu(gate) * up evaluated in fp32 on the oracle's gate / up (rounded to ydt)."""
    N = n_plain + 2 * inter
    x, q, s, m = synth.gemv_case(N, K, 13)
    x = x.to(xdt)
    xd, qd, sd, md = x.to(dev), q.to(dev), s.to(dev), m.to(dev)
    y = torch.full((max(n_plain, 1),), 5.0, device=dev, dtype=ydt)
    act = torch.full((inter + 3,), 5.0, device=dev, dtype=ydt)  # 3 guard values past the end
    H.check(H.lib().rk_gemv_int4_g128_silu(H.ptr(xd), H.dt(xd), H.ptr(qd), H.ptr(sd), H.ptr(md), H.ptr(y),
                                           H.ptr(act), H.dt(act), n_plain, inter, K, 0, H.stream(dev)))
    torch.cuda.synchronize()
    ref, floor = _oracle(x, q, s, m)
    if n_plain:
        _assert_parity(y[:n_plain], (ref[:n_plain], floor[:n_plain]), "plain rows")
    else:
        assert torch.all(y == 5.0)
    g = torch.tensor(ref[n_plain:n_plain + inter], dtype=torch.float64)
    u = torch.tensor(ref[n_plain + inter:], dtype=torch.float64)
    sg = torch.sigmoid(g)
    want = g * sg * u
    # first-order bound: d(act) = silu'(g) u dg + silu(g) du (|silu'| <= 1.1), where gate / up each carry the
    # output rounding (eps, twice: kernel vs reference may round to neighbouring values) plus the GEMV bar's
    # absolute part (<= the per-output floor), and act its own rounding
    eps = {torch.float32: 1e-6, torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}[ydt]
    eg = 2 * eps * g.abs() + torch.tensor(floor[n_plain:n_plain + inter])
    eu = 2 * eps * u.abs() + torch.tensor(floor[n_plain + inter:])
    tol = 1.1 * u.abs() * eg + (g * sg).abs() * eu + 2 * eps * want.abs()
    got = act[:inter].double().cpu()
    assert torch.all((got - want).abs() <= tol), float(((got - want).abs() - tol).max())
    assert torch.all(act[inter:] == 5.0)  # nothing written past inter


def test_silu_fused_rejects_bad_arguments(dev):
    x, q, s, m = (t.to(dev) for t in synth.gemv_case(48, 256, 14))
    with pytest.raises(RuntimeError):
        cuda_gemv.gemv_int4_silu_cuda(x, q, s, m, 47)  # 1 row left: not a gate / up pair
    with pytest.raises(RuntimeError):
        cuda_gemv.gemv_int4_silu_cuda(x, q, s, m, 48)  # no MLP rows at all
    L = H.lib()
    assert L.rk_gemv_int4_g128_silu(H.ptr(x), H.F16, H.ptr(q), H.ptr(s), H.ptr(m), None, H.ptr(x), H.F16, 8, 20,
                                    256, 0, H.stream(dev)) == -4  # y missing while n_plain > 0
    assert L.rk_gemv_int4_g128_silu(H.ptr(x), H.F16, H.ptr(q), H.ptr(s), H.ptr(m), H.ptr(x), H.ptr(x), H.F16, 8, 0,
                                    256, 0, H.stream(dev)) == -1


@pytest.mark.parametrize("N1,K1,N2,K2", [(2048, 2048, 2048, 11008), (17, 256, 5, 11008), (1001, 2048, 63, 16384),
                                         (300, 4096, 40, 2048)])
def test_pair_equals_two_gemvs(N1, K1, N2, K2, dev):
    """rk_gemv_int4_g128_pair (one launch: the o and down projections) against the oracle for both outputs, and
    bit-equal to rk_gemv_int4_g128_valu with its default plan for each (the last case, K1 = 4096 and K2 = 2048,
    takes the two-launch fallback)."""
    x1, q1, s1, m1 = synth.gemv_case(N1, K1, 31)
    x2, q2, s2, m2 = synth.gemv_case(N2, K2, 32)
    d1 = tuple(t.to(dev) for t in (x1, q1, s1, m1))
    d2 = tuple(t.to(dev) for t in (x2, q2, s2, m2))
    y1, y2 = cuda_gemv.gemv_int4_pair_cuda(d1[0], d1[1:], d2[0], d2[1:])
    torch.cuda.synchronize()
    _assert_parity(y1, _oracle(x1, q1, s1, m1), "first")
    _assert_parity(y2, _oracle(x2, q2, s2, m2), "second")
    # the same arithmetic per row as the single-GEMV VALU kernel's default plan: equal bits
    for (x, q, s, m), y in ((d1, y1), (d2, y2)):
        z = torch.full_like(y, 7.0)
        H.check(H.lib().rk_gemv_int4_g128_valu(H.ptr(x), H.dt(x), H.ptr(q), H.ptr(s), H.ptr(m), H.ptr(z), H.dt(z),
                                               q.shape[0], q.shape[1] * 2, 0, 0, H.stream(dev)))
        torch.cuda.synchronize()
        assert torch.equal(y, z)


def test_pair_rejects_bad_arguments(dev):
    x, q, s, m = (t.to(dev) for t in synth.gemv_case(48, 256, 14))
    L = H.lib()
    args = lambda K2, xdt=H.F16: (H.ptr(x), H.F16, H.ptr(q), H.ptr(s), H.ptr(m), H.ptr(x), H.F16, 48, 256,  # noqa
                                  H.ptr(x), xdt, H.ptr(q), H.ptr(s), H.ptr(m), H.ptr(x), H.F16, 48, K2, H.stream(dev))
    assert L.rk_gemv_int4_g128_pair(*args(200)) == -1  # K2 not a multiple of 128: RK_ERR_SHAPE
    assert L.rk_gemv_int4_g128_pair(*args(256, xdt=H.F32)) == -3  # fp32 x: RK_ERR_DTYPE
    with pytest.raises(RuntimeError):
        cuda_gemv.gemv_int4_pair_cuda(x[:128], (q, s, m), x, (q, s, m))
