"""int4 prefill matmul (config 3) on the GPU vs the CPU oracle X @ dequantize(W)^T in fp32
(reference kernels/mm_int4.py:92-106 checks the same product with a norm-relative error).
Bar: max relative error <= 1e-2 with the per-output floor max(2^-14, 256 u32 sum_k |X_mk w_nk|), cosine >= 0.9999."""
import numpy as np
import pytest
import torch

import cuda_gemv
import mm_int4
import synth
import _hiplib as H
from oracle import int4 as O

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().float().cpu().numpy()


def _ref(X, q, s, m):
    a = (_np(X), q.cpu().numpy(), s.cpu().numpy(), m.cpu().numpy())
    return O.mm_int4(*a), O.cond_floor(O.mm_int4_abs(*a))


def _check(Y, ref, label=""):
    rep = O.parity_report(_np(Y), *ref)
    assert rep["max_rel"] <= 1e-2 and rep["cosine"] >= 0.9999, f"{label} {rep}"
    return rep


@pytest.mark.parametrize("N,K", [(3072, 2048), (22016, 2048), (2048, 11008)])
@pytest.mark.parametrize("M", [34, 128])
def test_config3_shapes(M, N, K, dev):
    X, q, s, m = synth.prefill_case(M, N, K, 3)
    Y = mm_int4.mm_int4(X.to(dev), q.to(dev), s.to(dev), m.to(dev))
    assert Y.shape == (M, N) and Y.dtype == torch.float16
    rep = _check(Y, _ref(X, q, s, m), f"M={M} N={N} K={K}")
    print(f"M={M} N={N} K={K}: {rep}")


@pytest.mark.parametrize("N,K,kernel", [(3072, 2048, H.MM_TILE64), (22016, 2048, H.MM_WIDE128),
                                         (2048, 11008, H.MM_WIDE128)])
@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
def test_config3_m512(N, K, kernel, xdt, dev):
    """M = 512 on every config-3 shape through the drop-in (workspace entry); gate+up 22016 x 2048 runs the
    wide-wave prepared-X kernel and down 2048 x 11008 the same kernel split over K (asserted; their tile-kernel
    runs are in test_prepared_x_against_tile_kernels)."""
    assert H.mm_plan(512, N, K)[0] == kernel
    X, q, s, m = synth.prefill_case(512, N, K, 3)
    X = X.to(xdt)
    Y = mm_int4.mm_int4(X.to(dev), q.to(dev), s.to(dev), m.to(dev))
    rep = _check(Y, _ref(X, q, s, m), f"M=512 N={N} K={K} {xdt}")
    print(f"M=512 N={N} K={K} {xdt}: {rep}")


@pytest.mark.parametrize("T,kernel", [(34, H.MM_STREAM), (69, H.MM_WIDE128), (201, H.MM_WIDE128)])
def test_reference_w_in_prompts(T, kernel, dev):
    """The reference's own check (kernels/mm_int4.py:92-106): w_in 25088 x 2048 at T in {34, 69, 201}, bf16 X as
    the engine passes it, through the drop-in (the kernels the plan picks, asserted); T = 69 / 201 on the tile
    kernels are in test_prepared_x_against_tile_kernels."""
    N, K = 25088, 2048
    assert H.mm_plan(T, N, K) == (kernel, 1)
    X, q, s, m = synth.prefill_case(T, N, K, 30 + T)
    X = X.bfloat16()
    Y = mm_int4.mm_int4(X.to(dev), q.to(dev), s.to(dev), m.to(dev))
    assert Y.dtype == torch.bfloat16
    ref = _ref(X, q, s, m)
    rep = _check(Y, ref, f"T={T}")
    # the reference's own metric: norm-relative error against the fp32 dequantize-then-matmul (~0.0017 there)
    assert rep["norm_rel"] < 5e-3, rep
    print(f"T={T}: {rep}")


@pytest.mark.parametrize("M,N,K", [(1, 64, 128), (3, 17, 256), (17, 100, 384), (33, 48, 2048), (65, 129, 1152),
                                   (200, 33, 11008)])
def test_ragged(M, N, K, dev):
    X, q, s, m = synth.prefill_case(M, N, K, 4)
    Y = mm_int4.mm_int4(X.to(dev), q.to(dev), s.to(dev), m.to(dev))
    _check(Y, _ref(X, q, s, m), f"M={M} N={N} K={K}")


@pytest.mark.parametrize("M,N,K", [(34, 2048, 11008), (34, 3072, 4096), (5, 200, 4096), (128, 2048, 11008),
                                   (64, 2048, 11008)])
def test_split_k_matches_single_pass(M, N, K, dev):
    """The workspace entry's split-K plans (fp32 partials + ordered sum over K splits of the tile kernels; the stream
    kernel, which serves M <= 48 only for K <= 2048 and has no K split, takes none of these shapes) against the
    single-pass kernel of rk_mm_int4_g128 and the oracle; both calls go through the C ABI, the second twice into one
    workspace."""
    L = H.lib()
    nws = L.rk_mm_int4_workspace_bytes(M, N, K)
    assert nws > 0
    X, q, s, m = synth.prefill_case(M, N, K, 11)
    Xd, qd, sd, md = X.to(dev), q.to(dev), s.to(dev), m.to(dev)
    Y1 = torch.empty(M, N, device=dev, dtype=torch.float32)
    H.check(L.rk_mm_int4_g128(H.ptr(Xd), H.F16, K, H.ptr(qd), H.ptr(sd), H.ptr(md), H.ptr(Y1), H.F32, N, M, N, K,
                              H.stream(dev)))
    ws = torch.full((nws,), 0xFF, device=dev, dtype=torch.uint8)  # stale contents must not matter
    for _ in range(2):
        Y2 = torch.full((M, N), 3.0, device=dev, dtype=torch.float32)
        H.check(L.rk_mm_int4_g128_ws(H.ptr(Xd), H.F16, K, H.ptr(qd), H.ptr(sd), H.ptr(md), H.ptr(Y2), H.F32, N, M,
                                     N, K, H.ptr(ws), nws, H.stream(dev)))
        torch.cuda.synchronize()
        ref = _ref(X, q, s, m)
        _check(Y1, ref, "single pass")
        _check(Y2, ref, "split K")
        # the two differ only in fp32 summation order
        np.testing.assert_allclose(_np(Y2), _np(Y1), rtol=1e-4, atol=1e-6 * float(np.abs(_np(Y1)).max()))


def test_bf16_and_fp32_out(dev):
    X, q, s, m = synth.prefill_case(40, 256, 2048, 5)
    Xb = X.bfloat16()
    Y = mm_int4.mm_int4(Xb.to(dev), q.to(dev), s.to(dev), m.to(dev))
    assert Y.dtype == torch.bfloat16
    _check(Y, _ref(Xb, q, s, m), "bf16")
    Y32 = torch.empty(40, 256, device=dev, dtype=torch.float32)
    mm_int4.mm_int4(Xb.to(dev), q.to(dev), s.to(dev), m.to(dev), out=Y32)
    _check(Y32, _ref(Xb, q, s, m), "fp32 out")


def test_rows_match_gemv(dev):
    # row m of the prefill product is the batch-1 GEMV of X[m] (both within the bar of the same oracle)
    X, q, s, m = (t.to(dev) for t in synth.prefill_case(9, 3072, 2048, 6))
    Y = mm_int4.mm_int4(X, q, s, m, out=torch.empty(9, 3072, device=dev, dtype=torch.float32))
    for i in range(9):
        y = torch.empty(3072, device=dev, dtype=torch.float32)
        cuda_gemv.gemv_int4_cuda(X[i].contiguous(), q, s, m, out=y)
        np.testing.assert_allclose(_np(Y[i]), _np(y), rtol=1e-4, atol=2e-5)


def test_strided_rows_through_c_abi(dev):
    # X rows with a stride larger than K (a view into a wider buffer), Y with a padded row stride
    M, N, K = 20, 96, 512
    X, q, s, m = synth.prefill_case(M, N, K, 7)
    Xw = torch.zeros(M, K + 64, dtype=torch.float16)
    Xw[:, :K] = X
    Xd, qd, sd, md = Xw.to(dev), q.to(dev), s.to(dev), m.to(dev)
    Yw = torch.full((M, N + 16), 7.0, device=dev, dtype=torch.float32)
    H.check(H.lib().rk_mm_int4_g128(H.ptr(Xd), H.F16, K + 64, H.ptr(qd), H.ptr(sd), H.ptr(md), H.ptr(Yw), H.F32,
                                    N + 16, M, N, K, H.stream(dev)))
    torch.cuda.synchronize()
    _check(Yw[:, :N], _ref(X, q, s, m), "strided")
    assert torch.all(Yw[:, N:] == 7.0)  # nothing written outside the [M, N] window


def test_min_term_known_answer(dev):
    M, N, K = 37, 80, 2048
    X = torch.ones(M, K, dtype=torch.float16, device=dev)
    q = torch.zeros(N, K // 2, dtype=torch.uint8, device=dev)
    s = (torch.rand(N, K // 128, device=dev) * 0.02 + 0.001).half()
    m = torch.ones(N, K // 128, dtype=torch.float16, device=dev)
    Y = mm_int4.mm_int4(X, q, s, m, out=torch.empty(M, N, device=dev, dtype=torch.float32))
    assert torch.equal(Y.cpu(), torch.full((M, N), float(K)))


def test_errors_and_knobs(dev):
    X, q, s, m = (t.to(dev) for t in synth.prefill_case(4, 32, 256, 8))
    mm_int4.mm_int4(X, q, s, m, BM=16, BN=128, num_warps=8, num_stages=2)  # Triton knobs accepted
    with pytest.raises(AssertionError):
        mm_int4.mm_int4(X[:, :128], q, s, m)
    with pytest.raises(AssertionError):
        mm_int4.mm_int4(X, q, s, m, BN=0)


def test_warmup_and_graph(dev):
    mm_int4.warmup([(64, 256)])
    X, q, s, m = (t.to(dev) for t in synth.prefill_case(34, 512, 2048, 9))
    Y = torch.empty(34, 512, device=dev, dtype=torch.float16)
    mm_int4.mm_int4(X, q, s, m, out=Y)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        mm_int4.mm_int4(X, q, s, m, out=Y)
    for i in range(3):
        X.copy_(synth.prefill_case(34, 512, 2048, 20 + i)[0].to(dev))
        Y.zero_()
        g.replay()
        torch.cuda.synchronize()
        _check(Y, _ref(X.cpu(), q.cpu(), s.cpu(), m.cpu()), f"replay {i}")


# ---- the prepared-X kernels (workspace entry) against the tile kernels (plain entry) and the oracle
def _abi(X, q, s, m, Y, ws=None, ldx=None, ldy=None):
    L = H.lib()
    M, K = X.shape[0], q.shape[1] * 2
    N = q.shape[0]
    args = [H.ptr(X), H.dt(X), ldx or X.stride(0), H.ptr(q), H.ptr(s), H.ptr(m), H.ptr(Y), H.dt(Y), ldy or Y.stride(0),
            M, N, K]
    if ws is None:
        H.check(L.rk_mm_int4_g128(*args, H.stream(X.device)), "rk_mm_int4_g128")
    else:
        H.check(L.rk_mm_int4_g128_ws(*args, H.ptr(ws), ws.numel(), H.stream(X.device)), "rk_mm_int4_g128_ws")


def _ws(M, N, K, dev):
    n = H.lib().rk_mm_int4_workspace_bytes(M, N, K)
    return torch.full((max(n, 16),), 0xFF, device=dev, dtype=torch.uint8)  # stale contents must not matter


@pytest.mark.parametrize("M,N,K,prep,tile", [(512, 22016, 2048, H.MM_WIDE128, H.MM_TILE128),
                                             (201, 25088, 2048, H.MM_WIDE128, H.MM_TILE128),
                                             (69, 25088, 2048, H.MM_WIDE128, H.MM_TILE64),
                                             (40, 65536, 2048, H.MM_PREP48, H.MM_TILE64),
                                             (128, 22016, 2048, H.MM_WIDE128, H.MM_TILE64),
                                             (64, 22016, 4096, H.MM_PREP64, H.MM_TILE64),
                                             (512, 20480, 1152, H.MM_PREP128, H.MM_TILE128),
                                             (512, 2048, 11008, H.MM_WIDE128, H.MM_TILE64)])
def test_prepared_x_against_tile_kernels(M, N, K, prep, tile, dev):
    """Each benchmarked / reference prompt shape on both plans: both within the oracle bar, and equal to each other up
    to fp32 summation order."""
    assert H.mm_plan(M, N, K, use_workspace=True)[0] == prep
    assert H.mm_plan(M, N, K, use_workspace=False) == (tile, 1)
    X, q, s, m = synth.prefill_case(M, N, K, 21)
    X = X.bfloat16() if M in (40, 69, 201) else X  # the engine passes bf16 on the w_in prompts
    Xd, qd, sd, md = X.to(dev), q.to(dev), s.to(dev), m.to(dev)
    Yp = torch.full((M, N), 3.0, device=dev, dtype=torch.float32)
    Yt = torch.full((M, N), -3.0, device=dev, dtype=torch.float32)
    _abi(Xd, qd, sd, md, Yp, ws=_ws(M, N, K, dev))
    _abi(Xd, qd, sd, md, Yt)
    torch.cuda.synchronize()
    ref = _ref(X, q, s, m)
    rp = _check(Yp, ref, f"prepared M={M} N={N} K={K}")
    _check(Yt, ref, f"tile M={M} N={N} K={K}")
    np.testing.assert_allclose(_np(Yp), _np(Yt), rtol=1e-4, atol=1e-6 * float(np.abs(_np(Yt)).max()))
    print(f"M={M} N={N} K={K}: {rp}")


@pytest.mark.parametrize("M,N,K,xdt,ydt", [(49, 20488, 256, torch.float16, torch.float16),
                                           (63, 20480, 384, torch.bfloat16, torch.float32),
                                           (61, 20360, 1152, torch.float16, torch.bfloat16),
                                           (130, 20480, 256, torch.bfloat16, torch.bfloat16),
                                           (200, 20600, 512, torch.float16, torch.float32),
                                           (96, 20488, 1024, torch.bfloat16, torch.bfloat16),
                                           (77, 20520, 1536, torch.float16, torch.float16),
                                           (300, 1000, 4352, torch.bfloat16, torch.float32),
                                           (260, 1544, 3328, torch.float16, torch.bfloat16)])
def test_prepared_x_ragged_and_dtypes(M, N, K, xdt, ydt, dev):
    """Ragged rows (the last block's missing m tiles, rows past M), ragged columns (N not a multiple of 128 or 8),
    odd group counts, every input / output dtype; nothing is written outside [M, N]."""
    kernel, _ = H.mm_plan(M, N, K, use_workspace=True)
    assert kernel in H.MM_PREP, (M, N, K, kernel)
    X, q, s, m = synth.prefill_case(M, N, K, 22)
    X = X.to(xdt)
    Xd, qd, sd, md = X.to(dev), q.to(dev), s.to(dev), m.to(dev)
    Yw = torch.full((M + 1, N + 8), 7.0, device=dev, dtype=ydt)  # one guard row, eight guard columns
    Y = Yw[:M, :N]
    _abi(Xd, qd, sd, md, Y, ws=_ws(M, N, K, dev), ldy=N + 8)
    torch.cuda.synchronize()
    _check(Y, _ref(X, q, s, m), f"M={M} N={N} K={K} {xdt}->{ydt}")
    assert torch.all(Yw[M] == 7.0) and torch.all(Yw[:, N:] == 7.0)


@pytest.mark.parametrize("M,kernel", [(50, H.MM_PREP64), (100, H.MM_WIDE128)])
def test_prepared_x_strided_rows_and_scale_fallback(M, kernel, dev):
    """X rows with a stride beyond K; scale / min arrays that are not 16-byte aligned take the tile plan instead
    (same workspace size suffices) — both within the bar."""
    N, K = 20480, 512
    assert H.mm_plan(M, N, K, use_workspace=True) == (kernel, 1)
    X, q, s, m = synth.prefill_case(M, N, K, 23)
    Xw = torch.zeros(M, K + 64, dtype=torch.float16)
    Xw[:, :K] = X
    Xd, qd = Xw.to(dev), q.to(dev)
    sd, md = s.to(dev), m.to(dev)
    ws = _ws(M, N, K, dev)
    Y = torch.empty(M, N, device=dev, dtype=torch.float32)
    _abi(Xd, qd, sd, md, Y, ws=ws, ldx=K + 64)
    torch.cuda.synchronize()
    ref = _ref(X, q, s, m)
    _check(Y, ref, "strided X")
    # the same scales and mins, 2 bytes past a 16-byte boundary
    sb = torch.empty(s.numel() + 1, dtype=torch.float16, device=dev)[1:].view(N, K // 128)
    mb_ = torch.empty(m.numel() + 1, dtype=torch.float16, device=dev)[1:].view(N, K // 128)
    sb.copy_(sd)
    mb_.copy_(md)
    assert sb.data_ptr() % 16 and mb_.data_ptr() % 16
    Y2 = torch.empty_like(Y)
    _abi(Xd, qd, sb, mb_, Y2, ws=ws, ldx=K + 64)
    torch.cuda.synchronize()
    _check(Y2, ref, "unaligned scales")


# ---- the small-M stream kernel (M <= 48 and K <= 2048: X held in registers, code tiles streamed, no K split)
F16, BF16, F32 = torch.float16, torch.bfloat16, torch.float32


@pytest.mark.parametrize("M,N,K,xdt,ydt", [(34, 3072, 2048, F16, F16), (34, 22016, 2048, F16, F16),
                                           (34, 25088, 2048, BF16, BF16), (1, 64, 128, F16, F32),
                                           (16, 2048, 2048, BF16, F16), (17, 100, 384, F16, BF16),
                                           (48, 20360, 1152, BF16, F32), (33, 48, 2048, F16, F16),
                                           (3, 17, 256, BF16, F32), (32, 4104, 1920, F16, F16),
                                           (40, 30000, 1408, F16, F16)])
def test_stream_kernel(M, N, K, xdt, ydt, dev):
    """Every m-tile count (M = 1 .. 48), K from one group to 16 (K = 1920 / 1408: 15 / 11 groups, so waves own one
    or two groups; K = 128: seven waves with none), ragged columns (N % 16 != 0, a short last block), 1 .. 8 tiles
    per block, every dtype pairing, X rows with a stride beyond K; against the oracle, nothing written outside
    [M, N], and the three entries (workspace, no-alloc and plain) bit-identical."""
    kernel, splits = H.mm_plan(M, N, K, use_workspace=True)
    assert kernel == H.MM_STREAM and splits == 1
    X, q, s, m = synth.prefill_case(M, N, K, 40 + M)
    X = X.to(xdt)
    Xw = torch.zeros(M, K + 32, dtype=xdt)
    Xw[:, :K] = X
    Xd, qd, sd, md = Xw.to(dev), q.to(dev), s.to(dev), m.to(dev)
    Yw = torch.full((M + 1, N + 8), 7.0, device=dev, dtype=ydt)  # one guard row, eight guard columns
    Y = Yw[:M, :N]
    _abi(Xd, qd, sd, md, Y, ws=_ws(M, N, K, dev), ldx=K + 32, ldy=N + 8)
    torch.cuda.synchronize()
    rep = _check(Y, _ref(X, q, s, m), f"M={M} N={N} K={K} {xdt}->{ydt}")
    assert torch.all(Yw[M] == 7.0) and torch.all(Yw[:, N:] == 7.0)
    L = H.lib()
    Yn = torch.full((M, N), -7.0, device=dev, dtype=ydt)
    H.check(L.rk_mm_int4_g128_noalloc(H.ptr(Xd), H.dt(Xd), K + 32, H.ptr(qd), H.ptr(sd), H.ptr(md), H.ptr(Yn),
                                      H.dt(Yn), N, M, N, K, H.stream(dev)), "noalloc")
    assert H.mm_plan(M, N, K, use_workspace=False) == (H.MM_STREAM, 1)
    Yp = torch.full((M, N), 9.0, device=dev, dtype=ydt)
    _abi(Xd, qd, sd, md, Yp, ldx=K + 32)
    torch.cuda.synchronize()
    assert torch.equal(Yp, Y)
    torch.cuda.synchronize()
    assert torch.equal(Yn, Y)
    print(f"M={M} N={N} K={K} {xdt}->{ydt}: {rep}")


def test_stream_kernel_one_hot_codes(dev):
    """Exact known answers through the stream kernel: a single code 1 at column k of row n (all else 0), scale 1,
    min 0, X = integers, gives Y[:, n] = X[:, k] exactly, for k at both nibbles and in every quarter / group of a
    chunk; other columns are exactly 0."""
    M, N, K = 34, 64, 2048
    X = torch.randint(-8, 9, (M, K), dtype=torch.float32).half()
    q = torch.zeros(N, K // 2, dtype=torch.uint8)
    ks = [0, 1, 7, 8, 31, 32, 127, 128, 255, 1000, 1777, 2047]
    for n, k in enumerate(ks):
        q[n, k // 2] = 1 if k % 2 == 0 else 0x10
    s = torch.ones(N, K // 128, dtype=torch.float16)
    mn = torch.zeros(N, K // 128, dtype=torch.float16)
    assert H.mm_plan(M, N, K) == (H.MM_STREAM, 1)
    Y = mm_int4.mm_int4(X.to(dev), q.to(dev), s.to(dev), mn.to(dev), out=torch.empty(M, N, device=dev, dtype=F32))
    want = torch.zeros(M, N)
    for n, k in enumerate(ks):
        want[:, n] = X[:, k].float()
    assert torch.equal(Y.cpu(), want)
