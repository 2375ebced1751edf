"""The C-ABI library without a GPU: it loads, exports every function include/rumik_hip.h declares, the binding
table covers them, and argument validation answers before any device work (status codes and their texts are the
reference's error messages, kernels/cuda_gemv.py:121,135,190)."""
import ctypes
import re
import subprocess

import pytest

import _hiplib as HL
from conftest import ROOT

HEADER = ROOT / "include" / "rumik_hip.h"


def declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^[A-Za-z_][\w \t\*]*?\b(rk_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_drop_in_entry_points():
    names = declared()
    for n in ("rk_gemv_int4_g128", "rk_gemv_int8_rows", "rk_mm_int4_g128", "rk_embed_ln", "rk_add_ln", "rk_post",
              "rk_attn_split", "rk_attn_combine", "rk_decode_step_persistent"):
        assert n in names, n


def test_library_exports_every_declared_symbol():
    lib = HL.lib()
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", str(HL.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (\w+)$", out, flags=re.M))
    assert set(declared()) <= exported, sorted(set(declared()) - exported)
    # and nothing else: the library is built with hidden visibility, the header alone decides the exports
    assert exported == set(declared()), sorted(exported - set(declared()))


def test_binding_table_covers_the_header():
    assert set(declared()) == set(HL.exported_symbols())


def test_version_and_status_strings():
    lib = HL.lib()
    assert lib.rk_abi_version() == 5
    texts = {0: "ok", -1: "shape", -2: "unsupported block shape", -3: "unsupported dtype", -4: "null pointer",
             -6: "kernel launch failed"}
    for code, t in texts.items():
        assert lib.rk_status_string(code).decode() == t
    assert "misaligned" in lib.rk_status_string(-5).decode()


@pytest.mark.parametrize("M,N,K,splits", [(34, 2048, 11008, 8), (34, 3072, 2048, 1), (128, 2048, 11008, 4),
                                          (200, 33, 11008, 21), (34, 22016, 2048, 1), (512, 2048, 11008, 8),
                                          (512, 22016, 2048, 1), (4, 32, 256, 1), (64, 2048, 11008, 8),
                                          (5, 200, 4096, 8)])
def test_mm_int4_split_k_plan(M, N, K, splits):
    """fp32 partials only where 64 x 64 output tiles leave CUs idle: splits = min(ceil(256 / tiles), groups / 4);
    shapes on the prepared-X kernels hold the prepared X instead (the wide-wave kernel split over K, for M >= 256
    with long K and few 128 x 128 tiles, also its partials: splits = min(round(512 / tiles), groups / 4)), and the
    stream kernel (M <= 48, K <= 2048) none"""
    nbytes = HL.lib().rk_mm_int4_workspace_bytes(M, N, K)
    kernel, sp = HL.mm_plan(M, N, K)
    assert sp == splits
    if kernel in HL.MM_PREP:
        Mp = (M + 15) // 16 * 16
        prep = Mp * K * 2 + (K // 128) * Mp * 4
        if sp == 1:
            assert nbytes == prep
        else:
            assert kernel == HL.MM_WIDE128 and nbytes >= (prep + 255) // 256 * 256 + sp * M * N * 4
    else:
        assert nbytes == (splits * M * N * 4 if splits > 1 else 0)


def test_mm_int4_ws_rejects_small_workspace():
    lib = HL.lib()
    buf = ctypes.c_void_p(256)  # never dereferenced: validation comes first
    need = lib.rk_mm_int4_workspace_bytes(34, 2048, 11008)
    args = (buf, HL.F16, 11008, buf, buf, buf, buf, HL.F16, 2048, 34, 2048, 11008)
    assert lib.rk_mm_int4_g128_ws(*args, buf, need - 4, None) == -1
    assert lib.rk_mm_int4_g128_ws(*args, None, need, None) == -1
    assert lib.rk_mm_int4_g128_ws(*args, ctypes.c_void_p(264), need, None) == -5


def test_decode_params_struct_matches_the_binding():
    import decode
    assert HL.lib().rk_decode_params_size() == ctypes.sizeof(decode.RkDecodeParams)


@pytest.mark.parametrize("N,K", [(64, 100), (64, 0), (0, 256), (-1, 256)])
def test_gemv_int4_rejects_bad_shapes(N, K):
    lib = HL.lib()
    buf = ctypes.c_void_p(16)  # never dereferenced: validation comes first
    for fn in (lib.rk_gemv_int4_g128, lib.rk_gemv_int4_g128_valu, lib.rk_gemv_int4_g128_mfma):
        assert fn(buf, HL.F16, buf, buf, buf, buf, HL.F16, N, K, 0, 0, None) == -1


def test_gemv_int4_rejects_bad_dtype_and_block_shape():
    lib = HL.lib()
    buf = ctypes.c_void_p(16)
    assert lib.rk_gemv_int4_g128(buf, 7, buf, buf, buf, buf, HL.F16, 64, 256, 0, 0, None) == -3
    assert lib.rk_gemv_int4_g128_mfma(buf, HL.F16, buf, buf, buf, buf, HL.F16, 64, 256, 0, 3, None) == -2


def test_gemv_int4_rejects_null_and_misaligned():
    lib = HL.lib()
    buf, odd = ctypes.c_void_p(256), ctypes.c_void_p(258)
    assert lib.rk_gemv_int4_g128(None, HL.F16, buf, buf, buf, buf, HL.F16, 64, 256, 0, 0, None) == -4
    assert lib.rk_gemv_int4_g128(buf, HL.F16, odd, buf, buf, buf, HL.F16, 64, 256, 0, 0, None) == -5


def test_layer_projections_validate_before_launch():
    """rk_gemv_int4_g128_layer: workspace size query, then NULL / dtype / shape / alignment / workspace checks on the
    host (fake, never dereferenced pointers) in that order."""
    lib = HL.lib()
    assert lib.rk_gemv_int4_g128_layer_ws_bytes(11008) == (64 + 2 * 256 + 11008) * 4
    assert lib.rk_gemv_int4_g128_layer_ws_bytes(0) == 0
    buf, odd = ctypes.c_void_p(256), ctypes.c_void_p(258)
    nws = lib.rk_gemv_int4_g128_layer_ws_bytes(11008)

    def call(x=buf, ws=buf, xdt=HL.F16, ydt=HL.F16, n_plain=3072, inter=11008, hid=2048, nbytes=nws, q=buf, sc=buf):
        return lib.rk_gemv_int4_g128_layer(x, buf, xdt, q, sc, buf, buf, buf, buf, buf, buf, buf, buf, buf, buf,
                                           buf, ydt, n_plain, inter, hid, ws, nbytes, None)
    assert call(x=None) == -4 and call(ws=None) == -4
    assert call(xdt=HL.F32) == -3 and call(ydt=HL.F32) == -3
    assert call(hid=4096) == -1 and call(inter=11008 + 64) == -1 and call(inter=12416) == -1
    assert call(n_plain=-1) == -1 and call(nbytes=nws - 4) == -1
    assert call(q=odd) == -5 and call(sc=odd) == -5  # codes 16-byte, scales / mins 4-byte aligned


def test_decode_step_validates_before_launch():
    import decode
    p = decode.RkDecodeParams()
    assert HL.lib().rk_decode_step_persistent(None, 256, None) == -4
    p.L, p.NH, p.NKV, p.inter, p.S, p.nsp, p.n_audio = 2, 16, 4, 11008, 64, 64, 16385
    assert HL.lib().rk_decode_step_persistent(ctypes.byref(p), 256, None) == -4  # null buffers
    for n in (0, 512 * 256 + 1):  # head rows: 1 .. 64 per tile wave
        p.n_audio = n
        assert HL.lib().rk_decode_step_persistent(ctypes.byref(p), 256, None) == -1
    p.n_audio = 16385
    p.NH = 12  # 12 * 128 != 2048
    assert HL.lib().rk_decode_step_persistent(ctypes.byref(p), 256, None) == -1
    p.NH, p.inter = 16, 11000  # not a multiple of 128
    assert HL.lib().rk_decode_step_persistent(ctypes.byref(p), 256, None) == -1
    p.inter = 11008
    assert HL.lib().rk_decode_step_persistent(ctypes.byref(p), 200, None) == -2  # nblocks != NKV * nsp


def test_sampler_entry_points_validate_before_any_device_work():
    """rk_stop_hidden / rk_topk_partial / rk_pick / rk_sample_tail reject bad sizes, dtypes and NULLs on the host
    (fake, never dereferenced pointers): top_k above 32, a candidate list that is not a power of two or too small
    or above 4096 slots, unsupported dtypes (reference pick asserts top_k <= 32, engine/sample.py:111)."""
    lib = HL.lib()
    P = ctypes.c_void_p(256)
    S = None
    # rk_pick(keys, scratch, u, z1, w2, b2, ids, step, tok, out, inv_temp, end_id, min_new, nch, nc, topk, nz, s)
    pick = lambda nch, nc, topk, nz=512: lib.rk_pick(P, P, P, P, P, P, P, P, P, P, 1.25, 16384, 8, nch, nc, topk,  # noqa: E731
                                                     nz, S)
    assert pick(33, 2048, 33) == -1
    assert pick(33, 2048, 0) == -1
    assert pick(33, 1024, 30) == -1      # 33 * 32 candidates do not fit
    assert pick(33, 3000, 30) == -1      # not a power of two
    assert pick(200, 8192, 30) == -1     # above 128 chunks
    assert pick(33, 2048, 30, nz=0) == -1
    assert lib.rk_pick(None, P, P, P, P, P, P, P, P, P, 1.0, 1, 8, 33, 2048, 30, 512, S) == -4
    assert lib.rk_topk_partial(P, 7, P, P, 16385, 16384, 8, S) == -3
    assert lib.rk_topk_partial(P, 2, P, P, 0, 0, 8, S) == -1
    assert lib.rk_stop_hidden(P, 1, P, P, P, 5, P, P, 1e-5, 2048, 512, S) == -3
    assert lib.rk_stop_hidden(P, 1, P, P, P, 1, P, P, 1e-5, 0, 512, S) == -1
    assert lib.rk_stop_hidden(P, 1, P, P, ctypes.c_void_p(258), 1, P, P, 1e-5, 2048, 512, S) == -5
    # rk_sample_tail: same checks (nv = 16385 -> 33 chunks need nc >= 1056)
    tail = lambda nc, topk: lib.rk_sample_tail(P, 1, P, P, P, 1, P, P, P, 1e-5, 2048, 512, P, 2, 16385, 16384, P,  # noqa: E731
                                               P, P, P, P, 1.25, 16384, 8, topk, P, P, nc, P, P, S)
    assert tail(1024, 30) == -1 and tail(2048, 40) == -1
    assert lib.rk_sample_tail(P, 1, P, P, P, 1, P, P, P, 1e-5, 2048, 512, P, 2, 16385, 16384, P, P, P, P, P, 1.25,
                              16384, 8, 30, P, P, 2048, P, None, S) == -4


@pytest.mark.parametrize("M,N,K,kernel", [(512, 22016, 2048, HL.MM_WIDE128), (201, 25088, 2048, HL.MM_WIDE128),
                                          (69, 25088, 2048, HL.MM_WIDE128), (34, 22016, 2048, HL.MM_STREAM),
                                          (64, 22016, 4096, HL.MM_PREP64), (128, 22016, 2048, HL.MM_WIDE128),
                                          (512, 20480, 1152, HL.MM_PREP128), (130, 20480, 256, HL.MM_PREP128),
                                          (512, 22016, 4096, HL.MM_PREP128), (200, 20600, 512, HL.MM_WIDE128),
                                          (512, 3072, 2048, HL.MM_TILE64), (512, 2048, 11008, HL.MM_WIDE128),
                                          (256, 2048, 11008, HL.MM_WIDE128), (128, 2048, 11008, HL.MM_TILE64),
                                          (34, 3072, 2048, HL.MM_STREAM), (34, 22017, 128, HL.MM_STREAM),
                                          (34, 2048, 11008, HL.MM_TILE64), (48, 20480, 2048, HL.MM_STREAM),
                                          (49, 20480, 2048, HL.MM_PREP64), (40, 65536, 2048, HL.MM_PREP48),
                                          (50, 2048, 11008, HL.MM_TILE64)])
def test_mm_int4_workspace_plan(M, N, K, kernel):
    """With a workspace, M <= 48 at K <= 2048 takes the stream kernel unless a block's scale / min tables would
    exceed 2048 entries (very wide N); otherwise shapes with >= 160 column blocks of 128 take the prepared-X kernel
    (48 / 64 / 128-row blocks by M; for M > 64 the wide-wave kernel when K / 128 is even and >= 4, split over K
    for M >= 256 with long K and few tiles); too few blocks, K too long for the block's scale tables, or N * K / 128
    not a multiple of 8 keep the tile plan."""
    assert HL.mm_plan(M, N, K, use_workspace=True)[0] == kernel


@pytest.mark.parametrize("M,N,K,kernel", [(512, 22016, 2048, HL.MM_TILE128), (201, 25088, 2048, HL.MM_TILE128),
                                          (512, 2048, 11008, HL.MM_TILE64), (69, 25088, 2048, HL.MM_TILE64),
                                          (34, 22016, 2048, HL.MM_STREAM), (128, 22016, 2048, HL.MM_TILE64),
                                          (512, 3072, 2048, HL.MM_TILE64), (4, 32, 200064, HL.MM_REGS),
                                          (34, 2048, 11008, HL.MM_TILE64)])
def test_mm_int4_plan_query(M, N, K, kernel):
    """The plan query names the kernel each shape runs (the GPU tests assert it for the shapes they cover). Without
    a workspace the stream kernel (M <= 48, K <= 2048) needs none either."""
    k, sp = HL.mm_plan(M, N, K, use_workspace=False)
    assert k == kernel and sp == 1
    k2, sp2 = HL.mm_plan(M, N, K, use_workspace=True)
    nbytes = HL.lib().rk_mm_int4_workspace_bytes(M, N, K)
    if k2 in HL.MM_PREP:  # prepared X (fp16, rows padded to 16) and its per-group row sums (fp32)
        Mp = (M + 15) // 16 * 16
        prep = Mp * K * 2 + (K // 128) * Mp * 4
        if sp2 == 1:
            assert nbytes == prep
        else:  # the wide-wave kernel split over K: fp32 partial sums after the prepared X
            assert k2 == HL.MM_WIDE128 and nbytes >= (prep + 255) // 256 * 256 + sp2 * M * N * 4
        assert k2 == (HL.MM_PREP48 if M <= 48 else HL.MM_PREP64 if M <= 64 else k2)
    else:
        assert (sp2 > 1) == (nbytes > 0) and nbytes == (sp2 * M * N * 4 if sp2 > 1 else 0)
    with pytest.raises(RuntimeError):
        HL.mm_plan(M, N, 100, use_workspace=False)


def test_noalloc_rejects_shapes_beyond_its_scratch():
    """rk_mm_int4_g128_noalloc refuses, before touching any device, a shape whose split-K partials exceed the fixed
    scratch (the pointers below are never dereferenced), and names the reason."""
    M, N, K = 2048, 1024, 65536
    assert HL.lib().rk_mm_int4_workspace_bytes(M, N, K) > HL.MM_SCRATCH_BYTES
    buf = ctypes.create_string_buffer(64)
    p = ctypes.cast(ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 16, ctypes.c_void_p)
    st = HL.lib().rk_mm_int4_g128_noalloc(p, HL.F16, K, p, p, p, p, HL.F16, N, M, N, K, None)
    assert st == HL.ERR_SCRATCH
    assert "scratch" in HL.lib().rk_status_string(st).decode()
    assert HL.lib().rk_mm_int4_g128_noalloc(p, HL.F16, K, p, p, p, p, HL.F16, N, M, N, 100, None) == -1  # shape


def test_status_constants_match_the_header():
    text = HEADER.read_text()
    codes = {m.group(1): int(m.group(2)) for m in re.finditer(r"#define RK_(OK|ERR_\w+) \(?(-?\d+)\)?", text)}
    assert codes and all(getattr(HL, k) == v for k, v in codes.items()), codes
