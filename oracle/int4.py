"""numpy restatement of the int4 / int8 weight formats and their products (test infrastructure only).

References (neoandmatrix/rumik-fast):
  format     kernels/int4_gemv.py:1-4 (affine identity), :16-24 (quantize), :27-30 (dequantize);
             modal_export_int4.py:48-59 (exporter q4); hf_card/README.md:46-53 (format spec)
  int4 GEMV  kernels/bench_gemv.py:43 / bench_cuda.py:38 (dequantize(q,s,m) @ x.float() as the fp32 reference)
  int8 GEMV  kernels/cuda_gemv.py:234-249 (uint8 = int8 + 128, fp32 row scale, y = ((q - 128) * s) @ x)
  prefill    kernels/mm_int4.py:8-11, :96-97 (X @ dequantize(W)^T in fp32)
"""
import numpy as np

G = 128


def unpack_int4(q: np.ndarray) -> np.ndarray:
    """uint8 [N, K/2] -> codes uint8 [N, K]; byte j holds column 2j in its low nibble and 2j+1 in its high nibble
    (kernels/int4_gemv.py:23,29; kernels/mm_int4.py:39 "col 2j = low nibble")."""
    q = np.asarray(q, dtype=np.uint8)
    codes = np.empty((q.shape[0], q.shape[1] * 2), dtype=np.uint8)
    codes[:, 0::2] = q & 0x0F
    codes[:, 1::2] = q >> 4
    return codes


def pack_int4(codes: np.ndarray) -> np.ndarray:
    """codes [N, K] in 0..15 -> uint8 [N, K/2] (inverse of unpack_int4; kernels/int4_gemv.py:23)."""
    c = np.asarray(codes, dtype=np.uint8)
    if c.max(initial=0) > 15:
        raise ValueError("int4 codes must be in 0..15")
    return np.ascontiguousarray(c[:, 0::2] | (c[:, 1::2] << 4))


def quantize(w: np.ndarray, group: int = G):
    """[N, K] float -> (q uint8 [N, K/2], scale fp16 [N, K/g], min fp16 [N, K/g]); min/max round-to-nearest
    (half to even, as torch.round) per group, scale = max((max - min) / 15, 1e-8) (kernels/int4_gemv.py:16-24)."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    g = w.reshape(n, k // group, group)
    lo = g.min(axis=-1, keepdims=True)
    hi = g.max(axis=-1, keepdims=True)
    step = np.maximum((hi - lo) / np.float32(15), np.float32(1e-8)).astype(np.float32)
    code = np.clip(np.rint((g - lo) / step), 0, 15).astype(np.uint8).reshape(n, k)
    return pack_int4(code), step.astype(np.float16).reshape(n, -1), lo.astype(np.float16).reshape(n, -1)


def dequantize(q, s, m, group: int = G) -> np.ndarray:
    """w = code * scale + min in fp32 from fp16 scale / min (kernels/int4_gemv.py:27-30)."""
    codes = unpack_int4(q).astype(np.float32)
    n, k = codes.shape
    s32 = np.asarray(s, dtype=np.float16).astype(np.float32).reshape(n, k // group, 1)
    m32 = np.asarray(m, dtype=np.float16).astype(np.float32).reshape(n, k // group, 1)
    return (codes.reshape(n, k // group, group) * s32 + m32).reshape(n, k)


def gemv_int4(x, q, s, m) -> np.ndarray:
    """The reference's fp32 check: dequantize(q, s, m) @ x.float() (kernels/bench_cuda.py:38). Returns fp32 [N]."""
    return dequantize(q, s, m) @ np.asarray(x).astype(np.float32)


def dequantize_f64(q, s, m, group: int = G) -> np.ndarray:
    """dequantize() in float64: code * scale + min is exact there (4-bit code times an fp16 value, plus an fp16)."""
    codes = unpack_int4(q).astype(np.float64)
    n, k = codes.shape
    s64 = np.asarray(s, dtype=np.float16).astype(np.float64).reshape(n, k // group, 1)
    m64 = np.asarray(m, dtype=np.float16).astype(np.float64).reshape(n, k // group, 1)
    return (codes.reshape(n, k // group, group) * s64 + m64).reshape(n, k)


def gemv_int4_f64(x, q, s, m) -> np.ndarray:
    """Same product in float64 throughout (an error-free shadow for judging fp32 rounding)."""
    return dequantize_f64(q, s, m) @ np.asarray(x).astype(np.float64)


def int8_codes(q, q_kind: str) -> np.ndarray:
    """Signed codes from the two int8 layouts: 'u8' = uint8 holding int8 + 128 (kernels/cuda_gemv.py:238-241),
    's8' = plain int8."""
    if q_kind == "u8":
        return np.asarray(q, dtype=np.uint8).astype(np.int16) - 128
    if q_kind == "s8":
        return np.asarray(q, dtype=np.int8).astype(np.int16)
    raise ValueError(q_kind)


def gemv_int8_rows(x, q, s, q_kind: str = "u8") -> np.ndarray:
    """y = ((q - 128) * s) @ x, fp32 (kernels/cuda_gemv.py:246-249 semantics). Returns fp32 [N]."""
    w = int8_codes(q, q_kind).astype(np.float32) * np.asarray(s).astype(np.float32)[:, None]
    return w @ np.asarray(x).astype(np.float32)


def gemv_int8_rows_f64(x, q, s, q_kind: str = "u8") -> np.ndarray:
    """gemv_int8_rows in float64 throughout (the per-row scale applied to the exact code, as the fp32 form does)."""
    w = int8_codes(q, q_kind).astype(np.float64) * np.asarray(s).astype(np.float64)[:, None]
    return w @ np.asarray(x).astype(np.float64)


def quantize_int8_rows(w, pad_to: int = 16):
    """[N, K] -> (uint8 [N', K] = int8 + 128, fp32 scale [N']), rows zero-padded to a multiple of pad_to;
    scale = max(max|w| / 127, 1e-8), code = clip(round(w / scale), -127, 127) (kernels/cuda_gemv.py:234-242)."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    n_pad = -(-n // pad_to) * pad_to
    wf = np.zeros((n_pad, k), dtype=np.float32)
    wf[:n] = w
    scale = np.maximum(np.abs(wf).max(axis=1) / np.float32(127), np.float32(1e-8)).astype(np.float32)
    codes = np.clip(np.rint(wf / scale[:, None]), -127, 127)
    return (codes + 128).astype(np.uint8), scale


def mm_int4(X, q, s, m) -> np.ndarray:
    """Prefill product Y[T, N] = X[T, K] @ dequantize(W)^T in fp32 (kernels/mm_int4.py:96-97)."""
    return np.asarray(X).astype(np.float32) @ dequantize(q, s, m).T


def mm_int4_f64(X, q, s, m) -> np.ndarray:
    """The prefill product in float64 throughout."""
    return np.asarray(X).astype(np.float64) @ dequantize_f64(q, s, m).T


# ---------------------------------------------------------------- error metrics used by every parity test
FP16_TINY = 2.0 ** -14  # smallest normal fp16: below it the fp16 output grid itself has no 1e-2 relative precision
U32 = 2.0 ** -24        # fp32 unit roundoff
COND_MULT = 256         # floor = 256 unit roundoffs of the dot product's absolute sum (see cond_floor)


def gemv_int4_abs(x, q, s, m) -> np.ndarray:
    """sum_k |w[n,k] * x[k]| per row: the absolute sum that bounds any fp32 evaluation's rounding error."""
    return np.abs(dequantize(q, s, m)).astype(np.float64) @ np.abs(np.asarray(x).astype(np.float64))


def gemv_int8_abs(x, q, s, q_kind: str = "u8") -> np.ndarray:
    w = np.abs(int8_codes(q, q_kind).astype(np.float64)) * np.abs(np.asarray(s).astype(np.float64))[:, None]
    return w @ np.abs(np.asarray(x).astype(np.float64))


def mm_int4_abs(X, q, s, m) -> np.ndarray:
    return np.abs(np.asarray(X).astype(np.float64)) @ np.abs(dequantize(q, s, m)).astype(np.float64).T


def cond_floor(abs_sum) -> np.ndarray:
    """Per-output floor of the relative-error denominator: max(2^-14, 256 * u32 * sum_k |w_k x_k|).

    An fp32 dot product (the reference's own dequantize-then-matmul included) carries rounding error up to about
    u32 * sum|w x| (measured: the fp32 oracle reaches 0.96 of it against a float64 evaluation). For outputs smaller
    than ~100x that, relative error against an fp32 reference is set by the reference's rounding, not by the
    kernel; there the bar becomes absolute: |err| <= 1e-2 * 256 * u32 * sum|w x| = 2.56 u32 sum|w x|."""
    return np.maximum(FP16_TINY, COND_MULT * U32 * np.asarray(abs_sum, dtype=np.float64))


def rel_errors(y, ref, floor=FP16_TINY) -> np.ndarray:
    """Per-output relative error |y - ref| / max(|ref|, floor); floor may be a scalar or per-output array."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return np.abs(y - ref) / np.maximum(np.abs(ref), floor)


def cosine(y, ref) -> float:
    y = np.asarray(y, dtype=np.float64).ravel()
    ref = np.asarray(ref, dtype=np.float64).ravel()
    den = np.linalg.norm(y) * np.linalg.norm(ref)
    return float(np.dot(y, ref) / den) if den > 0 else float(np.array_equal(y, ref))


def parity_report(y, ref, floor=FP16_TINY) -> dict:
    """max relative error (with its |ref|), cosine, norm-relative error of y against ref; plus the max relative
    error with the fixed fp16 floor alone (`max_rel_strict`) for transparency when a per-output floor is given."""
    r = rel_errors(y, ref, floor).ravel()
    i = int(np.argmax(r)) if r.size else 0
    ref64 = np.asarray(ref, dtype=np.float64).ravel()
    y64 = np.asarray(y, dtype=np.float64).ravel()
    nrm = np.linalg.norm(ref64)
    strict = rel_errors(y64, ref64, FP16_TINY)
    return {
        "max_rel": float(r[i]) if r.size else 0.0,
        "worst_abs_ref": float(abs(ref64[i])) if r.size else 0.0,
        "max_rel_strict": float(strict.max()) if r.size else 0.0,
        "cosine": cosine(y, ref),
        "norm_rel": float(np.linalg.norm(y64 - ref64) / nrm) if nrm > 0 else 0.0,
        "n": int(r.size),
    }
