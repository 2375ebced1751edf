"""ctypes binding of librumik_hip.so (the C ABI in include/rumik_hip.h).

torch is imported first on purpose: its bundled HIP runtime carries the SONAME libamdhip64.so.7, so the dynamic
linker binds the library to that same runtime and torch's streams and device pointers are valid inside it.
There is no fallback: if the library is missing, every call raises.
"""
import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parents[1] / "lib" / "librumik_hip.so"

F16, BF16, F32 = 0, 1, 2
Q_S8, Q_U8 = 0, 1
DTYPE_CODE = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32}

_p, _i, _f, _l = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_longlong
_SIGS = {
    "rk_abi_version": ([], _i),
    "rk_status_string": ([_i], ctypes.c_char_p),
    "rk_gemv_int4_g128": ([_p, _i, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p], _i),
    "rk_gemv_int4_g128_mfma": ([_p, _i, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p], _i),
    "rk_gemv_int4_g128_valu": ([_p, _i, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p], _i),
    "rk_gemv_int4_g128_pair": ([_p, _i, _p, _p, _p, _p, _i, _i, _i, _p, _i, _p, _p, _p, _p, _i, _i, _i, _p], _i),
    "rk_gemv_int4_g128_silu": ([_p, _i, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p], _i),
    "rk_gemv_int4_g128_layer_ws_bytes": ([_i], ctypes.c_size_t),
    "rk_gemv_int4_g128_layer": ([_p, _p, _i, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _p,
                                 ctypes.c_size_t, _p], _i),
    "rk_gemv_int8_rows": ([_p, _i, _p, _i, _p, _i, _p, _i, _i, _i, _p], _i),
    "rk_gemv_int8_rows_ex": ([_p, _i, _p, _i, _p, _i, _p, _i, _i, _i, _i, _i, _p], _i),
    "rk_mm_int4_g128": ([_p, _i, _i, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p], _i),
    "rk_mm_int4_plan": ([_i, _i, _i, _i, ctypes.POINTER(_i), ctypes.POINTER(_i)], _i),
    "rk_read_only": ([_p, ctypes.c_size_t, _p, ctypes.c_size_t, _p, ctypes.c_size_t, _i, _i, _p, _p], _i),
    "rk_read_only_ex": ([_p, ctypes.c_size_t, _p, ctypes.c_size_t, _p, ctypes.c_size_t, _i, _i, _i, _p, _p], _i),
    "rk_mm_int4_workspace_bytes": ([_i, _i, _i], ctypes.c_size_t),
    "rk_mm_int4_g128_ws": ([_p, _i, _i, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p, ctypes.c_size_t, _p], _i),
    "rk_mm_int4_g128_noalloc": ([_p, _i, _i, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p], _i),
    "rk_embed_ln": ([_p, _p, _p, _p, _p, _p, _i, _i, _f, _p], _i),
    "rk_add_ln": ([_p, _p, _p, _p, _p, _i, _i, _f, _p], _i),
    "rk_post": ([_p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i, _p], _i),
    "rk_attn_split": ([_p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _f, _p], _i),
    "rk_attn_combine": ([_p, _p, _p, _p, _p, _i, _i, _i, _i, _p], _i),
    "rk_pos_advance": ([_p, _p], _i),
    "rk_silu_mul": ([_p, _p, _i, _i, _p], _i),
    "rk_decode_step_persistent": ([_p, _i, _p], _i),
    "rk_decode_params_size": ([], _i),
    "rk_decode_get_limits": ([_p], _i),
    "rk_decode_step_roles": ([_p, _p], _i),
    "rk_decode_roles_params_size": ([], _i),
    "rk_decode_roles_placement": ([_p, _p], _i),
    "rk_decode_roles_get_limits": ([_p], _i),
    "rk_embed_ln_rows": ([_p, _p, _p, _p, _p, _p, _i, _i, _i, _f, _p], _i),
    "rk_add_ln_rows": ([_p, _p, _p, _p, _p, _i, _i, _i, _f, _p], _i),
    "rk_post_rows": ([_p, _i, _i, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i, _i, _p], _i),
    "rk_prefill_attn": ([_p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i, _f, _p], _i),
    "rk_stop_hidden": ([_p, _i, _p, _p, _p, _i, _p, _p, _f, _i, _i, _p], _i),
    "rk_topk_partial": ([_p, _i, _p, _p, _i, _i, _i, _p], _i),
    "rk_pick": ([_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _f, _l, _i, _i, _i, _i, _i, _p], _i),
    "rk_sample_tail": ([_p, _i, _p, _p, _p, _i, _p, _p, _p, _f, _i, _i, _p, _i, _i, _i, _p, _p, _p, _p, _p, _f, _l,
                        _i, _i, _p, _p, _i, _p, _p, _p], _i),
}

_lib = None


def lib():
    """The loaded library (loaded once; raises RuntimeError if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built: run `python rumik-fast_amd/build.py` (or "
                               "__graft_entry__.build()) first; there is no non-HIP fallback")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (args, ret) in _SIGS.items():
            fn = getattr(L, name, None)
            if fn is None:
                continue
            fn.argtypes, fn.restype = args, ret
        _lib = L
    return _lib


MM_REGS, MM_TILE128, MM_TILE64, MM_PREP128, MM_PREP64, MM_PREP48, MM_STREAM, MM_WIDE128 = 0, 1, 2, 3, 4, 5, 6, 7
MM_PREP = (MM_PREP128, MM_PREP64, MM_PREP48, MM_WIDE128)  # the plans that prepare X into the workspace
MM_SCRATCH_BYTES = 8 << 20  # RK_MM_SCRATCH_BYTES: the fixed split-K scratch of rk_mm_int4_g128_noalloc
# status codes (RK_OK and RK_ERR_* of the header)
OK, ERR_SHAPE, ERR_BLOCK, ERR_DTYPE, ERR_NULL, ERR_ALIGN, ERR_LAUNCH, ERR_SCRATCH = 0, -1, -2, -3, -4, -5, -6, -7


def mm_plan(M: int, N: int, K: int, use_workspace: bool = True):
    """(kernel, splits) that rk_mm_int4_g128[_ws] runs for this shape (kernel: MM_REGS / MM_TILE128 / MM_TILE64, or
    with a workspace MM_PREP128 / MM_PREP64 / MM_PREP48 / MM_WIDE128)."""
    k, sp = _i(), _i()
    check(lib().rk_mm_int4_plan(M, N, K, int(use_workspace), ctypes.byref(k), ctypes.byref(sp)), "mm_int4_plan")
    return k.value, sp.value


def exported_symbols():
    """Names the C ABI declares, for the load/export check."""
    return list(_SIGS)


def check(status: int, what: str = ""):
    if status != 0:
        msg = lib().rk_status_string(status).decode()
        raise RuntimeError(f"{what}: {msg}" if what else msg)


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def dt(t: torch.Tensor) -> int:
    try:
        return DTYPE_CODE[t.dtype]
    except KeyError:
        raise RuntimeError(f"unsupported dtype {t.dtype}") from None


def stream(device: torch.device | None = None):
    """The current torch stream of `device` as a raw hipStream_t (so calls are graph-capturable)."""
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def require_gpu(*ts: torch.Tensor):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("rumik HIP kernels need GPU tensors (there is no CPU path)")
