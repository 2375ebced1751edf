"""int4-weight matrix product for the prefill on MI355X: drop-in for the reference's kernels/mm_int4.py.

Y[T, N] = X[T, K] @ W^T with W in the int4 g128 layout (qweight uint8 [N, K/2], fp16 scale / min [N, K/128]),
computed by a gfx950 kernel (csrc/mm_int4.hip) on the matrix cores: codes are dequantized exactly to fp16 inside
the kernel (weights never leave int4 in HBM), products accumulate in fp32, and each 128-column group's affine
(scale * dot + min * rowsum) is applied in fp32 — the algebra of the reference's _mm_int4 (kernels/mm_int4.py:8-11).

Same names and arguments as the reference (mm_int4(x, q, s, m, BM=None, BN=64, num_warps=4, num_stages=3), warmup,
G). The Triton tiling knobs BM / BN / num_warps / num_stages are accepted and validated but do not select anything:
the HIP kernel picks its own tiles (and, for shapes with few output tiles, a split over K whose fp32 partial sums
go to a workspace allocated per call from torch's caching allocator, like y). Extra keyword `out=` writes into a
preallocated [T, N] tensor (graph-capturable). The output dtype is x's dtype (bf16 for the reference engine, as before).
"""
import torch

try:
    from . import _hiplib as H
except ImportError:
    import _hiplib as H

G = 128


def mm_int4(x, q, s, m, BM=None, BN=64, num_warps=4, num_stages=3, out=None):
    """x [T, K] (fp16/bf16) -> y [T, N] = x @ dequantize(q, s, m)^T (reference kernels/mm_int4.py:59-73)."""
    for knob in (BN, num_warps, num_stages) + ((BM,) if BM is not None else ()):
        if not isinstance(knob, int) or knob <= 0:
            raise AssertionError("tiling knobs must be positive integers")
    x = x.contiguous()
    if x.dim() != 2 or q.dim() != 2 or q.dtype != torch.uint8:
        raise AssertionError("x must be [T, K] and q uint8 [N, K/2]")
    T, K = x.shape
    N = q.shape[0]
    if q.shape[1] * 2 != K or K % G:
        raise AssertionError("q.shape[1] * 2 must equal K and K % 128 == 0")
    if s.dtype != torch.float16 or m.dtype != torch.float16 or s.numel() != N * (K // G) or m.numel() != N * (K // G):
        raise AssertionError("scale / min must be fp16 [N, K/128]")
    if not (s.is_contiguous() and m.is_contiguous() and q.is_contiguous()):
        raise AssertionError("q, scale and min must be contiguous")
    y = out if out is not None else torch.empty(T, N, device=x.device, dtype=x.dtype)
    if y.shape != (T, N) or y.stride(1) != 1:
        raise AssertionError("out must be [T, N] with unit column stride")
    H.require_gpu(x, q, s, m, y)
    L = H.lib()
    nws = L.rk_mm_int4_workspace_bytes(T, N, K)
    # split-K partial sums for shapes with few output tiles (allocated per call like y, from torch's cache)
    ws = torch.empty(nws, device=x.device, dtype=torch.uint8) if nws else None
    st = L.rk_mm_int4_g128_ws(H.ptr(x), H.dt(x), x.stride(0), H.ptr(q), H.ptr(s), H.ptr(m), H.ptr(y), H.dt(y),
                              y.stride(0), T, N, K, H.ptr(ws), nws, H.stream(x.device))
    H.check(st, "mm_int4")
    return y


def warmup(shapes, max_T=512):
    """Run every (N, K) shape once per kernel plan a prompt of up to max_T rows can select (reference
    kernels/mm_int4.py:49-56 runs its Triton buckets; there is no JIT here, this loads the code objects and touches
    every plan: the 128 x 128 and 64 x 64 tile kernels, with and without the split over K)."""
    for n, k in shapes:
        q = torch.zeros(n, k // 2, device="cuda", dtype=torch.uint8)
        s = torch.zeros(n, k // G, device="cuda", dtype=torch.float16)
        for T in plan_lengths(n, k, max_T):
            mm_int4(torch.zeros(T, k, device="cuda", dtype=torch.bfloat16), q, s, s)
    torch.cuda.synchronize()


def plan_lengths(n, k, max_T=512):
    """The shortest prompt length in [1, max_T] for each distinct kernel plan of an (N, K) product."""
    first = {}
    for T in range(1, max_T + 1):
        first.setdefault(H.mm_plan(T, n, k, use_workspace=True), T)
    return sorted(first.values())
