"""int4 format maths and the generic batch-1 GEMV: drop-in for the reference's kernels/int4_gemv.py.

Layout ("rumik-int4-g128-minmax-v1", reference kernels/int4_gemv.py:1-4, modal_export_int4.py:48-59):
  qweight uint8 [N, K/2], low nibble = even column; scale, min fp16 [N, K/G]; w = code * scale + min.

quantize / dequantize are load-time format utilities (torch ops on the tensors' own device); the GEMV itself is the
HIP kernel of cuda_gemv.gemv_int4_cuda. The reference's Triton variants v2-v5 (kernels/int4_gemv.py:99-276) were
negative results kept for its write-up and have no counterpart here.
"""
import torch

try:
    from . import cuda_gemv as _cg
except ImportError:
    import cuda_gemv as _cg

G = 128


def quantize(w: torch.Tensor, group: int = G):
    """[N, K] (any float dtype) -> (qweight uint8 [N, K/2], scale fp16 [N, K/group], min fp16 [N, K/group]).
    Round-to-nearest min/max quantization per group of `group` columns, as the exporter writes it
    (reference kernels/int4_gemv.py:16-24): scale = (max - min) / 15 clamped to >= 1e-8, code = round((w - min) /
    scale) clamped to [0, 15] (torch.round: half to even), scale and min stored as fp16."""
    n, k = w.shape
    if k % group:
        raise ValueError(f"K={k} is not a multiple of the group size {group}")
    grp = w.float().reshape(n, k // group, group)
    lo = grp.amin(dim=-1, keepdim=True)
    step = torch.clamp((grp.amax(dim=-1, keepdim=True) - lo) / 15, min=1e-8)
    code = torch.clamp(torch.round((grp - lo) / step), 0, 15).to(torch.uint8).reshape(n, k)
    packed = code[:, 0::2] | (code[:, 1::2] << 4)
    return packed.contiguous(), step.half().reshape(n, -1).contiguous(), lo.half().reshape(n, -1).contiguous()


def dequantize(q, s, m, group: int = G):
    """(qweight, scale, min) -> fp32 [N, K]: w = code * scale + min (reference kernels/int4_gemv.py:27-30)."""
    n = q.shape[0]
    code = torch.empty(n, q.shape[1] * 2, device=q.device, dtype=torch.float32)
    code[:, 0::2] = (q & 0xF).float()
    code[:, 1::2] = (q >> 4).float()
    code = code.reshape(n, -1, group)
    return (code * s.float().unsqueeze(-1) + m.float().unsqueeze(-1)).reshape(n, -1)


def gemv_int4(x: torch.Tensor, q: torch.Tensor, s: torch.Tensor, m: torch.Tensor, out: torch.Tensor | None = None):
    """x [K] (bf16/fp16) -> y [N] in x's dtype (reference contract kernels/int4_gemv.py:84-96)."""
    if x.numel() != q.shape[1] * 2 or x.numel() % G:
        raise AssertionError("x.numel() must equal K and K % 128 == 0")
    return _cg.gemv_int4_cuda(x, q, s, m, out=out)
