"""Batch-1 GEMVs of the decode step on MI355X: drop-in for the reference's kernels/cuda_gemv.py.

Same names and arguments as the reference module (kernels/cuda_gemv.py:222-249): gemv_int4_cuda, gemv_int8_cuda,
quantize_int8_rows and the SHAPE table, so engine/rumik_fused.py:9 can import them unchanged. The work is done by
hand-written gfx950 kernels in librumik_hip.so (csrc/gemv_int4.hip, csrc/gemv_int8.hip), launched on the current
torch stream with no allocation when `out` is given, so the calls can be captured in a hipGraph.

Differences from the reference, all widening what is accepted:
  * x may be fp16 or bf16 (the reference reads bf16 only); y is x's dtype unless `out` says otherwise
    (for the reference's bf16 x that is bf16, as before); out may also be fp32;
  * any N (the reference needs N % (warps*rows) == 0) and, for int8, any K % 16 == 0 (reference: K % 512 == 0);
  * int8 codes may be the reference's uint8 = int8 + 128 or plain int8; the row scale fp32 or fp16.
Errors keep the reference's messages: RuntimeError("shape"), RuntimeError("unsupported block shape").
"""
import torch

try:
    from . import _hiplib as H
except ImportError:  # imported with this directory on sys.path, as the reference engine does
    import _hiplib as H

G = 128

# block shape (waves per block, rows per wave) per (N, K); an empty table means the library's tuned defaults.
# Same role as the reference's SHAPE (kernels/cuda_gemv.py:222-223).
SHAPE = {}


def _check_int4(x, q, s, m, y):
    H.require_gpu(x, q, s, m, y)
    if q.dim() != 2 or q.dtype != torch.uint8:
        raise RuntimeError("shape")
    N, K = q.shape[0], q.shape[1] * 2
    if K % G or x.numel() != K or y.numel() < N:
        raise RuntimeError("shape")
    if s.dtype != torch.float16 or m.dtype != torch.float16 or s.numel() != N * (K // G) or m.numel() != N * (K // G):
        raise RuntimeError("shape")
    for t in (x, q, s, m, y):
        if not t.is_contiguous():
            raise RuntimeError("shape")
    return N, K


def gemv_int4_cuda(x, q, s, m, out=None, warps=None, rows=None):
    """int4 g128 GEMV: x [K] (fp16/bf16) -> y [N] = dequant(q, s, m) @ x, fp32 accumulation.
    Reference contract: kernels/cuda_gemv.py:226-231 (x bf16 [K] -> y bf16 [N])."""
    y = out if out is not None else torch.empty(q.shape[0], device=x.device, dtype=x.dtype)
    N, K = _check_int4(x, q, s, m, y)
    w, r = SHAPE.get((N, K), (0, 0))
    st = H.lib().rk_gemv_int4_g128(H.ptr(x), H.dt(x), H.ptr(q), H.ptr(s), H.ptr(m), H.ptr(y), H.dt(y), N, K,
                                   int(warps or w), int(rows or r), H.stream(x.device))
    H.check(st)
    return y


def gemv_int4_pair_cuda(x1, w1, x2, w2, out1=None, out2=None):
    """Two independent int4 g128 GEMVs in one launch: (dequant(w1) @ x1, dequant(w2) @ x2), w = (q, s, m); the
    decode layer's o and down projections (the reference's two gemv_int4 calls, engine/rumik_fused.py:115-116).
    Same checks and outputs as two gemv_int4_cuda calls."""
    y1 = out1 if out1 is not None else torch.empty(w1[0].shape[0], device=x1.device, dtype=x1.dtype)
    y2 = out2 if out2 is not None else torch.empty(w2[0].shape[0], device=x2.device, dtype=x2.dtype)
    N1, K1 = _check_int4(x1, *w1, y1)
    N2, K2 = _check_int4(x2, *w2, y2)
    st = H.lib().rk_gemv_int4_g128_pair(H.ptr(x1), H.dt(x1), H.ptr(w1[0]), H.ptr(w1[1]), H.ptr(w1[2]), H.ptr(y1),
                                        H.dt(y1), N1, K1, H.ptr(x2), H.dt(x2), H.ptr(w2[0]), H.ptr(w2[1]),
                                        H.ptr(w2[2]), H.ptr(y2), H.dt(y2), N2, K2, H.stream(x1.device))
    H.check(st)
    return y1, y2


def gemv_int4_silu_cuda(x, q, s, m, n_plain, out=None, act=None):
    """The engine's w_in projection with SiLU(gate) * up fused: q = [n_plain rows | inter gate rows | inter up rows]
    (int4 g128) -> (y [n_plain] or None, act [inter]), equal to gemv_int4_cuda followed by act = silu(g) * u on the
    rounded outputs (the MLP part of the reference's post, engine/fused.py:44-84). Outputs in x's dtype by default."""
    if q.dim() != 2 or q.dtype != torch.uint8 or n_plain < 0 or q.shape[0] <= n_plain or (q.shape[0] - n_plain) % 2:
        raise RuntimeError("shape")
    N, K = q.shape[0], q.shape[1] * 2
    inter = (N - n_plain) // 2
    a = act if act is not None else torch.empty(inter, device=x.device, dtype=x.dtype)
    y = out if out is not None else (torch.empty(n_plain, device=x.device, dtype=a.dtype) if n_plain else None)
    H.require_gpu(x, q, s, m, a, y)
    if K % G or x.numel() != K or a.numel() < inter or (n_plain and (y.numel() < n_plain or y.dtype != a.dtype)):
        raise RuntimeError("shape")
    if s.dtype != torch.float16 or m.dtype != torch.float16 or s.numel() != N * (K // G) or m.numel() != N * (K // G):
        raise RuntimeError("shape")
    for t in (x, q, s, m, a) + ((y,) if y is not None else ()):
        if not t.is_contiguous():
            raise RuntimeError("shape")
    st = H.lib().rk_gemv_int4_g128_silu(H.ptr(x), H.dt(x), H.ptr(q), H.ptr(s), H.ptr(m), H.ptr(y), H.ptr(a),
                                        H.dt(a), n_plain, inter, K, 0, H.stream(x.device))
    H.check(st)
    return y, a


class LayerProjections:
    """One decoder layer's four decode projections in one launch (rk_gemv_int4_g128_layer): w_in over x with
    act = silu(gate) * up fused, o over ob, and down over that act -- the reference's gemv(h, w_in), the MLP part of
    post, gemv(ob, w_o) and gemv(act, w_down) (engine/rumik_fused.py:100-101, 115-116) when ob is already at hand.
    Owns the zeroed workspace the launch's exchange needs (one launch at a time per instance; hipGraph replays of a
    captured call need no reset). Outputs as gemv_int4_silu_cuda and gemv_int4_pair_cuda give them.

        lp = LayerProjections(n_plain, inter, device)
        y_plain, act, y_o, y_down = lp(x, w_in, ob, w_o, w_down)
    """

    def __init__(self, n_plain, inter, device):
        self.n_plain, self.inter = int(n_plain), int(inter)
        nbytes = H.lib().rk_gemv_int4_g128_layer_ws_bytes(self.inter)
        if nbytes == 0:
            raise RuntimeError("shape")
        self.ws = torch.zeros(nbytes // 4, device=device, dtype=torch.int32)

    def status(self):
        """The workspace's status word: 0, or bit 0 once a launch's exchange ran out of time."""
        return int(self.ws[0].item())

    def __call__(self, x, w_in, ob, w_o, w_down, out=None, act=None, out_o=None, out_d=None):
        n_plain, inter = self.n_plain, self.inter
        q, s, m = w_in
        Hd = x.numel()
        dt = x.dtype
        a = act if act is not None else torch.empty(inter, device=x.device, dtype=dt)
        y = out if out is not None else (torch.empty(n_plain, device=x.device, dtype=a.dtype) if n_plain else None)
        yo = out_o if out_o is not None else torch.empty(Hd, device=x.device, dtype=a.dtype)
        yd = out_d if out_d is not None else torch.empty(Hd, device=x.device, dtype=a.dtype)
        H.require_gpu(x, q, s, m, a, y)
        if q.dim() != 2 or q.dtype != torch.uint8 or q.shape[0] != n_plain + 2 * inter or q.shape[1] * 2 != Hd:
            raise RuntimeError("shape")
        ng = Hd // G
        if s.dtype != torch.float16 or m.dtype != torch.float16 or s.numel() != q.shape[0] * ng or m.numel() != s.numel():
            raise RuntimeError("shape")
        if not all(t.is_contiguous() for t in (x, q, s, m, a)):
            raise RuntimeError("shape")
        if _check_int4(ob, *w_o, yo) != (Hd, Hd) or _check_int4(a, *w_down, yd) != (Hd, inter):
            raise RuntimeError("shape")
        if ob.dtype != dt or any(t.dtype != a.dtype for t in (yo, yd) + ((y,) if y is not None else ())):
            raise RuntimeError("dtype")
        if a.numel() != inter or (y is not None and (y.numel() < n_plain or not y.is_contiguous())):
            raise RuntimeError("shape")
        st = H.lib().rk_gemv_int4_g128_layer(
            H.ptr(x), H.ptr(ob), H.dt(x), H.ptr(q), H.ptr(s), H.ptr(m), H.ptr(w_o[0]), H.ptr(w_o[1]),
            H.ptr(w_o[2]), H.ptr(w_down[0]), H.ptr(w_down[1]), H.ptr(w_down[2]), H.ptr(y), H.ptr(a), H.ptr(yo),
            H.ptr(yd), H.dt(a), n_plain, inter, Hd, H.ptr(self.ws), self.ws.numel() * 4, H.stream(x.device))
        H.check(st)
        return y, a, yo, yd


def quantize_int8_rows(w, pad_to=16):
    """[N, K] -> (uint8 [N', K] = int8 + 128, fp32 scale [N']), rows zero-padded to a multiple of pad_to.
    Symmetric per row: w ~ (q - 128) * scale, scale = max|w| / 127 (reference kernels/cuda_gemv.py:234-242)."""
    n, k = w.shape
    n_pad = -(-n // pad_to) * pad_to
    wf = torch.zeros(n_pad, k, device=w.device, dtype=torch.float32)
    wf[:n] = w.float()
    scale = torch.clamp(wf.abs().amax(dim=1) / 127.0, min=1e-8)
    codes = torch.clamp(torch.round(wf / scale[:, None]), -127, 127)
    return (codes + 128).to(torch.uint8).contiguous(), scale.contiguous()


def gemv_int8_cuda(x, q, s, out=None):
    """int8 per-row GEMV: x [K] -> y [N] = s * (codes @ x). codes are uint8 = int8 + 128 (reference layout) or
    int8. y defaults to bf16 as in the reference (kernels/cuda_gemv.py:245-249); pass an fp32 `out` for logits."""
    y = out if out is not None else torch.empty(q.shape[0], device=x.device, dtype=torch.bfloat16)
    H.require_gpu(x, q, s, y)
    if q.dim() != 2 or q.dtype not in (torch.uint8, torch.int8):
        raise RuntimeError("shape")
    N, K = q.shape
    if x.numel() != K or s.numel() != N or y.numel() < N or K % 16:
        raise RuntimeError("shape")
    if s.dtype not in (torch.float32, torch.float16):
        raise RuntimeError("unsupported dtype")
    for t in (x, q, s, y):
        if not t.is_contiguous():
            raise RuntimeError("shape")
    kind = H.Q_U8 if q.dtype == torch.uint8 else H.Q_S8
    st = H.lib().rk_gemv_int8_rows(H.ptr(x), H.dt(x), H.ptr(q), kind, H.ptr(s), H.dt(s), H.ptr(y), H.dt(y), N, K,
                                   H.stream(x.device))
    H.check(st)
    return y
