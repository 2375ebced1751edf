"""Decode-step glue on MI355X: the reference's engine/fused.py kernels as calls into librumik_hip.so.

Same kernel names, argument order and launch form as the reference (engine/fused.py, launched from
engine/rumik_fused.py:99-119): `fused.post[(grid,)](y, pos, cos, sin, kc, vc, q, act, S, INTER, NH=..., NKV=...,
HD=..., ROPE=..., BLOCK=..., num_warps=...)`. The launch grid and the Triton tuning arguments (BLOCK, BT,
num_warps, PV_BF16) are accepted and ignored: each HIP wrapper picks its own launch shape. The kernels can also be
called without a grid (`fused.post(...)`). Every call is asynchronous on the current torch stream, reads `pos` /
`tok` from device memory and allocates nothing (except `attn`'s one-time workspace), so a whole decode step can be
captured in one hipGraph. Activations are fp16 or bf16; the KV cache of a layer is [NKV, S, HD] in the activation
dtype; cos / sin tables are [S, HD] in the activation dtype.
"""
import functools
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "kernels"))
import _hiplib as HL  # noqa: E402  (not H: the reference's kernels take an H= keyword)


class _Kernel:
    """`kernel[grid](...)` as in the reference's Triton launches, or a plain call."""

    def __init__(self, fn):
        self._fn = fn
        functools.update_wrapper(self, fn)

    def __getitem__(self, grid):
        return self._fn

    def __call__(self, *args, **kwargs):
        return self._fn(*args, **kwargs)


def _s(t):
    return HL.stream(t.device)


def _check_h(x, Hsize):
    if Hsize is not None and Hsize != x.numel():
        raise AssertionError(f"H={Hsize} does not match the vector length {x.numel()}")


@_Kernel
def embed_ln(tok, emb_q, emb_s, ln_w, x, h, eps, H=None, num_warps=None):
    """x = dt(emb_q[tok] * emb_s[tok]); h = LayerNorm(x) * ln_w (reference engine/fused.py:16-30)."""
    _check_h(x, H)
    HL.check(HL.lib().rk_embed_ln(HL.ptr(tok), HL.ptr(emb_q), HL.ptr(emb_s), HL.ptr(ln_w), HL.ptr(x),
                                      HL.ptr(h), HL.dt(x), x.numel(), float(eps), _s(x)), "embed_ln")


@_Kernel
def add_ln(x, a, b, ln_w, h, eps, H=None, num_warps=None):
    """x = dt(x + a + b) in fp32; h = LayerNorm(x) * ln_w (reference engine/fused.py:33-48); b may be None."""
    _check_h(x, H)
    HL.check(HL.lib().rk_add_ln(HL.ptr(x), HL.ptr(a), HL.ptr(b), HL.ptr(ln_w), HL.ptr(h), HL.dt(x),
                                    x.numel(), float(eps), _s(x)), "add_ln")


@_Kernel
def post(y, pos, cos, sin, kc, vc, q, act, S, INTER, NH, NKV, HD, ROPE, BLOCK=None, num_warps=None):
    """RoPE (q, k), K/V cache write at pos, act = silu(gate) * up (reference engine/fused.py:51-90).
    kc / vc: this layer's cache [NKV, S, HD]."""
    if kc.shape[1] != S or INTER * 2 + (NH + 2 * NKV) * HD != y.numel():
        raise RuntimeError("shape")
    HL.check(HL.lib().rk_post(HL.ptr(y), HL.ptr(pos), HL.ptr(cos), HL.ptr(sin), HL.ptr(kc),
                                  HL.ptr(vc), HL.ptr(q), HL.ptr(act), HL.dt(y), NH, NKV, HD, S, INTER,
                                  int(bool(ROPE)), _s(y)), "post")


@_Kernel
def attn_split(q, kc, vc, pos, po, pm, pl, S, scale, REP, HD, NSPLIT, BT=None, num_warps=None, PV_BF16=None):
    """Flash-decoding partials (m, l, acc) per query head and split (reference engine/fused.py:127-171).
    PV_BF16 (the reference's bf16 p.V product) is accepted; p.V is computed in fp32 here."""
    NKV = kc.shape[0]
    if kc.shape[1] != S:
        raise RuntimeError("shape")
    HL.check(HL.lib().rk_attn_split(HL.ptr(q), HL.ptr(kc), HL.ptr(vc), HL.ptr(pos), HL.ptr(po),
                                        HL.ptr(pm), HL.ptr(pl), HL.dt(q), REP * NKV, NKV, HD, S, NSPLIT,
                                        float(scale), _s(q)), "attn_split")


@_Kernel
def attn_combine(po, pm, pl, pos, o, HD, NSPLIT, BT=None, num_warps=None):
    """Merge the split partials into the attention output (reference engine/fused.py:173-190)."""
    HL.check(HL.lib().rk_attn_combine(HL.ptr(po), HL.ptr(pm), HL.ptr(pl), HL.ptr(pos), HL.ptr(o),
                                          HL.dt(o), po.shape[0], HD, NSPLIT, _s(o)), "attn_combine")


_attn_ws = {}


@_Kernel
def attn(q, kc, vc, pos, o, S, scale, REP, HD, BT=None, num_warps=None):
    """Unsplit decode attention (reference engine/fused.py:92-125): one split over all slots, then the merge.
    Its fp32 workspace is allocated on the first call per (device, heads) — before graph capture, as the
    reference's warm-up does — and reused afterwards."""
    import torch
    NH = REP * kc.shape[0]
    key = (o.device, NH, HD)
    if key not in _attn_ws:
        _attn_ws[key] = (torch.empty(NH, 1, HD, dtype=torch.float32, device=o.device),
                         torch.empty(NH, 1, dtype=torch.float32, device=o.device),
                         torch.empty(NH, 1, dtype=torch.float32, device=o.device))
    po, pm, pl = _attn_ws[key]
    attn_split(q, kc, vc, pos, po, pm, pl, S, scale, REP=REP, HD=HD, NSPLIT=1)
    attn_combine(po, pm, pl, pos, o, HD=HD, NSPLIT=1)


def silu_mul(gate_up, act, inter):
    """act = silu(gate) * up for gate_up = [gate | up]."""
    HL.check(HL.lib().rk_silu_mul(HL.ptr(gate_up), HL.ptr(act), HL.dt(act), inter, _s(act)), "silu_mul")


def pos_advance(pos):
    """pos += 1 on the device (reference engine/rumik_fused.py:120)."""
    HL.check(HL.lib().rk_pos_advance(HL.ptr(pos), _s(pos)), "pos_advance")

