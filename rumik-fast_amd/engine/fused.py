"""Decode-step glue on MI355X: the reference's engine/fused.py kernels as Python calls into librumik_hip.so.

Same kernel names and the same tensors as the reference (engine/fused.py): embed_ln, post, attn_split,
attn_combine, add_ln — called as functions (no Triton launch grids); every call is asynchronous on the current
torch stream, reads `pos` / `tok` from device memory and allocates nothing, so a whole decode step can be captured
in one hipGraph. Activations are fp16 or bf16; the KV cache of a layer is [NKV, S, HD] in the activation dtype.
"""
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "kernels"))
import _hiplib as H  # noqa: E402


def _s(t):
    return H.stream(t.device)


def embed_ln(tok, emb_q, emb_s, ln_w, x, h, eps):
    """x = dt(emb_q[tok] * emb_s[tok]); h = LayerNorm(x) * ln_w (reference engine/fused.py:16-27)."""
    H.check(H.lib().rk_embed_ln(H.ptr(tok), H.ptr(emb_q), H.ptr(emb_s), H.ptr(ln_w), H.ptr(x), H.ptr(h), H.dt(x),
                                x.numel(), float(eps), _s(x)), "embed_ln")


def add_ln(x, a, b, ln_w, h, eps):
    """x = dt(x + a + b) in fp32; h = LayerNorm(x) * ln_w (reference engine/fused.py:30-41); b may be None."""
    H.check(H.lib().rk_add_ln(H.ptr(x), H.ptr(a), H.ptr(b), H.ptr(ln_w), H.ptr(h), H.dt(x), x.numel(), float(eps),
                              _s(x)), "add_ln")


def post(y, pos, cos, sin, kc, vc, q_out, act, NH, NKV, HD, inter, rope):
    """RoPE (q, k), K/V cache write at pos, act = silu(gate) * up (reference engine/fused.py:44-84).
    kc / vc: this layer's cache [NKV, S, HD]."""
    S = kc.shape[1]
    H.check(H.lib().rk_post(H.ptr(y), H.ptr(pos), H.ptr(cos), H.ptr(sin), H.ptr(kc), H.ptr(vc), H.ptr(q_out),
                            H.ptr(act), H.dt(y), NH, NKV, HD, S, inter, int(bool(rope)), _s(y)), "post")


def attn_split(q, kc, vc, pos, po, pm, pl, NH, NKV, HD, nsplit, scale):
    """Flash-decoding partials (m, l, acc) per query head and split (reference engine/fused.py:120-169)."""
    S = kc.shape[1]
    H.check(H.lib().rk_attn_split(H.ptr(q), H.ptr(kc), H.ptr(vc), H.ptr(pos), H.ptr(po), H.ptr(pm), H.ptr(pl),
                                  H.dt(q), NH, NKV, HD, S, nsplit, float(scale), _s(q)), "attn_split")


def attn_combine(po, pm, pl, pos, out, NH, HD, nsplit):
    """Merge the split partials into the attention output (reference engine/fused.py:172-187)."""
    H.check(H.lib().rk_attn_combine(H.ptr(po), H.ptr(pm), H.ptr(pl), H.ptr(pos), H.ptr(out), H.dt(out), NH, HD,
                                    nsplit, _s(out)), "attn_combine")


def silu_mul(gate_up, act, inter):
    """act = silu(gate) * up for gate_up = [gate | up]."""
    H.check(H.lib().rk_silu_mul(H.ptr(gate_up), H.ptr(act), H.dt(act), inter, _s(act)), "silu_mul")


def pos_advance(pos):
    """pos += 1 on the device (reference engine/rumik_fused.py:120)."""
    H.check(H.lib().rk_pos_advance(H.ptr(pos), _s(pos)), "pos_advance")
