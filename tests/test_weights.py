"""The int4 checkpoint loader (rumik-fast_amd/engine/weights.py) on the CPU, against a synthetic checkpoint written in
the reference's format (`rumik-int4-g128-minmax-v1`, hf_card/README.md:46-53) by the exporter mapping
(modal_export_int4.py:48-70):

- every key maps where the reference loader puts it (engine/rumik_int4.py:88-114): w_in = rows [q | k | v | gate |
  up] exactly as the file holds them, w_o, w_down, LayerNorm weights (bf16 -> fp16 exactly), the int8 embedding,
  the audio head and its ids, the stop predictor; config fields from config.json (rumik_int4.py:70-78);
- the dequantized projections are within half a quantization step of the float weights (the format's
  w = code * scale + min, every element), and the int8 head rows within half a row step;
- malformed files are rejected naming the key: missing tensor, wrong dtype, wrong shape, </audio> id absent or
  repeated, layer_types of the wrong length.
"""
import json

import numpy as np
import pytest
import torch

import weights as W

CFG = {"num_hidden_layers": 2, "hidden_size": 256, "num_attention_heads": 2, "num_key_value_heads": 1,
       "head_dim": 128, "intermediate_size": 384, "layer_norm_eps": 1e-5, "rope_theta": 50000.0,
       "layer_types": ["sliding_attention", "full_attention"], "audio_end_token_id": 60}
VOCAB, NAUDIO = 64, 50


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    d = tmp_path_factory.mktemp("ckpt")
    st = W.synthetic_float_model(CFG, VOCAB, NAUDIO, seed=3, nz=32)
    ex = W.export_int4(st)
    W.save(d / "m.safetensors", ex, CFG)
    return d, st, ex


def test_config_mapping(ckpt):
    d, st, ex = ckpt
    cfg, w, extras = W.load(d / "m.safetensors", d / "config.json", device="cpu", S=128)
    assert (cfg.L, cfg.H, cfg.NH, cfg.NKV, cfg.HD, cfg.inter, cfg.S) == (2, 256, 2, 1, 128, 384, 128)
    assert cfg.sliding == [True, False] and cfg.rope_theta == 50000.0 and cfg.eps == 1e-5
    assert cfg.vocab == VOCAB and cfg.n_audio == NAUDIO
    assert extras["end_id"] == 60 and int((extras["audio_ids"] == 60).sum()) == 1


def test_keys_land_where_the_reference_loader_puts_them(ckpt):
    d, st, ex = ckpt
    cfg, w, extras = W.load(d / "m.safetensors", CFG, device="cpu")
    for i in range(2):
        p = f"model.layers.{i}."
        for j, suf in enumerate((".qweight", ".scale", ".min")):
            cat = torch.cat([ex[p + n + suf] for n in W.W_IN])
            assert torch.equal(w["w_in"][i][j], cat)
            assert torch.equal(w["w_o"][i][j], ex[p + "self_attn.o_proj" + suf])
            assert torch.equal(w["w_down"][i][j], ex[p + "mlp.down_proj" + suf])
        assert w["ln"][i].dtype == torch.float16
        assert torch.equal(w["ln"][i].float(), st[p + "input_layernorm.weight"].float())
    assert torch.equal(w["norm"].float(), st["model.norm.weight"].float())
    assert torch.equal(w["emb"][0], ex["model.embed_tokens.qweight"]) and w["emb"][0].dtype == torch.int8
    assert torch.equal(w["emb"][1], ex["model.embed_tokens.scale"]) and w["emb"][1].dtype == torch.float16
    assert torch.equal(extras["audio_ids"], st["head.audio_ids"])
    for k in W.STOP_KEYS:
        assert torch.equal(extras["stop"][k], st["stop_predictor." + k])
    assert w["w_in"][0][0].shape == (2 * 128 + 2 * 128 + 2 * 384, 128)


def _deq(q, s, m):
    codes = torch.stack([q & 0xF, q >> 4], -1).reshape(q.shape[0], -1).float()
    step = s.float().repeat_interleave(128, 1)
    return codes * step + m.float().repeat_interleave(128, 1), step


def test_dequantized_weights_within_half_a_step(ckpt):
    d, st, ex = ckpt
    cfg, w, extras = W.load(d / "m.safetensors", CFG, device="cpu")
    wf = torch.cat([st[f"model.layers.1.{n}.weight"].float() for n in W.W_IN])
    deq, step = _deq(*w["w_in"][1])
    # the min and scale are rounded to fp16, so allow their rounding on top of half a step
    slack = 0.5 * step + 16 * 2.0 ** -11 * (wf.abs() + step)
    assert bool(((deq - wf).abs() <= slack).all()), float(((deq - wf).abs() / step).max())
    hq, hs = w["head"]
    hw = st["head.audio_weight"].float()
    assert hq.dtype == torch.int8 and hs.dtype == torch.float16
    assert int(hq.abs().amax(1).min()) == 127  # every row reaches the full code range
    err = (hq.float() * hs.float()[:, None] - hw).abs()
    assert bool((err <= 0.5 * hs.float()[:, None] + 2.0 ** -11 * hw.abs().amax(1, keepdim=True)).all())
    # the reference's uint8 + 128 head with fp32 scale for the CUDA-path head GEMV
    u8, s32 = extras["head_u8"]
    assert u8.dtype == torch.uint8 and s32.dtype == torch.float32 and u8.shape[0] % 16 == 0


def _write(tmp_path, tensors, cfg=CFG):
    p = tmp_path / "bad.safetensors"
    W.save(p, tensors)
    return p, cfg


def test_malformed_checkpoints_are_rejected(ckpt, tmp_path):
    d, st, ex = ckpt
    bad = dict(ex)
    del bad["model.layers.1.mlp.up_proj.min"]
    with pytest.raises(W.CheckpointError, match="model.layers.1.mlp.up_proj.min"):
        W.load(*_write(tmp_path, bad), device="cpu")
    bad = dict(ex)
    bad["model.layers.0.self_attn.k_proj.scale"] = bad["model.layers.0.self_attn.k_proj.scale"].float()
    with pytest.raises(W.CheckpointError, match="k_proj.scale: dtype"):
        W.load(*_write(tmp_path, bad), device="cpu")
    bad = dict(ex)
    bad["model.layers.0.mlp.down_proj.qweight"] = bad["model.layers.0.mlp.down_proj.qweight"][:, :-1].contiguous()
    with pytest.raises(W.CheckpointError, match="down_proj.qweight: shape"):
        W.load(*_write(tmp_path, bad), device="cpu")
    bad = dict(ex)
    bad["head.audio_ids"] = torch.where(bad["head.audio_ids"] == 60, 0, bad["head.audio_ids"])
    with pytest.raises(W.CheckpointError, match="exactly once"):
        W.load(*_write(tmp_path, bad), device="cpu")
    p, _ = _write(tmp_path, ex)
    with pytest.raises(W.CheckpointError, match="layer_types"):
        W.load(p, dict(CFG, layer_types=["sliding_attention"]), device="cpu")
    with pytest.raises(W.CheckpointError, match="config"):
        W.load(d / "m.safetensors", None, device="cpu")


def test_file_is_plain_safetensors(ckpt):
    """the file carries the format name and nothing that needs unpickling (safetensors' header is JSON)"""
    d, st, ex = ckpt
    raw = (d / "m.safetensors").read_bytes()
    n = int.from_bytes(raw[:8], "little")
    header = json.loads(raw[8:8 + n])
    assert header["__metadata__"]["format"] == W.FORMAT
    assert set(header) - {"__metadata__"} == set(ex)
    assert np.dtype("uint8").itemsize == 1


def test_drop_in_quantize_is_bit_exact_with_the_oracle():
    """kernels/int4_gemv.quantize (torch, load time) writes exactly the codes, scales and mins of the pinned oracle
    (oracle.int4.quantize, reference kernels/int4_gemv.py:16-24) on seeded inputs: random weights at several
    scales, groups whose values sit exactly on rounding ties (half to even), constant groups (the 1e-8 clamp) and
    bf16 / fp16 inputs."""
    import int4_gemv
    from oracle import int4 as O
    g = torch.Generator().manual_seed(31)
    cases = [torch.randn(64, 1024, generator=g) * sc for sc in (1e-3, 0.05, 1.0, 300.0)]
    ties = (torch.randint(0, 31, (32, 512), generator=g).float() * 0.5)  # k / 2 on [0, 15]: every odd k is a tie
    ties[:, ::128] = 0.0
    ties[:, 1::128] = 15.0                                              # min 0, max 15: step exactly 1
    cases.append(ties)
    const = torch.full((8, 256), 0.37)
    const[4:] = -2.0
    cases.append(const)
    cases.append((torch.randn(16, 2048, generator=g) * 0.02).bfloat16())
    cases.append((torch.randn(16, 2048, generator=g) * 0.02).half())
    for w in cases:
        q, s, m = int4_gemv.quantize(w)
        oq, os_, om = O.quantize(w.float().numpy())
        assert np.array_equal(q.numpy(), oq)
        assert np.array_equal(s.numpy().view(np.uint16), os_.view(np.uint16))
        assert np.array_equal(m.numpy().view(np.uint16), om.view(np.uint16))
    # the tie case really exercised ties, both directions
    codes = O.unpack_int4(O.quantize(ties.numpy())[0])
    half = (ties.numpy() * 2).astype(int) % 2 == 1
    assert half.sum() > 1000 and set(np.unique(codes[half] % 2)) == {0}  # ties went to the even code
