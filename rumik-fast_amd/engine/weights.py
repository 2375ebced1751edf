"""The reference's int4 checkpoint (format `rumik-int4-g128-minmax-v1`) -> this build's decode engines.

Loader (reference engine/rumik_int4.py:88-114, with the int8 head of engine/rumik_fused.py:27-33): one safetensors
file opened with safetensors' loader (no pickle), per layer
  w_in   = rows [q | k | v | gate | up]  (qweight uint8 [N, K/2], scale / min fp16 [N, K/128]) -- one GEMV for the
           five projections that all multiply the same h (a parallel block)
  w_o, w_down, input_layernorm.weight
then model.norm.weight, the int8 embedding (model.embed_tokens.qweight / .scale), the audio head (bf16 rows
head.audio_weight + their token ids head.audio_ids) and the stop predictor (stop_predictor.{0,1,3}.{weight,bias}).
The head is quantized per row to int8 at load time (symmetric, scale = max|w| / 127, the reference's
quantize_int8_rows, cuda_gemv.py:234-242); the one-launch step takes it as int8 codes with an fp16 row scale.
LayerNorm weights are converted to fp16 (the engines' activation dtype; bf16 -> fp16 is exact for values within fp16
range, which is checked).

Config (reference engine/rumik_int4.py:70-78): the HF config.json fields num_hidden_layers, hidden_size,
num_attention_heads, num_key_value_heads, head_dim, intermediate_size, layer_norm_eps, rope_theta, layer_types
("sliding_attention" = RoPE), audio_end_token_id.

Exporter mapping (reference modal_export_int4.py:48-70, format in hf_card/README.md:46-53), used to write
synthetic checkpoints in the same layout: every 2-D `<proj>.weight` of a q/k/v/o/gate/up/down projection ->
`<proj>.{qweight, scale, min}` with the group-128 min-max quantizer (kernels/int4_gemv.py::quantize); the token
embedding -> per-row int8; everything else copied as-is.
"""
import json
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "kernels"))
import int4_gemv  # noqa: E402

FORMAT = "rumik-int4-g128-minmax-v1"
PROJ = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")
STOP_KEYS = ("0.weight", "0.bias", "1.weight", "1.bias", "3.weight", "3.bias")
W_IN = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "mlp.gate_proj", "mlp.up_proj")


class CheckpointError(ValueError):
    """A key is missing or has the wrong dtype / shape for the config."""


def config_from_hf(cfg: dict, S: int = 2048, vocab: int | None = None, n_audio: int | None = None):
    """decode.Config from the HF config.json fields the reference engine reads (rumik_int4.py:70-78)."""
    import decode
    L = int(cfg["num_hidden_layers"])
    types = cfg.get("layer_types")
    sliding = [t == "sliding_attention" for t in types] if types is not None else None
    if sliding is not None and len(sliding) != L:
        raise CheckpointError(f"layer_types has {len(sliding)} entries for {L} layers")
    kw = dict(L=L, H=int(cfg["hidden_size"]), NH=int(cfg["num_attention_heads"]),
              NKV=int(cfg["num_key_value_heads"]), HD=int(cfg["head_dim"]), inter=int(cfg["intermediate_size"]),
              S=S, eps=float(cfg.get("layer_norm_eps", 1e-5)), rope_theta=float(cfg.get("rope_theta", 10000.0)),
              sliding=sliding)
    if vocab is not None:
        kw["vocab"] = int(vocab)
    if n_audio is not None:
        kw["n_audio"] = int(n_audio)
    return decode.Config(**kw)


def int8_rows(w: torch.Tensor):
    """bf16 / fp32 rows [N, K] -> (int8 codes [N, K], fp16 scale [N]): symmetric per row, scale = max|w| / 127
    clamped to 1e-8, codes = round(w / scale) clamped to [-127, 127] (the reference's quantize_int8_rows without the
    +128 offset and row padding; the scale stored in fp16)."""
    wf = w.float()
    scale = torch.clamp(wf.abs().amax(dim=1) / 127.0, min=1e-8)
    codes = torch.clamp(torch.round(wf / scale[:, None]), -127, 127).to(torch.int8)
    return codes.contiguous(), scale.half().contiguous()


def _to_f16(t: torch.Tensor, name: str):
    if t.dtype == torch.float16:
        return t.contiguous()
    tf = t.float()
    if tf.abs().max() > 65504:
        raise CheckpointError(f"{name}: values outside the fp16 range")
    return tf.half().contiguous()


def _expect(t, name, dtype, shape):
    if t.dtype != dtype:
        raise CheckpointError(f"{name}: dtype {t.dtype}, expected {dtype}")
    if tuple(t.shape) != tuple(shape):
        raise CheckpointError(f"{name}: shape {tuple(t.shape)}, expected {tuple(shape)}")


def load(path, cfg_json=None, device="cuda", S: int = 2048):
    """Load an int4 checkpoint. `cfg_json`: the HF config (dict or path to config.json). Returns (cfg, weights,
    extras): `weights` in the layout decode.DecodeStep / decode.PersistentDecode take (as decode.random_weights
    builds it), `extras` = {audio_ids, end_id, stop (state dict), head_u8 (the reference's uint8 + 128 head with
    fp32 row scale, for cuda_gemv.gemv_int8_cuda), head_bf16}."""
    from safetensors import safe_open
    if cfg_json is None:
        raise CheckpointError("the HF config (config.json) is needed: layer count, heads, sizes, layer types")
    if not isinstance(cfg_json, dict):
        cfg_json = json.loads(Path(cfg_json).read_text())
    with safe_open(str(path), "pt", device="cpu") as f:
        keys = set(f.keys())

        def get(name):
            if name not in keys:
                raise CheckpointError(f"missing tensor {name}")
            return f.get_tensor(name)

        L, H = int(cfg_json["num_hidden_layers"]), int(cfg_json["hidden_size"])
        NH, NKV, HD = int(cfg_json["num_attention_heads"]), int(cfg_json["num_key_value_heads"]), int(cfg_json["head_dim"])
        inter = int(cfg_json["intermediate_size"])
        rows = {"self_attn.q_proj": NH * HD, "self_attn.k_proj": NKV * HD, "self_attn.v_proj": NKV * HD,
                "mlp.gate_proj": inter, "mlp.up_proj": inter, "self_attn.o_proj": H, "mlp.down_proj": H}
        cols = {"self_attn.o_proj": NH * HD, "mlp.down_proj": inter}

        def proj(name, key):
            N, K = rows[key], cols.get(key, H)
            q, s, m = get(name + ".qweight"), get(name + ".scale"), get(name + ".min")
            _expect(q, name + ".qweight", torch.uint8, (N, K // 2))
            _expect(s, name + ".scale", torch.float16, (N, K // 128))
            _expect(m, name + ".min", torch.float16, (N, K // 128))
            return q, s, m

        w = {"w_in": [], "w_o": [], "w_down": [], "ln": []}
        for i in range(L):
            p = f"model.layers.{i}."
            parts = [proj(p + k, k) for k in W_IN]
            w["w_in"].append(tuple(torch.cat([t[j] for t in parts]).contiguous().to(device) for j in range(3)))
            w["w_o"].append(tuple(t.to(device) for t in proj(p + "self_attn.o_proj", "self_attn.o_proj")))
            w["w_down"].append(tuple(t.to(device) for t in proj(p + "mlp.down_proj", "mlp.down_proj")))
            ln = get(p + "input_layernorm.weight")
            _expect(ln, p + "input_layernorm.weight", ln.dtype, (H,))
            w["ln"].append(_to_f16(ln, p + "input_layernorm.weight").to(device))
        norm = get("model.norm.weight")
        _expect(norm, "model.norm.weight", norm.dtype, (H,))
        w["norm"] = _to_f16(norm, "model.norm.weight").to(device)
        eq, es = get("model.embed_tokens.qweight"), get("model.embed_tokens.scale")
        _expect(eq, "model.embed_tokens.qweight", torch.int8, (eq.shape[0], H))
        _expect(es, "model.embed_tokens.scale", torch.float16, (eq.shape[0],))
        w["emb"] = (eq.contiguous().to(device), es.contiguous().to(device))
        hw, ids = get("head.audio_weight"), get("head.audio_ids")
        _expect(hw, "head.audio_weight", hw.dtype, (hw.shape[0], H))
        _expect(ids, "head.audio_ids", torch.int64, (hw.shape[0],))
        if int(ids.min()) < 0 or int(ids.max()) >= eq.shape[0]:
            raise CheckpointError("head.audio_ids: token ids outside the embedding table")
        w["head"] = tuple(t.to(device) for t in int8_rows(hw))
        stop = {}
        for k in STOP_KEYS:
            stop[k] = get("stop_predictor." + k).to(device)
    end_id = int(cfg_json["audio_end_token_id"])
    if int((ids == end_id).sum()) != 1:
        raise CheckpointError("head.audio_ids must hold audio_end_token_id exactly once")
    import cuda_gemv
    extras = {"audio_ids": ids.to(device), "end_id": end_id, "stop": stop, "head_bf16": hw.to(device),
              "head_u8": tuple(t.to(device) for t in cuda_gemv.quantize_int8_rows(hw.float()))}
    cfg = config_from_hf(cfg_json, S=S, vocab=eq.shape[0], n_audio=hw.shape[0])
    return cfg, w, extras


def export_int4(state: dict) -> dict:
    """A float state dict (reference model key names) -> the int4 checkpoint's tensors (modal_export_int4.py:48-70):
    q/k/v/o/gate/up/down `<proj>.weight` -> `<proj>.{qweight, scale, min}`; `model.embed_tokens.weight` -> per-row
    int8 `.qweight` + fp16 `.scale`; everything else (norms, head.audio_*, stop_predictor.*) as-is."""
    out = {}
    for name, t in state.items():
        base = name[:-len(".weight")] if name.endswith(".weight") else None
        if base and base.split(".")[-1] in PROJ and t.dim() == 2:
            out[base + ".qweight"], out[base + ".scale"], out[base + ".min"] = int4_gemv.quantize(t)
        elif name == "model.embed_tokens.weight":
            out["model.embed_tokens.qweight"], out["model.embed_tokens.scale"] = int8_rows(t)
        else:
            out[name] = t.contiguous()
    return out


def save(path, tensors: dict, cfg_json: dict | None = None):
    """Write tensors as one safetensors file (and the HF config next to it as config.json when given)."""
    from safetensors.torch import save_file
    save_file({k: v.contiguous().cpu() for k, v in tensors.items()}, str(path), metadata={"format": FORMAT})
    if cfg_json is not None:
        (Path(path).parent / "config.json").write_text(json.dumps(cfg_json))


def synthetic_float_model(cfg_json: dict, vocab: int, n_audio: int, seed: int = 0, nz: int = 512):
    """A random float state dict with the reference model's key names and shapes (for tests and load timing)."""
    if n_audio > vocab:
        raise ValueError("the audio rows are token ids of the vocabulary: n_audio <= vocab")
    g = torch.Generator().manual_seed(seed)
    L, H = int(cfg_json["num_hidden_layers"]), int(cfg_json["hidden_size"])
    NH, NKV, HD = int(cfg_json["num_attention_heads"]), int(cfg_json["num_key_value_heads"]), int(cfg_json["head_dim"])
    inter = int(cfg_json["intermediate_size"])
    r = lambda *s, scale=1.0: (torch.randn(*s, generator=g) * scale).bfloat16()  # noqa: E731
    st = {}
    for i in range(L):
        p = f"model.layers.{i}."
        for name, (n, k) in {"self_attn.q_proj": (NH * HD, H), "self_attn.k_proj": (NKV * HD, H),
                             "self_attn.v_proj": (NKV * HD, H), "self_attn.o_proj": (H, NH * HD),
                             "mlp.gate_proj": (inter, H), "mlp.up_proj": (inter, H),
                             "mlp.down_proj": (H, inter)}.items():
            st[p + name + ".weight"] = r(n, k, scale=k ** -0.5)
        st[p + "input_layernorm.weight"] = (1 + 0.1 * torch.randn(H, generator=g)).bfloat16()
    st["model.norm.weight"] = (1 + 0.1 * torch.randn(H, generator=g)).bfloat16()
    st["model.embed_tokens.weight"] = r(vocab, H, scale=0.5)
    ids = torch.randperm(vocab, generator=g)[:n_audio].to(torch.int64)
    ids[-1] = int(cfg_json["audio_end_token_id"])
    ids[:-1][ids[:-1] == ids[-1]] = (ids[-1] + 1) % vocab
    st["head.audio_weight"] = r(n_audio, H, scale=H ** -0.5)
    st["head.audio_ids"] = ids
    st["stop_predictor.0.weight"] = torch.ones(H).bfloat16()
    st["stop_predictor.0.bias"] = torch.zeros(H).bfloat16()
    st["stop_predictor.1.weight"] = r(nz, H, scale=H ** -0.5)
    st["stop_predictor.1.bias"] = torch.zeros(nz).bfloat16()
    st["stop_predictor.3.weight"] = r(1, nz, scale=nz ** -0.5)
    st["stop_predictor.3.bias"] = torch.tensor([-4.0]).bfloat16()
    return st
