"""Local MLX-format checkpoints for the target (the on-disk format the reference loads through
mlx_lm.load, src/mlx_dspark/load.py:314-351).

A checkpoint directory holds ``config.json`` and ``model*.safetensors``. Each linear layer of a
quantized MLX checkpoint is three tensors: ``<name>.weight`` uint32 [N, K * bits / 32] (four
8-bit or eight 4-bit codes per word, lowest bits first), ``<name>.scales`` and
``<name>.biases`` [N, K/64] (w = s * q + b, group 64); ``config.json["quantization"]`` names
the bits (8 or 4) and group size. Unquantized checkpoints (bf16/f32 ``<name>.weight`` [N, K])
are quantized to W8 on load. The tensors are
read once, the q/k/v rows stacked into the fused projection and gate/up paired, and every
matrix repacked into the engine's tiled layout (dsk_w8_repack).

Key names follow mlx_lm's qwen3 module (the public Qwen3 layout): ``model.embed_tokens``,
``model.layers.<i>.self_attn.{q,k,v,o}_proj``, ``.self_attn.{q,k}_norm``,
``.mlp.{gate,up,down}_proj``, ``.input_layernorm``, ``.post_attention_layernorm``,
``model.norm`` and, when untied, ``lm_head``.
"""

from __future__ import annotations

import json
import os
from pathlib import Path

import torch

from .ops import W8Table, W8Weight
from .qwen3 import LayerWeights, Qwen3W8, TargetArgs

_ARG_KEYS = ("hidden_size", "num_hidden_layers", "intermediate_size", "num_attention_heads", "num_key_value_heads",
             "vocab_size", "rms_norm_eps", "rope_theta", "tie_word_embeddings", "max_position_embeddings")


def is_checkpoint_dir(path) -> bool:
    p = Path(str(path))
    return p.is_dir() and (p / "config.json").is_file() and any(p.glob("*.safetensors"))


def read_config(path) -> dict:
    with open(Path(str(path)) / "config.json") as f:
        return json.load(f)


def target_args_from_config(cfg: dict) -> TargetArgs:
    """TargetArgs of a Qwen3-family config.json (text_config is read when nested)."""
    c = cfg.get("text_config", cfg)
    mt = str(c.get("model_type", cfg.get("model_type", "")))
    if not mt.startswith("qwen3"):
        raise ValueError(f"checkpoint model_type {mt!r}: only qwen3-family targets load from a local path")
    missing = [k for k in ("hidden_size", "num_hidden_layers", "intermediate_size", "num_attention_heads",
                           "vocab_size") if k not in c]
    if missing:
        raise ValueError(f"config.json is missing {missing}")
    kw = {k: c[k] for k in _ARG_KEYS if k in c}
    kw.setdefault("num_key_value_heads", c["num_attention_heads"])
    kw["head_dim"] = int(c.get("head_dim") or c["hidden_size"] // c["num_attention_heads"])
    kw["model_type"] = "qwen3"
    args = TargetArgs(**kw)
    if args.hidden_size % 64 or args.intermediate_size % 128 or args.head_dim not in (128, 256):
        raise ValueError(f"unsupported shape: hidden {args.hidden_size} (multiple of 64), intermediate "
                         f"{args.intermediate_size} (multiple of 128), head_dim {args.head_dim} (128 or 256)")
    return args


def _quantization(cfg: dict):
    q = cfg.get("quantization") or cfg.get("quantization_config")
    if not q:
        return None
    bits, gs = int(q.get("bits", 0)), int(q.get("group_size", 0))
    if bits not in (4, 8) or gs != 64:
        raise ValueError(f"quantization bits={bits} group_size={gs}: this engine runs 8- or 4-bit codes "
                         f"with group 64 (or unquantized checkpoints, which it quantizes)")
    return bits, gs


class _Tensors:
    """Every tensor of the checkpoint's safetensors files, read on demand (to the device)."""

    def __init__(self, path, device):
        from safetensors import safe_open
        self.device = device
        self.files = {}
        for f in sorted(Path(str(path)).glob("*.safetensors")):
            h = safe_open(str(f), framework="pt")
            for k in h.keys():
                self.files[k] = h

    def has(self, key) -> bool:
        return key in self.files

    def get(self, key) -> torch.Tensor:
        if key not in self.files:
            raise ValueError(f"checkpoint tensor {key!r} not found")
        return self.files[key].get_tensor(key).to(self.device)


def _mlx_triplet(t: _Tensors, name: str, N: int, K: int, bits: int | None):
    """(codes u8 [N, K] one per byte, scales, biases bf16 [N, K/64]) of one linear (quantizing a
    plain weight when bits is None)."""
    w = t.get(name + ".weight")
    if bits:
        words = K * bits // 32
        if w.dtype not in (torch.uint32, torch.int32) or tuple(w.shape) != (N, words):
            raise ValueError(f"{name}.weight: expected {bits}-bit packed uint32 [{N}, {words}], got {w.dtype} "
                             f"{tuple(w.shape)}")
        by = w.contiguous().view(torch.uint8).view(N, K * bits // 8)
        if bits == 8:
            q = by
        else:   # two codes per byte, low nibble first
            q = torch.stack([by & 0xF, by >> 4], dim=-1).view(N, K)
        s = t.get(name + ".scales").to(torch.bfloat16)
        b = t.get(name + ".biases").to(torch.bfloat16)
        if tuple(s.shape) != (N, K // 64) or tuple(b.shape) != (N, K // 64):
            raise ValueError(f"{name}: scales/biases must be [{N}, {K // 64}]")
        return q, s.contiguous(), b.contiguous()
    if tuple(w.shape) != (N, K):
        raise ValueError(f"{name}.weight: expected [{N}, {K}], got {tuple(w.shape)}")
    return W8Weight.quantize_mlx(w.to(torch.bfloat16) if w.dtype != torch.float32 else w)


def _w8(t, names_rows, K, bits, paired=False) -> W8Weight:
    parts = [_mlx_triplet(t, n, rows, K, bits) for n, rows in names_rows]
    q = torch.cat([p[0] for p in parts]) if len(parts) > 1 else parts[0][0]
    s = torch.cat([p[1] for p in parts]) if len(parts) > 1 else parts[0][1]
    b = torch.cat([p[2] for p in parts]) if len(parts) > 1 else parts[0][2]
    return W8Weight.from_mlx(q, s, b, paired, bits or 8)


def _vec(t: _Tensors, name: str, n: int) -> torch.Tensor:
    v = t.get(name).to(torch.bfloat16).contiguous()
    if v.numel() != n:
        raise ValueError(f"{name}: expected {n} values, got {v.numel()}")
    return v.view(n)


def load_qwen3_w8(path, device="cuda") -> Qwen3W8:
    """The target of a local MLX checkpoint directory as the engine's W8 model."""
    cfg = read_config(path)
    args = target_args_from_config(cfg)
    qz = _quantization(cfg)
    quantized = qz[0] if qz is not None else None   # code width, or None: quantize to 8-bit
    device = torch.device(device)
    t = _Tensors(path, device)
    H, I = args.hidden_size, args.intermediate_size
    nq, nkv, hd = args.num_attention_heads, args.num_key_value_heads, args.head_dim
    layers = []
    for l in range(args.num_hidden_layers):
        p = f"model.layers.{l}."
        a, m = p + "self_attn.", p + "mlp."
        layers.append(LayerWeights(
            qkv=_w8(t, [(a + "q_proj", nq * hd), (a + "k_proj", nkv * hd), (a + "v_proj", nkv * hd)], H, quantized),
            o=_w8(t, [(a + "o_proj", H)], nq * hd, quantized),
            gate_up=_w8(t, [(m + "gate_proj", I), (m + "up_proj", I)], H, quantized, paired=True),
            down=_w8(t, [(m + "down_proj", H)], I, quantized),
            in_norm=_vec(t, p + "input_layernorm.weight", H),
            post_norm=_vec(t, p + "post_attention_layernorm.weight", H),
            q_norm=_vec(t, a + "q_norm.weight", hd), k_norm=_vec(t, a + "k_norm.weight", hd)))
    eq, es, eb = _mlx_triplet(t, "model.embed_tokens", args.vocab_size, H, quantized)
    embed = W8Table(eq, es, eb)
    if args.tie_word_embeddings or not t.has("lm_head.weight"):
        lm_head = W8Weight.from_mlx(eq, es, eb, bits=quantized or 8)
    else:
        lm_head = _w8(t, [("lm_head", args.vocab_size)], H, quantized)
    norm = _vec(t, "model.norm.weight", H)
    torch.cuda.synchronize(device)
    return Qwen3W8(args, layers, embed, lm_head, norm)


def has_tokenizer(path) -> bool:
    p = Path(str(path))
    return (p / "tokenizer.json").is_file() or (p / "tokenizer_config.json").is_file()


def load_tokenizer(path):
    """The checkpoint's Hugging Face tokenizer (tokenizer.json in the directory, read offline)."""
    from transformers import AutoTokenizer
    return AutoTokenizer.from_pretrained(str(path), local_files_only=True)


def save_qwen3_w8(model: Qwen3W8, path, config_extra: dict | None = None) -> None:
    """Write a model built with keep_mlx=True as a quantized MLX checkpoint (config.json +
    model.safetensors; 8- or 4-bit codes as the model's layers hold them; the embedding table
    is written at the same width) - the inverse of load_qwen3_w8, for tests and round trips."""
    from safetensors.torch import save_file
    a = model.args
    nq, nkv, hd, I = a.num_attention_heads, a.num_key_value_heads, a.head_dim, a.intermediate_size
    out = {}

    bits = model.layers[0].qkv.bits

    def put(name, trip, r0=None, r1=None):
        q, s, b = trip
        if r0 is not None:
            q, s, b = q[r0:r1], s[r0:r1], b[r0:r1]
        q = q.contiguous()
        if bits == 4:    # two codes per byte, low nibble first
            q = (q.view(q.shape[0], -1, 2)[..., 0] | (q.view(q.shape[0], -1, 2)[..., 1] << 4)).contiguous()
        out[name + ".weight"] = q.view(torch.uint32).cpu()
        out[name + ".scales"] = s.contiguous().cpu()
        out[name + ".biases"] = b.contiguous().cpu()

    for l, L in enumerate(model.layers):
        p = f"model.layers.{l}."
        put(p + "self_attn.q_proj", L.qkv.mlx, 0, nq * hd)
        put(p + "self_attn.k_proj", L.qkv.mlx, nq * hd, (nq + nkv) * hd)
        put(p + "self_attn.v_proj", L.qkv.mlx, (nq + nkv) * hd, (nq + 2 * nkv) * hd)
        put(p + "self_attn.o_proj", L.o.mlx)
        put(p + "mlp.gate_proj", L.gate_up.mlx, 0, I)
        put(p + "mlp.up_proj", L.gate_up.mlx, I, 2 * I)
        put(p + "mlp.down_proj", L.down.mlx)
        out[p + "input_layernorm.weight"] = L.in_norm.cpu()
        out[p + "post_attention_layernorm.weight"] = L.post_norm.cpu()
        out[p + "self_attn.q_norm.weight"] = L.q_norm.cpu()
        out[p + "self_attn.k_norm.weight"] = L.k_norm.cpu()
    put("model.embed_tokens", (model.embed.q, model.embed.s, model.embed.b))
    if not a.tie_word_embeddings:
        put("lm_head", model.lm_head.mlx)
    out["model.norm.weight"] = model.norm.cpu()
    os.makedirs(str(path), exist_ok=True)
    save_file(out, str(Path(str(path)) / "model.safetensors"))
    cfg = {"model_type": "qwen3", "hidden_size": a.hidden_size, "num_hidden_layers": a.num_hidden_layers,
           "intermediate_size": I, "num_attention_heads": nq, "num_key_value_heads": nkv, "head_dim": hd,
           "vocab_size": a.vocab_size, "rms_norm_eps": a.rms_norm_eps, "rope_theta": a.rope_theta,
           "tie_word_embeddings": a.tie_word_embeddings, "max_position_embeddings": a.max_position_embeddings,
           "quantization": {"group_size": 64, "bits": bits}}
    cfg.update(config_extra or {})
    with open(Path(str(path)) / "config.json", "w") as f:
        json.dump(cfg, f, indent=1)
