"""Local DSpark and DFlash drafter checkpoints (a directory of config.json + *.safetensors, the
inputs of src/mlx_dspark/load.py:155-215 and :224-289 in the reference).

Key names are the reference modules' parameter paths, so DeepSpec DSpark and z-lab DFlash
checkpoints load as they are:

  DSpark (src/mlx_dspark/model.py:196-245):
    embed_tokens.weight [V, H]   fc.weight [H, taps*H]   hidden_norm.weight   norm.weight
    lm_head.weight [V, H]
    layers.<i>.self_attn.{q,k,v,o}_proj.weight (no v_proj when k_eq_v), .self_attn.{q,k}_norm.weight
    layers.<i>.mlp.{gate,up,down}_proj.weight, .input_layernorm.weight, .post_attention_layernorm.weight
    gemma layers also: .pre_feedforward_layernorm.weight, .post_feedforward_layernorm.weight, .layer_scalar [1]
    markov_head.markov_w1.weight [V, R] (an embedding), markov_head.markov_w2.weight [V, R]
    confidence_head.proj.weight [1, H (+ R)], confidence_head.proj.bias [1]
  DFlash (src/mlx_dspark/dflash_model.py:100-208; embedding and head come from the target):
    fc.weight, hidden_norm.weight, norm.weight and the same per-layer attention / MLP / two-norm keys.

A checkpoint whose key set differs from the config's raises ValueError (strict, as the reference
does); ``strict=False`` loads the intersection (a DSpark drafter only, as in the reference), and a
missing parameter takes the value a fresh reference module gives it: norm weights one, a linear
matrix uniform in +-sqrt(1/K) (nn.Linear's initialiser), an embedding table normal with scale
sqrt(1/dims) (nn.Embedding's); a missing bias is zero (nn.Linear would draw it uniform too). Those draws are seeded by the key name, so a load is
reproducible; MLX's own random stream is not, so a partially loaded drafter drafts like some
fresh reference module, not like the one the reference would build. Weights in bf16/f16/f32 are quantized on load
with the engine's affine group-64 quantizer: every linear and embedding table (the reference's
nn.quantize over the DSpark drafter; the DFlash backbone linears only) at ``bits`` (4 by default,
as the reference). An MLX-quantized matrix (uint32 ``.weight`` with ``.scales`` / ``.biases``) is
taken with its own codes. Embedding and Markov tables are gathered row by row, so their codes are
held one per byte whatever the width; the Markov w2 projection runs on the 8-bit tile layout
with 4-bit code values (the Markov kernel streams byte codes).
"""

from __future__ import annotations

import hashlib

import json
import warnings
from pathlib import Path

import torch

from .checkpoint import _Tensors
from .config import DSparkConfig
from .ops import W8Table, W8Weight
from .qwen3 import LayerWeights

_FLOAT = (torch.bfloat16, torch.float16, torch.float32)


def _layer_keys(p: str, *, k_eq_v: bool, gemma: bool, bias: bool) -> list[str]:
    a = p + "self_attn."
    keys = [a + "q_proj.weight", a + "k_proj.weight", a + "o_proj.weight", a + "q_norm.weight", a + "k_norm.weight"]
    if not k_eq_v:
        keys.append(a + "v_proj.weight")
    if bias:
        keys += [a + f"{n}_proj.bias" for n in ("q", "k", "o")] + ([] if k_eq_v else [a + "v_proj.bias"])
    keys += [p + f"mlp.{n}_proj.weight" for n in ("gate", "up", "down")]
    keys += [p + "input_layernorm.weight", p + "post_attention_layernorm.weight"]
    if gemma:
        keys += [p + "pre_feedforward_layernorm.weight", p + "post_feedforward_layernorm.weight", p + "layer_scalar"]
    return keys


def dspark_keys(cfg: DSparkConfig) -> list[str]:
    """The parameter names of a DSpark drafter with this config (model.py:196-245)."""
    gemma = cfg.norm_style == "gemma"
    keys = ["embed_tokens.weight", "fc.weight", "hidden_norm.weight", "norm.weight", "lm_head.weight"]
    for l in range(cfg.num_hidden_layers):
        keys += _layer_keys(f"layers.{l}.", k_eq_v=cfg.attention_k_eq_v, gemma=gemma, bias=cfg.attention_bias)
    if cfg.markov_rank > 0:
        keys += ["markov_head.markov_w1.weight", "markov_head.markov_w2.weight"]
    if cfg.enable_confidence_head:
        keys += ["confidence_head.proj.weight", "confidence_head.proj.bias"]
    return keys


def dflash_keys(cfg) -> list[str]:
    """The parameter names of a DFlash drafter with this config (dflash_model.py:100-208)."""
    keys = ["fc.weight", "hidden_norm.weight", "norm.weight"]
    for l in range(cfg.num_hidden_layers):
        keys += _layer_keys(f"layers.{l}.", k_eq_v=False, gemma=False, bias=False)
    return keys


def _ckpt_keys(t: _Tensors) -> set[str]:
    """The checkpoint's parameter names (an MLX-quantized matrix's .scales / .biases belong to
    its .weight)."""
    keys = set(t.files)
    for k in list(keys):
        if k.endswith(".scales") and k[:-7] + ".weight" in keys:
            keys.discard(k)
            keys.discard(k[:-7] + ".biases")
    return keys


def _fresh_init(key: str, N: int, K: int, embedding: bool, device) -> torch.Tensor:
    """A fresh module's value for a parameter missing from a checkpoint: nn.Embedding's normal
    draw (scale sqrt(1/K)) or nn.Linear's uniform one (+-sqrt(1/K)), seeded by the key name."""
    g = torch.Generator().manual_seed(int.from_bytes(hashlib.sha256(key.encode()).digest()[:8], "little") >> 1)
    scale = (1.0 / K) ** 0.5
    if embedding:
        w = torch.randn((N, K), generator=g) * scale
    else:
        w = (torch.rand((N, K), generator=g) * 2.0 - 1.0) * scale
    return w.to(device)


def _check_keys(where: str, want: list[str], t: _Tensors, strict: bool, what: str) -> set[str]:
    have = _ckpt_keys(t)
    missing = sorted(set(want) - have)
    unexpected = sorted(have - set(want))
    if missing or unexpected:
        detail = ""
        if missing:
            detail += f"\n  missing in checkpoint ({len(missing)}): {missing[:8]}"
        if unexpected:
            detail += f"\n  unexpected in checkpoint ({len(unexpected)}): {unexpected[:8]}"
        if strict:
            raise ValueError(f"{where}: tensor names don't match a {what} with this config.json{detail}")
        warnings.warn(f"{where}: key mismatch, loading the intersection:{detail}")
    return set(want) & have


class _Loader:
    """Reads one checkpoint's tensors and quantizes them for the engine. keep_mlx keeps every
    matrix's MLX-layout (codes, scales, biases) on its engine weight (for checkers)."""

    def __init__(self, t: _Tensors, present: set[str], bits: int, device, keep_mlx: bool = False):
        self.t, self.present, self.bits, self.device, self.keep_mlx = t, present, bits, device, keep_mlx

    def _float(self, key: str, shape) -> torch.Tensor | None:
        if key not in self.present:
            return None
        w = self.t.get(key)
        if w.dtype not in _FLOAT:
            raise ValueError(f"{key}: expected a floating-point tensor, got {w.dtype}")
        if tuple(w.shape) != tuple(shape):
            raise ValueError(f"{key}: expected shape {tuple(shape)}, got {tuple(w.shape)}")
        return w

    def triplet(self, name: str, N: int, K: int, bits: int | None = None, embedding: bool = False):
        """(codes u8 [N, K] one per byte, scales, biases bf16 [N, K/64]) of a matrix: its own codes
        when MLX-quantized, else quantized here (a missing one, strict=False, a seeded draw of the
        module's initialiser: ``embedding`` tables normal, linears uniform)."""
        bits = bits or self.bits
        key = name + ".weight"
        if key in self.present and self.t.has(name + ".scales"):
            w = self.t.get(key)
            if w.dtype not in (torch.uint32, torch.int32):
                raise ValueError(f"{key}: quantized weights are packed uint32")
            words = w.shape[1]
            qbits = words * 32 // K
            if qbits not in (4, 8) or tuple(w.shape) != (N, K * qbits // 32):
                raise ValueError(f"{key}: packed shape {tuple(w.shape)} is not [{N}, K*bits/32] with K={K}")
            by = w.contiguous().view(torch.uint8).view(N, K * qbits // 8)
            q = by if qbits == 8 else torch.stack([by & 0xF, by >> 4], dim=-1).view(N, K)
            s = self.t.get(name + ".scales").to(torch.bfloat16).contiguous()
            b = self.t.get(name + ".biases").to(torch.bfloat16).contiguous()
            if tuple(s.shape) != (N, K // 64) or tuple(b.shape) != (N, K // 64):
                raise ValueError(f"{name}: scales / biases must be [{N}, {K // 64}]")
            return q.contiguous(), s, b, qbits
        w = self._float(key, (N, K))
        if w is None:
            w = _fresh_init(key, N, K, embedding, self.device)
        q, s, b = W8Weight.quantize_mlx(w.to(torch.bfloat16) if w.dtype != torch.float32 else w, bits)
        return q, s, b, bits

    def linear(self, names_rows: list[tuple[str, int]], K: int, *, paired: bool = False) -> W8Weight:
        """Rows of several matrices stacked into one engine weight (the fused q|k|v, gate|up)."""
        parts = [self.triplet(n, rows, K) for n, rows in names_rows]
        widths = {p[3] for p in parts}
        if len(widths) != 1:
            raise ValueError(f"{[n for n, _ in names_rows]}: mixed code widths {sorted(widths)}")
        q = torch.cat([p[0] for p in parts])
        s = torch.cat([p[1] for p in parts])
        b = torch.cat([p[2] for p in parts])
        W = W8Weight.from_mlx(q, s, b, paired, widths.pop())
        if self.keep_mlx:
            W.mlx = (q, s, b)
        return W

    def table(self, name: str, N: int, K: int) -> W8Table:
        q, s, b, _ = self.triplet(name, N, K, embedding=True)
        return W8Table(q, s, b)

    def vec(self, key: str, n: int, default: float = 1.0) -> torch.Tensor:
        w = self._float(key, (n,))
        if w is None:
            return torch.full((n,), default, dtype=torch.bfloat16, device=self.device)
        return w.to(torch.bfloat16).contiguous()

    def scalar(self, key: str, default: float = 1.0) -> float:
        w = self._float(key, (1,))
        return default if w is None else float(w.float().item())


def _layers(ld: _Loader, n_layers: int, H: int, I: int, nq: int, nkv: int, hd: int, *, k_eq_v: bool,
            gemma: bool) -> list[LayerWeights]:
    out = []
    for l in range(n_layers):
        p = f"layers.{l}."
        a = p + "self_attn."
        qkv_rows = [(a + "q_proj", nq * hd), (a + "k_proj", nkv * hd),
                    (a + ("k_proj" if k_eq_v else "v_proj"), nkv * hd)]   # k_eq_v: V comes from k_proj
        norm = (lambda k: ld.vec(p + k + ".weight", H))
        out.append(LayerWeights(
            qkv=ld.linear(qkv_rows, H),
            o=ld.linear([(a + "o_proj", H)], nq * hd),
            gate_up=ld.linear([(p + "mlp.gate_proj", I), (p + "mlp.up_proj", I)], H, paired=True),
            down=ld.linear([(p + "mlp.down_proj", H)], I),
            in_norm=norm("input_layernorm"),
            # gemma: the norm before the MLP is pre_feedforward_layernorm; post_attention_layernorm
            # and post_feedforward_layernorm norm the sublayer outputs before their residual adds
            post_norm=norm("pre_feedforward_layernorm" if gemma else "post_attention_layernorm"),
            q_norm=ld.vec(a + "q_norm.weight", hd), k_norm=ld.vec(a + "k_norm.weight", hd),
            attn_out_norm=norm("post_attention_layernorm") if gemma else None,
            ff_out_norm=norm("post_feedforward_layernorm") if gemma else None))
    return out


def load_dspark(path, *, bits: int = 4, strict: bool = True, device="cuda", keep_mlx: bool = False):
    """(DSparkDrafter, DSparkConfig) from a local DeepSpec-format directory (load.py:155-215)."""
    from .model import ConfidenceHead, DSparkDrafter, MarkovHead

    if bits not in (4, 8):
        raise ValueError("this engine runs 4- or 8-bit (group 64) drafters")
    path = Path(str(path))
    cfg = DSparkConfig.from_json(path / "config.json")
    if cfg.attention_bias:
        raise ValueError(f"{path}: attention_bias drafters are not supported by this engine")
    t = _Tensors(path, torch.device(device))
    present = _check_keys(str(path), dspark_keys(cfg), t, strict, "DeepSpec-format DSpark drafter")
    ld = _Loader(t, present, bits, torch.device(device), keep_mlx)
    H, V, I = cfg.hidden_size, cfg.vocab_size, cfg.intermediate_size
    gemma = cfg.norm_style == "gemma"
    nq, nkv, hd = cfg.num_attention_heads, cfg.n_kv_heads, cfg.attn_head_dim
    layers = _layers(ld, cfg.num_hidden_layers, H, I, nq, nkv, hd, k_eq_v=cfg.attention_k_eq_v, gemma=gemma)
    markov = None
    R = cfg.markov_rank
    if R > 0:
        q2, s2, b2, _ = ld.triplet("markov_head.markov_w2", V, R)
        w2 = W8Weight.from_mlx(q2, s2, b2, bits=8)
        if keep_mlx:
            w2.mlx = (q2, s2, b2)
        markov = MarkovHead(ld.table("markov_head.markov_w1", V, R), w2)
    conf = None
    if cfg.enable_confidence_head:
        K = H + (R if cfg.confidence_head_with_markov and R > 0 else 0)
        q, s, b, cb = ld.triplet("confidence_head.proj", 1, K)
        # one output row, padded to a 16-row tile with zero codes, unit scales and zero biases
        q = torch.cat([q, torch.zeros((15, K), dtype=q.dtype, device=q.device)])
        s = torch.cat([s, torch.ones((15, K // 64), dtype=s.dtype, device=s.device)])
        b = torch.cat([b, torch.zeros((15, K // 64), dtype=b.dtype, device=b.device)])
        cw = W8Weight.from_mlx(q, s, b, bits=cb)
        if keep_mlx:
            cw.mlx = (q, s, b)
        conf = ConfidenceHead(cw, ld.scalar("confidence_head.proj.bias", 0.0))
    d = DSparkDrafter(cfg, embed=ld.table("embed_tokens", V, H),
                      fc=ld.linear([("fc", H)], len(cfg.target_layer_ids) * H),
                      hidden_norm=ld.vec("hidden_norm.weight", H), layers=layers, norm=ld.vec("norm.weight", H),
                      lm_head=ld.linear([("lm_head", V)], H), markov=markov, confidence=conf,
                      layer_scalars=[ld.scalar(f"layers.{l}.layer_scalar") for l in range(cfg.num_hidden_layers)]
                      if gemma else None)
    torch.cuda.synchronize()
    return d, cfg


def dflash_config(path):
    """DFlashConfig of a z-lab DFlash config.json in directory ``path``."""
    return dflash_config_from_dict(json.loads((Path(str(path)) / "config.json").read_text()), str(path))


def dflash_config_from_dict(cfg: dict, path: str = "config"):
    """DFlashConfig of a z-lab DFlash config (load.py:242-263: a Markov-head hybrid is refused;
    the gemma4 layout nests RoPE under rope_parameters)."""
    from .dflash_model import DFlashConfig

    if cfg.get("markov_rank"):
        raise ValueError(f"{path}: this DFlash checkpoint carries a Markov head (markov_rank={cfg['markov_rank']}),"
                         f" a DFlash+DSpark hybrid this engine does not run")
    rope = cfg.get("rope_parameters") or {}
    dfc = cfg.get("dflash_config", {})
    return DFlashConfig(
        hidden_size=cfg["hidden_size"], num_hidden_layers=cfg["num_hidden_layers"],
        num_attention_heads=cfg["num_attention_heads"], num_key_value_heads=cfg["num_key_value_heads"],
        head_dim=cfg["head_dim"], intermediate_size=cfg["intermediate_size"], vocab_size=cfg["vocab_size"],
        rms_norm_eps=cfg["rms_norm_eps"], rope_theta=cfg.get("rope_theta", rope.get("rope_theta", 1_000_000.0)),
        max_position_embeddings=cfg["max_position_embeddings"], block_size=cfg["block_size"],
        target_layer_ids=tuple(dfc.get("target_layer_ids") or cfg["target_layer_ids"]),
        num_target_layers=cfg["num_target_layers"], mask_token_id=dfc.get("mask_token_id", cfg.get("mask_token_id", 0)),
        rope_scaling=cfg.get("rope_scaling"),
        layer_types=tuple(cfg.get("layer_types") or ["full_attention"] * cfg["num_hidden_layers"]),
        sliding_window=cfg.get("sliding_window"), final_logit_softcapping=cfg.get("final_logit_softcapping"))


def load_dflash(path, *, bits: int = 4, device="cuda", keep_mlx: bool = False):
    """(DFlashDraftModel, DFlashConfig) from a local z-lab-format directory (load.py:224-289): the
    key set must match exactly; the backbone linears are quantized, the embedding and head come
    from the target at bind()."""
    from .dflash_model import DFlashDraftModel

    if bits not in (4, 8):
        raise ValueError("this engine runs 4- or 8-bit (group 64) drafters")
    cfg = dflash_config(path)
    t = _Tensors(Path(str(path)), torch.device(device))
    present = _check_keys(str(path), dflash_keys(cfg), t, True, "z-lab DFlash drafter")
    ld = _Loader(t, present, bits, torch.device(device), keep_mlx)
    H, I = cfg.hidden_size, cfg.intermediate_size
    layers = _layers(ld, cfg.num_hidden_layers, H, I, cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim,
                     k_eq_v=False, gemma=False)
    fc = ld.linear([("fc", H)], len(cfg.target_layer_ids) * H)
    d = DFlashDraftModel(cfg, fc, ld.vec("hidden_norm.weight", H), layers, ld.vec("norm.weight", H))
    torch.cuda.synchronize()
    return d, cfg


# ----------------------------------------------------------------------------- saving
def _packed_u32(q: torch.Tensor, bits: int) -> torch.Tensor:
    """Codes one per byte [N, K] -> MLX uint32 words [N, K * bits / 32] (lowest bits first)."""
    q = q.contiguous().to(torch.uint8)
    N, K = q.shape
    if bits == 4:
        if int(q.max()) > 15:
            raise ValueError("4-bit packing of codes above 15")
        q = (q[:, 0::2] | (q[:, 1::2] << 4)).contiguous()
    return q.view(torch.int32).view(N, K * bits // 32)


def _put_matrix(out: dict, name: str, q, s, b, r0: int | None = None, r1: int | None = None) -> None:
    q, s, b = (x[r0:r1] for x in (q, s, b)) if r0 is not None else (q, s, b)
    bits = 4 if int(q.max()) <= 15 else 8
    out[name + ".weight"] = _packed_u32(q, bits).cpu()
    out[name + ".scales"] = s.contiguous().cpu()
    out[name + ".biases"] = b.contiguous().cpu()


def _mlx_of(W, what: str):
    trip = getattr(W, "mlx", None)
    if trip is None:
        raise ValueError(f"{what}: saving needs the MLX-layout codes (build or load with keep_mlx=True)")
    return trip


def _put_layers(out: dict, layers, nq: int, nkv: int, hd: int, I: int, *, k_eq_v: bool, gemma: bool) -> None:
    for l, L in enumerate(layers):
        p = f"layers.{l}."
        a = p + "self_attn."
        q, s, b = _mlx_of(L.qkv, "qkv")
        _put_matrix(out, a + "q_proj", q, s, b, 0, nq * hd)
        _put_matrix(out, a + "k_proj", q, s, b, nq * hd, (nq + nkv) * hd)
        if not k_eq_v:
            _put_matrix(out, a + "v_proj", q, s, b, (nq + nkv) * hd, (nq + 2 * nkv) * hd)
        _put_matrix(out, a + "o_proj", *_mlx_of(L.o, "o"))
        g, sg, bg = _mlx_of(L.gate_up, "gate_up")         # source order: gate rows, then up rows
        _put_matrix(out, p + "mlp.gate_proj", g, sg, bg, 0, I)
        _put_matrix(out, p + "mlp.up_proj", g, sg, bg, I, 2 * I)
        _put_matrix(out, p + "mlp.down_proj", *_mlx_of(L.down, "down"))
        out[a + "q_norm.weight"] = L.q_norm.cpu()
        out[a + "k_norm.weight"] = L.k_norm.cpu()
        out[p + "input_layernorm.weight"] = L.in_norm.cpu()
        if gemma:
            out[p + "post_attention_layernorm.weight"] = L.attn_out_norm.cpu()
            out[p + "pre_feedforward_layernorm.weight"] = L.post_norm.cpu()
            out[p + "post_feedforward_layernorm.weight"] = L.ff_out_norm.cpu()
        else:
            out[p + "post_attention_layernorm.weight"] = L.post_norm.cpu()


def dspark_config_dict(cfg: DSparkConfig) -> dict:
    """A DeepSpec config.json for a DSpark config (the fields DSparkConfig.from_dict reads)."""
    c = {"model_type": "qwen3" if cfg.family == "qwen3" else "gemma4_text", "hidden_size": cfg.hidden_size,
         "vocab_size": cfg.vocab_size, "num_hidden_layers": cfg.num_hidden_layers,
         "intermediate_size": cfg.intermediate_size, "rms_norm_eps": cfg.rms_norm_eps,
         "num_attention_heads": cfg.num_attention_heads, "num_key_value_heads": cfg.num_key_value_heads,
         "attention_bias": cfg.attention_bias, "block_size": cfg.block_size, "mask_token_id": cfg.mask_token_id,
         "target_layer_ids": list(cfg.target_layer_ids), "num_target_layers": cfg.num_target_layers,
         "markov_rank": cfg.markov_rank, "markov_head_type": cfg.markov_head_type,
         "enable_confidence_head": cfg.enable_confidence_head,
         "confidence_head_with_markov": cfg.confidence_head_with_markov,
         "final_logit_softcapping": cfg.final_logit_softcapping, "pad_token_id": cfg.pad_token_id,
         "head_dim": cfg.head_dim}
    if cfg.family == "qwen3":
        c["rope_theta"] = cfg.rope_theta
    else:
        c.update(num_global_key_value_heads=cfg.num_global_key_value_heads, global_head_dim=cfg.global_head_dim,
                 attention_k_eq_v=cfg.attention_k_eq_v,
                 rope_parameters={"full_attention": {"rope_theta": cfg.rope_theta, "rope_type": cfg.rope_type,
                                                     "partial_rotary_factor": cfg.partial_rotary_factor}})
    return c


def save_dspark(drafter, path) -> None:
    """Write an engine DSpark drafter (built with keep_mlx=True) as an MLX-quantized checkpoint
    with the reference's key names: the inverse of load_dspark."""
    from safetensors.torch import save_file
    cfg = drafter.config
    gemma = cfg.norm_style == "gemma"
    out: dict = {}
    t = drafter.embed_tokens
    _put_matrix(out, "embed_tokens", t.q, t.s, t.b)
    _put_matrix(out, "fc", *_mlx_of(drafter.fc, "fc"))
    _put_matrix(out, "lm_head", *_mlx_of(drafter.lm_head, "lm_head"))
    out["hidden_norm.weight"] = drafter.hidden_norm.cpu()
    out["norm.weight"] = drafter.norm.cpu()
    _put_layers(out, drafter.layers, cfg.num_attention_heads, cfg.n_kv_heads, cfg.attn_head_dim,
                cfg.intermediate_size, k_eq_v=cfg.attention_k_eq_v, gemma=gemma)
    if gemma:
        for l, x in enumerate(drafter.layer_scalars or [1.0] * cfg.num_hidden_layers):
            out[f"layers.{l}.layer_scalar"] = torch.tensor([x], dtype=torch.bfloat16)
    if drafter.markov_head is not None:
        w1 = drafter.markov_head.w1
        _put_matrix(out, "markov_head.markov_w1", w1.q, w1.s, w1.b)
        _put_matrix(out, "markov_head.markov_w2", *_mlx_of(drafter.markov_head.w2, "markov_w2"))
    if drafter.confidence_head is not None:
        _put_matrix(out, "confidence_head.proj", *_mlx_of(drafter.confidence_head.proj, "confidence"), 0, 1)
        out["confidence_head.proj.bias"] = torch.tensor([drafter.confidence_head.bias], dtype=torch.float32)
    path = Path(str(path))
    path.mkdir(parents=True, exist_ok=True)
    (path / "config.json").write_text(json.dumps(dspark_config_dict(cfg), indent=1))
    save_file(out, str(path / "model.safetensors"))


def save_dflash(drafter, path) -> None:
    """Write an engine DFlash drafter (built with keep_mlx=True) as an MLX-quantized z-lab-format
    checkpoint: the inverse of load_dflash."""
    from safetensors.torch import save_file
    c = drafter.config
    out: dict = {}
    _put_matrix(out, "fc", *_mlx_of(drafter.fc, "fc"))
    out["hidden_norm.weight"] = drafter.hidden_norm.cpu()
    out["norm.weight"] = drafter.norm.cpu()
    _put_layers(out, drafter.layers, c.num_attention_heads, c.num_key_value_heads, c.head_dim, c.intermediate_size,
                k_eq_v=False, gemma=False)
    cj = {"hidden_size": c.hidden_size, "num_hidden_layers": c.num_hidden_layers,
          "num_attention_heads": c.num_attention_heads, "num_key_value_heads": c.num_key_value_heads,
          "head_dim": c.head_dim, "intermediate_size": c.intermediate_size, "vocab_size": c.vocab_size,
          "rms_norm_eps": c.rms_norm_eps, "rope_theta": c.rope_theta,
          "max_position_embeddings": c.max_position_embeddings, "block_size": c.block_size,
          "target_layer_ids": list(c.target_layer_ids), "num_target_layers": c.num_target_layers,
          "mask_token_id": c.mask_token_id, "layer_types": list(c.layer_types), "sliding_window": c.sliding_window,
          "final_logit_softcapping": c.final_logit_softcapping}
    path = Path(str(path))
    path.mkdir(parents=True, exist_ok=True)
    (path / "config.json").write_text(json.dumps(cj, indent=1))
    save_file(out, str(path / "model.safetensors"))
