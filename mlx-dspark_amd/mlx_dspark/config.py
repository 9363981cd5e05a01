"""DSpark drafter configuration (drop-in for src/mlx_dspark/config.py).

Same fields, defaults and config.json schema as the reference's DSparkConfig (config.py:18-185),
so DeepSpec drafter configs parse identically: family detection from model_type, the
rejection of vLLM "speculators" packagings and of targets with an embedded drafter, the
required-field check, and the family-derived knobs (MLP activation, norm layout, v_norm,
attention scaling). The engine's drafter runs both families (model.py).
"""

from __future__ import annotations

import json
from dataclasses import dataclass, field
from pathlib import Path


@dataclass
class DSparkConfig:
    family: str = "gemma4"
    hidden_size: int = 3840
    vocab_size: int = 262144
    num_hidden_layers: int = 5
    intermediate_size: int = 15360
    rms_norm_eps: float = 1e-6
    num_attention_heads: int = 16
    num_key_value_heads: int = 8
    num_global_key_value_heads: int = 1
    head_dim: int = 256
    global_head_dim: int = 512
    attention_k_eq_v: bool = True
    attention_bias: bool = False
    rope_theta: float = 1_000_000.0
    partial_rotary_factor: float = 0.25
    rope_type: str = "proportional"
    block_size: int = 7
    mask_token_id: int = 4
    target_layer_ids: list = field(default_factory=lambda: [5, 17, 29, 41, 46])
    num_target_layers: int = 48
    markov_rank: int = 256
    markov_head_type: str = "vanilla"
    enable_confidence_head: bool = True
    confidence_head_with_markov: bool = True
    final_logit_softcapping: float | None = 30.0
    pad_token_id: int = 0
    mlp_activation: str = "gelu_tanh"
    norm_style: str = "gemma"
    use_v_norm: bool = True
    attention_scaling: float | None = None

    @property
    def attn_head_dim(self) -> int:
        return self.global_head_dim if self.family == "gemma4" else self.head_dim

    @property
    def n_kv_heads(self) -> int:
        return self.num_global_key_value_heads if (self.family == "gemma4" and self.attention_k_eq_v) \
            else self.num_key_value_heads

    @property
    def scaling(self) -> float:
        if self.attention_scaling is not None:
            return self.attention_scaling
        return self.attn_head_dim ** -0.5 if self.family == "qwen3" else 1.0

    @property
    def rope_parameters(self) -> dict:
        return {"rope_type": self.rope_type, "partial_rotary_factor": self.partial_rotary_factor}

    @classmethod
    def from_json(cls, path) -> "DSparkConfig":
        with open(path) as f:
            c = json.load(f)
        return cls.from_dict(c, str(path))

    @classmethod
    def from_dict(cls, c: dict, where: str = "config") -> "DSparkConfig":
        mt = c.get("model_type", "")
        if "speculators_config" in c or "speculators_model_type" in c:
            raise ValueError(f"{where}: this checkpoint is in the vLLM 'speculators' format, which this "
                             f"engine cannot load; use a DeepSpec-native standalone DSpark drafter")
        if "block_size" not in c and any(k.startswith("dspark_") for k in c):
            raise ValueError(f"{where}: this looks like a full target model with an embedded DSpark drafter "
                             f"(dspark_* fields), not a standalone drafter checkpoint")
        if "qwen3" in mt:
            family = "qwen3"
        elif "gemma4" in mt:
            family = "gemma4"
        else:
            raise ValueError(f"{where}: unsupported drafter family (model_type={mt!r}); supported drafter "
                             f"backbones: qwen3, gemma4")
        need = ("hidden_size", "vocab_size", "num_hidden_layers", "intermediate_size", "num_attention_heads",
                "block_size", "mask_token_id", "target_layer_ids")
        missing = [k for k in need if k not in c]
        if missing:
            raise ValueError(f"{where}: config is missing required DeepSpec drafter fields {missing}")
        common = dict(hidden_size=c["hidden_size"], vocab_size=c["vocab_size"],
                      num_hidden_layers=c["num_hidden_layers"], intermediate_size=c["intermediate_size"],
                      rms_norm_eps=c.get("rms_norm_eps", 1e-6), num_attention_heads=c["num_attention_heads"],
                      num_key_value_heads=c.get("num_key_value_heads", 8),
                      attention_bias=c.get("attention_bias", False), block_size=c["block_size"],
                      mask_token_id=c["mask_token_id"], target_layer_ids=list(c["target_layer_ids"]),
                      markov_rank=c.get("markov_rank", 256), markov_head_type=c.get("markov_head_type", "vanilla"),
                      enable_confidence_head=c.get("enable_confidence_head", True),
                      confidence_head_with_markov=c.get("confidence_head_with_markov", True))
        if family == "qwen3":
            rp = c.get("rope_parameters") or {}
            return cls(family="qwen3", **common,
                       head_dim=c.get("head_dim", c["hidden_size"] // c["num_attention_heads"]),
                       attention_k_eq_v=False, rope_theta=rp.get("rope_theta", c.get("rope_theta", 1_000_000.0)),
                       rope_type="default", num_target_layers=c.get("num_target_layers", 36),
                       final_logit_softcapping=c.get("final_logit_softcapping", None),
                       pad_token_id=c.get("pad_token_id") or 0, mlp_activation="silu", norm_style="qwen",
                       use_v_norm=False)
        rope = (c.get("rope_parameters") or {}).get("full_attention", {}) or {}
        return cls(family="gemma4", **common,
                   num_global_key_value_heads=c.get("num_global_key_value_heads", 1),
                   head_dim=c.get("head_dim", 256), global_head_dim=c.get("global_head_dim", 512),
                   attention_k_eq_v=c.get("attention_k_eq_v", True),
                   rope_theta=rope.get("rope_theta", 1_000_000.0),
                   partial_rotary_factor=rope.get("partial_rotary_factor", 0.25),
                   rope_type=rope.get("rope_type", "proportional"), num_target_layers=c.get("num_target_layers", 48),
                   final_logit_softcapping=c.get("final_logit_softcapping", 30.0), pad_token_id=c.get("pad_token_id", 0),
                   mlp_activation="gelu_tanh", norm_style="gemma", use_v_norm=True)
