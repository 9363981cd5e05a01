"""DFlash block-diffusion drafter on gfx950 kernels.

Behaviour follows the reference's DFlashDraftModel (src/mlx_dspark/dflash_model.py:52-208):
  - the drafter has no embedding or head of its own; ``bind`` lends it the target's
    (:168-184);
  - context: h_ctx = RMSNorm(fc(concat of tapped target hidden states)) (:199); each layer
    projects h_ctx to K/V (k_norm on K), ropes K at the cache offset and stores it (:111-123);
  - block: [anchor] + [mask] * (block_size - 1) embedded by the target table (:198); per layer
    q, k, v from RMSNorm(h), q/k norms, rope at offset + S (:115-122); the block K/V is not
    stored; attention over ctx ++ block is unmasked (bidirectional) on full-attention layers
    and causal within the window on sliding layers (:127-133);
  - logits = target_head(norm(h[:, logits_start:])) with an optional soft-cap (:202-208).
The context K/V lives in a PagedKVCache (one row); the block K/V is written after the
context in the same pages and left outside the cached length, so the next context append
overwrites it.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Dict, Optional, Tuple

import torch

from . import blockdraft, ops
from .kv import PagedKVCache
from .ops import W8Weight
from .qwen3 import LayerWeights, TargetArgs


@dataclass
class DFlashConfig:
    hidden_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    intermediate_size: int
    vocab_size: int
    rms_norm_eps: float
    rope_theta: float
    max_position_embeddings: int
    block_size: int
    target_layer_ids: Tuple[int, ...]
    num_target_layers: int
    mask_token_id: int = 0
    rope_scaling: Optional[Dict[str, Any]] = None
    layer_types: Tuple[str, ...] = field(default_factory=tuple)
    sliding_window: Optional[int] = None
    final_logit_softcapping: Optional[float] = None

    def __post_init__(self):
        if not self.layer_types:
            self.layer_types = ("full_attention",) * self.num_hidden_layers

    def as_args(self) -> TargetArgs:
        return TargetArgs(hidden_size=self.hidden_size, num_hidden_layers=self.num_hidden_layers,
                          intermediate_size=self.intermediate_size,
                          num_attention_heads=self.num_attention_heads,
                          num_key_value_heads=self.num_key_value_heads, head_dim=self.head_dim,
                          vocab_size=self.vocab_size, rms_norm_eps=self.rms_norm_eps,
                          rope_theta=self.rope_theta, sliding_window=self.sliding_window,
                          layer_types=tuple(self.layer_types))


class DFlashDraftModel:
    def __init__(self, config: DFlashConfig, fc: W8Weight, hidden_norm: torch.Tensor,
                 layers: list[LayerWeights], norm: torch.Tensor):
        if config.rope_scaling:
            raise ValueError("DFlash rope_scaling is not supported by this engine")
        self.config = config
        self.args = config.as_args()
        self.fc = fc
        self.hidden_norm = hidden_norm
        self.layers = layers
        self.norm = norm
        self.device = norm.device
        self.inv_freq = ops.rope_inv_freq(config.head_dim, config.rope_theta, self.device)
        self.act_epi = ops.DSK_EPI_SWIGLU
        self.target = None
        self.embed_tokens = None
        self.lm_head = None
        self.embed_scale = 1.0

    # ---------------------------------------------------------------- binding
    def bind(self, target_model) -> "DFlashDraftModel":
        """Borrow the target's embedding table and head (src/mlx_dspark/dflash_model.py:168-184)."""
        tm = getattr(target_model, "model", target_model)
        if not hasattr(tm, "embed"):
            raise AttributeError(f"Cannot find embed_tokens in {type(target_model).__name__}")
        self.target = tm
        self.embed_tokens = tm.embed
        self.lm_head = tm.lm_head
        self.embed_scale = tm.args.embed_scale
        return self

    def make_cache(self, max_ctx: int = 16384, B: int = 1) -> PagedKVCache:
        c = self.config
        return PagedKVCache(c.num_hidden_layers, B, c.num_key_value_heads, c.head_dim,
                            max_ctx + c.block_size, device=self.device)

    # ---------------------------------------------------------------- context
    def ingest(self, target_hidden: torch.Tensor, cache: PagedKVCache, n_valid=None) -> None:
        """Append context rows: target_hidden [S, n_tap*H] (or [1, S, .]) bf16 (see
        blockdraft.ingest_context; n_valid: device-counted append of n_valid + 1 rows)."""
        blockdraft.ingest_context(self, target_hidden, cache, n_valid)

    # ---------------------------------------------------------------- block
    def block_hidden(self, block_ids: torch.Tensor, cache: PagedKVCache) -> torch.Tensor:
        """block_ids [B, bs] int32 (device) -> final hidden [B*bs, H] before the drafter norm."""
        B, bs = block_ids.shape
        h = ops.w8_embed(block_ids.reshape(-1), self.embed_tokens, self.embed_scale)
        return blockdraft.block_layers(self, h, B, bs, cache, self.config.head_dim ** -0.5)

    def block_logits(self, block_ids: torch.Tensor, cache: PagedKVCache, logits_start: int = 1,
                     cap: int | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
        """Logits of block positions logits_start .. logits_start + cap - 1: [B, cap, V] f32."""
        c = self.config
        B, bs = block_ids.shape
        cap = bs - logits_start if cap is None else cap
        h = self.block_hidden(block_ids, cache).view(B, bs, -1)[:, logits_start:logits_start + cap]
        h = h.reshape(B * cap, -1) if B > 1 else h[0]
        out = blockdraft.head_rows(self, h, self.lm_head, out)
        return out.view(B, cap, c.vocab_size)

    def __call__(self, inputs, target_hidden, cache, logits_start: int = 0):
        """Reference-shaped call (src/mlx_dspark/dflash_model.py:197-208): ingest the new
        context rows, then return logits for the block positions from logits_start on."""
        if target_hidden is not None and target_hidden.numel():
            self.ingest(target_hidden, cache)
        ids = inputs if torch.is_tensor(inputs) else torch.tensor(inputs)
        ids = ids.to(self.device, torch.int32).reshape(1, -1)
        return self.block_logits(ids, cache, logits_start)
