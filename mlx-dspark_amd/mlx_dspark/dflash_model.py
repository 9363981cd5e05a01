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

from . import ops
from .kv import PagedKVCache
from .ops import W8Weight
from .qwen3 import MAX_ROWS, LayerWeights, TargetArgs


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
        """Append context rows: target_hidden [S, n_tap*H] (or [1, S, .]) bf16.

        n_valid (device int32 [1]) advances the cached length by n_valid + 1 instead of S:
        the fixed-shape form used when only a device-side prefix of the rows is committed."""
        c = self.config
        th = target_hidden.reshape(-1, target_hidden.shape[-1])
        S = th.shape[0]
        if n_valid is not None and S > MAX_ROWS:
            raise ValueError("a device-counted context append must fit one pass")
        cache.check_room(S + c.block_size)
        H = c.hidden_size
        for r0 in range(0, S, MAX_ROWS):
            r1 = min(S, r0 + MAX_ROWS)
            hcp = ops.w8_gemm(ops.pack(th[r0:r1]), self.fc, epi=ops.DSK_EPI_PARTIAL)     # fc(target_hidden)
            xc = ops.act_pack(M=r1 - r0, K=H, part=hcp, norm_w=self.hidden_norm, eps=c.rms_norm_eps)
            for l, L in enumerate(self.layers):
                kv = ops.w8_gemm(xc, L.kv_view(self.args), epi=ops.DSK_EPI_PARTIAL)
                k_pool, v_pool, k_sb, v_sb = cache.layer_args(l)
                ops.qkv_rope_append(kv, 1, r1 - r0, 0, c.num_key_value_heads, c.head_dim, None, L.k_norm,
                                    c.rms_norm_eps, self.inv_freq, cache.seq_lens, cache.block_table,
                                    cache.page, cache.kv_dtype, k_pool, v_pool, k_sb, v_sb, None)
            if n_valid is None:
                ops.lens_add(cache.seq_lens, None, r1 - r0)
                cache.note_lengths([cache.lengths[0] + (r1 - r0)])
        if n_valid is not None:
            ops.lens_add(cache.seq_lens, n_valid, 1)

    # ---------------------------------------------------------------- block
    def block_hidden(self, block_ids: torch.Tensor, cache: PagedKVCache) -> torch.Tensor:
        """block_ids [B, bs] int32 (device) -> final hidden [B*bs, H] before the drafter norm."""
        c, a = self.config, self.args
        B, bs = block_ids.shape
        M, H = B * bs, c.hidden_size
        eps = c.rms_norm_eps
        nq, nkv, hd = c.num_attention_heads, c.num_key_value_heads, c.head_dim
        h = ops.w8_embed(block_ids.reshape(-1), self.embed_tokens, self.embed_scale)
        x = ops.pack(h, self.layers[0].in_norm, eps)
        nl = len(self.layers)
        for l, L in enumerate(self.layers):
            qkv = ops.w8_gemm(x, L.qkv, epi=ops.DSK_EPI_PARTIAL)
            k_pool, v_pool, k_sb, v_sb = cache.layer_args(l)
            q = ops.qkv_rope_append(qkv, B, bs, nq, nkv, hd, L.q_norm, L.k_norm, eps, self.inv_freq, cache.seq_lens,
                                    cache.block_table, cache.page, cache.kv_dtype, k_pool, v_pool, k_sb, v_sb)
            win = a.window(l)
            o = ops.attention(q, B, bs, nq, nkv, hd, hd ** -0.5, cache.seq_lens, cache.max_ctx, cache.block_table,
                              cache.page, cache.kv_dtype, k_pool, v_pool, k_sb, v_sb, causal=bool(win), window=win,
                              packed=True)
            op = ops.w8_gemm(o, L.o, epi=ops.DSK_EPI_PARTIAL)
            x = ops.act_pack(M=M, K=H, part=op, h=h, norm_w=L.post_norm, eps=eps)
            act = ops.w8_gemm(x, L.gate_up, epi=ops.DSK_EPI_SWIGLU)
            dp = ops.w8_gemm(act, L.down, epi=ops.DSK_EPI_PARTIAL)
            last = l == nl - 1
            x = ops.act_pack(M=M, K=H, part=dp, h=h, norm_w=None if last else self.layers[l + 1].in_norm, eps=eps,
                             out=not last)
        return h

    def block_logits(self, block_ids: torch.Tensor, cache: PagedKVCache, logits_start: int = 1,
                     cap: int | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
        """Logits of block positions logits_start .. logits_start + cap - 1: [B, cap, V] f32."""
        c = self.config
        B, bs = block_ids.shape
        cap = bs - logits_start if cap is None else cap
        h = self.block_hidden(block_ids, cache).view(B, bs, -1)[:, logits_start:logits_start + cap]
        h = h.reshape(B * cap, -1) if B > 1 else h[0]
        x = ops.pack(h, self.norm, c.rms_norm_eps)
        out = out if out is not None else torch.empty((B * cap, c.vocab_size), dtype=torch.float32,
                                                      device=self.device)
        ops.w8_gemm(x, self.lm_head, out=out, softcap=c.final_logit_softcapping or 0.0)
        return out.view(B, cap, c.vocab_size)

    def __call__(self, inputs, target_hidden, cache, logits_start: int = 0):
        """Reference-shaped call (src/mlx_dspark/dflash_model.py:197-208): ingest the new
        context rows, then return logits for the block positions from logits_start on."""
        if target_hidden is not None and target_hidden.numel():
            self.ingest(target_hidden, cache)
        ids = inputs if torch.is_tensor(inputs) else torch.tensor(inputs)
        ids = ids.to(self.device, torch.int32).reshape(1, -1)
        return self.block_logits(ids, cache, logits_start)
