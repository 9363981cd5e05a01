"""DSpark drafter on gfx950 kernels (drop-in for src/mlx_dspark/model.py).

Behaviour follows the reference's DSparkDrafter (model.py:220-320), both families:
  - context: fused = RMSNorm(fc(concat of tapped target states)); per layer K = rope(k_norm(
    k_proj(fused)), ctx_offset + i), V = v_proj(fused) (qwen3) or, with gemma4's k_eq_v,
    V = v_norm(k_proj(fused)) (an RMSNorm without weight on the un-normed, un-roped k
    projection), appended to the layer's context cache (:113-128, :247-256);
  - block: [pending] + [mask] * (k-1) embedded (x embed_scale: sqrt(hidden) for gemma4), then
    the layers, attention bidirectional over context ++ block, roped at block_offset =
    committed length (:130-193, :258-262), final RMSNorm. qwen3: Llama 2-norm layers, SiLU MLP,
    scale head_dim^-1/2. gemma4: sandwich norms (post-attention and post-feedforward norms of
    the projection outputs before their residual adds) and the layer_scalar multiply (:172-184),
    tanh-GeLU MLP, attention scale 1, head_dim = global_head_dim over the global kv heads,
    proportional RoPE (the first partial_rotary_factor of the rotate-half frequencies, exponents
    over the full head_dim; the rest pass through);
  - heads: logits = lm_head(h[:cap]) (+ tanh soft-cap) (:264-268); Markov block sampling
    tok_i = argmax(logits_i + w2(w1[tok_{i-1}])) (:270-281) or its sampled form (:283-309); the
    confidence head sigmoid(Linear(concat(h, w1[prev]))) (:311-320).
The context cache is a PagedKVCache; the block's K/V sits past its cached length.
"""

from __future__ import annotations

import torch

from . import blockdraft, ops
from .config import DSparkConfig
from .kv import PagedKVCache
from .ops import W8Table, W8Weight
from .qwen3 import LayerWeights, TargetArgs


class MarkovHead:
    """Rank-R previous-token correction, logits += w2(w1[prev]) (model.py:196-208)."""

    def __init__(self, w1: W8Table, w2: W8Weight):
        self.w1, self.w2 = w1, w2

    def prev_embeddings(self, token_ids: torch.Tensor) -> torch.Tensor:
        return ops.w8_embed(token_ids.reshape(-1), self.w1)

    def step_bias(self, token_ids: torch.Tensor) -> torch.Tensor:
        """[n] token ids -> bf16-valued f32 [n, V] biases."""
        e = self.prev_embeddings(token_ids)
        y = ops.w8_gemm(ops.pack(e), self.w2, out_dtype=torch.float32)
        return y.to(torch.bfloat16).float()


class ConfidenceHead:
    """sigmoid(proj(features)) features -> scalar (model.py:211-217): a 1-row linear with bias,
    stored as a W8 weight padded to 16 rows (row 0 is the projection)."""

    def __init__(self, proj: W8Weight, bias: float):
        self.proj, self.bias = proj, float(bias)

    def __call__(self, features: torch.Tensor) -> torch.Tensor:
        y = ops.w8_gemm(ops.pack(features), self.proj, out_dtype=torch.float32)
        return y[:, 0] + self.bias


class DSparkDrafter:
    def __init__(self, config: DSparkConfig, *, embed: W8Table, fc: W8Weight, hidden_norm: torch.Tensor,
                 layers: list[LayerWeights], norm: torch.Tensor, lm_head: W8Weight,
                 markov: MarkovHead | None = None, confidence: ConfidenceHead | None = None,
                 layer_scalars: list[float] | None = None):
        """layers: the qkv projection is [q | k | v] rows; with k_eq_v the v rows repeat the k
        rows (the shared k_proj). layer_scalars: gemma4's per-layer output multipliers."""
        if config.family not in ("qwen3", "gemma4"):
            raise ValueError(f"DSpark family {config.family!r}: qwen3 or gemma4")
        gemma = config.family == "gemma4"
        if gemma and config.attention_k_eq_v and not config.use_v_norm:
            raise ValueError("gemma4 k_eq_v drafter without v_norm")
        self.config = config
        self.block_size = config.block_size
        self.mask_token_id = config.mask_token_id
        self.embed_scale = float(config.hidden_size) ** 0.5 if gemma else 1.0
        self.softcap = config.final_logit_softcapping
        self.embed_tokens = embed
        self.fc = fc
        self.hidden_norm = hidden_norm
        self.layers = layers
        self.norm = norm
        self.lm_head = lm_head
        self.markov_head = markov
        self.confidence_head = confidence
        self.device = norm.device
        hd, nkv = config.attn_head_dim, config.n_kv_heads
        self.args = TargetArgs(hidden_size=config.hidden_size, num_hidden_layers=config.num_hidden_layers,
                               intermediate_size=config.intermediate_size,
                               num_attention_heads=config.num_attention_heads,
                               num_key_value_heads=nkv, head_dim=hd,
                               vocab_size=config.vocab_size, rms_norm_eps=config.rms_norm_eps,
                               rope_theta=config.rope_theta)
        frac = config.partial_rotary_factor if config.rope_type == "proportional" else 1.0
        self.inv_freq = ops.rope_inv_freq(hd, config.rope_theta, self.device, rotary_fraction=frac)
        # RMSNorm without weight on V (gemma4 v_norm): a unit weight
        self.v_norm = torch.ones(hd, dtype=torch.bfloat16, device=self.device) if config.use_v_norm else None
        self.layer_scalars = [float(x) for x in layer_scalars] if layer_scalars is not None else None
        self.act_epi = ops.DSK_EPI_SWIGLU if config.mlp_activation == "silu" else ops.DSK_EPI_GEGLU

    # ---------------------------------------------------------------- context
    def embed(self, ids) -> torch.Tensor:
        ids = torch.as_tensor(ids, device=self.device).to(torch.int32)
        shape = tuple(ids.shape)
        out = ops.w8_embed(ids.reshape(-1), self.embed_tokens, self.embed_scale)
        return out.view(*shape, -1)

    def make_ctx_cache(self, max_ctx: int = 16384, B: int = 1, spare_rows: int = 0) -> PagedKVCache:
        """Per-layer context K/V (the reference's [CtxCache] * n_layers, model.py:48-80, 250-251)."""
        c = self.config
        return PagedKVCache(c.num_hidden_layers, B, c.n_kv_heads, c.attn_head_dim, max_ctx + c.block_size,
                            device=self.device, spare_rows=spare_rows)

    def update_context(self, target_hidden_cat: torch.Tensor, ctx_offset: int, ctx_caches: PagedKVCache,
                       n_valid=None) -> None:
        """Append the fused target states of committed positions ctx_offset.. (model.py:253-256).
        n_valid (device int32 [1]): only rows 0..n_valid are committed (device-side length)."""
        if n_valid is None and ctx_offset != ctx_caches.lengths[0]:
            raise ValueError(f"context offset {ctx_offset} != cached context length {ctx_caches.lengths[0]}")
        blockdraft.ingest_context(self, target_hidden_cat, ctx_caches, n_valid)

    # ---------------------------------------------------------------- block
    def block_hidden(self, block_ids: torch.Tensor, ctx_caches: PagedKVCache) -> torch.Tensor:
        """block_ids [B, k] int32 -> pre-norm hidden [B*k, H] bf16 (positions from the cache)."""
        B, k = block_ids.shape
        h = ops.w8_embed(block_ids.reshape(-1), self.embed_tokens, self.embed_scale)
        return blockdraft.block_layers(self, h, B, k, ctx_caches, self.config.scaling)

    def backbone(self, noise_embedding: torch.Tensor, block_offset, ctx_caches: PagedKVCache,
                 mask=None) -> torch.Tensor:
        """Reference-shaped backbone (model.py:258-262): noise [B, k, H] bf16 -> normed [B, k, H]."""
        if mask is not None:
            raise NotImplementedError("padding masks: batched drafting runs on per-row paged contexts")
        B, k, H = noise_embedding.shape
        lens = ctx_caches.lengths
        offs = [int(block_offset)] * B if isinstance(block_offset, int) else [int(x) for x in block_offset]
        if offs != lens[:B]:
            raise ValueError(f"block offset {offs} != cached context lengths {lens[:B]}")
        h = noise_embedding.reshape(B * k, H).to(torch.bfloat16).contiguous().clone()
        h = blockdraft.block_layers(self, h, B, k, ctx_caches, self.config.scaling)
        return ops.pack(h, self.norm, self.config.rms_norm_eps).unpack().view(B, k, H)

    def compute_logits(self, hidden: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        """lm_head(hidden) (+ soft-cap) for normed hidden [..., H] -> f32 [..., V] (model.py:264-268)."""
        shp = hidden.shape[:-1]
        x = ops.pack(hidden.reshape(-1, hidden.shape[-1]).to(torch.bfloat16))
        y = ops.w8_gemm(x, self.lm_head, out=out, out_dtype=torch.float32, softcap=self.softcap or 0.0)
        return y.view(*shp, -1)

    def block_logits(self, block_ids: torch.Tensor, ctx_caches: PagedKVCache, cap: int,
                     out: torch.Tensor | None = None) -> torch.Tensor:
        """Base logits of block positions 0 .. cap-1: [B, cap, V] f32 (the final norm fused
        into the head's activation pack)."""
        B, k = block_ids.shape
        h = self.block_hidden(block_ids, ctx_caches).view(B, k, -1)[:, :cap]
        h = h.reshape(B * cap, -1) if B > 1 else h[0]
        return blockdraft.head_rows(self, h, self.lm_head, out).view(B, cap, -1)

    # ---------------------------------------------------------------- heads
    def _first_prev(self, first_prev_token, B: int) -> torch.Tensor:
        if torch.is_tensor(first_prev_token):
            return first_prev_token.reshape(-1).to(self.device, torch.int32)
        vals = [int(first_prev_token)] * B if isinstance(first_prev_token, int) else [int(x) for x in first_prev_token]
        return torch.tensor(vals, dtype=torch.int32, device=self.device)

    def sample_block(self, base_logits: torch.Tensor, first_prev_token, out: torch.Tensor | None = None):
        """Greedy block tokens (model.py:270-281): base_logits [cap, V] or [B, cap, V] f32 ->
        int32 [cap] / [B, cap] on device (argmax per position without a Markov head)."""
        squeeze = base_logits.dim() == 2
        bl = base_logits.unsqueeze(0) if squeeze else base_logits
        B, cap, V = bl.shape
        if self.markov_head is None:
            tok, _ = ops.sample_rows(bl.reshape(B * cap, V), 0.0, token_out=None if out is None else out.view(-1))
            tok = tok.view(B, cap)
        else:
            tok = ops.markov_block(bl, self._first_prev(first_prev_token, B), self.markov_head.w1,
                                   self.markov_head.w2, tok_out=None if out is None else out.view(B, cap))
        return tok[0] if squeeze else tok

    def sample_block_probs(self, base_logits: torch.Tensor, first_prev_token, temperature: float,
                           top_p: float = 1.0, top_k: int = 0, *, seed: int = 0, offset: int = 0):
        """Sampled block (model.py:283-309): (tokens int32 [cap], q_logits f32 [cap, V]).

        Each token is drawn from truncate(softmax(l_i * (1/T))); the second value holds the l_i,
        whose distribution dsk_accept_sample rebuilds with q_mul_inv_t=1 (the reference returns
        the probabilities themselves)."""
        squeeze = base_logits.dim() == 2
        bl = base_logits.unsqueeze(0) if squeeze else base_logits
        B, cap, V = bl.shape
        if self.markov_head is None:
            ql = bl.float().contiguous()
            tok = torch.empty((B, cap), dtype=torch.int32, device=self.device)
            for b in range(B):
                ops.sample_rows(ql[b], temperature, top_p, top_k, mul_inv_t=True, seed=seed, offset=offset,
                                row0=b * cap, token_out=tok[b])
        else:
            tok, ql = ops.markov_block(bl, self._first_prev(first_prev_token, B), self.markov_head.w1,
                                       self.markov_head.w2, temperature=temperature, top_p=top_p, top_k=top_k,
                                       seed=seed, offset=offset)
        return (tok[0], ql[0]) if squeeze else (tok, ql)

    def confidence_logits(self, block_hidden: torch.Tensor, prev_token_ids) -> torch.Tensor | None:
        """Confidence logits of normed block rows [cap, H] given their previous tokens
        (model.py:311-320)."""
        if self.confidence_head is None:
            return None
        feats = block_hidden.reshape(-1, block_hidden.shape[-1]).to(torch.bfloat16)
        if self.config.confidence_head_with_markov:
            prev = torch.as_tensor(prev_token_ids, device=self.device).reshape(-1).to(torch.int32)
            feats = torch.cat([feats, self.markov_head.prev_embeddings(prev)], dim=-1)
        return self.confidence_head(feats.contiguous())


Gemma4DSparkDrafter = DSparkDrafter
