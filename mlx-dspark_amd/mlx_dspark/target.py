"""Target wrapper: KV cache factory + verify forward with a hidden-state tap.

Same surface as the reference's Target (src/mlx_dspark/target.py:16-128): ``make_cache()``,
``run(ids, cache, tap) -> (logits [1, L, V], fused [1, L, n_tap*H])``, ``plain(ids, cache)``,
``verify_tap()``, and the attributes callers read (model, tokenizer, is_vlm, family,
kv_bits, kv_group_size). Tensors are torch tensors on the HIP device.
"""

from __future__ import annotations

import torch

from .qwen3 import MAX_ROWS, Qwen3W8


def _as_ids(ids, device) -> torch.Tensor:
    if not torch.is_tensor(ids):
        ids = torch.tensor(ids)
    ids = ids.to(device=device, dtype=torch.int32)
    return ids.reshape(1, -1) if ids.dim() == 1 else ids


class Target:
    def __init__(self, model: Qwen3W8, tokenizer, *, kv_bits: int | None = None, kv_group_size: int = 64,
                 max_ctx: int | None = None):
        self.model = model
        self.tokenizer = tokenizer
        self.is_vlm = False
        mt = getattr(model.args, "model_type", "qwen3")
        self.family = "gemma4" if mt.startswith("gemma") else mt
        if kv_bits not in (None, 8):
            raise ValueError(f"kv_bits={kv_bits}: the engine supports 8-bit KV (or bf16)")
        if kv_group_size != 64:
            raise ValueError("KV quantization uses group size 64")
        self.kv_bits = int(kv_bits) if kv_bits else None
        self.kv_group_size = int(kv_group_size)
        self.max_ctx = max_ctx
        self._tied = bool(model.args.tie_word_embeddings)

    # -- cache --
    def make_cache(self, B: int = 1, max_ctx: int | None = None, spare_rows: int = 0):
        return self.model.make_cache(B, max_ctx or self.max_ctx, self.kv_bits, spare_rows=spare_rows)

    # -- forward with hidden-state tap --
    def run(self, ids, cache, tap):
        """ids [1, L] -> (logits [1, L, V] f32, fused [1, L, n_tap*H] bf16); advances cache by L."""
        ids = _as_ids(ids, self.model.device)
        L = ids.shape[1]
        cache.check_room(L)
        outs, fus = [], []
        for c0 in range(0, L, MAX_ROWS):
            lg, fu = self.model.forward(ids[:, c0:c0 + MAX_ROWS], cache, tap)
            outs.append(lg)
            fus.append(fu)
        logits = outs[0] if len(outs) == 1 else torch.cat(outs, dim=1)
        fused = None
        if fus[0] is not None:
            fused = fus[0] if len(fus) == 1 else torch.cat(fus, dim=1)
        return logits, fused

    # -- plain forward (no capture) --
    def plain(self, ids, cache):
        return self.run(ids, cache, None)[0]

    # -- tap sanity probe --
    def verify_tap(self) -> None:
        """The tapped forward and the plain forward are one code path here; the probe still
        checks structure (windowed layers cannot be tapped by one causal mask in the
        reference's generic loop) and that both give the same logits on 4 tokens."""
        a = self.model.args
        # The reference refuses windowed layers because its tap replays mlx_lm's loop with one
        # causal mask; this engine's forward is the model itself (per-layer windows included),
        # so only a family it does not implement is refused.
        if a.layer_types and any(t != "full_attention" for t in a.layer_types) and not a.sandwich_norms:
            raise ValueError(f"hidden-state tap unsupported for model_type {self.family!r}: it uses "
                             f"windowed/alternating attention layers")
        ids = [[1, 2, 3, 4]]
        ref = self.plain(ids, self.make_cache(max_ctx=64))
        got, _ = self.run(ids, self.make_cache(max_ctx=64), [0])
        diff = float((ref - got).abs().max())
        if diff > 1e-3:
            raise ValueError(f"hidden-state tap unsupported for model_type {self.family!r}: the tapped "
                             f"forward diverges from the plain one (max |dlogit| = {diff:.4g})")
