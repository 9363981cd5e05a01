"""Forward pieces shared by the block drafters (DSpark and DFlash) on gfx950 kernels.

Both drafters condition on the target's hidden states through an EAGLE-style context: the
tapped target states are fused (fc, then RMSNorm) and every drafter layer projects them to
K/V, K normed and roped at its absolute position, and keeps them in a per-layer cache
(src/mlx_dspark/model.py:113-128, :247-256; src/mlx_dspark/dflash_model.py:111-123, :199).
A drafted block then runs the drafter layers over [anchor] + [mask] * (k-1) with attention
over context ++ block, bidirectional (model.py:130-155, dflash_model.py:123-133).

Here the context K/V lives in a PagedKVCache. The block's own K/V is appended after the
cached context in the same pages but outside the cached length, so the next context append
overwrites it (the reference concatenates it on the fly and never stores it).
"""

from __future__ import annotations

import torch

from . import ops
from .kv import PagedKVCache
from .qwen3 import MAX_ROWS


def ingest_context(d, target_hidden: torch.Tensor, cache: PagedKVCache, n_valid=None) -> None:
    """Append context rows for drafter ``d``: target_hidden [S, n_tap*H] (or [1, S, .]) bf16.

    ``d`` provides config (hidden_size, rms_norm_eps, block_size), args (the attention shape:
    num_key_value_heads, head_dim), fc, hidden_norm, layers (with kv_view / k_norm), inv_freq
    and optionally v_norm (an RMSNorm on V). n_valid (device int32 [1]) advances the cached
    length by n_valid + 1 instead of S: the fixed-shape form used when only a device-side prefix
    of the rows is committed (speculative rounds)."""
    c, a = d.config, d.args
    v_norm = getattr(d, "v_norm", None)
    th = target_hidden.reshape(-1, target_hidden.shape[-1])
    S = th.shape[0]
    if n_valid is not None and S > MAX_ROWS:
        raise ValueError("a device-counted context append must fit one pass")
    cache.check_room(S + c.block_size)
    H = c.hidden_size
    for r0 in range(0, S, MAX_ROWS):
        r1 = min(S, r0 + MAX_ROWS)
        hcp = ops.w8_gemm(ops.pack(th[r0:r1]), d.fc, epi=ops.DSK_EPI_PARTIAL)          # fc(target_hidden)
        xc = ops.act_pack(M=r1 - r0, K=H, part=hcp, norm_w=d.hidden_norm, eps=c.rms_norm_eps)
        for l, L in enumerate(d.layers):
            kv = ops.w8_gemm(xc, L.kv_view(d.args), epi=ops.DSK_EPI_PARTIAL)
            k_pool, v_pool, k_sb, v_sb = cache.layer_args(l)
            ops.qkv_rope_append(kv, 1, r1 - r0, 0, a.num_key_value_heads, a.head_dim, None, L.k_norm,
                                c.rms_norm_eps, d.inv_freq, cache.seq_lens, cache.block_table,
                                cache.page, cache.kv_dtype, k_pool, v_pool, k_sb, v_sb, None, v_norm=v_norm)
        if n_valid is None:
            ops.lens_add(cache.seq_lens, None, r1 - r0)
            cache.note_lengths([cache.lengths[0] + (r1 - r0)])
    if n_valid is not None:
        ops.lens_add(cache.seq_lens, n_valid, 1)


def ingest_rows(d, fused: torch.Tensor, cache: PagedKVCache, n_valid: torch.Tensor) -> None:
    """Batched context append for rows 0 .. B-1 of a multi-row drafter cache: fused [B, W,
    n_tap*H] bf16 holds each row's W candidate positions (at its own cached length); row b
    keeps n_valid[b] + 1 of them (n_valid device int32 [B]), the rest lies past its length
    and is overwritten by the next append."""
    c, a = d.config, d.args
    v_norm = getattr(d, "v_norm", None)
    B, W = fused.shape[0], fused.shape[1]
    if B * W > MAX_ROWS:   # groups of whole batch rows, one kernel pass each
        for b0, b1 in _groups(B, W):
            ingest_rows(d, fused[b0:b1], cache.rows(b0, b1), n_valid[b0:b1])
        return
    H = c.hidden_size
    th = fused.reshape(B * W, -1)
    hcp = ops.w8_gemm(ops.pack(th), d.fc, epi=ops.DSK_EPI_PARTIAL)
    xc = ops.act_pack(M=B * W, K=H, part=hcp, norm_w=d.hidden_norm, eps=c.rms_norm_eps)
    for l, L in enumerate(d.layers):
        kv = ops.w8_gemm(xc, L.kv_view(d.args), epi=ops.DSK_EPI_PARTIAL)
        k_pool, v_pool, k_sb, v_sb = cache.layer_args(l)
        ops.qkv_rope_append(kv, B, W, 0, a.num_key_value_heads, a.head_dim, None, L.k_norm, c.rms_norm_eps,
                            d.inv_freq, cache.seq_lens, cache.block_table, cache.page, cache.kv_dtype, k_pool,
                            v_pool, k_sb, v_sb, None, v_norm=v_norm)
    ops.lens_add(cache.seq_lens[:B], n_valid, 1)


def _groups(B: int, W: int):
    """Groups of whole batch rows with at most 64 rows (B*W) each: one kernel pass per group."""
    if W > MAX_ROWS:
        raise ValueError(f"{W} rows per batch row > {MAX_ROWS}")
    g = MAX_ROWS // W
    return [(b0, min(B, b0 + g)) for b0 in range(0, B, g)]


def block_layers(d, h: torch.Tensor, B: int, bs: int, cache: PagedKVCache, scale: float) -> torch.Tensor:
    """Run drafter ``d``'s decoder layers over the block rows h [B*bs, H] (bf16, updated in
    place) attending to context ++ block; returns h before the final norm. Llama 2-norm layers,
    or sandwich norms when the layers carry attn_out_norm / ff_out_norm (gemma4), with
    d.layer_scalars multiplying each layer's output and d.v_norm normalising V. More than 64
    block rows run as groups of whole batch rows."""
    if B * bs > MAX_ROWS:
        for b0, b1 in _groups(B, bs):
            _block_layers(d, h[b0 * bs:b1 * bs], b1 - b0, bs, cache.rows(b0, b1), scale)
        return h
    return _block_layers(d, h, B, bs, cache, scale)


def _block_layers(d, h: torch.Tensor, B: int, bs: int, cache: PagedKVCache, scale: float) -> torch.Tensor:
    c, a = d.config, d.args
    M, H = B * bs, c.hidden_size
    eps = c.rms_norm_eps
    nq, nkv, hd = a.num_attention_heads, a.num_key_value_heads, a.head_dim
    v_norm = getattr(d, "v_norm", None)
    scalars = getattr(d, "layer_scalars", None)
    x = ops.pack(h, d.layers[0].in_norm, eps)
    nl = len(d.layers)
    for l, L in enumerate(d.layers):
        qkv = ops.w8_gemm(x, L.qkv, epi=ops.DSK_EPI_PARTIAL)
        k_pool, v_pool, k_sb, v_sb = cache.layer_args(l)
        q = ops.qkv_rope_append(qkv, B, bs, nq, nkv, hd, L.q_norm, L.k_norm, eps, d.inv_freq, cache.seq_lens,
                                cache.block_table, cache.page, cache.kv_dtype, k_pool, v_pool, k_sb, v_sb,
                                v_norm=v_norm)
        win = a.window(l)
        o = ops.attention(q, B, bs, nq, nkv, hd, scale, cache.seq_lens, cache.max_ctx, cache.block_table,
                          cache.page, cache.kv_dtype, k_pool, v_pool, k_sb, v_sb, causal=bool(win), window=win,
                          packed=True)
        op = ops.w8_gemm(o, L.o, epi=ops.DSK_EPI_PARTIAL)
        x = ops.act_pack(M=M, K=H, part=op, h=h, norm_w=L.post_norm, eps=eps, part_norm_w=L.attn_out_norm)
        act = ops.w8_gemm(x, L.gate_up, epi=d.act_epi)
        dp = ops.w8_gemm(act, L.down, epi=ops.DSK_EPI_PARTIAL)
        last = l == nl - 1
        x = ops.act_pack(M=M, K=H, part=dp, h=h, norm_w=None if last else d.layers[l + 1].in_norm, eps=eps,
                         out=not last, part_norm_w=L.ff_out_norm, scale=scalars[l] if scalars else 1.0)
    return h


def head_rows(d, h_rows: torch.Tensor, lm_head, out: torch.Tensor | None = None) -> torch.Tensor:
    """logits = lm_head(norm(h_rows)) (+ soft-cap) for h_rows [R, H] bf16 -> f32 [R, V]."""
    c = d.config
    out = out if out is not None else torch.empty((h_rows.shape[0], lm_head.N), dtype=torch.float32,
                                                  device=h_rows.device)
    for r0 in range(0, h_rows.shape[0], MAX_ROWS):
        r1 = min(h_rows.shape[0], r0 + MAX_ROWS)
        x = ops.pack(h_rows[r0:r1], d.norm, c.rms_norm_eps)
        ops.w8_gemm(x, lm_head, out=out[r0:r1], softcap=c.final_logit_softcapping or 0.0)
    return out
