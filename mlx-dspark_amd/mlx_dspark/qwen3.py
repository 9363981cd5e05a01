"""Qwen3-shaped W8 decoder (the speculative-decoding target) on gfx950 kernels.

The reference runs the target through mlx_lm (external) and replicates its layer loop to
tap hidden states (src/mlx_dspark/target.py:58-75). This module is the engine's own
forward over the same public Qwen3 architecture:
    h = embed(ids)
    per layer: h += o(attn(rope(q_norm(q)), rope(k_norm(k)), v))   q,k,v from RMSNorm(h)
               h += down(silu(gate) * up)                           from RMSNorm(h)
    logits = lm_head(RMSNorm(h))       (tied: embed_tokens.as_linear)
with the residual stream captured after the tapped layers. Every projection is W8 (affine
group 64, bf16 scale/bias); activations are bf16 between kernels, accumulation is fp32,
logits are fp32.

The same forward runs the Gemma-style layout (model_type gemma*): embedding scaled by
sqrt(hidden) (rounded to bf16), sandwich norms (the attention and MLP outputs are RMSNorm-ed
before their residual adds, fused into the act_pack that follows each projection), GeGLU
(tanh-approximated GeLU), sliding-window layers with their own RoPE base, a query scale of
query_pre_attn_scalar ** -0.5 and a final logit soft-cap. Norm gains are stored as the
effective multipliers (gemma's 1 + w).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import ops
from .kv import PagedKVCache
from .ops import DSK_EPI_GEGLU, DSK_EPI_SWIGLU, W8Table, W8Weight

MAX_ROWS = 64  # rows per kernel pass (M of the skinny GEMM)
DENSE_MIN_ROWS = 256   # prompts from this length prefill layer by layer through the library GEMM
PREFILL_CHUNK = 2048   # prompt rows handed to a drafter per on_chunk call (generate.py:613-656)


@dataclass
class TargetArgs:
    """The model-config fields the engine reads (names follow the HF / mlx_lm config)."""

    model_type: str = "qwen3"
    hidden_size: int = 1024
    num_hidden_layers: int = 28
    intermediate_size: int = 3072
    num_attention_heads: int = 16
    num_key_value_heads: int = 8
    head_dim: int = 128
    vocab_size: int = 151936
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    tie_word_embeddings: bool = False
    max_position_embeddings: int = 40960
    hidden_act: str = "silu"                       # "silu" | "gelu_tanh"
    embed_scale: float = 1.0                       # gemma: sqrt(hidden_size)
    sliding_window: int | None = None
    layer_types: tuple = field(default_factory=tuple)   # "full_attention" | "sliding_attention"
    final_logit_softcapping: float | None = None
    query_pre_attn_scalar: float | None = None    # attention scale = this ** -0.5 when set
    rope_local_base_freq: float | None = None     # RoPE base of the sliding-window layers

    @property
    def sandwich_norms(self) -> bool:
        return self.model_type.startswith("gemma")

    @property
    def n_qkv(self) -> int:
        return (self.num_attention_heads + 2 * self.num_key_value_heads) * self.head_dim

    @property
    def attn_scale(self) -> float:
        s = self.query_pre_attn_scalar or self.head_dim
        return float(s) ** -0.5

    def is_sliding(self, layer: int) -> bool:
        return bool(self.layer_types) and self.layer_types[layer] == "sliding_attention"

    def window(self, layer: int) -> int:
        if self.is_sliding(layer) and self.sliding_window:
            return int(self.sliding_window)
        return 0


@dataclass
class LayerWeights:
    qkv: W8Weight          # [q | k | v] rows, N = (nq + 2 nkv) * hd, K = hidden
    o: W8Weight            # N = hidden, K = nq * hd
    gate_up: W8Weight      # [gate | up] rows, N = 2 * intermediate, paired layout
    down: W8Weight         # N = hidden, K = intermediate
    in_norm: torch.Tensor  # bf16 [hidden]
    post_norm: torch.Tensor
    q_norm: torch.Tensor   # bf16 [head_dim]
    k_norm: torch.Tensor
    attn_out_norm: torch.Tensor | None = None  # sandwich norms: attention output before its add
    ff_out_norm: torch.Tensor | None = None    # sandwich norms: MLP output before its add

    def kv_view(self, args: TargetArgs) -> W8Weight:
        """The [k | v] rows of the fused projection, as a zero-copy W8 view."""
        nq_rows = args.num_attention_heads * args.head_dim
        return self.qkv.rows(nq_rows, nq_rows + 2 * args.num_key_value_heads * args.head_dim)


class Qwen3W8:
    """Weights + forward. Mirrors the pieces of an mlx_lm model that callers touch
    (``args``, ``layers``); ``model.embed_tokens`` / ``lm_head`` are W8 objects."""

    def __init__(self, args: TargetArgs, layers: list[LayerWeights], embed: W8Table,
                 lm_head: W8Weight, norm: torch.Tensor):
        self.args = args
        self.layers = layers
        self.embed = embed
        self.lm_head = lm_head
        self.norm = norm
        self.device = norm.device
        self.inv_freq = ops.rope_inv_freq(args.head_dim, args.rope_theta, self.device)
        self.inv_freq_local = (ops.rope_inv_freq(args.head_dim, args.rope_local_base_freq, self.device)
                               if args.rope_local_base_freq else self.inv_freq)
        self.act_epi = DSK_EPI_SWIGLU if args.hidden_act == "silu" else DSK_EPI_GEGLU
        self._dense_w = None   # bf16 rows of every layer's weights, when keep_dense_weights holds them
        self._prefetch = None  # (side stream, sink, workgroups) when prefetch_weights is on

    # ------------------------------------------------------------------ cache
    def make_cache(self, B: int = 1, max_ctx: int | None = None, kv_bits: int | None = None,
                   page: int = 64, spare_rows: int = 0) -> PagedKVCache:
        a = self.args
        max_ctx = max_ctx or min(a.max_position_embeddings, 16384)
        return PagedKVCache(a.num_hidden_layers, B, a.num_key_value_heads, a.head_dim, max_ctx,
                            page=page, kv_bits=kv_bits, device=self.device, spare_rows=spare_rows)

    @property
    def weight_bytes(self) -> int:
        t = self.lm_head.nbytes
        for L in self.layers:
            t += L.qkv.nbytes + L.o.nbytes + L.gate_up.nbytes + L.down.nbytes
        return t

    def prefetch_weights(self, on: bool = True, workgroups: int = 512) -> None:
        """Overlap experiment (off by default): each Qwen3-layout layer forks a side stream after
        its q/k/v projection that reads the layer's o and gate|up weights (dsk_prefetch) while the
        RoPE/append, attention and combine run, so those GEMMs find their weights in the
        memory-side cache; the forward joins the side stream before it returns."""
        if not on:
            self._prefetch = None
            return
        self._prefetch = (torch.cuda.Stream(device=self.device),
                          torch.zeros(4, dtype=torch.int32, device=self.device), int(workgroups))

    # ------------------------------------------------------------------ forward
    def embed_rows(self, ids: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        return ops.w8_embed(ids, self.embed, self.args.embed_scale, out=out)

    def layer(self, l: int, x: ops.Packed, h: torch.Tensor, B: int, W: int, cache: PagedKVCache, *,
              causal: bool = True, next_norm: torch.Tensor | None = None, copy: torch.Tensor | None = None,
              want_next: bool = True) -> ops.Packed | None:
        """One decoder layer. x: this layer's input, RMSNorm(h) packed (normed later in the
        Qwen3 layout); h [B*W, H] bf16 residual stream (updated in place). Returns the next
        projection's packed input, RMSNorm(h_out) with next_norm (the next layer's input norm or
        the final norm), or the plain packed h_out when next_norm is None; None when want_next is
        False. copy, when given, receives h_out (hidden-state tap)."""
        a = self.args
        L = self.layers[l]
        nq, nkv, hd = a.num_attention_heads, a.num_key_value_heads, a.head_dim
        M, H = B * W, a.hidden_size
        eps = a.rms_norm_eps
        # a normed-later x: the split-K partials take its row scale where they are summed
        qkv = ops.w8_gemm(x.plain(), L.qkv, epi=ops.DSK_EPI_PARTIAL)
        if self._prefetch is not None and not a.sandwich_norms:
            side, sink, wg = self._prefetch
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                ops.prefetch(L.o, sink, wg)
                ops.prefetch(L.gate_up, sink, wg)
        k_pool, v_pool, k_sb, v_sb = cache.layer_args(l)
        inv_freq = self.inv_freq_local if a.is_sliding(l) else self.inv_freq
        q = ops.qkv_rope_append(qkv, B, W, nq, nkv, hd, L.q_norm, L.k_norm, eps, inv_freq,
                                cache.seq_lens, cache.block_table, cache.page, cache.kv_dtype,
                                k_pool, v_pool, k_sb, v_sb, x=x)
        o = ops.attention(q, B, W, nq, nkv, hd, a.attn_scale, cache.seq_lens, cache.max_ctx,
                          cache.block_table, cache.page, cache.kv_dtype, k_pool, v_pool, k_sb, v_sb,
                          causal=causal, window=a.window(l), packed=True)
        if not a.sandwich_norms:
            # the residual adds run in the o / down epilogues, each next RMSNorm in the GEMM that
            # consumes it (normed later)
            x = ops.w8_residual(o, L.o, h, next_norm=L.post_norm, eps=eps)
            act = ops.w8_gemm(x, L.gate_up, epi=self.act_epi)
            return ops.w8_residual(act, L.down, h, next_norm=next_norm, eps=eps, copy=copy, out=want_next)
        op = ops.w8_gemm(o, L.o, epi=ops.DSK_EPI_PARTIAL)
        x = ops.act_pack(M=M, K=H, part=op, h=h, norm_w=L.post_norm, eps=eps, part_norm_w=L.attn_out_norm)
        act = ops.w8_gemm(x, L.gate_up, epi=self.act_epi)
        dp = ops.w8_gemm(act, L.down, epi=ops.DSK_EPI_PARTIAL)
        return ops.act_pack(M=M, K=H, part=dp, h=h, copy=copy, norm_w=next_norm, eps=eps, out=want_next,
                            part_norm_w=L.ff_out_norm)

    def forward(self, ids: torch.Tensor, cache: PagedKVCache, tap=None, *, advance: bool = True,
                logits: str = "all", logits_out: torch.Tensor | None = None,
                fused_out: torch.Tensor | None = None, h_out: torch.Tensor | None = None):
        """ids [B, W] int32 on device (W <= 64 rows per batch row).

        Positions come from cache.seq_lens (device). Returns (logits [B, W or 1, V] f32 or
        None, fused [B, W, n_tap*H] bf16 or None). advance=True moves seq_lens by W; the
        speculative loops pass False and let the acceptance kernel apply n + 1. A batch of
        more than 64 rows runs as groups of whole batch rows, at most 64 rows each (the row
        limit of one kernel pass), each group on a view of its rows of the cache."""
        a = self.args
        B, W = ids.shape
        M = B * W
        if W > MAX_ROWS:
            raise ValueError(f"forward pass of {W} rows per batch row > {MAX_ROWS}; chunk the prompt")
        if M > MAX_ROWS:
            return self._forward_groups(ids, cache, tap, advance=advance, logits=logits, logits_out=logits_out,
                                        fused_out=fused_out, h_out=h_out)
        H = a.hidden_size
        eps = a.rms_norm_eps
        tap = list(tap or [])
        slots: dict = {}
        for i, t in enumerate(tap):
            slots.setdefault(t, []).append(i)
        h = h_out if h_out is not None else torch.empty((M, H), dtype=torch.bfloat16, device=self.device)
        self.embed_rows(ids.reshape(-1), out=h)
        fused = None
        if tap:
            fused = fused_out if fused_out is not None else torch.empty(
                (M, len(tap) * H), dtype=torch.bfloat16, device=self.device)
        nl = a.num_hidden_layers
        if a.sandwich_norms:
            x = ops.pack(h, self.layers[0].in_norm, eps)
        else:
            x = ops.pack_rn(M=M, K=H, h=h, norm_w=self.layers[0].in_norm, eps=eps)
        for l in range(nl):
            last = l == nl - 1
            s = slots.get(l, ())
            copy = fused[:, s[0] * H:(s[0] + 1) * H] if s else None
            if not last:
                x = self.layer(l, x, h, B, W, cache, next_norm=self.layers[l + 1].in_norm, copy=copy)
            else:   # the final norm is fused into the last residual add when every row needs logits
                x = self.layer(l, x, h, B, W, cache, next_norm=self.norm, copy=copy, want_next=logits == "all")
            for extra in s[1:]:
                fused[:, extra * H:(extra + 1) * H].copy_(fused[:, s[0] * H:(s[0] + 1) * H])
        out = None
        if logits != "none":
            if logits != "all":
                hl = h.view(B, W, H)[:, -1]
                if a.sandwich_norms:
                    x = ops.pack(hl, self.norm, eps)
                else:   # normed later, as the all-rows head is: both round the same way
                    x = ops.pack_rn(M=B, K=H, h=hl, norm_w=self.norm, eps=eps)
            Mr = x.M
            out = logits_out if logits_out is not None else torch.empty(
                (Mr, a.vocab_size), dtype=torch.float32, device=self.device)
            ops.w8_gemm(x, self.lm_head, out=out, softcap=a.final_logit_softcapping or 0.0)
            out = out.view(B, W if logits == "all" else 1, a.vocab_size)
        if advance:
            ops.lens_add(cache.seq_lens, None, W)
            cache.note_lengths([l + W for l in cache.lengths])
        if self._prefetch is not None:
            torch.cuda.current_stream().wait_stream(self._prefetch[0])   # join the side stream
        return out, (fused.view(B, W, -1) if fused is not None else None)

    def _forward_groups(self, ids, cache, tap, *, advance, logits, logits_out, fused_out, h_out):
        """forward over groups of floor(64 / W) batch rows; outputs land in row slices of one
        buffer each, so the result is the same [B, ...] tensors a single pass returns."""
        a = self.args
        B, W = ids.shape
        g = MAX_ROWS // W
        per = W if logits == "all" else 1
        out = None
        if logits != "none":
            out = logits_out if logits_out is not None else torch.empty(
                (B * per, a.vocab_size), dtype=torch.float32, device=self.device)
            out = out.view(B * per, a.vocab_size)
        fused = None
        if tap:
            fused = fused_out if fused_out is not None else torch.empty(
                (B * W, len(tap) * a.hidden_size), dtype=torch.bfloat16, device=self.device)
            fused = fused.view(B * W, -1)
        h_all = h_out.view(B * W, -1) if h_out is not None else None
        for b0 in range(0, B, g):
            b1 = min(B, b0 + g)
            self.forward(ids[b0:b1], cache.rows(b0, b1), tap, advance=advance, logits=logits,
                         logits_out=None if out is None else out[b0 * per:b1 * per],
                         fused_out=None if fused is None else fused[b0 * W:b1 * W],
                         h_out=None if h_all is None else h_all[b0 * W:b1 * W])
        return (None if out is None else out.view(B, per, a.vocab_size),
                None if fused is None else fused.view(B, W, -1))

    def head_logits(self, h: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        """lm_head(norm(h)) for h [M, H] bf16 (DFlash reuses the target head)."""
        a = self.args
        out = out if out is not None else torch.empty((h.shape[0], a.vocab_size), dtype=torch.float32,
                                                      device=self.device)
        for m0 in range(0, h.shape[0], MAX_ROWS):
            m1 = min(h.shape[0], m0 + MAX_ROWS)
            x = ops.pack(h[m0:m1], self.norm, a.rms_norm_eps)
            ops.w8_gemm(x, self.lm_head, out=out[m0:m1], softcap=a.final_logit_softcapping or 0.0)
        return out

    def prefill(self, ids: list[int] | torch.Tensor, cache: PagedKVCache, tap=None, *, chunk: int = MAX_ROWS,
                on_chunk=None, dense: bool | None = None):
        """Single-row prefill. Returns (last-position logits [1, 1, V], fused of the whole prompt
        [1, L, n_tap*H] or None). on_chunk(fused_chunk, pos) lets a drafter ingest the hidden
        states chunk by chunk. A Qwen3-layout prompt of DENSE_MIN_ROWS rows or more runs layer
        by layer over all its rows (prefill_dense); shorter ones (or dense=False) in forward
        passes of ``chunk`` rows."""
        if not torch.is_tensor(ids):
            ids = torch.tensor(ids, dtype=torch.int32)
        ids = ids.reshape(1, -1).to(self.device, torch.int32)
        L = ids.shape[1]
        cache.check_room(L)
        if dense is None:
            dense = L >= DENSE_MIN_ROWS and not self.args.sandwich_norms
        if dense:
            return self.prefill_dense(ids, cache, tap, on_chunk=on_chunk)
        parts = []
        out = None
        pos = cache.lengths[0]
        for c0 in range(0, L, chunk):
            c1 = min(L, c0 + chunk)
            last = c1 == L
            out, fused = self.forward(ids[:, c0:c1], cache, tap, logits="last" if last else "none")
            if fused is not None:
                if on_chunk is not None:
                    on_chunk(fused, pos)
                else:
                    parts.append(fused)
            pos += c1 - c0
        fused_all = None
        if parts:
            fused_all = parts[0] if len(parts) == 1 else torch.cat(parts, dim=1)
        return out, fused_all


    # ------------------------------------------------------------------ dense prefill
    def keep_dense_weights(self, keep: bool = True) -> int:
        """Hold every layer's weights expanded to bf16 rows in HBM for the dense prefill (two
        bytes per weight: 15.1 GB for the Qwen3-8B shape, against 8 GB of 8-bit codes), so a
        prefill multiplies them directly instead of expanding each layer's four matrices first
        (4 ms of a 4096-token prefill). The rows are the ones the per-layer expansion writes, bit
        for bit. keep=False releases them. Returns the bytes held."""
        if not keep:
            self._dense_w = None
            return 0
        if self._dense_w is None:
            self._dense_w = [{k: ops.w8_dequant(getattr(Lw, k)) for k in ("qkv", "o", "gate_up", "down")}
                             for Lw in self.layers]
        return sum(t.numel() * t.element_size() for d in self._dense_w for t in d.values())

    def prefill_dense(self, ids: torch.Tensor, cache: PagedKVCache, tap=None, *, on_chunk=None,
                      chunk: int = PREFILL_CHUNK):
        """Prefill of a long prompt, layer by layer over all L rows (the reference's chunked
        _prefill_tapped, generate.py:613-656, computes the same causal result): each layer's W8
        weights are expanded to bf16 once (dsk_w8_dequant_rows; or held expanded, see
        keep_dense_weights) and multiplied by the library GEMM (hipBLASLt through torch.matmul /
        addmm, whose beta = 1 form is the fused residual add), between the engine's RMSNorm,
        q/k-norm + RoPE + KV append, many-query attention and SwiGLU kernels. The norms here
        normalise first. Returns what prefill() returns."""
        a = self.args
        if a.sandwich_norms:
            raise ValueError("prefill_dense: the Qwen3 layout only")
        ids = ids.reshape(1, -1)
        L = ids.shape[1]
        cache.check_room(L)
        H, I, eps = a.hidden_size, a.intermediate_size, a.rms_norm_eps
        nq, nkv, hd = a.num_attention_heads, a.num_key_value_heads, a.head_dim
        dev = self.device
        tap = list(tap or [])
        h = self.embed_rows(ids.reshape(-1))
        fused = torch.empty((L, len(tap) * H), dtype=torch.bfloat16, device=dev) if tap else None
        held = self._dense_w
        wbuf = None
        if held is None:
            wbuf = torch.empty(max(a.n_qkv * H, H * nq * hd, 2 * I * H, H * I), dtype=torch.bfloat16, device=dev)

        def rows(l, name):
            return held[l][name] if held is not None else ops.w8_dequant(getattr(self.layers[l], name), out=wbuf)
        x = torch.empty((L, H), dtype=torch.bfloat16, device=dev)
        qkv = torch.empty((L, a.n_qkv), dtype=torch.bfloat16, device=dev)
        gu = torch.empty((L, 2 * I), dtype=torch.bfloat16, device=dev)
        act = torch.empty((L, I), dtype=torch.bfloat16, device=dev)
        for l, Lw in enumerate(self.layers):
            ops.rows_rmsnorm(h, Lw.in_norm, eps, out=x)
            torch.matmul(x, rows(l, "qkv").t(), out=qkv)
            k_pool, v_pool, k_sb, v_sb = cache.layer_args(l)
            inv_freq = self.inv_freq_local if a.is_sliding(l) else self.inv_freq
            q = ops.qkv_rope_append(qkv, 1, L, nq, nkv, hd, Lw.q_norm, Lw.k_norm, eps, inv_freq, cache.seq_lens,
                                    cache.block_table, cache.page, cache.kv_dtype, k_pool, v_pool, k_sb, v_sb)
            o = ops.attention(q, 1, L, nq, nkv, hd, a.attn_scale, cache.seq_lens, cache.max_ctx, cache.block_table,
                              cache.page, cache.kv_dtype, k_pool, v_pool, k_sb, v_sb, causal=True, window=a.window(l))
            h.addmm_(o, rows(l, "o").t())
            ops.rows_rmsnorm(h, Lw.post_norm, eps, out=x)
            torch.matmul(x, rows(l, "gate_up").t(), out=gu)
            ops.rows_gated(gu, self.act_epi, out=act)
            h.addmm_(act, rows(l, "down").t())
            for i, t in enumerate(tap):
                if t == l:
                    fused[:, i * H:(i + 1) * H].copy_(h)
        pos = cache.lengths[0]
        ops.lens_add(cache.seq_lens, None, L)
        cache.note_lengths([pos + L])
        x = ops.pack_rn(M=1, K=H, h=h[L - 1:L], norm_w=self.norm, eps=eps)
        out = torch.empty((1, a.vocab_size), dtype=torch.float32, device=dev)
        ops.w8_gemm(x, self.lm_head, out=out, softcap=a.final_logit_softcapping or 0.0)
        if fused is not None and on_chunk is not None:
            for c0 in range(0, L, chunk):
                on_chunk(fused[c0:c0 + chunk].view(1, -1, len(tap) * H), pos + c0)
            return out.view(1, 1, -1), None
        return out.view(1, 1, -1), (fused.view(1, L, -1) if fused is not None else None)
