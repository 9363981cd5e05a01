"""CPU restatement of the verify forward, KV semantics and the DFlash drafter (torch, float32).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Restates (reference paths):
  - Target._run_mlxlm: embed -> layers -> norm -> lm_head with the residual captured after
    the tapped layers (src/mlx_dspark/target.py:58-75). The Qwen3 layer itself lives in
    mlx_lm (external); it follows the public Qwen3 architecture: RMSNorm -> q/k/v
    projections -> per-head q/k RMSNorm -> rotate-half RoPE (theta from config) -> GQA
    attention, causal with offset (mask grid of tests/test_batch_engine.py:87-103) ->
    o_proj + residual; RMSNorm -> down(silu(gate) * up) + residual. The Gemma-style layout
    (public Gemma 3 architecture; the reference runs it through mlx_vlm, target.py:53-55)
    adds the embedding scale, sandwich norms (the o_proj and down outputs RMSNorm-ed before
    their residual adds), GeGLU with tanh GeLU, sliding-window layers with their own RoPE base
    and a final tanh soft-cap on the logits.
  - KV append / trim as metadata (src/mlx_dspark/batch_engine.py:132-163).
  - DFlashDraftModel.__call__ (src/mlx_dspark/dflash_model.py:100-208).
Every intermediate is rounded to bf16 where a bf16 MLX graph produces a bf16 array, except
that a projection and the residual add it feeds round once (a fused add, as the engine
does); ``double_round=True`` rounds the projection output first, as an unfused bf16 graph
would. On a 256-wide 4-layer random model the two conventions alone differ by 0.022 in the
normalised-logit metric, which is the noise floor this oracle works at.

Pinning: with the bf16 rounding points switched off, every composition equals an independent
implementation of the public architecture on identical weights (tests/test_oracle_compose.py):
OracleTarget equals transformers' Qwen3ForCausalLM (GQA, q/k norms, RoPE base, tied and untied
heads, KV-cached continuation, hidden-state taps) and Gemma3ForCausalLM for the Gemma-style
layout (sandwich norms, GeGLU, sliding-window layers with their own RoPE base, query scale,
soft-cap, embedding scale); OracleDFlash and the qwen3 OracleDSpark equal stacks of
Qwen3DecoderLayer run without a mask over [context; block] rows (the context rows' input norm
made the identity), and the gemma4 OracleDSpark a stack of Gemma4TextDecoderLayer (k_eq_v,
v_norm, proportional RoPE, scale 1, layer_scalar); to 1e-5 in the normalised-logit metric, and
each comparison catches a planted mistake. Attention also equals an explicit loop over heads
with the GQA map h -> h // (nq/nkv) (tests/test_model.py:25-60 in the reference); the causal
mask reproduces the reference's exact grids; RMSNorm / RoPE / SiLU are checked against float64
closed forms in tests/test_oracle_model.py. What stays unpinned is the rounding: where a bf16
MLX graph rounds inside mlx_lm / mlx_vlm is external to the reference, so the rounding points
here are this build's choice, covered by the logits tolerance.
"""

from __future__ import annotations

import contextlib

import numpy as np
import torch

from . import w8 as W8


def bf(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).to(torch.float32)


# Float64 sums. Inside ``with exact_sums():`` every reduction (projections, attention, the
# norms' mean squares) and every elementwise chain between two rounding points runs in float64
# and is rounded once to float32: an evaluation of the same bf16 rounding points whose float32
# values are correctly rounded. Its distance from the plain float32 evaluation is how far two
# valid implementations of one rounding-point graph drift apart (other summation orders move a
# value by a few float32 ulp, and every later bf16 rounding that such a move flips passes on a
# whole bf16 step): the noise floor of the logits metric for that model and input.
_EXACT = [False]


@contextlib.contextmanager
def exact_sums(on: bool = True):
    prev = _EXACT[0]
    _EXACT[0] = on
    try:
        yield
    finally:
        _EXACT[0] = prev


def _dt():
    return torch.float64 if _EXACT[0] else torch.float32


def mm(x, w):
    """x [M, K] . w [N, K]^T in float32 (float64, rounded once, under exact_sums)."""
    if not _EXACT[0]:
        return x @ w.T
    xd = x.double()
    out = torch.empty(x.shape[0], w.shape[0], dtype=torch.float32)
    for n0 in range(0, w.shape[0], 16384):
        out[:, n0:n0 + 16384] = (xd @ w[n0:n0 + 16384].double().T).float()
    return out


def silu(x):
    if _EXACT[0]:
        xd = x.double()
        return (xd * torch.sigmoid(xd)).float()
    return x * torch.sigmoid(x)


def rmsnorm(x, w, eps):
    if _EXACT[0]:
        xd = x.double()
        return (xd * torch.rsqrt((xd * xd).mean(-1, keepdim=True) + eps) * w.double()).float()
    return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps) * w


def norm_later(x, w, eps):
    """The RMSNorm in front of a projection applied after it, where the engine's Qwen3 layout
    applies it (the consuming GEMM scales its output rows): returns (bf16(x * w), r) with
    r = rsqrt(mean(x^2) + eps) per row, so r * (bf16(x * w) @ W^T) is rmsnorm(x, w) @ W^T up
    to where the product is rounded."""
    if _EXACT[0]:
        xd = x.double()
        return bf(x * w), torch.rsqrt((xd * xd).mean(-1, keepdim=True) + eps).float()
    return bf(x * w), torch.rsqrt((x * x).mean(-1, keepdim=True) + eps)


def inv_freq(hd: int, theta: float, rotary_fraction: float = 1.0) -> torch.Tensor:
    """Rotate-half RoPE frequencies theta^(-2i/hd), i < hd/2 (float64, stored f32). A
    rotary_fraction below 1 is proportional RoPE (the gemma4 drafter's "proportional" rope
    type, src/mlx_dspark/config.py:38-42, :161-163; the public definition, as in transformers'
    _compute_proportional_rope_parameters): the first int(fraction * hd / 2) frequencies keep
    their full-head_dim exponents, the rest are 0, so those dims are not rotated."""
    inv = theta ** (-2.0 * np.arange(hd // 2) / hd)
    if rotary_fraction < 1.0:
        inv[int(rotary_fraction * hd // 2):] = 0.0
    return torch.from_numpy(inv.astype(np.float32))


def rope(x, pos, theta, inv=None, revolutions: bool = False):
    """rotate-half RoPE; x [..., n, hd], pos [n]; inv overrides the theta frequencies. The angle
    is pos * inv rounded to float32; its sine and cosine are those of that float32 angle.
    revolutions=True instead reduces the float32 angle to revolutions in float32 first
    (ang * 1/(2 pi), minus the nearest integer) and takes sin / cos of 2 pi times that: the
    hardware sine's argument form, off by up to |ang| * 2^-24 revolutions (a rounding source
    the decomposition in tests/test_rounding_sources.py measures)."""
    hd = x.shape[-1]
    if inv is None:
        inv = torch.from_numpy((theta ** (-2.0 * np.arange(hd // 2) / hd)).astype(np.float32))
    ang = pos.float()[:, None] * inv[None, :]
    if revolutions:
        rev = ang * torch.tensor(0.15915494309189535, dtype=torch.float32)
        ang = (rev - torch.round(rev)).double() * (2.0 * np.pi)
    if _EXACT[0] or revolutions:
        a = ang.double()
        c, s = torch.cos(a), torch.sin(a)
        if not _EXACT[0]:
            c, s = c.float(), s.float()
    else:
        c, s = torch.cos(ang), torch.sin(ang)
    x1, x2 = x[..., : hd // 2], x[..., hd // 2:]
    if _EXACT[0]:
        x1, x2 = x1.double(), x2.double()
        return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], dim=-1).float()
    return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], dim=-1)


def _blocks_attend(s, V, split, block, p_bf16, partial_bf16, exp2_c, terms=0):
    """Attention of score rows s [W, L] (scaled, -inf where masked) over V [L, hd] as split
    kernels compute it: keys in splits of ``split`` (one split: the whole range), inside a split
    one max per ``block`` keys (the offset the exponent is taken from, which decides how P rounds
    under p_bf16), each split's output normalised (rounded to bf16 with partial_bf16) and the
    splits merged with weights exp(m_s - M) * l_s. exp2_c: exp(s - m) as 2^(s c - m c) with
    c = log2(e) rounded to float32 (the kernels' exp2 form, scale already in s). terms=2: P
    weights V and is summed as bf16(p) + bf16(p - bf16(p)) (the two-term form)."""
    dt = s.dtype
    L = s.shape[1]
    step = split or L
    ninf = float("-inf")
    parts = []
    for j0 in range(0, L, step):
        sj, vj = s[:, j0:j0 + step], V[j0:j0 + step]
        bstep = block or sj.shape[1]
        bm, bl, bo = [], [], []
        for b0 in range(0, sj.shape[1], bstep):
            sb, vb = sj[:, b0:b0 + bstep], vj[b0:b0 + bstep]
            m = sb.max(dim=-1, keepdim=True).values
            m0 = torch.where(torch.isinf(m), torch.zeros_like(m), m)
            p = torch.exp2(sb * exp2_c - m0 * exp2_c) if exp2_c else torch.exp(sb - m0)
            if p_bf16:
                p = bf(p).to(dt)
            elif terms == 2:
                hi = bf(p).to(dt)
                p = hi + bf(p - hi).to(dt)
            bm.append(m)
            bl.append(p.sum(dim=-1, keepdim=True))
            bo.append(p @ vb)
        M = torch.stack(bm).max(0).values
        w = [torch.where(torch.isinf(m), torch.zeros_like(m), torch.exp(m - M)) for m in bm]
        l = sum(a * b for a, b in zip(bl, w))
        o = sum(a * b for a, b in zip(bo, w)) / torch.where(l > 0, l, torch.ones_like(l))
        if partial_bf16 and step < L:
            o = bf(o).to(dt)
        parts.append((M, l, o))
    if len(parts) == 1:
        return parts[0][2]
    M = torch.stack([p[0] for p in parts]).max(0).values
    w = [torch.where(torch.isinf(m), torch.zeros_like(m), torch.exp(m - M)) * l for m, l, _ in parts]
    den = sum(w)
    o = sum(p[2] * x for p, x in zip(parts, w))
    return o / torch.where(den > 0, den, torch.ones_like(den))


def sdpa(q, K, V, scale, mask=None, p_bf16=False, *, split=0, block=0, partial_bf16=False, exp2=False,
         terms=0):
    """q [W, nq, hd], K/V [L, nkv, hd] -> [W, nq, hd]; GQA by head index // (nq/nkv).
    p_bf16: the unnormalised probabilities exp(s - max) are rounded to bf16 before they weight
    V and before they are summed for the normaliser (where a bf16 attention kernel rounds them);
    otherwise the softmax stays float32. split / block / partial_bf16 / exp2 / terms: the split
    kernels' evaluation order (_blocks_attend), for the rounding-source decomposition."""
    W, nq, hd = q.shape
    nkv = K.shape[1]
    G = nq // nkv
    dt = _dt()
    out = torch.empty(W, nq, hd, dtype=dt)
    plain = not (split or block or partial_bf16 or exp2 or terms)
    c2 = float(np.float32(1.4426950408889634)) if exp2 else 0.0
    for h in range(nq):
        Kh, Vh = K[:, h // G].to(dt), V[:, h // G].to(dt)
        s = (q[:, h].to(dt) @ Kh.T) * scale
        if mask is not None:
            s = s.masked_fill(~mask, float("-inf"))
        if not plain:
            out[:, h] = _blocks_attend(s, Vh, split, block, p_bf16, partial_bf16, c2, terms)
        elif p_bf16:
            p = bf(torch.exp(s - s.max(dim=-1, keepdim=True).values)).to(dt)
            out[:, h] = (p @ Vh) / p.sum(dim=-1, keepdim=True)
        else:
            out[:, h] = torch.softmax(s, dim=-1) @ Vh
    return out.float()


def causal_mask(offset: int, W: int, window: int = 0) -> torch.Tensor:
    """[W, offset + W] boolean: query i (absolute offset + i) sees key j iff j <= offset + i,
    and, for a sliding-window layer, j > offset + i - window."""
    j = torch.arange(offset + W)[None, :]
    i = torch.arange(W)[:, None]
    m = j <= offset + i
    if window:
        m &= j > offset + i - window
    return m


def gelu_tanh(x: torch.Tensor) -> torch.Tensor:
    """tanh-approximated GeLU (gemma's gelu_pytorch_tanh)."""
    if _EXACT[0]:
        xd = x.double()
        return (0.5 * xd * (1.0 + torch.tanh(0.7978845608028654 * (xd + 0.044715 * xd * xd * xd)))).float()
    return 0.5 * x * (1.0 + torch.tanh(0.7978845608028654 * (x + 0.044715 * x * x * x)))


def deq_codes(q: torch.Tensor, s: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """float32 w = s * q + b per group of 64 columns (q uint8 [N, K], s / b bf16 [N, K/64]), on
    the CPU. s * q is exact in float32 (a bf16 times an integer below 256), so the one rounding
    of the sum gives the float32 value of oracle/w8.py's float64 dequantize, bit for bit."""
    q, s, b = q.cpu(), s.cpu(), b.cpu()
    N, K = q.shape
    w = q.view(N, K // 64, 64).float() * s.float().unsqueeze(-1) + b.float().unsqueeze(-1)
    return w.view(N, K)


def deq(wobj) -> torch.Tensor:
    return deq_codes(*wobj.mlx)


def deq_table(t) -> torch.Tensor:
    return deq_codes(t.q, t.s, t.b)


def kv_quant_roundtrip(x: torch.Tensor) -> torch.Tensor:
    """8-bit group-64 affine round trip along the last axis (same rule as the weights)."""
    shp = x.shape
    flat = x.reshape(-1, shp[-1]).numpy().astype(np.float32)
    q, s, b = W8.quantize(flat)
    return bf(torch.from_numpy(W8.dequantize(q, s, b).astype(np.float32)).reshape(shp))


class OracleLayer:
    def __init__(self, L, nq, nkv, hd):
        self.wq = deq(L.qkv)
        self.wo = deq(L.o)
        self.wgu = deq(L.gate_up)
        self.wd = deq(L.down)
        self.in_norm = L.in_norm.float().cpu()
        self.post_norm = L.post_norm.float().cpu()
        self.q_norm = L.q_norm.float().cpu()
        self.k_norm = L.k_norm.float().cpu()
        an, fn = getattr(L, "attn_out_norm", None), getattr(L, "ff_out_norm", None)
        self.attn_out_norm = None if an is None else an.float().cpu()
        self.ff_out_norm = None if fn is None else fn.float().cpu()
        self.nq, self.nkv, self.hd = nq, nkv, hd


class OracleTarget:
    """Dense-KV CPU model built from a GPU model created with keep_mlx=True."""

    def __init__(self, model, kv_bits=None, double_round: bool = False, p_bf16: bool = False, *,
                 norm_first: bool = False, split: int = 0, p_block: int = 0, partial_bf16: bool = False,
                 exp2: bool = False, p_terms: int = 0, rope_revolutions: bool = False, requant_new: bool = True):
        """Rounding-point options (each default is the reference-order evaluation; the others
        exist to measure one source at a time): double_round rounds a projection's output to
        bf16 before its residual add; p_bf16 rounds the attention probabilities to bf16;
        norm_first normalises the Qwen3 layout's rows before their projections (bf16 normalised
        rows, as an unfused graph does) instead of after them; split / p_block / partial_bf16 /
        exp2 / p_terms evaluate attention the way split kernels do (sdpa); rope_revolutions takes the
        RoPE sine in float32 revolutions (rope); requant_new=False keeps the new K/V rows in
        bf16 in an 8-bit cache (the re-quantisation of the new rows switched off)."""
        a = model.args
        self.a = a
        self.kv_bits = kv_bits
        self.rr = bf if double_round else (lambda x: x)
        self.p_bf16 = p_bf16
        self.norm_first = norm_first
        self.attn_opts = dict(split=split, block=p_block, partial_bf16=partial_bf16, exp2=exp2, terms=p_terms)
        self.rope_revolutions = rope_revolutions
        self.requant_new = requant_new
        self.layers = [OracleLayer(L, a.num_attention_heads, a.num_key_value_heads, a.head_dim) for L in model.layers]
        self.embed = deq_table(model.embed)
        self.lm_head = deq(model.lm_head)
        self.norm = model.norm.float().cpu()
        self.K = [torch.zeros(0, a.num_key_value_heads, a.head_dim) for _ in self.layers]
        self.V = [torch.zeros(0, a.num_key_value_heads, a.head_dim) for _ in self.layers]
        self.offset = 0
        # dense=True: the rounding of the engine's dense prefill (the norms normalise first and the
        # projections multiply weights rounded to bf16, as a bf16 library GEMM over expanded
        # weights does); the final norm and head keep the engine's normed-later form
        self.dense = False
        self._bf_w: dict = {}

    def _w(self, l: int, name: str) -> torch.Tensor:
        w = getattr(self.layers[l], name)
        if not self.dense:
            return w
        key = (l, name)
        if key not in self._bf_w:
            self._bf_w[key] = bf(w)
        return self._bf_w[key]

    def trim(self, n: int) -> None:
        """Roll back n tokens (metadata in the engine; a truncation here)."""
        self.offset = max(0, self.offset - n)
        self.K = [k[: self.offset] for k in self.K]
        self.V = [v[: self.offset] for v in self.V]

    def forward(self, ids, tap=()):
        a = self.a
        ids = torch.as_tensor(ids).reshape(-1).long()
        W = ids.numel()
        nq, nkv, hd, eps = a.num_attention_heads, a.num_key_value_heads, a.head_dim, a.rms_norm_eps
        h = bf(bf(self.embed[ids]) * a.embed_scale)   # bf16 embedding rows, then the bf16 scale
        pos = torch.arange(self.offset, self.offset + W)
        gelu = getattr(a, "hidden_act", "silu") != "silu"
        # the Qwen3 layout's norms are applied after their projections (norm_later); the
        # Gemma-style layout normalises before them
        sandwich = bool(getattr(a, "sandwich_norms", False))
        first = sandwich or self.dense or self.norm_first
        rev = self.rope_revolutions
        captured = []
        for l, L in enumerate(self.layers):
            win = a.window(l)
            theta = (a.rope_local_base_freq or a.rope_theta) if a.is_sliding(l) else a.rope_theta
            if first:
                qkv = bf(mm(bf(rmsnorm(h, L.in_norm, eps)), self._w(l, "wq")))
            else:
                xg, r = norm_later(h, L.in_norm, eps)
                qkv = bf(r * mm(xg, L.wq))
            q = qkv[:, : nq * hd].view(W, nq, hd)
            k = qkv[:, nq * hd:(nq + nkv) * hd].view(W, nkv, hd)
            v = qkv[:, (nq + nkv) * hd:].view(W, nkv, hd)
            q = bf(rope(bf(rmsnorm(q, L.q_norm, eps)).transpose(0, 1), pos, theta, revolutions=rev).transpose(0, 1))
            k = bf(rope(bf(rmsnorm(k, L.k_norm, eps)).transpose(0, 1), pos, theta, revolutions=rev).transpose(0, 1))
            if self.kv_bits == 8 and self.requant_new:
                k, v = kv_quant_roundtrip(k), kv_quant_roundtrip(v)
            self.K[l] = torch.cat([self.K[l], k])
            self.V[l] = torch.cat([self.V[l], v])
            o = bf(sdpa(q, self.K[l], self.V[l], a.attn_scale, causal_mask(self.offset, W, win), self.p_bf16,
                        **self.attn_opts))
            if L.attn_out_norm is not None:     # sandwich: norm the projection output, then add
                h = bf(h + bf(rmsnorm(bf(mm(o.reshape(W, -1), L.wo)), L.attn_out_norm, eps)))
            else:
                h = bf(h + self.rr(mm(o.reshape(W, -1), self._w(l, "wo"))))
            if first:
                gu = bf(mm(bf(rmsnorm(h, L.post_norm, eps)), self._w(l, "wgu")))
            else:
                xg, r = norm_later(h, L.post_norm, eps)
                gu = bf(r * mm(xg, L.wgu))
            I = gu.shape[1] // 2
            g, u = gu[:, :I], gu[:, I:]
            act = bf(bf(gelu_tanh(g) if gelu else silu(g)) * u)
            if L.ff_out_norm is not None:
                h = bf(h + bf(rmsnorm(bf(mm(act, L.wd)), L.ff_out_norm, eps)))
            else:
                h = bf(h + self.rr(mm(act, self._w(l, "wd"))))
            if l in tap:
                captured.append(h)
        self.offset += W
        if sandwich or self.norm_first:
            logits = mm(bf(rmsnorm(h, self.norm, eps)), self.lm_head)
        else:
            xg, r = norm_later(h, self.norm, eps)
            logits = r * mm(xg, self.lm_head)
        cap = getattr(a, "final_logit_softcapping", None)
        if cap:
            logits = torch.tanh(logits / cap) * cap
        fused = torch.cat(captured, dim=-1) if captured else None
        return logits, fused


class OracleDFlash:
    """CPU DFlash drafter (src/mlx_dspark/dflash_model.py:100-208) bound to an OracleTarget.

    Full-attention layers attend over every stored context row and the whole block without a
    mask. Sliding layers (layer_types[l] == "sliding_attention", :90-92) attend causally with
    a window of ``sliding_window`` positions: the block query at absolute position P sees the
    keys at positions P - window + 1 .. P (:103-109 keep the last window - 1 context rows, and
    :128-132 mask the block causally within the window). Context K is roped at its absolute
    position and the block after the stored context (:118-122)."""

    def __init__(self, drafter, target: OracleTarget, p_bf16: bool = False):
        c = drafter.config
        self.c = c
        self.p_bf16 = p_bf16
        self.fc = deq(drafter.fc)
        self.hidden_norm = drafter.hidden_norm.float().cpu()
        self.norm = drafter.norm.float().cpu()
        self.layers = [OracleLayer(L, c.num_attention_heads, c.num_key_value_heads, c.head_dim)
                       for L in drafter.layers]
        self.target = target
        self.K = [torch.zeros(0, c.num_key_value_heads, c.head_dim) for _ in self.layers]
        self.V = [torch.zeros(0, c.num_key_value_heads, c.head_dim) for _ in self.layers]

    @property
    def offset(self) -> int:
        return self.K[0].shape[0]

    def _sliding(self, l: int) -> bool:
        lt = getattr(self.c, "layer_types", None) or ()
        return l < len(lt) and lt[l] == "sliding_attention"

    def __call__(self, block_ids, target_hidden, logits_start=1):
        c = self.c
        nq, nkv, hd, eps = c.num_attention_heads, c.num_key_value_heads, c.head_dim, c.rms_norm_eps
        ids = torch.as_tensor(block_ids).reshape(-1).long()
        L = ids.numel()
        h = bf(self.target.embed[ids] * self.target.a.embed_scale)
        th = target_hidden.reshape(-1, target_hidden.shape[-1]).float()
        S = th.shape[0]
        h_ctx = bf(rmsnorm(bf(mm(th, self.fc)), self.hidden_norm, eps))
        off = self.offset
        for l, Lw in enumerate(self.layers):
            x = bf(rmsnorm(h, Lw.in_norm, eps))
            qkv = bf(mm(x, Lw.wq))
            q = qkv[:, : nq * hd].view(L, nq, hd)
            kb = qkv[:, nq * hd:(nq + nkv) * hd].view(L, nkv, hd)
            vb = qkv[:, (nq + nkv) * hd:].view(L, nkv, hd)
            kvc = bf(mm(h_ctx, Lw.wq[nq * hd:]))
            kc = kvc[:, : nkv * hd].view(S, nkv, hd)
            vc = kvc[:, nkv * hd:].view(S, nkv, hd)
            pq = torch.arange(off + S, off + S + L)
            q = bf(rope(bf(rmsnorm(q, Lw.q_norm, eps)).transpose(0, 1), pq, c.rope_theta).transpose(0, 1))
            kb = bf(rope(bf(rmsnorm(kb, Lw.k_norm, eps)).transpose(0, 1), pq, c.rope_theta).transpose(0, 1))
            kc = bf(rope(bf(rmsnorm(kc, Lw.k_norm, eps)).transpose(0, 1), torch.arange(off, off + S),
                         c.rope_theta).transpose(0, 1))
            self.K[l] = torch.cat([self.K[l], kc])
            self.V[l] = torch.cat([self.V[l], vc])
            K = torch.cat([self.K[l], kb])
            Vv = torch.cat([self.V[l], vb])
            mask = None
            if self._sliding(l):
                mask = causal_mask(off + S, L, int(c.sliding_window))
            o = bf(sdpa(q, K, Vv, hd ** -0.5, mask, self.p_bf16))
            h = bf(h + mm(o.reshape(L, -1), Lw.wo))
            x = bf(rmsnorm(h, Lw.post_norm, eps))
            gu = bf(mm(x, Lw.wgu))
            I = gu.shape[1] // 2
            act = bf(bf(silu(gu[:, :I])) * gu[:, I:])
            h = bf(h + mm(act, Lw.wd))
        h = h[logits_start:]
        return mm(bf(rmsnorm(h, self.norm, eps)), self.target.lm_head)


def normalized_maxdiff(a: torch.Tensor, b: torch.Tensor) -> float:
    """max |a/rms(a) - b/rms(b)| over rows: the logits tolerance metric."""
    a = a.detach().float().cpu().reshape(-1, a.shape[-1])
    b = b.detach().float().cpu().reshape(-1, b.shape[-1])
    an = a / a.pow(2).mean(-1, keepdim=True).sqrt()
    bn = b / b.pow(2).mean(-1, keepdim=True).sqrt()
    return float((an - bn).abs().max())


def logit_diff(a: torch.Tensor, b: torch.Tensor):
    """(max-abs, rms) of the difference of RMS-normalised logit rows."""
    a = a.detach().float().cpu().reshape(-1, a.shape[-1])
    b = b.detach().float().cpu().reshape(-1, b.shape[-1])
    d = a / a.pow(2).mean(-1, keepdim=True).sqrt() - b / b.pow(2).mean(-1, keepdim=True).sqrt()
    return float(d.abs().max()), float(d.pow(2).mean().sqrt())


def greedy_decode(target: OracleTarget, prompt, n_new: int):
    """Plain greedy decoding (what speculative greedy decoding must reproduce); returns the
    tokens and the top-2 margin (after RMS normalisation) of every decision."""
    logits, _ = target.forward(prompt)
    out, margins = [], []
    row = logits[-1]
    for _ in range(n_new):
        rn = row / row.pow(2).mean().sqrt()
        top = torch.topk(rn, 2).values
        margins.append(float(top[0] - top[1]))
        t = int(torch.argmax(row))
        out.append(t)
        row = target.forward([t])[0][-1]
    return out, margins


class OracleDSpark:
    """CPU DSpark drafter, qwen3 and gemma4 families (src/mlx_dspark/model.py:83-320), built
    from a GPU drafter created with keep_mlx=True.

    Context rows: fused = RMSNorm(fc(target_hidden)); per layer K = rope(k_norm(k_proj(fused)),
    ctx position), V = v_proj(fused) or, gemma4 with k_eq_v, V = v_norm(k_proj(fused)) (RMSNorm
    without weight, not roped) (model.py:113-128, :247-256). Block: embed (x sqrt(hidden) for
    gemma4, :244-245) -> layers with attention over context ++ block, no mask, roped at
    block_offset + i (:130-155); the qwen3 layer is Llama 2-norm with SiLU, the gemma4 layer has
    sandwich norms, tanh-GeLU and the layer_scalar multiply (:172-193) -> final RMSNorm. gemma4
    attends over the global kv heads at global_head_dim with scale 1 and proportional RoPE
    (config.py:64-84). Heads: lm_head (+ tanh soft-cap) (:264-268), Markov block sampling
    (:270-281) with bf16 rounding points (logits, bias and their sum are bf16, as in a bf16
    graph), confidence logits (:311-320)."""

    def __init__(self, drafter, p_bf16: bool = False):
        c = drafter.config
        self.c = c
        self.p_bf16 = p_bf16
        self.gemma = c.family == "gemma4"
        self.nq, self.nkv, self.hd = c.num_attention_heads, c.n_kv_heads, c.attn_head_dim
        frac = c.partial_rotary_factor if c.rope_type == "proportional" else 1.0
        self.inv = inv_freq(self.hd, c.rope_theta, frac)
        self.embed_scale = float(c.hidden_size) ** 0.5 if self.gemma else 1.0
        self.scalars = list(drafter.layer_scalars) if getattr(drafter, "layer_scalars", None) else None
        self.embed = deq_table(drafter.embed_tokens)
        self.fc = deq(drafter.fc)
        self.hidden_norm = drafter.hidden_norm.float().cpu()
        self.norm = drafter.norm.float().cpu()
        self.lm_head = deq(drafter.lm_head)
        self.layers = [OracleLayer(L, self.nq, self.nkv, self.hd) for L in drafter.layers]
        self.w1 = deq_table(drafter.markov_head.w1) if drafter.markov_head is not None else None
        self.w2 = deq(drafter.markov_head.w2) if drafter.markov_head is not None else None
        self.conf_w = deq(drafter.confidence_head.proj)[0] if drafter.confidence_head is not None else None
        self.conf_b = drafter.confidence_head.bias if drafter.confidence_head is not None else 0.0
        self.K = [torch.zeros(0, self.nkv, self.hd) for _ in self.layers]
        self.V = [torch.zeros(0, self.nkv, self.hd) for _ in self.layers]

    @property
    def length(self) -> int:
        return self.K[0].shape[0]

    def _kv(self, L, x, n, pos):
        """(roped normed K, V) [n, nkv, hd] of rows x (model.py:113-124)."""
        c = self.c
        nq, nkv, hd, eps = self.nq, self.nkv, self.hd, c.rms_norm_eps
        kp = bf(mm(x, L.wq[nq * hd:(nq + nkv) * hd])).view(n, nkv, hd)
        if self.gemma and c.attention_k_eq_v:
            v = bf(rmsnorm(kp, torch.ones(hd), eps))
        else:
            v = bf(mm(x, L.wq[(nq + nkv) * hd:])).view(n, nkv, hd)
            if c.use_v_norm:
                v = bf(rmsnorm(v, torch.ones(hd), eps))
        k = bf(rope(bf(rmsnorm(kp, L.k_norm, eps)).transpose(0, 1), pos, c.rope_theta, self.inv).transpose(0, 1))
        return k, v

    def update_context(self, target_hidden):
        c = self.c
        eps = c.rms_norm_eps
        th = torch.as_tensor(target_hidden).reshape(-1, self.fc.shape[1]).float()
        S = th.shape[0]
        fused = bf(rmsnorm(bf(mm(th, self.fc)), self.hidden_norm, eps))
        pos = torch.arange(self.length, self.length + S)
        for l, L in enumerate(self.layers):
            k, v = self._kv(L, fused, S, pos)
            self.K[l] = torch.cat([self.K[l], k])
            self.V[l] = torch.cat([self.V[l], v])

    def block_hidden(self, block_ids):
        """normed block hidden [k, H]"""
        c = self.c
        nq, hd, eps = self.nq, self.hd, c.rms_norm_eps
        ids = torch.as_tensor(block_ids).reshape(-1).long()
        k = ids.numel()
        h = bf(self.embed[ids])
        if self.embed_scale != 1.0:
            h = bf(h * self.embed_scale)
        pos = torch.arange(self.length, self.length + k)
        for l, L in enumerate(self.layers):
            x = bf(rmsnorm(h, L.in_norm, eps))
            q = bf(mm(x, L.wq[: nq * hd])).view(k, nq, hd)
            q = bf(rope(bf(rmsnorm(q, L.q_norm, eps)).transpose(0, 1), pos, c.rope_theta, self.inv).transpose(0, 1))
            kb, vb = self._kv(L, x, k, pos)
            o = bf(sdpa(q, torch.cat([self.K[l], kb]), torch.cat([self.V[l], vb]), c.scaling, None, self.p_bf16))
            if self.gemma:     # sandwich norms, tanh-GeLU, layer_scalar (model.py:172-184)
                h = bf(h + bf(rmsnorm(bf(mm(o.reshape(k, -1), L.wo)), L.attn_out_norm, eps)))
                x = bf(rmsnorm(h, L.post_norm, eps))
                gu = bf(mm(x, L.wgu))
                I = gu.shape[1] // 2
                act = bf(bf(gelu_tanh(gu[:, :I])) * gu[:, I:])
                h = bf(h + bf(rmsnorm(bf(mm(act, L.wd)), L.ff_out_norm, eps)))
                if self.scalars is not None and self.scalars[l] != 1.0:
                    h = bf(h * self.scalars[l])
            else:
                h = bf(h + mm(o.reshape(k, -1), L.wo))
                x = bf(rmsnorm(h, L.post_norm, eps))
                gu = bf(mm(x, L.wgu))
                I = gu.shape[1] // 2
                h = bf(h + mm(bf(bf(silu(gu[:, :I])) * gu[:, I:]), L.wd))
        return bf(rmsnorm(h, self.norm, eps))

    def base_logits(self, block_ids, cap):
        logits = mm(self.block_hidden(block_ids)[:cap], self.lm_head)
        cap_ = self.c.final_logit_softcapping
        return torch.tanh(logits / cap_) * cap_ if cap_ else logits

    def step_logits(self, base_row, prev):
        """bf16(bf16(base) + bf16(w2 . bf16(w1[prev])))"""
        if getattr(self, "_w2_src", None) is not self.w2:        # float64 copy, made once per table
            self._w2d, self._w2_src = self.w2.double(), self.w2
        bias = bf(self._w2d @ bf(self.w1[int(prev)]).double())
        return bf(bf(torch.as_tensor(base_row).float()) + bias.float())

    def sample_block(self, base, first_prev):
        """greedy Markov block: argmax (lowest index on ties) of step_logits, sequentially."""
        toks, prev = [], int(first_prev)
        for i in range(base.shape[0]):
            row = self.step_logits(base[i], prev) if self.w1 is not None else bf(torch.as_tensor(base[i]).float())
            t = int(torch.argmax(row))
            toks.append(t)
            prev = t
        return toks

    def confidence_logits(self, hidden_rows, prev_ids):
        """proj(feats) + bias per row (src/mlx_dspark/model.py:211-217, :311-320): feats are the
        block hidden rows, followed by the Markov head's previous-token embeddings w1[prev]
        (bf16 rows) when config.confidence_head_with_markov is set."""
        feats = torch.as_tensor(hidden_rows).float()
        if self.c.confidence_head_with_markov:
            feats = torch.cat([feats, bf(self.w1[torch.as_tensor(prev_ids).long()])], dim=-1)
        return feats @ self.conf_w + self.conf_b


def markov_sample_block(base, first_prev, step_bias):
    """Sequential greedy Markov sampling with an arbitrary step_bias(prev) -> [V] (the control
    flow of src/mlx_dspark/model.py:270-281 and batch_engine.py:414-428)."""
    toks, prev = [], first_prev
    for i in range(base.shape[0]):
        t = int(torch.argmax(torch.as_tensor(base[i]) + step_bias(prev)))
        toks.append(t)
        prev = t
    return toks


def penalty_rows(counts: dict, presence: float, frequency: float, draft_prefix) -> list:
    """Per-row {token: penalty} of a verify block (src/mlx_dspark/generate.py:202-228): base
    completion counts, then each draft-prefix token adds frequency, plus presence the first
    time it appears."""
    base = {t: presence + frequency * c for t, c in counts.items()}
    rows, seen = [base], dict(counts)
    for d in draft_prefix:
        r = dict(rows[-1])
        r[d] = r.get(d, 0.0) + frequency + (presence if seen.get(d, 0) == 0 else 0.0)
        seen[d] = seen.get(d, 0) + 1
        rows.append(r)
    return rows
