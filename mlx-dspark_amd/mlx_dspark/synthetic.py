"""Seeded random-init W8 models at the benchmark shapes (no checkpoints are needed).

Weights are N(0, 0.02) drawn on the device from a per-tensor seed (so a tensor does not
depend on the order tensors are built in), quantized with dsk_w8_quantize (affine 8-bit,
group 64, bf16 scale/bias) and repacked into the engine's tiled layout.
q/k norm gains are hd**-0.25 (see qk_norm), other norm weights are 1. With ``keep_mlx=True`` every W8 weight also keeps its MLX-layout (q, scales, biases) so a
CPU checker can dequantize exactly the same numbers.
"""

from __future__ import annotations

import hashlib
import math

import torch

from .ops import W8Table, W8Weight
from .qwen3 import LayerWeights, Qwen3W8, TargetArgs

STD = 0.02

# Target shapes (HF config field names).
TARGETS = {
    "qwen3-0.6b": dict(hidden_size=1024, num_hidden_layers=28, intermediate_size=3072,
                       num_attention_heads=16, num_key_value_heads=8, head_dim=128,
                       vocab_size=151936, tie_word_embeddings=True),
    "qwen3-8b": dict(hidden_size=4096, num_hidden_layers=36, intermediate_size=12288,
                     num_attention_heads=32, num_key_value_heads=8, head_dim=128,
                     vocab_size=151936, tie_word_embeddings=False),
    # small shapes for tests and smoke runs
    "tiny": dict(hidden_size=256, num_hidden_layers=4, intermediate_size=512,
                 num_attention_heads=4, num_key_value_heads=2, head_dim=128, vocab_size=1024,
                 tie_word_embeddings=False),
    "tiny-tied": dict(hidden_size=256, num_hidden_layers=3, intermediate_size=512,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=128, vocab_size=1024,
                      tie_word_embeddings=True),
    # Gemma-style 12B shape: sandwich norms, GeGLU, 5 sliding (1024) : 1 global layers, soft-cap 30
    "gemma-12b": dict(model_type="gemma4_text", hidden_size=3840, num_hidden_layers=48, intermediate_size=15360,
                      num_attention_heads=16, num_key_value_heads=8, head_dim=256, vocab_size=262144,
                      tie_word_embeddings=True, hidden_act="gelu_tanh", sliding_window=1024,
                      final_logit_softcapping=30.0, query_pre_attn_scalar=256.0, rope_local_base_freq=10_000.0),
    "tiny-gemma": dict(model_type="gemma4_text", hidden_size=512, num_hidden_layers=6, intermediate_size=1024,
                       num_attention_heads=4, num_key_value_heads=2, head_dim=256, vocab_size=1024,
                       tie_word_embeddings=True, hidden_act="gelu_tanh", sliding_window=32,
                       final_logit_softcapping=30.0, query_pre_attn_scalar=256.0, rope_local_base_freq=10_000.0),
}


def target_args(name: str) -> TargetArgs:
    """TargetArgs of a named synthetic shape (Gemma-style shapes get their embedding scale,
    bf16(sqrt(hidden)), and the 5:1 sliding/global layer pattern)."""
    spec = {"model_type": "qwen3", **TARGETS[name]}
    a = TargetArgs(**spec)
    if a.sandwich_norms:
        a.embed_scale = float(torch.tensor(a.hidden_size ** 0.5).to(torch.bfloat16))
        a.layer_types = tuple("full_attention" if (l + 1) % 6 == 0 else "sliding_attention"
                              for l in range(a.num_hidden_layers))
    return a


def _seed(seed: int, name: str) -> int:
    h = hashlib.sha256(f"{seed}:{name}".encode()).digest()
    return int.from_bytes(h[:8], "little") & ((1 << 63) - 1)


def randn(shape, seed: int, name: str, device, std: float = STD) -> torch.Tensor:
    g = torch.Generator(device=device)
    g.manual_seed(_seed(seed, name))
    return torch.randn(shape, generator=g, device=device, dtype=torch.float32) * std


def w8(N: int, K: int, seed: int, name: str, device, keep_mlx: bool = False, paired: bool = False,
       bits: int = 8) -> W8Weight:
    """A seeded random [N, K] weight quantized affine group 64 (8-bit, or 4-bit codes)."""
    w = randn((N, K), seed, name, device)
    q, s, b = W8Weight.quantize_mlx(w, bits)
    del w
    W = W8Weight.from_mlx(q, s, b, paired, bits)
    if keep_mlx:
        W.mlx = (q, s, b)
    return W


def w8_table(V: int, H: int, seed: int, name: str, device, bits: int = 8) -> W8Table:
    w = randn((V, H), seed, name, device)
    q, s, b = W8Weight.quantize_mlx(w, bits)
    return W8Table(q, s, b)


def ones(n: int, device) -> torch.Tensor:
    return torch.ones(n, dtype=torch.bfloat16, device=device)


def qk_norm(hd: int, device) -> torch.Tensor:
    """q/k RMSNorm gains of hd**-0.25, so normalised q.k / sqrt(hd) has unit variance (with
    unit gains a random model's attention is nearly one-hot, unlike a trained model's)."""
    return torch.full((hd,), hd ** -0.25, dtype=torch.bfloat16, device=device)


def build_target(name_or_args, seed: int = 0, device="cuda", keep_mlx: bool = False, bits: int = 8) -> Qwen3W8:
    """A seeded random-init target; bits = 4 quantizes every linear and the embedding to 4-bit
    codes (an MLX 4-bit checkpoint's layout)."""
    if isinstance(name_or_args, TargetArgs):
        args = name_or_args
    else:
        args = target_args(name_or_args)
    device = torch.device(device)
    H, I = args.hidden_size, args.intermediate_size
    nq, nkv, hd = args.num_attention_heads, args.num_key_value_heads, args.head_dim
    layers = []
    for l in range(args.num_hidden_layers):
        p = f"layers.{l}."
        layers.append(LayerWeights(
            qkv=w8(args.n_qkv, H, seed, p + "qkv", device, keep_mlx, bits=bits),
            o=w8(H, nq * hd, seed, p + "o", device, keep_mlx, bits=bits),
            gate_up=w8(2 * I, H, seed, p + "gate_up", device, keep_mlx, paired=True, bits=bits),
            down=w8(H, I, seed, p + "down", device, keep_mlx, bits=bits),
            in_norm=ones(H, device), post_norm=ones(H, device),
            q_norm=qk_norm(hd, device), k_norm=qk_norm(hd, device),
            attn_out_norm=ones(H, device) if args.sandwich_norms else None,
            ff_out_norm=ones(H, device) if args.sandwich_norms else None))
    embed = w8_table(args.vocab_size, H, seed, "embed_tokens", device, bits=bits)
    if args.tie_word_embeddings:
        lm_head = W8Weight.from_mlx(embed.q, embed.s, embed.b, bits=bits)
        if keep_mlx:
            lm_head.mlx = (embed.q, embed.s, embed.b)
    else:
        lm_head = w8(args.vocab_size, H, seed, "lm_head", device, keep_mlx, bits=bits)
    torch.cuda.synchronize(device)
    return Qwen3W8(args, layers, embed, lm_head, ones(H, device))


def randomize_norms(model, seed: int, spread: float = 0.25) -> None:
    """Scale every RMSNorm gain of a built model (target or drafter: layer norms, q/k norms,
    sandwich norms, final and hidden norms) by 1 + spread * N(0, 1), in place, seeded: models
    whose gains are not all equal, so a norm applied to the wrong tensor or left out changes the
    output."""
    g = torch.Generator().manual_seed(seed)
    tensors = []
    for L in getattr(model, "layers", []):
        for name in ("in_norm", "post_norm", "q_norm", "k_norm", "attn_out_norm", "ff_out_norm"):
            t = getattr(L, name, None)
            if t is not None:
                tensors.append(t)
    for name in ("norm", "hidden_norm"):
        t = getattr(model, name, None)
        if torch.is_tensor(t):
            tensors.append(t)
    for t in tensors:
        f = 1.0 + spread * torch.randn(t.shape, generator=g)
        t.copy_((t.float().cpu() * f).to(t.dtype))


def evenly_spaced_layers(n_target_layers: int, n: int) -> list[int]:
    """n distinct tap layers spread over the target: from layer 1 to layer L-3 (the DFlash
    convention) when the target is deep enough, else over all layers."""
    if n > n_target_layers:
        raise ValueError(f"{n} taps from a {n_target_layers}-layer target")
    if n == 1:
        return [n_target_layers // 2]
    lo, hi = (1, n_target_layers - 3) if n_target_layers - 3 - 1 >= n - 1 else (0, n_target_layers - 1)
    return [int(round(lo + i * (hi - lo) / (n - 1))) for i in range(n)]


def _w8_k_eq_v(nq_rows: int, k_rows: int, K: int, seed: int, name: str, device, keep_mlx: bool,
               bits: int = 8) -> W8Weight:
    """The [q | k | k] projection of a k_eq_v attention: the shared k_proj rows twice (the
    second copy is V's input), quantized row by row, so both copies are identical."""
    q1, s1, b1 = W8Weight.quantize_mlx(randn((nq_rows, K), seed, name + ".q_proj", device), bits)
    q2, s2, b2 = W8Weight.quantize_mlx(randn((k_rows, K), seed, name + ".k_proj", device), bits)
    q, s, b = torch.cat([q1, q2, q2]), torch.cat([s1, s2, s2]), torch.cat([b1, b2, b2])
    W = W8Weight.from_mlx(q, s, b, bits=bits)
    if keep_mlx:
        W.mlx = (q, s, b)
    return W


def build_dspark(target_args: TargetArgs, seed: int = 2, device="cuda", keep_mlx: bool = False,
                 num_hidden_layers: int = 1, block_size: int = 7, taps=None, markov_rank: int = 256,
                 confidence: bool = True, mask_token_id: int | None = None, family: str = "qwen3",
                 global_head_dim: int = 512, bits: int = 4):
    """A DSpark drafter of the target's width, with its own embedding and head, a
    rank-``markov_rank`` Markov head and a confidence head, conditioned on the target layers
    ``taps`` (default: 3 spread over the target).
    family "qwen3": heads and MLP shaped like the target, Llama 2-norm layers.
    family "gemma4": the target's q heads over one global kv head of ``global_head_dim``
    (k_eq_v, v_norm, proportional RoPE over a quarter of the dims), sandwich norms with
    layer_scalar 1, tanh-GeLU MLP, soft-cap 30, embedding scale sqrt(hidden).
    bits: the code width of every linear and embedding table (4, the reference's drafter default,
    or 8). Tables are gathered row by row and hold one code per byte; the Markov w2 projection
    keeps 4-bit code values in the 8-bit tile layout its kernel streams."""
    from .config import DSparkConfig
    from .model import ConfidenceHead, DSparkDrafter, MarkovHead

    a = target_args
    device = torch.device(device)
    L = a.num_hidden_layers
    taps = list(taps) if taps is not None else [1, L // 2, L - 1] if L >= 3 else list(range(L))
    gemma = family == "gemma4"
    if family not in ("qwen3", "gemma4"):
        raise ValueError(f"unknown DSpark family {family!r}")
    common = dict(hidden_size=a.hidden_size, vocab_size=a.vocab_size, num_hidden_layers=num_hidden_layers,
                  intermediate_size=a.intermediate_size, rms_norm_eps=a.rms_norm_eps,
                  num_attention_heads=a.num_attention_heads, block_size=block_size,
                  mask_token_id=a.vocab_size - 2 if mask_token_id is None else mask_token_id,
                  target_layer_ids=taps, num_target_layers=L, markov_rank=markov_rank,
                  enable_confidence_head=confidence, confidence_head_with_markov=markov_rank > 0)
    if gemma:
        cfg = DSparkConfig(family="gemma4", num_key_value_heads=a.num_key_value_heads, num_global_key_value_heads=1,
                           head_dim=a.head_dim, global_head_dim=global_head_dim, attention_k_eq_v=True,
                           rope_theta=1_000_000.0, partial_rotary_factor=0.25, rope_type="proportional",
                           final_logit_softcapping=30.0, mlp_activation="gelu_tanh", norm_style="gemma",
                           use_v_norm=True, **common)
    else:
        cfg = DSparkConfig(family="qwen3", num_key_value_heads=a.num_key_value_heads, head_dim=a.head_dim,
                           attention_k_eq_v=False, rope_theta=a.rope_theta, rope_type="default",
                           final_logit_softcapping=None, mlp_activation="silu", norm_style="qwen", use_v_norm=False,
                           **common)
    H, I = a.hidden_size, a.intermediate_size
    nq, nkv, hd = cfg.num_attention_heads, cfg.n_kv_heads, cfg.attn_head_dim
    layers = []
    for l in range(num_hidden_layers):
        p = f"dspark.layers.{l}."
        qkv = (_w8_k_eq_v(nq * hd, nkv * hd, H, seed, p + "attn", device, keep_mlx, bits) if gemma
               else w8(a.n_qkv, H, seed, p + "qkv", device, keep_mlx, bits=bits))
        layers.append(LayerWeights(
            qkv=qkv,
            o=w8(H, nq * hd, seed, p + "o", device, keep_mlx, bits=bits),
            gate_up=w8(2 * I, H, seed, p + "gate_up", device, keep_mlx, paired=True, bits=bits),
            down=w8(H, I, seed, p + "down", device, keep_mlx, bits=bits),
            in_norm=ones(H, device), post_norm=ones(H, device),
            q_norm=qk_norm(hd, device), k_norm=qk_norm(hd, device),
            attn_out_norm=ones(H, device) if gemma else None, ff_out_norm=ones(H, device) if gemma else None))
    markov = None
    if markov_rank > 0:
        w1 = w8_table(a.vocab_size, markov_rank, seed, "dspark.markov_w1", device, bits=bits)
        q2, s2, b2 = W8Weight.quantize_mlx(randn((a.vocab_size, markov_rank), seed, "dspark.markov_w2", device), bits)
        w2 = W8Weight.from_mlx(q2, s2, b2, bits=8)
        if keep_mlx:
            w2.mlx = (q2, s2, b2)
        markov = MarkovHead(w1, w2)
    conf = None
    if confidence:
        K = H + (markov_rank if markov_rank > 0 else 0)
        w = randn((1, K), seed, "dspark.confidence", device)
        w = torch.cat([w, torch.zeros((15, K), device=device)])
        q, s_, b_ = W8Weight.quantize_mlx(w, bits)
        cw = W8Weight.from_mlx(q, s_, b_, bits=bits)
        if keep_mlx:
            cw.mlx = (q, s_, b_)
        conf = ConfidenceHead(cw, 0.5)
    d = DSparkDrafter(cfg, embed=w8_table(a.vocab_size, H, seed, "dspark.embed_tokens", device, bits=bits),
                      fc=w8(H, len(taps) * H, seed, "dspark.fc", device, keep_mlx, bits=bits),
                      hidden_norm=ones(H, device),
                      layers=layers, norm=ones(H, device),
                      lm_head=w8(a.vocab_size, H, seed, "dspark.lm_head", device, keep_mlx, bits=bits),
                      markov=markov, confidence=conf, layer_scalars=[1.0] * num_hidden_layers if gemma else None)
    torch.cuda.synchronize(device)
    return d, cfg


def build_dflash(target_args: TargetArgs, seed: int = 1, device="cuda", keep_mlx: bool = False,
                 num_hidden_layers: int = 2, block_size: int = 16, n_taps: int = 5,
                 mask_token_id: int | None = None, bits: int = 4, layer_types: tuple | None = None,
                 sliding_window: int | None = None):
    """A DFlash drafter shaped like the target (same width, heads and MLP), conditioned on
    n_taps evenly spaced target layers, with a block of block_size positions; its linear
    layers quantized to ``bits`` (4, the reference's default, or 8). ``layer_types`` /
    ``sliding_window``: per-layer "sliding_attention" / "full_attention" as in the reference's
    config (src/mlx_dspark/dflash_model.py:90-92); default all full."""
    from .dflash_model import DFlashConfig, DFlashDraftModel

    a = target_args
    device = torch.device(device)
    cfg = DFlashConfig(
        hidden_size=a.hidden_size, num_hidden_layers=num_hidden_layers,
        num_attention_heads=a.num_attention_heads, num_key_value_heads=a.num_key_value_heads,
        head_dim=a.head_dim, intermediate_size=a.intermediate_size, vocab_size=a.vocab_size,
        rms_norm_eps=a.rms_norm_eps, rope_theta=a.rope_theta,
        max_position_embeddings=a.max_position_embeddings, block_size=block_size,
        target_layer_ids=tuple(evenly_spaced_layers(a.num_hidden_layers, n_taps)),
        num_target_layers=a.num_hidden_layers,
        mask_token_id=a.vocab_size - 1 if mask_token_id is None else mask_token_id,
        layer_types=tuple(layer_types or ()), sliding_window=sliding_window)
    H, I = a.hidden_size, a.intermediate_size
    nq, nkv, hd = a.num_attention_heads, a.num_key_value_heads, a.head_dim
    layers = []
    for l in range(num_hidden_layers):
        p = f"dflash.layers.{l}."
        layers.append(LayerWeights(
            qkv=w8(a.n_qkv, H, seed, p + "qkv", device, keep_mlx, bits=bits),
            o=w8(H, nq * hd, seed, p + "o", device, keep_mlx, bits=bits),
            gate_up=w8(2 * I, H, seed, p + "gate_up", device, keep_mlx, paired=True, bits=bits),
            down=w8(H, I, seed, p + "down", device, keep_mlx, bits=bits),
            in_norm=ones(H, device), post_norm=ones(H, device),
            q_norm=qk_norm(hd, device), k_norm=qk_norm(hd, device)))
    fc = w8(H, n_taps * H, seed, "dflash.fc", device, keep_mlx, bits=bits)
    torch.cuda.synchronize(device)
    return DFlashDraftModel(cfg, fc, ones(H, device), layers, ones(H, device)), cfg
