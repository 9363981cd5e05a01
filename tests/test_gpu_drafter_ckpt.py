"""GPU: drafter checkpoints (src/mlx_dspark/load.py:155-215, :224-289). An engine drafter saved in
the MLX-quantized checkpoint format and loaded back is the same drafter bit for bit (every matrix,
table, norm and layer scalar) and drafts bit-identical logits; a bf16 checkpoint under the
reference's key names is quantized on load to 4-bit codes, each engine matrix holding exactly the
named tensors' rows (fused q|k|v, paired gate|up; gemma's sandwich norms in their places), the
embedding and Markov tables included; strict=False loads a partial checkpoint with a warning."""

import warnings

import pytest
import torch

pytestmark = pytest.mark.gpu


def _same_w(a, b, what):
    assert (a.N, a.K, a.bits, a.paired) == (b.N, b.K, b.bits, b.paired), what
    assert torch.equal(a.wt, b.wt) and torch.equal(a.sb, b.sb), what


def _same_t(a, b, what):
    assert torch.equal(a.q, b.q) and torch.equal(a.s, b.s) and torch.equal(a.b, b.b), what


def _same_drafter(d, e):
    _same_t(d.embed_tokens, e.embed_tokens, "embed")
    _same_w(d.fc, e.fc, "fc")
    _same_w(d.lm_head, e.lm_head, "lm_head")
    assert torch.equal(d.hidden_norm, e.hidden_norm) and torch.equal(d.norm, e.norm)
    for l, (a, b) in enumerate(zip(d.layers, e.layers)):
        for n in ("qkv", "o", "gate_up", "down"):
            _same_w(getattr(a, n), getattr(b, n), f"layer {l} {n}")
        for n in ("in_norm", "post_norm", "q_norm", "k_norm", "attn_out_norm", "ff_out_norm"):
            x, y = getattr(a, n), getattr(b, n)
            assert (x is None and y is None) or torch.equal(x, y), f"layer {l} {n}"
    if getattr(d, "markov_head", None) is not None:
        _same_t(d.markov_head.w1, e.markov_head.w1, "markov w1")
        _same_w(d.markov_head.w2, e.markov_head.w2, "markov w2")
    if getattr(d, "confidence_head", None) is not None:
        _same_w(d.confidence_head.proj, e.confidence_head.proj, "confidence")
        assert d.confidence_head.bias == pytest.approx(e.confidence_head.bias, rel=1e-2)


@pytest.mark.parametrize("family", ["qwen3", "gemma4"])
def test_dspark_save_load_round_trip(dev, tmp_path, family):
    from mlx_dspark import drafter_ckpt as DC
    from mlx_dspark import synthetic
    from mlx_dspark.load import load_drafter
    print(f"DSpark checkpoint round trip, {family}", flush=True)
    args = synthetic.target_args("tiny" if family == "qwen3" else "tiny-gemma")
    d, cfg = synthetic.build_dspark(args, seed=5, keep_mlx=True, num_hidden_layers=2, block_size=4, family=family)
    synthetic.randomize_norms(d, seed=6)
    if family == "gemma4":
        d.layer_scalars = [1.25, 0.75]
    DC.save_dspark(d, tmp_path)
    e, ecfg = load_drafter(str(tmp_path), keep_mlx=True)
    assert ecfg == cfg
    _same_drafter(d, e)
    if family == "gemma4":
        assert e.layer_scalars == [1.25, 0.75]
    # the same context and block draft the same logits
    H = args.hidden_size
    g = torch.Generator().manual_seed(7)
    th = (torch.randn(40, len(cfg.target_layer_ids) * H, generator=g)).to(torch.bfloat16).to(dev)
    block = torch.randint(0, args.vocab_size, (1, cfg.block_size), generator=g).to(dev, torch.int32)
    outs = []
    for x in (d, e):
        cache = x.make_ctx_cache(max_ctx=128)
        x.update_context(th, 0, cache)
        outs.append(x.block_logits(block, cache, cfg.block_size - 1).clone())
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])


def _ref_tensors(cfg, gen):
    """Random bf16 tensors under the reference's parameter names and shapes (model.py:83-245)."""
    H, V, I, R = cfg.hidden_size, cfg.vocab_size, cfg.intermediate_size, cfg.markov_rank
    nq, nkv, hd = cfg.num_attention_heads, cfg.n_kv_heads, cfg.attn_head_dim
    gemma = cfg.norm_style == "gemma"
    rnd = lambda *s: (torch.randn(*s, generator=gen) * 0.05).to(torch.bfloat16)
    gain = lambda n: (1 + 0.3 * torch.randn(n, generator=gen)).to(torch.bfloat16)
    t = {"embed_tokens.weight": rnd(V, H), "fc.weight": rnd(H, len(cfg.target_layer_ids) * H),
         "hidden_norm.weight": gain(H), "norm.weight": gain(H), "lm_head.weight": rnd(V, H),
         "markov_head.markov_w1.weight": rnd(V, R), "markov_head.markov_w2.weight": rnd(V, R),
         "confidence_head.proj.weight": rnd(1, H + R), "confidence_head.proj.bias": rnd(1)}
    for l in range(cfg.num_hidden_layers):
        p, a = f"layers.{l}.", f"layers.{l}.self_attn."
        t.update({a + "q_proj.weight": rnd(nq * hd, H), a + "k_proj.weight": rnd(nkv * hd, H),
                  a + "o_proj.weight": rnd(H, nq * hd), a + "q_norm.weight": gain(hd), a + "k_norm.weight": gain(hd),
                  p + "mlp.gate_proj.weight": rnd(I, H), p + "mlp.up_proj.weight": rnd(I, H),
                  p + "mlp.down_proj.weight": rnd(H, I), p + "input_layernorm.weight": gain(H),
                  p + "post_attention_layernorm.weight": gain(H)})
        if not cfg.attention_k_eq_v:
            t[a + "v_proj.weight"] = rnd(nkv * hd, H)
        if gemma:
            t.update({p + "pre_feedforward_layernorm.weight": gain(H), p + "post_feedforward_layernorm.weight": gain(H),
                      p + "layer_scalar": torch.tensor([0.8], dtype=torch.bfloat16)})
    return t


@pytest.mark.parametrize("family", ["qwen3", "gemma4"])
def test_dspark_bf16_checkpoint_quantized_on_load(dev, tmp_path, family):
    import json

    from safetensors.torch import save_file

    from mlx_dspark import drafter_ckpt as DC
    from mlx_dspark import synthetic
    from mlx_dspark.load import load_drafter
    from mlx_dspark.ops import W8Weight
    print(f"DSpark bf16 checkpoint, {family}", flush=True)
    args = synthetic.target_args("tiny" if family == "qwen3" else "tiny-gemma")
    _, cfg = synthetic.build_dspark(args, seed=1, num_hidden_layers=2, block_size=4, family=family)
    t = _ref_tensors(cfg, torch.Generator().manual_seed(3))
    (tmp_path / "config.json").write_text(json.dumps(DC.dspark_config_dict(cfg)))
    save_file(t, str(tmp_path / "model.safetensors"))
    d, _ = load_drafter(str(tmp_path))          # bits 4 (the reference's default)
    on = lambda k: t[k].to(dev)
    q4 = lambda *ks, paired=False: W8Weight.quantize(torch.cat([on(k) for k in ks]), paired=paired, bits=4)
    _same_w(d.fc, q4("fc.weight"), "fc")
    _same_w(d.lm_head, q4("lm_head.weight"), "lm_head")
    qe = W8Weight.quantize_mlx(on("embed_tokens.weight"), 4)
    assert torch.equal(d.embed_tokens.q, qe[0]) and int(d.embed_tokens.q.max()) <= 15
    q1 = W8Weight.quantize_mlx(on("markov_head.markov_w1.weight"), 4)
    assert torch.equal(d.markov_head.w1.q, q1[0]) and int(d.markov_head.w1.q.max()) <= 15
    _same_w(d.markov_head.w2, W8Weight.from_mlx(*W8Weight.quantize_mlx(on("markov_head.markov_w2.weight"), 4), bits=8),
            "markov w2 (4-bit codes, byte tiles)")
    assert d.confidence_head.bias == pytest.approx(float(t["confidence_head.proj.bias"]), rel=1e-3)
    gemma = family == "gemma4"
    for l, L in enumerate(d.layers):
        p, a = f"layers.{l}.", f"layers.{l}.self_attn."
        v = a + ("k_proj.weight" if gemma else "v_proj.weight")       # k_eq_v: V from k_proj
        _same_w(L.qkv, q4(a + "q_proj.weight", a + "k_proj.weight", v), f"layer {l} qkv")
        _same_w(L.o, q4(a + "o_proj.weight"), f"layer {l} o")
        _same_w(L.gate_up, q4(p + "mlp.gate_proj.weight", p + "mlp.up_proj.weight", paired=True), f"layer {l} gate_up")
        _same_w(L.down, q4(p + "mlp.down_proj.weight"), f"layer {l} down")
        assert torch.equal(L.in_norm, on(p + "input_layernorm.weight"))
        assert torch.equal(L.q_norm, on(a + "q_norm.weight")) and torch.equal(L.k_norm, on(a + "k_norm.weight"))
        if gemma:   # input -> attention -> post_attention norm -> add; pre_feedforward -> MLP -> post_feedforward
            assert torch.equal(L.attn_out_norm, on(p + "post_attention_layernorm.weight"))
            assert torch.equal(L.post_norm, on(p + "pre_feedforward_layernorm.weight"))
            assert torch.equal(L.ff_out_norm, on(p + "post_feedforward_layernorm.weight"))
            assert d.layer_scalars[l] == pytest.approx(0.8, rel=1e-2)
        else:
            assert torch.equal(L.post_norm, on(p + "post_attention_layernorm.weight"))
    # a partial checkpoint: strict refuses it, strict=False warns and loads (the missing matrix a
    # seeded draw of nn.Linear's initialiser: uniform in +-sqrt(1/K), not zero)
    del t["layers.1.mlp.up_proj.weight"]
    save_file(t, str(tmp_path / "model.safetensors"))
    with pytest.raises(ValueError, match="missing in checkpoint"):
        load_drafter(str(tmp_path))
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        e, _ = load_drafter(str(tmp_path), strict=False, keep_mlx=True)
    assert any("key mismatch" in str(x.message) for x in w)
    _same_w(e.layers[0].gate_up, d.layers[0].gate_up, "intact layer")
    I, H = d.config.intermediate_size, d.config.hidden_size
    from oracle import model as OM
    up = OM.deq(e.layers[1].gate_up)[I:]
    bound = (1.0 / H) ** 0.5
    assert float(up.abs().max()) <= 1.01 * bound and float(up.std()) > 0.5 * bound / 3 ** 0.5


def test_dflash_save_load_round_trip(dev, tmp_path):
    import numpy as np

    from mlx_dspark import drafter_ckpt as DC
    from mlx_dspark import synthetic
    from mlx_dspark.generate import dflash_generate
    from mlx_dspark.load import load_dflash
    from mlx_dspark.target import Target
    from mlx_dspark.tokenizer import SyntheticTokenizer
    print("DFlash checkpoint round trip", flush=True)
    model = synthetic.build_target("tiny", seed=3)
    d, cfg = synthetic.build_dflash(model.args, seed=9, keep_mlx=True, num_hidden_layers=2, block_size=8, n_taps=2)
    synthetic.randomize_norms(d, seed=4)
    DC.save_dflash(d, tmp_path)
    e, ecfg = load_dflash(str(tmp_path))
    assert ecfg == cfg
    _same_w(d.fc, e.fc, "fc")
    assert torch.equal(d.hidden_norm, e.hidden_norm) and torch.equal(d.norm, e.norm)
    for l, (a, b) in enumerate(zip(d.layers, e.layers)):
        for n in ("qkv", "o", "gate_up", "down"):
            _same_w(getattr(a, n), getattr(b, n), f"layer {l} {n}")
        for n in ("in_norm", "post_norm", "q_norm", "k_norm"):
            assert torch.equal(getattr(a, n), getattr(b, n)), (l, n)
    tok = SyntheticTokenizer(model.args.vocab_size)
    prompt = np.random.default_rng(5).integers(0, model.args.vocab_size, 40).tolist()
    streams = []
    for x in (d, e):
        x.bind(model)
        streams.append(dflash_generate(Target(model, tok), tok, x, prompt_ids=prompt, max_new_tokens=12).token_ids)
    assert streams[0] == streams[1]
