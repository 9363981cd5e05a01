"""Local MLX-format checkpoints: config parsing (CPU) and, on the GPU, a save -> load round trip
whose forward is bit-identical to the model it was written from, plus an unquantized (bf16)
checkpoint that the loader quantizes."""

import json

import numpy as np
import pytest
import torch

QWEN3_8B_CONFIG = {     # the fields of mlx-community/Qwen3-8B-8bit's config.json that the loader reads
    "model_type": "qwen3", "hidden_size": 4096, "num_hidden_layers": 36, "intermediate_size": 12288,
    "num_attention_heads": 32, "num_key_value_heads": 8, "head_dim": 128, "vocab_size": 151936,
    "rms_norm_eps": 1e-6, "rope_theta": 1000000, "tie_word_embeddings": False,
    "max_position_embeddings": 40960, "quantization": {"group_size": 64, "bits": 8}}


def test_target_args_from_qwen3_config():
    from mlx_dspark import checkpoint, synthetic
    a = checkpoint.target_args_from_config(QWEN3_8B_CONFIG)
    b = synthetic.target_args("qwen3-8b")
    for k in ("hidden_size", "num_hidden_layers", "intermediate_size", "num_attention_heads",
              "num_key_value_heads", "head_dim", "vocab_size", "tie_word_embeddings"):
        assert getattr(a, k) == getattr(b, k), k
    assert a.rope_theta == 1e6 and a.rms_norm_eps == 1e-6
    assert checkpoint._quantization(QWEN3_8B_CONFIG) == (8, 64)
    nested = {"model_type": "qwen3", "text_config": dict(QWEN3_8B_CONFIG, head_dim=None)}
    assert checkpoint.target_args_from_config(nested).head_dim == 128     # hidden / heads


@pytest.mark.parametrize("bad, what", [
    ({"model_type": "llama"}, "qwen3-family"),
    ({"hidden_size": 4000}, "unsupported shape"),
    ({"head_dim": 64}, "unsupported shape"),
    ({"vocab_size": None}, "missing"),
])
def test_config_rejections(bad, what):
    from mlx_dspark import checkpoint
    cfg = {k: v for k, v in {**QWEN3_8B_CONFIG, **bad}.items() if v is not None}
    with pytest.raises(ValueError, match=what):
        checkpoint.target_args_from_config(cfg)


@pytest.mark.parametrize("q", [{"bits": 3, "group_size": 64}, {"bits": 8, "group_size": 32},
                               {"bits": 6, "group_size": 64}])
def test_quantization_rejections(q):
    from mlx_dspark import checkpoint
    with pytest.raises(ValueError, match="8- or 4-bit codes with group 64"):
        checkpoint._quantization(dict(QWEN3_8B_CONFIG, quantization=q))
    assert checkpoint._quantization(dict(QWEN3_8B_CONFIG, quantization={"bits": 4, "group_size": 64})) == (4, 64)


def test_checkpoint_dir_detection(tmp_path):
    from mlx_dspark import checkpoint
    from mlx_dspark.load import load_target
    assert not checkpoint.is_checkpoint_dir(tmp_path)
    (tmp_path / "config.json").write_text(json.dumps(QWEN3_8B_CONFIG))
    assert not checkpoint.is_checkpoint_dir(tmp_path)          # no safetensors yet
    (tmp_path / "model.safetensors").write_bytes(b"")
    assert checkpoint.is_checkpoint_dir(tmp_path)
    assert not checkpoint.has_tokenizer(tmp_path)
    with pytest.raises(ValueError, match="not a synthetic"):
        load_target(str(tmp_path / "missing"))


def _logits(model, prompt, block):
    cache = model.make_cache(max_ctx=256)
    l0, _ = model.prefill(prompt, cache, [])
    ids = torch.tensor([block], dtype=torch.int32, device=model.device)
    l1, _ = model.forward(ids, cache, None, advance=False)
    return l0[0, -1].float().cpu(), l1[0].float().cpu()


@pytest.mark.gpu
@pytest.mark.parametrize("name,bits", [("tiny", 8), ("tiny-tied", 8), ("tiny", 4), ("tiny-tied", 4)])
def test_mlx_checkpoint_round_trip_is_bit_exact(dev, tmp_path, name, bits):
    from mlx_dspark import checkpoint, synthetic
    from mlx_dspark.load import load_target
    print(f"checkpoint round trip {name} {bits}-bit", flush=True)
    model = synthetic.build_target(name, seed=11, keep_mlx=True, bits=bits)
    checkpoint.save_qwen3_w8(model, tmp_path)
    target, tok = load_target(str(tmp_path))
    loaded = target.model
    assert loaded.args.num_hidden_layers == model.args.num_hidden_layers
    assert loaded.layers[0].qkv.bits == bits and loaded.lm_head.bits == bits
    assert loaded.args.tie_word_embeddings == model.args.tie_word_embeddings
    for La, Lb in zip(model.layers, loaded.layers):
        for f in ("qkv", "o", "gate_up", "down"):
            wa, wb = getattr(La, f), getattr(Lb, f)
            assert torch.equal(wa.wt, wb.wt) and torch.equal(wa.sb, wb.sb), f
    assert torch.equal(model.lm_head.wt, loaded.lm_head.wt)
    rng = np.random.default_rng(1)
    prompt = rng.integers(0, model.args.vocab_size, 40).tolist()
    block = rng.integers(0, model.args.vocab_size, 9).tolist()
    a0, a1 = _logits(model, prompt, block)
    b0, b1 = _logits(loaded, prompt, block)
    assert torch.equal(a0, b0) and torch.equal(a1, b1)
    assert tok.encode("1 2 3") is not None


@pytest.mark.gpu
def test_unquantized_checkpoint_is_quantized_on_load(dev, tmp_path):
    """A bf16 checkpoint of the model's dequantized weights loads (quantized to W8 group 64)
    exactly as quantizing the stacked bf16 rows directly would, with logits close to the source
    model's."""
    from safetensors.torch import save_file
    from mlx_dspark import checkpoint, synthetic
    from mlx_dspark.load import load_target
    model = synthetic.build_target("tiny", seed=12, keep_mlx=True)
    checkpoint.save_qwen3_w8(model, tmp_path)
    from safetensors import safe_open
    out = {}
    with safe_open(str(tmp_path / "model.safetensors"), framework="pt") as f:
        keys = list(f.keys())
        for k in keys:
            if k.endswith(".scales") or k.endswith(".biases"):
                continue
            t = f.get_tensor(k)
            if k.endswith(".weight") and t.dtype == torch.uint32:
                base = k[:-len(".weight")]
                q = t.view(torch.uint8).float()
                s, b = f.get_tensor(base + ".scales").float(), f.get_tensor(base + ".biases").float()
                N, K = q.shape
                w = q.view(N, K // 64, 64) * s[..., None] + b[..., None]
                out[k] = w.view(N, K).to(torch.bfloat16)
            else:
                out[k] = t
    save_file(out, str(tmp_path / "model.safetensors"))
    cfg = json.loads((tmp_path / "config.json").read_text())
    del cfg["quantization"]
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    target, _ = load_target(str(tmp_path))
    from mlx_dspark.ops import W8Weight
    w = {k: v.to(dev) for k, v in out.items()}
    p = "model.layers.1."
    want = W8Weight.quantize(torch.cat([w[p + "self_attn.q_proj.weight"], w[p + "self_attn.k_proj.weight"],
                                        w[p + "self_attn.v_proj.weight"]]))
    got = target.model.layers[1].qkv
    assert torch.equal(got.wt, want.wt) and torch.equal(got.sb, want.sb)
    want = W8Weight.quantize(torch.cat([w[p + "mlp.gate_proj.weight"], w[p + "mlp.up_proj.weight"]]), paired=True)
    got = target.model.layers[1].gate_up
    assert got.paired and torch.equal(got.wt, want.wt) and torch.equal(got.sb, want.sb)
    # Requantizing bf16-rounded dequantized weights moves each weight by up to half a step, so
    # the logits agree to that perturbation rather than to kernel noise: max-abs 0.1, RMS 0.03
    # on RMS-normalised rows (a wrong row order or pairing gives O(1)).
    rng = np.random.default_rng(2)
    prompt = rng.integers(0, model.args.vocab_size, 40).tolist()
    block = rng.integers(0, model.args.vocab_size, 9).tolist()
    a0, a1 = _logits(model, prompt, block)
    b0, b1 = _logits(target.model, prompt, block)
    for got, ref, what in ((b0, a0, "prefill row"), (b1, a1, "verify block")):
        a = got.reshape(-1, got.shape[-1])
        b = ref.reshape(-1, ref.shape[-1])
        d = a / a.pow(2).mean(-1, keepdim=True).sqrt() - b / b.pow(2).mean(-1, keepdim=True).sqrt()
        mx, rms = float(d.abs().max()), float(d.pow(2).mean().sqrt())
        print(f"bf16 checkpoint {what}: normalised max-abs {mx:.4f} rms {rms:.5f}", flush=True)
        assert mx < 0.1 and rms < 0.03, (what, mx, rms)
