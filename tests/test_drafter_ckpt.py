"""Drafter checkpoint format on the CPU: the parameter names the loader expects are the reference
modules' (src/mlx_dspark/model.py:196-245, dflash_model.py:100-208), a checkpoint with other names
is refused before anything is read to the device (load.py:175-199, :271-279), DeepSpec config.json
round trips, and a DFlash checkpoint with a Markov head is refused (load.py:242-249)."""

import json

import pytest
import torch

from mlx_dspark import drafter_ckpt as DC
from mlx_dspark.config import DSparkConfig


def _cfg(family):
    base = dict(hidden_size=256, vocab_size=1024, num_hidden_layers=1, intermediate_size=512,
                num_attention_heads=4, num_key_value_heads=2, block_size=4, mask_token_id=3,
                target_layer_ids=[0, 2], num_target_layers=3, markov_rank=64)
    if family == "qwen3":
        return DSparkConfig.from_dict({"model_type": "qwen3", "head_dim": 128, **base})
    return DSparkConfig.from_dict({"model_type": "gemma4_text", "head_dim": 256, "global_head_dim": 512, **base})


def test_dspark_key_names_follow_the_reference_modules():
    # a 1-layer qwen3-family drafter: DSparkDrafter's parameter tree (model.py:220-245)
    want = {"embed_tokens.weight", "fc.weight", "hidden_norm.weight", "norm.weight", "lm_head.weight",
            "layers.0.self_attn.q_proj.weight", "layers.0.self_attn.k_proj.weight",
            "layers.0.self_attn.v_proj.weight", "layers.0.self_attn.o_proj.weight",
            "layers.0.self_attn.q_norm.weight", "layers.0.self_attn.k_norm.weight",
            "layers.0.mlp.gate_proj.weight", "layers.0.mlp.up_proj.weight", "layers.0.mlp.down_proj.weight",
            "layers.0.input_layernorm.weight", "layers.0.post_attention_layernorm.weight",
            "markov_head.markov_w1.weight", "markov_head.markov_w2.weight",
            "confidence_head.proj.weight", "confidence_head.proj.bias"}
    assert set(DC.dspark_keys(_cfg("qwen3"))) == want
    # gemma4: k_eq_v drops v_proj (model.py:99-100), sandwich norms and layer_scalar (:167-170)
    g = set(DC.dspark_keys(_cfg("gemma4")))
    assert "layers.0.self_attn.v_proj.weight" not in g
    assert {"layers.0.pre_feedforward_layernorm.weight", "layers.0.post_feedforward_layernorm.weight",
            "layers.0.layer_scalar"} <= g
    # no Markov / confidence heads when the config turns them off (model.py:238-242)
    c = _cfg("qwen3")
    c.markov_rank, c.enable_confidence_head = 0, False
    assert not any(k.startswith(("markov_head", "confidence_head")) for k in DC.dspark_keys(c))


def test_config_json_round_trip():
    for fam in ("qwen3", "gemma4"):
        c = _cfg(fam)
        assert DSparkConfig.from_dict(DC.dspark_config_dict(c)) == c


def _write(tmp_path, cfg_dict, tensors):
    from safetensors.torch import save_file
    (tmp_path / "config.json").write_text(json.dumps(cfg_dict))
    save_file(tensors, str(tmp_path / "model.safetensors"))


def test_mismatched_names_are_refused(tmp_path):
    c = _cfg("qwen3")
    keys = DC.dspark_keys(c)
    tensors = {k: torch.zeros(1) for k in keys if k != "fc.weight"}
    tensors["fc_proj.weight"] = torch.zeros(1)       # a renamed tensor
    _write(tmp_path, DC.dspark_config_dict(c), tensors)
    with pytest.raises(ValueError, match=r"(?s)missing in checkpoint \(1\): \[.fc.weight.\].*unexpected in checkpoint"):
        DC.load_dspark(tmp_path, device="cpu")


def test_dflash_with_a_markov_head_is_refused(tmp_path):
    cfg = {"hidden_size": 256, "num_hidden_layers": 1, "num_attention_heads": 4, "num_key_value_heads": 2,
           "head_dim": 128, "intermediate_size": 512, "vocab_size": 1024, "rms_norm_eps": 1e-6,
           "max_position_embeddings": 4096, "block_size": 8, "target_layer_ids": [0], "num_target_layers": 2,
           "markov_rank": 256}
    _write(tmp_path, cfg, {"fc.weight": torch.zeros(1)})
    with pytest.raises(ValueError, match="Markov head"):
        DC.load_dflash(tmp_path, device="cpu")


def test_dflash_key_names_and_exact_match(tmp_path):
    cfg = {"hidden_size": 256, "num_hidden_layers": 2, "num_attention_heads": 4, "num_key_value_heads": 2,
           "head_dim": 128, "intermediate_size": 512, "vocab_size": 1024, "rms_norm_eps": 1e-6,
           "max_position_embeddings": 4096, "block_size": 8, "dflash_config": {"target_layer_ids": [0, 1],
                                                                               "mask_token_id": 7},
           "num_target_layers": 3}
    c = DC.dflash_config_from_dict(cfg)
    assert c.target_layer_ids == (0, 1) and c.mask_token_id == 7
    keys = DC.dflash_keys(c)
    assert "layers.1.mlp.down_proj.weight" in keys and "embed_tokens.weight" not in keys
    _write(tmp_path, cfg, {k: torch.zeros(1) for k in keys[:-1]})
    with pytest.raises(ValueError, match="missing in checkpoint"):
        DC.load_dflash(tmp_path, device="cpu")
