"""Loaders and the drafter registry (drop-in for src/mlx_dspark/load.py).

``load_pair`` / ``load_dflash_pair`` / ``load_target`` / ``load_dflash`` keep the reference's
signatures and return values (load.py:155-373). Model names under ``synthetic/`` build seeded
random-init W8 models at the benchmark shapes on the GPU (there is no network for hub
downloads): a target name picks its shape, a drafter name ``synthetic/dspark-<target>`` or
``synthetic/dflash-<target>`` builds a drafter matched to that target.
"""

from __future__ import annotations

import os

from . import synthetic
from .qwen3 import TargetArgs
from .target import Target
from .tokenizer import SyntheticTokenizer

# registry: target name -> matched drafters (same role as the reference's REGISTRY, load.py:54-64)
REGISTRY = [
    {"id": "qwen3-0.6b", "target": "synthetic/qwen3-0.6b", "dspark": "synthetic/dspark-qwen3-0.6b",
     "dflash": "synthetic/dflash-qwen3-0.6b", "ram": "~0.7 GB"},
    {"id": "qwen3-8b", "target": "synthetic/qwen3-8b", "dspark": "synthetic/dspark-qwen3-8b",
     "dflash": "synthetic/dflash-qwen3-8b", "ram": "~9 GB"},
    {"id": "tiny", "target": "synthetic/tiny", "dspark": "synthetic/dspark-tiny",
     "dflash": "synthetic/dflash-tiny", "ram": "~1 MB"},
    {"id": "gemma-12b", "target": "synthetic/gemma-12b", "dspark": "synthetic/dspark-gemma-12b",
     "ram": "~13 GB"},
    {"id": "tiny-gemma", "target": "synthetic/tiny-gemma", "dspark": "synthetic/dspark-tiny-gemma", "ram": "~2 MB"},
]
PRESETS = {"qwen3": {"target": "synthetic/qwen3-0.6b", "drafter": "synthetic/dspark-qwen3-0.6b"},
           "gemma4": {"target": "synthetic/gemma-12b", "drafter": "synthetic/dspark-gemma-12b"}}
DFLASH_PRESETS = {"qwen3": {"target": "synthetic/qwen3-8b", "drafter": "synthetic/dflash-qwen3-8b"}}
DEFAULT_TARGET = PRESETS["qwen3"]["target"]
DEFAULT_DRAFTER = PRESETS["qwen3"]["drafter"]
_FAMILY_ALIASES = {"qwen3": "synthetic/qwen3-0.6b", "gemma4": "synthetic/gemma-12b"}


def _registry_entry(target: str):
    key = os.path.basename(str(target).rstrip("/")).lower()
    for e in sorted(REGISTRY, key=lambda e: -len(e["id"])):
        if e["id"] == key or e["id"] in key.split("-", 1)[-1] or key.endswith(e["id"]):
            return e
    return None


def resolve(model=None, *, mode="dspark", drafter=None, family=None, target=None):
    """(target_name, drafter_name) for a target and a mode (load.py:85-112)."""
    tgt = model or target or family
    tgt = _FAMILY_ALIASES.get(tgt, tgt) or DEFAULT_TARGET
    if mode in ("baseline", "lookup"):
        return tgt, None
    if drafter:
        return tgt, drafter
    e = _registry_entry(tgt)
    if e is not None and e.get(mode):
        return tgt, e[mode]
    raise ValueError(f"no built-in {mode} drafter is registered for target {tgt!r} — pass drafter=...")


def resolve_mode(model=None, *, mode="auto", drafter=None, family=None, target=None):
    if mode != "auto":
        t, d = resolve(model, mode=mode, drafter=drafter, family=family, target=target)
        return mode, t, d
    if drafter:
        t, d = resolve(model, mode="dspark", drafter=drafter, family=family, target=target)
        return "dspark", t, d
    t, _ = resolve(model, mode="baseline", family=family, target=target)
    e = _registry_entry(t)
    if e is not None:
        for m in ("dspark", "dflash"):
            if e.get(m):
                return m, t, e[m]
    return "lookup", t, None


def _synthetic_key(name: str) -> str:
    if not str(name).startswith("synthetic/"):
        raise ValueError(f"{name!r}: not a synthetic/* model name, nor a local checkpoint directory "
                         f"(config.json + *.safetensors); hub downloads are not available offline")
    return str(name).split("/", 1)[1]


def apply_wired_limit() -> None:
    """No-op on this engine (HBM residency needs no wiring)."""


def load_target(repo_or_path: str = DEFAULT_TARGET, *, require_tap: bool = False, kv_bits=None,
                kv_group_size: int = 64, seed: int = 0, keep_mlx: bool = False, max_ctx=None):
    """(Target, tokenizer) for a synthetic target or a local MLX checkpoint directory
    (config.json + safetensors, 8-bit group-64 or unquantized qwen3; load.py:314-351)."""
    from . import checkpoint
    if checkpoint.is_checkpoint_dir(repo_or_path):
        model = checkpoint.load_qwen3_w8(repo_or_path)
        if checkpoint.has_tokenizer(repo_or_path):
            tok = checkpoint.load_tokenizer(repo_or_path)
        else:                               # weights-only directory: token ids in and out
            tok = SyntheticTokenizer(model.args.vocab_size)
    else:
        key = _synthetic_key(repo_or_path)
        if key not in synthetic.TARGETS:
            raise ValueError(f"unknown synthetic target {key!r}; known: {sorted(synthetic.TARGETS)}")
        model = synthetic.build_target(key, seed=seed, keep_mlx=keep_mlx)
        tok = SyntheticTokenizer(model.args.vocab_size)
    target = Target(model, tok, kv_bits=kv_bits, kv_group_size=kv_group_size, max_ctx=max_ctx)
    if require_tap:
        target.verify_tap()
    return target, tok


def load_dflash(repo_or_path: str, *, quantize: bool = True, bits: int = 4, group_size: int = 64,
                target_args: TargetArgs | None = None, seed: int = 1, keep_mlx: bool = False):
    """(drafter, config) for a DFlash drafter (load.py:224-289): a local z-lab-format checkpoint
    directory (exact key match; drafter_ckpt.py) or a synthetic name; its linear layers 4-bit by
    default, as the reference quantizes them (8 also runs)."""
    if bits not in (4, 8) or group_size != 64 or not quantize:
        raise ValueError("this engine runs 4- or 8-bit (group 64) drafters")
    from . import checkpoint, drafter_ckpt
    if checkpoint.is_checkpoint_dir(repo_or_path):
        return drafter_ckpt.load_dflash(repo_or_path, bits=bits, keep_mlx=keep_mlx)
    key = _synthetic_key(repo_or_path)
    if not key.startswith("dflash-"):
        raise ValueError(f"{repo_or_path!r} is not a DFlash drafter name")
    tkey = key[len("dflash-"):]
    if target_args is None:
        target_args = synthetic.target_args(tkey)
    # 5 tapped layers, or every layer of a shallower target
    n_taps = min(5, target_args.num_hidden_layers)
    return synthetic.build_dflash(target_args, seed=seed, keep_mlx=keep_mlx, bits=bits, n_taps=n_taps)


def load_drafter(repo_or_path: str = DEFAULT_DRAFTER, *, quantize: bool = True, bits: int = 4,
                 group_size: int = 64, strict: bool = True, target_args: TargetArgs | None = None, seed: int = 2,
                 keep_mlx: bool = False, **shape):
    """(drafter, config) for a DSpark drafter (load.py:155-215): a local DeepSpec-format
    checkpoint directory (key names checked, strict by default; drafter_ckpt.py) or a synthetic
    name. Every linear and embedding table is quantized to ``bits`` (4 by default, as the
    reference quantizes them; 8 also runs). ``shape`` overrides the synthetic builder's drafter
    knobs (num_hidden_layers, block_size, taps, markov_rank, confidence, family: gemma4 by default
    for Gemma-style targets)."""
    if bits not in (4, 8) or group_size != 64 or not quantize:
        raise ValueError("this engine runs 4- or 8-bit (group 64) drafters")
    from . import checkpoint, drafter_ckpt
    if checkpoint.is_checkpoint_dir(repo_or_path):
        if shape:
            raise ValueError(f"drafter shape overrides {sorted(shape)} apply to synthetic drafters only")
        return drafter_ckpt.load_dspark(repo_or_path, bits=bits, strict=strict, keep_mlx=keep_mlx)
    key = _synthetic_key(repo_or_path)
    if not key.startswith("dspark-"):
        raise ValueError(f"{repo_or_path!r} is not a DSpark drafter name")
    tkey = key[len("dspark-"):]
    if target_args is None:
        if tkey not in synthetic.TARGETS:
            raise ValueError(f"unknown synthetic target {tkey!r} for drafter {repo_or_path!r}")
        target_args = synthetic.target_args(tkey)
    # Gemma-family targets get the gemma4 drafter layout, as their DeepSpec drafters have
    shape.setdefault("family", "gemma4" if str(target_args.model_type).startswith("gemma") else "qwen3")
    return synthetic.build_dspark(target_args, seed=seed, keep_mlx=keep_mlx, bits=bits, **shape)


def load_pair(model: str = DEFAULT_TARGET, *, drafter=None, kv_bits=None, keep_mlx: bool = False, max_ctx=None,
              **drafter_shape):
    """(target, tokenizer, DSpark drafter, cfg) (load.py:354-363)."""
    target_name, drafter_name = resolve(model, mode="dspark", drafter=drafter)
    target, tok = load_target(target_name, require_tap=True, kv_bits=kv_bits, keep_mlx=keep_mlx, max_ctx=max_ctx)
    d, cfg = load_drafter(drafter_name, target_args=target.model.args, keep_mlx=keep_mlx, **drafter_shape)
    return target, tok, d, cfg


def load_dflash_pair(model: str = "synthetic/qwen3-8b", *, drafter=None, kv_bits=None, keep_mlx: bool = False,
                     max_ctx=None):
    """(target, tokenizer, DFlash drafter, cfg), drafter bound to the target (load.py:366-373)."""
    target_name, drafter_name = resolve(model, mode="dflash", drafter=drafter)
    target, tok = load_target(target_name, require_tap=True, kv_bits=kv_bits, keep_mlx=keep_mlx, max_ctx=max_ctx)
    d, cfg = load_dflash(drafter_name, target_args=target.model.args, keep_mlx=keep_mlx)
    d.bind(target.model)
    return target, tok, d, cfg
