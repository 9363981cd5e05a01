"""mlx_dspark on MI355X: the speculative-decoding verify engine of regeter/mlx-dspark,
rebuilt on hand-written gfx950 HIP kernels (libdspark_hip.so) with a PyTorch-ROCm host.

The public names mirror the reference package's exports (src/mlx_dspark/__init__.py:54-116)
for the decode path: loaders, Target, the drafters, the decode loops and GenResult."""

__version__ = "0.1.0"

from .batch_engine import SpecSlots, batch_generate_baseline, batch_spec_generate, batchable
from .config import DSparkConfig
from .dflash_model import DFlashConfig, DFlashDraftModel
from .generate import (GenResult, StopStreaming, dflash_generate, encode_messages, encode_prompt,
                       greedy_generate, speculative_generate)
from .load import (DEFAULT_DRAFTER, DEFAULT_TARGET, DFLASH_PRESETS, PRESETS, REGISTRY, apply_wired_limit,
                   load_dflash, load_dflash_pair, load_drafter, load_pair, load_target, resolve, resolve_mode)
from .lookup import NGramIndex, lookup_generate
from .model import DSparkDrafter, Gemma4DSparkDrafter
from .target import Target

__all__ = [
    "DSparkConfig", "DSparkDrafter", "Gemma4DSparkDrafter", "DFlashConfig", "DFlashDraftModel", "Target",
    "load_pair", "load_drafter", "load_dflash", "load_target", "load_dflash_pair",
    "speculative_generate", "dflash_generate", "greedy_generate", "StopStreaming", "encode_messages",
    "encode_prompt", "GenResult", "NGramIndex", "lookup_generate", "PRESETS", "DFLASH_PRESETS", "REGISTRY", "resolve", "resolve_mode",
    "apply_wired_limit", "DEFAULT_TARGET", "DEFAULT_DRAFTER", "SpecSlots", "batch_spec_generate",
    "batch_generate_baseline", "batchable",
]
