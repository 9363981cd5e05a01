"""CPU checks of the engine's argument validation (no models are built)."""

import pytest

from mlx_dspark.engine import MODES, Engine


def test_modes_and_drafter_requirement():
    assert MODES == ("dspark", "dflash", "lookup", "baseline")
    with pytest.raises(ValueError):
        Engine(None, None, None, mode="bogus", model_id="m")
    for mode in ("dspark", "dflash"):
        with pytest.raises(ValueError):
            Engine(None, None, None, mode=mode, model_id="m")


def test_auto_cap_needs_a_controller():
    with pytest.raises(ValueError):
        Engine.load(mode="dspark", model="synthetic/tiny", max_draft_tokens="auto")
