"""Logit agreement for the GPU parity tests, bounded by the bf16 noise floor of the metric.

Two oracles that differ only in whether the attention probabilities are rounded to bf16 (as the
attention kernel rounds them) or kept float32 are both valid bf16 evaluations of the same
forward. How far apart they are in the RMS-normalised logit metric is the metric's noise floor for
that model, input and width: 0.046-0.050 max-abs / 0.009 rms at the Qwen3-8B and Qwen3-0.6B
widths over the full 151936-entry vocabulary (tests/test_gpu_fullwidth.py prints it), 0.02-0.04
max-abs on the narrow test models. The kernels have several such rounding choices (the RoPE
angle reduction, the exp of the softmax, bf16 split partials, the 8-bit KV quantizer on slightly
different inputs) where the floor measures one, so the GPU logits must agree with the
kernel-matching oracle within 1.5x the floor; the floor replaces the nominal 2e-2 max-abs /
3e-3 rms only where it is larger."""

from oracle import model as OM

HEADROOM = 1.5
NOMINAL_MAX, NOMINAL_RMS = 2e-2, 3e-3


def check_logits(got, want, want_alt, what=""):
    """got: GPU logits; want: the oracle with bf16 attention probabilities; want_alt: the same
    oracle with float32 probabilities (the floor's second evaluation)."""
    fmax, frms = OM.logit_diff(want, want_alt)
    mx, rms = OM.logit_diff(got, want)
    bmax, brms = HEADROOM * max(fmax, NOMINAL_MAX), HEADROOM * max(frms, NOMINAL_RMS)
    print(f"{what}: normalised max-abs {mx:.4f} rms {rms:.5f} (floor {fmax:.4f} / {frms:.5f}; "
          f"bound {bmax:.4f} / {brms:.5f})", flush=True)
    assert mx <= bmax and rms <= brms, (what, mx, rms, fmax, frms)
    return bmax
