"""CPU restatement of greedy speculative rounds over the oracle models.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): the CPU baseline of the benchmark and the
tests run these loops; the engine never imports them.

dspark_generate follows src/mlx_dspark/generate.py:691-978 with lookup drafts off and a fixed
cap: prefill the prompt through the target with the drafter's tap layers, append the fused
states to the drafter context (model.py:253-256), then every round
  - draft the block [pending, mask x (k - 1)] and Markov-sample ``cap`` tokens
    (model.py:130-155, :270-281);
  - verify [pending] + drafts in one target forward;
  - greedy acceptance: the longest prefix of drafts equal to the target's argmax picks, plus
    the target's pick after it (generate.py:904-921);
  - roll the target KV back by the rejected rows (:928-933) and append the committed rows'
    fused states to the drafter context.
dflash_round is one greedy round of src/mlx_dspark/generate.py:468-601: the DFlash drafter
takes the context rows committed since its last call and the block [pending, mask x (bs - 1)],
its rows 1 .. cap are the drafts (argmax), then verify, accept and roll back as above.

Pinning: speculative greedy decoding reproduces plain greedy decoding token for token
whatever the drafts are (tests/test_oracle_spec.py compares both loops with
model.greedy_decode, and plants a drafter that is always right and one that is always wrong).
"""

from __future__ import annotations

import torch


def greedy_accept(target_picks, drafts) -> int:
    """Number of leading drafts equal to the target's picks at their positions."""
    n = 0
    while n < len(drafts) and int(drafts[n]) == int(target_picks[n]):
        n += 1
    return n


def _verify(target, pending: int, drafts, tap):
    vl, vf = target.forward([pending] + list(drafts), tap)
    picks = vl.argmax(dim=-1).tolist()
    n = greedy_accept(picks, drafts)
    target.trim(len(drafts) - n)
    return n, int(picks[n]), vf


def dspark_generate(target, dspark, prompt, n_new: int, cap: int, tap, mask_id: int, block_size: int):
    """(tokens, accept lengths): greedy DSpark speculative decoding of ``n_new`` tokens or more
    (a round commits all its tokens)."""
    logits, fused = target.forward(list(prompt), tap)
    dspark.update_context(fused)
    pending = int(logits[-1].argmax())
    out, accepts = [pending], []
    while len(out) < n_new:
        base = dspark.base_logits([pending] + [mask_id] * (block_size - 1), cap)
        drafts = dspark.sample_block(base, pending)
        n, token, vf = _verify(target, pending, drafts, tap)
        dspark.update_context(vf[: n + 1])
        committed = drafts[:n] + [token]
        out += committed
        accepts.append(len(committed))
        pending = token
    return out, accepts


def dflash_round(target, dflash, pending: int, new_ctx: torch.Tensor, cap: int, tap, mask_id: int,
                 block_size: int):
    """One greedy DFlash round: (n accepted, token, drafts, fused rows of the committed
    positions, which are the drafter's next context rows)."""
    logits = dflash([pending] + [mask_id] * (block_size - 1), new_ctx, logits_start=1)
    drafts = logits[:cap].argmax(dim=-1).tolist()
    n, token, vf = _verify(target, pending, drafts, tap)
    return n, token, drafts, vf[: n + 1]


def dflash_generate(target, dflash, prompt, n_new: int, cap: int, tap, mask_id: int, block_size: int):
    """(tokens, accept lengths): greedy DFlash speculative decoding of ``n_new`` tokens or more."""
    logits, ctx = target.forward(list(prompt), tap)
    pending = int(logits[-1].argmax())
    out, accepts = [pending], []
    while len(out) < n_new:
        n, token, drafts, ctx = dflash_round(target, dflash, pending, ctx, cap, tap, mask_id, block_size)
        committed = drafts[:n] + [token]
        out += committed
        accepts.append(len(committed))
        pending = token
    return out, accepts
