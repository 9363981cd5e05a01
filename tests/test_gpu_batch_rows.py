"""GPU: ragged rows of one paged cache, against the fixtures of the reference's batch-cache tests
(tests/test_batch_engine.py).

  - after a per-row trim, each row's next write lands at its trimmed offset and overwrites what
    was there, while the positions before it keep their values (:60-71)
  - the causal + padding mask of rows at different offsets (build_batch_mask, :80-106;
    src/mlx_dspark/batch_engine.py:170-180): the reference's literal grids, as the attention
    kernels see them through per-row lengths
  - the drafter's context + block mask (_ctx_block_mask, :185-191; batch_engine.py:401-410): a row
    with no context sees its block only

Both attention kernels run: pages of 64 keys take the verify kernel (keys straight from the
pool), pages of 16 the LDS-staged kernel."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

NQ, NKV, HD = 4, 2, 128


def _cache(B, page, dev, max_ctx=64):
    from mlx_dspark.kv import PagedKVCache
    return PagedKVCache(1, B, NKV, HD, max_ctx, page=page, device=dev)


def _put(c, b, pos, k, v):
    """K/V rows [NKV, HD] at position pos of row b (bf16 pools)."""
    pg = int(c.block_table[b, pos // c.page])
    c.k[0][pg, :, pos % c.page] = k
    c.v[0][pg, :, pos % c.page] = v


def _get(c, b, pos, which):
    pg = int(c.block_table[b, pos // c.page])
    return (c.k if which == "k" else c.v)[0][pg, :, pos % c.page].float().cpu()


@pytest.mark.parametrize("page", [16, 64])
def test_next_write_after_a_trim_lands_at_the_trimmed_offset(dev, page):
    from mlx_dspark.ops import qkv_rope_append, rope_inv_freq
    print(f"trim then write page={page}", flush=True)
    g = torch.Generator().manual_seed(7)
    c = _cache(3, page, dev)
    inv = rope_inv_freq(HD, 1e6, dev)
    qn = torch.ones(HD, dtype=torch.bfloat16, device=dev)
    nh = NQ + 2 * NKV

    def append(x):
        qkv_rope_append(x.to(dev), 3, 1, NQ, NKV, HD, qn, qn, 1e-6, inv, c.seq_lens, c.block_table, c.page,
                        c.kv_dtype, c.k[0], c.v[0], c.k_sb[0], c.v_sb[0])
        torch.cuda.synchronize()

    c.set_lengths([4, 4, 4])
    for b in range(3):
        for p in range(4):
            _put(c, b, p, torch.randn(NKV, HD, generator=g).to(torch.bfloat16).to(dev),
                 torch.randn(NKV, HD, generator=g).to(torch.bfloat16).to(dev))
    x1 = torch.randn(3, nh * HD, generator=g).to(torch.bfloat16)
    append(x1)
    c.set_lengths([5, 5, 5])
    before = {(b, p): _get(c, b, p, "v") for b in range(3) for p in range(5)}
    c.trim_rows([0, 1, 2])
    assert c.lengths == [5, 4, 3]
    x2 = torch.randn(3, nh * HD, generator=g).to(torch.bfloat16)
    append(x2)
    for b, off in enumerate([5, 4, 3]):
        # the new V row (stored as given) at the trimmed offset
        assert torch.equal(_get(c, b, off, "v"), x2[b, (NQ + NKV) * HD:].view(NKV, HD).float())
        for p in range(off):                    # everything before it untouched
            assert torch.equal(_get(c, b, p, "v"), before[(b, p)])


def _attend(c, q, lens, W, causal):
    from mlx_dspark.ops import attention
    out = attention(q.to(c.k[0].device), len(lens), W, NQ, NKV, HD, HD ** -0.5, c.seq_lens, c.max_ctx,
                    c.block_table, c.page, c.kv_dtype, c.k[0], c.v[0], causal=causal)
    torch.cuda.synchronize()
    return out.view(len(lens), W, NQ, HD).float().cpu()


def _reference(c, q, lens, W, grid):
    """softmax over the keys grid[b][i] allows (grid columns are key positions of row b)."""
    B = len(lens)
    G = NQ // NKV
    ref = torch.zeros(B, W, NQ, HD)
    qf = q.view(B, W, NQ, HD).float()
    for b in range(B):
        allowed = torch.tensor(grid[b], dtype=torch.bool)          # [W, cols]
        n = allowed.shape[1]
        K = torch.stack([_get(c, b, p, "k") if p < lens[b] + W else torch.zeros(NKV, HD) for p in range(n)])
        V = torch.stack([_get(c, b, p, "v") if p < lens[b] + W else torch.zeros(NKV, HD) for p in range(n)])
        for h in range(NQ):
            s = (qf[b, :, h] @ K[:, h // G].T) * HD ** -0.5
            s = s.masked_fill(~allowed, float("-inf"))
            ref[b, :, h] = torch.softmax(s, -1) @ V[:, h // G]
    return ref


def _fill(c, lens, W, g, dev):
    for b, L in enumerate(lens):
        for p in range(L + W):
            _put(c, b, p, torch.randn(NKV, HD, generator=g).to(torch.bfloat16).to(dev),
                 torch.randn(NKV, HD, generator=g).to(torch.bfloat16).to(dev))


@pytest.mark.parametrize("page", [16, 64])
@pytest.mark.parametrize("case", ["block", "decode"])
def test_causal_mask_of_ragged_rows_is_the_reference_grid(dev, page, case):
    # build_batch_mask([2, 0], T=2) and build_batch_mask([5, 3, 0], T=1), as literal grids
    if case == "block":
        lens, W = [2, 0], 2
        grid = [[[1, 1, 1, 0], [1, 1, 1, 1]],
                [[1, 0, 0, 0], [1, 1, 0, 0]]]
    else:
        lens, W = [5, 3, 0], 1
        grid = [[[1, 1, 1, 1, 1, 1]],
                [[1, 1, 1, 1, 0, 0]],
                [[1, 0, 0, 0, 0, 0]]]
    print(f"ragged causal grid {case} page={page}", flush=True)
    g = torch.Generator().manual_seed(11 + W)
    c = _cache(len(lens), page, dev)
    _fill(c, lens, W, g, dev)
    c.set_lengths(lens)
    q = torch.randn(len(lens) * W, NQ * HD, generator=g).to(torch.bfloat16)
    got = _attend(c, q, lens, W, causal=True)
    want = _reference(c, q, lens, W, grid)
    err = (got - want).abs().max().item()
    assert err < 2e-2, err


@pytest.mark.parametrize("page", [16, 64])
def test_context_block_mask_hides_the_missing_context(dev, page):
    # _ctx_block_mask([2, 0], k=2): row 0 sees its 2 context rows and the block, row 1 (no
    # context) the block only; the block is not causal. Row 1's block sits at its positions 0, 1.
    lens, W = [2, 0], 2
    grid = [[[1, 1, 1, 1], [1, 1, 1, 1]],
            [[1, 1], [1, 1]]]
    print(f"context block mask page={page}", flush=True)
    g = torch.Generator().manual_seed(5)
    c = _cache(2, page, dev)
    _fill(c, lens, W, g, dev)
    c.set_lengths(lens)
    q = torch.randn(2 * W, NQ * HD, generator=g).to(torch.bfloat16)
    got = _attend(c, q, lens, W, causal=False)
    want = _reference(c, q, lens, W, grid)
    err = (got - want).abs().max().item()
    assert err < 2e-2, err
    # the same rows with the context hidden differ: the mask is live
    hidden = _reference(c, q, lens, W, [[[0, 0, 1, 1], [0, 0, 1, 1]], grid[1]])
    assert (got[0] - hidden[0]).abs().max().item() > 0.1
