"""Per-row metadata of the paged cache under continuous batching, checked against the fixtures
the reference's batch-cache tests hold (tests/test_batch_engine.py). The reference keeps one
dense buffer per batch with per-row offsets; here every row owns a block-table row and a length,
so trims, admissions and compaction are metadata: lengths and page lists, never K/V copies.

  - per-row trim is metadata and clamps at zero (:60-77; BatchCache.trim,
    src/mlx_dspark/batch_engine.py:159-167)
  - admission into an empty slot (:139-148; BatchCache.set_row, :106-114)
  - compaction moves a row into a vacated slot (:161-167; BatchCache.move_row, :116-125): here
    the block-table rows and lengths swap, and the vacated slot's length is zero
  - a one-row view narrows every operation to its row (:170-176)

The writes that follow a trim (the next token lands at the trimmed offset) and the attention
masks of ragged rows run on the GPU in tests/test_gpu_batch_rows.py."""

import pytest

from mlx_dspark.kv import PagedKVCache


def _cache(B: int) -> PagedKVCache:
    return PagedKVCache(2, B, 2, 64, 64, page=16, device="cpu")


def test_trim_is_per_row_metadata():
    c = _cache(3)
    c.set_lengths([5, 5, 5])
    pages = [c.row_pages(b) for b in range(3)]
    c.trim_rows([0, 1, 2])                      # roll rows back by 0 / 1 / 2
    assert c.lengths == [5, 4, 3]
    assert c.seq_lens.tolist() == [5, 4, 3]
    assert [c.row_pages(b) for b in range(3)] == pages   # no page moves


def test_trim_clamps_at_zero():
    c = _cache(3)
    c.set_lengths([2, 1, 3])
    c.trim_rows([5, 0, 1])
    assert c.lengths == [0, 1, 2]
    assert c.seq_lens.tolist() == [0, 1, 2]


def test_trim_rows_needs_one_amount_per_row():
    c = _cache(3)
    c.set_lengths([2, 2, 2])
    with pytest.raises(ValueError):
        c.trim_rows([1, 1])
    with pytest.raises(ValueError):
        c.trim_rows([1, -1, 0])
    assert c.lengths == [2, 2, 2]


def test_admit_into_an_empty_slot():
    c = _cache(3)
    assert c.lengths == [0, 0, 0]
    c.set_row_length(1, 5)
    assert c.lengths == [0, 5, 0]
    assert c.seq_lens.tolist() == [0, 5, 0]


def test_compaction_moves_the_last_row_into_a_vacated_slot():
    c = _cache(3)
    c.set_lengths([3, 2, 4])
    p0, p2 = c.row_pages(0), c.row_pages(2)
    c.swap_rows(0, 2)                           # retire row 0: the last row takes its slot
    c.set_row_length(2, 0)
    assert c.lengths == [4, 2, 0]
    assert c.seq_lens.tolist() == [4, 2, 0]
    assert c.row_pages(0) == p2 and c.row_pages(2) == p0


def test_row_view_narrows_to_its_row():
    c = _cache(3)
    c.set_lengths([3, 1, 4])
    r = c.row(1)
    assert r.B == 1 and r.lengths == [1] and r.seq_lens.tolist() == [1]
    r.set_lengths([2])                          # an update through the view touches row 1 only
    assert c.lengths == [3, 2, 4]
    assert c.seq_lens.tolist() == [3, 2, 4]
    assert r.row_pages(0) == c.row_pages(1)


def test_views_of_views_write_through_to_the_root_cache():
    # a view of a view addresses the root cache's rows: lengths set, noted, swapped or set per row
    # on it land in the root's host lengths and device seq_lens alike
    c = _cache(6)
    c.set_lengths([1, 2, 3, 4, 5, 6])
    outer = c.rows(1, 5)                         # root rows 1..4
    inner = outer.rows(1, 3)                     # root rows 2..3
    assert inner.parent is c and (inner.b, inner.b1) == (2, 4)
    assert inner.lengths == [3, 4]
    inner.note_lengths([13, 14])
    assert c.lengths == [1, 2, 13, 14, 5, 6]
    inner.set_lengths([23, 24])
    assert c.lengths == [1, 2, 23, 24, 5, 6] and c.seq_lens.tolist() == [1, 2, 23, 24, 5, 6]
    pages = [c.row_pages(b) for b in range(6)]
    inner.swap_rows(0, 1)
    assert c.lengths == [1, 2, 24, 23, 5, 6] and c.seq_lens.tolist() == [1, 2, 24, 23, 5, 6]
    assert c.row_pages(2) == pages[3] and c.row_pages(3) == pages[2]
    outer.row(3).set_row_length(0, 9)            # root row 4
    assert c.lengths == [1, 2, 24, 23, 9, 6] and int(c.seq_lens[4]) == 9
    with pytest.raises(ValueError):
        outer.rows(2, 5)                         # past the outer view's 4 rows
