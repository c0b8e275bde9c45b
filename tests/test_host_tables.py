"""Host-side tables of the GDN scan (no GPU): the per-segment chunk table and
the packed table that puts several whole branches into one 64-token chunk."""
import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.join(os.path.dirname(__file__), "..", "cu-jev_amd"))
from cujev import ops  # noqa: E402


def test_chunk_table_cuts_segments_at_64():
    tok0, clen, seg0, segn = ops.chunk_table([1, 64, 65, 130])
    assert tok0.tolist() == [0, 1, 65, 129, 130, 194, 258]
    assert clen.tolist() == [1, 64, 64, 1, 64, 64, 2]
    assert seg0.tolist() == [0, 1, 2, 4]
    assert segn.tolist() == [1, 1, 2, 3]


def test_packed_table_fills_chunks_in_order():
    tok0, clen, starts = ops.packed_chunk_table([16] * 5)
    assert tok0.tolist() == [0, 64] and clen.tolist() == [64, 16]
    assert starts.view(np.uint64).tolist() == [1 | 1 << 16 | 1 << 32 | 1 << 48, 1]


def test_packed_table_ragged():
    lens = [1, 2, 3, 5, 16, 37, 64, 20, 20, 20, 63, 1]
    tok0, clen, starts = ops.packed_chunk_table(lens)
    # every chunk <= 64 tokens, chunks tile the tokens, segments never split
    assert (clen <= 64).all() and clen.sum() == sum(lens)
    assert (np.diff(tok0) == clen[:-1]).all() and tok0[0] == 0
    bounds = set(np.cumsum([0] + lens[:-1]).tolist())
    seen = set()
    for t0, n, m in zip(tok0.tolist(), clen.tolist(), starts.view(np.uint64).tolist()):
        assert m & 1 and m >> n == 0  # a chunk starts a segment; no bit past its tokens
        seen |= {t0 + b for b in range(n) if m >> b & 1}
    assert seen == bounds
    # greedy: a segment joins the open chunk whenever it still fits
    assert clen.tolist() == [64, 64, 60, 64]


def test_packed_table_rejects_long_segments():
    with pytest.raises(ValueError):
        ops.packed_chunk_table([10, 65])
