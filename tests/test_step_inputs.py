"""Step inputs (``tinyserve_amd.step_inputs``) on the CPU.

Mirrors the reference's tests/test_batched_forward.py:33-102, :202-212 (``build_batch``)
and tests/test_decode_inputs.py:33-77 (``fill_decode_inputs``) case by case. Tables come
from ``Tables`` below, which hands out block ids like the reference's allocator (next
free ids, optionally with gaps) and appends tokens like its ``BlockTable.append``.
"""

from __future__ import annotations

import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

from tinyserve_amd.step_inputs import DecodeInputs, PagedTable, build_batch, fill_decode_inputs


class Tables:
    """Block ids 0, 1, 2, ... in order of request (a fresh allocator's order)."""

    def __init__(self, block_size: int) -> None:
        self.block_size = block_size
        self.next = 0

    def skip(self, n: int) -> None:
        self.next += n

    def new(self) -> PagedTable:
        return PagedTable([], self.block_size, 0)

    def append(self, t: PagedTable, n: int) -> None:
        total = t.num_tokens + n
        while len(t.blocks) * self.block_size < total:
            t.blocks.append(self.next)
            self.next += 1
        t.num_tokens = total


def test_build_batch_flattens_positions_and_slots() -> None:
    tb = Tables(4)
    a, b = tb.new(), tb.new()
    tb.append(a, 3)
    tb.append(b, 5)
    tb.append(b, 1)
    batch = build_batch([([7, 8, 9], a), ([4], b)])
    assert batch.token_ids.tolist() == [7, 8, 9, 4]
    assert batch.positions.tolist() == [0, 1, 2, 5]
    assert batch.new_slots.tolist() == [a.slot(0), a.slot(1), a.slot(2), b.slot(5)]
    assert batch.seq_slots[1].tolist() == [b.slot(p) for p in range(6)]
    assert batch.query_lens == [3, 1]
    assert batch.num_seqs == 2
    assert batch.last_rows.tolist() == [2, 3]
    # The prefill kernel's view of the same batch.
    assert batch.q_starts.tolist() == [0, 3] and batch.q_lens.tolist() == [3, 1]
    assert batch.q_starts.dtype == batch.q_lens.dtype == torch.int32


@settings(max_examples=60, deadline=None)
@given(
    lens=st.lists(st.tuples(st.integers(1, 40), st.integers(1, 40)), min_size=1, max_size=5),
    block_size=st.sampled_from([1, 2, 4, 16]),
    first=st.integers(0, 50),
)
def test_slots_from_block_lists_equal_the_per_token_slots(lens: list[tuple[int, int]], block_size: int,
                                                          first: int) -> None:  # fmt: skip
    tb = Tables(block_size)
    tb.skip(first)
    items = []
    for cached, new in lens:
        t = tb.new()
        tb.append(t, cached)
        tb.skip(1)  # a gap: the next table's blocks are not contiguous with these
        tb.append(t, new)
        items.append(([1] * new, t))
    batch = build_batch(items)
    want_new = []
    for (toks, t), got in zip(items, batch.seq_slots):
        every = [t.slot(p) for p in range(t.num_tokens)]
        assert got.tolist() == every
        want_new += every[t.num_tokens - len(toks) :]
    assert batch.new_slots.tolist() == want_new
    assert batch.new_slots.dtype == torch.int64


def test_build_batch_reads_the_tables_only() -> None:
    tb = Tables(4)
    t = tb.new()
    tb.append(t, 5)
    blocks = list(t.blocks)
    build_batch([([1, 2, 3, 4, 5], t)])
    assert t.blocks == blocks and t.num_tokens == 5


def test_build_batch_rejects_bad_input() -> None:
    tb = Tables(4)
    t = tb.new()
    tb.append(t, 2)
    with pytest.raises(ValueError):
        build_batch([])
    with pytest.raises(ValueError):
        build_batch([([], t)])  # no new tokens
    with pytest.raises(ValueError):
        build_batch([([1, 2, 3], t)])  # more new tokens than the table holds


def test_build_batch_block_tables_and_lengths_for_the_kernel() -> None:
    tb = Tables(4)
    a, b = tb.new(), tb.new()
    tb.append(a, 9)
    tb.append(b, 2)
    tb.append(b, 1)
    batch = build_batch([([7] * 9, a), ([4], b)])
    assert batch.block_tables.dtype == batch.context_lens.dtype == torch.int32
    assert batch.block_tables.tolist() == [a.blocks, [*b.blocks, 0, 0]]
    assert batch.context_lens.tolist() == [9, 3]


def tables(tb: Tables, cached: list[int], new: list[int]) -> list[PagedTable]:
    out = []
    for c, n in zip(cached, new):
        t = tb.new()
        tb.append(t, c)
        tb.append(t, n)
        out.append(t)
    return out


def test_fill_writes_each_sequence_then_padding() -> None:
    a, b = tables(Tables(4), [5, 0], [1, 1])  # a: 6 tokens over 2 blocks; b: 1 token
    inp = DecodeInputs.empty(4, 3, "cpu")
    fill_decode_inputs(inp, [(7, a), (9, b)], pad_block=16)
    assert inp.token_ids.tolist() == [7, 9, 0, 0]
    assert inp.positions.tolist() == [5, 0, 0, 0]
    assert inp.slots.tolist() == [a.slot(5), b.slot(0), 64, 64]  # padding: block 16, slot 0
    assert inp.context_lens.tolist() == [6, 1, 1, 1]
    assert inp.block_tables[:, :2].tolist() == [a.blocks, [*b.blocks, 16], [16] * 2, [16] * 2]
    assert inp.block_tables[:, 2].tolist() == [0] * 4  # past the longest table: untouched
    assert inp.block_tables.dtype == inp.context_lens.dtype == torch.int32


def test_fill_overwrites_the_previous_step() -> None:
    a, b, c = tables(Tables(4), [2, 3, 4], [1, 1, 1])
    inp = DecodeInputs.empty(4, 3, "cpu")
    fill_decode_inputs(inp, [(1, a), (2, b), (3, c)], pad_block=16)
    fill_decode_inputs(inp, [(4, b)], pad_block=16)
    assert inp.token_ids.tolist() == [4, 0, 0, 0]
    assert inp.context_lens.tolist() == [4, 1, 1, 1]


def test_head_is_a_view() -> None:
    inp = DecodeInputs.empty(8, 2, "cpu")
    (a,) = tables(Tables(4), [0], [1])
    fill_decode_inputs(inp.head(2), [(5, a)], pad_block=4)
    assert inp.head(2).num_rows == 2
    assert inp.token_ids.tolist()[:2] == [5, 0]
    assert inp.slots.tolist()[1] == 16  # the padding row written through the view


def test_fill_rejects_what_does_not_fit() -> None:
    a, b = tables(Tables(4), [9, 0], [1, 1])  # a holds 3 blocks of 4
    with pytest.raises(ValueError, match="do not fit"):
        fill_decode_inputs(DecodeInputs.empty(1, 4, "cpu"), [(1, a), (2, b)], pad_block=16)
    with pytest.raises(ValueError, match="do not fit"):
        fill_decode_inputs(DecodeInputs.empty(1, 4, "cpu"), [], pad_block=16)
    with pytest.raises(ValueError, match="3 blocks"):
        fill_decode_inputs(DecodeInputs.empty(2, 2, "cpu"), [(1, a)], pad_block=16)
    with pytest.raises(ValueError, match="already be appended"):
        fill_decode_inputs(DecodeInputs.empty(2, 2, "cpu"), [(1, PagedTable([], 4, 0))], 16)


def test_paged_table_slot_matches_the_block_table_docstring() -> None:
    # block_table.py:6-12: block_size 4, blocks [7, 2].
    t = PagedTable([7, 2], 4, 8)
    assert [t.slot(p) for p in range(8)] == [28, 29, 30, 31, 8, 9, 10, 11]
    with pytest.raises(IndexError):
        t.slot(8)
