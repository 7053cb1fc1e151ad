"""PagedKVCache host logic on the CPU (model/kv_cache.py): page allocation,
the tables of a forward, popn, sequence removal and the errors -- the
bookkeeping of mlc-llm's PagedKVCache as the reference's engine drives it
(engine.py:41-53,109-131)."""
import pytest
import torch

from model.kv_cache import PAGE_SIZE, PagedKVCache


def make(pages=8, batch=2, tokens=64):
    return PagedKVCache(num_layers=2, num_pages=pages, max_batch=batch, max_tokens=tokens,
                        device="cpu")


def test_tables_of_a_ragged_forward():
    c = make()
    c.add_sequence(0)
    c.add_sequence(7)
    t = c.begin_forward([0, 7], [20, 3])
    assert (t.batch, t.num_tokens, t.max_q_len, t.max_kv_len) == (2, 23, 20, 20)
    assert t.q_indptr.tolist() == [0, 20, 23]
    assert t.kv_len.tolist() == [20, 3]
    assert t.page_indptr.tolist() == [0, 2, 3]
    pages0 = t.page_indices[:2].tolist()
    pages7 = t.page_indices[2:3].tolist()
    assert len(set(pages0 + pages7)) == 3
    assert t.positions.tolist() == list(range(20)) + [0, 1, 2]
    slots = t.slots.tolist()
    for i, p in enumerate(range(20)):
        assert slots[i] == pages0[p // PAGE_SIZE] * PAGE_SIZE + p % PAGE_SIZE
    assert slots[20:] == [pages7[0] * PAGE_SIZE + j for j in range(3)]
    assert not t.is_decode
    c.end_forward()
    t = c.begin_forward([7, 0], [1, 1])        # decode step: one token each
    assert t.is_decode and t.kv_len.tolist() == [4, 21]
    assert t.positions.tolist() == [3, 20]


def test_popn_frees_pages_and_positions_resume():
    c = make()
    c.add_sequence(0)
    c.begin_forward([0], [40])
    assert len(c.seqs[0].pages) == 3 and len(c.free) == 5
    c.popn(0, 10)                                # 30 tokens: still 2 pages
    assert c.seq_len(0) == 30 and len(c.seqs[0].pages) == 2 and len(c.free) == 6
    t = c.begin_forward([0], [3])
    assert t.positions.tolist() == [30, 31, 32] and t.kv_len.tolist() == [33]
    with pytest.raises(ValueError):
        c.popn(0, 34)
    c.remove_sequence(0)
    assert len(c.free) == 8 and c.total_sequence_length() == 0


def test_errors():
    c = make(pages=2, batch=1, tokens=40)
    c.add_sequence(0)
    with pytest.raises(ValueError):
        c.add_sequence(0)
    with pytest.raises(MemoryError):
        c.begin_forward([0], [33])              # 3 pages needed, 2 in the pool
    with pytest.raises(ValueError):
        c.begin_forward([0], [41])              # more tokens than the forward buffers
    with pytest.raises(ValueError):
        c.begin_forward([0], [0])
    with pytest.raises(ValueError):
        c.enable_sliding_window(0, 128, sink_size=4)
    c.enable_sliding_window(0, 128)
    t = c.begin_forward([0], [5])
    assert t.windows == (128,)
    assert c.data.shape == (2, 2, 2, 8, PAGE_SIZE, 64) and c.data.dtype == torch.bfloat16


def test_clear():
    c = make()
    for s in range(2):
        c.add_sequence(s)
    c.begin_forward([0, 1], [17, 5])
    c.clear()
    assert c.seqs == {} and sorted(c.free) == list(range(8))
