"""Paged KV cache for the attention block (host side).

Mirrors the part of mlc-llm's PagedKVCache the reference drives
(engine.py:41-53,97-131,133-174; model/transformer.py:153-175): sequences
are added, optionally given a sliding window, extended by ``begin_forward``
with the number of tokens each one appends, and shortened by ``popn``.  The
data live on the GPU in one bf16 tensor [layers, pages, 2 (k, v), kv_heads,
16, head_dim] (mlc's per-layer page layout, stacked), pages of 16 tokens
shared by all layers of a sequence, allocated from a free list.

``begin_forward`` builds the tables the kernels read -- each sequence's page
list, its length after the append, the positions and cache slots of the
appended tokens -- and copies them into device buffers allocated once at
construction, so the forward itself allocates nothing and can be captured in
a HIP graph (the tables are inputs of the graph: refresh them with
``begin_forward`` before each replay; ``static_span`` fixes the decode
attention's split count at the pool's capacity for a captured forward, whose
empty splits return at once and merge to the same result).

Sliding window: the reference's cache keeps only the window's pages for its
"mha_sliding" layers; this cache keeps every token and the kernels attend to
the last ``window`` positions in those layers, which gives the same result
with one page table for all layers.
"""
from __future__ import annotations

import dataclasses

import torch

PAGE_SIZE = 16


@dataclasses.dataclass
class _Seq:
    length: int = 0
    pages: list = dataclasses.field(default_factory=list)
    window: int = 0


@dataclasses.dataclass
class ForwardTables:
    """Device tables of one forward (views into the cache's buffers)."""
    batch: int
    num_tokens: int
    max_q_len: int
    max_kv_len: int
    q_indptr: torch.Tensor      # [batch + 1] int32
    positions: torch.Tensor     # [num_tokens] int32
    slots: torch.Tensor         # [num_tokens] int32 (page * 16 + offset)
    page_indptr: torch.Tensor   # [batch + 1] int32
    page_indices: torch.Tensor  # [pages] int32
    kv_len: torch.Tensor        # [batch] int32
    windows: tuple              # per sequence: sliding window (0 = none)

    @property
    def is_decode(self) -> bool:
        return self.max_q_len == 1


class PagedKVCache:
    def __init__(self, num_layers: int, num_pages: int, max_batch: int, max_tokens: int,
                 kv_heads: int = 8, head_dim: int = 64, device="cuda",
                 dtype=torch.bfloat16):
        self.num_layers = num_layers
        self.num_pages = num_pages
        self.max_batch = max_batch
        self.max_tokens = max_tokens
        self.data = torch.zeros((num_layers, num_pages, 2, kv_heads, PAGE_SIZE, head_dim),
                                dtype=dtype, device=device)
        self.free = list(range(num_pages - 1, -1, -1))  # pop() hands out page 0 first
        self.seqs: dict[int, _Seq] = {}
        # The forward tables live in one device buffer at fixed offsets (kernels
        # captured in a graph keep their addresses), uploaded from a pinned
        # staging buffer of the same layout.  A forward of at most max_batch
        # tokens (every decode step) keeps its positions and slots in short
        # arrays ahead of the page indices, so its tables are one contiguous
        # range and one copy; a longer forward uses the long arrays at the end
        # (three copies, each spanning only what the forward uses).
        sizes = (max_batch + 1, max_batch + 1, max_batch, max_batch, max_batch, num_pages,
                 max_tokens, max_tokens)
        self._tables_dev = torch.zeros(sum(sizes), dtype=torch.int32, device=device)
        # two staging buffers used in turn: a forward waits only for the copy
        # made from its buffer two forwards ago (an event), not for the stream
        self._pinned = [torch.zeros(sum(sizes), dtype=torch.int32,
                                    pin_memory=torch.cuda.is_available()) for _ in range(2)]
        self._stage_events: list = [None, None]
        self._stage = 0
        self._table_offsets, views, off = [], [], 0
        for k in sizes:
            self._table_offsets.append(off)
            views.append(self._tables_dev[off:off + k])
            off += k
        (self._q_indptr, self._page_indptr, self._kv_len, self._positions_short,
         self._slots_short, self._page_indices, self._positions, self._slots) = views
        self.tables: ForwardTables | None = None
        self._decode_ws: torch.Tensor | None = None
        self._decode_ws_held: list = []
        # decode attention's key bound for a captured forward (0: per forward)
        self.static_span = 0

    def decode_workspace(self, batch: int, span: int) -> torch.Tensor:
        """The decode attention's split buffers for `batch` sequences attending
        to at most `span` keys; grown here only (``reserve_decode`` sizes it
        up front for callers that capture the forward in a graph)."""
        import attn_native
        need = attn_native.decode_workspace_bytes(batch, span)
        if self._decode_ws is None or self._decode_ws.numel() < need:
            # a buffer a captured graph holds stays alive in _decode_ws_held
            self._decode_ws = attn_native.decode_workspace(batch, span, self.data.device)
        return self._decode_ws

    def reserve_decode(self, batch: int, span: int, for_graph: bool = False) -> None:
        """Size the decode workspace now.  With ``for_graph`` the buffer is
        kept alive as long as the cache: a graph captured after this call
        holds its address, and a later, larger call gets a new buffer rather
        than freeing the captured one."""
        ws = self.decode_workspace(batch, span)
        if for_graph and all(h is not ws for h in self._decode_ws_held):
            self._decode_ws_held.append(ws)

    # -- sequences (vm.builtin.kv_state_* of engine.py:41-53) -------------------
    def layer(self, i: int) -> torch.Tensor:
        return self.data[i]

    def add_sequence(self, seq_id: int) -> None:
        if seq_id in self.seqs:
            raise ValueError(f"sequence {seq_id} exists")
        self.seqs[seq_id] = _Seq()

    def enable_sliding_window(self, seq_id: int, window: int, sink_size: int = 0) -> None:
        if sink_size:
            raise ValueError("attention sinks in the cache (sink_size > 0) are not supported; "
                             "the reference runs with 0 (engine.py:62, 120)")
        self.seqs[seq_id].window = int(window)

    def remove_sequence(self, seq_id: int) -> None:
        self.free.extend(reversed(self.seqs.pop(seq_id).pages))

    def clear(self) -> None:
        for sid in list(self.seqs):
            self.remove_sequence(sid)

    def popn(self, seq_id: int, n: int) -> None:
        s = self.seqs[seq_id]
        if not 0 <= n <= s.length:
            raise ValueError(f"popn({n}) on a sequence of {s.length} tokens")
        s.length -= n
        keep = -(-s.length // PAGE_SIZE)
        self.free.extend(reversed(s.pages[keep:]))
        del s.pages[keep:]

    def total_sequence_length(self) -> int:
        return sum(s.length for s in self.seqs.values())

    def seq_len(self, seq_id: int) -> int:
        return self.seqs[seq_id].length

    # -- one forward ---------------------------------------------------------------
    def begin_forward(self, seq_ids, append_lengths) -> ForwardTables:
        """Append ``append_lengths[i]`` tokens to sequence ``seq_ids[i]``
        (pages allocated as needed) and upload the tables of this forward."""
        seq_ids, append_lengths = list(seq_ids), [int(a) for a in append_lengths]
        batch, n = len(seq_ids), sum(append_lengths)
        if batch > self.max_batch or n > self.max_tokens:
            raise ValueError(f"forward of {batch} sequences / {n} tokens exceeds the cache's "
                             f"{self.max_batch} / {self.max_tokens}")
        if min(append_lengths, default=1) < 1:
            raise ValueError("every sequence of a forward appends at least one token")
        need = sum(max(0, -(-(self.seqs[s].length + a) // PAGE_SIZE) - len(self.seqs[s].pages))
                   for s, a in zip(seq_ids, append_lengths))
        if need > len(self.free):
            raise MemoryError(f"KV cache full: {need} pages needed, {len(self.free)} free")
        q_indptr, positions, slots, page_indptr, page_indices, kv_len = [0], [], [], [0], [], []
        for sid, a in zip(seq_ids, append_lengths):
            s = self.seqs[sid]
            while len(s.pages) * PAGE_SIZE < s.length + a:
                s.pages.append(self.free.pop())
            for p in range(s.length, s.length + a):
                positions.append(p)
                slots.append(s.pages[p // PAGE_SIZE] * PAGE_SIZE + p % PAGE_SIZE)
            s.length += a
            q_indptr.append(q_indptr[-1] + a)
            page_indices.extend(s.pages)
            page_indptr.append(len(page_indices))
            kv_len.append(s.length)
        j = self._stage
        if self._stage_events[j] is not None:
            self._stage_events[j].synchronize()  # this buffer's previous copy is done
        host, offs = self._pinned[j], self._table_offsets
        short = n <= self.max_batch
        parts = [q_indptr, page_indptr, kv_len, page_indices]
        part_offs = [offs[0], offs[1], offs[2], offs[5]]
        pos_off, slot_off = (offs[3], offs[4]) if short else (offs[6], offs[7])
        for vals, off in zip(parts + [positions, slots], part_offs + [pos_off, slot_off]):
            host[off:off + len(vals)] = torch.tensor(vals, dtype=torch.int32)
        ranges = [(0, offs[5] + len(page_indices))]
        if not short:
            ranges += [(pos_off, pos_off + n), (slot_off, slot_off + n)]
        for a, b in ranges:
            self._tables_dev[a:b].copy_(host[a:b], non_blocking=True)
        if self.data.is_cuda:
            ev = torch.cuda.Event()
            ev.record()
            self._stage_events[j] = ev
            self._stage = j ^ 1
        self.tables = ForwardTables(
            batch=batch, num_tokens=n, max_q_len=max(append_lengths),
            max_kv_len=max(kv_len), q_indptr=self._q_indptr[:batch + 1],
            positions=(self._positions_short if short else self._positions)[:n],
            slots=(self._slots_short if short else self._slots)[:n],
            page_indptr=self._page_indptr[:batch + 1],
            page_indices=self._page_indices[:max(1, len(page_indices))],
            kv_len=self._kv_len[:batch],
            windows=tuple(self.seqs[s].window for s in seq_ids))
        return self.tables

    def end_forward(self) -> None:
        self.tables = None
