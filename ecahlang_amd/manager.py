"""AutoKVCacheManager with a device-resident page pool (ecahlang/manager.py:13-280).

Same constructor, methods, attribute names and exception messages as the reference, which
``ecahlang/main.py`` calls by name.  What changes is where the page ids live:

* The free-page stack and each sequence's page list are int32 tensors on the GPU
  (``csrc/pool.hip``).  The host keeps counts only: free pages, pages and last-page length per
  sequence, sequence slots.  So every check the reference makes (and its exceptions) happens
  on the host before anything is mutated, and every stack position is known on the host
  without reading the device.
* allocate / append_tokens / free / init_cuda_graph_buffers queue their pops and pushes;
  one ``pkv_pool_apply`` launch applies the queue, in order, before the page lists are next
  read.  The page ids are exactly the reference's: LIFO pops from the end of the free list,
  frees pushed back in page order.
* get_append_metadata / fill_cuda_graph_metadata compute ``kv_indptr`` and
  ``kv_last_page_len`` on the host in O(batch) from the counts and gather ``kv_indices`` on
  the device (``pkv_pool_gather``).  The reference's per-page Python walk and blocking H2D
  copies (manager.py:124-137, 231-253) become one asynchronous copy of O(batch) integers and
  one kernel.  Nothing here synchronises the device except the attributes that hand page ids
  back to Python (``free_blocks`` contents, ``batch_to_blocks``, ``padding_pages``), which
  ``main.py`` reads only for ``len(free_blocks)``, and the staging ring of pinned buffers
  those copies go through, which waits for a copy only when all eight of its buffers are
  still queued behind unfinished device work.

One deliberate divergence, shared with the oracle (oracle/manager_ref.py): ``allocate(T)``
with ``T % block_size == 0`` records ``block_size`` as the last page's length instead of 0
(manager.py:106).  The reference's 0 makes ``get_seq_lens`` report ``T - block_size`` while
``T`` tokens are held; ``strict_reference_q1=True`` restores it.

One extension with no counterpart in the reference (which has no page refcounting, so its
sequences cannot share pages): radix-style page sharing.  ``allocate(b, T, prefix=p)`` starts
sequence b's page list with the pages of the live sequence p that cover its first min(T,
len(p)) tokens (copied on the device, not popped; p's partial last page included, and p may
itself share pages, so prefixes nest) and pops pages for the rest.  Every page has a count of
the lists that hold it (on the host, under a handle given out at each pop): a sequence whose
tokens would go into a page others hold first takes a private copy of it (one pop; the page's
K/V copied on the device for every layer), at allocate or at append_tokens; ``free(b)``
returns, in page order, the pages only b held (a tail of its list) and drops the counts of
the rest.  The oracle restates the same rules; the graph metadata's shared-page hint for the
decode plan is computed on the device from the page lists.

A second extension, also without a counterpart (the reference frees every page of a finished
sequence and keeps no index of what pages hold, manager.py:99-120): a token-keyed prefix cache,
enabled by ``prefix_cache_rows``.  ``free(b, tokens=ids)`` keeps b's full pages in a tree keyed
by their token ids (one node per page, a path from the root per page-aligned prefix) under a
count of their own; ``allocate(b, T, tokens=ids)`` starts b with the pages of the longest
cached prefix of ids (the caller then prefills only the tokens after it); pages only the tree
holds are evicted, least recently used leaf first, when an allocation or an append is short
of free pages, or by ``evict``.  The tree lives on the host; each insert's page ids are kept
on the device in a cache row of the page table (the inserting sequence's row copied there), so
a match is one device copy from that row.  The oracle (``RefRadixKVCacheManager``) states the
rules.

The sampling helpers (init_sampling_buffers, fill_sampling_params,
fill_cuda_graph_sampling_params, ``mask_penalty``) are outside the paged-KV path; they are
kept, as plain tensor code, so that ``main.py`` finds the attributes it uses.
"""
from __future__ import annotations

import math
from typing import Iterable

import numpy as np
import torch

from ._lib import check, lib, stream_ptr
from .ops import (append_paged_kv_cache, append_paged_kv_cache_slots, get_batch_indices_positions,
                  get_seq_lens)

_POP, _PUSH, _COPY, _COW = 0, 1, 2, 3


class _CacheNode:
    """A page of the prefix cache: its block_size token ids (its key under its parent), the
    page's handle, its place on the device (cache row and column) and its last use."""
    __slots__ = ("key", "handle", "parent", "children", "last", "id", "row", "col")

    def __init__(self, key, handle, parent, nid, col):
        self.key, self.handle, self.parent, self.id, self.col = key, handle, parent, nid, col
        self.children: dict = {}
        self.last = 0
        self.row = -1


def get_total_free_memory(index: int = 0) -> int:
    """Free bytes of device ``index`` (the reference reads them through NVML, manager.py:7-11)."""
    return torch.cuda.mem_get_info(index)[0]


class _Staging:
    """Host -> device copies of int32 arrays through a ring of reused pinned buffers, queued on
    the current stream.  ``host(n)`` hands out the next buffer once the event recorded behind
    its last copy has completed (so a queued copy never sees its source change); ``send`` queues
    the copy and records the buffer's event.  Arrays beyond the ring's capacity go through a
    fresh pinned buffer instead, which the caching host allocator keeps until its copy has run.
    Nothing is staged while the stream is being captured: a pinned allocation is not allowed
    then, and a recorded copy would read its buffer again at every replay, so ``host`` raises
    before anything is enqueued (the callers fill their metadata before capture, as the
    reference's loop does, or use the device-resident steps)."""

    def __init__(self, device: torch.device, slots: int = 8, cap: int = 1 << 15):
        self.device, self.cap = device, cap
        self.bufs = [torch.empty(cap, dtype=torch.int32, pin_memory=True) for _ in range(slots)]
        self.views = [b.numpy() for b in self.bufs]
        self.events = [torch.cuda.Event() for _ in range(slots)]
        self.used = [False] * slots
        self.i = 0

    def host(self, n: int) -> tuple:
        """(slot, int32 array of n to fill); slot -1 means the array is not a ring buffer."""
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("page-pool metadata is staged from host arrays and cannot be recorded into a "
                               "graph: fill it before capture (fill_cuda_graph_metadata) or capture the "
                               "device-resident step (begin_device_steps / device_step)")
        if n > self.cap:
            return -1, np.empty(n, dtype=np.int32)
        i = self.i
        self.i = (i + 1) % len(self.bufs)
        if self.used[i]:
            self.events[i].synchronize()
        return i, self.views[i][:n]

    def send(self, slot: int, arr: np.ndarray, dst: torch.Tensor | None = None) -> torch.Tensor:
        """Queue ``arr`` (from ``host``) into ``dst[:len(arr)]``, a new device tensor when
        ``dst`` is None."""
        n = len(arr)
        src = self.bufs[slot][:n] if slot >= 0 else torch.from_numpy(arr).pin_memory()
        if dst is None:
            dst = torch.empty(n, dtype=torch.int32, device=self.device)
        dst[:n].copy_(src, non_blocking=True)
        if slot >= 0:
            self.events[slot].record(torch.cuda.current_stream(self.device))
            self.used[slot] = True
        return dst

    def copy(self, values: list, dst: torch.Tensor | None = None) -> torch.Tensor:
        slot, arr = self.host(len(values))
        arr[:] = values
        return self.send(slot, arr, dst)


class _FreeBlocks:
    """``manager.free_blocks``: its length is known on the host; its contents (the free-page
    stack, bottom to top) are read from the device on demand."""

    __slots__ = ("_m",)

    def __init__(self, m: "AutoKVCacheManager"):
        self._m = m

    def __len__(self) -> int:
        return self._m._n_free

    def tolist(self) -> list:
        m = self._m
        m._flush()
        return m._stack[: m._n_free].tolist()

    def __iter__(self):
        return iter(self.tolist())

    def __getitem__(self, i):
        return self.tolist()[i]

    def __eq__(self, other):
        return self.tolist() == list(other)

    def __repr__(self) -> str:
        return repr(self.tolist())


class _Pages:
    """The page list ``allocate`` returns, read from the device on first use (the pages the
    sequence held when it was allocated)."""

    __slots__ = ("_m", "_row", "_n", "_list")

    def __init__(self, m: "AutoKVCacheManager", row: int, n: int):
        self._m, self._row, self._n, self._list = m, row, n, None

    def tolist(self) -> list:
        if self._list is None:
            self._m._flush()
            self._list = self._m._table[self._row, : self._n].tolist() if self._n else []
        return self._list

    def __len__(self) -> int:
        return self._n

    def __iter__(self):
        return iter(self.tolist())

    def __getitem__(self, i):
        return self.tolist()[i]

    def __eq__(self, other):
        return self.tolist() == list(other)

    def __repr__(self) -> str:
        return repr(self.tolist())


class AutoKVCacheManager:
    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, vocab_size: int = 10000,
                 seq_lens: int = 128, block_size: int = 16, dtype: torch.dtype = torch.float16,
                 layout: str = "NHD", total_gpu_mem_bytes: int | None = None,
                 mem_utilization: float = 0.9, *, device=None, max_pages_per_seq: int = 512,
                 strict_reference_q1: bool = False, prefix_cache_rows: int = 0):
        """manager.py:14-72.  Extensions (keyword-only): ``device`` (default: the current
        CUDA device), ``max_pages_per_seq`` (initial width of the per-sequence page table; it
        grows on demand), ``strict_reference_q1`` (see the module docstring) and
        ``prefix_cache_rows`` (0: no prefix cache; otherwise how many inserts the cache keeps
        at once, each in a row of the page table)."""
        if layout.upper() != "NHD":
            raise NotImplementedError("only the NHD cache layout is implemented (the reference uses NHD)")
        self.device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        if self.device.type != "cuda":
            raise ValueError("the page pool lives on a CUDA (HIP) device")
        lib()  # no fallback: a missing library fails here, not at the first step
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.vocab_size = vocab_size
        self.seq_lens = max(seq_lens, 128)
        self.block_size = block_size
        self.dtype = dtype
        self.layout = layout.upper()
        self.dtype_size = torch.tensor([], dtype=dtype).element_size()
        self.strict_reference_q1 = strict_reference_q1
        if prefix_cache_rows < 0 or (prefix_cache_rows and strict_reference_q1):
            raise ValueError("prefix_cache_rows must be >= 0, and the prefix cache needs full last pages "
                             "(strict_reference_q1=False)")
        self._mask_resets: list = []  # slots whose mask_penalty row allocate set back to 1
        self.mask_penalty = torch.ones(self.seq_lens, vocab_size, dtype=dtype, device=self.device)

        if total_gpu_mem_bytes is None:
            total_gpu_mem_bytes = get_total_free_memory(self.device.index or 0)
        usable_mem = int(total_gpu_mem_bytes * mem_utilization)
        per_token_bytes = num_kv_heads * head_dim * self.dtype_size * 2
        per_block_per_layer = block_size * per_token_bytes
        self.max_blocks = usable_mem // (num_layers * per_block_per_layer)
        self.kv_cache = torch.zeros((num_layers, self.max_blocks, 2, block_size, num_kv_heads, head_dim),
                                    dtype=dtype, device=self.device)

        # device pool: free-page stack (bottom = page 0) and one page-list row per sequence
        # slot, then a row for the CUDA-graph padding pages, then the prefix cache's rows
        self._stack = torch.arange(self.max_blocks, dtype=torch.int32, device=self.device)
        self._n_free = self.max_blocks
        self._pad_row = self.seq_lens
        self._rows = self.seq_lens + 1 + prefix_cache_rows
        self._stride = max(1, min(max(self.max_blocks, 1), max_pages_per_seq))
        self._table = torch.full((self._rows, self._stride), -1, dtype=torch.int32, device=self.device)
        self._err = torch.zeros(1, dtype=torch.int32, device=self.device)
        # device-resident decode steps (begin_device_steps): each slot's page count and
        # last-page length, and the free-stack size, as the device advances them
        self._dev_npages = torch.zeros(self._rows, dtype=torch.int32, device=self.device)
        self._dev_plen = torch.zeros(self._rows, dtype=torch.int32, device=self.device)
        self._dev_nfree = torch.zeros(1, dtype=torch.int32, device=self.device)
        self._dev = None  # the batch handed to the device, or None
        self._staging = _Staging(self.device)
        self._ops: list = []
        self._n_padding = 0
        # page sharing (an extension): each page in a list has a host-side handle (one per pop)
        # and a count of the lists that hold it; the page ids themselves stay on the device
        self._pg: dict = {}      # batch_id -> handles of its pages, in page order
        self._rc: dict = {}      # handle -> lists holding that page
        self._next_handle = 0
        self._n_multi = 0        # handles held by more than one list
        self._n_cow = 0          # copies on write queued since the last flush
        self._cow_cap = 1024
        self._pairs = torch.zeros(2 * self._cow_cap, dtype=torch.int32, device=self.device)
        # prefix cache (an extension): the tree on the host, each insert's pages in a cache row
        self._cache_rows = prefix_cache_rows
        self._root = _CacheNode(None, None, None, -1, -1)
        self._nodes: dict = {}   # id -> node
        self._clock = 0
        self._next_node = 0
        self._free_crows = list(range(prefix_cache_rows))  # handed out from the end
        self._crow_nodes: dict = {}  # cache row -> nodes homed there

        # host bookkeeping: counts only
        self.free_seq_lens = list(range(self.seq_lens))
        self._npages: dict = {}
        self.batch_to_page_lengths: dict = {}
        self.batch_to_total_tokens: dict = {}
        self.batch_to_seq_len: dict = {}
        self.prefill_layer_idx = 0
        self.decode_layer_idx = 0

        self.cuda_graph_mode = False
        self._cg_kv_indices: dict = {}
        self._cg_kv_indptr: dict = {}
        self._cg_kv_last_page_len: dict = {}
        self._cg_batch_indices: dict = {}
        self._cg_positions: dict = {}
        self._cg_append_indptr: dict = {}
        self._cg_meta: dict = {}  # bucket -> [desc | indptr | last_page_len | positions] (the three are views)
        self._cg_slots: dict = {}  # bucket -> each row's append slot, page * block_size + position % block_size
        # bucket -> for each row, the leading pages it shares with the row before it (the
        # decode plan's kv_shared_pages)
        self._cg_kv_shared: dict = {}
        self._cg_rows: dict = {}   # bucket -> table row of each batch entry (-1: padding), device steps
        self._cg_desc: dict = {}   # bucket -> gather descriptor scratch of the device step
        # The pool's initial state (free stack, page table, cache) is written on the current
        # stream; a caller may go on to drive the pool from another stream, so it is complete
        # before the constructor returns.
        torch.cuda.current_stream(self.device).synchronize()

    # ------------------------------------------------------------------ device pool plumbing

    def _ensure_stride(self, need: int) -> None:
        self._end_dev()
        if need <= self._stride:
            return
        new = max(need, 2 * self._stride)
        table = torch.full((self._rows, new), -1, dtype=torch.int32, device=self.device)
        table[:, : self._stride].copy_(self._table)
        self._table, self._stride = table, new

    @property
    def mask_penalty(self) -> torch.Tensor:
        """manager.py:56: one row per sequence slot, set back to 1 by ``allocate``.  The resets
        of a batch of allocations are applied together (one launch), at the next pool flush
        or read of this attribute, on the current stream."""
        if self._mask_resets:
            self._reset_mask_rows(self._staging.copy(self._reset_words()), 0)
        return self._mask_penalty

    @mask_penalty.setter
    def mask_penalty(self, value: torch.Tensor) -> None:
        if self._mask_resets:
            self._reset_mask_rows(self._staging.copy(self._reset_words()), 0)
        self._mask_penalty = value

    def _reset_words(self) -> list:
        """The pending reset slots as int32 word pairs (little-endian int64 indices)."""
        return [w for r in self._mask_resets for w in (r, 0)]

    def _reset_mask_rows(self, staged: torch.Tensor, off: int) -> None:
        idx = staged[off: off + 2 * len(self._mask_resets)].view(torch.int64)
        self._mask_resets = []
        self._mask_penalty.index_fill_(0, idx, 1.0)

    def _flush(self) -> None:
        """Apply the queued pops, pushes and copies (one launch, with the effect of applying
        them in order, on the current stream) and the queued mask_penalty resets, from one
        staged copy; then copy the K/V data of the queued copies on write."""
        self._end_dev()
        if not self._ops and not self._mask_resets:
            return
        flat = [x for op in self._ops for x in op]
        off = len(flat) + len(flat) % 2  # (the resets' int64 words start 8-byte aligned)
        if self._mask_resets:
            flat += [0] * (off - len(flat)) + self._reset_words()
        ops = self._staging.copy(flat)
        if self._ops:
            check(lib().pkv_pool_apply(self._stack.data_ptr(), self.max_blocks, self._table.data_ptr(),
                                       self._stride, self._rows, ops.data_ptr(), len(self._ops),
                                       self._pairs.data_ptr(), self._cow_cap, self._err.data_ptr(),
                                       stream_ptr(self.device)), "page pool update")
        if self._mask_resets:
            self._reset_mask_rows(ops, off)
        self._ops = []
        if self._n_cow:
            c = self.kv_cache
            check(lib().pkv_pool_copy_pages(c.data_ptr(), c.stride(0) * c.element_size(), c.shape[0],
                                            c.stride(1) * c.element_size(), self._pairs.data_ptr(), self._n_cow,
                                            self.max_blocks, self._err.data_ptr(), stream_ptr(self.device)),
                  "page copy")
            self._n_cow = 0

    # ------------------------------------------------------------------ page handles (sharing)

    def _new_handles(self, n: int) -> list:
        h = list(range(self._next_handle, self._next_handle + n))
        self._next_handle += n
        for x in h:
            self._rc[x] = 1
        return h

    def _hold(self, handles) -> None:
        for x in handles:
            self._rc[x] += 1
            if self._rc[x] == 2:
                self._n_multi += 1

    def _drop(self, x) -> None:
        self._rc[x] -= 1
        if self._rc[x] == 1:
            self._n_multi -= 1
        elif self._rc[x] == 0:
            del self._rc[x]

    def _shares_last_page(self, batch_id) -> bool:
        """Whether new tokens of batch_id would go into a page other lists hold."""
        h = self._pg.get(batch_id)
        return bool(h) and self._rc[h[-1]] > 1 and self.batch_to_page_lengths[batch_id] < self.block_size

    def _queue_cow(self, batch_id) -> None:
        """Replace batch_id's (shared) last page by a private copy: one pop from the top of the
        stack; the page's K/V is copied for every layer when the queue is applied."""
        if self._n_cow == self._cow_cap:
            self._flush()
        h = self._pg[batch_id]
        self._ops.append((_COW, self.batch_to_seq_len[batch_id], self._n_free, len(h) - 1, self._n_cow))
        self._n_cow += 1
        self._n_free -= 1
        self._drop(h[-1])
        h[-1] = self._new_handles(1)[0]

    def _stage_tables(self, ids: list, bucket: int = 0, positions: bool = False) -> tuple:
        """The gather's input for the sequences ``ids`` followed by ``bucket - len(ids)``
        padding rows (one padding page each, last_page_len 1, position 0), staged in one host
        array: [desc (4 per row) | kv_indptr (rows + 1) | kv_last_page_len (rows)] plus
        [positions (rows) | shared (rows)] (each row's newest token, and how many leading pages
        it shares with the row before it) when asked.  Returns (slot, array, rows, pages)."""
        self._end_dev()
        r = len(ids)
        b = max(bucket, r)
        if b - r > self._n_padding:
            raise IndexError("list index out of range")
        slots = np.fromiter(map(self.batch_to_seq_len.__getitem__, ids), np.int32, r)
        npages = np.fromiter(map(self._npages.__getitem__, ids), np.int32, r)
        plen = np.fromiter(map(self.batch_to_page_lengths.__getitem__, ids), np.int32, r)
        slot, out = self._staging.host((8 if positions else 6) * b + 1)
        desc = out[: 4 * b].reshape(b, 4)
        desc[:r, 0] = slots
        desc[r:, 0] = self._pad_row
        desc[:r, 1] = 0
        desc[r:, 1] = np.arange(b - r, dtype=np.int32)
        desc[:r, 2] = npages
        desc[r:, 2] = 1
        desc[:, 3] = 0
        indptr = out[4 * b: 5 * b + 1]
        indptr[0] = 0
        np.cumsum(desc[:, 2], out=indptr[1:])
        last = out[5 * b + 1: 6 * b + 1]
        last[:r] = plen
        last[r:] = 1
        if positions:
            pos = out[6 * b + 1: 7 * b + 1]
            np.multiply(npages - 1, self.block_size, out=pos[:r])
            pos[:r] += plen - 1
            pos[r:] = 0
            shared = out[7 * b + 1: 8 * b + 1]
            shared[:] = 0  # (filled on the device from the gathered lists when pages are shared)
        return slot, out, b, int(indptr[-1])

    def _gather(self, slot: int, staged: np.ndarray, b: int, pages: int, out_indices: torch.Tensor,
                dst: torch.Tensor | None = None, slots: torch.Tensor | None = None) -> torch.Tensor:
        """Copy the staged [desc | indptr | extra] to the device (into ``dst`` when given) and
        gather out_indices[indptr[r] + k] = table[desc...]; returns the device [indptr | extra].
        With ``slots``, extra is [last_page_len | positions] and each row's append slot
        (page * block_size + position % block_size) is written there too."""
        self._flush()
        dev = self._staging.send(slot, staged, dst)
        d_desc, d_rest = dev[: 4 * b], dev[4 * b:]
        if pages or slots is not None:
            pos_ptr, slots_ptr = 0, 0
            if slots is not None:
                pos_ptr = d_rest[2 * b + 1:].data_ptr()
                slots_ptr = slots.data_ptr()
            check(lib().pkv_pool_gather(self._table.data_ptr(), self._stride, self._rows, d_desc.data_ptr(),
                                        d_rest.data_ptr(), b, out_indices.data_ptr(), out_indices.numel(),
                                        pages, pos_ptr, self.block_size, slots_ptr, self._err.data_ptr(),
                                        stream_ptr(self.device)),
                  "page table gather")
        return d_rest

    def pool_errors(self) -> int:
        """Operations or gathers the device had to skip (0 unless the host bookkeeping and the
        device pool disagree); reading it synchronises."""
        return int(self._err.item())

    # ------------------------------------------------------------------ reference attributes

    @property
    def free_blocks(self) -> _FreeBlocks:
        return _FreeBlocks(self)

    @property
    def batch_to_blocks(self) -> dict:
        """Page lists by sequence, read back from the device (synchronises)."""
        self._flush()
        if not self._npages:
            return {}
        rows = self._table.cpu()
        return {b: rows[self.batch_to_seq_len[b], :n].tolist() for b, n in self._npages.items()}

    @property
    def padding_pages(self) -> list:
        self._flush()
        return self._table[self._pad_row, : self._n_padding].tolist() if self._n_padding else []

    # ------------------------------------------------------------------ page pool (A3-A5)

    def _counts(self, batch_id) -> tuple:
        """(pages, last-page length) of a sequence, also while the device runs its steps."""
        d = self._dev
        if d is not None and batch_id in d["at"]:
            i = d["at"][batch_id]
            return self._advanced(d["npages0"][i], d["plen0"][i], d["k"] * d["n"])
        return self._npages[batch_id], self.batch_to_page_lengths[batch_id]

    def _advanced(self, npages: int, last: int, tokens: int) -> tuple:
        """(pages, last-page length) after appending `tokens` tokens one step at a time, each
        step as append_tokens does it: t = last + n, pop t // block_size, keep t % block_size.
        With last <= block_size that is (last + tokens) // block_size pops in all (the last
        page may start full: allocate's last_page_len of block_size)."""
        if tokens == 0:
            return npages, last
        t = last + tokens
        return npages + t // self.block_size, t % self.block_size

    def _seq_len(self, batch_id) -> int:
        n, last = self._counts(batch_id)
        return (n - 1) * self.block_size + last if n else 0

    def allocate(self, batch_id, total_tokens: int, *, prefix=None, tokens=None) -> _Pages:
        """manager.py:99-112: pop ceil(T / block_size) pages, take a sequence slot.  With
        ``prefix`` (an extension), the pages of that live sequence covering the first
        min(T, len(prefix)) tokens come first (a partial last page included; copied, if this
        sequence's tokens continue into it) and only the rest are popped.  With ``tokens``
        (the prefix cache, an extension: the sequence's token ids), the cached pages of the
        longest page-aligned prefix of tokens[:T] come first; ``match_prefix`` tells how many
        tokens that is beforehand.  With the prefix cache, pages only the cache holds are
        evicted first when the free pages are too few."""
        self._end_dev()
        bs = self.block_size
        k, cow, path = 0, False, []
        if prefix is not None:
            if prefix not in self._npages:
                raise ValueError(f"{prefix} not allocated")
            if tokens is not None:
                raise ValueError("prefix and tokens are exclusive")
            ts = min(total_tokens, self._seq_len(prefix))
            k = math.ceil(ts / bs)
            cow = total_tokens > ts and ts % bs != 0
        elif tokens is not None:
            if not self._cache_rows:
                raise ValueError("allocate(tokens=) needs the prefix cache (prefix_cache_rows > 0)")
            self._clock += 1
            path = self._match(tokens, total_tokens)
            k = len(path)
        num_pages = math.ceil(total_tokens / bs) - k
        if self._n_free < num_pages + cow and self._cache_rows:
            self.evict(num_pages + cow - self._n_free, _protect=set(path))
        if self._n_free < num_pages + cow:
            raise RuntimeError("Not enough KV cache blocks available")
        if not self.free_seq_lens:
            raise IndexError("pop from empty list")
        slot = self.free_seq_lens.pop()
        self._ensure_stride(k + num_pages)
        handles = []
        if path:
            handles = [n.handle for n in path]
            self._hold(handles)
            for n in path:
                n.last = self._clock
            # the deepest node's cache row holds the whole path from column 0
            self._ops.append((_COPY, slot, path[-1].row, 0, k))
        elif k:
            handles = self._pg[prefix][:k]
            self._hold(handles)
            self._ops.append((_COPY, slot, self.batch_to_seq_len[prefix], 0, k))
        self._pg[batch_id] = handles
        self.batch_to_seq_len[batch_id] = slot
        if cow:
            self.batch_to_page_lengths[batch_id] = 0  # (read by nothing before it is set below)
            self._queue_cow(batch_id)
        if num_pages:
            self._ops.append((_POP, slot, self._n_free, k, num_pages))
            self._n_free -= num_pages
            handles += self._new_handles(num_pages)
        self._npages[batch_id] = k + num_pages
        page_len = total_tokens % bs
        if page_len == 0 and total_tokens > 0 and not self.strict_reference_q1:
            page_len = bs
        self.batch_to_page_lengths[batch_id] = page_len
        self.batch_to_total_tokens[batch_id] = total_tokens
        self._mask_resets.append(slot)  # (mask_penalty[slot] = 1: applied with the next flush or read)
        return _Pages(self, slot, k + num_pages)

    def free(self, batch_id, *, tokens=None) -> None:
        """manager.py:114-120: push the pages back in page order, release the slot.  With
        shared pages (an extension), only the pages no other list holds go back: always a tail
        of the list, since a list holding one of this sequence's pages holds all before it.
        With ``tokens`` (the prefix cache, an extension: the sequence's token ids), its full
        pages are first kept in the cache (see ``_insert``)."""
        self._end_dev()
        if tokens is not None:
            if not self._cache_rows:
                raise ValueError("free(tokens=) needs the prefix cache (prefix_cache_rows > 0)")
            if batch_id in self._npages:
                self._insert(batch_id, tokens)
        handles = self._pg.pop(batch_id, [])
        n = self._npages.pop(batch_id, 0)
        self.batch_to_page_lengths.pop(batch_id, None)
        slot = self.batch_to_seq_len.pop(batch_id, None)
        t = len(handles)
        while t > 0 and self._rc[handles[t - 1]] == 1:
            t -= 1
        if any(self._rc[x] == 1 for x in handles[:t]):
            raise RuntimeError("page sharing bookkeeping is inconsistent")
        for x in handles:
            self._drop(x)
        if n > t and slot is not None:
            self._ops.append((_PUSH, slot, self._n_free, t, n - t))
            self._n_free += n - t
        if slot is not None:
            self.free_seq_lens.append(slot)

    def append_tokens(self, batch_id, num_new_tokens: int) -> None:
        """manager.py:187-205: a page is popped as soon as the last one fills (an empty
        trailing page with last_page_len 0 is kept, as the reference does).  New tokens that
        would go into a page other sequences hold (an extension) first get a private copy of it."""
        self._end_dev()
        if batch_id not in self._npages:
            raise ValueError(f"{batch_id} not allocated")
        current_len = self.batch_to_page_lengths.get(batch_id, 0)
        total_tokens = current_len + num_new_tokens
        full_new_pages = total_tokens // self.block_size
        remaining = total_tokens % self.block_size
        cow = num_new_tokens > 0 and self._shares_last_page(batch_id)
        if full_new_pages + cow > self._n_free and self._cache_rows:
            self.evict(full_new_pages + cow - self._n_free)
        if full_new_pages + cow > self._n_free:
            raise RuntimeError("Not enough free blocks to append tokens")
        if cow:
            self._queue_cow(batch_id)
        if full_new_pages:
            col = self._npages[batch_id]
            self._ensure_stride(col + full_new_pages)
            self._ops.append((_POP, self.batch_to_seq_len[batch_id], self._n_free, col, full_new_pages))
            self._n_free -= full_new_pages
            self._npages[batch_id] = col + full_new_pages
            self._pg[batch_id] += self._new_handles(full_new_pages)
        self.batch_to_page_lengths[batch_id] = remaining

    # ------------------------------------------------------------------ prefix cache (extension)

    def _keys(self, tokens, limit: int) -> list:
        bs = self.block_size
        n = min(len(tokens), limit) // bs
        return [tuple(int(t) for t in tokens[i * bs:(i + 1) * bs]) for i in range(n)]

    def _match(self, tokens, limit: int) -> list:
        path, node = [], self._root
        for key in self._keys(tokens, limit):
            node = node.children.get(key)
            if node is None:
                break
            path.append(node)
        return path

    def match_prefix(self, tokens) -> int:
        """How many leading tokens of ``tokens`` the prefix cache holds (whole pages); what
        ``allocate(..., tokens=tokens)`` would start the sequence with.  Touches nothing."""
        if not self._cache_rows:
            return 0
        return len(self._match(tokens, len(tokens))) * self.block_size

    @property
    def prefix_cache_pages(self) -> int:
        """Pages the prefix cache holds (whether or not live sequences hold them too)."""
        return len(self._nodes)

    def _insert(self, batch_id, tokens) -> None:
        """Keep batch_id's full pages (those whose tokens ``tokens`` gives) in the cache.
        Walking from the root, a block cached with this sequence's own page is followed, a
        block cached with another page ends the walk, and the blocks after the last one
        followed become new nodes holding this sequence's pages, all homed in one cache row:
        the sequence's row up to the last new node copied there (it holds the whole path).
        With no cache row free, least recently used pages are evicted until one is; if none
        is, nothing is inserted."""
        self._clock += 1
        handles = self._pg[batch_id]
        node, created = self._root, []
        for i, key in enumerate(self._keys(tokens, self._seq_len(batch_id))):
            child = node.children.get(key) if not created else None
            if child is not None:
                if child.handle != handles[i]:
                    break
                child.last = self._clock
                node = child
                continue
            new = _CacheNode(key, handles[i], node, self._next_node, i)
            self._next_node += 1
            created.append(new)
            node = new
        if not created:
            return
        while not self._free_crows and self._evict_one(()):
            pass
        if not self._free_crows:
            return
        r = self._free_crows.pop()
        row = self._pad_row + 1 + r
        self._crow_nodes[row] = len(created)
        for n in created:
            n.parent.children[n.key] = n
            n.row, n.last = row, self._clock
            self._nodes[n.id] = n
        self._hold([n.handle for n in created])
        self._ops.append((_COPY, row, self.batch_to_seq_len[batch_id], 0, created[-1].col + 1))

    def _evict_one(self, protect) -> bool:
        best = None
        for n in self._nodes.values():
            if n.children or self._rc[n.handle] != 1 or n in protect:
                continue
            if best is None or (n.last, n.id) < (best.last, best.id):
                best = n
        if best is None:
            return False
        del best.parent.children[best.key]
        del self._nodes[best.id]
        self._drop(best.handle)
        self._ops.append((_PUSH, best.row, self._n_free, best.col, 1))
        self._n_free += 1
        self._crow_nodes[best.row] -= 1
        if self._crow_nodes[best.row] == 0:
            del self._crow_nodes[best.row]
            self._free_crows.append(best.row - self._pad_row - 1)
        return True

    def evict(self, n: int, *, _protect=()) -> int:
        """Return up to ``n`` pages that only the prefix cache holds to the free stack, least
        recently used first (a page is evictable once no sequence and no longer cached prefix
        holds it); returns how many."""
        self._end_dev()
        k = 0
        while k < n and self._evict_one(_protect):
            k += 1
        return k

    def cached_prefixes(self) -> dict:
        """page id -> the token ids of the cached prefix ending with that page (reads the
        device; for checks)."""
        self._flush()
        out = {}
        for nd in self._nodes.values():
            keys, m = [], nd
            while m is not self._root:
                keys.append(m.key)
                m = m.parent
            page = int(self._table[nd.row, nd.col].item())
            out[page] = [t for k in reversed(keys) for t in k]
        return out

    # ------------------------------------------------------------------ page tables (A6-A9)

    def get_append_metadata(self, batch_ids: Iterable) -> tuple:
        """manager.py:122-138: (kv_indices, kv_indptr, kv_last_page_len), int32 on the device."""
        batch_ids = list(batch_ids)
        self._flush()  # (the staging ring hands out buffers in order)
        slot, staged, b, pages = self._stage_tables(batch_ids)
        kv_indices = torch.empty(pages, dtype=torch.int32, device=self.device)
        rest = self._gather(slot, staged, b, pages, kv_indices)
        return kv_indices, rest[: b + 1], rest[b + 1: 2 * b + 1]

    def prepare_append_metadata(self, batch_ids, append_indptr: torch.Tensor, nnz=None) -> None:
        """manager.py:140-151: the page table, seq_lens, and each appended token's sequence
        and position, cached for every layer of the step.  ``nnz`` (an extension) is the
        number of appended tokens; without it ``append_indptr[-1]`` is read back, a device
        synchronisation, as in the reference."""
        kv_indices, kv_indptr, kv_last_page_len = self.get_append_metadata(batch_ids)
        seq_lens = get_seq_lens(kv_indptr, kv_last_page_len, self.block_size)
        batch_indices, positions = get_batch_indices_positions(
            append_indptr, seq_lens, append_indptr[-1] if nnz is None else nnz)
        self._cached_kv_indices = kv_indices
        self._cached_kv_indptr = kv_indptr
        self._cached_kv_last_page_len = kv_last_page_len
        self._cached_batch_indices = batch_indices
        self._cached_positions = positions

    def append_paged_kv_cache_cached(self, key, value, layer_idx: int) -> None:
        """manager.py:153-165."""
        append_paged_kv_cache(append_key=key, append_value=value,
                              batch_indices=self._cached_batch_indices, positions=self._cached_positions,
                              paged_kv_cache=self.kv_cache[layer_idx], kv_indices=self._cached_kv_indices,
                              kv_indptr=self._cached_kv_indptr,
                              kv_last_page_len=self._cached_kv_last_page_len, kv_layout=self.layout)

    def append_paged_kv_cache(self, batch_ids, key, value, append_indptr, layer_idx: int, nnz=None) -> None:
        """manager.py:167-185 (the uncached variant)."""
        kv_indices, kv_indptr, kv_last_page_len = self.get_append_metadata(batch_ids)
        seq_lens = get_seq_lens(kv_indptr, kv_last_page_len, self.block_size)
        batch_indices, positions = get_batch_indices_positions(
            append_indptr, seq_lens, append_indptr[-1] if nnz is None else nnz)
        append_paged_kv_cache(append_key=key, append_value=value, batch_indices=batch_indices,
                              positions=positions, paged_kv_cache=self.kv_cache[layer_idx],
                              kv_indices=kv_indices, kv_indptr=kv_indptr,
                              kv_last_page_len=kv_last_page_len, kv_layout=self.layout)

    # ------------------------------------------------------------------ CUDA-graph buckets (A10-A12)

    def init_cuda_graph_buffers(self, bucket_sizes, *, max_indices: int | None = None) -> None:
        """manager.py:207-226: reserve max(bucket) padding pages and the static per-bucket
        buffers the captured step reads.  ``max_indices`` (an extension) sizes the static
        ``kv_indices`` buffers; the reference's ``max_blocks`` is too small once sequences
        share prefix pages (a shared page appears in every table that holds it)."""
        self._end_dev()
        max_bucket = max(bucket_sizes)
        if self._n_free < max_bucket:
            raise RuntimeError(f"Not enough free blocks for {max_bucket} padding pages")
        self._ensure_stride(max_bucket)
        self._ops.append((_POP, self._pad_row, self._n_free, 0, max_bucket))
        self._n_free -= max_bucket
        self._n_padding = max_bucket
        dev = self.device
        self._cg_temperature, self._cg_top_k, self._cg_top_p = {}, {}, {}
        for bs in bucket_sizes:
            self._cg_kv_indices[bs] = torch.zeros(max(self.max_blocks, max_indices or 0), dtype=torch.int32,
                                                  device=dev)
            # indptr, last_page_len, positions and the shared-prefix hint are views of one block
            # laid out as the metadata build stages them, so one host copy fills all four
            meta = torch.zeros(8 * bs + 1, dtype=torch.int32, device=dev)
            self._cg_meta[bs] = meta
            self._cg_kv_indptr[bs] = meta[4 * bs: 5 * bs + 1]
            self._cg_kv_last_page_len[bs] = meta[5 * bs + 1: 6 * bs + 1]
            self._cg_batch_indices[bs] = torch.arange(bs, dtype=torch.int32, device=dev)
            self._cg_positions[bs] = meta[6 * bs + 1: 7 * bs + 1]
            self._cg_kv_shared[bs] = meta[7 * bs + 1: 8 * bs + 1]
            self._cg_rows[bs] = torch.full((bs,), -1, dtype=torch.int32, device=dev)
            self._cg_desc[bs] = torch.zeros(4 * bs, dtype=torch.int32, device=dev)
            self._cg_slots[bs] = torch.full((bs,), -1, dtype=torch.int32, device=dev)
            self._cg_append_indptr[bs] = torch.arange(bs + 1, dtype=torch.int32, device=dev)
            self._cg_temperature[bs] = torch.ones(bs, 1, dtype=torch.float32, device=dev)
            self._cg_top_k[bs] = torch.full((bs,), self.vocab_size, dtype=torch.int32, device=dev)
            self._cg_top_p[bs] = torch.ones(bs, dtype=torch.float32, device=dev)

    def fill_cuda_graph_metadata(self, bucket_size: int, real_uuids) -> None:
        """manager.py:228-253: the real sequences' page tables and the position of each one's
        newest token, then ``bucket - n`` padding rows (one padding page, last_page_len 1,
        position 0), written into the bucket's static buffers on the device.  Also fills
        ``_cg_kv_shared[bucket]``: for each row, the leading pages it has in common with the
        row before it (the decode plan's ``kv_shared_pages``; all zero unless pages are
        shared)."""
        real_uuids = list(real_uuids)
        self._flush()
        slot, staged, b, pages = self._stage_tables(real_uuids, bucket_size, positions=True)
        if pages > self._cg_kv_indices[bucket_size].numel():
            raise RuntimeError("page table larger than the bucket's kv_indices buffer")
        # [desc | indptr | last | positions | shared] lands in the bucket's block: the buffers
        # the step reads are views of it
        self._gather(slot, staged, b, pages, self._cg_kv_indices[bucket_size], dst=self._cg_meta[bucket_size],
                     slots=self._cg_slots[bucket_size])
        if self._n_multi:
            idx = self._cg_kv_indices[bucket_size]
            check(lib().pkv_shared_prefix_pages(self._cg_kv_indptr[bucket_size].data_ptr(), idx.data_ptr(),
                                                idx.numel(), b, self._cg_kv_shared[bucket_size].data_ptr(),
                                                stream_ptr(self.device)), "shared-page hint")

    def append_paged_kv_cache_cuda_graph(self, key, value, bucket_size: int, layer_idx: int) -> None:
        """manager.py:270-280: the append through the bucket's static metadata.  Each row's
        destination (the page and slot its ``positions`` entry selects through ``kv_indptr`` /
        ``kv_indices``) is resolved once per step by ``fill_cuda_graph_metadata``, so every
        layer's append reads one slot per token."""
        append_paged_kv_cache_slots(key, value, self._cg_slots[bucket_size], self.kv_cache[layer_idx],
                                    kv_layout=self.layout)

    # ------------------------------------------------------------------ device-resident decode steps

    def begin_device_steps(self, bucket_size: int, real_uuids, steps: int, num_new_tokens: int = 1) -> None:
        """Extension: hand the next ``steps`` decode steps of this batch to the device.

        Each step is the serving loop's ``append_tokens(b, num_new_tokens)`` for every sequence
        of ``real_uuids`` (in that order) followed by ``fill_cuda_graph_metadata(bucket_size,
        real_uuids)`` (ecahlang/main.py:328-347), done by ``device_step`` on the device with no
        host work, so it can be captured in a graph together with the plan and the model and
        replayed.  Per replay the host calls ``advance_device_step`` (O(1): it advances the free
        count by the pages the step pops, which it knows in advance).  Sets up the bucket's
        buffers for the current state (as ``fill_cuda_graph_metadata`` would) and widens the
        page table for ``steps`` steps, before any capture: the table must not move while a
        graph holds its address.  Any other method of the manager first brings the host
        counts up to date (``end_device_steps``)."""
        self._end_dev()
        ids = list(real_uuids)
        bs = self.block_size
        if steps < 0 or num_new_tokens < 0:
            raise ValueError("steps and num_new_tokens must be non-negative")
        if steps and num_new_tokens:
            # A row whose new tokens would go into a page other lists hold takes its private
            # copy now (the copy on write its first append would make), in row order, so the
            # device steps only ever write pages their rows hold alone.
            rc, need = {}, 0
            for i in ids:  # (a copy drops the old page's count for the rows after it)
                h = self._pg[i]
                if h and self.batch_to_page_lengths[i] < bs:
                    c = rc.get(h[-1], self._rc[h[-1]])
                    if c > 1:
                        rc[h[-1]] = c - 1
                        need += 1
            if need > self._n_free:
                raise RuntimeError("Not enough free blocks to append tokens")
            for i in ids:
                if self._shares_last_page(i):
                    self._queue_cow(i)
        grow = -(-(steps * num_new_tokens) // bs) + 1  # pages a sequence can gain
        if ids:
            self._ensure_stride(max(self._npages[i] for i in ids) + grow)
        cap = self._cg_kv_indices[bucket_size].numel()
        if sum(self._npages[i] for i in ids) + len(ids) * grow + bucket_size - len(ids) > cap:
            raise RuntimeError("page table of the device steps larger than the bucket's kv_indices buffer")
        self.fill_cuda_graph_metadata(bucket_size, ids)
        npages = [self._npages[i] for i in ids]
        plen = [self.batch_to_page_lengths[i] for i in ids]
        # the device's counts, from the metadata just written (one launch)
        check(lib().pkv_pool_steps_begin(self._cg_meta[bucket_size].data_ptr(),
                                         self._cg_kv_last_page_len[bucket_size].data_ptr(), bucket_size, len(ids),
                                         self._n_free, self._cg_rows[bucket_size].data_ptr(),
                                         self._dev_npages.data_ptr(), self._dev_plen.data_ptr(), self._rows,
                                         self._dev_nfree.data_ptr(), self._err.data_ptr(), stream_ptr(self.device)),
              "device steps hand-over")
        # one token a step: a row with last-page length p pops at the steps k with p + k a
        # multiple of bs, and a row whose last page starts full (p == bs) also pops at step 1
        hist = np.zeros(bs, dtype=np.int64)
        for p in plen:
            hist[p % bs] += 1
        self._dev = {"bucket": bucket_size, "ids": ids, "at": {i: j for j, i in enumerate(ids)},
                     "npages0": npages, "plen0": plen, "hist": hist, "full": sum(p == bs for p in plen),
                     "n": num_new_tokens, "k": 0, "max": steps}

    def device_step(self, bucket_size: int) -> None:
        """Enqueue one device step of the batch given to ``begin_device_steps`` (no host work;
        safe to capture): ``pkv_pool_step`` over the bucket's static buffers."""
        d = self._dev
        if d is None or d["bucket"] != bucket_size:
            raise RuntimeError("begin_device_steps must be called for this bucket first")
        idx = self._cg_kv_indices[bucket_size]
        check(lib().pkv_pool_step(self._stack.data_ptr(), self._dev_nfree.data_ptr(), self._table.data_ptr(),
                                  self._stride, self._rows, self._cg_rows[bucket_size].data_ptr(), bucket_size,
                                  d["n"], self.block_size, self._dev_npages.data_ptr(), self._dev_plen.data_ptr(),
                                  self._pad_row, self._cg_desc[bucket_size].data_ptr(),
                                  self._cg_kv_indptr[bucket_size].data_ptr(),
                                  self._cg_kv_last_page_len[bucket_size].data_ptr(),
                                  self._cg_positions[bucket_size].data_ptr(), idx.data_ptr(), idx.numel(),
                                  idx.numel(), self._cg_slots[bucket_size].data_ptr(), self._err.data_ptr(),
                                  stream_ptr(self.device)), "device decode step")

    def advance_device_step(self, bucket_size: int) -> None:
        """The host side of one replay of ``device_step`` (call it once per replay, before it).
        When the step would need more free pages than the pool has, the host counts are
        brought up to date and the reference's per-sequence path runs instead, which raises
        ``RuntimeError("Not enough free blocks to append tokens")`` at the same sequence as the
        reference (the sequences before it are appended); the graph must then not be
        replayed."""
        d = self._dev
        if d is None or d["bucket"] != bucket_size:
            raise RuntimeError("begin_device_steps must be called for this bucket first")
        k = d["k"] + 1
        if k > d["max"]:
            raise RuntimeError(f"begin_device_steps was given {d['max']} steps")
        bs, n = self.block_size, d["n"]
        if n == 1:
            pops = int(d["hist"][(-k) % bs]) + (d["full"] if k == 1 else 0)
        else:
            pops = sum(self._advanced(0, p, k * n)[0] - self._advanced(0, p, (k - 1) * n)[0] for p in d["plen0"])
        if pops > self._n_free:
            ids = d["ids"]
            self._end_dev()
            for i in ids:  # raises at the first sequence the pool cannot serve
                self.append_tokens(i, n)
            raise RuntimeError("Not enough free blocks to append tokens")
        self._n_free -= pops
        d["k"] = k

    def end_device_steps(self) -> None:
        """Bring the host counts of the device's batch up to date (the steps it has run)."""
        self._end_dev()

    def _end_dev(self) -> None:
        d = self._dev
        if d is None:
            return
        self._dev = None
        for i, n0, p0 in zip(d["ids"], d["npages0"], d["plen0"]):
            self._npages[i], self.batch_to_page_lengths[i] = self._advanced(n0, p0, d["k"] * d["n"])
            if self._npages[i] > n0:  # the pages the device steps popped
                self._pg[i] += self._new_handles(self._npages[i] - n0)

    # ------------------------------------------------------------------ sampling buffers (outside the path)
    # main.py reads sampling_{temperature,top_k,top_p}_gpu and the bucket's _cg_* copies of
    # them (main.py:360, 375-378, 462, 477-479); they are kept so it finds them.  Each call
    # stages its values in a fresh pinned buffer, so a queued copy never sees them change.

    def init_sampling_buffers(self, max_batch_size: int) -> None:
        dev = self.device
        self.sampling_temperature_gpu = torch.ones(max_batch_size, 1, dtype=torch.float32, device=dev)
        self.sampling_top_k_gpu = torch.full((max_batch_size,), self.vocab_size, dtype=torch.int32, device=dev)
        self.sampling_top_p_gpu = torch.ones(max_batch_size, dtype=torch.float32, device=dev)

    @staticmethod
    def _stage(dst: torch.Tensor, values, n: int) -> None:
        src = torch.as_tensor(values, dtype=dst.dtype).reshape(-1)[:n].pin_memory()
        dst.reshape(-1)[:n].copy_(src, non_blocking=True)

    def fill_sampling_params(self, n: int, temperatures, top_ks, top_ps) -> None:
        self._stage(self.sampling_temperature_gpu, temperatures, n)
        self._stage(self.sampling_top_k_gpu, top_ks, n)
        self._stage(self.sampling_top_p_gpu, top_ps, n)

    def fill_cuda_graph_sampling_params(self, bucket_size: int, n: int, temperatures, top_ks, top_ps) -> None:
        t, k, p = self._cg_temperature[bucket_size], self._cg_top_k[bucket_size], self._cg_top_p[bucket_size]
        t.fill_(1.0)  # padding rows keep neutral values
        k.fill_(self.vocab_size)
        p.fill_(1.0)
        self._stage(t, temperatures, n)
        self._stage(k, top_ks, n)
        self._stage(p, top_ps, n)
