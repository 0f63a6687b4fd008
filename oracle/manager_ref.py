"""Restatement of the reference's page-pool bookkeeping with plain Python lists.

Test infrastructure only (see oracle/__init__.py).  Follows ecahlang/manager.py line by line
for the list semantics; the GPU tensors and sampling buffers of the original are left out.

One deliberate divergence, shared with the product manager: ``allocate(T)`` with
``T % block_size == 0`` records ``page_len = block_size`` instead of 0.  The reference's
0 (manager.py:106) makes ``get_seq_lens`` report T - block_size while T tokens are held
(and a following append overwrites slot 0 of the last full page); block_size is the only
value consistent with the pages it pops.  The page ids popped are unchanged.

One extension with no counterpart in the reference (which has no page refcounting): shared
pages, radix style.  Every page in a sequence's list has a reference count (the number of
lists that hold it).  ``allocate(b, T, prefix=p)`` gives sequence b the pages of the live
sequence p that cover b's first min(T, len(p)) tokens -- p's partial last page included --
then pops pages for the rest of its T tokens; p may itself share pages with others, so
prefixes nest.  A sequence that writes into a page others still hold first takes a private
copy of it ("copy on write": one page popped, the old page's count dropped; the device copies
the page's K/V for every layer): at allocate, when b's tokens continue past a shared partial
page, and at append_tokens, when new tokens go into a shared last page.  Those pops come
before the others of the same call.  ``free(b)`` returns, in page order, the pages only b
held (always a tail of b's list: every sequence that holds one of b's pages holds all of b's
pages before it) and drops the counts of the rest.  This is the restatement the device
manager's sharing is checked against.
"""
from __future__ import annotations

import math


class RefKVCacheManager:
    def __init__(self, max_blocks: int, seq_lens: int = 128, block_size: int = 16,
                 strict_reference_q1: bool = False):
        # manager.py:31, :47-49 (pool size given directly), :56-61
        self.block_size = block_size
        self.max_blocks = max_blocks
        self.seq_lens = max(seq_lens, 128)
        self.free_blocks = list(range(max_blocks))
        self.free_seq_lens = list(range(self.seq_lens))
        self.batch_to_blocks: dict = {}
        self.batch_to_page_lengths: dict = {}
        self.batch_to_total_tokens: dict = {}
        self.batch_to_seq_len: dict = {}
        self.padding_pages: list = []
        self.strict_reference_q1 = strict_reference_q1
        self.refs: dict = {}    # page id -> number of sequences whose list holds it
        self.cow_pairs: list = []  # (old page, new page) of every copy on write, in order

    def _pop(self) -> int:
        page = self.free_blocks.pop()
        self.refs[page] = 1
        return page

    def _cow(self, blocks: list, i: int) -> None:
        """Replace the shared page blocks[i] by a private copy."""
        old, new = blocks[i], self._pop()
        self.refs[old] -= 1
        blocks[i] = new
        self.cow_pairs.append((old, new))

    def shares_last_page(self, batch_id) -> bool:
        """Whether new tokens would go into a page other sequences hold."""
        pages = self.batch_to_blocks[batch_id]
        return bool(pages) and self.refs[pages[-1]] > 1 and self.batch_to_page_lengths[batch_id] < self.block_size

    # manager.py:99-112 (+ the sharing extension)
    def allocate(self, batch_id, total_tokens: int, prefix=None) -> list:
        shared, cow = [], False
        if prefix is not None:
            if prefix not in self.batch_to_blocks:
                raise ValueError(f"{prefix} not allocated")
            ts = min(total_tokens, self.seq_len(prefix))
            shared = self.batch_to_blocks[prefix][: math.ceil(ts / self.block_size)]
            cow = total_tokens > ts and ts % self.block_size != 0
        num_pages = math.ceil(total_tokens / self.block_size) - len(shared)
        if len(self.free_blocks) < num_pages + cow:
            raise RuntimeError("Not enough KV cache blocks available")
        blocks = list(shared)
        for page in shared:
            self.refs[page] += 1
        if cow:
            self._cow(blocks, len(blocks) - 1)
        blocks += [self._pop() for _ in range(num_pages)]
        self.batch_to_blocks[batch_id] = blocks
        page_len = total_tokens % self.block_size
        if page_len == 0 and total_tokens > 0 and not self.strict_reference_q1:
            page_len = self.block_size
        self.batch_to_page_lengths[batch_id] = page_len
        self.batch_to_total_tokens[batch_id] = total_tokens
        seq_slot = self.free_seq_lens.pop()
        self.batch_to_seq_len[batch_id] = seq_slot
        return blocks

    # manager.py:114-120 (+ the sharing extension)
    def free(self, batch_id) -> None:
        blocks = self.batch_to_blocks.pop(batch_id, [])
        t = len(blocks)
        while t > 0 and self.refs[blocks[t - 1]] == 1:
            t -= 1
        assert all(self.refs[p] > 1 for p in blocks[:t]), "pages only this list holds form its tail"
        for p in blocks[:t]:
            self.refs[p] -= 1
        for p in blocks[t:]:
            del self.refs[p]
        self.free_blocks.extend(blocks[t:])
        self.batch_to_page_lengths.pop(batch_id, None)
        seq_slot = self.batch_to_seq_len.pop(batch_id, None)
        if seq_slot is not None:
            self.free_seq_lens.append(seq_slot)

    # manager.py:187-205 (+ copy on write into a shared last page)
    def append_tokens(self, batch_id, num_new_tokens: int) -> None:
        if batch_id not in self.batch_to_blocks:
            raise ValueError(f"{batch_id} not allocated")
        current_len = self.batch_to_page_lengths.get(batch_id, 0)
        total_tokens = current_len + num_new_tokens
        full_new_pages = total_tokens // self.block_size
        remaining = total_tokens % self.block_size
        cow = num_new_tokens > 0 and self.shares_last_page(batch_id)
        if full_new_pages + cow > len(self.free_blocks):
            raise RuntimeError("Not enough free blocks to append tokens")
        if cow:
            self._cow(self.batch_to_blocks[batch_id], len(self.batch_to_blocks[batch_id]) - 1)
        for _ in range(full_new_pages):
            self.batch_to_blocks[batch_id].append(self._pop())
        self.batch_to_page_lengths[batch_id] = remaining

    def make_last_pages_private(self, batch_ids) -> None:
        """Copy on write, in list order, for every sequence whose new tokens would go into a
        shared page (what each one's next append_tokens would do first)."""
        refs, need = dict(self.refs), 0
        for b in batch_ids:  # (a copy drops the old page's count for the rows after it)
            pages = self.batch_to_blocks[b]
            if pages and refs[pages[-1]] > 1 and self.batch_to_page_lengths[b] < self.block_size:
                refs[pages[-1]] -= 1
                need += 1
        if need > len(self.free_blocks):
            raise RuntimeError("Not enough free blocks to append tokens")
        for b in batch_ids:
            if self.shares_last_page(b):
                self._cow(self.batch_to_blocks[b], len(self.batch_to_blocks[b]) - 1)

    @staticmethod
    def shared_prefix_pages(kv_indices: list, kv_indptr: list) -> list:
        """Entry b >= 1: how many leading pages row b has in common with row b - 1 (the
        decode plan's kv_shared_pages); entry 0 is 0."""
        out = [0] * (len(kv_indptr) - 1)
        for b in range(1, len(out)):
            x = kv_indices[kv_indptr[b]:kv_indptr[b + 1]]
            y = kv_indices[kv_indptr[b - 1]:kv_indptr[b]]
            k = 0
            while k < min(len(x), len(y)) and x[k] == y[k]:
                k += 1
            out[b] = k
        return out

    # manager.py:122-138 (lists instead of device tensors)
    def get_append_metadata(self, batch_ids) -> tuple:
        kv_indices, kv_indptr, kv_last_page_len = [], [0], []
        for bid in batch_ids:
            pages = self.batch_to_blocks[bid]
            kv_indices.extend(pages)
            kv_indptr.append(kv_indptr[-1] + len(pages))
            kv_last_page_len.append(self.batch_to_page_lengths[bid])
        return kv_indices, kv_indptr, kv_last_page_len

    # manager.py:207-212 (padding-page reservation; the buffers themselves are device-side)
    def init_cuda_graph_buffers(self, bucket_sizes) -> None:
        max_bucket = max(bucket_sizes)
        if len(self.free_blocks) < max_bucket:
            raise RuntimeError(f"Not enough free blocks for {max_bucket} padding pages")
        self.padding_pages = [self.free_blocks.pop() for _ in range(max_bucket)]

    # manager.py:228-253 (lists instead of device tensors)
    def fill_cuda_graph_metadata(self, bucket_size: int, real_uuids) -> tuple:
        kv_indices, kv_indptr, kv_last_page_len, positions = [], [0], [], []
        for uid in real_uuids:
            pages = self.batch_to_blocks[uid]
            kv_indices.extend(pages)
            kv_indptr.append(kv_indptr[-1] + len(pages))
            kv_last_page_len.append(self.batch_to_page_lengths[uid])
            total = (len(pages) - 1) * self.block_size + self.batch_to_page_lengths[uid]
            positions.append(total - 1)
        for i in range(bucket_size - len(real_uuids)):
            kv_indices.append(self.padding_pages[i])
            kv_indptr.append(kv_indptr[-1] + 1)
            kv_last_page_len.append(1)
            positions.append(0)
        return kv_indices, kv_indptr, kv_last_page_len, positions

    def seq_len(self, batch_id) -> int:
        pages = self.batch_to_blocks[batch_id]
        if not pages:
            return 0
        return (len(pages) - 1) * self.block_size + self.batch_to_page_lengths[batch_id]


class _Node:
    """One cached page of a prefix tree: the page's block_size token ids (its key under its
    parent), the page, and its last use."""
    __slots__ = ("key", "page", "parent", "children", "last", "id", "row")

    def __init__(self, key, page, parent, nid, row=None):
        self.key, self.page, self.parent, self.id, self.row = key, page, parent, nid, row
        self.children: dict = {}
        self.last = 0


class RefRadixKVCacheManager(RefKVCacheManager):
    """The page pool with a token-keyed prefix cache (an extension: the reference frees every
    page of a finished sequence at once, manager.py:114-120, and keeps no index of what the
    pages hold).  The rules, which the device manager (AutoKVCacheManager with
    ``prefix_cache_rows``) follows exactly:

    * The cache is a tree of full pages: a node is one page whose block_size token ids are its
      key under its parent; a path from the root is a page-aligned token prefix.
    * ``allocate(b, T, tokens=ids)`` starts b with the pages of the longest cached path that
      matches ids[:T] block by block (only blocks wholly inside both), each page's count going
      up by one, then pops ceil(T / block_size) - k pages as ``allocate`` does.
    * ``free(b, tokens=ids)`` first inserts b's full pages whose tokens ids gives (blocks wholly
      inside min(len(ids), seq_len(b))): walking from the root, a block already cached with
      b's own page is followed, a block cached with another page ends the walk, and every block
      after the last one followed becomes a new node holding b's page (the tree's hold counts
      like a list's).  The new nodes of one insert share one of ``cache_rows`` cache slots; with
      none free, least recently used nodes are evicted until one is, and if none is, nothing
      is inserted.  Then b is freed as ``free`` does: the pages the tree keeps stay allocated.
    * A clock advances at every allocate and free given tokens; the nodes an allocate matched
      and the nodes a free walked or created take its value.
    * Eviction: a node whose page only the tree holds and which has no children is evictable;
      the one with the smallest (last use, creation number) goes first, its page back on the
      free stack; its parent may become evictable.  ``allocate`` and ``append_tokens`` evict
      while the free stack is short of the pages they need (never the nodes the allocate
      matched), before raising the reference's exception if it still is; evictions made stay
      made.  ``evict(n)`` evicts up to n pages.
    """

    def __init__(self, max_blocks: int, seq_lens: int = 128, block_size: int = 16, cache_rows: int | None = None):
        super().__init__(max_blocks, seq_lens, block_size)
        self.root = _Node(None, None, None, -1)
        self.clock = 0
        self.next_id = 0
        self.cache_rows = self.seq_lens if cache_rows is None else cache_rows
        self.free_rows = list(range(self.cache_rows))  # handed out from the end
        self.row_nodes: dict = {}
        self.evicted: list = []  # pages evicted, in order

    # ---- tree
    def _keys(self, tokens, limit: int) -> list:
        bs = self.block_size
        n = min(len(tokens), limit) // bs
        return [tuple(tokens[i * bs:(i + 1) * bs]) for i in range(n)]

    def match(self, tokens, limit: int | None = None) -> list:
        """The nodes of the longest cached path matching tokens (blocks within limit)."""
        path, node = [], self.root
        for key in self._keys(tokens, len(tokens) if limit is None else limit):
            node = node.children.get(key)
            if node is None:
                break
            path.append(node)
        return path

    def nodes(self) -> list:
        out, stack = [], list(self.root.children.values())
        while stack:
            n = stack.pop()
            out.append(n)
            stack.extend(n.children.values())
        return out

    def cached_pages(self) -> dict:
        """page -> the token ids of the path ending at it."""
        out = {}
        for n in self.nodes():
            keys, m = [], n
            while m is not self.root:
                keys.append(m.key)
                m = m.parent
            out[n.page] = [t for k in reversed(keys) for t in k]
        return out

    def _evict_one(self, protect=()) -> bool:
        best = None
        for n in self.nodes():
            if n.children or self.refs[n.page] != 1 or n in protect:
                continue
            if best is None or (n.last, n.id) < (best.last, best.id):
                best = n
        if best is None:
            return False
        del best.parent.children[best.key]
        del self.refs[best.page]
        self.free_blocks.append(best.page)
        self.evicted.append(best.page)
        self.row_nodes[best.row] -= 1
        if self.row_nodes[best.row] == 0:
            del self.row_nodes[best.row]
            self.free_rows.append(best.row)
        return True

    def evict(self, n: int, protect=()) -> int:
        k = 0
        while k < n and self._evict_one(protect):
            k += 1
        return k

    # ---- the pool's calls
    def allocate(self, batch_id, total_tokens: int, prefix=None, tokens=None) -> list:
        bs = self.block_size
        if prefix is not None and prefix not in self.batch_to_blocks:
            raise ValueError(f"{prefix} not allocated")
        if tokens is None:
            need = math.ceil(total_tokens / bs)
            if prefix is not None:
                ts = min(total_tokens, self.seq_len(prefix))
                need += -math.ceil(ts / bs) + (total_tokens > ts and ts % bs != 0)
            if len(self.free_blocks) < need:
                self.evict(need - len(self.free_blocks))
            return super().allocate(batch_id, total_tokens, prefix)
        if prefix is not None:
            raise ValueError("prefix and tokens are exclusive")
        self.clock += 1
        path = self.match(tokens, total_tokens)
        need = math.ceil(total_tokens / bs) - len(path)
        if len(self.free_blocks) < need:
            self.evict(need - len(self.free_blocks), protect=set(path))
        if len(self.free_blocks) < need:
            raise RuntimeError("Not enough KV cache blocks available")
        blocks = [n.page for n in path]
        for n in path:
            self.refs[n.page] += 1
            n.last = self.clock
        blocks += [self._pop() for _ in range(need)]
        self.batch_to_blocks[batch_id] = blocks
        page_len = total_tokens % bs
        if page_len == 0 and total_tokens > 0:
            page_len = bs
        self.batch_to_page_lengths[batch_id] = page_len
        self.batch_to_total_tokens[batch_id] = total_tokens
        self.batch_to_seq_len[batch_id] = self.free_seq_lens.pop()
        return blocks

    def free(self, batch_id, tokens=None) -> None:
        if tokens is not None and batch_id in self.batch_to_blocks:
            self.clock += 1
            blocks = self.batch_to_blocks[batch_id]
            node, created = self.root, []
            for i, key in enumerate(self._keys(tokens, self.seq_len(batch_id))):
                child = node.children.get(key) if not created else None
                if child is not None:
                    if child.page != blocks[i]:
                        break
                    child.last = self.clock
                    node = child
                    continue
                new = _Node(key, blocks[i], node, self.next_id)
                self.next_id += 1
                created.append(new)
                node = new
            if created:
                while not self.free_rows and self._evict_one():
                    pass
                if self.free_rows:
                    row = self.free_rows.pop()
                    self.row_nodes[row] = len(created)
                    for n in created:
                        n.parent.children[n.key] = n
                        n.row, n.last = row, self.clock
                        self.refs[n.page] += 1
        super().free(batch_id)

    def append_tokens(self, batch_id, num_new_tokens: int) -> None:
        if batch_id in self.batch_to_blocks:
            t = self.batch_to_page_lengths.get(batch_id, 0) + num_new_tokens
            need = t // self.block_size + (num_new_tokens > 0 and self.shares_last_page(batch_id))
            if need > len(self.free_blocks):
                self.evict(need - len(self.free_blocks))
        super().append_tokens(batch_id, num_new_tokens)
