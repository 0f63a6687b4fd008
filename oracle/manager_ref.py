"""Restatement of the reference's page-pool bookkeeping with plain Python lists.

Test infrastructure only (see oracle/__init__.py).  Follows ecahlang/manager.py line by line
for the list semantics; the GPU tensors and sampling buffers of the original are left out.

One deliberate divergence, shared with the product manager: ``allocate(T)`` with
``T % block_size == 0`` records ``page_len = block_size`` instead of 0.  The reference's
0 (manager.py:106) makes ``get_seq_lens`` report T - block_size while T tokens are held
(and a following append overwrites slot 0 of the last full page); block_size is the only
value consistent with the pages it pops.  The page ids popped are unchanged.

One extension with no counterpart in the reference (which has no page refcounting): prefix
sharing.  ``allocate(b, T, prefix=p)`` gives sequence b the full pages of the live sequence p
first (shared, not popped), then pops the pages for the rest of its T tokens; ``free(b)``
returns only b's own pages; ``free(p)`` while sequences share p raises.  This is the
restatement the device manager's prefix sharing is checked against.
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
        self.shared: dict = {}  # batch_id -> (prefix id, number of leading shared pages)
        self.refs: dict = {}    # prefix id -> live sequences sharing its pages

    # manager.py:99-112 (+ the prefix extension)
    def allocate(self, batch_id, total_tokens: int, prefix=None) -> list:
        shared = []
        if prefix is not None:
            if prefix not in self.batch_to_blocks:
                raise ValueError(f"{prefix} not allocated")
            shared = self.batch_to_blocks[prefix][: self.seq_len(prefix) // self.block_size]
            if total_tokens < len(shared) * self.block_size:
                raise ValueError("a sequence cannot be shorter than its shared prefix")
        num_pages = math.ceil(total_tokens / self.block_size) - len(shared)
        if len(self.free_blocks) < num_pages:
            raise RuntimeError("Not enough KV cache blocks available")
        blocks = shared + [self.free_blocks.pop() for _ in range(num_pages)]
        self.batch_to_blocks[batch_id] = blocks
        if prefix is not None:
            self.shared[batch_id] = (prefix, len(shared))
            self.refs[prefix] = self.refs.get(prefix, 0) + 1
        page_len = total_tokens % self.block_size
        if page_len == 0 and total_tokens > 0 and not self.strict_reference_q1:
            page_len = self.block_size
        self.batch_to_page_lengths[batch_id] = page_len
        self.batch_to_total_tokens[batch_id] = total_tokens
        seq_slot = self.free_seq_lens.pop()
        self.batch_to_seq_len[batch_id] = seq_slot
        return blocks

    # manager.py:114-120 (+ the prefix extension)
    def free(self, batch_id) -> None:
        if self.refs.get(batch_id):
            raise RuntimeError(f"{batch_id} is the shared prefix of {self.refs[batch_id]} live sequences")
        blocks = self.batch_to_blocks.pop(batch_id, [])
        prefix, n_shared = self.shared.pop(batch_id, (None, 0))
        if prefix is not None:
            self.refs[prefix] -= 1
        self.free_blocks.extend(blocks[n_shared:])
        self.batch_to_page_lengths.pop(batch_id, None)
        seq_slot = self.batch_to_seq_len.pop(batch_id, None)
        if seq_slot is not None:
            self.free_seq_lens.append(seq_slot)

    # manager.py:187-205
    def append_tokens(self, batch_id, num_new_tokens: int) -> None:
        if batch_id not in self.batch_to_blocks:
            raise ValueError(f"{batch_id} not allocated")
        current_len = self.batch_to_page_lengths.get(batch_id, 0)
        total_tokens = current_len + num_new_tokens
        full_new_pages = total_tokens // self.block_size
        remaining = total_tokens % self.block_size
        if full_new_pages > len(self.free_blocks):
            raise RuntimeError("Not enough free blocks to append tokens")
        for _ in range(full_new_pages):
            self.batch_to_blocks[batch_id].append(self.free_blocks.pop())
        self.batch_to_page_lengths[batch_id] = remaining

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
