"""The manager's host-side page-table staging (``AutoKVCacheManager._stage_tables``: the array
that one copy takes to the device before the page gather) against the oracle's list
restatement of get_append_metadata / fill_cuda_graph_metadata (ecahlang/manager.py:122-138,
:228-253).  CPU only: the method reads the host bookkeeping alone, so the manager's state is
set from the oracle's after a random sequence of pool operations."""
import random

import numpy as np
import pytest

from ecahlang_amd.manager import AutoKVCacheManager
from oracle.manager_ref import RefKVCacheManager


class _HostStaging:  # hands out plain host arrays where the manager uses its pinned ring
    def host(self, n):
        return -1, np.full(n, -7, dtype=np.int32)  # (poisoned: every entry must be written)


def _mirror(ref: RefKVCacheManager) -> AutoKVCacheManager:
    m = object.__new__(AutoKVCacheManager)
    m.block_size = ref.block_size
    m.batch_to_seq_len = dict(ref.batch_to_seq_len)
    m.batch_to_page_lengths = dict(ref.batch_to_page_lengths)
    m._npages = {b: len(p) for b, p in ref.batch_to_blocks.items()}
    m._n_padding = len(ref.padding_pages)
    m._rows = ref.seq_lens + 1
    m._pad_row = ref.seq_lens
    m._dev = None
    m._staging = _HostStaging()
    return m


def _random_pool(seed):
    rng = random.Random(seed)
    ref = RefKVCacheManager(400)
    ref.init_cuda_graph_buffers([1, 2, 4, 8, 16, 32])
    ids = list(range(24))
    for _ in range(300):
        sid = rng.choice(ids)
        n = rng.choice([0, 1, 1, 2, 15, 16, 17, 40])
        try:
            if sid not in ref.batch_to_blocks:
                pre = [p for p in ref.batch_to_blocks if ref.seq_len(p) >= 16]
                if pre and rng.random() < 0.5:  # on a live sequence's full pages
                    p = rng.choice(pre)
                    ref.allocate(sid, ref.seq_len(p) // 16 * 16 + n, prefix=p)
                else:
                    ref.allocate(sid, n)
            elif rng.random() < 0.15:
                ref.free(sid)
            else:
                ref.append_tokens(sid, rng.choice([1, 1, 1, 3, 16]))
        except RuntimeError:  # pool exhausted: the oracle is unchanged, go on
            pass
    return rng, ref


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_staged_tables_match_oracle(seed):
    rng, ref = _random_pool(seed)
    m = _mirror(ref)
    live = list(ref.batch_to_blocks)
    for it in range(20):
        ids = rng.sample(live, rng.randint(0, len(live)))
        if it % 2:  # rows on one prefix next to each other, as a serving batch groups them
            ids.sort(key=lambda i: ref.batch_to_blocks[i][:1])
        # get_append_metadata: [desc | indptr | last_page_len]
        _, out, b, pages = m._stage_tables(ids)
        idx, ptr, last = ref.get_append_metadata(ids)
        assert b == len(ids) and pages == len(idx) and out.size == 6 * b + 1
        assert out[4 * b: 5 * b + 1].tolist() == ptr
        assert out[5 * b + 1:].tolist() == last
        desc = out[: 4 * b].reshape(b, 4).tolist()
        assert desc == [[ref.batch_to_seq_len[i], 0, len(ref.batch_to_blocks[i]), 0] for i in ids]
        # fill_cuda_graph_metadata: padded to the bucket, plus each row's newest-token position
        bucket = next(s for s in (1, 2, 4, 8, 16, 32) if s >= len(ids)) if len(ids) <= 32 else None
        if bucket is None:
            continue
        _, out, b, pages = m._stage_tables(ids, bucket, positions=True)
        idx, ptr, last, pos = ref.fill_cuda_graph_metadata(bucket, ids)
        assert b == bucket and pages == len(idx) and out.size == 8 * b + 1
        assert out[4 * b: 5 * b + 1].tolist() == ptr
        assert out[5 * b + 1: 6 * b + 1].tolist() == last
        assert out[6 * b + 1: 7 * b + 1].tolist() == pos
        # the decode plan's hint is left zero here: the device fills it from the gathered lists
        assert out[7 * b + 1:].tolist() == [0] * bucket
        desc = out[: 4 * b].reshape(b, 4).tolist()
        real = [[ref.batch_to_seq_len[i], 0, len(ref.batch_to_blocks[i]), 0] for i in ids]
        pad = [[m._pad_row, i, 1, 0] for i in range(bucket - len(ids))]
        assert desc == real + pad


def test_staging_errors_match_the_reference():
    _, ref = _random_pool(5)
    m = _mirror(ref)
    live = list(ref.batch_to_blocks)[:3]
    with pytest.raises(IndexError, match="list index out of range"):  # more padding rows than pages
        m._stage_tables(live, 64, positions=True)
    with pytest.raises(KeyError):
        m._stage_tables(live + ["never allocated"])
