"""Device-resident decode steps (AutoKVCacheManager.begin_device_steps / device_step /
advance_device_step): every step's page table (kv_indices, kv_indptr, kv_last_page_len, the
newest-token positions and the append slots) against the oracle pool running the reference's
loop (append_tokens for every sequence, then fill_cuda_graph_metadata), for one and several
tokens a step, sequences whose last page starts empty, partial or full, padding rows, eager and
graph-replayed steps; then the pool itself (page lists, free stack) after the steps, and the
reference's exception, at the same sequence, when the pool runs dry."""
import numpy as np
import pytest
import torch

from ecahlang_amd.manager import AutoKVCacheManager
from oracle.manager_ref import RefKVCacheManager

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
BUCKET = 16


def _pair(pages):
    per_block = 16 * 2 * 64 * 2 * 2  # block_size * Hkv * D * 2 (K, V) * fp16
    m = AutoKVCacheManager(1, 2, 64, dtype=torch.float16, device=DEV, total_gpu_mem_bytes=pages * per_block,
                           mem_utilization=1.0, max_pages_per_seq=8)
    ref = RefKVCacheManager(m.max_blocks, seq_lens=m.seq_lens)
    return m, ref


def _allocate(m, ref, lens, prefix_at=None):
    ids = []
    for i, n in enumerate(lens):
        sid = f"s{i}"
        m.allocate(sid, n)
        ref.allocate(sid, n)
        ids.append(sid)
    return ids


def _expected_slots(idx, ptr, pos, bs=16):
    out = []
    for b in range(len(pos)):
        p = pos[b]
        n = ptr[b + 1] - ptr[b]
        out.append(idx[ptr[b] + p // bs] * bs + p % bs if 0 <= p and p // bs < n else -1)
    return out


def _check_meta(m, ref, ids, step):
    idx, ptr, last, pos = ref.fill_cuda_graph_metadata(BUCKET, ids)
    b = BUCKET
    assert m._cg_kv_indptr[b].tolist() == ptr, step
    assert m._cg_kv_indices[b][:len(idx)].tolist() == idx, step
    assert m._cg_kv_last_page_len[b].tolist() == last, step
    assert m._cg_positions[b].tolist() == pos, step
    assert m._cg_slots[b].tolist() == _expected_slots(idx, ptr, pos), step


# last-page lengths 16 (full: allocate of a multiple of 16), 15 (fills at the first step), 1,
# and longer sequences; 10 real rows in a bucket of 16 (6 padding rows)
LENS = [32, 15, 1, 47, 64, 100, 17, 16, 250, 3]


@pytest.mark.parametrize("n_tokens,graph", [(1, False), (1, True), (3, False), (17, True)])
def test_device_steps_match_the_reference_loop(n_tokens, graph):
    print(f"device steps: n_tokens={n_tokens} graph={graph}", flush=True)
    m, ref = _pair(600)
    ids = _allocate(m, ref, LENS)
    m.init_cuda_graph_buffers([BUCKET], max_indices=4096)
    ref.init_cuda_graph_buffers([BUCKET])
    steps = 40
    m.begin_device_steps(BUCKET, ids, steps=steps, num_new_tokens=n_tokens)
    g = None
    if graph:
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream(device=DEV)
        s.wait_stream(torch.cuda.current_stream(DEV))
        with torch.cuda.graph(g, stream=s):
            m.device_step(BUCKET)
    for step in range(steps):
        m.advance_device_step(BUCKET)
        if graph:
            g.replay()
        else:
            m.device_step(BUCKET)
        torch.cuda.synchronize()
        for sid in ids:
            ref.append_tokens(sid, n_tokens)
        _check_meta(m, ref, ids, step)
        # the host's counts of the device's batch, without ending the device steps
        assert [m._seq_len(i) for i in ids] == [ref.seq_len(i) for i in ids]
        assert len(m.free_blocks) == len(ref.free_blocks)
    m.end_device_steps()
    assert m.batch_to_blocks == ref.batch_to_blocks
    assert list(m.free_blocks) == ref.free_blocks
    assert {i: m.batch_to_page_lengths[i] for i in ids} == {i: ref.batch_to_page_lengths[i] for i in ids}
    # the host path takes over where the device stopped
    for sid in ids:
        m.append_tokens(sid, 1)
        ref.append_tokens(sid, 1)
    m.free(ids[3])
    ref.free(ids[3])
    assert m.batch_to_blocks == ref.batch_to_blocks
    assert list(m.free_blocks) == ref.free_blocks
    assert m.pool_errors() == 0


def test_device_steps_raise_like_the_reference_when_the_pool_runs_dry():
    m, ref = _pair(60)
    ids = _allocate(m, ref, [31, 47, 15, 30, 14])  # pops due at steps 1, 1, 1, 2, 2 ...
    m.init_cuda_graph_buffers([BUCKET], max_indices=1024)
    ref.init_cuda_graph_buffers([BUCKET])
    m.begin_device_steps(BUCKET, ids, steps=200)
    err = None
    for step in range(200):
        try:
            for sid in ids:
                ref.append_tokens(sid, 1)
        except RuntimeError as e:
            err = e
        if err is None:
            m.advance_device_step(BUCKET)
            m.device_step(BUCKET)
            continue
        with pytest.raises(RuntimeError, match="^Not enough free blocks to append tokens$"):
            m.advance_device_step(BUCKET)
        break
    assert err is not None and str(err) == "Not enough free blocks to append tokens"
    # the same sequences were appended before the one that found the pool empty
    assert m.batch_to_blocks == ref.batch_to_blocks
    assert {i: m.batch_to_page_lengths[i] for i in ids} == {i: ref.batch_to_page_lengths[i] for i in ids}
    assert list(m.free_blocks) == ref.free_blocks
    assert m.pool_errors() == 0


def test_steps_begin_hand_over_through_the_c_abi():
    """pkv_pool_steps_begin: from a bucket's gather descriptor and kv_last_page_len, the real
    entries' rows go to the row list and their page counts and last-page lengths to the
    per-row arrays, the padding entries get row -1, the free count is written, rows outside
    the table are counted in err; a real count above the batch is refused."""
    from ecahlang_amd._lib import lib, stream_ptr
    dev = torch.device("cuda:0")
    batch, real, rows_total = 6, 4, 10
    # desc: 4 words per entry (row, column, pages, unused); entry 2 names a row outside the table
    desc = torch.tensor([[3, 0, 5, 0], [7, 0, 1, 0], [12, 0, 2, 0], [0, 0, 9, 0], [10, 0, 1, 0], [10, 1, 1, 0]],
                        dtype=torch.int32, device=dev).reshape(-1)
    last = torch.tensor([16, 1, 7, 3, 1, 1], dtype=torch.int32, device=dev)
    out_rows = torch.full((batch,), 99, dtype=torch.int32, device=dev)
    npages = torch.full((rows_total,), -5, dtype=torch.int32, device=dev)
    plen = torch.full((rows_total,), -5, dtype=torch.int32, device=dev)
    nfree = torch.zeros(1, dtype=torch.int32, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    args = (desc.data_ptr(), last.data_ptr(), batch, real, 1234, out_rows.data_ptr(), npages.data_ptr(),
            plen.data_ptr(), rows_total, nfree.data_ptr(), err.data_ptr(), stream_ptr(dev))
    assert lib().pkv_pool_steps_begin(*args) == 0
    torch.cuda.synchronize()
    assert out_rows.tolist() == [3, 7, 12, 0, -1, -1]
    want_np, want_pl = [-5] * rows_total, [-5] * rows_total
    for r, n, p in ((3, 5, 16), (7, 1, 1), (0, 9, 3)):
        want_np[r], want_pl[r] = n, p
    assert npages.tolist() == want_np and plen.tolist() == want_pl
    assert nfree.item() == 1234 and err.item() == 1
    bad = list(args)
    bad[3] = batch + 1
    assert lib().pkv_pool_steps_begin(*bad) < 0
