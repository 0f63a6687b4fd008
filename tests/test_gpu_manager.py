"""Device page pool (ecahlang_amd.manager.AutoKVCacheManager) against the oracle's list
restatement of the reference manager: page ids, page lengths and page tables bit-exact, the
same exceptions with the pool untouched, and an end-to-end step (allocate, append through the
cached metadata, decode) against the attention oracle."""
import random

import numpy as np
import pytest
import torch

from ecahlang_amd.manager import AutoKVCacheManager
from ecahlang_amd.wrappers import BatchDecodeWithPagedKVCacheWrapper
from oracle import kv_ref
from oracle.manager_ref import RefKVCacheManager

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _pool(pages, strict=False, stride=4, layers=1, hkv=1, d=64, dtype=torch.float16):
    es = torch.tensor([], dtype=dtype).element_size()
    per_page = 16 * hkv * d * es * 2
    m = AutoKVCacheManager(layers, hkv, d, total_gpu_mem_bytes=pages * per_page * layers, mem_utilization=1.0,
                           dtype=dtype, device=DEV, max_pages_per_seq=stride, strict_reference_q1=strict)
    assert m.max_blocks == pages
    return m


def _same_state(dev, ref):
    assert list(dev.free_blocks) == ref.free_blocks
    assert len(dev.free_blocks) == len(ref.free_blocks)
    assert dev.batch_to_blocks == ref.batch_to_blocks
    assert dev.batch_to_page_lengths == ref.batch_to_page_lengths
    assert dev.batch_to_seq_len == ref.batch_to_seq_len
    assert dev.free_seq_lens == ref.free_seq_lens


def _run_trace(trace, strict):
    m = _pool(trace["pool"], strict)
    for op in trace["ops"]:
        if strict and op.get("product_only"):
            break
        kind = op["op"]
        if "error" in op:
            exc = {"RuntimeError": RuntimeError, "ValueError": ValueError}[op["error"]]
            before = list(m.free_blocks)
            with pytest.raises(exc, match=op["message"]):
                getattr(m, kind)(op["id"], op["n"])
            assert list(m.free_blocks) == before
            if "free_blocks" in op:
                assert list(m.free_blocks) == op["free_blocks"]
            continue
        if kind in ("allocate", "append_tokens"):
            got = getattr(m, kind)(op["id"], op["n"])
            pages = op.get("reference_pages", op["pages"]) if strict else op["pages"]
            plen = op.get("reference_page_len", op["page_len"]) if strict else op["page_len"]
            if kind == "allocate":
                assert list(got) == pages
            assert m.batch_to_blocks[op["id"]] == pages, (trace["name"], op)
            assert m.batch_to_page_lengths[op["id"]] == plen, (trace["name"], op)
        elif kind == "free":
            m.free(op["id"])
            assert list(m.free_blocks) == op["free_blocks"], (trace["name"], op)
        elif kind == "init_cuda_graph_buffers":
            m.init_cuda_graph_buffers(op["buckets"])
            assert m.padding_pages == op["padding_pages"]
        elif kind == "fill_cuda_graph_metadata":
            b = op["bucket"]
            m.fill_cuda_graph_metadata(b, op["ids"])
            n = len(op["kv_indices"])
            assert m._cg_kv_indices[b][:n].tolist() == op["kv_indices"]
            assert m._cg_kv_indptr[b].tolist() == op["kv_indptr"]
            assert m._cg_kv_last_page_len[b].tolist() == op["kv_last_page_len"]
            assert m._cg_positions[b].tolist() == op["positions"]
        elif kind == "get_append_metadata":
            idx, ptr, last = m.get_append_metadata(op["ids"])
            assert (idx.tolist(), ptr.tolist(), last.tolist()) == (
                op["kv_indices"], op["kv_indptr"], op["kv_last_page_len"])
        else:
            raise AssertionError(kind)
    assert m.pool_errors() == 0


@pytest.mark.parametrize("strict", [False, True])
def test_hand_traces(golden, strict):
    for trace in golden("manager_traces.json")["traces"]:
        print(f"trace {trace['name']} strict={strict}", flush=True)
        _run_trace(trace, strict)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_random_operations_match_oracle(seed):
    # small pages-per-row start (stride 4) so page-table growth is exercised too
    rng = random.Random(seed)
    P = 60
    dev, ref = _pool(P), RefKVCacheManager(P)
    ids = list(range(8))
    for step in range(250):
        kind = rng.choice(["alloc", "alloc", "append", "append", "append", "free", "meta"])
        sid = rng.choice(ids)
        n = rng.choice([0, 1, 1, 1, 2, 15, 16, 17, 31, 33, 70])
        if kind == "alloc" and sid not in ref.batch_to_blocks:
            calls = ("allocate", (sid, n))
        elif kind == "append" and sid in ref.batch_to_blocks:
            calls = ("append_tokens", (sid, n))
        elif kind == "append":
            calls = ("append_tokens", (sid, n))  # unknown id: ValueError in both
        elif kind == "free":
            calls = ("free", (sid,))
        else:
            live = [s for s in ids if s in ref.batch_to_blocks]
            rng.shuffle(live)
            idx, ptr, last = dev.get_append_metadata(live)
            assert (idx.tolist(), ptr.tolist(), last.tolist()) == tuple(map(list, ref.get_append_metadata(live)))
            continue
        name, args = calls
        err_ref = err_dev = None
        try:
            getattr(ref, name)(*args)
        except (RuntimeError, ValueError) as e:
            err_ref = (type(e), str(e))
        try:
            getattr(dev, name)(*args)
        except (RuntimeError, ValueError) as e:
            err_dev = (type(e), str(e))
        assert err_dev == err_ref, (step, name, args)
        if step % 10 == 0 or err_ref:
            _same_state(dev, ref)
    _same_state(dev, ref)
    assert dev.pool_errors() == 0


def test_graph_buckets_match_oracle():
    P = 200
    dev, ref = _pool(P), RefKVCacheManager(P)
    for m in (dev, ref):
        m.init_cuda_graph_buffers([1, 2, 4, 8])
    assert dev.padding_pages == ref.padding_pages
    for i, t in enumerate([5, 16, 33, 100, 1]):
        dev.allocate(i, t)
        ref.allocate(i, t)
    for i in range(5):
        dev.append_tokens(i, 1)
        ref.append_tokens(i, 1)
    for bucket, real in ((8, [3, 0, 4, 1, 2]), (4, [2, 1]), (1, [4])):
        dev.fill_cuda_graph_metadata(bucket, real)
        idx, ptr, last, pos = ref.fill_cuda_graph_metadata(bucket, real)
        assert dev._cg_kv_indices[bucket][: len(idx)].tolist() == idx
        assert dev._cg_kv_indptr[bucket].tolist() == ptr
        assert dev._cg_kv_last_page_len[bucket].tolist() == last
        assert dev._cg_positions[bucket].tolist() == pos
        # each row's append slot: the page its position selects through the table, and the
        # slot inside it (what append_paged_kv_cache_cuda_graph writes to)
        slots = [idx[ptr[r] + p // 16] * 16 + p % 16 for r, p in enumerate(pos)]
        assert dev._cg_slots[bucket].tolist() == slots
    # a sequence that holds no page (allocate(b, 0)) gets no slot: its position points before
    # its pages, and the graph-bucket append skips its row, as the reference's append does
    dev.allocate(9, 0)
    ref.allocate(9, 0)
    dev.fill_cuda_graph_metadata(4, [9, 3])
    idx, ptr, last, pos = ref.fill_cuda_graph_metadata(4, [9, 3])
    assert dev._cg_positions[4].tolist() == pos and pos[0] < 0
    assert dev._cg_slots[4].tolist() == [-1] + [idx[ptr[r] + p // 16] * 16 + p % 16 for r, p in enumerate(pos)][1:]
    with pytest.raises(RuntimeError, match="Not enough free blocks for 400 padding pages"):
        dev.init_cuda_graph_buffers([400])
    assert dev.pool_errors() == 0


def test_end_to_end_prefill_then_decode_steps():
    """allocate -> prepare_append_metadata -> cached append per layer -> decode plan/run,
    for a prefill and three decode steps; every step checked against the oracle on the K/V
    the test appended (tracked on the host)."""
    L, hkv, hq, d, dt = 2, 2, 16, 128, torch.float16
    P = 400
    m = _pool(P, layers=L, hkv=hkv, d=d, stride=8)
    gen = torch.Generator().manual_seed(11)
    lens = [40, 1, 16, 250, 97]
    ids = [f"r{i}" for i in range(len(lens))]
    hist = {i: [[], []] for i in ids}  # per sequence: K rows, V rows (per layer stacked)

    def append_step(new):  # new: tokens per sequence this step
        append_indptr = torch.tensor(np.concatenate([[0], np.cumsum(new)]), dtype=torch.int32, device=DEV)
        m.prepare_append_metadata(ids, append_indptr)
        nnz = int(sum(new))
        k = (torch.randn(L, nnz, hkv, d, generator=gen) * 0.5).to(dt)
        v = (torch.randn(L, nnz, hkv, d, generator=gen) * 0.5).to(dt)
        for layer in range(L):
            m.append_paged_kv_cache_cached(k[layer].to(DEV), v[layer].to(DEV), layer)
        off = 0
        for sid, n in zip(ids, new):
            hist[sid][0].append(k[:, off:off + n])
            hist[sid][1].append(v[:, off:off + n])
            off += n

    for sid, n in zip(ids, lens):
        m.allocate(sid, n)
    append_step(lens)
    ws = torch.empty(64 << 20, dtype=torch.uint8, device=DEV)
    w = BatchDecodeWithPagedKVCacheWrapper(ws, "NHD")
    for step in range(4):
        if step:
            for sid in ids:
                m.append_tokens(sid, 1)
            append_step([1] * len(ids))
        w.plan(m._cached_kv_indptr, m._cached_kv_indices, m._cached_kv_last_page_len, hq, hkv, d, 16,
               pos_encoding_mode="NONE", q_data_type=dt)
        q = (torch.randn(len(ids), hq, d, generator=gen) * 0.5).to(dt)
        for layer in range(L):
            out = w.run(q.to(DEV), m.kv_cache[layer]).float().cpu().numpy()
            for b, sid in enumerate(ids):
                kk = torch.cat(hist[sid][0], 1)[layer].float().numpy()  # [len, hkv, d]
                vv = torch.cat(hist[sid][1], 1)[layer].float().numpy()
                ref = kv_ref._attend(q[b:b + 1].float().numpy().astype(np.float64), kk, vv,
                                     [kk.shape[0]], d ** -0.5)[0]
                np.testing.assert_allclose(out[b], ref, atol=2e-3, rtol=1e-2,
                                           err_msg=f"step {step} layer {layer} seq {sid}")
    assert m.pool_errors() == 0


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_prefix_sharing_matches_oracle(seed):
    """Page sharing (allocate(..., prefix=), nested, shorter and longer than the prefix, with
    copies on write at allocate and at append) against the oracle's restatement: page lists,
    free stack and exceptions under random allocate / share / append / free; the graph
    metadata's shared-page hint against the lists the oracle holds."""
    rng = random.Random(100 + seed)
    P = 120
    dev, ref = _pool(P, stride=16), RefKVCacheManager(P)
    dev.init_cuda_graph_buffers([16], max_indices=4096)
    ref.init_cuda_graph_buffers([16])
    ids = list(range(12))
    for step in range(400):
        kind = rng.choice(["alloc", "share", "share", "share", "append", "append", "free", "meta", "hint"])
        sid = rng.choice(ids)
        n = rng.choice([0, 1, 2, 15, 16, 17, 33, 70])
        live = sorted(s for s in ids if s in ref.batch_to_blocks)
        if kind == "meta":
            idx, ptr, last = dev.get_append_metadata(live)
            assert (idx.tolist(), ptr.tolist(), last.tolist()) == tuple(map(list, ref.get_append_metadata(live)))
            continue
        if kind == "hint":
            rows = rng.sample(live, min(len(live), 16))
            rows.sort(key=lambda i: ref.batch_to_blocks[i][:1])  # sharers next to each other
            dev.fill_cuda_graph_metadata(16, rows)
            idx, ptr, _, _ = ref.fill_cuda_graph_metadata(16, rows)
            assert dev._cg_kv_shared[16].tolist() == ref.shared_prefix_pages(idx, ptr), step
            continue
        if kind == "share":
            if not live or sid in ref.batch_to_blocks:
                continue
            p = rng.choice(live + [99])  # 99: not allocated (ValueError in both)
            tokens = (ref.seq_len(p) if p in ref.batch_to_blocks else 0) + rng.choice([-20, -5, -1, 0, 0, 1, 7, 20])
            name, args, kw = "allocate", (sid, max(tokens, 0)), {"prefix": p}
        elif kind == "alloc" and sid not in ref.batch_to_blocks:
            name, args, kw = "allocate", (sid, n), {}
        elif kind == "append":
            name, args, kw = "append_tokens", (sid, n), {}
        elif kind == "free":
            name, args, kw = "free", (sid,), {}
        else:
            continue
        err_ref = err_dev = None
        try:
            getattr(ref, name)(*args, **kw)
        except (RuntimeError, ValueError) as e:
            err_ref = (type(e), str(e))
        try:
            getattr(dev, name)(*args, **kw)
        except (RuntimeError, ValueError) as e:
            err_dev = (type(e), str(e))
        assert err_dev == err_ref, (step, name, args, kw)
        if step % 10 == 0 or err_ref:
            _same_state(dev, ref)
    _same_state(dev, ref)
    assert len(ref.cow_pairs) > 5  # the sequence did exercise copies on write
    assert dev.pool_errors() == 0


def test_copy_on_write_copies_every_layer_of_the_page():
    """A sequence that shares a partial last page and then appends gets a private copy: a new
    page id whose K/V, in every layer, equal the shared page's, while the shared page and its
    other holder are untouched; a sequence allocated past a shared partial page copies it at
    allocate; freeing the sharers returns the pages only they held."""
    L, hkv, d = 3, 2, 64
    m, ref = _pool(40, layers=L, hkv=hkv, d=d), RefKVCacheManager(40)
    gen = torch.Generator().manual_seed(5)
    m.kv_cache.copy_(torch.randn(m.kv_cache.shape, generator=gen).to(m.kv_cache.dtype))
    before = m.kv_cache.clone()
    for mm in (m, ref):
        mm.allocate("p", 40)           # 3 pages, the last holds 8 tokens
        mm.allocate("a", 40, prefix="p")
        mm.allocate("b", 45, prefix="p")  # continues past p's partial page: copied at allocate
    for mm in (m, ref):
        mm.append_tokens("a", 1)          # into the shared page: copied first
    _same_state(m, ref)
    torch.cuda.synchronize()
    pa, pb, pp = m.batch_to_blocks["a"], m.batch_to_blocks["b"], m.batch_to_blocks["p"]
    assert pa[:2] == pp[:2] == pb[:2] and len({pa[2], pb[2], pp[2]}) == 3
    for layer in range(L):
        for copy in (pa[2], pb[2]):
            assert torch.equal(m.kv_cache[layer, copy].view(torch.int16), before[layer, pp[2]].view(torch.int16))
    # every page but the two copies holds what it held before
    others = [x for x in range(40) if x not in (pa[2], pb[2])]
    assert torch.equal(m.kv_cache[:, others].view(torch.int16), before[:, others].view(torch.int16))
    for mm in (m, ref):
        mm.free("p")
        mm.free("a")
    _same_state(m, ref)
    assert m.pool_errors() == 0


def test_device_steps_on_a_shared_last_page():
    """begin_device_steps gives each row whose new tokens would go into a shared page its copy
    first (in row order, as each row's first append would), then the steps run on the device:
    page tables against the oracle doing the same copies and appends."""
    m, ref = _pool(200, stride=8), RefKVCacheManager(200)
    m.init_cuda_graph_buffers([8])
    ref.init_cuda_graph_buffers([8])
    for mm in (m, ref):
        mm.allocate("p", 37)
        mm.allocate("x", 37, prefix="p")
        mm.allocate("y", 20, prefix="p")
        mm.allocate("z", 64, prefix="p")
    ids = ["p", "x", "y", "z"]
    m.begin_device_steps(8, ids, steps=20)
    ref.make_last_pages_private(ids)
    for step in range(20):
        m.advance_device_step(8)
        m.device_step(8)
        for sid in ids:
            ref.append_tokens(sid, 1)
        torch.cuda.synchronize()
        idx, ptr, last, pos = ref.fill_cuda_graph_metadata(8, ids)
        assert m._cg_kv_indptr[8].tolist() == ptr, step
        assert m._cg_kv_indices[8][:len(idx)].tolist() == idx, step
        assert m._cg_kv_last_page_len[8].tolist() == last, step
    m.end_device_steps()
    _same_state(m, ref)
    assert m.pool_errors() == 0


def test_uncached_append_matches_oracle_and_cached_path():
    """manager.py:167-185, the uncached append (metadata, seq lens, positions and the scatter in
    one call): bitwise over the whole NaN-poisoned pool against the oracle's scatter on the
    oracle manager's page tables, and against the cached path on a second pool."""
    P, hkv, d, dt = 90, 2, 64, torch.float16
    gen = torch.Generator().manual_seed(21)
    lens = [5, 16, 33, 1, 70]       # allocated tokens; the last `new` of each are this call's
    new = [5, 3, 33, 1, 2]
    ids = [f"u{i}" for i in range(len(lens))]
    pools = [_pool(P, hkv=hkv, d=d, stride=8) for _ in range(2)]
    ref = RefKVCacheManager(P)
    for m in pools:
        m.kv_cache.view(torch.int16).fill_(0x7E00)  # NaN in fp16: untouched slots stay NaN
    for sid, n in zip(ids, lens):
        for m in pools:
            m.allocate(sid, n)
        ref.allocate(sid, n)
    nnz = sum(new)
    k = (torch.randn(nnz, hkv, d, generator=gen) * 0.5).to(dt)
    v = (torch.randn(nnz, hkv, d, generator=gen) * 0.5).to(dt)
    append_indptr = torch.tensor(np.concatenate([[0], np.cumsum(new)]), dtype=torch.int32, device=DEV)
    pools[0].append_paged_kv_cache(ids, k.to(DEV), v.to(DEV), append_indptr, 0)
    pools[1].prepare_append_metadata(ids, append_indptr)
    pools[1].append_paged_kv_cache_cached(k.to(DEV), v.to(DEV), 0)
    torch.cuda.synchronize()
    idx, ptr, last = ref.get_append_metadata(ids)
    sl = kv_ref.seq_lens(ptr, last, 16)
    bidx, pos = kv_ref.batch_indices_positions(append_indptr.cpu().numpy(), sl, nnz)
    want = kv_ref.append(np.full(pools[0].kv_cache[0].shape, 0x7E00, dtype=np.int16), k.view(torch.int16).numpy(),
                         v.view(torch.int16).numpy(), bidx, pos, np.asarray(idx), np.asarray(ptr), 16)
    got = [m.kv_cache[0].view(torch.int16).cpu().numpy() for m in pools]
    assert np.array_equal(got[0], want)
    assert np.array_equal(got[1], want)
    assert all(m.pool_errors() == 0 for m in pools)


def test_default_pool_sizing_from_free_device_memory():
    """manager.py:38-49: without total_gpu_mem_bytes the pool is sized from the device's free
    memory: max_blocks = int(free * mem_utilization) // (layers * 16 * Hkv * D * es * 2)."""
    L, hkv, d, vocab, util = 2, 2, 64, 64, 0.002
    # the constructor's first allocation (the penalty table) must come from torch's cache, so
    # that the free memory it reads is the one read here
    torch.ones(128, vocab, dtype=torch.float16, device=DEV)
    torch.cuda.synchronize()
    free = torch.cuda.mem_get_info(DEV.index or 0)[0]
    m = AutoKVCacheManager(L, hkv, d, vocab_size=vocab, dtype=torch.float16, device=DEV, mem_utilization=util)
    per_block = 16 * hkv * d * 2 * 2
    assert m.max_blocks == int(free * util) // (L * per_block)
    assert m.kv_cache.shape == (L, m.max_blocks, 2, 16, hkv, d)
    assert len(m.free_blocks) == m.max_blocks
    # the pool hands out its last pages first, as the reference's free list does
    assert list(m.allocate("a", 40)) == [m.max_blocks - 1, m.max_blocks - 2, m.max_blocks - 3]
    m.free("a")
    assert m.pool_errors() == 0


def test_metadata_staging_refuses_graph_capture():
    """Staging host arrays cannot be recorded into a graph (no pinned allocation during capture,
    and a recorded copy would re-read its buffer at every replay): the call raises before
    anything is enqueued, and the pool is unchanged and usable afterwards."""
    m = _pool(64, stride=8)
    m.allocate(0, 40)
    m.allocate(1, 20)
    want = [t.clone() for t in m.get_append_metadata([0, 1])]
    m.allocate(2, 33)  # a queued pop, flushed by the next staging call
    torch.cuda.synchronize()
    s = torch.cuda.Stream(device=DEV)
    g = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="cannot be recorded into a graph"):
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                m.get_append_metadata([0, 1])
    got = m.get_append_metadata([0, 1])
    for a, b in zip(got, want):
        assert torch.equal(a, b)
    ref = RefKVCacheManager(m.max_blocks)
    for i, n in ((0, 40), (1, 20), (2, 33)):
        ref.allocate(i, n)
    assert m.batch_to_blocks[2] == ref.batch_to_blocks[2]
    assert list(m.free_blocks) == ref.free_blocks
    assert m.pool_errors() == 0


def test_long_operation_queue_matches_oracle():
    """Over a thousand queued pops and pushes applied by one flush (the device stages them a
    chunk of 1024 at a time): the same pages as the oracle's in-order lists."""
    rng = random.Random(7)
    P = 60
    dev, ref = _pool(P), RefKVCacheManager(P)
    queued = 0
    while queued < 1300:
        sid = rng.randrange(8)
        if sid in ref.batch_to_blocks:
            dev.free(sid)
            ref.free(sid)
            queued += 1
        else:
            n = rng.choice([1, 15, 16, 17, 33, 48])
            try:
                ref.allocate(sid, n)
            except RuntimeError:
                with pytest.raises(RuntimeError):
                    dev.allocate(sid, n)
                continue
            dev.allocate(sid, n)
            queued += 1
    assert len(dev._ops) > 1024
    _same_state(dev, ref)
    assert dev.pool_errors() == 0


def test_mask_penalty_rows_reset_on_allocate():
    """manager.py:56, 110: allocate sets the sequence slot's mask_penalty row back to 1.  The
    resets of several allocations are applied together: at the next flush of the pool (seen
    through a tensor taken before the allocations) or at the next read of the attribute."""
    m = AutoKVCacheManager(1, 1, 64, vocab_size=96, total_gpu_mem_bytes=64 * 16 * 64 * 2 * 2,
                           mem_utilization=1.0, dtype=torch.float16, device=DEV, max_pages_per_seq=8)
    t = m.mask_penalty
    t.fill_(0.5)
    m.allocate("a", 20)
    m.allocate("b", 0)
    m.get_append_metadata(["a", "b"])  # a flush
    slots = [m.batch_to_seq_len["a"], m.batch_to_seq_len["b"]]
    want = torch.full_like(t, 0.5)
    want[slots] = 1.0
    assert torch.equal(t, want)
    t[slots] = 0.25
    m.free("a")
    m.allocate("c", 5)
    m.allocate("d", 40)
    got = m.mask_penalty  # a read, no flush
    assert got is t
    for s in (m.batch_to_seq_len["c"], m.batch_to_seq_len["d"]):
        want[s] = 1.0
    want[m.batch_to_seq_len["b"]] = 0.25
    if m.batch_to_seq_len["c"] != slots[0] and m.batch_to_seq_len["d"] != slots[0]:
        want[slots[0]] = 0.25
    assert torch.equal(got, want)
    assert m.pool_errors() == 0
