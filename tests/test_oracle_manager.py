"""Pins the oracle's page-pool restatement against hand-derived traces and invariants."""
import pytest
from hypothesis import given, settings, strategies as st

from oracle.manager_ref import RefKVCacheManager


def _run_trace(trace, strict):
    m = RefKVCacheManager(trace["pool"], strict_reference_q1=strict)
    for op in trace["ops"]:
        if strict and op.get("product_only"):
            break
        kind = op["op"]
        if "error" in op:
            exc = {"RuntimeError": RuntimeError, "ValueError": ValueError}[op["error"]]
            before = list(m.free_blocks)
            with pytest.raises(exc, match=op["message"]):
                getattr(m, kind)(op["id"], op["n"])
            assert m.free_blocks == before
            if "free_blocks" in op:
                assert m.free_blocks == op["free_blocks"]
            continue
        if kind in ("allocate", "append_tokens"):
            getattr(m, kind)(op["id"], op["n"])
            pages = op.get("reference_pages", op["pages"]) if strict else op["pages"]
            plen = op.get("reference_page_len", op["page_len"]) if strict else op["page_len"]
            assert m.batch_to_blocks[op["id"]] == pages, (trace["name"], op)
            assert m.batch_to_page_lengths[op["id"]] == plen, (trace["name"], op)
        elif kind == "free":
            m.free(op["id"])
            assert m.free_blocks == op["free_blocks"], (trace["name"], op)
        elif kind == "init_cuda_graph_buffers":
            m.init_cuda_graph_buffers(op["buckets"])
            assert m.padding_pages == op["padding_pages"]
        elif kind == "fill_cuda_graph_metadata":
            idx, ptr, last, pos = m.fill_cuda_graph_metadata(op["bucket"], op["ids"])
            assert (idx, ptr, last, pos) == (op["kv_indices"], op["kv_indptr"],
                                             op["kv_last_page_len"], op["positions"])
        elif kind == "get_append_metadata":
            idx, ptr, last = m.get_append_metadata(op["ids"])
            assert (idx, ptr, last) == (op["kv_indices"], op["kv_indptr"], op["kv_last_page_len"])
        else:
            raise AssertionError(kind)


def test_hand_traces(golden):
    for trace in golden("manager_traces.json")["traces"]:
        _run_trace(trace, strict=False)


def test_hand_traces_reference_q1_mode(golden):
    # the same traces under the reference's own allocate(T % 16 == 0) rule
    for trace in golden("manager_traces.json")["traces"]:
        _run_trace(trace, strict=True)


ops = st.lists(st.tuples(st.sampled_from(["alloc", "append", "free"]), st.integers(0, 5),
                         st.integers(0, 70)), max_size=60)


@settings(max_examples=200, deadline=None)
@given(ops)
def test_pool_invariants(seq):
    P = 40
    m = RefKVCacheManager(P)
    for kind, sid, n in seq:
        try:
            if kind == "alloc" and sid not in m.batch_to_blocks:
                m.allocate(sid, n)
            elif kind == "append" and sid in m.batch_to_blocks:
                m.append_tokens(sid, n)
            elif kind == "free":
                m.free(sid)
        except RuntimeError:
            pass
        live = [p for pages in m.batch_to_blocks.values() for p in pages]
        # pages are conserved and never shared
        assert len(live) == len(set(live))
        assert sorted(live + m.free_blocks) == list(range(P))
        for sid2, pages in m.batch_to_blocks.items():
            plen = m.batch_to_page_lengths[sid2]
            assert 0 <= plen <= 16
            if pages:
                assert m.seq_len(sid2) == (len(pages) - 1) * 16 + plen


def test_seq_len_tracks_token_count():
    m = RefKVCacheManager(100)
    total = 0
    m.allocate("s", 37)
    total = 37
    for n in [1, 1, 11, 16, 0, 5, 32, 1]:
        m.append_tokens("s", n)
        total += n
        assert m.seq_len("s") == total


def test_prefix_sharing_hand_trace():
    """The sharing extension on a 10-page pool, derived by hand: shared pages (a partial last
    page included), copies on write at allocate and at append, nested prefixes, and frees that
    return only the pages no other list holds."""
    m = RefKVCacheManager(10)
    assert m.allocate("p", 40) == [9, 8, 7]              # 2 full pages + 8 tokens
    assert m.allocate("a", 40, prefix="p") == [9, 8, 7]  # all of p, its partial page too
    assert m.allocate("b", 45, prefix="p") == [9, 8, 6]  # continues past p's partial page: copy
    assert m.batch_to_page_lengths["b"] == 13
    assert m.allocate("c", 20, prefix="p") == [9, 8]     # p's pages for its first 20 tokens
    m.append_tokens("c", 1)                              # into the shared page 8: copy
    assert m.batch_to_blocks["c"] == [9, 5] and m.batch_to_page_lengths["c"] == 5
    m.append_tokens("a", 8)                              # copy of 7, then the page after
    assert m.batch_to_blocks["a"] == [9, 8, 4, 3] and m.batch_to_page_lengths["a"] == 0
    assert m.cow_pairs == [(7, 6), (8, 5), (7, 4)]
    assert m.refs == {9: 4, 8: 3, 7: 1, 6: 1, 5: 1, 4: 1, 3: 1}
    assert m.shared_prefix_pages(*m.get_append_metadata(["p", "a", "b", "c"])[:2]) == [0, 2, 2, 1]
    m.free("p")                                          # only page 7 was p's alone
    assert m.free_blocks == [0, 1, 2, 7]
    assert m.allocate("d", 64, prefix="a") == [9, 8, 4, 7]  # nested: a's pages hold p's
    m.free("a")
    assert m.free_blocks == [0, 1, 2, 3]
    m.free("b")
    assert m.free_blocks == [0, 1, 2, 3, 6]
    with pytest.raises(ValueError, match="q not allocated"):
        m.allocate("e", 40, prefix="q")
    with pytest.raises(RuntimeError, match="Not enough KV cache blocks available"):
        m.allocate("e", 16 * 10, prefix="d")             # 6 pages of its own, 5 free
    m.free("c")
    m.free("d")
    assert m.free_blocks == [0, 1, 2, 3, 6, 5, 9, 8, 4, 7] and m.refs == {}
    # append with the pool empty and a copy due: the reference's exception, nothing changed
    m2 = RefKVCacheManager(2)
    m2.allocate("x", 5)
    m2.allocate("y", 5, prefix="x")
    m2.append_tokens("y", 0)                             # no token: no copy
    m2.allocate("z", 16)
    with pytest.raises(RuntimeError, match="Not enough free blocks to append tokens"):
        m2.append_tokens("x", 1)
    assert m2.batch_to_blocks == {"x": [1], "y": [1], "z": [0]} and m2.refs == {1: 2, 0: 1}


prefix_ops = st.lists(st.tuples(st.sampled_from(["alloc", "share", "share", "append", "free"]), st.integers(0, 5),
                                st.integers(0, 70)), max_size=60)


@settings(max_examples=200, deadline=None)
@given(prefix_ops)
def test_prefix_pool_invariants(seq):
    """Under random allocate / share (nested, shorter and longer than the prefix) / append /
    free: every page is either free or held, each count equals the lists that hold it, the
    counts never rise along a list (the pages a free returns are a tail), copies on write pop
    pages that were free, and lengths stay consistent."""
    P = 60
    m = RefKVCacheManager(P)
    for kind, sid, n in seq:
        try:
            if kind == "alloc" and sid not in m.batch_to_blocks:
                m.allocate(sid, n)
            elif kind == "share" and sid not in m.batch_to_blocks:
                live = sorted(m.batch_to_blocks)
                if live:
                    p = live[n % len(live)]
                    m.allocate(sid, max(0, m.seq_len(p) + n % 40 - 20), prefix=p)
            elif kind == "append" and sid in m.batch_to_blocks:
                m.append_tokens(sid, n % 20)
            elif kind == "free":
                m.free(sid)
        except RuntimeError:
            pass
        held = {}
        for b, pages in m.batch_to_blocks.items():
            for pg in pages:
                held[pg] = held.get(pg, 0) + 1
        assert held == m.refs
        assert not set(held) & set(m.free_blocks)
        assert sorted(list(held) + m.free_blocks) == list(range(P))
        for b, pages in m.batch_to_blocks.items():
            counts = [m.refs[pg] for pg in pages]
            assert counts == sorted(counts, reverse=True)
            if pages:
                assert m.seq_len(b) == (len(pages) - 1) * 16 + m.batch_to_page_lengths[b]


def test_radix_cache_hand_trace():
    """The prefix cache's rules on a hand-derived trace (block_size 4, eight pages, pops from
    the end of the free list): insert on free, match on allocate, a walk that follows its own
    cached pages, pages the tree keeps counted like a list's, eviction only of leaves no list
    holds (least recently used first, the parent after its child), and the exception when
    eviction cannot make room."""
    from oracle.manager_ref import RefRadixKVCacheManager
    m = RefRadixKVCacheManager(8, block_size=4, cache_rows=2)
    A = list(range(1, 11))
    assert m.allocate("a", 10, tokens=A) == [7, 6, 5]
    m.free("a", tokens=A)  # blocks (1..4) -> page 7 and (5..8) -> page 6 cached; page 5 freed
    assert m.free_blocks == [0, 1, 2, 3, 4, 5]
    assert m.cached_pages() == {7: [1, 2, 3, 4], 6: [1, 2, 3, 4, 5, 6, 7, 8]}
    assert m.refs == {7: 1, 6: 1}
    B = [1, 2, 3, 4, 5, 6, 7, 8, 9, 9, 9]
    assert m.allocate("b", 11, tokens=B) == [7, 6, 5]  # two pages matched, one popped
    assert m.refs == {7: 2, 6: 2, 5: 1}
    assert m.allocate("c", 6, tokens=[1, 2, 3, 4, 0, 0]) == [7, 4]
    m.free("c", tokens=[1, 2, 3, 4, 0, 0])  # follows the cached page 7; page 4 freed
    assert m.free_blocks == [0, 1, 2, 3, 4] and m.refs == {7: 2, 6: 2, 5: 1}
    assert m.allocate("d", 20) == [4, 3, 2, 1, 0]
    with pytest.raises(RuntimeError, match="Not enough free blocks to append tokens"):
        m.append_tokens("b", 2)  # nothing evictable: b holds both cached pages
    assert m.free_blocks == [] and m.evicted == []
    m.free("b", tokens=B)
    assert m.free_blocks == [5] and m.refs == {7: 1, 6: 1, 4: 1, 3: 1, 2: 1, 1: 1, 0: 1}
    assert m.allocate("e", 12) == [7, 6, 5]  # evicts page 6 (the leaf), then 7 (now a leaf)
    assert m.evicted == [6, 7] and m.cached_pages() == {} and m.free_rows == [0, 1]
    # the same tokens cached with another sequence's pages end the walk: nothing of g is kept
    m.free("e")
    m.free("d")
    X = [9, 9, 9, 9, 8, 8, 8, 8]
    f = m.allocate("f", 8, tokens=X)
    g = m.allocate("g", 8, tokens=X)
    assert f == [0, 1] and g == [2, 3]
    m.free("f", tokens=X)
    m.free("g", tokens=X)
    assert m.cached_pages() == {0: [9, 9, 9, 9], 1: X}
    assert m.free_blocks[-2:] == [2, 3]
    # least recently used first: touch f's path, then cache another path and evict one page
    h = m.allocate("h", 4, tokens=[5, 5, 5, 5])
    m.free("h", tokens=[5, 5, 5, 5])
    assert m.allocate("x", 4, tokens=X) == [0]  # touches page 0 only (one block asked for)
    m.free("x")
    assert m.evict(1) == 1 and m.evicted[-1] == 1  # page 1: untouched since f's free
    assert m.evict(1) == 1 and m.evicted[-1] == h[0]  # then h's page (older than page 0's touch)
    assert m.cached_pages() == {0: [9, 9, 9, 9]}


radix_ops = st.lists(st.tuples(st.sampled_from(["alloc", "alloc", "append", "free", "free_plain", "evict"]),
                               st.integers(0, 6), st.integers(0, 3), st.integers(0, 90)), max_size=60)


@settings(max_examples=200, deadline=None)
@given(radix_ops)
def test_radix_cache_invariants(seq):
    """Random allocates over a few shared token streams, appends, frees with and without
    tokens, evictions, under pool pressure (48 pages, 3 cache rows): every page is free, held by
    lists or kept by the tree, each count equals its lists plus the tree's hold, a matched page
    holds exactly the tokens it was matched on, and the tree's pages hold their paths."""
    from oracle.manager_ref import RefRadixKVCacheManager
    P, bs = 48, 16
    m = RefRadixKVCacheManager(P, cache_rows=3)
    streams = [[(s * 7 + i // 40) % 5 for i in range(400)] for s in range(4)]
    content = {}  # page -> token ids written into it
    toks = {}
    for kind, sid, stream, n in seq:
        try:
            if kind == "alloc" and sid not in m.batch_to_blocks:
                ids = streams[stream][: 5 + n * 3]
                T = len(ids)
                k = len(m.match(ids, T))
                pages = m.allocate(sid, T, tokens=ids)
                for i, pg in enumerate(pages):
                    block = tuple(ids[i * bs:(i + 1) * bs])
                    if i < k:
                        assert content[pg] == block, "a matched page holds other tokens"
                    else:
                        content[pg] = block
                toks[sid] = ids
            elif kind == "append" and sid in m.batch_to_blocks:
                m.append_tokens(sid, n % 20)
                toks[sid] = toks[sid] + [99] * (n % 20)
                L = m.seq_len(sid)
                for i, pg in enumerate(m.batch_to_blocks[sid]):
                    content[pg] = tuple(toks[sid][i * bs:min((i + 1) * bs, L)])
            elif kind in ("free", "free_plain") and sid in m.batch_to_blocks:
                m.free(sid, tokens=toks[sid] if kind == "free" else None)
                del toks[sid]
            elif kind == "evict":
                m.evict(n % 4)
        except RuntimeError:
            pass
        tree = m.cached_pages()
        held = {}
        for pages in m.batch_to_blocks.values():
            for pg in pages:
                held[pg] = held.get(pg, 0) + 1
        for pg in tree:
            held[pg] = held.get(pg, 0) + 1
        assert held == m.refs
        assert not set(held) & set(m.free_blocks)
        assert sorted(list(held) + m.free_blocks) == list(range(P))
        for pg, path in tree.items():
            assert content[pg] == tuple(path[-bs:]), "a cached page holds other tokens"
        assert len(m.free_rows) + len(m.row_nodes) == 3
