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
    """The prefix extension on a 10-page pool, derived by hand: shared pages are the
    prefix's full pages, never popped or pushed by the sequences that share them."""
    m = RefKVCacheManager(10)
    assert m.allocate("p", 40) == [9, 8, 7]           # 2 full pages + 8 tokens
    assert m.allocate("a", 40, prefix="p") == [9, 8, 6]  # shares [9, 8]; its own page 6
    assert m.allocate("b", 32, prefix="p") == [9, 8]     # nothing of its own yet
    assert m.batch_to_page_lengths["b"] == 16
    m.append_tokens("b", 1)                              # 17th token of its last page: pops 5
    assert m.batch_to_blocks["b"] == [9, 8, 5] and m.batch_to_page_lengths["b"] == 1
    with pytest.raises(RuntimeError, match="p is the shared prefix of 2 live sequences"):
        m.free("p")
    with pytest.raises(ValueError, match="q not allocated"):
        m.allocate("c", 40, prefix="q")
    with pytest.raises(ValueError, match="shorter than its shared prefix"):
        m.allocate("c", 31, prefix="p")
    with pytest.raises(RuntimeError, match="Not enough KV cache blocks available"):
        m.allocate("c", 32 + 16 * 6, prefix="p")  # 6 own pages, 5 free
    assert m.free_blocks == [0, 1, 2, 3, 4]
    m.free("a")
    assert m.free_blocks == [0, 1, 2, 3, 4, 6]
    m.free("b")
    m.free("p")
    assert m.free_blocks == [0, 1, 2, 3, 4, 6, 5, 9, 8, 7]
    # a prefix whose last page is partial shares only its full pages
    m.allocate("p2", 20)                                  # pops 7, 8
    assert m.allocate("d", 20, prefix="p2") == [7, 9]


prefix_ops = st.lists(st.tuples(st.sampled_from(["alloc", "share", "append", "free"]), st.integers(0, 5),
                                st.integers(0, 70)), max_size=60)


@settings(max_examples=200, deadline=None)
@given(prefix_ops)
def test_prefix_pool_invariants(seq):
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
                    m.allocate(sid, m.seq_len(p) + n % 20, prefix=p)
            elif kind == "append" and sid in m.batch_to_blocks:
                m.append_tokens(sid, n)
            elif kind == "free":
                m.free(sid)
        except RuntimeError:
            pass
        own = {b: pages[m.shared.get(b, (None, 0))[1]:] for b, pages in m.batch_to_blocks.items()}
        flat = [p for pages in own.values() for p in pages]
        # own pages are disjoint and conserved with the free list
        assert len(flat) == len(set(flat))
        assert sorted(flat + m.free_blocks) == list(range(P))
        for b, (p, k) in m.shared.items():
            # shared pages are the prefix's own leading pages, and the prefix is live
            assert m.batch_to_blocks[b][:k] == m.batch_to_blocks[p][:k]
            assert m.refs[p] >= 1
        for b, pages in m.batch_to_blocks.items():
            if pages:
                assert m.seq_len(b) == (len(pages) - 1) * 16 + m.batch_to_page_lengths[b]
