"""Pins the oracle's metadata and append restatements (CPU only)."""
import numpy as np
import pytest

from oracle import kv_ref


def test_seq_lens_known_answers(golden):
    for case in golden("metadata_kat.json")["seq_lens"]:
        got = kv_ref.seq_lens(case["indptr"], case["last"], case["page_size"])
        assert got.tolist() == case["expected"], case["derivation"]


def test_batch_indices_positions_known_answers(golden):
    for case in golden("metadata_kat.json")["batch_indices_positions"]:
        bidx, pos = kv_ref.batch_indices_positions(case["append_indptr"], case["seq_lens"], case["nnz"])
        assert bidx.tolist() == case["batch_indices"], case["derivation"]
        assert pos.tolist() == case["positions"], case["derivation"]


def test_positions_end_at_seq_len():
    # Invariant: each request's appended positions are the last n_b slots of its sequence.
    rng = np.random.default_rng(0)
    n = rng.integers(0, 9, size=20)
    sl = n + rng.integers(0, 50, size=20)
    ai = np.concatenate([[0], np.cumsum(n)])
    bidx, pos = kv_ref.batch_indices_positions(ai, sl, int(ai[-1]))
    for b in range(20):
        sel = pos[bidx == b]
        assert sel.tolist() == list(range(sl[b] - n[b], sl[b]))


def test_append_matches_brute_force_elementwise():
    rng = np.random.default_rng(1)
    P, ps, H, D = 6, 4, 2, 3
    cache = rng.integers(-1000, 1000, size=(P, 2, ps, H, D)).astype(np.int16)
    indptr = [0, 2, 3]
    indices = [4, 1, 5]
    # seq 0 holds 6 tokens (pages 4,1), seq 1 holds 3 (page 5); append 2 + 1 tokens
    bidx = [0, 0, 1]
    pos = [4, 5, 2]
    k = rng.integers(-1000, 1000, size=(3, H, D)).astype(np.int16)
    v = rng.integers(-1000, 1000, size=(3, H, D)).astype(np.int16)
    got = kv_ref.append(cache, k, v, bidx, pos, indices, indptr, ps)
    want = cache.copy()
    # brute force with the NHD element formula written out for each element
    flat = want.reshape(-1)
    for i in range(3):
        page = indices[indptr[bidx[i]] + pos[i] // ps]
        slot = pos[i] % ps
        for h in range(H):
            for d in range(D):
                flat[(((page * 2 + 0) * ps + slot) * H + h) * D + d] = k[i, h, d]
                flat[(((page * 2 + 1) * ps + slot) * H + h) * D + d] = v[i, h, d]
    assert np.array_equal(got, want)
    # untouched pages are bit-identical
    assert np.array_equal(got[[0, 2, 3]], cache[[0, 2, 3]])


def test_gather_respects_page_order_and_last_len():
    P, ps, H, D = 5, 2, 1, 1
    cache = np.arange(P * 2 * ps * H * D, dtype=np.float32).reshape(P, 2, ps, H, D)
    k, v = kv_ref.gather(cache, [3, 0, 2], [0, 3], [1], 0, ps)
    # pages 3,0,2 -> K rows: page3 slots 0,1; page0 slots 0,1; page2 slot 0 (last_len 1)
    assert k[:, 0, 0].tolist() == [12.0, 13.0, 0.0, 1.0, 8.0]
    assert v[:, 0, 0].tolist() == [14.0, 15.0, 2.0, 3.0, 10.0]
