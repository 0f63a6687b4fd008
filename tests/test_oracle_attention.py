"""Pins the oracle's attention restatement (CPU only).

Each check is chosen so that a plausible mistake fails it: a wrong GQA head mapping, a
dropped scale, a wrong causal offset, reading past last_page_len or the wrong page order.
"""
import math

import numpy as np
import pytest
import torch

from oracle import kv_ref
from ecahlang_amd import workloads


def _pool(rng, P, ps, H, D, scale=1.0):
    return (rng.standard_normal((P, 2, ps, H, D)) * scale).astype(np.float32)


def test_hand_computed_two_tokens():
    # one sequence, 2 tokens, Hq = Hkv = 1, D = 2, scale 1/sqrt(2)
    cache = np.full((1, 2, 4, 1, 2), np.nan, np.float32)
    cache[0, 0, 0, 0] = [1.0, 0.0]   # k0
    cache[0, 0, 1, 0] = [0.0, 1.0]   # k1
    cache[0, 1, 0, 0] = [2.0, 4.0]   # v0
    cache[0, 1, 1, 0] = [6.0, 8.0]   # v1
    q = np.array([[[math.sqrt(2) * math.log(3.0), 0.0]]], np.float32)
    # scores: q.k0 / sqrt2 = ln 3, q.k1 / sqrt2 = 0 -> weights 3/4, 1/4
    o = kv_ref.decode(q, cache, [0, 1], [0], [2], 4)
    np.testing.assert_allclose(o[0, 0], [0.75 * 2 + 0.25 * 6, 0.75 * 4 + 0.25 * 8], rtol=1e-6)


def test_single_token_returns_v0():
    rng = np.random.default_rng(2)
    cache = _pool(rng, 3, 16, 2, 8)
    q = rng.standard_normal((1, 4, 8)).astype(np.float32)
    o = kv_ref.decode(q, cache, [0, 1], [2], [1], 16)
    for h in range(4):
        np.testing.assert_array_equal(o[0, h], cache[2, 1, 0, h // 2].astype(np.float64))


def test_constant_v_and_identical_keys():
    rng = np.random.default_rng(3)
    P, ps, H, D = 4, 16, 1, 8
    cache = _pool(rng, P, ps, H, D)
    cache[:, 1] = 0.625  # constant V -> output exactly V whatever the weights
    q = rng.standard_normal((1, 2, D)).astype(np.float32)
    o = kv_ref.decode(q, cache, [0, 3], [1, 3, 0], [5], ps)
    np.testing.assert_allclose(o, 0.625, rtol=0, atol=1e-12)
    cache = _pool(rng, P, ps, H, D)
    cache[:, 0] = cache[0, 0, 0]  # identical keys -> uniform weights -> mean of V rows
    o = kv_ref.decode(q, cache, [0, 2], [2, 0], [7], ps)
    vrows = np.concatenate([cache[2, 1], cache[0, 1, :7]]).astype(np.float64)
    np.testing.assert_allclose(o[0, 0], vrows.mean(axis=0)[0], rtol=1e-10)


def test_page_permutation_invariance():
    rng = np.random.default_rng(4)
    P, ps, H, D = 8, 4, 2, 4
    cache = _pool(rng, P, ps, H, D)
    q = rng.standard_normal((1, 4, D)).astype(np.float32)
    o1 = kv_ref.decode(q, cache, [0, 3], [6, 1, 3], [2], ps)
    perm = np.array([5, 7, 0, 2, 1, 4, 3, 6])  # physical page moved: new id of old page i
    cache2 = np.empty_like(cache)
    cache2[perm] = cache
    o2 = kv_ref.decode(q, cache2, [0, 3], [perm[6], perm[1], perm[3]], [2], ps)
    np.testing.assert_array_equal(o1, o2)


def test_gqa_mapping_equals_duplicated_heads():
    rng = np.random.default_rng(5)
    P, ps, Hkv, D, g = 4, 4, 2, 8, 3
    cache = _pool(rng, P, ps, Hkv, D)
    q = rng.standard_normal((1, Hkv * g, D)).astype(np.float32)
    o = kv_ref.decode(q, cache, [0, 2], [3, 1], [3], ps)
    dup = np.repeat(cache, g, axis=3)  # MHA cache: head h holds kv head h // g
    o_mha = kv_ref.decode(q, dup, [0, 2], [3, 1], [3], ps)
    np.testing.assert_array_equal(o, o_mha)


def test_scale_argument():
    rng = np.random.default_rng(6)
    cache = _pool(rng, 2, 4, 1, 4)
    q = rng.standard_normal((1, 1, 4)).astype(np.float32)
    a = kv_ref.decode(q, cache, [0, 2], [0, 1], [4], 4, sm_scale=0.3)
    b = kv_ref.decode(q * np.float32(0.6), cache, [0, 2], [0, 1], [4], 4, sm_scale=0.5)
    np.testing.assert_allclose(a, b, rtol=1e-6)


def test_empty_sequence_is_zero():
    cache = np.zeros((2, 2, 4, 1, 2), np.float32)
    q = np.ones((2, 1, 2), np.float32)
    o = kv_ref.decode(q, cache, [0, 0, 1], [1], [0, 0], 4)
    assert not o.any()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_decode_agrees_with_torch_sdpa(dtype):
    wb = workloads.build_batch([5, 33, 16, 70], [1] * 4, 8, 2, 64, dtype, seed=11, scale=0.7)
    # write the new tokens in with the oracle append, then compare the two restatements
    iv = torch.int16 if dtype != torch.float32 else torch.int32
    raw = wb.cache.view(iv).numpy()
    kraw, vraw = wb.k_new.view(iv).numpy(), wb.v_new.view(iv).numpy()
    raw2 = kv_ref.append(raw, kraw, vraw, wb.batch_indices.numpy(), wb.positions.numpy(),
                         wb.indices.numpy(), wb.indptr.numpy(), wb.ps)
    cache = torch.from_numpy(raw2).view(dtype)
    ref_np = kv_ref.decode(wb.q.float().numpy(), cache.float().numpy(), wb.indptr.numpy(),
                           wb.indices.numpy(), wb.last.numpy(), wb.ps)
    ref_t = kv_ref.sdpa_decode(wb.q, cache, wb.indptr, wb.indices, wb.last, wb.ps)
    np.testing.assert_allclose(ref_t.numpy(), ref_np, rtol=1e-5, atol=1e-5)
    assert np.isfinite(ref_np).all()  # NaN-poisoned slots never reached


def test_prefill_square_causal_matches_sdpa_is_causal():
    # qo_len == kv_len: bottom-right and top-left causal coincide -> torch's is_causal
    rng = np.random.default_rng(7)
    P, ps, Hkv, D, L, Hq = 3, 4, 2, 8, 10, 4
    cache = _pool(rng, P, ps, Hkv, D)
    q = rng.standard_normal((L, Hq, D)).astype(np.float32)
    o = kv_ref.prefill(q, [0, L], cache, [0, 3], [2, 0, 1], [2], ps, causal=True)
    kk, vv = kv_ref.gather(cache, [2, 0, 1], [0, 3], [2], 0, ps)
    qt = torch.from_numpy(q).transpose(0, 1)[None]
    kt = torch.from_numpy(np.ascontiguousarray(kk)).repeat_interleave(2, 1).transpose(0, 1)[None]
    vt = torch.from_numpy(np.ascontiguousarray(vv)).repeat_interleave(2, 1).transpose(0, 1)[None]
    ref = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, is_causal=True)[0].transpose(0, 1)
    np.testing.assert_allclose(o, ref.numpy(), rtol=1e-5, atol=1e-5)


def test_prefill_last_row_equals_decode_and_bottom_right_offset():
    rng = np.random.default_rng(8)
    P, ps, Hkv, D, Hq = 4, 4, 1, 8, 2
    cache = _pool(rng, P, ps, Hkv, D)
    indptr, indices, last = [0, 4], [3, 0, 2, 1], [3]  # kv_len 15
    q = rng.standard_normal((5, Hq, D)).astype(np.float32)  # last 5 tokens of the sequence
    o = kv_ref.prefill(q, [0, 5], cache, indptr, indices, last, ps, causal=True)
    # row i sees keys [0, 11 + i): its output equals decode over a sequence truncated there
    for i in range(5):
        n = 11 + i
        npg = (n + ps - 1) // ps
        d = kv_ref.decode(q[i:i + 1], cache, [0, npg], indices[:npg], [(n - 1) % ps + 1], ps)
        np.testing.assert_allclose(o[i], d[0], rtol=1e-12, atol=1e-12)
    onc = kv_ref.prefill(q, [0, 5], cache, indptr, indices, last, ps, causal=False)
    d = kv_ref.decode(q, cache, [0, 4, 8, 12, 16, 20], indices * 5, last * 5, ps)
    np.testing.assert_allclose(onc, d, rtol=1e-12, atol=1e-12)


def test_sdpa_prefill_agrees_with_numpy_prefill():
    wb = workloads.build_batch([40, 17, 64], [8, 17, 3], 8, 2, 64, torch.float32, seed=12)
    raw = wb.cache.view(torch.int32).numpy()
    raw2 = kv_ref.append(raw, wb.k_new.view(torch.int32).numpy(), wb.v_new.view(torch.int32).numpy(),
                         wb.batch_indices.numpy(), wb.positions.numpy(), wb.indices.numpy(),
                         wb.indptr.numpy(), wb.ps)
    cache = torch.from_numpy(raw2).view(torch.float32)
    o_np = kv_ref.prefill(wb.q.numpy(), wb.append_indptr.numpy(), cache.numpy(), wb.indptr.numpy(),
                          wb.indices.numpy(), wb.last.numpy(), wb.ps, causal=True)
    o_t = kv_ref.sdpa_prefill(wb.q, wb.append_indptr, cache, wb.indptr, wb.indices, wb.last, wb.ps)
    np.testing.assert_allclose(o_t.numpy(), o_np, rtol=1e-5, atol=1e-5)
    assert np.isfinite(o_np).all()
