"""HIP kernels through the C ABI against the CPU oracle (run on the MI355X with -m gpu).

Bar: bit-exact for metadata and the append (whole NaN-poisoned pool compared as integers);
attention within atol 2e-3 / rtol 1e-2 for fp16/bf16 and 1e-5 for fp32 against the float64
gather-then-softmax oracle computed from the same input bits.
"""
import numpy as np
import pytest
import torch

from ecahlang_amd import ops, workloads
from ecahlang_amd.wrappers import (BatchDecodeWithPagedKVCacheWrapper,
                                   BatchPrefillWithPagedKVCacheWrapper)
from oracle import kv_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float32: dict(atol=1e-5, rtol=1e-5), torch.float16: dict(atol=2e-3, rtol=1e-2),
       torch.bfloat16: dict(atol=2e-3, rtol=1e-2)}


def _iv(dtype):
    return torch.int32 if dtype == torch.float32 else torch.int16


def _bits(t):
    return t.view(_iv(t.dtype)).cpu().numpy()


def _oracle_appended(wb):
    """numpy bit view of the cache after the batch's append, and its float64 values."""
    raw = kv_ref.append(_bits(wb.cache), _bits(wb.k_new), _bits(wb.v_new),
                        wb.batch_indices.numpy(), wb.positions.numpy(), wb.indices.numpy(),
                        wb.indptr.numpy(), wb.ps)
    vals = torch.from_numpy(raw).view(wb.dtype).float().numpy()
    return raw, vals


def _append_dev(dv):
    ops.append_paged_kv_cache(dv.k_new, dv.v_new, dv.batch_indices, dv.positions, dv.cache,
                              dv.indices, dv.indptr, dv.last)


def _decode_dev(dv, q, force_valu=False, num_ctas=None, cache=None, indices=None,
                deterministic=True):
    ws = torch.empty(128 << 20, dtype=torch.uint8, device=DEV)
    w = BatchDecodeWithPagedKVCacheWrapper(ws, "NHD")
    w.plan(dv.indptr, dv.indices if indices is None else indices, dv.last, dv.hq, dv.hkv, dv.d,
           dv.ps, pos_encoding_mode="NONE", q_data_type=dv.dtype, num_ctas=num_ctas,
           deterministic=deterministic)
    return w.run(q, dv.cache if cache is None else cache, force_valu=force_valu)


# ---------------------------------------------------------------- metadata

def test_seq_lens_golden(golden):
    for case in golden("metadata_kat.json")["seq_lens"]:
        ip = torch.tensor(case["indptr"], dtype=torch.int32, device=DEV)
        la = torch.tensor(case["last"], dtype=torch.int32, device=DEV)
        got = ops.get_seq_lens(ip, la, case["page_size"])
        assert got.cpu().tolist() == case["expected"], case["derivation"]


def test_batch_indices_positions_golden(golden):
    for case in golden("metadata_kat.json")["batch_indices_positions"]:
        ai = torch.tensor(case["append_indptr"], dtype=torch.int32, device=DEV)
        sl = torch.tensor(case["seq_lens"], dtype=torch.int32, device=DEV)
        bidx, pos = ops.get_batch_indices_positions(ai, sl, ai[-1])
        assert bidx.cpu().tolist() == case["batch_indices"], case["derivation"]
        assert pos.cpu().tolist() == case["positions"], case["derivation"]


def test_metadata_random_vs_oracle():
    g = torch.Generator().manual_seed(5)
    B = 300
    npages = torch.randint(0, 40, (B,), generator=g)
    indptr = torch.zeros(B + 1, dtype=torch.int32)
    indptr[1:] = torch.cumsum(npages, 0)
    last = torch.randint(0, 17, (B,), generator=g).to(torch.int32)
    sl = ops.get_seq_lens(indptr.to(DEV), last.to(DEV), 16).cpu().numpy()
    assert np.array_equal(sl, kv_ref.seq_lens(indptr.numpy(), last.numpy(), 16))
    n = torch.randint(0, 5, (B,), generator=g)
    ai = torch.zeros(B + 1, dtype=torch.int32)
    ai[1:] = torch.cumsum(n, 0)
    s = torch.from_numpy(sl) + 4
    bidx, pos = ops.get_batch_indices_positions(ai.to(DEV), s.to(DEV), int(ai[-1]))
    rb, rp = kv_ref.batch_indices_positions(ai.numpy(), s.numpy(), int(ai[-1]))
    assert np.array_equal(bidx.cpu().numpy(), rb) and np.array_equal(pos.cpu().numpy(), rp)


# ---------------------------------------------------------------- append

APPEND_CASES = {
    "llama32_1b_fp32": lambda: workloads.llama32_1b_decode(),
    "qwen25_3b_fp16_b64": lambda: workloads.qwen25_3b_decode(batch=64, lo=16, hi=300),
    "llama31_8b_bf16_b8": lambda: workloads.build_batch([33, 1, 16, 17, 100, 2, 64, 5], [1] * 8,
                                                        32, 8, 128, torch.bfloat16, 44),
    "prefill_chunks_fp16": lambda: workloads.qwen25_3b_prefill(requests=4, chunk=64, max_prefix=300),
    # rows of 32 and 64 chunks of 16 bytes: 2 and 1 tokens per wave, token counts that leave
    # a partial last round
    "hkv1_d128_fp16_37tok": lambda: workloads.build_batch([40, 3, 17], [30, 3, 4], 8, 1, 128, torch.float16, 45),
    "hkv4_d64_bf16_23tok": lambda: workloads.build_batch([9, 50, 16], [6, 16, 1], 16, 4, 64, torch.bfloat16, 46),
    # rows of 16 and 8 chunks: 4 and 8 tokens per wave
    "hkv1_d64_fp16_29tok": lambda: workloads.build_batch([30, 7, 12], [20, 7, 2], 4, 1, 64, torch.float16, 47),
    "hkv1_d32_bf16_45tok": lambda: workloads.build_batch([64, 21], [40, 5], 2, 1, 32, torch.bfloat16, 48),
}


@pytest.mark.parametrize("name", list(APPEND_CASES))
def test_append_bit_exact_whole_pool(name):
    wb = APPEND_CASES[name]()
    print(f"case {name}: nnz={wb.k_new.shape[0]} pages={wb.num_pages}", flush=True)
    dv = wb.to(DEV)
    _append_dev(dv)
    torch.cuda.synchronize()
    want, _ = _oracle_appended(wb)
    assert np.array_equal(_bits(dv.cache), want)


def test_append_strided_hf_layout_and_misaligned():
    wb = workloads.qwen25_3b_prefill(requests=3, chunk=40, max_prefix=100)
    want, _ = _oracle_appended(wb)
    dv = wb.to(DEV)
    nnz, H, D = dv.k_new.shape
    # HF hands the hook [1, H, L, D]; the hook passes key[0].transpose(0, 1) (strided)
    k_hf = dv.k_new.transpose(0, 1).contiguous()[None]
    v_hf = dv.v_new.transpose(0, 1).contiguous()[None]
    k, v = k_hf[0].transpose(0, 1), v_hf[0].transpose(0, 1)
    assert not k.is_contiguous()
    c1 = dv.cache.clone()
    ops.append_paged_kv_cache(k, v, dv.batch_indices, dv.positions, c1, dv.indices, dv.indptr, dv.last)
    # 2-byte misaligned rows take the element-wise path
    buf = torch.empty(2 * nnz * H * D + 1, dtype=dv.dtype, device=DEV)
    km = buf[1:1 + nnz * H * D].view(nnz, H, D)
    vm = buf[1 + nnz * H * D:].view(nnz, H, D)
    km.copy_(dv.k_new)
    vm.copy_(dv.v_new)
    c2 = dv.cache.clone()
    ops.append_paged_kv_cache(km, vm, dv.batch_indices, dv.positions, c2, dv.indices, dv.indptr, dv.last)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(c1), want)
    assert np.array_equal(_bits(c2), want)


def test_append_split_kv_tuple_form():
    wb = workloads.build_batch([20, 3], [4, 3], 4, 2, 64, torch.float16, 9)
    want, _ = _oracle_appended(wb)
    dv = wb.to(DEV)
    kc = dv.cache[:, 0].contiguous()
    vc = dv.cache[:, 1].contiguous()
    ops.append_paged_kv_cache(dv.k_new, dv.v_new, dv.batch_indices, dv.positions, (kc, vc),
                              dv.indices, dv.indptr, dv.last)
    torch.cuda.synchronize()
    got = torch.stack([kc, vc], 1)
    assert np.array_equal(_bits(got), want)


def test_append_out_of_range_metadata_is_skipped_and_counted():
    wb = workloads.build_batch([20, 3], [2, 1], 4, 2, 64, torch.float16, 10)
    dv = wb.to(DEV)
    before = _bits(dv.cache)
    pos = dv.positions.clone()
    pos[0] = 10_000  # beyond the sequence's pages
    pos[1] = -3      # negative (what the reference's allocate(T % 16 == 0) quirk produces)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    ops.append_paged_kv_cache(dv.k_new[:2], dv.v_new[:2], dv.batch_indices, pos, dv.cache,
                              dv.indices, dv.indptr, dv.last, err_count=err)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(dv.cache), before)
    assert err.item() == 2 * 2 * 2  # one count per token, K or V, and head


def _index_put_append(cache, k, v, page, slot, keep):
    """The append as torch's index_put on the device: the expected pool for large batches."""
    want = cache.clone()
    want[page[keep], 0, slot[keep]] = k[keep]
    want[page[keep], 1, slot[keep]] = v[keep]
    return want


@pytest.mark.parametrize("by_slot", [False, True])
def test_append_many_rounds_per_wave_with_bad_tokens(by_slot):
    """40960 tokens (several pipelined rounds per wave at one workgroup per 8th of a CU's
    slots), with tokens whose metadata is out of range scattered through the batch: every
    other token lands bit for bit, the bad ones are skipped and counted."""
    wb = workloads.build_batch([512] * 80, [512] * 80, 2, 2, 128, torch.float16, 49, fill_old=False)
    dv = wb.to(DEV)
    nnz, ps = dv.k_new.shape[0], wb.ps
    bidx, pos = dv.batch_indices.clone(), dv.positions.clone()
    page = dv.indices.long()[dv.indptr.long()[bidx.long()] + pos.long() // ps]
    slot = pos.long() % ps
    keep = torch.ones(nnz, dtype=torch.bool, device=DEV)
    bad = [0, 777, 12345, 40959]
    keep[bad] = False
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    want = _index_put_append(dv.cache, dv.k_new, dv.v_new, page, slot, keep)
    if by_slot:
        slots = (page * ps + slot).to(torch.int32)
        slots[0], slots[777], slots[12345], slots[40959] = -1, wb.num_pages * ps, -16, 2 ** 31 - 1
        ops.append_paged_kv_cache_slots(dv.k_new, dv.v_new, slots, dv.cache, err_count=err)
    else:
        pos[0] = 10 ** 6      # past the sequence's pages
        bidx[777] = wb.batch  # no such sequence
        bidx[12345] = -1
        pos[40959] = -2
        ops.append_paged_kv_cache(dv.k_new, dv.v_new, bidx, pos, dv.cache, dv.indices, dv.indptr, dv.last,
                                  err_count=err)
    torch.cuda.synchronize()
    assert torch.equal(dv.cache.view(torch.int16), want.view(torch.int16))
    assert err.item() == len(bad) * 2 * 2


def _host_slots(wb):
    ind, ptr, ps = wb.indices.tolist(), wb.indptr.tolist(), wb.ps
    return torch.tensor([ind[ptr[b] + p // ps] * ps + p % ps
                         for b, p in zip(wb.batch_indices.tolist(), wb.positions.tolist())], dtype=torch.int32)


@pytest.mark.parametrize("name", list(APPEND_CASES))
def test_append_by_slot_bit_exact_whole_pool(name):
    wb = APPEND_CASES[name]()
    print(f"case {name}: nnz={wb.k_new.shape[0]} pages={wb.num_pages}", flush=True)
    want, _ = _oracle_appended(wb)
    dv = wb.to(DEV)
    ops.append_paged_kv_cache_slots(dv.k_new, dv.v_new, _host_slots(wb).to(DEV), dv.cache)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(dv.cache), want)


def test_append_by_slot_misaligned_rows_and_bad_slots():
    wb = workloads.build_batch([20, 3, 40], [2, 1, 3], 4, 2, 64, torch.float16, 12)
    want, _ = _oracle_appended(wb)
    dv = wb.to(DEV)
    nnz, H, D = dv.k_new.shape
    buf = torch.empty(2 * nnz * H * D + 1, dtype=dv.dtype, device=DEV)  # 2-byte misaligned rows
    km = buf[1:1 + nnz * H * D].view(nnz, H, D)
    vm = buf[1 + nnz * H * D:].view(nnz, H, D)
    km.copy_(dv.k_new)
    vm.copy_(dv.v_new)
    c = dv.cache.clone()
    ops.append_paged_kv_cache_slots(km, vm, _host_slots(wb).to(DEV), c)
    # slots that are negative or past the pool are skipped and counted (one count per token,
    # K or V, and head)
    bad = torch.tensor([-1, wb.num_pages * wb.ps, 2 ** 31 - 1, -16, 0, 0], dtype=torch.int32, device=DEV)[:nnz]
    bad[4:] = -5
    before = _bits(dv.cache)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    ops.append_paged_kv_cache_slots(dv.k_new, dv.v_new, bad, dv.cache, err_count=err)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(c), want)
    assert np.array_equal(_bits(dv.cache), before)
    assert err.item() == nnz * 2 * H


# ---------------------------------------------------------------- decode

DECODE_CASES = {
    "llama32_1b_fp32": lambda: workloads.llama32_1b_decode(),
    "qwen25_3b_fp16_b64": lambda: workloads.qwen25_3b_decode(),
    "llama31_8b_bf16_b16": lambda: workloads.llama31_8b_decode(batch=16, lo=100, hi=3000),
    "mha_fp16_d64": lambda: workloads.build_batch([5, 70, 300, 1], [1] * 4, 4, 4, 64, torch.float16, 21),
    "g16_bf16_d64": lambda: workloads.build_batch([50, 17, 900], [1] * 3, 16, 1, 64, torch.bfloat16, 22),
    # one KV head at head_dim 128: eight waves share the head
    "mqa_fp16_d128": lambda: workloads.build_batch([700, 33, 1200, 16], [1] * 4, 8, 1, 128, torch.float16, 23),
    # three KV heads: two waves per head, two waves idle
    "gqa3_bf16_d128": lambda: workloads.build_batch([90, 640, 5], [1] * 3, 12, 3, 128, torch.bfloat16, 24),
    # two KV heads at head_dim 64: four waves per head
    "gqa2_fp16_d64": lambda: workloads.build_batch([260, 31, 77, 1000], [1] * 4, 8, 2, 64, torch.float16, 25),
}


@pytest.mark.parametrize("name", list(DECODE_CASES))
@pytest.mark.parametrize("force_valu", [False, True])
def test_decode_matches_oracle(name, force_valu):
    wb = DECODE_CASES[name]()
    print(f"case {name} force_valu={force_valu}: B={wb.batch} pages={int(wb.indptr[-1])}", flush=True)
    dv = wb.to(DEV)
    _append_dev(dv)
    o = _decode_dev(dv, dv.q, force_valu=force_valu)
    torch.cuda.synchronize()
    _, vals = _oracle_appended(wb)
    ref = kv_ref.decode(wb.q.float().numpy(), vals, wb.indptr.numpy(), wb.indices.numpy(),
                        wb.last.numpy(), wb.ps)
    np.testing.assert_allclose(o.float().cpu().numpy(), ref, **TOL[wb.dtype])


@pytest.mark.parametrize("name", [n for n in DECODE_CASES if "fp32" not in n])
def test_decode_dynamic_pages_match_oracle(name):
    # waves take pages on demand: same result within tolerance, any partition of the pages
    wb = DECODE_CASES[name]()
    dv = wb.to(DEV)
    _append_dev(dv)
    _, vals = _oracle_appended(wb)
    ref = kv_ref.decode(wb.q.float().numpy(), vals, wb.indptr.numpy(), wb.indices.numpy(),
                        wb.last.numpy(), wb.ps)
    for ctas in (None, 7):
        o = _decode_dev(dv, dv.q, num_ctas=ctas, deterministic=False)
        torch.cuda.synchronize()
        np.testing.assert_allclose(o.float().cpu().numpy(), ref, **TOL[wb.dtype])


@pytest.mark.parametrize("force_valu", [False, True])
def test_decode_pages_before_first_sequence(force_valu):
    # kv_indptr[0] > 0: the leading page-list entries belong to no sequence
    wb = workloads.build_batch([40, 300, 17], [1] * 3, 16, 2, 128, torch.float16, 41)
    dv = wb.to(DEV)
    _append_dev(dv)
    _, vals = _oracle_appended(wb)
    ref = kv_ref.decode(wb.q.float().numpy(), vals, wb.indptr.numpy(), wb.indices.numpy(),
                        wb.last.numpy(), wb.ps)
    lead = 37
    # valid pages holding other sequences' data: counting them would change the result
    pick = torch.randint(0, wb.indices.numel(), (lead,), generator=torch.Generator().manual_seed(2))
    junk = wb.indices[pick]
    indices = torch.cat([junk, wb.indices]).to(DEV)
    indptr = (wb.indptr + lead).to(DEV)
    for ctas in (1, 5, 64):
        ws = torch.empty(64 << 20, dtype=torch.uint8, device=DEV)
        w = BatchDecodeWithPagedKVCacheWrapper(ws)
        w.plan(indptr, indices, dv.last, dv.hq, dv.hkv, dv.d, 16, q_data_type=dv.dtype,
               num_ctas=ctas)
        o = w.run(dv.q, dv.cache, force_valu=force_valu)
        torch.cuda.synchronize()
        np.testing.assert_allclose(o.float().cpu().numpy(), ref, **TOL[wb.dtype],
                                   err_msg=f"num_ctas={ctas}")


@pytest.mark.parametrize("ctas", [1, 3, 17, 256, 1000])
def test_decode_split_counts(ctas):
    wb = workloads.qwen25_3b_decode(batch=12, lo=1, hi=700, seed=77)
    dv = wb.to(DEV)
    _append_dev(dv)
    _, vals = _oracle_appended(wb)
    ref = kv_ref.decode(wb.q.float().numpy(), vals, wb.indptr.numpy(), wb.indices.numpy(),
                        wb.last.numpy(), wb.ps)
    for rep in range(2):  # the second call checks the counters were left at zero
        o = _decode_dev(dv, dv.q, num_ctas=ctas)
        torch.cuda.synchronize()
        np.testing.assert_allclose(o.float().cpu().numpy(), ref, **TOL[wb.dtype])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_decode_edge_sequences(dtype):
    # lengths 1, 16 (full page), 17, 32 as [full, full, empty trailing page], and an empty row
    lens = [1, 16, 17, 32, 5]
    wb = workloads.build_batch(lens, [1] * 5, 8, 2, 128, dtype, 31)
    dv = wb.to(DEV)
    _append_dev(dv)
    torch.cuda.synchronize()
    # rebuild the table: seq 3 gets an extra page with last_page_len 0, seq 4 becomes empty
    ip = wb.indptr.tolist()
    idx = wb.indices.tolist()
    spare = [p for p in range(wb.num_pages) if p not in set(idx)][0]
    rows = [idx[ip[b]:ip[b + 1]] for b in range(5)]
    rows[3] = rows[3] + [spare]
    rows[4] = []
    last = [1, 16, 1, 0, 0]
    indptr = torch.tensor(np.concatenate([[0], np.cumsum([len(r) for r in rows])]), dtype=torch.int32)
    indices = torch.tensor(sum(rows, []), dtype=torch.int32)
    lastt = torch.tensor(last, dtype=torch.int32)
    _, vals = _oracle_appended(wb)
    ref = kv_ref.decode(wb.q.float().numpy(), vals, indptr.numpy(), indices.numpy(), lastt.numpy(), 16)
    for ctas in (1, 4, 64):
        ws = torch.empty(64 << 20, dtype=torch.uint8, device=DEV)
        w = BatchDecodeWithPagedKVCacheWrapper(ws)
        w.plan(indptr.to(DEV), indices.to(DEV), lastt.to(DEV), 8, 2, 128, 16, q_data_type=dtype,
               num_ctas=ctas)
        o = w.run(dv.q, dv.cache)
        torch.cuda.synchronize()
        got = o.float().cpu().numpy()
        np.testing.assert_allclose(got, ref, **TOL[dtype])
        assert not got[4].any()  # empty sequence -> zeros
        # single token: softmax weight exactly 1 -> output is exactly v0
        v0 = vals[int(indices[0]), 1, 0]  # [Hkv, D]
        np.testing.assert_array_equal(got[0], np.repeat(v0, 4, axis=0))


def test_decode_page_permutation_bitwise_invariant():
    wb = workloads.qwen25_3b_decode(batch=8, lo=30, hi=400, seed=5)
    dv = wb.to(DEV)
    _append_dev(dv)
    o1 = _decode_dev(dv, dv.q, num_ctas=16)
    perm = torch.randperm(wb.num_pages, generator=torch.Generator().manual_seed(1)).to(DEV)
    cache2 = torch.empty_like(dv.cache)
    cache2[perm] = dv.cache
    idx2 = perm[dv.indices.long()].to(torch.int32)
    o2 = _decode_dev(dv, dv.q, num_ctas=16, cache=cache2, indices=idx2)
    torch.cuda.synchronize()
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))


def test_decode_strided_q_and_out():
    wb = workloads.qwen25_3b_decode(batch=6, lo=10, hi=200, seed=6)
    dv = wb.to(DEV)
    _append_dev(dv)
    ref = _decode_dev(dv, dv.q.contiguous())
    qs = dv.q.transpose(0, 1).contiguous().transpose(0, 1)  # [B, Hq, D], strides (D, B*D, 1)
    o = _decode_dev(dv, qs)
    torch.cuda.synchronize()
    assert torch.equal(o, ref)


def test_decode_graph_replays_match_eager():
    wb = workloads.qwen25_3b_decode(batch=32, lo=100, hi=1500, seed=8)
    dv = wb.to(DEV)
    _append_dev(dv)
    ws = torch.empty(128 << 20, dtype=torch.uint8, device=DEV)
    w = BatchDecodeWithPagedKVCacheWrapper(ws)
    w.plan(dv.indptr, dv.indices, dv.last, dv.hq, dv.hkv, dv.d, 16, q_data_type=torch.float16)
    q = dv.q.clone()
    out = torch.empty_like(q)
    w.run(q, dv.cache, out=out)  # warm-up outside capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            w.run(q, dv.cache, out=out)
    torch.cuda.synchronize()
    gen = torch.Generator(device=DEV).manual_seed(3)
    for rep in range(4):
        q.copy_(torch.randn(q.shape, generator=gen, device=DEV, dtype=torch.float32).to(q.dtype))
        eager = w.run(q, dv.cache)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep}"


# ---------------------------------------------------------------- prefill

PREFILL_CASES = {
    "qwen25_3b_fp16": lambda: workloads.qwen25_3b_prefill(requests=4, chunk=96, max_prefix=700),
    "bf16_ragged": lambda: workloads.build_batch([40, 200, 1, 64], [40, 17, 1, 3], 32, 8, 128,
                                                 torch.bfloat16, 51),
    "fp32_d64": lambda: workloads.build_batch([30, 90], [12, 30], 32, 8, 64, torch.float32, 52),
    # matrix-core shapes: MHA at head_dim 64, a 16-head group, a query tile cut short
    "mha_fp16_d64": lambda: workloads.build_batch([300, 70, 513], [300, 5, 100], 8, 8, 64, torch.float16, 53),
    "g16_bf16_d64": lambda: workloads.build_batch([33, 600], [33, 40], 16, 1, 64, torch.bfloat16, 54),
    # a request with no new tokens between two that have some (qo_indptr repeats a value)
    "zero_chunk_bf16": lambda: workloads.build_batch([40, 200, 1, 64], [40, 0, 1, 3], 32, 8, 128,
                                                     torch.bfloat16, 55),
}


@pytest.mark.parametrize("name", list(PREFILL_CASES))
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_matches_oracle(name, causal):
    wb = PREFILL_CASES[name]()
    print(f"case {name} causal={causal}: nnz={wb.q.shape[0]}", flush=True)
    dv = wb.to(DEV)
    _append_dev(dv)
    ws = torch.empty(64 << 20, dtype=torch.uint8, device=DEV)
    w = BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
    w.plan(dv.append_indptr, dv.indptr, dv.indices, dv.last, dv.hq, dv.hkv, dv.d, dv.ps,
           causal=causal, q_data_type=dv.dtype)
    o = w.run(dv.q, dv.cache)
    torch.cuda.synchronize()
    _, vals = _oracle_appended(wb)
    ref = kv_ref.prefill(wb.q.float().numpy(), wb.append_indptr.numpy(), vals, wb.indptr.numpy(),
                         wb.indices.numpy(), wb.last.numpy(), wb.ps, causal=causal)
    np.testing.assert_allclose(o.float().cpu().numpy(), ref, **TOL[wb.dtype])


@pytest.mark.parametrize("causal", [True, False])
def test_prefill_chunked_qwen_full_size(causal):
    # C3 at full size: 8 requests x 512-token chunks onto prefixes U[0, 8192]; the key ranges are
    # cut into chunks whose partials the merge kernel folds, and the matrix-core result also
    # agrees with the vector-ALU kernel
    wb = workloads.qwen25_3b_prefill()
    print(f"C3 causal={causal}: nnz={wb.q.shape[0]} kv={sum(wb.kv_len)}", flush=True)
    dv = wb.to(DEV)
    _append_dev(dv)
    ws = torch.empty(128 << 20, dtype=torch.uint8, device=DEV)
    w = BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
    w.plan(dv.append_indptr, dv.indptr, dv.indices, dv.last, dv.hq, dv.hkv, dv.d, dv.ps,
           causal=causal, q_data_type=dv.dtype)
    assert w._mfma and w._n_groups > 0  # split groups exercised
    o = w.run(dv.q, dv.cache)
    ov = w.run(dv.q, dv.cache, force_valu=True)
    torch.cuda.synchronize()
    _, vals = _oracle_appended(wb)
    ref = kv_ref.prefill(wb.q.float().numpy(), wb.append_indptr.numpy(), vals, wb.indptr.numpy(),
                         wb.indices.numpy(), wb.last.numpy(), wb.ps, causal=causal)
    np.testing.assert_allclose(o.float().cpu().numpy(), ref, **TOL[wb.dtype])
    np.testing.assert_allclose(ov.float().cpu().numpy(), ref, **TOL[wb.dtype])


def test_read_probe_reads_in_bounds_and_checks_arguments():
    """pkv_probe_stream_read (the bench's achievable-bandwidth probe): slices of any size over
    any workgroup count, including more workgroups than 16-byte words, run and leave the guard
    words around the buffer alone; bad arguments are refused before anything is enqueued."""
    from ecahlang_amd._lib import lib, stream_ptr
    dev = torch.device("cuda:0")
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    for words, blocks in ((1, 1), (7, 3), (1000, 256), (4099, 2048), (65536, 256)):
        buf = torch.full((words * 4 + 8,), 0x5A5A5A5A, dtype=torch.int32, device=dev)
        inner = buf[4: 4 + words * 4]
        assert lib().pkv_probe_stream_read(inner.data_ptr(), words * 16, blocks, sink.data_ptr(),
                                           stream_ptr(dev)) == 0
        torch.cuda.synchronize()
        assert int(sink.item()) in (0, 1)
        assert bool((buf == 0x5A5A5A5A).all())
    x = torch.zeros(64, dtype=torch.int32, device=dev)
    s = stream_ptr(dev)
    assert lib().pkv_probe_stream_read(x.data_ptr(), 24, 4, sink.data_ptr(), s) < 0      # not 16-byte words
    assert lib().pkv_probe_stream_read(x.data_ptr() + 4, 32, 4, sink.data_ptr(), s) < 0  # misaligned
    assert lib().pkv_probe_stream_read(x.data_ptr(), 64, 0, sink.data_ptr(), s) < 0      # no workgroups
    assert lib().pkv_probe_stream_read(x.data_ptr(), 64, 4, 0, s) < 0                    # no sink
