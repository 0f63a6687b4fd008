"""The decode schedule pkv_decode_plan writes on the device, read back and checked with no
tolerance (tests/sched_check.py: every page of every sequence exactly once and in order, valid
rows, append marks, part numbering and disjoint slots, the range heads) for the
page tables of the benchmark workloads and for edge tables.  The decode reads exactly this
schedule, so these checks pin its index work directly rather than through attention outputs."""
import numpy as np
import pytest
import torch

import sched_check as sc
from ecahlang_amd import workloads
from ecahlang_amd.wrappers import BatchDecodeWithPagedKVCacheWrapper
from test_sched_check import CASES, _table

pytestmark = pytest.mark.gpu
DEV = "cuda"
PS = 16


def _plan_check(indptr, indices, last, hq, hkv, d, dtype, ctas=None, hint=None, num_indices=None,
                ws_bytes=128 << 20):
    indptr = np.asarray(indptr, dtype=np.int64)
    indices = np.asarray(indices, dtype=np.int64)
    last = np.asarray(last, dtype=np.int64)
    B = len(last)
    n_idx = len(indices) if num_indices is None else num_indices
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    w = BatchDecodeWithPagedKVCacheWrapper(ws, "NHD")
    ip = torch.tensor(indptr, dtype=torch.int32, device=DEV)
    idx = torch.tensor(np.clip(indices[:n_idx], -2**31, 2**31 - 1), dtype=torch.int32, device=DEV)
    lt = torch.tensor(last, dtype=torch.int32, device=DEV)
    sh = None if hint is None else torch.tensor(hint, dtype=torch.int32, device=DEV)
    w.plan(ip, idx, lt, hq, hkv, d, PS, q_data_type=dtype, num_ctas=ctas, kv_shared_pages=sh)
    assert w._mfma
    torch.cuda.synchronize()
    lay = sc.layout(B, hq, d, w._ctas, n_idx, ws_bytes)
    s = sc.parse(ws.cpu().numpy(), lay, B)
    return sc.check_plain(s, indptr, indices, last, n_idx, PS, hint=hint is not None)


@pytest.mark.parametrize("ctas", [None, 16, 3, 1000])
def test_schedule_of_qwen25_3b_b64_decode(ctas):
    """The headline decode's page table (Qwen2.5-3B, B=64, context U[512, 4096])."""
    lens = workloads.qwen25_3b_lengths()
    pool = int(np.ceil(1.25 * sum((L + 15) // 16 for L in lens)))
    ip, idx, lt = workloads.paged_table(lens, pool, seed=1002)
    out = _plan_check(ip.numpy(), idx.numpy(), lt.numpy(), 16, 2, 128, torch.float16, ctas=ctas)
    print(f"C2 ctas={ctas}: {out}", flush=True)
    assert out["appends"] == 64


@pytest.mark.parametrize("ctas", [None, 64])
def test_schedule_of_llama31_8b_long_context(ctas):
    """The long-context decode's page table (Llama-3.1-8B, B=128, ~73k pages in a 20 GB pool)."""
    lens = workloads.llama31_8b_lengths()
    ip, idx, lt = workloads.paged_table(lens, workloads.LLAMA31_8B_POOL_PAGES, seed=1004)
    out = _plan_check(ip.numpy(), idx.numpy(), lt.numpy(), 32, 8, 128, torch.bfloat16, ctas=ctas)
    print(f"C4 ctas={ctas}: {out}", flush=True)
    assert out["appends"] == 128 and out["split"] > 0


def _shared_prefix_table(rng, B=128, prefix_pages=128, lo=64, hi=1024, steps=0):
    """Every sequence's page list starts with the same prefix pages, then pages of its own
    (the 36-layer step's tables); hint[b] = prefix_pages for b >= 1."""
    lens = rng.integers(lo, hi + 1, size=B) + steps
    own = [(int(L) + 15) // 16 for L in lens]
    perm = rng.permutation(prefix_pages + sum(own) + 64)
    pre = perm[:prefix_pages]
    rows, k = [], prefix_pages
    for n in own:
        rows.append(np.concatenate([pre, perm[k:k + n]]))
        k += n
    indptr = np.concatenate([[0], np.cumsum([len(r) for r in rows])])
    last = np.array([(int(L) - 1) % 16 + 1 for L in lens])
    hint = np.array([0] + [prefix_pages] * (B - 1))
    return indptr, np.concatenate(rows), last, hint


@pytest.mark.parametrize("hinted", [True, False])
def test_schedule_of_the_shared_prefix_step(hinted):
    """The 36-layer step's tables (B=128, a 128-page prefix in every table, own suffixes of
    U[64, 1024] tokens), with and without the shared-prefix hint."""
    rng = np.random.default_rng(1005)
    ip, idx, lt, hint = _shared_prefix_table(rng)
    out = _plan_check(ip, idx, lt, 16, 2, 128, torch.float16, hint=hint if hinted else None)
    print(f"C5 hint={hinted}: {out}", flush=True)


@pytest.mark.parametrize("k", range(len(CASES)))
@pytest.mark.parametrize("geom", [(16, 2, 128, torch.float16), (32, 8, 128, torch.bfloat16),
                                  (32, 8, 64, torch.float16), (16, 1, 128, torch.bfloat16)])
def test_schedule_of_edge_tables(k, geom):
    """Empty rows, empty trailing pages, full last pages, entries before indptr[0], a page list cut
    by num_indices, ranges forced past 512 pages, one-page sequences, ids outside the pool; four
    head geometries."""
    c = CASES[k]
    rng = np.random.default_rng(100 + k)
    indptr, indices, last = _table(rng, c["lens"], c.get("lp"), c.get("lead", 0), bad_ids=c.get("bad", 0))
    n_idx = int(indptr[-1]) - c.get("cut", 0)
    hq, hkv, d, dt = geom
    _plan_check(indptr, indices, last, hq, hkv, d, dt, ctas=c["R"], num_indices=n_idx)
