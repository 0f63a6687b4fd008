"""Shared prefixes in the matrix-core decode (plan's kv_shared_pages): sequences in runs that
share their leading pages, with prefixes from 16 pages (the smallest that is grouped) past 2048
pages (past sixteen chunks of 64 pages, where chunks grow towards 128), runs of 1 to 17
sequences (partial groups), hints
that understate the sharing, and head layouts whose prefix items group 2, 4 and 8 sequences.
With the hint alone the shared pages only change load policy, so the output is bit-identical
to the plain schedule's; with the cascade every output row is checked against the float64
oracle and against the plain schedule."""
import numpy as np
import pytest
import torch

import sched_check as sc

from ecahlang_amd.wrappers import BatchDecodeWithPagedKVCacheWrapper
from oracle import kv_ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
PS = 16


def _batch(runs, hq, hkv, d, dtype, seed):
    """runs: list of (sequences, shared pages, hinted pages).  Returns the device page table,
    cache, q and hint, plus the host copies the oracle reads."""
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    pages, hint, last = [], [], []
    nxt = 0
    for n, shared, hinted in runs:
        pre = list(range(nxt, nxt + shared))
        nxt += shared
        for i in range(n):
            own = int(rng.integers(1, 40))
            pages.append(pre + list(range(nxt, nxt + own)))
            nxt += own
            hint.append(hinted if i > 0 else 0)
            last.append(int(rng.integers(1, PS + 1)))
    perm = torch.randperm(nxt + 64, generator=g).tolist()  # scatter the pages over the pool
    pages = [[perm[p] for p in row] for row in pages]
    indptr = np.cumsum([0] + [len(r) for r in pages]).astype(np.int32)
    indices = np.array([p for r in pages for p in r], dtype=np.int32)
    cache = (torch.randn((nxt + 64, 2, PS, hkv, d), generator=g) * 0.5).to(dtype)
    used = torch.zeros(nxt + 64, dtype=torch.bool)
    used[torch.from_numpy(indices).long()] = True
    cache[~used] = float("nan")
    for r, L in zip(pages, last):  # slots past each sequence's end are NaN
        cache[r[-1], :, L:] = float("nan")
    q = (torch.randn((len(pages), hq, d), generator=g) * 0.5).to(dtype)
    dv = dict(indptr=torch.from_numpy(indptr).to(DEV), indices=torch.from_numpy(indices).to(DEV),
              last=torch.tensor(last, dtype=torch.int32, device=DEV), cache=cache.to(DEV), q=q.to(DEV),
              hint=torch.tensor(hint, dtype=torch.int32, device=DEV))
    return dv, dict(indptr=indptr, indices=indices, last=last, cache=cache, q=q)


def _decode(dv, hq, hkv, d, dtype, hint, cascade=False):
    ws = torch.empty(128 << 20, dtype=torch.uint8, device=DEV)
    w = BatchDecodeWithPagedKVCacheWrapper(ws, "NHD")
    w.plan(dv["indptr"], dv["indices"], dv["last"], hq, hkv, d, PS, q_data_type=dtype,
           kv_shared_pages=dv["hint"] if hint else None, cascade=cascade)
    assert w._mfma
    out = w.run(dv["q"], dv["cache"])
    torch.cuda.synchronize()
    # global schedule header (after the per-sequence counters, 256-byte aligned): R, prefix items
    off = sc.layout(dv["q"].shape[0], hq, d, w._ctas, dv["indices"].numel(), ws.numel())["ghdr"]
    hdr = ws[off:off + 32].view(torch.int32).tolist()
    return out.float().cpu().numpy(), hdr[0], hdr[4]


QWEN_RUNS = [(1, 0, 0), (2, 16, 16), (9, 100, 100), (8, 17, 16), (17, 600, 600), (3, 2100, 2100),
             (4, 40, 15), (5, 30, 30)]


@pytest.mark.parametrize("hq,hkv,d,dtype,runs,group", [
    (16, 2, 128, torch.float16, QWEN_RUNS + [(40, 64, 64)], 4),              # Qwen2.5-3B
    (32, 8, 128, torch.bfloat16, [(5, 40, 40), (1, 0, 0), (3, 20, 20)], 8),  # Llama-3.1-8B
    (32, 8, 64, torch.float16, [(6, 33, 33), (2, 70, 70)], 8),               # Llama-3.2-1B
    (16, 1, 128, torch.bfloat16, [(10, 50, 50), (3, 16, 16)], 2),            # one KV head, g 16
    (8, 2, 64, torch.float16, [(11, 64, 64)], 8),                            # 256-byte unit rows
])
@torch.no_grad()
def test_cascade_matches_oracle_and_plain_schedule(hq, hkv, d, dtype, runs, group):
    dv, host = _batch(runs, hq, hkv, d, dtype, seed=hq * 1000 + hkv * 10 + d)
    B = len(host["last"])
    print(f"cascade: hq={hq} hkv={hkv} d={d} {dtype} B={B} pages={len(host['indices'])}", flush=True)
    got, R, items = _decode(dv, hq, hkv, d, dtype, hint=True, cascade=True)
    plain, R0, items0 = _decode(dv, hq, hkv, d, dtype, hint=False)
    marked, _, items1 = _decode(dv, hq, hkv, d, dtype, hint=True)
    # prefix items only with the cascade
    assert items0 == 0 and items1 == 0 and items > 0
    assert np.array_equal(marked, plain)  # the hint alone changes the load policy, not the math
    np.testing.assert_allclose(got, plain, atol=4e-3, rtol=2e-2)
    cache = host["cache"].float().numpy()
    q = host["q"].float().numpy().astype(np.float64)
    ref = kv_ref.decode(q, cache, host["indptr"], host["indices"], host["last"], PS)
    for b in range(B):
        np.testing.assert_allclose(got[b], ref[b], atol=2e-3, rtol=1e-2, err_msg=f"sequence {b}")


@torch.no_grad()
def test_cascade_hint_of_unshared_or_short_runs_changes_nothing():
    """Runs that share fewer than 16 pages are not grouped: the schedule has no prefix items
    and the result is the plain one."""
    dv, host = _batch([(3, 15, 15), (2, 0, 0)], 16, 2, 128, torch.float16, seed=5)
    got, _, items = _decode(dv, 16, 2, 128, torch.float16, hint=True, cascade=True)
    assert items == 0
    ref = kv_ref.decode(host["q"].float().numpy().astype(np.float64), host["cache"].float().numpy(),
                        host["indptr"], host["indices"], host["last"], PS)
    np.testing.assert_allclose(got, ref, atol=2e-3, rtol=1e-2)
