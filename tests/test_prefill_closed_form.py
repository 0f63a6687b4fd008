"""The closed-form prefill check (tests/test_gpu_prefill_exact.py) discriminates: on the same
tables, moving every row's causal limit by one key, or dropping one page of a request, changes
rows by more than the two ulps the GPU check allows.  Host arithmetic only."""
import numpy as np
import torch

from ecahlang_amd import workloads
from test_gpu_prefill_exact import expected_rows, ulps


def _beyond(a, b, dtype):
    return int((np.abs(a - b) > 2 * ulps(a, dtype)).any(axis=2).sum())


def test_off_by_one_causal_limit_is_detected():
    wb = workloads.qwen25_3b_prefill()
    exp = expected_rows(wb, True)
    for shift in (-1, 1):
        moved = _beyond(exp, expected_rows(wb, True, shift), torch.float16)
        assert moved >= 0.9 * exp.shape[0] * exp.shape[1], f"shift {shift}: only {moved} rows differ"


def test_a_dropped_page_is_detected():
    wb = workloads.build_batch([3000, 40, 2, 700, 64], [64, 0, 1, 600, 48], 32, 8, 128, torch.bfloat16, 77)
    exp = expected_rows(wb, True)
    ip = wb.indptr.clone()
    idx = wb.indices.clone()
    # request 3's 10th page replaced by a page no request owns (its rows select other classes:
    # page ids that agree mod D - 1 select the same ones, so one that does not is taken)
    was = int(idx[int(ip[3]) + 9])
    unused = [p for p in sorted(set(range(wb.cache.shape[0])) - set(idx.tolist())) if (p - was) % (wb.d - 1)]
    idx[int(ip[3]) + 9] = unused[0]
    bad = workloads.PagedBatch(**{**wb.__dict__, "indices": idx})
    moved = _beyond(exp, expected_rows(bad, True), torch.bfloat16)
    assert moved > 0
