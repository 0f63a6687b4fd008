"""Chunked prefill outputs in closed form at full size.

With q = 0 every key a query row sees weighs the same, so each output row is the mean of the V
rows of exactly the keys it sees: keys 0 .. t + kv_len - qo_len of its request for query token t
when causal (bottom-right aligned), all kv_len keys otherwise.  V rows are one-hot: the row of
key j (page p, row r of the page, KV head h) selects dimension (5 p + 31 h + 7 r) mod (D - 1),
so each output dimension is count / L_t, exact on the host.  A key seen that should not be, or
missed, moves its dimension by 1 / L_t, about (D - 1) / L_t relative to its value: many ulps at
these sizes, while the kernel's own rounding (exact fp32 sums of ones and counts, one division,
fp16 partials of split key ranges merged with equal maxima) stays within two ulps.  Checked on the
Qwen2.5-3B chunked-prefill batch (8 x 512-token chunks on prefixes U[0, 8192], key ranges split
across workgroups), causal and not, and on a ragged bf16 batch with a request that adds no
tokens, one-token prefixes and pages shared by nothing.  K rows are random; slots no token owns
are NaN, so reading one shows."""
import numpy as np
import pytest
import torch

from ecahlang_amd import workloads
from ecahlang_amd.wrappers import BatchPrefillWithPagedKVCacheWrapper

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
PS = 16
MANT = {torch.float16: 10, torch.bfloat16: 7}


def _cls(pages, rows, h, d):
    return (5 * pages + 31 * h + 7 * rows) % (d - 1)


def expected_rows(wb, causal, shift=0):
    """The closed-form output rows [nnz, Hq, D] (float64) of a batch whose V rows are one-hot
    by _cls and whose queries are zero; ``shift`` moves every row's causal limit (a planted
    mistake, for the check that these rows discriminate)."""
    ip = wb.indptr.numpy().astype(np.int64)
    idx = wb.indices.numpy().astype(np.int64)
    qo = wb.append_indptr.numpy().astype(np.int64)
    kv_len = np.array(wb.kv_len, dtype=np.int64)
    hkv, hq, d = wb.hkv, wb.hq, wb.d
    g = hq // hkv
    exp = np.zeros((int(qo[-1]), hq, d), dtype=np.float64)
    for b in range(len(kv_len)):
        L, n = int(kv_len[b]), int(qo[b + 1] - qo[b])
        pages, rows = idx[ip[b] + np.arange(L) // PS], np.arange(L) % PS
        t = np.arange(n)
        seen = np.clip(t + L - n + 1 + shift, 1, L) if causal else np.full(n, L)
        for h in range(hkv):
            onehot = np.zeros((L + 1, d), dtype=np.int64)
            onehot[np.arange(1, L + 1), _cls(pages, rows, h, d)] = 1
            counts = np.cumsum(onehot, axis=0)  # counts[m] = classes of keys 0 .. m - 1
            exp[qo[b]:qo[b] + n, h * g:(h + 1) * g] = (counts[seen] / seen[:, None])[:, None, :]
    return exp


def ulps(exp, dtype):
    e = np.abs(exp)
    return np.where(e > 0, 2.0 ** (np.floor(np.log2(np.where(e > 0, e, 1))) - MANT[dtype]), 0)


def _case(wb, causal, seed):
    ip = wb.indptr.numpy().astype(np.int64)
    idx = wb.indices.numpy().astype(np.int64)
    qo = wb.append_indptr.numpy().astype(np.int64)
    kv_len = np.array(wb.kv_len, dtype=np.int64)
    B, hkv, hq, d = len(kv_len), wb.hkv, wb.hq, wb.d
    g = hq // hkv
    # every valid key's page and row
    tok_page = np.concatenate([idx[ip[b] + np.arange(kv_len[b]) // PS] for b in range(B)])
    tok_row = np.concatenate([np.arange(kv_len[b]) % PS for b in range(B)])
    cache = torch.full(tuple(wb.cache.shape), float("nan"), dtype=wb.dtype, device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(seed)
    tp = torch.from_numpy(tok_page).to(DEV)
    tr = torch.from_numpy(tok_row).to(DEV)
    cls = torch.stack([torch.from_numpy(_cls(tok_page, tok_row, h, d)).to(DEV) for h in range(hkv)], 1)  # [tok, hkv]
    cache[tp, 0, tr] = torch.randn((len(tok_page), hkv, d), generator=gen, device=DEV).to(wb.dtype)
    cache[tp, 1, tr] = torch.nn.functional.one_hot(cls, d).to(wb.dtype)
    q = torch.zeros((int(qo[-1]), hq, d), dtype=wb.dtype, device=DEV)
    exp = expected_rows(wb, causal)
    dv = wb.to(DEV)
    w = BatchPrefillWithPagedKVCacheWrapper(torch.empty(128 << 20, dtype=torch.uint8, device=DEV), "NHD")
    w.plan(dv.append_indptr, dv.indptr, dv.indices, dv.last, hq, hkv, d, PS, causal=causal, q_data_type=wb.dtype)
    assert w._mfma
    out = w.run(q, cache)
    torch.cuda.synchronize()
    got = out.double().cpu().numpy()
    bad = ~(np.abs(got - exp) <= 2 * ulps(exp, wb.dtype))
    if bad.any():
        r, hh, dd = np.argwhere(bad)[0]
        raise AssertionError(f"{int(bad.sum())} of {bad.size} values off by more than two ulps; first at query row {r} "
                             f"head {hh} dim {dd}: {got[r, hh, dd]!r} vs {exp[r, hh, dd]!r}")
    return w


@pytest.mark.parametrize("causal", [True, False])
@torch.no_grad()
def test_qwen25_3b_chunked_prefill_closed_form(causal):
    wb = workloads.qwen25_3b_prefill()
    print(f"C3 closed form causal={causal}: kv={sum(wb.kv_len)}", flush=True)
    w = _case(wb, causal, 3003)
    assert w._n_groups > 0  # split key ranges exercised


@pytest.mark.parametrize("causal", [True, False])
@torch.no_grad()
def test_ragged_bf16_prefill_closed_form(causal):
    # requests: a long prefix, no new tokens, a one-token prefix, a chunk longer than its prefix,
    # and a chunk that starts a page
    wb = workloads.build_batch([3000, 40, 2, 700, 16 + 48], [64, 0, 1, 600, 48], 32, 8, 128, torch.bfloat16, 77)
    print(f"ragged closed form causal={causal}", flush=True)
    _case(wb, causal, 3004)
