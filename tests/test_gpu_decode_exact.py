"""Decode outputs in closed form at full size.

With q = 0 every valid token of a sequence gets the same weight, so each output row is the mean
of the sequence's V rows.  Here V rows are one-hot: the rows of a page select dimension
(5 * page + 31 * head) mod (D - 1), and the page holding a sequence's last token selects D - 1.
Each output row is then count_d / L per dimension, exact on the host.  A dropped, repeated or
misplaced page moves some dimension by at least 1 / L (a dimension holds about L / 127 tokens, so
that is ~127 / pages relative: many ulps at these sizes), and a wrong valid-row count on the last
page moves dimension D - 1 by 1 / nv relative; the kernel's own rounding (fp32 sums of exact
counts, one division, a merge of partials with equal maxima) stays within one ulp of the output
type.  Checked at the headline decode (Qwen2.5-3B, B=64, fp16) and the long-context decode
(Llama-3.1-8B, B=128, bf16), with the step's append fused into the launch and without, and on
the shared-prefix step's tables with the hint.  K rows are random: with q = 0 they must not
matter; slots no token owns are NaN, so reading one shows."""
import numpy as np
import pytest
import torch

from ecahlang_amd import workloads
from ecahlang_amd.wrappers import BatchDecodeWithPagedKVCacheWrapper
from test_gpu_decode_schedule import _shared_prefix_table

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
PS = 16
MANT = {torch.float16: 10, torch.bfloat16: 7}
TINY = {torch.float16: 2.0 ** -24, torch.bfloat16: 2.0 ** -133}


def _classes(pids, hkv, d):
    return (np.asarray(pids, dtype=np.int64)[:, None] * 5 + np.arange(hkv)[None, :] * 31) % (d - 1)


def _build(indptr, indices, last, hq, hkv, d, dtype, pool_pages, seed, hole_last=False):
    """Device cache with one-hot V rows and random K rows on the listed pages; the expected
    outputs; with hole_last, each sequence's last token slot is left NaN and its rows returned
    for the fused append."""
    indptr = np.asarray(indptr, dtype=np.int64)
    indices = np.asarray(indices, dtype=np.int64)
    last = np.asarray(last, dtype=np.int64)
    B = len(last)
    lastpage = indices[indptr[1:] - 1]
    valid = {}  # rows of each used page: 16, or the sequence's last-page length
    for p in indices.tolist():
        valid[p] = PS
    for b in range(B):
        valid[int(lastpage[b])] = int(last[b])
    pages = np.array(sorted(valid), dtype=np.int64)
    nvalid = np.array([valid[p] for p in pages.tolist()], dtype=np.int64)
    cls = _classes(pages, hkv, d)
    is_last = np.isin(pages, lastpage)
    cls[is_last] = d - 1
    cache = torch.full((pool_pages, 2, PS, hkv, d), float("nan"), dtype=dtype, device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(seed)
    pg_d = torch.from_numpy(pages).to(DEV)
    nv_d = torch.from_numpy(nvalid).to(DEV)
    cls_d = torch.from_numpy(cls).to(DEV)
    slot = torch.arange(PS, device=DEV)
    for s in range(0, len(pages), 8192):
        p, nv, c = pg_d[s:s + 8192], nv_d[s:s + 8192], cls_d[s:s + 8192]
        n = p.numel()
        ok = (slot[None, :] < nv[:, None])[:, :, None, None]
        k = torch.randn((n, PS, hkv, d), generator=gen, device=DEV, dtype=torch.float32)
        v = torch.nn.functional.one_hot(c, d).to(torch.float32)[:, None].expand(n, PS, hkv, d)
        nan = torch.tensor(float("nan"), device=DEV)
        cache[p, 0] = torch.where(ok, k, nan).to(dtype)
        cache[p, 1] = torch.where(ok, v, nan).to(dtype)
    # expected: count of valid tokens per (sequence, head, dimension) / L
    counts = np.zeros((B, hkv, d), dtype=np.float64)
    L = np.zeros(B, dtype=np.int64)
    pos = {int(p): i for i, p in enumerate(pages.tolist())}
    for b in range(B):
        for p in indices[indptr[b]:indptr[b + 1]].tolist():
            i = pos[p]
            nv = nvalid[i] if p == lastpage[b] else PS
            counts[b, np.arange(hkv), cls[i]] += nv
            L[b] += nv
    g = hq // hkv
    exp = np.repeat(counts / L[:, None, None], g, axis=1)  # [B, hq, d]
    app = None
    if hole_last:
        # the last token of each sequence: its slot goes back to NaN, its rows are appended
        ks = torch.randn((B, hkv, d), generator=gen, device=DEV, dtype=torch.float32).to(dtype)
        vs = torch.zeros((B, hkv, d), device=DEV, dtype=dtype)
        vs[:, :, d - 1] = 1
        lp = torch.from_numpy(lastpage).to(DEV)
        lr = torch.from_numpy(last - 1).to(DEV)
        cache[lp, 0, lr] = float("nan")
        cache[lp, 1, lr] = float("nan")
        app = (ks, vs, lp, lr)
    tables = (torch.tensor(indptr, dtype=torch.int32, device=DEV), torch.tensor(indices, dtype=torch.int32, device=DEV),
              torch.tensor(last, dtype=torch.int32, device=DEV))
    return cache, tables, exp, app


def _check(got, exp, dtype, what):
    got = got.double().cpu().numpy()
    e = np.abs(exp)
    ulp = np.where(e > 0, np.maximum(2.0 ** (np.floor(np.log2(np.where(e > 0, e, 1))) - MANT[dtype]), TINY[dtype]), 0)
    err = np.abs(got - exp)
    bad = ~(err <= ulp)
    if bad.any():
        b, h, dd = np.argwhere(bad)[0]
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} values off by more than one ulp; first at "
                             f"sequence {b} head {h} dim {dd}: {got[b, h, dd]!r} vs {exp[b, h, dd]!r}")


def _run(tables, cache, hq, hkv, d, dtype, ctas=None, hint=None, append=None):
    ip, idx, lt = tables
    B = lt.numel()
    ws = torch.empty(128 << 20, dtype=torch.uint8, device=DEV)
    w = BatchDecodeWithPagedKVCacheWrapper(ws, "NHD")
    w.plan(ip, idx, lt, hq, hkv, d, PS, q_data_type=dtype, num_ctas=ctas, kv_shared_pages=hint)
    assert w._mfma
    q = torch.zeros((B, hq, d), dtype=dtype, device=DEV)
    if append is None:
        out = w.run(q, cache)
    else:
        out = w.run(q, cache, append_kv=(append[0], append[1]))
    torch.cuda.synchronize()
    return out


def _decode_case(lens, hq, hkv, d, dtype, seed, ctas):
    pool = int(np.ceil(1.25 * sum((L + 15) // 16 for L in lens)))
    ip, idx, lt = workloads.paged_table(lens, pool, seed=seed)
    cache, tables, exp, app = _build(ip.numpy(), idx.numpy(), lt.numpy(), hq, hkv, d, dtype, pool, seed,
                                     hole_last=True)
    # fused: the append writes each sequence's last token, then the decode attends it
    out = _run(tables, cache, hq, hkv, d, dtype, ctas=ctas, append=app)
    ks, vs, lp, lr = app
    assert torch.equal(cache[lp, 0, lr].view(torch.int16), ks.view(torch.int16)), "appended K rows"
    assert torch.equal(cache[lp, 1, lr].view(torch.int16), vs.view(torch.int16)), "appended V rows"
    _check(out, exp, dtype, f"fused append + decode (ctas={ctas})")
    # unfused, on the cache the fused launch completed
    out2 = _run(tables, cache, hq, hkv, d, dtype, ctas=ctas)
    _check(out2, exp, dtype, f"decode (ctas={ctas})")
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16)), "fused and plain decode differ"


@pytest.mark.parametrize("ctas", [None, 16])
@torch.no_grad()
def test_qwen25_3b_b64_decode_closed_form(ctas):
    lens = workloads.qwen25_3b_lengths()
    print(f"C2 closed form: B={len(lens)} tokens={sum(lens)} ctas={ctas}", flush=True)
    _decode_case(lens, 16, 2, 128, torch.float16, 1002, ctas)


@torch.no_grad()
def test_llama31_8b_long_context_closed_form():
    lens = workloads.llama31_8b_lengths()
    print(f"C4 closed form: B={len(lens)} tokens={sum(lens)}", flush=True)
    _decode_case(lens, 32, 8, 128, torch.bfloat16, 1004, None)


@torch.no_grad()
def test_shared_prefix_step_closed_form():
    """The 36-layer step's tables (every table starts with the same 128 pages) with the
    shared-prefix hint: the prefix pages' rows count once per sequence."""
    rng = np.random.default_rng(1005)
    ip, idx, lt, hint = _shared_prefix_table(rng)
    pool = int(idx.max()) + 1
    cache, tables, exp, _ = _build(ip, idx, lt, 16, 2, 128, torch.float16, pool, 1005)
    h = torch.tensor(hint, dtype=torch.int32, device=DEV)
    out = _run(tables, cache, 16, 2, 128, torch.float16, hint=h)
    _check(out, exp, torch.float16, "shared-prefix decode with the hint")
    plain = _run(tables, cache, 16, 2, 128, torch.float16)
    assert torch.equal(out.view(torch.int16), plain.view(torch.int16)), "the hint changed the result"


@pytest.mark.parametrize("ctas,hq,hkv,dtype", [(2, 16, 2, torch.float16), (3, 32, 8, torch.bfloat16)])
@torch.no_grad()
def test_many_short_sequences_closed_form(ctas, hq, hkv, dtype):
    """300 sequences of 2-4 pages on 2-3 workgroups: ranges of a hundred and more segments (far
    past the range heads' first segments), sequences split between ranges."""
    rng = np.random.default_rng(77 + ctas)
    lens = [int(x) for x in rng.integers(17, 61, size=300)]
    print(f"short sequences: B={len(lens)} tokens={sum(lens)} ctas={ctas}", flush=True)
    pool = int(np.ceil(1.25 * sum((L + 15) // 16 for L in lens)))
    ip, idx, lt = workloads.paged_table(lens, pool, seed=78 + ctas)
    cache, tables, exp, app = _build(ip.numpy(), idx.numpy(), lt.numpy(), hq, hkv, 128, dtype, pool, 79, hole_last=True)
    out = _run(tables, cache, hq, hkv, 128, dtype, ctas=ctas, append=app)
    _check(out, exp, dtype, f"fused append + decode, {ctas} workgroups")
    out2 = _run(tables, cache, hq, hkv, 128, dtype, ctas=ctas)
    _check(out2, exp, dtype, f"decode, {ctas} workgroups")
