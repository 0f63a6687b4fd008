"""The decode step's append fused with the decode (BatchDecodeWithPagedKVCacheWrapper.run(...,
append_kv=), pkv_batch_decode_append): token b's K and V rows go to the last slot of sequence
b's last page (the previous page's, when the last page is still empty), then attention runs
over the caches that hold them.  Checked against the two
launches the reference's graph step makes (append_paged_kv_cache at positions seq_len - 1, then
run): the output and the whole NaN-poisoned pool, bit for bit.  Covered: the matrix-core path
with the append inside the decode launch (head blocks of 1, 2 and 4 KV heads, sequences split
across workgroups, last pages holding 1 and 16 tokens); the paths that append with a launch of
their own (vector-ALU shapes, waves that take pages on demand, a cascade plan); rows whose
metadata names no slot, which get no append; and the fused call captured in a graph and
replayed with new rows."""
import numpy as np
import pytest
import torch

from ecahlang_amd import ops, workloads
from ecahlang_amd.wrappers import BatchDecodeWithPagedKVCacheWrapper
from oracle import kv_ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")

# context lengths after the step's token: last pages of 1, 16 and partial lengths, and a few
# long sequences that 16 workgroups split into several parts
LENS = [1, 16, 17, 32, 33, 100, 255, 2900, 5000, 7, 64, 65, 1500, 16, 3, 4097]

CASES = {
    # (hq, hkv, d, dtype): head block of 2 (Qwen2.5-3B), 2 (Llama-3.1-8B: 4 blocks), 1 (g 16),
    # 4 (d 64, g 4), and fp32 (the vector-ALU kernel)
    "qwen_fp16": (16, 2, 128, torch.float16),
    "llama8b_bf16": (32, 8, 128, torch.bfloat16),
    "hkv1_g16_fp16": (16, 1, 128, torch.float16),
    "d64_g4_bf16": (32, 8, 64, torch.bfloat16),
    "fp32_valu": (32, 8, 64, torch.float32),
    "hq4_hkv2_d64_fp16": (4, 2, 64, torch.float16),
}


def _iv(t):
    return t.view(torch.int32 if t.dtype == torch.float32 else torch.int16)


def _wrapper(dv, deterministic=True, cascade=False, ctas=16):
    w = BatchDecodeWithPagedKVCacheWrapper(torch.empty(128 << 20, dtype=torch.uint8, device=DEV), "NHD")
    w.plan(dv.indptr, dv.indices, dv.last, dv.hq, dv.hkv, dv.d, dv.ps, q_data_type=dv.dtype, num_ctas=ctas,
           deterministic=deterministic, cascade=cascade)
    return w


def _two_launches(dv, w, keep=None):
    """The reference's step: append at positions seq_len - 1 (rows in `keep` only), then run."""
    cache = dv.cache.clone()
    rows = slice(None) if keep is None else keep
    ops.append_paged_kv_cache(dv.k_new[rows], dv.v_new[rows], dv.batch_indices[rows], dv.positions[rows], cache,
                              dv.indices, dv.indptr, dv.last)
    out = w.run(dv.q, cache)
    return out, cache


def _fused(dv, w):
    cache = dv.cache.clone()
    out = w.run(dv.q, cache, append_kv=(dv.k_new, dv.v_new))
    return out, cache


def _head_major(t):
    """The same rows as the model hands them: [tokens, heads, D] views of a [heads, tokens, D]
    tensor (head stride = tokens * D)."""
    return t.transpose(0, 1).contiguous().transpose(0, 1)


@pytest.mark.parametrize("name,ctas,strided", [(n, 16, False) for n in CASES] +
                         [("qwen_fp16", None, True), ("hq4_hkv2_d64_fp16", None, True),
                          ("hq4_hkv2_d64_fp16", None, False), ("llama8b_bf16", None, True)])
def test_fused_append_matches_append_then_decode(name, ctas, strided):
    hq, hkv, d, dtype = CASES[name]
    print(f"case {name} ctas={ctas} strided={strided}", flush=True)
    wb = workloads.build_batch(LENS, [1] * len(LENS), hq, hkv, d, dtype, 61, scale=0.5)
    dv = wb.to(DEV)
    if strided:
        dv.k_new, dv.v_new = _head_major(dv.k_new), _head_major(dv.v_new)
    w = _wrapper(dv, ctas=ctas)
    assert w._mfma == (dtype != torch.float32)
    want_out, want_cache = _two_launches(dv, w)
    out, cache = _fused(dv, w)
    torch.cuda.synchronize()
    assert torch.equal(_iv(cache), _iv(want_cache))
    assert torch.equal(_iv(out), _iv(want_out))
    # the two-launch result itself against the oracle (the append is bit-exact elsewhere)
    raw = kv_ref.append(_iv(wb.cache).numpy(), _iv(wb.k_new).numpy(), _iv(wb.v_new).numpy(),
                        wb.batch_indices.numpy(), wb.positions.numpy(), wb.indices.numpy(), wb.indptr.numpy(), wb.ps)
    assert np.array_equal(_iv(cache).cpu().numpy(), raw)
    for b in (0, 7, 8, 15):
        pages = wb.indices[wb.indptr[b]:wb.indptr[b + 1]].long()
        L = LENS[b]
        kv = torch.from_numpy(raw).view(dtype)[pages].float().numpy()
        k = kv[:, 0].reshape(-1, hkv, d)[:L]
        v = kv[:, 1].reshape(-1, hkv, d)[:L]
        ref = kv_ref._attend(wb.q[b:b + 1].float().numpy().astype(np.float64), k, v, [L], d ** -0.5)[0]
        tol = dict(atol=1e-5, rtol=1e-5) if dtype == torch.float32 else dict(atol=2e-3, rtol=1e-2)
        np.testing.assert_allclose(out[b].float().cpu().numpy(), ref, **tol, err_msg=f"row {b}")


@pytest.mark.parametrize("mode", ["dynamic", "cascade", "valu"])
def test_fused_append_on_paths_with_a_separate_launch(mode):
    """Waves that take pages on demand, a cascade plan and the forced vector-ALU kernel append
    with a launch of their own: the same bits as the two launches."""
    hq, hkv, d, dtype = CASES["qwen_fp16"]
    wb = workloads.build_batch(LENS, [1] * len(LENS), hq, hkv, d, dtype, 62, scale=0.5)
    dv = wb.to(DEV)
    w = _wrapper(dv, deterministic=mode != "dynamic", cascade=mode == "cascade")
    if mode == "valu":
        c1 = dv.cache.clone()
        ops.append_paged_kv_cache(dv.k_new, dv.v_new, dv.batch_indices, dv.positions, c1, dv.indices, dv.indptr,
                                  dv.last)
        want_out, want_cache = w.run(dv.q, c1, force_valu=True), c1
        cache = dv.cache.clone()
        out = w.run(dv.q, cache, append_kv=(dv.k_new, dv.v_new), force_valu=True)
    else:
        want_out, want_cache = _two_launches(dv, w)
        out, cache = _fused(dv, w)
    torch.cuda.synchronize()
    assert torch.equal(_iv(cache), _iv(want_cache))
    if mode == "dynamic":  # the summation order varies from call to call
        torch.testing.assert_close(out.float(), want_out.float(), atol=2e-3, rtol=1e-2)
    else:
        assert torch.equal(_iv(out), _iv(want_out))


def _positions(indptr, last, ps=16):
    """Position seq_len - 1 = (n - 1) * ps + last - 1 of each row, or -1 when the row gets no
    append (empty list, last outside [0, ps], negative position)."""
    out = []
    for b in range(len(last)):
        n, lp = int(indptr[b + 1] - indptr[b]), int(last[b])
        at = (n - 1) * ps + lp - 1
        out.append(at if n >= 1 and 0 <= lp <= ps and at >= 0 else -1)
    return out


@pytest.mark.parametrize("name", ["qwen_fp16", "fp32_valu"])
def test_rows_whose_metadata_names_no_slot_get_no_append(name):
    """kv_last_page_len past the page size, 0 on a one-page sequence (position -1) and a token
    page id outside the pool: those rows' tokens are not written anywhere.  kv_last_page_len 0
    on a two-page sequence puts the token at the first page's last slot, as the reference's
    append at position seq_len - 1 does."""
    hq, hkv, d, dtype = CASES[name]
    wb = workloads.build_batch(LENS, [1] * len(LENS), hq, hkv, d, dtype, 63, scale=0.5)
    dv = wb.to(DEV)
    last = wb.last.clone()
    last[0] = 0   # one page: position -1
    last[3] = 0   # two pages: position 15
    last[5] = 17
    indices = dv.indices.clone()
    indices[int(wb.indptr[11]) - 1] = wb.num_pages + 5  # row 10's token page
    pos = _positions(wb.indptr.tolist(), last.tolist())
    assert pos[0] == -1 and pos[3] == 15 and pos[5] == -1
    keep = torch.tensor([p >= 0 and b != 10 for b, p in enumerate(pos)], device=DEV)
    dv.last, dv.indices = last.to(DEV), indices
    dv.positions = torch.tensor([max(p, 0) for p in pos], dtype=torch.int32, device=DEV)
    w = _wrapper(dv)
    want_out, want_cache = _two_launches(dv, w, keep)
    out, cache = _fused(dv, w)
    torch.cuda.synchronize()
    assert torch.equal(_iv(cache), _iv(want_cache))
    assert torch.equal(_iv(out), _iv(want_out))


@pytest.mark.parametrize("ctas", [16, 7, None])
def test_token_on_the_page_before_an_empty_last_page(ctas):
    """The pool's append_tokens pops an empty page as soon as a page fills (kv_last_page_len 0):
    the step's token then lands in the previous page's last slot, which may sit in another range
    (another workgroup) than the empty page.  Sequences of whole pages get that empty page here,
    including long ones that the plan splits across ranges."""
    hq, hkv, d, dtype = CASES["qwen_fp16"]
    lens = [16, 32, 4096, 7, 2048, 48, 1, 8192, 100, 512, 17, 1024]
    wb = workloads.build_batch(lens, [1] * len(lens), hq, hkv, d, dtype, 66, scale=0.5)
    ind, ptr, last = wb.indices.tolist(), wb.indptr.tolist(), wb.last.tolist()
    spare = sorted(set(range(wb.num_pages)) - set(ind))
    rows, nptr, nlast = [], [0], []
    for b, L in enumerate(lens):
        pages = ind[ptr[b]:ptr[b + 1]]
        if L % 16 == 0:
            pages = pages + [spare.pop()]
            nlast.append(0)
        else:
            nlast.append(last[b])
        rows += pages
        nptr.append(len(rows))
    assert _positions(nptr, nlast) == [L - 1 for L in lens]
    dv = wb.to(DEV)
    dv.indices = torch.tensor(rows, dtype=torch.int32, device=DEV)
    dv.indptr = torch.tensor(nptr, dtype=torch.int32, device=DEV)
    dv.last = torch.tensor(nlast, dtype=torch.int32, device=DEV)
    w = _wrapper(dv, ctas=ctas)
    want_out, want_cache = _two_launches(dv, w)
    out, cache = _fused(dv, w)
    torch.cuda.synchronize()
    assert torch.equal(_iv(cache), _iv(want_cache))
    assert torch.equal(_iv(out), _iv(want_out))


def test_fused_append_captured_in_a_graph():
    """Captured once, replayed three times with new K/V/Q rows written into the captured inputs
    between replays (and eager work in between): every replay matches the two launches."""
    hq, hkv, d, dtype = CASES["qwen_fp16"]
    wb = workloads.build_batch(LENS, [1] * len(LENS), hq, hkv, d, dtype, 64, scale=0.5)
    dv = wb.to(DEV)
    w = _wrapper(dv)
    base = dv.cache.clone()
    cache = dv.cache.clone()
    out = torch.empty_like(dv.q)
    s = torch.cuda.Stream(device=DEV)
    s.wait_stream(torch.cuda.current_stream(DEV))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        w.run(dv.q, cache, out=out, append_kv=(dv.k_new, dv.v_new))
        s.synchronize()
        with torch.cuda.graph(g, stream=s):
            w.run(dv.q, cache, out=out, append_kv=(dv.k_new, dv.v_new))
    gen = torch.Generator(device=DEV).manual_seed(65)
    for rep in range(3):
        for t in (dv.q, dv.k_new, dv.v_new):
            t.copy_((torch.randn(t.shape, generator=gen, device=DEV) * 0.5).to(dtype))
        cache.copy_(base)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        dv.cache = base
        want_out, want_cache = _two_launches(dv, w)
        torch.cuda.synchronize()
        assert torch.equal(_iv(cache), _iv(want_cache)), rep
        assert torch.equal(_iv(out), _iv(want_out)), rep
