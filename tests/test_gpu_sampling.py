"""The device sampler (ecahlang_amd.sampling, flashinfer.sampling.top_k_top_p_sampling_from_logits
at ecahlang/main.py:377-379, 489-491) against the oracle's rule: for a given uniform number
the token is the oracle's inverse-CDF draw over the same kept set (up to the fixed-point
rounding of the boundaries), it is always inside the kept set, and many draws reproduce the
oracle's distribution."""
import numpy as np
import pytest
import torch

from ecahlang_amd.sampling import top_k_top_p_sampling_from_logits as sample
from oracle import sampling_ref as sr

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _check_rows(x: torch.Tensor, ks, ps, u: torch.Tensor, got: torch.Tensor):
    xs = x.float().cpu().numpy().astype(np.float64)
    for r in range(xs.shape[0]):
        keep = sr.kept_set(xs[r], int(ks[r]), float(ps[r]))
        tok = int(got[r])
        assert 0 <= tok < xs.shape[1] and keep[tok], (r, tok)
        p = sr.probabilities(xs[r], int(ks[r]), float(ps[r]))
        c = np.cumsum(p)
        lo = c[tok - 1] if tok > 0 else 0.0
        uu = float(u[r])
        assert lo - 1e-6 <= uu * c[-1] <= c[tok] + 1e-6, (r, tok, uu, lo, c[tok])


@pytest.mark.parametrize("dtype,vocab,rows", [(torch.float16, 151936, 12), (torch.bfloat16, 32000, 16),
                                              (torch.float32, 1000, 16), (torch.float16, 1001, 8)])
def test_draw_matches_oracle(dtype, vocab, rows):
    g = torch.Generator().manual_seed(vocab + rows)
    x = (torch.randn(rows, vocab, generator=g) * 3).to(dtype)
    ks = torch.tensor([0, 1, 5, 50, vocab, vocab + 7, 20, 1000] * 2, dtype=torch.int32)[:rows]
    ps = torch.tensor([1.0, 1.0, 0.9, 0.5, 0.8, 0.05, 1.0, 0.95] * 2, dtype=torch.float32)[:rows]
    u = torch.rand(rows, generator=g)
    got = sample(x.to(DEV), ks.to(DEV), ps.to(DEV), uniform=u.to(DEV)).cpu()
    _check_rows(x, ks, ps, u, got)
    # scalars for every row
    got2 = sample(x.to(DEV), 40, 0.9, uniform=u.to(DEV)).cpu()
    _check_rows(x, [40] * rows, [0.9] * rows, u, got2)


def test_argmax_cases_and_strided_rows():
    g = torch.Generator().manual_seed(3)
    base = torch.randn(6, 5003, generator=g).half()
    x = torch.zeros(6, 5010, dtype=torch.float16)
    x[:, :5003] = base
    xd = x.to(DEV)[:, :5003]  # row stride 5010: rows not 16-byte aligned
    am = base.float().argmax(1)
    for k, p in ((1, 1.0), (0, 1e-6), (3, 1e-6)):
        got = sample(xd, k, p).cpu()
        assert torch.equal(got.long(), am), (k, p)


def test_ties_nan_and_masked_logits():
    x = torch.full((4, 64), -float("inf"))
    x[:, 10] = 2.0
    x[:, 20] = 2.0
    x[:, 30] = 1.0
    x[0, 5] = float("nan")
    u = torch.tensor([0.0, 0.49, 0.51, 0.999])
    got = sample(x.half().to(DEV), 1, 1.0, uniform=u.to(DEV)).cpu().tolist()
    assert got == [10, 10, 20, 20]  # top-1 keeps both tied maxima, each half the mass
    got = sample(x.half().to(DEV), 0, 1.0, uniform=u.to(DEV)).cpu().tolist()
    assert set(got) <= {10, 20, 30}


def test_distribution_of_many_draws():
    V, n = 16, 40000
    g = torch.Generator().manual_seed(11)
    row = torch.randn(V, generator=g) * 1.5
    x = row.expand(n, V).contiguous().to(DEV)
    for k, p in ((0, 1.0), (6, 1.0), (0, 0.7), (5, 0.8)):
        got = sample(x, k, p, generator=torch.Generator(device=DEV).manual_seed(k + 1)).cpu().numpy()
        freq = np.bincount(got, minlength=V) / n
        ref = sr.probabilities(row.numpy().astype(np.float64), k, p)
        assert np.all(freq[ref == 0] == 0), (k, p)
        assert np.abs(freq - ref).max() < 0.012, (k, p, np.abs(freq - ref).max())


def test_graph_captured_sampling_replays():
    """As the reference captures it (main.py:377-379 inside the decode graph): the default
    device generator, whose offset the graph advances on every replay."""
    x = torch.randn(8, 4096, device=DEV).half()
    torch.manual_seed(5)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        out = sample(x, 50, 0.9)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            out = sample(x, 50, 0.9)
    draws = []
    for _ in range(6):
        graph.replay()
        torch.cuda.synchronize()
        draws.append(out.cpu().clone())
    xs = x.float().cpu().numpy()
    for d in draws:
        for r in range(8):
            assert sr.kept_set(xs[r], 50, 0.9)[int(d[r])]
    assert len({tuple(d.tolist()) for d in draws}) > 1  # fresh uniforms on every replay


def _scaled_reference(x, table, rows, temp):
    """The serving loop's eager scaling (ecahlang/main.py:483-487): logits / mask_penalty rows
    in the logits' dtype, then / temperature [n, 1] float32 (which promotes to float32)."""
    y = x
    if table is not None:
        y = y / table[rows.long()]
    if temp is not None:
        y = y / temp.reshape(-1, 1)
    return y


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("which", ["both", "penalty", "temperature"])
def test_scaled_sampling_equals_sampling_the_scaled_logits(dtype, which):
    """Fused penalty + temperature: the token is exactly the one the plain sampler draws from
    the eagerly scaled logits, for the same uniforms (so every filter sees identical values)."""
    rows, vocab, slots = 16, 32000, 40
    g = torch.Generator().manual_seed(77)
    x = (torch.randn(rows, vocab, generator=g) * 3).to(dtype).to(DEV)
    table = torch.ones(slots, vocab, dtype=dtype)
    # repetition penalties on some tokens of some slots (main.py:522, 597: divided in place)
    for s in range(0, slots, 3):
        idx = torch.randint(0, vocab, (200,), generator=g)
        table[s, idx] = (1.0 / torch.empty(200).uniform_(1.05, 1.5, generator=g)).to(dtype)
        table[s, idx[:20]] = torch.tensor(1.3, dtype=dtype)
    table = table.to(DEV)
    prow = torch.randperm(slots, generator=g)[:rows].to(torch.int32).to(DEV)
    temp = torch.tensor([1.0, 0.7, 1.3, 0.05, 2.0, 1.0, 0.9, 1.1] * 2, dtype=torch.float32).to(DEV)
    pen_arg = table if which in ("both", "penalty") else None
    temp_arg = temp if which in ("both", "temperature") else None
    ref_logits = _scaled_reference(x, pen_arg, prow, temp_arg)
    ks = torch.tensor([0, 1, 5, 50, vocab, 20, 1000, 0] * 2, dtype=torch.int32).to(DEV)
    ps = torch.tensor([1.0, 1.0, 0.9, 0.5, 0.8, 0.95, 1.0, 0.3] * 2, dtype=torch.float32).to(DEV)
    for trial in range(4):
        u = torch.rand(rows, generator=g).to(DEV)
        got = sample(x, ks, ps, uniform=u, penalty=pen_arg, penalty_rows=prow if pen_arg is not None else None,
                     temperature=temp_arg)
        want = sample(ref_logits.contiguous(), ks, ps, uniform=u)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (dtype, which, trial, got.tolist(), want.tolist())
    # and the draw is the oracle's for the scaled row
    _check_rows(ref_logits.float().cpu(), ks.cpu(), ps.cpu(), u.cpu(), got.cpu())


def test_scaled_sampling_neutral_scaling_is_plain_sampling():
    """A penalty table of ones and temperature 1 change nothing (x / 1 == x)."""
    rows, vocab = 8, 4099  # (odd vocab: the element path for the row tails)
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(rows, vocab, generator=g) * 2).half().to(DEV)
    table = torch.ones(4, vocab, dtype=torch.float16, device=DEV)
    prow = torch.tensor([0, 1, 2, 3, 0, 1, 2, 3], dtype=torch.int32, device=DEV)
    u = torch.rand(rows, generator=g).to(DEV)
    a = sample(x, 30, 0.9, uniform=u, penalty=table, penalty_rows=prow, temperature=1.0)
    b = sample(x, 30, 0.9, uniform=u)
    assert torch.equal(a, b)


def test_scaled_sampling_argument_checks():
    x = torch.randn(4, 100, device=DEV).half()
    table = torch.ones(4, 100, dtype=torch.float16, device=DEV)
    with pytest.raises(ValueError):
        sample(x, 5, 0.9, penalty=table)  # no penalty_rows
    with pytest.raises(ValueError):
        sample(x, 5, 0.9, penalty=table.float(), penalty_rows=torch.zeros(4, dtype=torch.int32, device=DEV))
    with pytest.raises(ValueError):
        sample(x, 5, 0.9, temperature=torch.ones(3, device=DEV))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_scale_logits_is_bitwise_the_eager_scaling(dtype):
    """scale_logits against the serving loop's own tensor ops, value for value."""
    from ecahlang_amd.sampling import scale_logits
    rows, vocab, slots = 12, 50001, 20  # (odd vocab: a partial last group of 8)
    g = torch.Generator().manual_seed(9)
    x = (torch.randn(rows, vocab, generator=g) * 4).to(dtype)
    x[0, :5] = torch.tensor([0.0, -0.0, float("inf"), float("-inf"), 1e-7]).to(dtype)
    x = x.to(DEV)
    table = torch.ones(slots, vocab, dtype=dtype)
    idx = torch.randint(0, vocab, (slots, 500), generator=g)
    table.scatter_(1, idx, (1.0 / torch.empty(slots, 500).uniform_(1.01, 2.0, generator=g)).to(dtype))
    table = table.to(DEV)
    prow = torch.randint(0, slots, (rows,), generator=g).to(torch.int32).to(DEV)
    temp = torch.tensor([1.0, 0.7, 1.3, 0.05, 2.0, 0.99999994, 1.9999999, 0.3, 1.0, 3.7, 0.1, 1.1],
                        dtype=torch.float32).to(DEV)
    for pen, t in ((table, temp), (table, None), (None, temp), (None, 0.8)):
        got = scale_logits(x, pen, prow if pen is not None else None, t)
        want = x
        if pen is not None:
            want = want / pen[prow.long()]
        if t is not None:
            tt = t if isinstance(t, torch.Tensor) else torch.full((rows,), t, dtype=torch.float32, device=DEV)
            want = want / tt.reshape(-1, 1)
        want = want.float()
        torch.cuda.synchronize()
        assert got.dtype == torch.float32
        assert torch.equal(got.view(torch.int32), want.contiguous().view(torch.int32)), (dtype, pen is None, t)


def test_scale_logits_bad_penalty_row_reads_as_nan():
    from ecahlang_amd.sampling import scale_logits
    x = torch.randn(3, 1000, device=DEV).half()
    table = torch.ones(4, 1000, dtype=torch.float16, device=DEV)
    rows = torch.tensor([0, 9, -1], dtype=torch.int32, device=DEV)
    y = scale_logits(x, table, rows, 0.5)
    assert torch.equal(y[0], x[0].float() / 0.5)
    assert torch.isnan(y[1]).all() and torch.isnan(y[2]).all()
    tok = sample(x, 0, 1.0, uniform=torch.full((3,), 0.5, device=DEV), penalty=table, penalty_rows=rows)
    assert tok[1].item() == -1 and tok[2].item() == -1 and 0 <= tok[0].item() < 1000


def _single_wg(x, ks, ps, u):
    """The one-workgroup-per-row kernel (the entry point without a workspace)."""
    from ecahlang_amd._lib import dtype_code, lib, stream_ptr
    rows, vocab = x.shape
    out = torch.empty(rows, dtype=torch.int32, device=DEV)
    k_t = ks if isinstance(ks, torch.Tensor) else None
    p_t = ps if isinstance(ps, torch.Tensor) else None
    rc = lib().pkv_top_k_top_p_sampling(
        x.data_ptr(), x.stride(0), rows, vocab, dtype_code(x.dtype),
        k_t.data_ptr() if k_t is not None else None, 0 if k_t is not None else int(ks),
        p_t.data_ptr() if p_t is not None else None, 1.0 if p_t is not None else float(ps),
        u.data_ptr(), out.data_ptr(), stream_ptr(DEV))
    assert rc == 0
    return out


@pytest.mark.parametrize("dtype,vocab", [(torch.float16, 151936), (torch.bfloat16, 32003), (torch.float32, 50000),
                                         (torch.float16, 2048), (torch.float16, 7)])
def test_whole_row_split_path_equals_single_workgroup(dtype, vocab):
    """Rows sampled from their whole distribution run on many workgroups per row; the token
    must be the one-workgroup kernel's, bit for bit, for the same uniforms."""
    rows = 24
    g = torch.Generator().manual_seed(vocab)
    x = (torch.randn(rows, vocab, generator=g) * 3).to(dtype)
    x[1] = float("nan")                     # no mass: -1
    x[2, : vocab // 2] = float("nan")       # half NaN
    x[3] = 0.0                              # uniform distribution
    x[4, vocab // 3] = 50.0                 # one dominant logit
    x = x.to(DEV)
    u = torch.rand(rows, generator=g).to(DEV)
    u[5], u[6] = 0.0, 0.9999999
    want = _single_wg(x, 0, 1.0, u)
    got = sample(x, 0, 1.0, uniform=u)
    torch.cuda.synchronize()
    assert torch.equal(got, want), (got.tolist(), want.tolist())
    assert got[1].item() == -1
    assert got[4].item() == vocab // 3 or vocab < 3
    # per-row parameters mixing whole rows with filtered ones: both paths in one call
    ks = torch.tensor([0, vocab, 5, 0, 1, 0] * 4, dtype=torch.int32, device=DEV)
    ps = torch.tensor([1.0, 1.0, 1.0, 0.7, 1.0, 1.5] * 4, dtype=torch.float32, device=DEV)
    got2 = sample(x, ks, ps, uniform=u)
    want2 = _single_wg(x, ks, ps, u)
    torch.cuda.synchronize()
    assert torch.equal(got2, want2)


def test_whole_row_split_path_strided_rows_and_graph_replays():
    vocab = 40001
    base = (torch.randn(6, vocab + 5) * 2).half().to(DEV)
    x = base[:, 3:3 + vocab]                 # rows not 16-byte aligned: element loads
    u = torch.rand(6, device=DEV)
    assert torch.equal(sample(x, 0, 1.0, uniform=u), _single_wg(x, 0, 1.0, u))
    torch.manual_seed(11)
    s = torch.cuda.Stream()
    xc = base[:, :vocab].contiguous()
    with torch.cuda.stream(s):
        out = sample(xc, 0, 1.0)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            out = sample(xc, 0, 1.0)
    seen = []
    for _ in range(5):
        graph.replay()
        torch.cuda.synchronize()
        seen.append(out.cpu().clone())
        assert ((seen[-1] >= 0) & (seen[-1] < vocab)).all()
    assert len({tuple(t.tolist()) for t in seen}) > 1


@pytest.mark.parametrize("dtype,vocab", [(torch.float16, 151936), (torch.bfloat16, 32003), (torch.float32, 20000),
                                         (torch.float16, 300)])
def test_top_k_split_path_equals_single_workgroup(dtype, vocab):
    """Top-k rows (k <= 256, any top-p) run on many workgroups per row through per-slice
    candidates; the token must be the one-workgroup kernel's, bit for bit, including rows the
    split path hands back (ties beyond a slice's capacity, fewer than k finite logits)."""
    rows = 32
    g = torch.Generator().manual_seed(vocab + 1)
    x = (torch.randn(rows, vocab, generator=g) * 3).to(dtype)
    x[1] = torch.round(x[1])                          # heavy ties at every threshold
    x[2] = 0.5                                        # one value everywhere: handed back
    x[3, : vocab - 10] = float("nan")                 # fewer than k finite logits: handed back
    x[4, 7] = 40.0                                    # one dominant logit
    x[5, : vocab // 2] = float("-inf")
    x[6] = x[6].sort(descending=True).values           # the top-k all in the first slice
    x = x.to(DEV)
    ks = torch.tensor([50, 1, 20, 5, 256, 3, 200, 2] * 4, dtype=torch.int32, device=DEV)
    ps = torch.tensor([0.9, 1.0, 0.5, 1.0, 0.95, 0.3, 1.0, 0.99] * 4, dtype=torch.float32, device=DEV)
    ks = torch.minimum(ks, torch.tensor(vocab - 1, dtype=torch.int32, device=DEV))
    for trial in range(3):
        u = torch.rand(rows, generator=g).to(DEV)
        got = sample(x, ks, ps, uniform=u)
        want = _single_wg(x, ks, ps, u)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (trial, (got != want).nonzero().flatten().tolist())
    # scalar parameters (only the top-k kernels launched), and k = 257 (the one-workgroup kernel)
    for kk, pp in ((50, 0.9), (1, 1.0), (256, 0.5), (257, 0.9)):
        u = torch.rand(rows, generator=g).to(DEV)
        got = sample(x, min(kk, vocab - 1), pp, uniform=u)
        want = _single_wg(x, min(kk, vocab - 1), pp, u)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (kk, pp)


def test_top_k_split_path_graph_replays():
    x = (torch.randn(16, 151936, device=DEV) * 3).half()
    torch.manual_seed(3)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        out = sample(x, 50, 0.9)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            out = sample(x, 50, 0.9)
    xs = x.float().cpu().numpy()
    seen = []
    for _ in range(4):
        graph.replay()
        torch.cuda.synchronize()
        d = out.cpu().clone()
        seen.append(tuple(d.tolist()))
        for r in range(16):
            assert sr.kept_set(xs[r], 50, 0.9)[int(d[r])]
    assert len(set(seen)) > 1
