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
