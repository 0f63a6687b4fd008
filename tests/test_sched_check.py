"""The decode-schedule checker (tests/sched_check.py) pinned on the CPU: it accepts valid plain
schedules written by an independent rule, over page tables with the edge cases the plan must
handle, and rejects each kind of planted mistake.  The GPU tests then apply it to the schedules
pkv_decode_plan writes."""
import copy

import numpy as np
import pytest

import sched_check as sc

PS = 16


def _table(rng, lens, lp_override=None, lead=0, pool=None, bad_ids=0):
    """CSR page table of sequences of `lens` tokens (FlashInfer convention), pages a random
    permutation; `lead` unused entries before indptr[0]; `bad_ids` ids set outside the pool."""
    npages = [0 if L == 0 else (L + PS - 1) // PS for L in lens]
    total = sum(npages)
    pool = pool or total + lead + 8
    perm = rng.permutation(pool)[: total + lead]
    indptr = np.concatenate([[lead], lead + np.cumsum(npages)]).astype(np.int64)
    last = np.array([0 if L == 0 else (L - 1) % PS + 1 for L in lens], dtype=np.int64)
    if lp_override:
        for b, v in lp_override.items():
            last[b] = v
    indices = perm.astype(np.int64)
    for i in rng.choice(len(indices), size=bad_ids, replace=False) if bad_ids else []:
        indices[i] = -5 if i % 2 else (1 << 30) + 3
    return indptr, indices, last


CASES = [
    dict(lens=[17, 64, 129, 300], R=8),
    dict(lens=[513, 4097, 900, 2048, 16, 1], R=16),
    dict(lens=[0, 40, 0, 33, 0], R=4),                       # empty rows
    dict(lens=[32, 48, 16], R=3, lp={0: 0, 1: 16}),          # empty trailing page, full page
    dict(lens=[100, 200, 300], R=5, lead=7),                 # entries before indptr[0]
    dict(lens=[3 * 16, 5 * 16, 7 * 16], R=4, cut=10),        # num_indices cuts the list
    dict(lens=[16 * 600, 16 * 50], R=1),                     # ranges forced past 512 pages
    dict(lens=[1] * 40, R=5),                                # one-page sequences
    dict(lens=[2000, 17, 3000], R=7, bad=5),                 # ids outside the pool
]


def _case(c, seed):
    rng = np.random.default_rng(seed)
    indptr, indices, last = _table(rng, c["lens"], c.get("lp"), c.get("lead", 0), bad_ids=c.get("bad", 0))
    num_indices = int(indptr[-1]) - c.get("cut", 0)
    s = sc.build_plain(indptr, indices, last, num_indices, PS, c["R"])
    return s, (indptr, indices, last, num_indices, PS)


def test_constants_parse_from_the_schedule_header():
    C = sc.C
    assert C["kRecPidOff"] == C["kRecSegOff"] + 4 * C["kRangePages"]
    assert C["kRecStride"] % 64 == 0 and C["kRecStride"] >= C["kRecPidOff"] + C["kRangePages"]
    assert C["kHeadPidOff"] + C["kHeadPids"] <= C["kHeadWords"]
    assert C["kPidShared"] == 1 << 30


@pytest.mark.parametrize("k", range(len(CASES)))
def test_checker_accepts_valid_schedules(k):
    s, args = _case(CASES[k], seed=k)
    out = sc.check_plain(s, *args)
    assert out["ranges"] >= 1


def _mutations(s):
    """(name, mutated schedule) pairs, each one plausible planning mistake."""
    RO, PO, HP = sc.C["kRecSegOff"], sc.C["kRecPidOff"], sc.C["kHeadPidOff"]
    out = []

    def mut(name, fn):
        t = copy.deepcopy(s)
        fn(t)
        out.append((name, t))

    def seg(t, w, k):
        return sc._seg_fields(*t["recs"][w, RO + 4 * k: RO + 4 * k + 4])

    def put(t, w, k, **kw):
        f = seg(t, w, k)
        f.update(kw)
        words = (f["b"] | (f["nv"] << sc.SEG_B_BITS) | (f["np"] << (sc.SEG_B_BITS + 5)),
                 f["beg"] | (f["app"] << 10) | (f["end"] << 16), f["slot0"], f["part"] | ((f["nparts"] - 1) << 16))
        t["recs"][w, RO + 4 * k: RO + 4 * k + 4] = np.array(words, dtype=np.int64).astype(np.int32)
        if k < sc.C["kHeadSegs"]:
            t["heads"][w, RO + 4 * k: RO + 4 * k + 4] = t["recs"][w, RO + 4 * k: RO + 4 * k + 4]

    w = 0
    L = int(s["heads"][w, 0])
    nseg = int(s["heads"][w, 1])
    lastk = nseg - 1

    def drop_last_page(t):  # the range forgets its last page
        put(t, w, lastk, end=seg(t, w, lastk)["end"] - 1)
        t["heads"][w, 0] = L - 1
    mut("dropped page", drop_last_page)

    def dup_page(t):
        t["recs"][w, PO + 1] = t["recs"][w, PO]
        t["heads"][w, HP + 1] = t["heads"][w, HP]
    mut("duplicated page id", dup_page)
    mut("valid rows", lambda t: put(t, w, 0, nv=(seg(t, w, 0)["nv"] % 16) + 1))
    mut("part count", lambda t: put(t, w, 0, nparts=seg(t, w, 0)["nparts"] + 1))
    mut("first slot", lambda t: put(t, w, 0, slot0=seg(t, w, 0)["slot0"] + 1))
    mut("part number", lambda t: put(t, w, 0, part=seg(t, w, 0)["part"] + 1))

    def app_move(t):
        f = seg(t, w, 0)
        put(t, w, 0, app=0 if f["app"] else 1)
    mut("append mark", app_move)

    def head_copy(t):
        t["heads"][w, HP] = t["heads"][w, HP] ^ 1
    mut("head page id", head_copy)

    def empty_list(t):
        t["ghdr"][sc.C["kGhEmpty"]] += 1
    mut("empty list", empty_list)

    def shared_flag(t):
        t["recs"][w, PO] |= sc.PID_SHARED
        t["heads"][w, HP] |= sc.PID_SHARED
    mut("shared flag without a hint", shared_flag)
    return out


def test_checker_rejects_each_planted_mistake():
    c = dict(lens=[100, 300, 77, 640, 33], R=6)
    s, args = _case(c, seed=11)
    sc.check_plain(s, *args)
    muts = _mutations(s)
    assert len(muts) >= 10
    for name, t in muts:
        with pytest.raises(AssertionError):
            sc.check_plain(t, *args)


def test_checker_rejects_overlapping_slots():
    c = dict(lens=[100, 300, 77], R=4)
    s, args = _case(c, seed=3)
    RO = sc.C["kRecSegOff"]
    # give the last range's segments the slots of the first sequence
    w = int(s["ghdr"][0]) - 1
    f0 = sc._seg_fields(*s["recs"][0, RO: RO + 4])
    nseg = int(s["heads"][w, 1])
    for k in range(nseg):
        r = s["recs"][w, RO + 4 * k: RO + 4 * k + 4].copy()
        if sc._seg_fields(*r)["b"] != f0["b"]:
            s["recs"][w, RO + 4 * k + 2] = f0["slot0"]
            s["heads"][w, RO + 4 * k + 2] = f0["slot0"]
    with pytest.raises(AssertionError):
        sc.check_plain(s, *args)


def test_schedule_layout_fits_the_workspace():
    from ecahlang_amd._lib import lib

    need = int(lib().pkv_decode_workspace_bytes(64, 16, 128, 256, 12000))
    lay = sc.layout(64, 16, 128, 256, 12000, need)
    assert 0 < lay["ghdr"] < lay["heads"] < lay["recs"] < lay["precs"] < need
    assert lay["head_words"] == sc.C["kHeadWords"] and lay["rec_words"] == sc.C["kRecStride"]
    assert lay["rcap"] >= 256 and lay["slots"] >= lay["rcap"] + 64
    assert lay["recs"] + 4 * lay["rcap"] * lay["rec_words"] <= lay["precs"]
