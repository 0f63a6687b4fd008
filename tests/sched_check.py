"""Exact checks of a decode schedule against the page table it was planned from.

pkv_decode_plan writes the matrix-core decode's schedule into the workspace (record formats in
ecahlang_amd/csrc/decode_sched.h); the decode attends exactly the pages the schedule lists, so a
schedule that drops, repeats or misplaces a page, or that miscounts a sequence's parts, gives a
wrong result that attention's tolerance may not show.  :func:`check_plain` checks the schedule's
invariants with no tolerance:

* every page of every sequence appears exactly once, in the sequence's order, in the segments
  of consecutive ranges, each segment's page-id words equal to ``kv_indices`` (ids outside
  ``[0, 2^30)`` as -1), segments tiling their range in sequence order;
* a segment's valid-row count is ``kv_last_page_len`` exactly when it holds its sequence's last
  listed page (of an uncut list), else the page size;
* the fused append's mark: exactly one segment of every sequence whose position
  ``seq_len - 1`` exists names that page and row, and no other segment has a mark;
* a sequence's parts are numbered 0 .. n-1 in range order, all with its n and its first slot,
  and the sequences' slot intervals are disjoint and inside the workspace's slot capacity;
* ranges may be empty (no pages, no segments); each range head repeats its record's first
  segments and page ids;
* sequences with no pages are exactly those listed as empty;
* with a shared-prefix hint: a page flagged as shared is read by at least two sequences.

:func:`build_plain` writes a valid plain schedule by a different rule (equal page ranges), so
that the checker can be pinned on the CPU: it accepts that schedule and rejects each planted
mistake (tests/test_sched_check.py).
"""
from __future__ import annotations

import re
from pathlib import Path

import numpy as np

_SCHED_H = Path(__file__).resolve().parents[1] / "ecahlang_amd" / "csrc" / "decode_sched.h"


def consts() -> dict:
    """The integer constants of decode_sched.h (constexpr ints and enum members)."""
    text = re.sub(r"//[^\n]*", "", _SCHED_H.read_text())
    env: dict = {}
    for m in re.finditer(r"constexpr\s+(?:int|int64_t)\s+(\w+\s*=[^;]+);", text):
        for decl in m.group(1).split(","):  # (one declaration may define several names)
            k, v = decl.split("=", 1)
            v = v.replace("/", "//")  # (C integer division; every operand is non-negative)
            env[k.strip()] = int(eval(v, {"__builtins__": {}}, dict(env)))
    for m in re.finditer(r"enum\s+\w+\s*\{([^}]*)\}", text):
        for item in m.group(1).split(","):
            if "=" in item:
                k, v = item.split("=")
                env[k.strip()] = int(eval(v, {"__builtins__": {}}, dict(env)))
    return env


C = consts()
PID_SHARED = C["kPidShared"]
SEG_B_BITS = C["kSegBBits"]


def layout(batch, hq, d, ctas, num_indices, ws_bytes) -> dict:
    """Byte offsets and sizes of the schedule inside a workspace (pkv_decode_schedule_layout)."""
    import ctypes

    from ecahlang_amd._lib import check, lib

    out = (ctypes.c_int64 * 8)()
    check(lib().pkv_decode_schedule_layout(batch, hq, d, ctas, num_indices, ws_bytes, out), "schedule layout")
    keys = ["ghdr", "heads", "recs", "precs", "rcap", "slots", "head_words", "rec_words"]
    return dict(zip(keys, (int(x) for x in out)))


def parse(ws: np.ndarray, lay: dict, batch: int) -> dict:
    """The schedule's arrays from a workspace's bytes (uint8 numpy array)."""
    w32 = ws.view(np.int32)
    g0 = lay["ghdr"] // 4
    ghdr = w32[g0:g0 + C["kGlobHdr"] + batch].copy()
    rc, hw, rw = lay["rcap"], lay["head_words"], lay["rec_words"]
    heads = w32[lay["heads"] // 4: lay["heads"] // 4 + rc * hw].reshape(rc, hw).copy()
    recs = w32[lay["recs"] // 4: lay["recs"] // 4 + rc * rw].reshape(rc, rw).copy()
    return dict(ghdr=ghdr, heads=heads, recs=recs, rcap=rc, slots=lay["slots"])


def _seg_fields(x, y, z, w):
    u = int(x) & 0xFFFFFFFF
    return dict(b=u & ((1 << SEG_B_BITS) - 1), nv=(u >> SEG_B_BITS) & 31, np=u >> (SEG_B_BITS + 5),
                beg=int(y) & 0x3FF, app=(int(y) >> 10) & 63, end=(int(y) >> 16) & 0xFFFF,
                slot0=int(z), part=int(w) & 0xFFFF, nparts=((int(w) >> 16) & 0xFFFF) + 1)


def check_plain(s: dict, indptr, indices, last, num_indices: int, page_size: int,
                hint: bool = False) -> dict:
    """Assert every invariant of a plain (no prefix item) schedule; returns a few counts."""
    indptr = np.asarray(indptr, dtype=np.int64)
    indices = np.asarray(indices, dtype=np.int64)
    last = np.asarray(last, dtype=np.int64)
    B = len(last)
    ghdr, heads, recs = s["ghdr"], s["heads"], s["recs"]
    kGH = C["kGlobHdr"]
    R = int(ghdr[C["kGhRanges"]])
    total = int(min(max(indptr[B], 0), num_indices))
    first = int(min(max(indptr[0], 0), total))
    assert int(ghdr[C["kGhTotal"]]) == total and int(ghdr[C["kGhFirst"]]) == first
    assert int(ghdr[C["kGhItems"]]) == 0, "a plain schedule has no prefix items"
    assert 0 <= R <= s["rcap"], (R, s["rcap"])
    s0 = np.clip(indptr[:-1], first, total)
    s1 = np.clip(indptr[1:], first, total)
    npg = np.maximum(s1 - s0, 0)
    ne = int(ghdr[C["kGhEmpty"]])
    assert sorted(int(b) for b in ghdr[kGH:kGH + ne]) == [b for b in range(B) if npg[b] == 0], "empty list"
    # pages read by more than one sequence (for the shared flags)
    readers: dict = {}
    for b in range(B):
        for pid in set(indices[s0[b]:s1[b]].tolist()):
            readers[pid] = readers.get(pid, 0) + 1
    covered = np.zeros(B, dtype=np.int64)
    parts: dict = {b: [] for b in range(B)}
    apps: dict = {b: [] for b in range(B)}
    RO, PO = C["kRecSegOff"], C["kRecPidOff"]
    HP = C["kHeadPidOff"]
    pages_total = 0
    for w in range(R):
        h, rec = heads[w], recs[w]
        L, nseg = int(h[C["kHdrLen"]]), int(h[C["kHdrNseg"]])
        assert int(h[C["kHdrRanges"]]) == R and int(h[C["kHdrPrefix"]]) == 0, f"range {w} header"
        assert 0 <= L <= C["kRangePages"] and (1 <= nseg <= L or L == nseg == 0), f"range {w}: len {L} nseg {nseg}"
        pages_total += L
        if L == 0:  # (weighted cuts can leave a range empty; the decode skips it)
            continue
        ns_head = min(nseg, C["kHeadSegs"])
        assert np.array_equal(h[RO:RO + 4 * ns_head], rec[RO:RO + 4 * ns_head]), f"range {w} head segments"
        nph = min(L, C["kHeadPids"])
        assert np.array_equal(h[HP:HP + nph], rec[PO:PO + nph]), f"range {w} head page ids"
        segs = [_seg_fields(*rec[RO + 4 * k: RO + 4 * k + 4]) for k in range(nseg)]
        prev_end, prev_b = 0, -1
        for k, sg in enumerate(segs):
            b, beg, end = sg["b"], sg["beg"], sg["end"]
            assert sg["np"] == 0, f"range {w} segment {k}: prefix chunks in a plain schedule"
            assert beg == prev_end and end > beg, f"range {w} segment {k}: [{beg}, {end}) after {prev_end}"
            assert 0 <= b < B and b > prev_b, f"range {w} segment {k}: sequence {b} after {prev_b}"
            prev_end, prev_b = end, b
            k0 = int(covered[b])
            assert k0 + (end - beg) <= npg[b], f"sequence {b}: more pages than listed"
            want = indices[s0[b] + k0: s0[b] + k0 + (end - beg)]
            got = rec[PO + beg: PO + end].astype(np.int64)
            exp = np.where((want < 0) | (want >= PID_SHARED), -1, want)
            flag = (got >= 0) & ((got & PID_SHARED) != 0)
            assert np.array_equal(np.where(got < 0, -1, got & ~PID_SHARED), exp), \
                f"range {w} segment {k}: page ids of sequence {b} pages {k0}..{k0 + end - beg}"
            if hint:
                for pid in exp[flag[: len(exp)]]:
                    assert readers.get(int(pid), 0) >= 2, f"page {pid} flagged shared but read once"
            else:
                assert not flag.any(), f"range {w}: shared flags without a hint"
            covered[b] += end - beg
            uncut = indptr[b + 1] <= total
            holds_last = covered[b] == npg[b] and uncut
            assert sg["nv"] == (int(np.clip(last[b], 0, page_size)) if holds_last else page_size), \
                f"range {w} segment {k} (sequence {b}): valid rows {sg['nv']}"
            if sg["app"]:
                back = (sg["app"] - 1) >> 4
                row = (sg["app"] - 1) & 15
                page = end - 1 - back
                assert beg <= page < end, f"range {w} segment {k}: append page outside the segment"
                apps[b].append((k0 + page - beg, row))
            parts[b].append((sg["part"], sg["nparts"], sg["slot0"]))
        assert prev_end == L, f"range {w}: segments end at {prev_end} of {L}"
    assert pages_total == total - first, f"ranges hold {pages_total} pages of {total - first}"
    assert np.array_equal(covered, npg), "pages of some sequence missing"
    # parts and slots
    intervals = []
    for b in range(B):
        ps = parts[b]
        if npg[b] == 0:
            assert not ps
            continue
        n = len(ps)
        assert [p[0] for p in ps] == list(range(n)), f"sequence {b}: parts {[p[0] for p in ps]}"
        assert all(p[1] == n for p in ps), f"sequence {b}: part counts {[p[1] for p in ps]} for {n} parts"
        slot0 = ps[0][2]
        assert all(p[2] == slot0 for p in ps), f"sequence {b}: first slots differ"
        intervals.append((slot0, slot0 + n, b))
    intervals.sort()
    for (a0, a1, ba), (b0, b1, bb) in zip(intervals, intervals[1:]):
        assert a1 <= b0, f"slots of sequences {ba} and {bb} overlap"
    if intervals:
        assert intervals[0][0] >= 0 and intervals[-1][1] <= s["slots"], "slots outside the workspace"
    # append marks
    n_app = 0
    for b in range(B):
        n = int(indptr[b + 1] - indptr[b])
        lp = int(last[b])
        at = (n - 1) * page_size + lp - 1
        ok = indptr[b + 1] <= total and indptr[b] >= 0 and n >= 1 and 0 <= lp <= page_size and at >= 0
        if ok:
            assert apps[b] == [(at // page_size, at % page_size)], f"sequence {b}: append marks {apps[b]}"
            n_app += 1
        else:
            assert apps[b] == [], f"sequence {b}: append mark without a position"
    return dict(ranges=R, appends=n_app, split=sum(1 for b in range(B) if len(parts[b]) > 1))


def build_plain(indptr, indices, last, num_indices, page_size, R_target, slot_cap=None) -> dict:
    """A valid plain schedule by its own rule (the page list cut into equal ranges), in the
    layout check_plain reads.  For pinning the checker on the CPU only."""
    indptr = np.asarray(indptr, dtype=np.int64)
    indices = np.asarray(indices, dtype=np.int64)
    last = np.asarray(last, dtype=np.int64)
    B = len(last)
    total = int(min(max(indptr[B], 0), num_indices))
    first = int(min(max(indptr[0], 0), total))
    s0 = np.clip(indptr[:-1], first, total)
    s1 = np.clip(indptr[1:], first, total)
    n = total - first
    R = min(R_target, n) if n > 0 else 0
    R = max(R, -(-n // C["kRangePages"])) if n > 0 else 0
    starts = [first + (w * n) // R for w in range(R + 1)] if R else [first]
    hw, rw = C["kHeadWords"], C["kRecStride"]
    heads = np.zeros((max(R, 1), hw), dtype=np.int32)
    recs = np.zeros((max(R, 1), rw), dtype=np.int32)
    ghdr = np.zeros(C["kGlobHdr"] + B, dtype=np.int32)
    empty = [b for b in range(B) if s1[b] <= s0[b]]
    ghdr[C["kGhRanges"]], ghdr[C["kGhEmpty"]] = R, len(empty)
    ghdr[C["kGhTotal"]], ghdr[C["kGhFirst"]] = total, first
    ghdr[C["kGlobHdr"]:C["kGlobHdr"] + len(empty)] = empty
    # parts: ranges each sequence touches
    touch = {b: [w for w in range(R) if s0[b] < starts[w + 1] and s1[b] > starts[w]] for b in range(B)}
    slot0, nxt = {}, 0
    for b in range(B):
        slot0[b] = nxt
        nxt += len(touch[b])
    RO, PO, HP = C["kRecSegOff"], C["kRecPidOff"], C["kHeadPidOff"]
    for w in range(R):
        rs, re_ = starts[w], starts[w + 1]
        L = re_ - rs
        segs = []
        for b in range(B):
            a, e = max(s0[b], rs), min(s1[b], re_)
            if e <= a:
                continue
            beg, end = a - rs, e - rs
            uncut = indptr[b + 1] <= total
            nv = int(np.clip(last[b], 0, page_size)) if (e == s1[b] and uncut) else page_size
            nb = int(indptr[b + 1] - indptr[b])
            lp = int(last[b])
            at = (nb - 1) * page_size + lp - 1
            app = 0
            if uncut and nb >= 1 and 0 <= lp <= page_size and at >= 0:
                tp = s0[b] + at // page_size  # list position of the token's page
                if a <= tp < e:
                    app = 1 + (((end - 1 - (tp - rs)) << 4) | (at % page_size))
            part = touch[b].index(w)
            segs.append((b | (nv << SEG_B_BITS), beg | (app << 10) | (end << 16), slot0[b],
                         part | ((len(touch[b]) - 1) << 16)))
            for i in range(a, e):
                pid = int(indices[i])
                recs[w, PO + i - rs] = -1 if (pid < 0 or pid >= PID_SHARED) else pid
        for k, sg in enumerate(segs):
            recs[w, RO + 4 * k: RO + 4 * k + 4] = sg
        heads[w, :4] = (L, len(segs), R, 0)
        nh = min(len(segs), C["kHeadSegs"])
        heads[w, RO:RO + 4 * nh] = recs[w, RO:RO + 4 * nh]
        heads[w, HP:HP + min(L, C["kHeadPids"])] = recs[w, PO:PO + min(L, C["kHeadPids"])]
    return dict(ghdr=ghdr, heads=heads, recs=recs, rcap=max(R, 1),
                slots=slot_cap if slot_cap is not None else max(nxt, 1))

