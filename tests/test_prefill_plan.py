"""The matrix-core prefill's work list (``wrappers.prefill_work_list``, the host half of
BatchPrefillWithPagedKVCacheWrapper.plan) on the CPU: every (request, KV head, query tile) sees
exactly the keys causal (bottom-right aligned) or full attention gives it, cut into chunks that
tile that range without gaps or overlaps, and every split group's record matches its chunks."""
import random

import pytest

from ecahlang_amd.wrappers import prefill_work_list


def _batch(rng, n):
    qo, kv, last = [0], [0], []
    for _ in range(n):
        q = rng.choice([0, 1, 7, 64, 300, 512])
        L = q + rng.choice([0, 1, 15, 16, 200, 3000, 9000])  # keys after the append
        pages = -(-L // 16)
        qo.append(qo[-1] + q)
        kv.append(kv[-1] + pages)
        last.append(L - 16 * (pages - 1) if pages else 0)
    return qo, kv, last


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("causal", [True, False])
def test_work_list_covers_each_tile_exactly(seed, causal):
    rng = random.Random(seed)
    g, hkv, rows = rng.choice([(8, 2, 256), (4, 8, 256), (16, 1, 256), (1, 8, 256)])
    qo, kv, last = _batch(rng, rng.randint(1, 9))
    ncu = rng.choice([8, 64, 256])
    wl = prefill_work_list(qo, kv, last, g, hkv, 16, causal, 128, ncu, 1 << 30, rows)
    chunk, items, groups = wl["chunk"], wl["items"], wl["groups"]
    assert chunk % 64 == 0 and 256 <= chunk <= 8192
    tq_max = rows // g
    want = {}
    for b in range(len(qo) - 1):
        qo_len, pages = qo[b + 1] - qo[b], kv[b + 1] - kv[b]
        kv_len = (pages - 1) * 16 + last[b] if pages else 0
        for t0 in range(0, qo_len, tq_max):
            tq = min(tq_max, qo_len - t0)
            # brute force: the most keys any query token of the tile sees
            see = max(min(kv_len, max(0, t + kv_len - qo_len + 1)) if causal else kv_len for t in range(t0, t0 + tq))
            for h in range(hkv):
                want[(b, h, t0)] = (tq, see, kv_len, qo_len, qo[b], kv[b])
    got = {}
    for it in items:
        b, h, t0, tq, k0, k1, slot, kv_len, qo_len, qo_start, kp0, z = it
        assert (tq, kv_len, qo_len, qo_start, kp0) == tuple(want[(b, h, t0)][i] for i in (0, 2, 3, 4, 5))
        assert z == 0 and 0 <= k0 <= k1 and k1 - k0 <= chunk and k0 % chunk == 0
        got.setdefault((b, h, t0), []).append((k0, k1, slot))
    assert set(got) == set(want)
    for key, parts in got.items():
        parts.sort()
        see = want[key][1]
        assert parts[0][0] == 0 and parts[-1][1] == see, (key, parts, see)
        assert all(parts[i][1] == parts[i + 1][0] for i in range(len(parts) - 1))
        if len(parts) == 1:
            assert parts[0][2] == -1
        else:  # a split group: consecutive slots, and its record names them
            slots = [p[2] for p in parts]
            assert slots == list(range(slots[0], slots[0] + len(parts)))
            b, h, t0 = key
            rec = [gr for gr in groups if gr[0] == slots[0]]
            assert rec == [[slots[0], len(parts), qo[b], t0, want[key][0], h, 0, 0]]
    assert wl["slots"] == sum(gr[1] for gr in groups)
    lens = [it[5] - it[4] for it in items]
    assert lens == sorted(lens, reverse=True)
    assert wl["off_groups"] % 256 == 0 and wl["off_ml"] % 256 == 0 and wl["off_o"] % 256 == 0
    assert wl["off_groups"] >= 48 * len(items) and wl["off_ml"] - wl["off_groups"] >= 32 * len(groups)


def test_chunks_grow_to_fit_the_workspace_or_the_plan_fails():
    qo, kv, last = [0, 512, 1024], [0, 600, 1200], [16, 16]  # two 512-row chunks on 9600 keys
    small = prefill_work_list(qo, kv, last, 8, 2, 16, True, 128, 256, 1 << 30, chunk=512)
    tight = prefill_work_list(qo, kv, last, 8, 2, 16, True, 128, 256, small["bytes"] // 2)
    assert tight["chunk"] > small["chunk"] and tight["bytes"] <= small["bytes"] // 2
    with pytest.raises(RuntimeError, match="prefill workspace too small"):
        prefill_work_list(qo, kv, last, 8, 2, 16, True, 128, 256, 4096)
    # fp16 partials take half the bytes of fp32 ones: a workspace that fp32 partials overflow at
    # the roomy chunk holds the fp16 plan unchanged
    roomy = prefill_work_list(qo, kv, last, 8, 2, 16, True, 128, 256, 1 << 30)
    fits_half = roomy["off_o"] + (roomy["bytes"] - roomy["off_o"]) // 2
    assert fits_half < roomy["bytes"]
    half = prefill_work_list(qo, kv, last, 8, 2, 16, True, 128, 256, fits_half, partial_bytes=2)
    assert half["chunk"] == roomy["chunk"] and half["slots"] == roomy["slots"]
    assert half["bytes"] - half["off_o"] == (roomy["bytes"] - roomy["off_o"]) // 2


# A restatement of the list for a given chunk (the tiles, their key ranges, the chunks and their
# slots, the longest-first order) and of the makespan model the planner minimises.
def _groups(qo, kv, last, g, hkv, causal, rows=256):
    tq_max, out = rows // g, []
    for b in range(len(qo) - 1):
        qo_len, npg = qo[b + 1] - qo[b], kv[b + 1] - kv[b]
        kv_len = (npg - 1) * 16 + last[b] if npg > 0 else 0
        for t0 in range(0, qo_len, tq_max):
            tq = min(tq_max, qo_len - t0)
            kv_end = min(kv_len, max(0, t0 + tq + kv_len - qo_len)) if causal else kv_len
            for h in range(hkv):
                out.append((h, t0, tq, kv_end, kv_len, qo_len, qo[b], kv[b], b))
    return out


def _list_for(groups, chunk):
    items, merges, nslots = [], [], 0
    for (h, t0, tq, kv_end, kv_len, qo_len, qo_start, kp0, b) in groups:
        nch = max(1, -(-kv_end // chunk))
        if nch == 1:
            items.append([b, h, t0, tq, 0, kv_end, -1, kv_len, qo_len, qo_start, kp0, 0])
            continue
        for c in range(nch):
            items.append([b, h, t0, tq, c * chunk, min(kv_end, (c + 1) * chunk), nslots + c, kv_len, qo_len,
                          qo_start, kp0, 0])
        merges.append([nslots, nch, qo_start, t0, tq, h, 0, 0])
        nslots += nch
    items.sort(key=lambda it: it[4] - it[5])  # (stable) longest first
    return items, merges


def _makespan(items, ncu):
    import heapq
    load = [0.0] * ncu
    for it in items:
        t = heapq.heappop(load) + 11.0 + (6.0 if it[6] >= 0 else 0.0) + 1.9 * -(-(it[5] - it[4]) // 64)
        heapq.heappush(load, t)
    return max(load)


@pytest.mark.parametrize("seed", range(4))
def test_given_chunk_and_chosen_chunk_match_the_restatement(seed):
    rng = random.Random(100 + seed)
    qo, kv, last = _batch(rng, rng.randint(2, 9))
    g, hkv = rng.choice([(8, 2), (4, 8), (1, 8)])
    causal = bool(seed % 2)
    ncu = rng.choice([64, 256])
    groups = _groups(qo, kv, last, g, hkv, causal)
    for chunk in (256, 1024, 4096):
        wl = prefill_work_list(qo, kv, last, g, hkv, 16, causal, 128, ncu, 1 << 40, chunk=chunk)
        items, merges = _list_for(groups, chunk)
        assert wl["chunk"] == chunk and wl["items"] == items and wl["groups"] == merges
    # without a chunk: the candidate with the lowest simulated kernel time (ties to the longer)
    total = sum(gr[3] for gr in groups)
    per_cu = -(-total // ncu)
    cands = sorted({min(8192, max(256, (per_cu * f // 16 + 32) // 64 * 64)) for f in (8, 10, 12, 14, 16, 17, 18, 20, 24)})
    times = {c: _makespan(_list_for(groups, c)[0], ncu) for c in cands}
    want = min(cands, key=lambda c: (times[c], -c))
    wl = prefill_work_list(qo, kv, last, g, hkv, 16, causal, 128, ncu, 1 << 40)
    assert wl["chunk"] == want, (wl["chunk"], times)
    assert (wl["items"], wl["groups"]) == _list_for(groups, want)
