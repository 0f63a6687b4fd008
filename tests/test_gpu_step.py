"""The multi-layer decode step over a shared prefix (workloads.SharedPrefixDecodeLoop):
page tables from the device pool against the oracle's pool replaying the same operations
(prefix sharing, per-step appends with on-device page pops, frees and refills), every
layer's appended K/V in place bit for bit, and the graph-replayed decode outputs against the
oracle's attention over the pages read back."""
import numpy as np
import pytest
import torch

import sched_check as sc

from ecahlang_amd import workloads
from oracle import kv_ref
from oracle.manager_ref import RefKVCacheManager

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _replay_log(loop, ref, start):
    """Apply loop.log[start:] to the oracle pool; return the last graph metadata it built."""
    meta = None
    for op in loop.log[start:]:
        if op[0] == "allocate":
            ref.allocate(op[1], op[2], prefix=op[3])
        elif op[0] == "append_tokens":
            ref.append_tokens(op[1], op[2])
        elif op[0] == "free":
            ref.free(op[1])
        elif op[0] == "init_cuda_graph_buffers":
            ref.init_cuda_graph_buffers(op[1])
        elif op[0] == "fill_cuda_graph_metadata":
            meta = ref.fill_cuda_graph_metadata(op[1], op[2])
        else:
            raise AssertionError(op)
    return meta


def _check_layer(loop, layer, rows, idx, ptr, last):
    """Append in place (bitwise) and decode output (oracle tolerance) for batch rows."""
    cache = loop.mgr.kv_cache[layer]
    for r in rows:
        pages = torch.tensor(idx[ptr[r]:ptr[r + 1]], dtype=torch.long, device=DEV)
        L = (len(pages) - 1) * 16 + last[r]
        p, s = pages[(L - 1) // 16], (L - 1) % 16
        assert torch.equal(cache[p, 0, s], loop.k[layer, r]), (layer, r)
        assert torch.equal(cache[p, 1, s], loop.v[layer, r]), (layer, r)
        kv = cache[pages].float().cpu().numpy()
        k = kv[:, 0].reshape(-1, loop.hkv, loop.d)[:L]
        v = kv[:, 1].reshape(-1, loop.hkv, loop.d)[:L]
        q = loop.q[layer, r:r + 1].float().cpu().numpy().astype(np.float64)
        ref = kv_ref._attend(q, k, v, [L], loop.d ** -0.5)[0]
        got = loop.out[layer, r].float().cpu().numpy()
        np.testing.assert_allclose(got, ref, atol=2e-3, rtol=1e-2, err_msg=f"layer {layer} row {r}")


@pytest.mark.parametrize("hint,cascade,device_steps", [(True, False, False), (False, False, False),
                                                       (True, True, False), (True, False, True),
                                                       (True, True, True)])
def test_small_loop_matches_oracle_every_step(hint, cascade, device_steps):
    """With the manager's shared-prefix hint (the prefix's pages kept in L2), without it, with
    the cascade (the prefix read once per group), with the whole step in the graph (the
    page-table step on the device), and with both (the shared-prefix step's bench setting)."""
    loop = workloads.SharedPrefixDecodeLoop(DEV, layers=3, batch=16, prefix_tokens=256, suffix=(1, 200),
                                            finish=4, max_steps=12, seed=7, record=True,
                                            shared_hint=hint, cascade=cascade, device_steps=device_steps)
    ref = RefKVCacheManager(loop.mgr.max_blocks, seq_lens=loop.mgr.seq_lens)
    done = 0
    for step in range(8):
        print(f"small loop step {step}", flush=True)
        loop.new_inputs()
        loop.begin_step()
        loop.replay()
        torch.cuda.synchronize()
        idx, ptr, last, pos = _replay_log(loop, ref, done)
        done = len(loop.log)
        b = loop.batch
        assert loop.mgr._cg_kv_indices[b][:len(idx)].tolist() == idx
        assert loop.mgr._cg_kv_indptr[b].tolist() == ptr
        assert loop.mgr._cg_kv_last_page_len[b].tolist() == last
        assert loop.mgr._cg_positions[b].tolist() == pos
        # every sequence starts with the prefix's 16 full pages
        pre = ref.batch_to_blocks["prefix"][:16]
        assert all(idx[ptr[r]:ptr[r] + 16] == pre for r in range(b))
        for layer in range(loop.layers):
            _check_layer(loop, layer, range(b), idx, ptr, last)
        loop.retire()
    _replay_log(loop, ref, done)
    assert list(loop.mgr.free_blocks) == ref.free_blocks
    assert loop.mgr.pool_errors() == 0


@pytest.mark.parametrize("device_steps", [False, True])
def test_full_size_step_qwen_36_layers(device_steps):
    """Qwen2.5-3B attention shape, 36 layers, batch 128, 2048-token shared prefix: three steps
    (the graph captured on the first), then layers 0 and 17 checked on 8 sequences and layer 35
    on all 128; between steps, 8 sequences retired and replaced, their tokens written after the
    pool's part of the batch change."""
    loop = workloads.SharedPrefixDecodeLoop(DEV, max_steps=6, record=True, device_steps=device_steps)
    ref = RefKVCacheManager(loop.mgr.max_blocks, seq_lens=loop.mgr.seq_lens)
    done = 0
    for step in range(3):
        print(f"full loop step {step}", flush=True)
        loop.begin_step()
        loop.replay()
        torch.cuda.synchronize()
        idx, ptr, last, pos = _replay_log(loop, ref, done)
        done = len(loop.log)
        assert loop.mgr._cg_kv_indptr[loop.batch].tolist() == ptr
        assert loop.mgr._cg_kv_indices[loop.batch][:len(idx)].tolist() == idx
        if step == 2:
            rows = list(range(0, loop.batch, loop.batch // 8))
            for layer in (0, 17, 35):
                _check_layer(loop, layer, rows if layer < 35 else list(range(loop.batch)), idx, ptr, last)
        # the batch change as the benchmark times it: the pool's part, then the new sequences'
        # tokens written (with device steps, after the new batch is on the device)
        _, new = loop.retire(write_tokens=False)
        loop.write_tokens(new)
        if device_steps:
            assert loop.mgr._dev is not None
    assert loop.mgr.pool_errors() == 0


def test_full_size_cascade_and_hint_match_plain():
    """Qwen2.5-3B shape, batch 128 on a 2048-token shared prefix: the cascade plan (prefix items
    carried by ranges that also hold suffix pages) and the shared-page hint give the plain plan's
    outputs, and rows of all three match the oracle."""
    loop = workloads.SharedPrefixDecodeLoop(DEV, layers=1, max_steps=2)
    loop.begin_step()
    loop.mgr.append_paged_kv_cache_cuda_graph(loop.k[0], loop.v[0], loop.batch, 0)
    torch.cuda.synchronize()
    m, w, B = loop.mgr, loop.wrapper, loop.batch
    outs = {}
    items = {}
    for mode in ("plain", "hint", "cascade"):
        print(f"full-size shared prefix: {mode}", flush=True)
        w.plan(m._cg_kv_indptr[B], m._cg_kv_indices[B], m._cg_kv_last_page_len[B], loop.hq, loop.hkv, loop.d, 16,
               q_data_type=loop.dtype, kv_shared_pages=m._cg_kv_shared[B] if mode != "plain" else None,
               cascade=mode == "cascade")
        out = torch.empty_like(loop.out[0])
        w.run(loop.q[0], m.kv_cache[0], out=out)
        torch.cuda.synchronize()
        outs[mode] = out.float()
        # the plan's global header (after the per-sequence words): [ranges, ..., prefix items]
        off = sc.layout(B, loop.hq, loop.d, w._ctas, m._cg_kv_indices[B].numel(), w._workspace.numel())["ghdr"]
        items[mode] = w._workspace[off:off + 32].view(torch.int32).tolist()[4]
    assert items["plain"] == 0 and items["cascade"] > 0, items
    assert torch.isfinite(outs["cascade"]).all()
    torch.testing.assert_close(outs["hint"], outs["plain"], atol=0, rtol=0)
    # the plans differ only in fp32 summation order (3e-5 apart at this shape); a suffix read
    # through the wrong page list lands ~7e-3 away
    torch.testing.assert_close(outs["cascade"], outs["plain"], atol=5e-4, rtol=0)
    idx = m._cg_kv_indices[B].tolist()
    ptr = m._cg_kv_indptr[B].tolist()
    last = m._cg_kv_last_page_len[B].tolist()
    cache = m.kv_cache[0]
    for r in (0, 37, 64, 127):
        pages = torch.tensor(idx[ptr[r]:ptr[r + 1]], dtype=torch.long, device=DEV)
        L = (len(pages) - 1) * 16 + last[r]
        kv = cache[pages].float().cpu().numpy()
        k = kv[:, 0].reshape(-1, loop.hkv, loop.d)[:L]
        v = kv[:, 1].reshape(-1, loop.hkv, loop.d)[:L]
        q = loop.q[0, r:r + 1].float().cpu().numpy().astype(np.float64)
        ref = kv_ref._attend(q, k, v, [L], loop.d ** -0.5)[0]
        for mode in ("plain", "cascade"):
            np.testing.assert_allclose(outs[mode][r].cpu().numpy(), ref, atol=2e-3, rtol=1e-2,
                                       err_msg=f"{mode} row {r}")
