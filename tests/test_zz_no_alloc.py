"""pkv_batch_decode_noalloc (the decode entry point that allocates nothing: its workspace is a
file-scope device array) against the planned decode through a caller workspace
(BatchDecodeWithPagedKVCacheWrapper.plan + run, i.e. pkv_decode_plan + pkv_batch_decode), on two
calls in a row, the second with a smaller batch, and against the oracle."""
import numpy as np
import pytest
import torch

from ecahlang_amd import _lib, ops, workloads
from ecahlang_amd.wrappers import BatchDecodeWithPagedKVCacheWrapper
from oracle import kv_ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _noalloc(dv, ctas):
    out = torch.empty_like(dv.q)
    k, v = dv.cache[:, 0], dv.cache[:, 1]
    rc = _lib.lib().pkv_batch_decode_noalloc(
        dv.q.data_ptr(), dv.q.stride(0), dv.q.stride(1), k.data_ptr(), v.data_ptr(), dv.cache.stride(0),
        dv.cache.shape[0], dv.indptr.data_ptr(), dv.indices.data_ptr(), dv.indices.numel(), dv.last.data_ptr(),
        dv.batch, dv.hq, dv.hkv, dv.d, dv.ps, dv.d ** -0.5, ctas, out.data_ptr(), out.stride(0), out.stride(1),
        _lib.dtype_code(dv.dtype), _lib.stream_ptr(DEV))
    _lib.check(rc, "pkv_batch_decode_noalloc")
    return out


@pytest.mark.parametrize("case", ["qwen", "llama"])
def test_noalloc_decode_matches_workspace_decode_twice(case):
    if case == "qwen":  # the Qwen2.5-3B B=64 batch, then a smaller one
        batches = [workloads.qwen25_3b_decode(), workloads.qwen25_3b_decode(batch=9, lo=20, hi=900, seed=4)]
    else:  # Llama-3.1-8B shape (four head blocks), bf16
        batches = [workloads.llama31_8b_decode(batch=16, lo=100, hi=3000),
                   workloads.llama31_8b_decode(batch=5, lo=10, hi=400, seed=9)]
    for i, wb in enumerate(batches):
        print(f"{case} call {i}: B={wb.batch} pages={int(wb.indptr[-1])}", flush=True)
        dv = wb.to(DEV)
        ops.append_paged_kv_cache(dv.k_new, dv.v_new, dv.batch_indices, dv.positions, dv.cache, dv.indices,
                                  dv.indptr, dv.last)
        ctas = torch.cuda.get_device_properties(DEV).multi_processor_count
        w = BatchDecodeWithPagedKVCacheWrapper(torch.empty(128 << 20, dtype=torch.uint8, device=DEV))
        w.plan(dv.indptr, dv.indices, dv.last, wb.hq, wb.hkv, wb.d, wb.ps, q_data_type=wb.dtype, num_ctas=ctas)
        want = w.run(dv.q, dv.cache)
        got = _noalloc(dv, ctas)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"{case} call {i}"
        iv = torch.int16
        raw = kv_ref.append(wb.cache.view(iv).numpy(), wb.k_new.view(iv).numpy(), wb.v_new.view(iv).numpy(),
                            wb.batch_indices.numpy(), wb.positions.numpy(), wb.indices.numpy(),
                            wb.indptr.numpy(), wb.ps)
        vals = torch.from_numpy(raw).view(wb.dtype).float().numpy()
        ref = kv_ref.decode(wb.q.float().numpy(), vals, wb.indptr.numpy(), wb.indices.numpy(), wb.last.numpy(),
                            wb.ps)
        np.testing.assert_allclose(got.float().cpu().numpy(), ref, atol=2e-3, rtol=1e-2)


def test_noalloc_vector_alu_path_matches_workspace_decode_twice():
    """fp32 takes the vector-ALU decode (no plan): the array's split counters and partials
    against a caller workspace, bitwise, on two calls in a row, the second smaller."""
    for i, (lens, seed) in enumerate([([37, 900, 1500, 16, 333, 1200, 64, 700, 2048, 5, 480, 1001], 21),
                                      ([300, 17, 90], 22)]):
        wb = workloads.build_batch(lens, [1] * len(lens), 8, 2, 64, torch.float32, seed=seed)
        print(f"fp32 call {i}: B={wb.batch} pages={int(wb.indptr[-1])}", flush=True)
        dv = wb.to(DEV)
        ops.append_paged_kv_cache(dv.k_new, dv.v_new, dv.batch_indices, dv.positions, dv.cache, dv.indices,
                                  dv.indptr, dv.last)
        ctas = 64
        w = BatchDecodeWithPagedKVCacheWrapper(torch.empty(128 << 20, dtype=torch.uint8, device=DEV))
        w.plan(dv.indptr, dv.indices, dv.last, wb.hq, wb.hkv, wb.d, wb.ps, q_data_type=wb.dtype, num_ctas=ctas)
        assert not w._mfma
        want = w.run(dv.q, dv.cache)
        got = _noalloc(dv, ctas)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int32), want.view(torch.int32)), f"fp32 call {i}"
        ref = kv_ref.decode(wb.q.numpy(), dv.cache.cpu().numpy(), wb.indptr.numpy(), wb.indices.numpy(),
                            wb.last.numpy(), wb.ps)
        np.testing.assert_allclose(got.cpu().numpy(), ref, atol=1e-4, rtol=1e-4)
