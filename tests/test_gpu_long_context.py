"""Long-context decode at full size: Llama-3.1-8B shape (32 q / 8 kv heads, head_dim 128,
bf16), batch 128, contexts log-uniform in [1024, 32768] (~73k pages, ~4.8 GB of K/V) scattered
over a ~20 GB pool.  Every sequence is split across many workgroups.  The matrix-core output is
checked against the float64 oracle for every sequence, its K/V read back from the device, and
against the vector-ALU kernel (tests/test_gpu_decode_exact.py checks the same shape's outputs in
closed form, which a dropped or repeated page cannot pass)."""
import numpy as np
import pytest
import torch

from ecahlang_amd import workloads
from ecahlang_amd.wrappers import BatchDecodeWithPagedKVCacheWrapper
from oracle import kv_ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@torch.no_grad()
def test_llama31_8b_long_context_decode_full_size():
    wb = workloads.llama31_8b_decode_device(DEV)
    B = wb.batch
    print(f"C4: B={B} pages={int(wb.indptr[-1])} pool={wb.num_pages} tokens={sum(wb.kv_len)}", flush=True)
    ws = torch.empty(256 << 20, dtype=torch.uint8, device=DEV)
    w = BatchDecodeWithPagedKVCacheWrapper(ws, "NHD")
    w.plan(wb.indptr, wb.indices, wb.last, wb.hq, wb.hkv, wb.d, wb.ps, q_data_type=wb.dtype)
    assert w._mfma
    o = w.run(wb.q, wb.cache).float()
    wsv = torch.empty(256 << 20, dtype=torch.uint8, device=DEV)
    wv = BatchDecodeWithPagedKVCacheWrapper(wsv, "NHD")
    wv.plan(wb.indptr, wb.indices, wb.last, wb.hq, wb.hkv, wb.d, wb.ps, q_data_type=wb.dtype)
    ov = wv.run(wb.q, wb.cache, force_valu=True).float()
    torch.cuda.synchronize()
    assert torch.isfinite(o).all()
    # two bf16 results, each within the oracle tolerance: within twice it of each other
    np.testing.assert_allclose(o.cpu().numpy(), ov.cpu().numpy(), atol=4e-3, rtol=2e-2)

    lens = np.array(wb.kv_len)
    indptr = wb.indptr.cpu().numpy()
    for b in range(B):
        pages = wb.indices[indptr[b]:indptr[b + 1]].long()
        L = int(lens[b])
        k = wb.cache[pages, 0].reshape(-1, wb.hkv, wb.d)[:L].float().cpu().numpy()
        v = wb.cache[pages, 1].reshape(-1, wb.hkv, wb.d)[:L].float().cpu().numpy()
        ref = kv_ref._attend(wb.q[b:b + 1].float().cpu().numpy().astype(np.float64), k, v, [L],
                             wb.d ** -0.5)[0]
        np.testing.assert_allclose(o[b].cpu().numpy(), ref, atol=2e-3, rtol=1e-2, err_msg=f"sequence {b} (L={L})")
