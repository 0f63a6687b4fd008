"""Fused rotary embedding + append (pkv_append_paged_kv_cache_rope) through the C ABI.

Bar: bit-exact.  The expected result is the model's own sequence run on the same device:
transformers' apply_rotary_pos_emb (the function the reference's model calls right before
the attention hook, modeling_qwen2.py:210-211) on [1, H, nnz, D] views, then the plain append;
and, independently, the CPU oracle (oracle/rope_ref.py rotation + oracle/kv_ref.py append).
The whole NaN-poisoned pool is compared as integers.
"""
import numpy as np
import pytest
import torch

from ecahlang_amd import ops, workloads
from oracle import kv_ref, rope_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"
_NAME = {torch.float16: "float16", torch.bfloat16: "bfloat16", torch.float32: "float32"}


def _bits(t):
    iv = torch.int32 if t.dtype == torch.float32 else torch.int16
    return t.contiguous().view(iv).cpu().numpy()


def _cos_sin(positions, dtype, d):
    from transformers import Qwen2Config
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RotaryEmbedding

    cfg = Qwen2Config(hidden_size=16 * d, num_attention_heads=16, num_key_value_heads=2,
                      rope_theta=1000000.0, max_position_embeddings=32768)
    x = torch.zeros(1, positions.numel(), 1, dtype=dtype)
    cos, sin = Qwen2RotaryEmbedding(cfg)(x, positions.long()[None])
    return cos[0].contiguous(), sin[0].contiguous()


def _model_path(dv, cos, sin):
    """transformers' rotation on the device, then the plain append; returns (q_rot, cache)."""
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb

    cache = dv.cache.clone()
    q4 = dv.q.transpose(0, 1)[None]          # [1, Hq, nnz, D], the model's layout
    k4 = dv.k_new.transpose(0, 1)[None]
    qe, ke = apply_rotary_pos_emb(q4, k4, cos[None], sin[None])
    k_rot = ke[0].transpose(0, 1)
    ops.append_paged_kv_cache(k_rot, dv.v_new, dv.batch_indices, dv.positions, cache,
                              dv.indices, dv.indptr, dv.last)
    return qe[0].transpose(0, 1), cache


def _oracle(wb, cos, sin):
    name = _NAME[wb.dtype]
    c, s = _bits(cos)[:, None], _bits(sin)[:, None]
    q_rot = rope_ref.rotate(_bits(wb.q), c, s, name)
    k_rot = rope_ref.rotate(_bits(wb.k_new), c, s, name)
    iv = np.int32 if wb.dtype == torch.float32 else np.int16
    raw = kv_ref.append(_bits(wb.cache), k_rot.view(iv), _bits(wb.v_new), wb.batch_indices.numpy(),
                        wb.positions.numpy(), wb.indices.numpy(), wb.indptr.numpy(), wb.ps)
    return q_rot.view(iv), raw


CASES = {
    # decode step of Qwen2.5-3B's attention (Hq 16, Hkv 2, D 128) at mixed context lengths
    "decode_fp16": dict(kv=[1, 17, 300, 4096, 32000, 900] * 2, new=[1] * 12, hq=16, hkv=2, d=128,
                        dtype=torch.float16),
    # chunked prefill rows of three sequences
    "prefill_bf16": dict(kv=[700, 64, 129], new=[300, 64, 17], hq=16, hkv=2, d=128, dtype=torch.bfloat16),
    "fp32_d64": dict(kv=[33, 5, 100], new=[9, 5, 2], hq=8, hkv=4, d=64, dtype=torch.float32),
    # head_dim a multiple of 8 but not 16: the element path
    "fp16_d72": dict(kv=[30, 7], new=[3, 7], hq=4, hkv=2, d=72, dtype=torch.float16),
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_matches_model_rotation_then_append(case):
    c = CASES[case]
    wb = workloads.build_batch(c["kv"], c["new"], c["hq"], c["hkv"], c["d"], c["dtype"], seed=21, scale=2.0)
    cos, sin = _cos_sin(wb.positions, c["dtype"], c["d"])
    dv = wb.to(DEV)
    cd, sd = cos.to(DEV), sin.to(DEV)
    want_q, want_cache = _model_path(dv, cd, sd)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    got_q = ops.append_paged_kv_cache_with_rope(dv.q, dv.k_new, dv.v_new, cd, sd, dv.batch_indices,
                                                dv.positions, dv.cache, dv.indices, dv.indptr, dv.last,
                                                err_count=err)
    torch.cuda.synchronize()
    assert err.item() == 0
    assert np.array_equal(_bits(got_q), _bits(want_q)), f"{case}: q differs from the model's rotation"
    assert np.array_equal(_bits(dv.cache), _bits(want_cache)), f"{case}: pool differs"
    oq, ocache = _oracle(wb, cos, sin)
    assert np.array_equal(_bits(got_q), oq), f"{case}: q differs from the oracle"
    assert np.array_equal(_bits(dv.cache), ocache), f"{case}: pool differs from the oracle"


def test_in_place_on_the_model_layout():
    """q, k, v as the model hands them over: [1, H, L, D] tensors viewed as [L, H, D]."""
    wb = workloads.build_batch([200], [64], 16, 2, 128, torch.float16, seed=4)
    cos, sin = _cos_sin(wb.positions, torch.float16, 128)
    dv = wb.to(DEV)
    cd, sd = cos.to(DEV), sin.to(DEV)
    q4 = dv.q.transpose(0, 1).contiguous()[None]
    k4 = dv.k_new.transpose(0, 1).contiguous()[None]
    v4 = dv.v_new.transpose(0, 1).contiguous()[None]
    dv.k_new = k4[0].transpose(0, 1)
    dv.v_new = v4[0].transpose(0, 1)
    dv.q = q4[0].transpose(0, 1)
    want_q, want_cache = _model_path(dv, cd, sd)
    q_view = q4[0].transpose(0, 1)
    out = ops.append_paged_kv_cache_with_rope(q_view, dv.k_new, dv.v_new, cd, sd, dv.batch_indices,
                                              dv.positions, dv.cache, dv.indices, dv.indptr, dv.last,
                                              q_out=q_view)
    torch.cuda.synchronize()
    assert out.data_ptr() == q4.data_ptr()
    assert np.array_equal(_bits(q_view), _bits(want_q))
    assert np.array_equal(_bits(dv.cache), _bits(want_cache))


def test_unaligned_views_take_the_element_path():
    """Row views starting one element into their buffers (no 8-byte vectors possible)."""
    wb = workloads.build_batch([40, 9], [8, 3], 4, 2, 64, torch.bfloat16, seed=8)
    cos, sin = _cos_sin(wb.positions, torch.bfloat16, 64)
    dv = wb.to(DEV)
    n = dv.q.shape[0]

    def shifted(t):
        buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=DEV)
        v = buf[1:].view(t.shape)
        v.copy_(t)
        return v

    dv.q, dv.k_new, dv.v_new = shifted(dv.q), shifted(dv.k_new), shifted(dv.v_new)
    cd, sd = shifted(cos.to(DEV)), shifted(sin.to(DEV))
    assert dv.q.data_ptr() % 8 != 0
    want_q, want_cache = _model_path(dv, cd, sd)
    got_q = ops.append_paged_kv_cache_with_rope(dv.q, dv.k_new, dv.v_new, cd, sd, dv.batch_indices,
                                                dv.positions, dv.cache, dv.indices, dv.indptr, dv.last)
    torch.cuda.synchronize()
    assert got_q.shape == (n, 4, 64)
    assert np.array_equal(_bits(got_q), _bits(want_q))
    assert np.array_equal(_bits(dv.cache), _bits(want_cache))


def test_out_of_range_metadata_is_skipped_and_counted_once_per_token():
    wb = workloads.build_batch([20, 3], [2, 1], 4, 2, 64, torch.float16, seed=10)
    cos, sin = _cos_sin(wb.positions, torch.float16, 64)
    dv = wb.to(DEV)
    before = _bits(dv.cache)
    pos = dv.positions.clone()
    pos[0] = 10_000
    pos[1] = -3
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    cd, sd = cos.to(DEV)[:2], sin.to(DEV)[:2]
    q = ops.append_paged_kv_cache_with_rope(dv.q[:2], dv.k_new[:2], dv.v_new[:2], cd, sd, dv.batch_indices,
                                            pos, dv.cache, dv.indices, dv.indptr, dv.last, err_count=err)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(dv.cache), before)
    assert err.item() == 2
    # the queries are still rotated (they do not depend on the pages)
    want = rope_ref.rotate(_bits(wb.q[:2]), _bits(cos[:2])[:, None], _bits(sin[:2])[:, None], "float16")
    assert np.array_equal(_bits(q), want.view(np.int16))


def test_argument_checks():
    wb = workloads.build_batch([20], [2], 4, 2, 64, torch.float16, seed=1)
    cos, sin = _cos_sin(wb.positions, torch.float16, 64)
    dv = wb.to(DEV)
    cd, sd = cos.to(DEV), sin.to(DEV)
    with pytest.raises(ValueError):
        ops.append_paged_kv_cache_with_rope(dv.q, dv.k_new, dv.v_new, cd.float(), sd, dv.batch_indices,
                                            dv.positions, dv.cache, dv.indices, dv.indptr, dv.last)
    with pytest.raises(ValueError):
        ops.append_paged_kv_cache_with_rope(dv.q[:1], dv.k_new, dv.v_new, cd, sd, dv.batch_indices,
                                            dv.positions, dv.cache, dv.indices, dv.indptr, dv.last)
