"""The transformers attention hook that routes a CausalLM's attention through the paged-KV
path (ecahlang/main.py:25-98, registered at :200).

transformers calls it as ``fn(module, q[1,Hq,L,D], k[1,Hkv,L,D], v[1,Hkv,L,D],
attention_mask, dropout=, scaling=, sliding_window=, **model_kwargs)`` and expects
``(o[1,L,Hq,D], None)``.  The caller passes ``wrapper`` (the decode or prefill wrapper,
already planned for the step), ``manager`` (an AutoKVCacheManager whose step metadata is
prepared) and ``prefill`` through the model call's keyword arguments, as main.py does.

Per call (one layer): append this layer's new K/V into its pages, through the bucket's static
buffers when a CUDA graph is being captured or replayed for decode (main.py:62-64) and
through the step's cached metadata otherwise (:66); attend with the wrapper over the layer's
cache (:68); advance the manager's layer counter (:89).  In the bucketed decode path, with the
wrapper planned on the bucket's buffers as main.py plans it, the append rides in the decode's
launch (``run(..., append_kv=)``: the same bytes land in the same slots).  Inputs in another dtype than the
cache (an fp32 model over an fp16 cache) are cast to the cache's dtype and the output cast
back (the reference's ``need_autocast``, :50-53, :95-96).  ``attention_mask``, ``dropout``,
``scaling`` and ``sliding_window`` are ignored as in the reference: the wrapper's plan holds
the causal structure and the 1/sqrt(head_dim) scale.  The reference's optional SDPA
cross-check (:70-87) is a debugging aid and is not reproduced.
"""
from __future__ import annotations

import torch

HOOK_NAME = "ecah_attention"


@torch.compiler.disable
def ecah_attention(module, query, key, value, attention_mask, **kwargs):
    wrapper = kwargs.get("wrapper")
    manager = kwargs.get("manager")
    prefill = bool(kwargs.get("prefill"))
    if wrapper is None or manager is None:
        raise ValueError("ecah_attention needs wrapper= and manager= in the model call's kwargs")
    in_dtype = query.dtype
    if in_dtype != manager.dtype:
        query, key, value = (t.to(manager.dtype) for t in (query, key, value))
    # [1, H, L, D] -> [L, H, D] views (unit inner stride; the kernels take the strides)
    q = query[0].transpose(0, 1)
    k = key[0].transpose(0, 1)
    v = value[0].transpose(0, 1)
    layer_attr = "prefill_layer_idx" if prefill else "decode_layer_idx"
    layer_idx = getattr(manager, layer_attr)
    if manager.cuda_graph_mode and not prefill:
        if _planned_on_bucket(wrapper, manager, q.shape[0]):
            # the bucket's append (positions = seq_len - 1) in the decode's own launch
            o = wrapper.run(q, manager.kv_cache[layer_idx], append_kv=(k, v))
        else:
            manager.append_paged_kv_cache_cuda_graph(k, v, q.shape[0], layer_idx)
            o = wrapper.run(q, manager.kv_cache[layer_idx])
    else:
        manager.append_paged_kv_cache_cached(k, v, layer_idx)
        o = wrapper.run(q, manager.kv_cache[layer_idx])
    setattr(manager, layer_attr, layer_idx + 1)
    o = o[None]
    if o.dtype != in_dtype:
        o = o.to(in_dtype)
    return o, None


def _planned_on_bucket(wrapper, manager, bucket: int) -> bool:
    """Whether ``wrapper`` is a decode wrapper planned on the bucket's own metadata buffers
    (main.py:341-347 plans it so), whose rows then put each token at its sequence's last slot:
    the append the bucket's positions select."""
    from .wrappers import BatchDecodeWithPagedKVCacheWrapper

    if not isinstance(wrapper, BatchDecodeWithPagedKVCacheWrapper) or not getattr(wrapper, "_planned", False):
        return False
    meta = (getattr(manager, "_cg_kv_indptr", {}).get(bucket), getattr(manager, "_cg_kv_indices", {}).get(bucket),
            getattr(manager, "_cg_kv_last_page_len", {}).get(bucket))
    mine = (wrapper._indptr, wrapper._indices, wrapper._last)
    return all(a is not None and a.data_ptr() == b.data_ptr() and a.numel() == b.numel() for a, b in zip(meta, mine))


def register(name: str = HOOK_NAME) -> None:
    """Register the hook with transformers (main.py:200); then load a model with
    ``attn_implementation=name``."""
    from transformers import AttentionInterface

    AttentionInterface.register(name, ecah_attention)
