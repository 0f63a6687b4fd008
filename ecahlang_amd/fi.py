"""The FlashInfer names the reference calls on the paged-KV path, in one namespace.

``import ecahlang_amd.fi as flashinfer`` makes these call sites resolve here unchanged:
``flashinfer.get_seq_lens`` and ``flashinfer.get_batch_indices_positions``
(ecahlang/manager.py:143-146, 170-173), ``flashinfer.page.append_paged_kv_cache``
(manager.py:155-165, 175-185, 271-280), the two wrappers (ecahlang/main.py:201-204),
and ``flashinfer.sampling.top_k_top_p_sampling_from_logits`` (main.py:377, 400, 489, 582).
"""
from __future__ import annotations

import types

from .ops import append_paged_kv_cache, get_batch_indices_positions, get_seq_lens
from .sampling import top_k_top_p_sampling_from_logits
from .wrappers import BatchDecodeWithPagedKVCacheWrapper, BatchPrefillWithPagedKVCacheWrapper

page = types.SimpleNamespace(append_paged_kv_cache=append_paged_kv_cache,
                             get_seq_lens=get_seq_lens,
                             get_batch_indices_positions=get_batch_indices_positions)

sampling = types.SimpleNamespace(top_k_top_p_sampling_from_logits=top_k_top_p_sampling_from_logits)

__all__ = ["get_seq_lens", "get_batch_indices_positions", "page", "sampling",
           "BatchDecodeWithPagedKVCacheWrapper", "BatchPrefillWithPagedKVCacheWrapper"]
