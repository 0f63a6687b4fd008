"""The FlashInfer names the reference calls on the paged-KV path, in one namespace.

``import ecahlang_amd.fi as flashinfer`` makes these call sites resolve here unchanged:
``flashinfer.get_seq_lens`` and ``flashinfer.get_batch_indices_positions``
(ecahlang/manager.py:143-146, 170-173), ``flashinfer.page.append_paged_kv_cache``
(manager.py:155-165, 175-185, 271-280), and the two wrappers (ecahlang/main.py:201-204).
Sampling (``flashinfer.sampling``, main.py:377, 400, 489, 582) is outside the paged-KV path
and is not provided: asking for it raises.
"""
from __future__ import annotations

import types

from .ops import append_paged_kv_cache, get_batch_indices_positions, get_seq_lens
from .wrappers import BatchDecodeWithPagedKVCacheWrapper, BatchPrefillWithPagedKVCacheWrapper

page = types.SimpleNamespace(append_paged_kv_cache=append_paged_kv_cache,
                             get_seq_lens=get_seq_lens,
                             get_batch_indices_positions=get_batch_indices_positions)

__all__ = ["get_seq_lens", "get_batch_indices_positions", "page",
           "BatchDecodeWithPagedKVCacheWrapper", "BatchPrefillWithPagedKVCacheWrapper"]


def __getattr__(name: str):
    if name == "sampling":
        raise AttributeError("ecahlang_amd.fi provides the paged-KV path only; flashinfer.sampling "
                             "is not part of it")
    raise AttributeError(f"module 'ecahlang_amd.fi' has no attribute {name!r}")
