"""FlashInfer-shaped page-table and append functions, backed by libpagedkv.so.

Same names, argument order, keywords and result shapes as the FlashInfer 0.6.5 calls the
reference makes (ecahlang/manager.py:143-146, 155-165, 170-185, 271-280), so the manager and
any FlashInfer caller can switch by changing the import.
"""
from __future__ import annotations

from typing import Tuple, Union

import torch

from ._lib import check, dtype_code, lib, stream_ptr

CacheT = Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]


def _i32(t: torch.Tensor, name: str) -> torch.Tensor:
    if not isinstance(t, torch.Tensor) or t.dtype != torch.int32 or not t.is_cuda:
        raise ValueError(f"{name} must be an int32 CUDA tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t


class CacheView:
    """K/V base pointers and geometry of one layer's paged cache.

    Accepts the single-tensor NHD form ``[pages, 2, page_size, Hkv, D]`` the reference
    allocates (ecahlang/manager.py:51-54, indexed per layer at :160) or a ``(k_cache,
    v_cache)`` pair of ``[pages, page_size, Hkv, D]`` tensors.
    """

    __slots__ = ("k_ptr", "v_ptr", "page_stride", "num_pages", "page_size", "num_kv_heads",
                 "head_dim", "dtype", "device")

    def __init__(self, paged_kv_cache: CacheT, kv_layout: str = "NHD"):
        if kv_layout.upper() != "NHD":
            raise NotImplementedError("only the NHD cache layout is implemented (the reference uses NHD)")
        if isinstance(paged_kv_cache, (tuple, list)):
            k, v = paged_kv_cache
            if k.dim() != 4 or k.shape != v.shape or k.dtype != v.dtype:
                raise ValueError("(k_cache, v_cache) must both be [pages, page_size, Hkv, D]")
            for t in (k, v):
                if not t.is_contiguous():
                    raise ValueError("k_cache / v_cache must be contiguous")
            self.k_ptr, self.v_ptr = k.data_ptr(), v.data_ptr()
            self.num_pages, self.page_size, self.num_kv_heads, self.head_dim = k.shape
            self.page_stride = k.stride(0)
            self.dtype, self.device = k.dtype, k.device
        else:
            c = paged_kv_cache
            if c.dim() != 5 or c.shape[1] != 2:
                raise ValueError("paged_kv_cache must be [pages, 2, page_size, Hkv, D] (NHD)")
            if not c.is_contiguous():
                raise ValueError("paged_kv_cache must be contiguous")
            self.num_pages, _, self.page_size, self.num_kv_heads, self.head_dim = c.shape
            self.k_ptr = c.data_ptr()
            self.v_ptr = c[:, 1].data_ptr()
            self.page_stride = c.stride(0)
            self.dtype, self.device = c.dtype, c.device
        if not (self.device.type == "cuda"):
            raise ValueError("paged_kv_cache must live on a CUDA (HIP) device")


def get_seq_lens(kv_indptr: torch.Tensor, kv_last_page_len: torch.Tensor, page_size: int) -> torch.Tensor:
    """seq_len[b] = max(indptr[b+1]-indptr[b]-1, 0) * page_size + last_page_len[b] (int32)."""
    _i32(kv_indptr, "kv_indptr")
    _i32(kv_last_page_len, "kv_last_page_len")
    b = kv_last_page_len.numel()
    if kv_indptr.numel() != b + 1:
        raise ValueError("kv_indptr must have batch+1 entries")
    out = torch.empty(b, dtype=torch.int32, device=kv_indptr.device)
    check(lib().pkv_get_seq_lens(kv_indptr.data_ptr(), kv_last_page_len.data_ptr(), b,
                                 int(page_size), out.data_ptr(), stream_ptr(kv_indptr.device)),
          "get_seq_lens")
    return out


def get_batch_indices_positions(append_indptr: torch.Tensor, seq_lens: torch.Tensor, nnz) -> tuple:
    """(batch_indices, positions) of the nnz appended tokens, both int32 [nnz].

    ``nnz`` may be an int or a 0-d tensor (the reference passes ``append_indptr[-1]``,
    ecahlang/manager.py:145); a device tensor costs one host sync, as in the reference.
    """
    _i32(append_indptr, "append_indptr")
    _i32(seq_lens, "seq_lens")
    nnz = int(nnz)
    b = seq_lens.numel()
    if append_indptr.numel() != b + 1:
        raise ValueError("append_indptr must have batch+1 entries")
    dev = append_indptr.device
    bidx = torch.empty(nnz, dtype=torch.int32, device=dev)
    pos = torch.empty(nnz, dtype=torch.int32, device=dev)
    if nnz:
        check(lib().pkv_get_batch_indices_positions(append_indptr.data_ptr(), seq_lens.data_ptr(), b,
                                                    nnz, bidx.data_ptr(), pos.data_ptr(),
                                                    stream_ptr(dev)),
              "get_batch_indices_positions")
    return bidx, pos


def _row_strides(t: torch.Tensor, name: str) -> tuple:
    if t.dim() != 3 or t.stride(2) != 1:
        raise ValueError(f"{name} must be [nnz, heads, head_dim] with a unit inner stride")
    return t.stride(0), t.stride(1)


def append_paged_kv_cache(append_key: torch.Tensor, append_value: torch.Tensor,
                          batch_indices: torch.Tensor, positions: torch.Tensor,
                          paged_kv_cache: CacheT, kv_indices: torch.Tensor, kv_indptr: torch.Tensor,
                          kv_last_page_len: torch.Tensor, kv_layout: str = "NHD",
                          err_count: torch.Tensor | None = None) -> None:
    """Scatter ``append_key/value[i]`` into page ``kv_indices[kv_indptr[b] + pos // ps]`` slot
    ``pos % ps`` with b = batch_indices[i], pos = positions[i].  Bit-exact copy.

    ``kv_last_page_len`` is accepted for signature parity and, as in the reference's
    dependency, not used by the scatter.  ``err_count`` (optional int32 [1]) counts tokens
    whose metadata falls outside their sequence's pages; they are skipped.
    """
    cv = CacheView(paged_kv_cache, kv_layout)
    for t, n in ((append_key, "append_key"), (append_value, "append_value")):
        if t.dtype != cv.dtype:
            raise ValueError(f"{n} dtype {t.dtype} differs from the cache dtype {cv.dtype}")
        if t.shape[1:] != (cv.num_kv_heads, cv.head_dim):
            raise ValueError(f"{n} must be [nnz, {cv.num_kv_heads}, {cv.head_dim}]")
    nnz = append_key.shape[0]
    if append_value.shape[0] != nnz or batch_indices.numel() < nnz or positions.numel() < nnz:
        raise ValueError("append_key, append_value, batch_indices and positions disagree on nnz")
    _i32(batch_indices, "batch_indices")
    _i32(positions, "positions")
    _i32(kv_indices, "kv_indices")
    _i32(kv_indptr, "kv_indptr")
    ksn, ksh = _row_strides(append_key, "append_key")
    vsn, vsh = _row_strides(append_value, "append_value")
    err_ptr = 0
    if err_count is not None:
        err_ptr = _i32(err_count, "err_count").data_ptr()
    if nnz == 0:
        return
    check(lib().pkv_append_paged_kv_cache(
        append_key.data_ptr(), ksn, ksh, append_value.data_ptr(), vsn, vsh,
        batch_indices.data_ptr(), positions.data_ptr(), nnz, cv.k_ptr, cv.v_ptr, cv.page_stride,
        cv.num_pages, kv_indices.data_ptr(), kv_indices.numel(), kv_indptr.data_ptr(),
        kv_indptr.numel() - 1,
        cv.num_kv_heads, cv.head_dim, cv.page_size, dtype_code(cv.dtype), err_ptr,
        stream_ptr(cv.device)), "append_paged_kv_cache")


def append_paged_kv_cache_slots(append_key: torch.Tensor, append_value: torch.Tensor, slots: torch.Tensor,
                                paged_kv_cache: CacheT, kv_layout: str = "NHD",
                                err_count: torch.Tensor | None = None) -> None:
    """``append_paged_kv_cache`` with each token's destination resolved beforehand: token i goes
    to page ``slots[i] // ps``, slot ``slots[i] % ps`` (``slots`` as the page-table gather of
    ``AutoKVCacheManager.fill_cuda_graph_metadata`` writes them).  One lookup per token instead
    of the three dependent ones through batch_indices / positions, kv_indptr and kv_indices;
    the bytes written are the same.  Tokens with a negative or out-of-pool slot are skipped and
    counted in ``err_count``.
    """
    cv = CacheView(paged_kv_cache, kv_layout)
    for t, n in ((append_key, "append_key"), (append_value, "append_value")):
        if t.dtype != cv.dtype:
            raise ValueError(f"{n} dtype {t.dtype} differs from the cache dtype {cv.dtype}")
        if t.shape[1:] != (cv.num_kv_heads, cv.head_dim):
            raise ValueError(f"{n} must be [nnz, {cv.num_kv_heads}, {cv.head_dim}]")
    nnz = append_key.shape[0]
    if append_value.shape[0] != nnz or slots.numel() < nnz:
        raise ValueError("append_key, append_value and slots disagree on nnz")
    _i32(slots, "slots")
    ksn, ksh = _row_strides(append_key, "append_key")
    vsn, vsh = _row_strides(append_value, "append_value")
    err_ptr = 0
    if err_count is not None:
        err_ptr = _i32(err_count, "err_count").data_ptr()
    if nnz == 0:
        return
    check(lib().pkv_append_paged_kv_cache_slots(
        append_key.data_ptr(), ksn, ksh, append_value.data_ptr(), vsn, vsh, slots.data_ptr(), nnz,
        cv.k_ptr, cv.v_ptr, cv.page_stride, cv.num_pages, cv.num_kv_heads, cv.head_dim, cv.page_size,
        dtype_code(cv.dtype), err_ptr, stream_ptr(cv.device)), "append_paged_kv_cache_slots")


def append_paged_kv_cache_with_rope(q: torch.Tensor, append_key: torch.Tensor, append_value: torch.Tensor,
                                    cos: torch.Tensor, sin: torch.Tensor, batch_indices: torch.Tensor,
                                    positions: torch.Tensor, paged_kv_cache: CacheT,
                                    kv_indices: torch.Tensor, kv_indptr: torch.Tensor,
                                    kv_last_page_len: torch.Tensor, kv_layout: str = "NHD",
                                    q_out: torch.Tensor | None = None,
                                    err_count: torch.Tensor | None = None) -> torch.Tensor:
    """The model's rotary embedding on the new tokens, then the append, in one launch.

    Equivalent, bit for bit, to ``q, k = apply_rotary_pos_emb(q, k, cos, sin)`` as the model
    runs it (transformers/models/qwen2/modeling_qwen2.py:210-211) followed by
    ``append_paged_kv_cache(k, append_value, ...)`` (ecahlang/main.py:62-66).  ``q``,
    ``append_key`` and ``append_value`` are ``[nnz, heads, head_dim]`` row views; ``cos`` /
    ``sin`` are the tokens' ``[nnz, head_dim]`` position-embedding rows in the cache dtype.
    The rotated queries go to ``q_out`` (default: a new tensor; pass ``q`` to rotate in
    place) and are returned.  The rotated keys exist only in the cache.
    """
    cv = CacheView(paged_kv_cache, kv_layout)
    for t, n in ((append_key, "append_key"), (append_value, "append_value")):
        if t.dtype != cv.dtype:
            raise ValueError(f"{n} dtype {t.dtype} differs from the cache dtype {cv.dtype}")
        if t.shape[1:] != (cv.num_kv_heads, cv.head_dim):
            raise ValueError(f"{n} must be [nnz, {cv.num_kv_heads}, {cv.head_dim}]")
    nnz = append_key.shape[0]
    if q.dtype != cv.dtype or q.dim() != 3 or q.shape[0] != nnz or q.shape[2] != cv.head_dim:
        raise ValueError(f"q must be [{nnz}, Hq, {cv.head_dim}] in {cv.dtype}")
    for t, n in ((cos, "cos"), (sin, "sin")):
        if t.dtype != cv.dtype or t.dim() != 2 or t.shape != (nnz, cv.head_dim) or t.stride(1) != 1:
            raise ValueError(f"{n} must be [{nnz}, {cv.head_dim}] in {cv.dtype} with a unit inner stride")
    if cos.stride(0) != sin.stride(0):
        raise ValueError("cos and sin must share a row stride")
    if cv.head_dim % 8:
        raise ValueError("head_dim must be a multiple of 8")
    if append_value.shape[0] != nnz or batch_indices.numel() < nnz or positions.numel() < nnz:
        raise ValueError("q, append_key, append_value, batch_indices and positions disagree on nnz")
    if q_out is None:
        q_out = torch.empty_like(q)
    elif q_out.shape != q.shape or q_out.dtype != q.dtype:
        raise ValueError("q_out must match q's shape and dtype")
    _i32(batch_indices, "batch_indices")
    _i32(positions, "positions")
    _i32(kv_indices, "kv_indices")
    _i32(kv_indptr, "kv_indptr")
    qsn, qsh = _row_strides(q, "q")
    osn, osh = _row_strides(q_out, "q_out")
    ksn, ksh = _row_strides(append_key, "append_key")
    vsn, vsh = _row_strides(append_value, "append_value")
    for t, n in ((q, "q"), (q_out, "q_out"), (append_key, "append_key"), (append_value, "append_value"),
                 (cos, "cos"), (sin, "sin"), (batch_indices, "batch_indices"), (positions, "positions")):
        if t.device != cv.device:
            raise ValueError(f"{n} is on {t.device}, the cache on {cv.device}")
    err_ptr = 0
    if err_count is not None:
        err_ptr = _i32(err_count, "err_count").data_ptr()
    if nnz == 0:
        return q_out
    check(lib().pkv_append_paged_kv_cache_rope(
        q.data_ptr(), qsn, qsh, q_out.data_ptr(), osn, osh, q.shape[1],
        append_key.data_ptr(), ksn, ksh, append_value.data_ptr(), vsn, vsh,
        cos.data_ptr(), sin.data_ptr(), cos.stride(0),
        batch_indices.data_ptr(), positions.data_ptr(), nnz, cv.k_ptr, cv.v_ptr, cv.page_stride,
        cv.num_pages, kv_indices.data_ptr(), kv_indices.numel(), kv_indptr.data_ptr(),
        kv_indptr.numel() - 1, cv.num_kv_heads, cv.head_dim, cv.page_size, dtype_code(cv.dtype), err_ptr,
        stream_ptr(cv.device)), "append_paged_kv_cache_with_rope")
    return q_out
