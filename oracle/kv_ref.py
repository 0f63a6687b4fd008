"""numpy restatement of the paged-KV contract the reference calls (FlashInfer 0.6.5).

Test infrastructure only (see oracle/__init__.py).  FlashInfer is an external dependency of
the reference (uv.lock:324-325), absent from this machine; the semantics below follow the
reference's call sites and FlashInfer's published API:

  seq_lens                  flashinfer.get_seq_lens            ecahlang/manager.py:143, 170
  batch_indices_positions   flashinfer.get_batch_indices_positions  manager.py:144-146, 171-173
  append                    flashinfer.page.append_paged_kv_cache   manager.py:155-165, 271-280
  decode                    BatchDecodeWithPagedKVCacheWrapper.run  ecahlang/main.py:68
  prefill                   BatchPrefillWithPagedKVCacheWrapper.run main.py:68 (causal plan :432-443)
  sdpa_decode / sdpa_prefill  the reference's CPU path: gather the pages, then
                            torch.nn.functional.scaled_dot_product_attention in fp32 (the
                            cross-check the reference runs at main.py:70-87, done per request)

Arrays: cache [pages, 2, page_size, Hkv, D] (K at [:,0], V at [:,1]); q [rows, Hq, D];
indptr [B+1], indices [indptr[B]], last [B] int32.  Attention is computed in float64.
"""
from __future__ import annotations

import math

import numpy as np


def seq_lens(indptr, last, page_size: int) -> np.ndarray:
    indptr = np.asarray(indptr, dtype=np.int64)
    last = np.asarray(last, dtype=np.int64)
    npages = indptr[1:] - indptr[:-1]
    return (np.maximum(npages - 1, 0) * page_size + last).astype(np.int32)


def batch_indices_positions(append_indptr, seq_lens_, nnz: int) -> tuple:
    ai = np.asarray(append_indptr, dtype=np.int64)
    sl = np.asarray(seq_lens_, dtype=np.int64)
    bidx = np.empty(nnz, dtype=np.int32)
    pos = np.empty(nnz, dtype=np.int32)
    for b in range(len(sl)):
        lo, hi = ai[b], ai[b + 1]
        n = hi - lo
        bidx[lo:hi] = b
        pos[lo:hi] = sl[b] - n + np.arange(n)
    return bidx, pos


def append(cache: np.ndarray, k: np.ndarray, v: np.ndarray, bidx, pos, indices, indptr,
           page_size: int) -> np.ndarray:
    """Returns a copy of ``cache`` with token rows scattered in.  Works on raw bit views
    (e.g. int16 for fp16/bf16) so the comparison is bitwise."""
    out = cache.copy()
    indices = np.asarray(indices)
    indptr = np.asarray(indptr)
    for i in range(k.shape[0]):
        b, p = int(bidx[i]), int(pos[i])
        page = int(indices[int(indptr[b]) + p // page_size])
        slot = p % page_size
        out[page, 0, slot] = k[i]
        out[page, 1, slot] = v[i]
    return out


def gather(cache: np.ndarray, indices, indptr, last, b: int, page_size: int) -> tuple:
    """Contiguous K, V [L, Hkv, D] of sequence b, L = seq_len_b."""
    lo, hi = int(indptr[b]), int(indptr[b + 1])
    if hi == lo:
        shp = (0,) + cache.shape[3:]
        return np.zeros(shp, cache.dtype), np.zeros(shp, cache.dtype)
    pages = np.asarray(indices[lo:hi])
    L = (hi - lo - 1) * page_size + int(last[b])
    kk = cache[pages, 0].reshape((-1,) + cache.shape[3:])[:L]
    vv = cache[pages, 1].reshape((-1,) + cache.shape[3:])[:L]
    return kk, vv


def _attend(q: np.ndarray, k: np.ndarray, v: np.ndarray, limits, scale: float) -> np.ndarray:
    """q [R, Hq, D]; k, v [L, Hkv, D]; row r attends keys [0, limits[r]).  float64 out."""
    R, Hq, D = q.shape
    Hkv = k.shape[1] if k.ndim == 3 else 1
    g = Hq // Hkv
    out = np.zeros((R, Hq, D), dtype=np.float64)
    if k.shape[0] == 0:
        return out
    q64, k64, v64 = q.astype(np.float64), k.astype(np.float64), v.astype(np.float64)
    for h in range(Hq):
        kh, vh = k64[:, h // g, :], v64[:, h // g, :]
        s = q64[:, h, :] @ kh.T * scale  # [R, L]
        for r in range(R):
            n = int(limits[r])
            if n <= 0:
                continue
            sr = s[r, :n]
            w = np.exp(sr - sr.max())
            out[r, h] = (w / w.sum()) @ vh[:n]
    return out


def decode(q: np.ndarray, cache: np.ndarray, indptr, indices, last, page_size: int,
           sm_scale: float | None = None) -> np.ndarray:
    B, Hq, D = q.shape
    scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(D)
    out = np.zeros((B, Hq, D), dtype=np.float64)
    for b in range(B):
        kk, vv = gather(cache, indices, indptr, last, b, page_size)
        out[b] = _attend(q[b:b + 1], kk, vv, [kk.shape[0]], scale)[0]
    return out


def prefill(q: np.ndarray, qo_indptr, cache: np.ndarray, indptr, indices, last, page_size: int,
            causal: bool = True, sm_scale: float | None = None) -> np.ndarray:
    nnz, Hq, D = q.shape
    scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(D)
    out = np.zeros((nnz, Hq, D), dtype=np.float64)
    B = len(qo_indptr) - 1
    for b in range(B):
        lo, hi = int(qo_indptr[b]), int(qo_indptr[b + 1])
        if hi == lo:
            continue
        kk, vv = gather(cache, indices, indptr, last, b, page_size)
        kv_len, qo_len = kk.shape[0], hi - lo
        if causal:
            limits = [min(max(i + kv_len - qo_len + 1, 0), kv_len) for i in range(qo_len)]
        else:
            limits = [kv_len] * qo_len
        out[lo:hi] = _attend(q[lo:hi], kk, vv, limits, scale)
    return out


# ---- the reference's CPU path, in torch (used as the CPU baseline and as a library check) ----

def sdpa_decode(q, cache, indptr, indices, last, page_size: int, sm_scale=None):
    """q [B,Hq,D], cache [pages,2,ps,Hkv,D] torch CPU tensors; returns fp32 [B,Hq,D]."""
    import torch
    import torch.nn.functional as F

    B, Hq, D = q.shape
    out = torch.zeros(B, Hq, D, dtype=torch.float32)
    ip = indptr.tolist()
    for b in range(B):
        lo, hi = ip[b], ip[b + 1]
        if hi == lo:
            continue
        pages = indices[lo:hi].long()
        L = (hi - lo - 1) * page_size + int(last[b])
        kv = cache.index_select(0, pages)  # [n, 2, ps, Hkv, D]
        k = kv[:, 0].reshape(-1, *cache.shape[3:])[:L].float().transpose(0, 1)  # [Hkv, L, D]
        v = kv[:, 1].reshape(-1, *cache.shape[3:])[:L].float().transpose(0, 1)
        qb = q[b].float().unsqueeze(1)  # [Hq, 1, D]
        o = F.scaled_dot_product_attention(qb.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0),
                                           scale=sm_scale, enable_gqa=Hq != cache.shape[3])
        out[b] = o[0, :, 0]
    return out


def sdpa_prefill(q, qo_indptr, cache, indptr, indices, last, page_size: int, causal=True,
                 sm_scale=None):
    import torch
    import torch.nn.functional as F

    nnz, Hq, D = q.shape
    out = torch.zeros(nnz, Hq, D, dtype=torch.float32)
    qi, ip = qo_indptr.tolist(), indptr.tolist()
    for b in range(len(qi) - 1):
        lo, hi = qi[b], qi[b + 1]
        if hi == lo or ip[b + 1] == ip[b]:
            continue
        pages = indices[ip[b]:ip[b + 1]].long()
        L = (ip[b + 1] - ip[b] - 1) * page_size + int(last[b])
        kv = cache.index_select(0, pages)
        k = kv[:, 0].reshape(-1, *cache.shape[3:])[:L].float().transpose(0, 1)
        v = kv[:, 1].reshape(-1, *cache.shape[3:])[:L].float().transpose(0, 1)
        qb = q[lo:hi].float().transpose(0, 1)  # [Hq, qo, D]
        mask = None
        if causal:
            qo = hi - lo
            i = torch.arange(qo).unsqueeze(1)
            j = torch.arange(L).unsqueeze(0)
            mask = j <= i + (L - qo)  # bottom-right aligned
        o = F.scaled_dot_product_attention(qb.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0),
                                           attn_mask=mask, scale=sm_scale,
                                           enable_gqa=Hq != cache.shape[3])
        out[lo:hi] = o[0].transpose(0, 1)
    return out
