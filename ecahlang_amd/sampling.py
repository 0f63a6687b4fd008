"""Top-k / top-p sampling from logits on the device (the sampler the serving loop calls after the
last layer: flashinfer.sampling.top_k_top_p_sampling_from_logits at ecahlang/main.py:377-379,
400-402, 489-491, 582-584).

Same call shape: ``top_k_top_p_sampling_from_logits(logits, top_k, top_p, ...)`` with per-row
tensors or scalars, returning int32 token ids [batch].  The filter order is FlashInfer's
default, top-k first, then top-p on the renormalised top-k distribution; ties at a threshold are
kept.  The draw: one uniform number per row from ``generator`` (torch's device generator by
default: graph-capturable) selects the token by inverse CDF over the kept tokens in vocabulary
order, so for a given uniform the result is exact and bitwise reproducible (the kernel sums
masses as integers).  FlashInfer's own random stream is not reproduced.
"""
from __future__ import annotations

import torch

from ._lib import check, dtype_code, lib, stream_ptr


def _per_row(v, n: int, dtype, device, name: str):
    """(device tensor or None, scalar) for a per-row argument given as a tensor or a number."""
    if isinstance(v, torch.Tensor):
        if v.numel() == 1 and n != 1:
            return None, v.item()
        t = v.reshape(-1)
        if t.numel() != n:
            raise ValueError(f"{name} must have one entry per row ({n}), got {t.numel()}")
        if t.device != device:
            raise ValueError(f"{name} must be on {device}")
        return t.to(dtype).contiguous(), 0
    return None, v


def top_k_top_p_sampling_from_logits(logits: torch.Tensor, top_k, top_p, indices=None,
                                     filter_apply_order: str = "top_k_first", deterministic: bool = True,
                                     generator: torch.Generator | None = None, check_nan: bool = False,
                                     *, uniform: torch.Tensor | None = None) -> torch.Tensor:
    """Sample one token per row of ``logits`` [batch, vocab] (fp16, bf16 or fp32, unit inner
    stride).  ``uniform`` (an extension) supplies the per-row uniform numbers in [0, 1) instead
    of drawing them from ``generator``."""
    if indices is not None:
        raise NotImplementedError("indices (a row per request mapping) is not implemented")
    if filter_apply_order != "top_k_first":
        raise NotImplementedError("only filter_apply_order='top_k_first' (FlashInfer's default) is implemented")
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be [batch, vocab] with a unit inner stride")
    if logits.device.type != "cuda":
        raise ValueError("logits must be a CUDA (HIP) tensor")
    rows, vocab = logits.shape
    dev = logits.device
    if check_nan and bool(torch.isnan(logits).any()):
        raise ValueError("logits contain NaN")
    k_t, k_all = _per_row(top_k, rows, torch.int32, dev, "top_k")
    p_t, p_all = _per_row(top_p, rows, torch.float32, dev, "top_p")
    if uniform is None:
        uniform = torch.rand(rows, device=dev, dtype=torch.float32, generator=generator)
    else:
        uniform = uniform.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
        if uniform.numel() != rows:
            raise ValueError("uniform must have one entry per row")
    out = torch.empty(rows, dtype=torch.int32, device=dev)
    check(lib().pkv_top_k_top_p_sampling(
        logits.data_ptr(), logits.stride(0), rows, vocab, dtype_code(logits.dtype),
        k_t.data_ptr() if k_t is not None else None, int(k_all),
        p_t.data_ptr() if p_t is not None else None, float(p_all),
        uniform.data_ptr(), out.data_ptr(), stream_ptr(dev)), "top-k / top-p sampling")
    return out
