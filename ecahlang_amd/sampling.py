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
                                     *, uniform: torch.Tensor | None = None,
                                     penalty: torch.Tensor | None = None,
                                     penalty_rows: torch.Tensor | None = None,
                                     temperature=None) -> torch.Tensor:
    """Sample one token per row of ``logits`` [batch, vocab] (fp16, bf16 or fp32, unit inner
    stride).  ``uniform`` (an extension) supplies the per-row uniform numbers in [0, 1) instead
    of drawing them from ``generator``.

    ``penalty`` / ``penalty_rows`` / ``temperature`` (extensions) fold in the scaling the
    serving loop applies before sampling (ecahlang/main.py:169-170, 483-487):
    ``logits / penalty[penalty_rows]`` in the logits' dtype, then ``/ temperature`` in float32,
    rounded exactly as those tensor ops round, in one pass (:func:`scale_logits`) before the
    sampler.
    ``penalty`` is the [slots, vocab] table in the logits' dtype (the manager's
    ``mask_penalty``), ``penalty_rows`` the int32 slot of each row (``batch_to_seq_len``), and
    ``temperature`` a float32 tensor with one entry per row, or a number."""
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
    if penalty is not None or temperature is not None:
        logits = scale_logits(logits, penalty, penalty_rows, temperature)
    ws_bytes = lib().pkv_sampling_workspace_bytes(rows, vocab)
    ws = torch.empty(max(ws_bytes, 8), dtype=torch.uint8, device=dev)
    check(lib().pkv_top_k_top_p_sampling_ws(
        logits.data_ptr(), logits.stride(0), rows, vocab, dtype_code(logits.dtype),
        k_t.data_ptr() if k_t is not None else None, int(k_all),
        p_t.data_ptr() if p_t is not None else None, float(p_all),
        uniform.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(), stream_ptr(dev)), "top-k / top-p sampling")
    return out


def scale_logits(logits: torch.Tensor, penalty: torch.Tensor | None = None,
                 penalty_rows: torch.Tensor | None = None, temperature=None) -> torch.Tensor:
    """``(logits / penalty[penalty_rows]) / temperature`` as the serving loop computes it
    (ecahlang/main.py:169-170, 483-487: the first division in the logits' dtype, the second with
    a float32 temperature, so the result is float32), bit-identical, in one pass and without
    materialising ``penalty[penalty_rows]``.  Returns a new float32 [rows, vocab] tensor; a row
    whose ``penalty_rows`` entry is not a row of ``penalty`` comes back as NaN (and samples as
    -1), where the tensor expression would raise an indexing error."""
    if logits.dim() != 2 or logits.stride(1) != 1 or logits.device.type != "cuda":
        raise ValueError("logits must be a [batch, vocab] CUDA tensor with a unit inner stride")
    rows, vocab = logits.shape
    dev = logits.device
    pen_ptr, pen_stride, rows_ptr, slots = None, 0, None, 0
    if penalty is not None:
        if (penalty.dim() != 2 or penalty.shape[1] != vocab or penalty.stride(1) != 1
                or penalty.dtype != logits.dtype or penalty.device != dev):
            raise ValueError("penalty must be [slots, vocab] in the logits' dtype and device, unit inner stride")
        if penalty_rows is None:
            raise ValueError("penalty needs penalty_rows (the penalty row of each logits row)")
        penalty_rows = penalty_rows.reshape(-1)
        if (penalty_rows.dtype != torch.int32 or penalty_rows.numel() != rows
                or penalty_rows.device != dev or not penalty_rows.is_contiguous()):
            raise ValueError("penalty_rows must be a contiguous int32 tensor with one entry per row")
        pen_ptr, pen_stride, rows_ptr = penalty.data_ptr(), penalty.stride(0), penalty_rows.data_ptr()
        slots = penalty.shape[0]
    temp = None
    if temperature is not None:
        if isinstance(temperature, torch.Tensor):
            temp = temperature.reshape(-1)
            if temp.numel() == 1 and rows != 1:
                temp = temp.expand(rows)
            if temp.numel() != rows or temp.dtype != torch.float32 or temp.device != dev:
                raise ValueError("temperature must be float32 with one entry per row")
            temp = temp.contiguous()
        else:
            temp = torch.full((rows,), float(temperature), dtype=torch.float32, device=dev)
    out = torch.empty(rows, vocab, dtype=torch.float32, device=dev)
    check(lib().pkv_scale_logits(logits.data_ptr(), logits.stride(0), rows, vocab, dtype_code(logits.dtype),
                                 pen_ptr, pen_stride, slots, rows_ptr, temp.data_ptr() if temp is not None else None,
                                 out.data_ptr(), out.stride(0), stream_ptr(dev)), "scale_logits")
    return out
