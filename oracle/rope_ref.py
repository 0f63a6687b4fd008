"""numpy restatement of the model's rotary position embedding, for the tests only.

The reference's model applies it to q and k just before the attention hook:
``apply_rotary_pos_emb(q, k, cos, sin)`` (transformers 5.2.0 pinned at uv.lock:1554-1556,
transformers/models/qwen2/modeling_qwen2.py:210-211 at the call site), whose published body is

  rotate_half(x) = cat(-x[..., D/2:], x[..., :D/2])
  x_embed        = (x * cos) + (rotate_half(x) * sin)

run as eager tensor ops in the activations' dtype: each product is computed in float32 and
rounded to the dtype, then the sum likewise.  ``rotate`` below restates exactly that rounding
sequence (float32 arithmetic, round-to-nearest-even to fp16 / bf16 after every op), so that it
can be compared bit for bit.  Pinned in tests/test_oracle_rope.py against the installed
transformers function on CPU tensors and against closed forms (cos = 1, sin = 0 is the
identity; cos = 0, sin = 1 is rotate_half; two quarter turns negate).

Arrays: x [..., D] and cos / sin broadcastable to it, given as raw bit patterns of ``dtype``
(16-bit integers for fp16 / bf16, 32-bit integers or float32 values for fp32).  The result is
uint16 bits for fp16 / bf16 and float32 values for fp32.
"""
from __future__ import annotations

import numpy as np


def _to_f32(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "float16":
        return np.asarray(x).view(np.float16).astype(np.float32)
    if dtype == "bfloat16":
        return (np.asarray(x).view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    x = np.asarray(x)
    return x.view(np.float32) if x.dtype.kind in "iu" else x.astype(np.float32)  # raw bits or values


def _round(x: np.ndarray, dtype: str) -> np.ndarray:
    """float32 -> dtype (RNE) -> float32."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "float16":
        return x.astype(np.float16).astype(np.float32)
    if dtype == "bfloat16":
        u = x.view(np.uint32).astype(np.uint64)
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
        nan = np.isnan(x)
        r = np.where(nan, (u >> 16) | 0x40, r).astype(np.uint32)
        return (r << 16).view(np.float32)
    return x


def _from_f32(x: np.ndarray, dtype: str) -> np.ndarray:
    """float32 values already representable in dtype -> raw bits (uint16) or float32."""
    if dtype == "float16":
        return x.astype(np.float16).view(np.uint16)
    if dtype == "bfloat16":
        return (np.asarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)
    return np.asarray(x, dtype=np.float32)


def rotate(x, cos, sin, dtype: str) -> np.ndarray:
    """x * cos + rotate_half(x) * sin with the model's per-op rounding; same encoding as x."""
    xf, c, s = _to_f32(x, dtype), _to_f32(cos, dtype), _to_f32(sin, dtype)
    h = xf.shape[-1] // 2
    rot = np.concatenate([-xf[..., h:], xf[..., :h]], axis=-1)
    out = _round(_round(xf * c, dtype) + _round(rot * s, dtype), dtype)
    return _from_f32(out, dtype)
