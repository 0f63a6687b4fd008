"""Pins the rotary-embedding restatement (oracle/rope_ref.py).

Against the installed transformers function the reference's model calls
(transformers/models/qwen2/modeling_qwen2.py, apply_rotary_pos_emb, with cos / sin from the
model's own Qwen2RotaryEmbedding), bit for bit on CPU tensors in fp16, bf16 and fp32; and
against closed forms that a dropped term, a swapped half or a wrong sign would fail.  A
variant that rounds once instead of after every op is shown to differ, so the comparison does
pin the rounding sequence.
"""
import numpy as np
import pytest
import torch

from oracle import rope_ref

_DT = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.contiguous()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def _model_cos_sin(positions, dtype, d=128, theta=1000000.0):
    from transformers import Qwen2Config
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RotaryEmbedding

    cfg = Qwen2Config(hidden_size=16 * d, num_attention_heads=16, num_key_value_heads=2, rope_theta=theta,
                      max_position_embeddings=32768)
    emb = Qwen2RotaryEmbedding(cfg)
    x = torch.zeros(1, len(positions), 1, dtype=dtype)
    cos, sin = emb(x, torch.tensor([positions]))
    return cos[0], sin[0]  # [L, D] in dtype


@pytest.mark.parametrize("name", ["float16", "bfloat16", "float32"])
def test_matches_transformers_bitwise(name):
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb

    dt = _DT[name]
    g = torch.Generator().manual_seed(11)
    pos = [0, 1, 7, 100, 4095, 20000, 32767]
    cos, sin = _model_cos_sin(pos, dt)
    q = (torch.randn(1, 16, len(pos), 128, generator=g) * 3).to(dt)
    k = (torch.randn(1, 2, len(pos), 128, generator=g) * 3).to(dt)
    qe, ke = apply_rotary_pos_emb(q, k, cos[None], sin[None])
    c, s = _bits(cos)[None, None], _bits(sin)[None, None]
    assert np.array_equal(rope_ref.rotate(_bits(q), c, s, name), _bits(qe))
    assert np.array_equal(rope_ref.rotate(_bits(k), c, s, name), _bits(ke))


def test_per_op_rounding_is_what_is_pinned():
    """Rounding the whole expression once disagrees with the model on fp16 data; the oracle does not."""
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb

    g = torch.Generator().manual_seed(3)
    cos, sin = _model_cos_sin(list(range(0, 4096, 37)), torch.float16)
    q = (torch.randn(1, 16, cos.shape[0], 128, generator=g) * 3).half()
    qe, _ = apply_rotary_pos_emb(q, q[:, :2], cos[None], sin[None])
    xf, c, s = q.float().numpy(), cos.float().numpy(), sin.float().numpy()
    rot = np.concatenate([-xf[..., 64:], xf[..., :64]], axis=-1)
    once = (xf * c + rot * s).astype(np.float16).view(np.uint16)
    assert not np.array_equal(once, _bits(qe))
    assert np.array_equal(rope_ref.rotate(_bits(q), _bits(cos), _bits(sin), "float16"), _bits(qe))


@pytest.mark.parametrize("name", ["float16", "bfloat16", "float32"])
def test_closed_forms(name):
    dt = _DT[name]
    g = torch.Generator().manual_seed(5)
    x = torch.randn(3, 4, 64, generator=g).to(dt)
    one, zero = torch.ones(64, dtype=dt), torch.zeros(64, dtype=dt)
    xb = _bits(x)
    # cos = 1, sin = 0: identity
    assert np.array_equal(rope_ref.rotate(xb, _bits(one), _bits(zero), name), xb)
    # cos = 0, sin = 1: rotate_half exactly, cat(-x2, x1)
    r = rope_ref.rotate(xb, _bits(zero), _bits(one), name)
    assert np.array_equal(r, _bits(torch.cat((-x[..., 32:], x[..., :32]), -1)))
    # two quarter turns: -x
    assert np.array_equal(rope_ref.rotate(r, _bits(zero), _bits(one), name), _bits(-x))
    # cos = -1, sin = 0: -x
    assert np.array_equal(rope_ref.rotate(xb, _bits(-one), _bits(zero), name), _bits(-x))


def test_bf16_rounding_is_nearest_even():
    # 1 + 2^-8 lies halfway between bf16 neighbours 1 and 1 + 2^-7: ties go to the even one (1)
    # 1 + 3 * 2^-8 is halfway between 1 + 2^-7 and 1 + 2^-6: ties to 1 + 2^-6
    v = np.array([1 + 2.0 ** -8, 1 + 3 * 2.0 ** -8, 1 + 2.0 ** -8 + 2.0 ** -20], dtype=np.float32)
    assert rope_ref._round(v, "bfloat16").tolist() == [1.0, 1 + 2.0 ** -6, 1 + 2.0 ** -7]
    t = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
    assert rope_ref._round(v, "bfloat16").tolist() == t.tolist()


def test_fp32_accepts_raw_bits():
    x = np.array([[1.5, -2.25, 3.0, 0.5]], dtype=np.float32)
    c = np.array([0.5, 0.25, 0.5, 0.25], dtype=np.float32)
    s = np.array([0.75, 1.0, 0.75, 1.0], dtype=np.float32)
    by_value = rope_ref.rotate(x, c, s, "float32")
    by_bits = rope_ref.rotate(x.view(np.int32), c.view(np.int32), s.view(np.int32), "float32")
    assert np.array_equal(by_value, by_bits)
    # hand-computed: [1.5*.5 - 3*.75, -2.25*.25 - .5*1, 3*.5 + 1.5*.75, .5*.25 + -2.25*1]
    assert by_value.tolist() == [[-1.5, -1.0625, 2.625, -2.125]]
