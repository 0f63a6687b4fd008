"""ctypes binding of libpagedkv.so (declarations in include/pagedkv.h).

``torch`` is imported first so that the library's libamdhip64.so.7 dependency resolves to the
HIP runtime PyTorch already loaded: kernels launched here and PyTorch's own work then share
one runtime, one set of streams and one graph-capture state.

There is no fallback.  :func:`lib` raises if the library was not built, and every wrapper in
this package goes through it, so a missing extension fails loudly instead of silently
computing something else.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import torch  # noqa: F401  (must precede the dlopen below)

LIB_PATH = Path(__file__).resolve().parent / "libpagedkv.so"

_i32, _i64, _f32, _vp = C.c_int32, C.c_int64, C.c_float, C.c_void_p

# name -> (restype, argtypes); mirrors include/pagedkv.h
SIGNATURES: dict[str, tuple] = {
    "pkv_get_seq_lens": (_i32, [_vp, _vp, _i32, _i32, _vp, _vp]),
    "pkv_get_batch_indices_positions": (_i32, [_vp, _vp, _i32, _i32, _vp, _vp, _vp]),
    "pkv_append_paged_kv_cache": (
        _i32,
        [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _i32, _vp, _vp, _i64, _i64, _vp, _i64, _vp,
         _i32, _i32, _i32, _i32, _i32, _vp, _vp],
    ),
    "pkv_append_paged_kv_cache_slots": (
        _i32, [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i32, _vp, _vp, _i64, _i64, _i32, _i32, _i32, _i32, _vp, _vp]),
    "pkv_append_paged_kv_cache_rope": (
        _i32,
        [_vp, _i64, _i64, _vp, _i64, _i64, _i32, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _i64,
         _vp, _vp, _i32, _vp, _vp, _i64, _i64, _vp, _i64, _vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp],
    ),
    "pkv_decode_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32, _i64]),
    "pkv_decode_workspace_init": (_i32, [_vp, _i32, _vp]),
    "pkv_decode_schedule_layout": (_i32, [_i32, _i32, _i32, _i32, _i64, _i64, _vp]),
    "pkv_decode_plan": (_i32, [_vp, _vp, _i64, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _i64, _vp]),
    "pkv_decode_uses_mfma": (_i32, [_i32, _i32, _i32, _i32, _i32]),
    "pkv_batch_decode": (
        _i32,
        [_vp, _i64, _i64, _vp, _vp, _i64, _i64, _vp, _vp, _i64, _vp, _i32, _i32, _i32, _i32, _i32,
         _f32, _i32, _vp, _i64, _vp, _i64, _i64, _i32, _i32, _vp],
    ),
    "pkv_batch_decode_append": (
        _i32,
        [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _i64, _i64, _vp, _vp, _i64, _vp, _i32,
         _i32, _i32, _i32, _i32, _f32, _i32, _vp, _i64, _vp, _i64, _i64, _i32, _i32, _vp],
    ),
    "pkv_batch_decode_noalloc": (
        _i32,
        [_vp, _i64, _i64, _vp, _vp, _i64, _i64, _vp, _vp, _i64, _vp, _i32, _i32, _i32, _i32, _i32,
         _f32, _i32, _vp, _i64, _i64, _i32, _vp],
    ),
    "pkv_prefill_mfma_supported": (_i32, [_i32, _i32, _i32, _i32, _i32]),
    "pkv_prefill_work_list": (
        _i32, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i64, _i32, _i32, _i32, _vp, _i64, _vp, _i64,
               _vp]),
    "pkv_batch_prefill_mfma": (
        _i32,
        [_vp, _i64, _i64, _vp, _vp, _i64, _i64, _vp, _i64, _i32, _i32, _i32, _i32, _i32, _f32,
         _vp, _i32, _vp, _i32, _vp, _vp, _vp, _i64, _i64, _i32, _vp],
    ),
    "pkv_pool_apply": (_i32, [_vp, _i32, _vp, _i64, _i32, _vp, _i32, _vp, _i32, _vp, _vp]),
    "pkv_pool_copy_pages": (_i32, [_vp, _i64, _i32, _i64, _vp, _i32, _i64, _vp, _vp]),
    "pkv_shared_prefix_pages": (_i32, [_vp, _vp, _i64, _i32, _vp, _vp]),
    "pkv_pool_gather": (_i32, [_vp, _i64, _i32, _vp, _vp, _i32, _vp, _i64, _i64, _vp, _i32, _vp, _vp, _vp]),
    "pkv_pool_step": (
        _i32, [_vp, _vp, _vp, _i64, _i32, _vp, _i32, _i32, _i32, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _i64,
               _i64, _vp, _vp, _vp]),
    "pkv_probe_stream_read": (_i32, [_vp, _i64, _i32, _vp, _vp]),
    "pkv_pool_steps_begin": (_i32, [_vp, _vp, _i32, _i32, _i32, _vp, _vp, _vp, _i32, _vp, _vp, _vp]),
    "pkv_top_k_top_p_sampling": (_i32, [_vp, _i64, _i32, _i32, _i32, _vp, _i32, _vp, _f32, _vp, _vp, _vp]),
    "pkv_sampling_workspace_bytes": (_i64, [_i32, _i32]),
    "pkv_top_k_top_p_sampling_ws": (
        _i32, [_vp, _i64, _i32, _i32, _i32, _vp, _i32, _vp, _f32, _vp, _vp, _vp, _i64, _vp]),
    "pkv_scale_logits": (_i32, [_vp, _i64, _i32, _i32, _i32, _vp, _i64, _i32, _vp, _vp, _vp, _i64, _vp]),
    "pkv_batch_prefill_valu": (
        _i32,
        [_vp, _i64, _i64, _vp, _i32, _vp, _vp, _i64, _i64, _vp, _vp, _i64, _vp, _i32, _i32, _i32,
         _i32, _i32, _i32, _f32, _vp, _i64, _i64, _i32, _vp],
    ),
}

ERRORS = {
    -1: "unsupported dtype",
    -2: "unsupported head_dim",
    -3: "unsupported GQA group (num_qo_heads / num_kv_heads)",
    -4: "misaligned tensor",
    -5: "invalid argument",
    -6: "workspace buffer too small",
    -7: "unsupported page_size",
}

_LIB = None


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m ecahlang_amd.build` "
                "(there is no CPU or PyTorch fallback for the paged-KV kernels)")
        h = C.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_GLOBAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = h
    return _LIB


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = ERRORS.get(rc, f"HIP error {rc}")
        raise RuntimeError(f"{what} failed: {msg}")


DTYPE_CODE = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


def dtype_code(dt: torch.dtype) -> int:
    try:
        return DTYPE_CODE[dt]
    except KeyError:
        raise ValueError(f"unsupported dtype {dt}; expected float16, bfloat16 or float32") from None


def stream_ptr(device: torch.device | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream
