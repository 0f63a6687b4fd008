"""FlashInfer-shaped batch attention wrappers over the paged cache, backed by libpagedkv.so.

The reference builds one wrapper of each kind on a 128 MiB workspace (ecahlang/main.py:201-204),
calls ``plan`` once per scheduler step with the step's page table (main.py:341-347, 431-455,
538-548, 916-922, 963-969) and ``run(q, kv_cache[layer])`` once per layer from the attention
hook (main.py:68), also inside captured CUDA graphs (main.py:146-148).  The classes below
keep that call shape:

* ``plan`` reads no device data on the host: the decode schedule is built on the device (two
  small kernels, plus a fill kernel that zeroes the split counters when the batch grows), so
  it stays cheap, never synchronises and can be captured.
* ``run`` only enqueues kernels on the current stream and is safe to capture in a hipGraph;
  its geometry (workgroup count, kernel choice) is fixed by ``plan``'s arguments alone.
"""
from __future__ import annotations


import math
import os

import numpy as np

import torch

from ._lib import check, dtype_code, lib, stream_ptr
from .ops import CacheView, _i32

_STR_DTYPES = {"float16": torch.float16, "half": torch.float16, "bfloat16": torch.bfloat16,
               "float32": torch.float32, "float": torch.float32}


def _as_dtype(d) -> torch.dtype:
    if isinstance(d, torch.dtype):
        return d
    try:
        return _STR_DTYPES[str(d).replace("torch.", "")]
    except KeyError:
        raise ValueError(f"unsupported data type {d!r}") from None


def _num_cus(device: torch.device) -> int:
    return torch.cuda.get_device_properties(device).multi_processor_count


def _unsupported(pos_encoding_mode, window_left, logits_soft_cap, rope_scale, rope_theta):
    if str(pos_encoding_mode).upper() != "NONE":
        raise NotImplementedError("pos_encoding_mode must be 'NONE' (RoPE is applied before the hook)")
    if window_left is not None and window_left >= 0:
        raise NotImplementedError("sliding-window attention (window_left >= 0) is not implemented")
    if logits_soft_cap not in (None, 0, 0.0):
        raise NotImplementedError("logits_soft_cap is not implemented")
    if rope_scale is not None or rope_theta is not None:
        raise NotImplementedError("in-kernel RoPE is not implemented")


_DECODE_VALU, _DECODE_DYNAMIC, _DECODE_PLANNED = 1, 2, 4  # pkv_batch_decode flags (include/pagedkv.h)
_PLAN_CASCADE = 1  # pkv_decode_plan flag
_INIT_COUNTERS = 8192  # decode split counters zeroed when a workspace is given

class BatchDecodeWithPagedKVCacheWrapper:
    """Paged decode attention: one query token per sequence (FlashInfer contract)."""

    def __init__(self, float_workspace_buffer: torch.Tensor, kv_layout: str = "NHD",
                 use_cuda_graph: bool = False, use_tensor_cores: bool = False,
                 paged_kv_indptr_buffer=None, paged_kv_indices_buffer=None,
                 paged_kv_last_page_len_buffer=None, backend: str = "auto", jit_args=None):
        if kv_layout.upper() != "NHD":
            raise NotImplementedError("only the NHD layout is implemented (the reference uses NHD)")
        if float_workspace_buffer.device.type != "cuda":
            raise ValueError("workspace must be a CUDA (HIP) tensor")
        self._workspace = float_workspace_buffer
        self._kv_layout = "NHD"
        self._use_cuda_graph = use_cuda_graph
        self._planned = False
        self._zero_counters()
        # Whether this wrapper's schedules carry cascade prefix items.  run() picks the kernel
        # variant from it when it is enqueued, so a run captured in a graph keeps the variant of
        # its plan: once a run has been captured, a plan that changes it is refused (replays
        # would run the wrong variant on the new schedule).
        self._cascade_mode = False
        self._captured_mode: bool | None = None

    @property
    def is_cuda_graph_enabled(self) -> bool:
        return self._use_cuda_graph

    def reset_workspace_buffer(self, float_workspace_buffer: torch.Tensor, *_args) -> None:
        self._workspace = float_workspace_buffer
        self._zero_counters()
        self._captured_mode = None

    def _zero_counters(self) -> None:
        """The workspace starts with one split counter per sequence (int32), which the decode
        leaves at zero (each sequence's last arrival resets its own).  The first
        ``_INIT_COUNTERS`` are zeroed here, when the workspace is given, so that a plan
        captured in a graph does not record the fill.  ``_counters_ready``: how many leading
        counters are known to be zero; a plan's schedule overwrites the words after its own
        batch's counters, so it lowers the count to that batch."""
        self._counters_ready = 0
        n = min(_INIT_COUNTERS, self._workspace.numel() * self._workspace.element_size() // 4)
        if n > 0 and not torch.cuda.is_current_stream_capturing():
            dev = self._workspace.device
            check(lib().pkv_decode_workspace_init(self._workspace.data_ptr(), n, stream_ptr(dev)),
                  "decode workspace")
            # (complete before any stream's plan or run reads the counters)
            torch.cuda.current_stream(dev).synchronize()
            self._counters_ready = n

    def plan(self, indptr: torch.Tensor, indices: torch.Tensor, last_page_len: torch.Tensor,
             num_qo_heads: int, num_kv_heads: int, head_dim: int, page_size: int,
             pos_encoding_mode: str = "NONE", window_left: int = -1, logits_soft_cap=None,
             q_data_type="float16", kv_data_type=None, data_type=None, sm_scale=None,
             rope_scale=None, rope_theta=None, non_blocking: bool = True,
             num_ctas: int | None = None, deterministic: bool = True,
             kv_shared_pages: torch.Tensor | None = None, cascade: bool = False, **_unused) -> None:
        """Extensions: ``num_ctas`` fixes the number of workgroups that share the batch's
        pages (by default one per compute unit for the matrix-core kernel);
        ``deterministic=False`` lets the waves of a workgroup take pages on demand, which is
        a little faster but makes the last bits of the result vary from call to call (with
        the default the result is bitwise reproducible, as FlashInfer's is);
        ``kv_shared_pages`` (int32 [batch] on the device, as
        ``AutoKVCacheManager.fill_cuda_graph_metadata`` leaves it in ``_cg_kv_shared``) says,
        for each sequence b >= 1, how many of its leading pages are the same pages as sequence
        b - 1's (the caller guarantees the pages agree, as it does for the rest of the page
        table): a prefix that runs of sequences share is then kept in L2 for its readers after
        the first, and with ``cascade=True`` it is read once per group of 2 * (16 / g) sequences
        (g = num_qo_heads / num_kv_heads) instead (include/pagedkv.h, pkv_decode_plan)."""
        _unsupported(pos_encoding_mode, window_left, logits_soft_cap, rope_scale, rope_theta)
        self._indptr = _i32(indptr, "indptr")
        self._indices = _i32(indices, "indices")
        self._last = _i32(last_page_len, "last_page_len")
        self._batch = indptr.numel() - 1
        if self._last.numel() != self._batch:
            raise ValueError("last_page_len must have one entry per sequence")
        if num_qo_heads % num_kv_heads:
            raise ValueError("num_qo_heads must be a multiple of num_kv_heads")
        self._hq, self._hkv, self._d, self._ps = int(num_qo_heads), int(num_kv_heads), int(head_dim), int(page_size)
        if data_type is not None:
            q_data_type = data_type
        self._q_dtype = _as_dtype(q_data_type)
        self._kv_dtype = _as_dtype(kv_data_type) if kv_data_type is not None else self._q_dtype
        if self._kv_dtype != self._q_dtype:
            raise NotImplementedError("q and kv must share one dtype")
        self._sm_scale = float(sm_scale) if sm_scale is not None else 1.0 / math.sqrt(self._d)
        dev = indptr.device
        self._mfma = bool(lib().pkv_decode_uses_mfma(dtype_code(self._q_dtype), self._d, self._hq,
                                                     self._hkv, self._batch)) and self._ps == 16
        env = os.environ.get("PKV_DECODE_CTAS")
        if num_ctas is not None:
            self._ctas = int(num_ctas)
        elif env:
            self._ctas = int(env)
        else:
            self._ctas = _num_cus(dev) if self._mfma else 2 * _num_cus(dev)
        if self._ctas <= 0:
            raise ValueError("num_ctas must be positive")
        need = lib().pkv_decode_workspace_bytes(self._batch, self._hq, self._d, self._ctas,
                                                self._indices.numel())
        if need < 0:
            check(int(need), "decode plan")
        if need > self._workspace.numel() * self._workspace.element_size():
            raise RuntimeError(f"decode workspace too small: need {need} bytes")
        if self._batch > self._counters_ready:
            check(lib().pkv_decode_workspace_init(self._workspace.data_ptr(), self._batch,
                                                  stream_ptr(dev)), "decode plan")
        self._counters_ready = self._batch  # (the schedule is written after these)
        self._flags = 0 if deterministic else _DECODE_DYNAMIC
        shared = 0
        if kv_shared_pages is not None:
            self._shared = _i32(kv_shared_pages, "kv_shared_pages")
            if self._shared.numel() < self._batch:
                raise ValueError("kv_shared_pages must have one entry per sequence")
            shared = self._shared.data_ptr()
        cascade = bool(cascade) and kv_shared_pages is not None
        if self._captured_mode is not None and cascade != self._captured_mode:
            raise ValueError("plan(cascade=...) must not change after a run of this wrapper was captured "
                             "in a graph (replays keep the kernel variant of the captured plan); "
                             "use another wrapper or reset_workspace_buffer()")
        self._cascade_mode = cascade
        if self._mfma:
            # the matrix-core kernel's schedule, built on the device from this page table
            check(lib().pkv_decode_plan(self._indptr.data_ptr(), self._indices.data_ptr(),
                                        self._indices.numel(), self._last.data_ptr(), shared, self._batch,
                                        self._hq, self._hkv, self._d, self._ps, self._ctas,
                                        _PLAN_CASCADE if cascade else 0,
                                        self._workspace.data_ptr(),
                                        self._workspace.numel() * self._workspace.element_size(),
                                        stream_ptr(dev)), "decode plan")
            self._flags |= _DECODE_PLANNED
        self._planned = True

    def run(self, q: torch.Tensor, paged_kv_cache, *args, q_scale=None, k_scale=None,
            v_scale=None, out: torch.Tensor | None = None, lse=None, return_lse: bool = False,
            window_left=None, enable_pdl=None, force_valu: bool = False, append_kv=None) -> torch.Tensor:
        """FlashInfer's run (ecahlang/main.py:68).  Extension: ``append_kv=(k, v)``, each
        [batch, num_kv_heads, head_dim] with unit inner stride, first appends token b's rows at
        position seq_len_b - 1 (the decode step's append through the CUDA-graph metadata,
        ecahlang/manager.py:270-280) -- in the same launch on the matrix-core path."""
        if not self._planned:
            raise RuntimeError("plan() must be called before run()")
        if torch.cuda.is_current_stream_capturing():
            self._captured_mode = self._cascade_mode
        if return_lse or lse is not None:
            raise NotImplementedError("return_lse is not implemented")
        if q_scale is not None or k_scale is not None or v_scale is not None:
            raise NotImplementedError("fp8 scales are not implemented")
        cv = CacheView(paged_kv_cache, self._kv_layout)
        if q.dim() != 3 or q.shape != (self._batch, self._hq, self._d) or q.stride(2) != 1:
            raise ValueError(f"q must be [{self._batch}, {self._hq}, {self._d}] with unit inner stride")
        if q.dtype != self._q_dtype or cv.dtype != self._q_dtype:
            raise ValueError(f"q / cache dtype must be {self._q_dtype}")
        if (cv.num_kv_heads, cv.head_dim, cv.page_size) != (self._hkv, self._d, self._ps):
            raise ValueError("cache geometry differs from plan()")
        if out is None:
            out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        elif out.shape != q.shape or out.dtype != q.dtype or out.stride(2) != 1:
            raise ValueError("out must match q's shape and dtype")
        if append_kv is not None:
            k, v = append_kv
            for t, n in ((k, "k"), (v, "v")):
                if t.shape != (self._batch, self._hkv, self._d) or t.stride(2) != 1 or t.dtype != self._q_dtype:
                    raise ValueError(f"append {n} must be [{self._batch}, {self._hkv}, {self._d}] "
                                     f"{self._q_dtype} with unit inner stride")
            check(lib().pkv_batch_decode_append(
                q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
                v.data_ptr(), v.stride(0), v.stride(1), cv.k_ptr, cv.v_ptr, cv.page_stride, cv.num_pages,
                self._indptr.data_ptr(), self._indices.data_ptr(), self._indices.numel(),
                self._last.data_ptr(), self._batch,
                self._hq, self._hkv, self._d, self._ps, self._sm_scale, self._ctas,
                self._workspace.data_ptr(), self._workspace.numel() * self._workspace.element_size(),
                out.data_ptr(), out.stride(0), out.stride(1), dtype_code(q.dtype),
                self._flags | (_DECODE_VALU if force_valu else 0),
                stream_ptr(q.device)), "BatchDecodeWithPagedKVCacheWrapper.run(append_kv=)")
            return out
        check(lib().pkv_batch_decode(
            q.data_ptr(), q.stride(0), q.stride(1), cv.k_ptr, cv.v_ptr, cv.page_stride, cv.num_pages,
            self._indptr.data_ptr(), self._indices.data_ptr(), self._indices.numel(),
            self._last.data_ptr(), self._batch,
            self._hq, self._hkv, self._d, self._ps, self._sm_scale, self._ctas,
            self._workspace.data_ptr(), self._workspace.numel() * self._workspace.element_size(),
            out.data_ptr(), out.stride(0), out.stride(1), dtype_code(q.dtype),
            self._flags | (_DECODE_VALU if force_valu else 0),
            stream_ptr(q.device)), "BatchDecodeWithPagedKVCacheWrapper.run")
        return out

    forward = run


def prefill_work_list(qo_indptr, kv_indptr, last_page_len, g: int, hkv: int, page_size: int,
                      causal: bool, head_dim: int, num_cus: int, ws_bytes: int, rows: int = 256,
                      partial_bytes: int = 4, chunk: int | None = None) -> dict:
    """The matrix-core prefill kernel's work list, built on the host by the library
    (``pkv_prefill_work_list``).  Items are (request, KV head, rows/g query tokens, chunk of the
    keys those tokens see): the 12 int32 fields
    [b, h, t0, tq, k0, k1, slot, kv_len, qo_len, qo_start, kv_indptr[b], 0].  A key range longer
    than the chunk is cut into chunks (slot >= 0) that form a split group
    [first slot, chunks, qo_start, t0, tq, h, 0, 0], whose partials a second kernel merges.
    Chunks are whole steps of the kernel (64 keys); unless ``chunk`` fixes it, the chunk is the
    one among a few around total keys / CUs whose simulated kernel time (items longest first,
    each to the least loaded CU) is lowest, and it is doubled while the partials would not fit
    in ``ws_bytes``.  ``partial_bytes`` is the size of one element of a partial output row: 2
    for fp16 caches (the kernel keeps their partials in fp16), 4 otherwise.  Items are issued
    longest first.  ``items`` / ``groups`` are lists of records; ``items_np`` / ``groups_np``
    the same as int32 arrays."""
    qo = np.ascontiguousarray(np.asarray(qo_indptr, dtype=np.int64), dtype=np.int32)
    kv = np.ascontiguousarray(np.asarray(kv_indptr, dtype=np.int64), dtype=np.int32)
    last = np.ascontiguousarray(np.asarray(last_page_len, dtype=np.int64), dtype=np.int32)
    B = len(qo) - 1
    if len(kv) != B + 1 or len(last) < B:
        raise ValueError("indptr / last_page_len lengths do not match")
    # capacity: every (request, query tile, KV head) holds at most max(1, kv_len / 256) chunks
    tq_max = max(1, rows // max(1, g))
    qn = np.diff(qo.astype(np.int64))
    npg = np.diff(kv.astype(np.int64))
    kvl = np.where(npg > 0, (npg - 1) * page_size + last[:B], 0)
    tiles = -(-np.maximum(qn, 0) // tq_max)
    n_groups_cap = int((tiles * hkv).sum())
    n_items_cap = int((tiles * hkv * np.maximum(1, -(-np.maximum(kvl, 0) // 256))).sum())
    items = np.zeros((max(1, n_items_cap), 12), dtype=np.int32)
    groups = np.zeros((max(1, n_groups_cap), 8), dtype=np.int32)
    info = np.zeros(8, dtype=np.int64)
    L = lib()
    rc = L.pkv_prefill_work_list(qo.ctypes.data, kv.ctypes.data, last.ctypes.data, B, int(g), int(hkv),
                                 int(page_size), 1 if causal else 0, int(head_dim), int(num_cus), int(ws_bytes),
                                 int(rows), int(partial_bytes), int(chunk or 0), items.ctypes.data,
                                 items.shape[0], groups.ctypes.data, groups.shape[0], info.ctypes.data)
    if rc == -6:
        raise RuntimeError(f"prefill workspace too small: need {int(info[7])} bytes")
    check(int(rc), "prefill plan")
    ni, ng = int(info[0]), int(info[1])
    items, groups = items[:ni], groups[:ng]
    return {"items": items.tolist(), "groups": groups.tolist(), "items_np": items, "groups_np": groups,
            "chunk": int(info[2]), "slots": int(info[3]), "off_groups": int(info[4]), "off_ml": int(info[5]),
            "off_o": int(info[6]), "bytes": int(info[7])}


class BatchPrefillWithPagedKVCacheWrapper:
    """Paged (chunked) prefill attention over ragged query rows (FlashInfer contract)."""

    def __init__(self, float_workspace_buffer: torch.Tensor, kv_layout: str = "NHD",
                 use_cuda_graph: bool = False, qo_indptr_buf=None, paged_kv_indptr_buf=None,
                 paged_kv_indices_buf=None, paged_kv_last_page_len_buf=None, custom_mask_buf=None,
                 mask_indptr_buf=None, backend: str = "auto", jit_args=None):
        if kv_layout.upper() != "NHD":
            raise NotImplementedError("only the NHD layout is implemented (the reference uses NHD)")
        self._workspace = float_workspace_buffer
        self._kv_layout = "NHD"
        self._use_cuda_graph = use_cuda_graph
        self._planned = False

    @property
    def is_cuda_graph_enabled(self) -> bool:
        return self._use_cuda_graph

    def plan(self, qo_indptr: torch.Tensor, paged_kv_indptr: torch.Tensor,
             paged_kv_indices: torch.Tensor, paged_kv_last_page_len: torch.Tensor,
             num_qo_heads: int, num_kv_heads: int, head_dim_qk: int, page_size: int,
             head_dim_vo: int | None = None, custom_mask=None, packed_custom_mask=None,
             causal: bool = False, pos_encoding_mode: str = "NONE",
             use_fp16_qk_reduction: bool = False, sm_scale=None, window_left: int = -1,
             logits_soft_cap=None, rope_scale=None, rope_theta=None, q_data_type="float16",
             kv_data_type=None, non_blocking: bool = True, **_unused) -> None:
        _unsupported(pos_encoding_mode, window_left, logits_soft_cap, rope_scale, rope_theta)
        if custom_mask is not None or packed_custom_mask is not None:
            raise NotImplementedError("custom masks are not implemented")
        if head_dim_vo is not None and head_dim_vo != head_dim_qk:
            raise NotImplementedError("head_dim_vo must equal head_dim_qk")
        self._qo_indptr = _i32(qo_indptr, "qo_indptr")
        self._indptr = _i32(paged_kv_indptr, "paged_kv_indptr")
        self._indices = _i32(paged_kv_indices, "paged_kv_indices")
        self._last = _i32(paged_kv_last_page_len, "paged_kv_last_page_len")
        self._batch = paged_kv_indptr.numel() - 1
        if qo_indptr.numel() != self._batch + 1 or self._last.numel() != self._batch:
            raise ValueError("qo_indptr / last_page_len disagree with the batch size")
        if num_qo_heads % num_kv_heads:
            raise ValueError("num_qo_heads must be a multiple of num_kv_heads")
        self._hq, self._hkv, self._d, self._ps = int(num_qo_heads), int(num_kv_heads), int(head_dim_qk), int(page_size)
        self._causal = bool(causal)
        self._q_dtype = _as_dtype(q_data_type)
        self._kv_dtype = _as_dtype(kv_data_type) if kv_data_type is not None else self._q_dtype
        if self._kv_dtype != self._q_dtype:
            raise NotImplementedError("q and kv must share one dtype")
        self._sm_scale = float(sm_scale) if sm_scale is not None else 1.0 / math.sqrt(self._d)
        self._mfma = bool(lib().pkv_prefill_mfma_supported(dtype_code(self._q_dtype), self._d, self._hq,
                                                          self._hkv, self._ps))
        if self._mfma:
            self._schedule(qo_indptr.device)
        self._planned = True

    # rows per matrix-core work item (8 waves x 32 rows): 256 / g query tokens of one KV head
    _ROWS = 256

    def _schedule(self, dev: torch.device) -> None:
        """The matrix-core kernel's work list (``prefill_work_list``) copied into the
        workspace.  Like FlashInfer's plan, this reads the (small) indptr arrays back to the
        host once per batch."""
        qo = self._qo_indptr.cpu().tolist()
        kp = self._indptr.cpu().tolist()
        last = self._last.cpu().tolist()
        self._nnz_q = qo[-1]
        ws_bytes = self._workspace.numel() * self._workspace.element_size()
        # (the kernel keeps an fp16 cache's split partials in fp16)
        wl = prefill_work_list(qo, kp, last, self._hq // self._hkv, self._hkv, self._ps, self._causal, self._d,
                               _num_cus(dev), ws_bytes, self._ROWS,
                               partial_bytes=2 if self._q_dtype == torch.float16 else 4)
        items, merges = wl["items_np"], wl["groups_np"]
        off_g, off_ml, off_o = wl["off_groups"], wl["off_ml"], wl["off_o"]
        if len(items):
            flat = np.zeros(off_g // 4 + merges.size, dtype=np.int32)
            flat[: items.size] = items.reshape(-1)
            flat[off_g // 4:] = merges.reshape(-1)
            host = torch.from_numpy(flat).pin_memory()
            self._workspace.view(torch.uint8)[: 4 * flat.size].view(torch.int32).copy_(host, non_blocking=True)
        base = self._workspace.data_ptr()
        self._n_items, self._n_groups = len(items), len(merges)
        self._items_ptr, self._groups_ptr = base, base + off_g
        self._ml_ptr, self._o_ptr = base + off_ml, base + off_o
        self._chunk = wl["chunk"]

    def run(self, q: torch.Tensor, paged_kv_cache, *args, q_scale=None, k_scale=None,
            v_scale=None, out: torch.Tensor | None = None, lse=None, return_lse: bool = False,
            enable_pdl=None, window_left=None, force_valu: bool = False) -> torch.Tensor:
        if not self._planned:
            raise RuntimeError("plan() must be called before run()")
        if return_lse or lse is not None:
            raise NotImplementedError("return_lse is not implemented")
        cv = CacheView(paged_kv_cache, self._kv_layout)
        if q.dim() != 3 or q.shape[1:] != (self._hq, self._d) or q.stride(2) != 1:
            raise ValueError(f"q must be [nnz, {self._hq}, {self._d}] with unit inner stride")
        if q.dtype != self._q_dtype or cv.dtype != self._q_dtype:
            raise ValueError(f"q / cache dtype must be {self._q_dtype}")
        if (cv.num_kv_heads, cv.head_dim, cv.page_size) != (self._hkv, self._d, self._ps):
            raise ValueError("cache geometry differs from plan()")
        nnz = q.shape[0]
        if out is None:
            out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        elif out.shape != q.shape or out.dtype != q.dtype or out.stride(2) != 1:
            raise ValueError("out must match q's shape and dtype")
        aligned = q.data_ptr() % 16 == 0 and (q.stride(0) * q.element_size()) % 16 == 0 and \
            (q.stride(1) * q.element_size()) % 16 == 0
        if self._mfma and aligned and not force_valu:
            if nnz < self._nnz_q:
                raise ValueError(f"q has {nnz} rows, qo_indptr needs {self._nnz_q}")
            check(lib().pkv_batch_prefill_mfma(
                q.data_ptr(), q.stride(0), q.stride(1), cv.k_ptr, cv.v_ptr, cv.page_stride, cv.num_pages,
                self._indices.data_ptr(), self._indices.numel(), self._hq, self._hkv, self._d, self._ps,
                int(self._causal), self._sm_scale, self._items_ptr, self._n_items, self._groups_ptr,
                self._n_groups, self._ml_ptr, self._o_ptr, out.data_ptr(), out.stride(0), out.stride(1),
                dtype_code(q.dtype), stream_ptr(q.device)), "BatchPrefillWithPagedKVCacheWrapper.run")
            return out
        check(lib().pkv_batch_prefill_valu(
            q.data_ptr(), q.stride(0), q.stride(1), self._qo_indptr.data_ptr(), nnz, cv.k_ptr,
            cv.v_ptr, cv.page_stride, cv.num_pages, self._indptr.data_ptr(),
            self._indices.data_ptr(), self._indices.numel(), self._last.data_ptr(), self._batch, self._hq, self._hkv, self._d, self._ps,
            int(self._causal), self._sm_scale, out.data_ptr(), out.stride(0), out.stride(1),
            dtype_code(q.dtype), stream_ptr(q.device)), "BatchPrefillWithPagedKVCacheWrapper.run")
        return out

    forward = run
