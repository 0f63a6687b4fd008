"""Seeded synthetic paged-KV workloads: decode and chunked-prefill batches.

Each batch is built the way the serving loop leaves the cache just before the attention
call: every sequence owns a run of pages taken from a seeded random permutation of the pool,
the page table follows the FlashInfer convention (last_page_len = (L-1) % page_size + 1), the
existing context is written into its slots, every other slot of the pool is NaN so a read of
anything outside the page table shows up in the output, and the new tokens' K/V (plus their
batch indices and positions) are ready for the append.  Values are generated on the CPU from
torch.Generator(seed) in fp32 and cast, so a CPU check sees the same bits as the device.

Named shapes (heads q / kv, head_dim, dtype):
  llama32_1b_fp32   32 / 8 / 64,  float32   (decode, batch 4, context 17, 64, 129, 300)
  qwen25_3b_fp16    16 / 2 / 128, float16   (decode, batch 64, context U[512, 4096])
  llama31_8b_bf16   32 / 8 / 128, bfloat16  (decode, batch 128, context log-U[1024, 32768])
"""
from __future__ import annotations

import contextlib
import math
from dataclasses import dataclass, field

import torch


@dataclass
class PagedBatch:
    hq: int
    hkv: int
    d: int
    ps: int
    dtype: torch.dtype
    num_pages: int
    kv_len: list            # tokens per sequence after the append
    new_len: list           # appended tokens per sequence (1 for decode, the chunk for prefill)
    cache: torch.Tensor     # [pages, 2, ps, hkv, d]
    indptr: torch.Tensor    # int32 [B+1]
    indices: torch.Tensor   # int32 [sum pages]
    last: torch.Tensor      # int32 [B]
    append_indptr: torch.Tensor  # int32 [B+1]
    batch_indices: torch.Tensor  # int32 [nnz]
    positions: torch.Tensor      # int32 [nnz]
    k_new: torch.Tensor     # [nnz, hkv, d]
    v_new: torch.Tensor     # [nnz, hkv, d]
    q: torch.Tensor         # [nnz, hq, d] (one row per appended token)
    extra: dict = field(default_factory=dict)

    @property
    def batch(self) -> int:
        return len(self.kv_len)

    def kv_bytes(self) -> int:
        es = torch.tensor([], dtype=self.dtype).element_size()
        return sum(self.kv_len) * 2 * self.hkv * self.d * es

    def to(self, device) -> "PagedBatch":
        kw = {}
        for name in self.__dataclass_fields__:
            v = getattr(self, name)
            kw[name] = v.to(device) if isinstance(v, torch.Tensor) else v
        return PagedBatch(**kw)


def _randn(gen, shape, scale, dtype):
    return (torch.randn(shape, generator=gen, dtype=torch.float32) * scale).to(dtype)


def build_batch(kv_len, new_len, hq, hkv, d, dtype, seed, *, ps=16, scale=1.0,
                pool_pages=None, pool_factor=1.25, fill_old=True) -> PagedBatch:
    """CPU-resident batch; call ``.to("cuda")`` for the device copy (bits unchanged)."""
    gen = torch.Generator().manual_seed(seed)
    kv_len = [int(x) for x in kv_len]
    new_len = [int(x) for x in new_len]
    B = len(kv_len)
    npages = [(L + ps - 1) // ps for L in kv_len]
    total_pages = sum(npages)
    P = pool_pages if pool_pages is not None else max(int(math.ceil(pool_factor * total_pages)), 1)
    if P < total_pages:
        raise ValueError("pool smaller than the pages the batch needs")
    perm = torch.randperm(P, generator=gen).to(torch.int32)
    indices = perm[:total_pages].clone()
    indptr = torch.zeros(B + 1, dtype=torch.int32)
    indptr[1:] = torch.cumsum(torch.tensor(npages, dtype=torch.int64), 0).to(torch.int32)
    last = torch.tensor([((L - 1) % ps) + 1 if L > 0 else 0 for L in kv_len], dtype=torch.int32)

    cache = torch.full((P, 2, ps, hkv, d), float("nan"), dtype=dtype)
    old_len = [L - n for L, n in zip(kv_len, new_len)]
    if fill_old and sum(old_len):
        tok_page, tok_slot = [], []
        for b in range(B):
            pos = torch.arange(old_len[b])
            tok_page.append(indices[indptr[b] + pos // ps].long())
            tok_slot.append(pos % ps)
        tp, ts = torch.cat(tok_page), torch.cat(tok_slot)
        n_old = tp.numel()
        cache[tp, 0, ts] = _randn(gen, (n_old, hkv, d), scale, dtype)
        cache[tp, 1, ts] = _randn(gen, (n_old, hkv, d), scale, dtype)

    nnz = sum(new_len)
    append_indptr = torch.zeros(B + 1, dtype=torch.int32)
    append_indptr[1:] = torch.cumsum(torch.tensor(new_len, dtype=torch.int64), 0).to(torch.int32)
    bidx = torch.repeat_interleave(torch.arange(B, dtype=torch.int32),
                                   torch.tensor(new_len, dtype=torch.int64))
    pos = torch.cat([torch.arange(o, L, dtype=torch.int32) for o, L in zip(old_len, kv_len)]) \
        if nnz else torch.zeros(0, dtype=torch.int32)
    k_new = _randn(gen, (nnz, hkv, d), scale, dtype)
    v_new = _randn(gen, (nnz, hkv, d), scale, dtype)
    q = _randn(gen, (nnz, hq, d), scale, dtype)
    return PagedBatch(hq, hkv, d, ps, dtype, P, kv_len, new_len, cache, indptr, indices, last,
                      append_indptr, bidx, pos, k_new, v_new, q)


def llama32_1b_decode(seed=1001) -> PagedBatch:
    """32 q / 8 kv heads, head_dim 64, fp32; batch 4 with context 17, 64, 129, 300; pool 256."""
    ctx = [17, 64, 129, 300]
    return build_batch([c + 1 for c in ctx], [1] * 4, 32, 8, 64, torch.float32, seed,
                       pool_pages=256, scale=1.0)


def qwen25_3b_lengths(seed=1002, batch=64, lo=512, hi=4096) -> list:
    """Tokens per sequence after the step's append: context U[lo, hi] + 1."""
    g = torch.Generator().manual_seed(seed + 7919)
    return [c + 1 for c in torch.randint(lo, hi + 1, (batch,), generator=g).tolist()]


def qwen25_3b_decode(seed=1002, batch=64, lo=512, hi=4096) -> PagedBatch:
    """16 q / 2 kv heads, head_dim 128, fp16; context U[lo, hi]; pool 1.25x the pages used."""
    return build_batch(qwen25_3b_lengths(seed, batch, lo, hi), [1] * batch, 16, 2, 128, torch.float16, seed,
                       scale=0.5)


def paged_table(kv_len, pool_pages, seed, ps=16):
    """(indptr, indices, last) int32 host tensors: each sequence's pages a run of a seeded random
    permutation of the pool (the page table device_decode_batch builds for the same arguments)."""
    gen = torch.Generator().manual_seed(seed)
    npages = [(int(L) + ps - 1) // ps for L in kv_len]
    total = sum(npages)
    if pool_pages < total:
        raise ValueError("pool smaller than the pages the batch needs")
    indices = torch.randperm(pool_pages, generator=gen)[:total].to(torch.int32)
    indptr = torch.zeros(len(kv_len) + 1, dtype=torch.int32)
    indptr[1:] = torch.cumsum(torch.tensor(npages, dtype=torch.int64), 0).to(torch.int32)
    last = torch.tensor([((int(L) - 1) % ps) + 1 if L else 0 for L in kv_len], dtype=torch.int32)
    return indptr, indices, last


def qwen25_3b_prefill(seed=1003, requests=8, chunk=512, max_prefix=8192) -> PagedBatch:
    """16 q / 2 kv heads, head_dim 128, fp16; each request appends a `chunk`-token chunk onto a
    paged prefix of U[0, max_prefix] tokens; causal ragged attention over prefix + chunk."""
    g = torch.Generator().manual_seed(seed + 7919)
    prefix = torch.randint(0, max_prefix + 1, (requests,), generator=g).tolist()
    return build_batch([p + chunk for p in prefix], [chunk] * requests, 16, 2, 128,
                       torch.float16, seed, scale=0.5)


def llama31_8b_decode(seed=1004, batch=128, lo=1024, hi=32768, pool_pages=None) -> PagedBatch:
    """32 q / 8 kv heads, head_dim 128, bf16; context log-uniform in [lo, hi]."""
    g = torch.Generator().manual_seed(seed + 7919)
    u = torch.rand(batch, generator=g, dtype=torch.float64)
    ctx = torch.floor(torch.exp(math.log(lo) + u * (math.log(hi) - math.log(lo)))).long().tolist()
    return build_batch([c + 1 for c in ctx], [1] * batch, 32, 8, 128, torch.bfloat16, seed,
                       scale=1.0, pool_pages=pool_pages)


@dataclass
class DeviceDecodeBatch:
    """A decode batch generated directly in device memory (pools too large to build on the
    host): the page table is built on the host, the K/V values with a device generator."""
    hq: int
    hkv: int
    d: int
    ps: int
    dtype: torch.dtype
    num_pages: int
    kv_len: list
    cache: torch.Tensor      # [P, 2, ps, Hkv, D] on the device, unused slots NaN
    indptr: torch.Tensor     # device int32
    indices: torch.Tensor
    last: torch.Tensor
    q: torch.Tensor          # [B, Hq, D] on the device

    @property
    def batch(self) -> int:
        return len(self.kv_len)


def device_decode_batch(kv_len, hq, hkv, d, dtype, seed, pool_pages, device, *, ps=16,
                        scale=1.0) -> DeviceDecodeBatch:
    """Pages of each sequence scattered by a seeded permutation of the pool (host); the used
    pages filled with N(0,1)*scale on the device, every other slot (unused pages and the
    slots past each sequence's last token) NaN."""
    kv_len = [int(x) for x in kv_len]
    indptr, indices, last = paged_table(kv_len, pool_pages, seed, ps)
    total = int(indptr[-1])
    dgen = torch.Generator(device=device).manual_seed(seed)
    cache = torch.full((pool_pages, 2, ps, hkv, d), float("nan"), dtype=dtype, device=device)
    idx = indices.to(device).long()
    chunk = 8192  # pages per fill (bounded temporary)
    for s in range(0, total, chunk):
        pg = idx[s:s + chunk]
        cache[pg] = (torch.randn((pg.numel(), 2, ps, hkv, d), generator=dgen, device=device,
                                 dtype=torch.float32) * scale).to(dtype)
    for b, L in enumerate(kv_len):  # poison the tail of each last page
        if L and last[b] < ps:
            cache[int(indices[indptr[b + 1] - 1]), :, int(last[b]):] = float("nan")
    q = (torch.randn((len(kv_len), hq, d), generator=dgen, device=device, dtype=torch.float32)
         * scale).to(dtype)
    return DeviceDecodeBatch(hq, hkv, d, ps, dtype, pool_pages, kv_len, cache, indptr.to(device),
                             indices.to(device), last.to(device), q)


def llama31_8b_lengths(seed=1004, batch=128, lo=1024, hi=32768) -> list:
    """Tokens per sequence after the step's append: context log-uniform in [lo, hi] + 1."""
    g = torch.Generator().manual_seed(seed + 7919)
    u = torch.rand(batch, generator=g, dtype=torch.float64)
    ctx = torch.floor(torch.exp(math.log(lo) + u * (math.log(hi) - math.log(lo)))).long().tolist()
    return [c + 1 for c in ctx]


LLAMA31_8B_POOL_PAGES = 20_000_000_000 // (2 * 16 * 8 * 128 * 2)  # a ~20 GB pool of 64 KiB pages


def llama31_8b_decode_device(device, seed=1004, batch=128, lo=1024, hi=32768,
                             pool_bytes=20_000_000_000) -> DeviceDecodeBatch:
    """Long-context decode at Llama-3.1-8B shape (32 q / 8 kv heads, head_dim 128, bf16):
    context log-uniform in [lo, hi], pages scattered over a pool of ~pool_bytes."""
    page_bytes = 2 * 16 * 8 * 128 * 2
    return device_decode_batch(llama31_8b_lengths(seed, batch, lo, hi), 32, 8, 128, torch.bfloat16, seed,
                               pool_bytes // page_bytes, device)


class SharedPrefixDecodeLoop:
    """Repeated decode steps of every layer of a model over one page pool, driven through
    AutoKVCacheManager and the decode wrapper the way the serving loop drives them
    (ecahlang/main.py:320-381): per step, ``append_tokens(b, 1)`` for every sequence (a page is
    popped on the device when the last one fills), ``fill_cuda_graph_metadata`` for the
    batch's bucket, ``plan``, then one graph replay of every layer's append + decode.

    Every sequence starts with the full pages of one shared prefix (``allocate(...,
    prefix=)``), followed by pages of its own.  ``retire`` frees ``finish`` randomly chosen
    sequences (their own pages go back to the pool; the prefix's stay) and starts as many new
    ones on the same prefix, whose tokens are written into their pages as a prefill would
    leave them.  Default shape: Qwen2.5-3B attention (36 layers, 16 q / 2 kv heads, head_dim
    128, fp16), batch 128, a 2048-token prefix and own suffixes of U[64, 1024] tokens.

    Values are N(0,1)*scale from a device generator; every slot no token owns is NaN.  Lengths
    and the finished sequences come from a host generator.  With ``record=True`` every pool
    operation is logged in ``log`` (so a test can replay it on the oracle's pool).  With
    ``shared_hint`` (the default) the plan is given the manager's shared-prefix hint, so the
    prefix pages stay in L2 for their readers after the first; ``cascade`` asks the plan to read
    the prefix once per group of sequences instead.  With ``device_steps`` the step's
    append_tokens and metadata run on the device (AutoKVCacheManager.begin_device_steps) and the
    graph holds the whole step: page-table step, plan, and every layer's append + decode; the
    host's per-step work is ``advance_device_step``.  With ``fused_append`` (the default) each
    layer's append rides in its decode launch (``run(..., append_kv=)``); without it the append
    is a launch of its own through the bucket's slots, as the reference's step makes it."""

    def __init__(self, device, *, layers=36, batch=128, hq=16, hkv=2, d=128, dtype=torch.float16,
                 prefix_tokens=2048, suffix=(64, 1024), finish=8, max_steps=64, seed=1005, scale=0.5,
                 record=False, shared_hint=True, cascade=False, device_steps=False, fused_append=True):
        from .manager import AutoKVCacheManager
        from .wrappers import BatchDecodeWithPagedKVCacheWrapper

        self.device = torch.device(device)
        self.layers, self.batch, self.hq, self.hkv, self.d, self.dtype = layers, batch, hq, hkv, d, dtype
        self.ps = 16
        self.prefix_tokens, self.suffix, self.finish, self.scale = prefix_tokens, suffix, finish, scale
        self.shared_hint, self.cascade, self.fused_append = shared_hint, cascade, fused_append
        self.device_steps, self.max_steps = device_steps, max_steps
        self.gen = torch.Generator().manual_seed(seed + 7919)
        self.dgen = torch.Generator(device=self.device).manual_seed(seed)
        es = torch.tensor([], dtype=dtype).element_size()
        self.page_bytes = 2 * self.ps * hkv * d * es  # one page of one layer
        own_max = -(-(suffix[1] + max_steps + 1) // self.ps)
        # (device steps widen the table for max_steps more tokens before capture)
        width = -(-prefix_tokens // self.ps) + own_max + (-(-max_steps // self.ps) + 2 if device_steps else 0)
        pool = int(math.ceil(1.25 * (-(-prefix_tokens // self.ps) + batch * own_max))) + batch
        self.mgr = AutoKVCacheManager(layers, hkv, d, dtype=dtype, device=self.device,
                                      total_gpu_mem_bytes=pool * layers * self.page_bytes, mem_utilization=1.0,
                                      max_pages_per_seq=width,
                                      seq_lens=max(128, batch + 1))
        self.mgr.kv_cache.fill_(float("nan"))
        self.log: list = []
        self.record = record
        self.stream = torch.cuda.Stream(device=self.device)
        # the pool's tensors were initialised on the current stream; everything below runs on
        # self.stream
        self.stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(self.stream):
            self.mgr.allocate("prefix", prefix_tokens)
            self._note(("allocate", "prefix", prefix_tokens, None))
            self._write_tokens("prefix", 0)
            self.ids = []
            self._next_id = 0
            for _ in range(batch):
                self.ids.append(self._start_sequence())
            self.mgr.init_cuda_graph_buffers([batch], max_indices=batch * self.mgr._stride)
            self._note(("init_cuda_graph_buffers", [batch]))
            shape = (layers, batch)
            self.q = self._randn(shape + (hq, d))
            self.k = self._randn(shape + (hkv, d))
            self.v = self._randn(shape + (hkv, d))
            self.out = torch.empty_like(self.q)
            self.wrapper = BatchDecodeWithPagedKVCacheWrapper(
                torch.empty(128 << 20, dtype=torch.uint8, device=self.device), "NHD")
        self.graph = None
        self._on_stream = False

    def _note(self, op) -> None:
        if self.record:
            self.log.append(op)

    # ---------------------------------------------------------------- synthetic contents
    def _randn(self, shape):
        return (torch.randn(shape, generator=self.dgen, device=self.device, dtype=torch.float32)
                * self.scale).to(self.dtype)

    def _write_tokens(self, sid, first_page: int) -> None:
        """Fill sequence sid's pages from first_page on (every layer) with fresh values; the
        slots past its last token stay NaN."""
        m = self.mgr
        if m._ops:  # (queued pool operations land first; device-step mode stays on otherwise)
            m._flush()
        n = m._npages[sid]
        if n <= first_page:
            return
        pages = m._table[m.batch_to_seq_len[sid], first_page:n].long()
        cache = m.kv_cache
        cache[:, pages] = self._randn((self.layers, n - first_page, 2, self.ps, self.hkv, self.d))
        last = m.batch_to_page_lengths[sid]
        if last < self.ps:
            cache[:, pages[-1:], :, last:] = float("nan")

    def _start_sequence(self, write: bool = True):
        sid = f"s{self._next_id}"
        self._next_id += 1
        lo, hi = self.suffix
        n = int(torch.randint(lo, hi + 1, (1,), generator=self.gen))
        tokens = self.prefix_tokens + n
        self.mgr.allocate(sid, tokens, prefix="prefix")
        self._note(("allocate", sid, tokens, "prefix"))
        if write:
            self.write_tokens([sid])
        return sid

    def write_tokens(self, sids) -> None:
        """Write the tokens of newly started sequences (their pages after the prefix's full
        ones), as their prefill would leave them."""
        with torch.cuda.stream(self.stream):
            for sid in sids:
                self._write_tokens(sid, self.prefix_tokens // self.ps)

    # ---------------------------------------------------------------- one step
    @contextlib.contextmanager
    def on_stream(self):
        """Make the loop's stream current for a run of steps, so that ``begin_step`` and
        ``replay`` skip switching to it on every call (a few microseconds of host time each)."""
        with torch.cuda.stream(self.stream):
            self._on_stream = True
            try:
                yield self
            finally:
                self._on_stream = False

    def _stream_ctx(self):
        return contextlib.nullcontext() if self._on_stream else torch.cuda.stream(self.stream)

    def begin_step(self) -> None:
        """Host bookkeeping and device metadata for one decode step (main.py:328-347)."""
        m = self.mgr
        if self.device_steps:
            if m._dev is None:
                with self._stream_ctx():
                    self._begin_device()
            m.advance_device_step(self.batch)  # (host counts only: no device work)
            if self.record:
                for sid in self.ids:
                    self._note(("append_tokens", sid, 1))
                self._note(("fill_cuda_graph_metadata", self.batch, list(self.ids)))
            return
        with torch.cuda.stream(self.stream):
            for sid in self.ids:
                m.append_tokens(sid, 1)
                self._note(("append_tokens", sid, 1))
            m.fill_cuda_graph_metadata(self.batch, self.ids)
            self._note(("fill_cuda_graph_metadata", self.batch, list(self.ids)))
            self._plan()

    def _begin_device(self) -> None:
        self.mgr.begin_device_steps(self.batch, self.ids, steps=self.max_steps)

    def _plan(self) -> None:
        m = self.mgr
        self.wrapper.plan(m._cg_kv_indptr[self.batch], m._cg_kv_indices[self.batch],
                          m._cg_kv_last_page_len[self.batch], self.hq, self.hkv, self.d, self.ps,
                          pos_encoding_mode="NONE", q_data_type=self.dtype,
                          kv_shared_pages=m._cg_kv_shared[self.batch] if self.shared_hint else None,
                          cascade=self.cascade)

    def layers_fn(self) -> None:
        """Every layer's append of the step's token and its decode (what the graph holds); with
        device steps, first the page-table step and the plan."""
        m = self.mgr
        if self.device_steps:
            m.device_step(self.batch)
            self._plan()
        for layer in range(self.layers):
            if self.fused_append:
                self.wrapper.run(self.q[layer], m.kv_cache[layer], out=self.out[layer],
                                 append_kv=(self.k[layer], self.v[layer]))
            else:
                m.append_paged_kv_cache_cuda_graph(self.k[layer], self.v[layer], self.batch, layer)
                self.wrapper.run(self.q[layer], m.kv_cache[layer], out=self.out[layer])

    def replay(self) -> None:
        """Run the step's layers from the captured graph (captured on the first call, after
        an eager warm-up: a repeated append writes the same values to the same slots; with
        device steps there is no warm-up, since each run of the graph is a step)."""
        if self.graph is not None and self._on_stream:
            if self.mgr._table.data_ptr() != self._table_ptr:
                raise RuntimeError("the page table moved after the graph was captured")
            self.graph.replay()
            return
        with torch.cuda.stream(self.stream):
            if self.graph is None:
                if not self.device_steps:
                    self.layers_fn()
                self.stream.synchronize()
                self.graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(self.graph, stream=self.stream):
                    self.layers_fn()
                self._table_ptr = self.mgr._table.data_ptr()
            elif self.mgr._table.data_ptr() != self._table_ptr:
                raise RuntimeError("the page table moved after the graph was captured")
            self.graph.replay()

    def retire(self, write_tokens: bool = True) -> list:
        """Finish ``finish`` random sequences and start new ones in their batch rows: the
        pool's work of a batch change (frees, allocations on the prefix and, with device steps,
        handing the new batch to the device).  With ``write_tokens`` the new sequences' tokens
        are written too (the work of their prefill, not of the decode step); otherwise the
        caller writes them with ``write_tokens(new)`` before the next step.  Returns the rows
        and the new sequences."""
        with torch.cuda.stream(self.stream):
            rows = torch.randperm(self.batch, generator=self.gen)[: self.finish].tolist()
            new = []
            for r in sorted(rows):
                self.mgr.free(self.ids[r])
                self._note(("free", self.ids[r]))
                self.ids[r] = self._start_sequence(write=write_tokens)
                new.append(self.ids[r])
            if self.device_steps:  # the new batch goes back to the device
                self._begin_device()
        return rows, new

    def new_inputs(self) -> None:
        with torch.cuda.stream(self.stream):
            for t in (self.q, self.k, self.v):
                t.copy_(self._randn(t.shape))

    # ---------------------------------------------------------------- accounting
    def seq_lens(self) -> list:
        return [self.mgr._seq_len(s) for s in self.ids]

    def step_bytes(self, ahead: int = 0) -> dict:
        """Bytes one step's attention reads and writes per layer: ``unique`` counts every
        distinct valid token once (the shared prefix once), ``logical`` once per sequence.
        ``ahead``: the lengths after that many more steps (1 before a step: the step's own)."""
        es = torch.tensor([], dtype=self.dtype).element_size()
        tok = 2 * self.hkv * self.d * es
        lens = [L + ahead for L in self.seq_lens()]
        io = 2 * self.batch * self.hq * self.d * es + self.batch * tok  # q in, o out, appended K/V
        unique = (self.prefix_tokens + sum(L - self.prefix_tokens for L in lens)) * tok + io
        return {"unique": unique, "logical": sum(lens) * tok + io}
