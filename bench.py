"""Paged-KV hot-path benchmark on one MI355X.

Workload (default): one attention layer at Qwen2.5-3B shape (16 q / 2 kv heads, head_dim 128,
fp16), batch 64, contexts U[512, 4096], page_size 16, pages scattered by a seeded permutation
over a pool 1.25x the pages used, values N(0,1)*0.5.  A step is one pass of the hot path over
that batch: append one token per sequence into its page, then paged decode attention (one
launch: the decode kernel writes each token as it attends its page).

Steps rotate over --layers independent layer pools (4 x ~200 MB) so every step streams its
pages from HBM rather than from the 256 MB Infinity Cache.  Each layer's step is captured once
in a hipGraph and replayed, so host launch overhead does not gap the GPU.

Printed JSON line:
  value           decode GB/s = algorithmic bytes per decode launch / average decode launch
                  time (HIP events on the launch stream around back-to-back graph-replayed
                  decode launches; the median of 5 samples, each after a warm-up burst)
  roofline        the decode kernel against MI355X's 8 TB/s HBM peak
  append_mtok_s   appended tokens per second of the append kernel (nnz = batch)
  decode_append_fused_us  the decode launch with the step's append fused in (run(append_kv=):
                  one launch where the reference's step makes two)
  cpu_baseline    the reference's CPU path (gather pages, then torch SDPA, in fp32) on this
                  host's cores, on the same batch
  ms_per_step     append + decode per step (one launch, the append fused in), over exactly
                  --steps timed steps
  extras          the other hot-path workloads, each at its own default size, summarised (its
                  metric, value, roofline fraction, the times behind them, its CPU baseline):
                  chunked prefill, long-context decode, the 36-layer shared-prefix step and the
                  bulk append; --no-extras leaves them out, --workload <name> prints one in full

roofline.traffic is the decode kernel's HBM bytes per launch measured with hardware counters
(rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE, over `bench.py --profile-launches N`, each
scaled by the same counter's reading for a plain copy of known size run in the same
process); it is read from profiles/decode_traffic.json, where those runs were recorded, and is
reported only when that record was taken on this workload and on these exact decode kernel
sources (a SHA-256 over them), null otherwise.  The long-context decode, the 36-layer step and
the bulk append read their own records (profiles/*_traffic.json) the same way.  A record is
written from the two counter runs' CSV files by
`bench.py --workload W --traffic-record FETCH.csv WRITE.csv PROFILE.log`, PROFILE.log being
the output of the counter run (its profile_launches line).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time

HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "decode_traffic.json")


def decode_bytes(wb) -> int:
    es = wb.cache.element_size()
    B = wb.batch
    npages = int(wb.indptr[-1])
    return (sum(wb.kv_len) * 2 * wb.hkv * wb.d * es + 2 * B * wb.hq * wb.d * es
            + 4 * (2 * B + 1 + npages))


def append_bytes(wb) -> int:
    es = wb.cache.element_size()
    nnz = wb.k_new.shape[0]
    return nnz * (4 * wb.hkv * wb.d * es + 12)


DECODE_SOURCES = ("decode.hip", "decode_mfma.hip", "decode_plan.hip", "decode_sched.h", "decode_tile.h",
                  "attn_common.h", "mfma_common.h", "common.h")
APPEND_SOURCES = ("append.hip", "common.h")
APPEND_TRAFFIC_FILE = os.path.join(os.path.dirname(TRAFFIC_FILE), "append_traffic.json")
LONG_TRAFFIC_FILE = os.path.join(os.path.dirname(TRAFFIC_FILE), "decode_traffic_llama31_8b.json")
STEP36_TRAFFIC_FILE = os.path.join(os.path.dirname(TRAFFIC_FILE), "step36_traffic.json")
# per workload: (record file, kernel whose dispatches are counted, its sources, workload text)
TRAFFIC_RECORDS = {
    "qwen25_3b_b64": (TRAFFIC_FILE, "decode_mfma_kernel", DECODE_SOURCES,
                      "qwen2.5-3b paged decode, 1 layer, B=64, fp16 (bench.py default)"),
    "llama31_8b_b128": (LONG_TRAFFIC_FILE, "decode_mfma_kernel", DECODE_SOURCES,
                        "llama-3.1-8b long-context paged decode, 1 layer, B=128, bf16"),
    "qwen25_3b_step36": (STEP36_TRAFFIC_FILE, "decode_mfma_kernel", DECODE_SOURCES,
                         "qwen2.5-3b 36-layer decode step, B=128, 2048-token shared prefix, fp16: each "
                         "layer's decode launch (the step's append fused in)"),
    "qwen25_3b_bulk_append": (APPEND_TRAFFIC_FILE, "append_wave_kernel", APPEND_SOURCES,
                              "append_paged_kv_cache, 128 requests x 512 tokens (nnz 65536), fp16"),
}


def source_hash(names=DECODE_SOURCES) -> str:
    """SHA-256 over a kernel's sources (for the decode: the kernel, its schedule and the shared
    headers), so a counter record is only used for the code it was taken on."""
    import hashlib
    h = hashlib.sha256()
    root = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ecahlang_amd", "csrc")
    for name in names:
        with open(os.path.join(root, name), "rb") as f:
            h.update(name.encode() + b"\0" + f.read())
    return h.hexdigest()


def _traffic_record(path):
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return {}


def measured_traffic(wb, w):
    """HBM bytes per decode launch from the committed counter runs, when they were taken on
    this workload, this workgroup count and these decode sources (None otherwise)."""
    return recorded_traffic("qwen25_3b_b64", decode_bytes(wb), key={"decode_ctas": w._ctas})


def measured_append_traffic(wb):
    """HBM bytes per append launch from the committed counter runs (rocprofv3 FETCH_SIZE and
    WRITE_SIZE over `--workload qwen25_3b_bulk_append --profile-launches N`, scaled by a copy
    of the same byte count), when taken on this token batch and these append sources."""
    return recorded_traffic("qwen25_3b_bulk_append", append_bytes(wb))


def record_traffic(workload, fetch_csv, write_csv, profile_log):
    """Write a workload's traffic record from its two counter runs: the kernel's FETCH_SIZE and
    WRITE_SIZE (KiB per dispatch, averaged over the run's last `kernel_dispatches` dispatches of
    it, the profiled launches), each scaled by the same counter's reading for the plain copies
    of `copy_bytes` the run made after them (true bytes / reading).  Returns the record."""
    import csv
    path, kernel, sources, text = TRAFFIC_RECORDS[workload]

    with open(profile_log) as f:
        prof = [json.loads(ln) for ln in f if ln.startswith('{"profile_launches"')][-1]

    def readings(fn, counter):
        kern, copy = [], []
        with open(fn) as f:
            for r in csv.DictReader(f):
                if r["Counter_Name"] != counter:
                    continue
                if kernel in r["Kernel_Name"]:
                    kern.append((int(r["Dispatch_Id"]), float(r["Counter_Value"])))
                elif "copyBuffer" in r["Kernel_Name"]:
                    copy.append(float(r["Counter_Value"]))
        kern = [v for _, v in sorted(kern)][-prof["kernel_dispatches"]:]
        return kern, copy

    copy_kib = prof["copy_bytes"] / 1024
    fk, fc = readings(fetch_csv, "FETCH_SIZE")
    wk, wc = readings(write_csv, "WRITE_SIZE")
    fc = [v for v in fc if v > 0.4 * copy_kib]  # (the calibration copies, not small ones)
    wc = [v for v in wc if v > 0.4 * copy_kib]
    if not (fk and wk and fc and wc):
        raise SystemExit(f"no {kernel} or calibration-copy dispatches in the counter files")
    fs, ws = copy_kib / statistics.mean(fc), copy_kib / statistics.mean(wc)
    traffic = round((statistics.mean(fk) * fs + statistics.mean(wk) * ws) * 1024)
    algo = prof["algorithmic_bytes"]
    rec = {"kernel": kernel, "workload": text, "algorithmic_bytes": algo,
           "fetch_kib_per_dispatch": round(statistics.mean(fk), 1),
           "write_kib_per_dispatch": round(statistics.mean(wk), 1), "dispatches": len(fk),
           "copy_bytes": prof["copy_bytes"], "copy_fetch_kib_per_dispatch": round(statistics.mean(fc), 1),
           "copy_write_kib_per_dispatch": round(statistics.mean(wc), 1),
           "fetch_scale": round(fs, 5), "write_scale": round(ws, 5), "traffic_bytes": traffic,
           "traffic_over_algorithmic": round(traffic / algo, 4),
           "source_sha256": source_hash(sources)}
    for k in ("key", "logical_bytes"):
        if k in prof:
            rec[k] = prof[k]
    if "logical_bytes" in prof:
        rec["traffic_over_logical"] = round(traffic / prof["logical_bytes"], 4)
    with open(path, "w") as f:
        json.dump(rec, f, indent=1)
        f.write("\n")
    return rec


def recorded_traffic(workload, algorithmic_bytes=None, key=None):
    """HBM bytes per launch from a workload's traffic record, when it was taken on these
    kernel sources and on this workload (its algorithmic bytes or its key); None otherwise."""
    path, _, sources, _ = TRAFFIC_RECORDS[workload]
    t = _traffic_record(path)
    if t.get("source_sha256") != source_hash(sources):
        return None
    if algorithmic_bytes is not None and t.get("algorithmic_bytes") != algorithmic_bytes:
        return None
    if key is not None and t.get("key") != key:
        return None
    return t.get("traffic_bytes")


def graph_time(torch, stream, graph, reps, launches, samples=5):
    """Seconds per launch of a captured graph of `launches` launches: HIP events around `reps`
    back-to-back replays on `stream`, the median of `samples` samples.  Each sample follows a
    burst of 3 untimed replays with no synchronisation in between: the first milliseconds
    after the GPU has idled run ~10 % slow, and a sample taken then is not the kernel's rate."""
    times = []
    for _ in range(samples):
        with torch.cuda.stream(stream):
            for _ in range(3):
                graph.replay()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(reps):
                graph.replay()
            e1.record(stream)
        e1.synchronize()
        times.append(e0.elapsed_time(e1) / 1e3 / (reps * launches))
    return statistics.median(times)


def read_probe(torch, dev, stream, nbytes, nbuf, blocks, per_buf=8):
    """Seconds per launch of the library's streaming-read probe (pkv_probe_stream_read) over
    nbytes with `blocks` workgroups, `nbuf` buffers read in turn (more than the 256 MB MALL
    holds, as the decode's rotated pools are), timed like the kernels: a captured graph of
    per_buf x nbuf launches replayed back to back."""
    from ecahlang_amd._lib import check, lib, stream_ptr
    nb = -(-nbytes // 16) * 16
    bufs = [torch.empty(nb, dtype=torch.uint8, device=dev) for _ in range(nbuf)]
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        def launch(b):
            check(lib().pkv_probe_stream_read(b.data_ptr(), nb, blocks, sink.data_ptr(), stream_ptr(dev)),
                  "read probe")
        for b in bufs:
            launch(b)
        with torch.cuda.graph(graph, stream=stream):
            for _ in range(per_buf):
                for b in bufs:
                    launch(b)
    t = graph_time(torch, stream, graph, 3, per_buf * nbuf)
    del graph, bufs
    return t


def long_context(args, torch, workloads, Wrapper, dev):
    """Decode-only timing of the long-context workload (K/V far beyond the 256 MB MALL, so
    no pool rotation is needed); the CPU baseline runs on a bounded sample of sequences."""
    import numpy as np
    print("bench: building Llama-3.1-8B B=128 long-context batch on the device", file=sys.stderr, flush=True)
    wb = workloads.llama31_8b_decode_device(dev)
    es = wb.cache.element_size()
    npages = int(wb.indptr[-1])
    dbytes = (sum(wb.kv_len) * 2 * wb.hkv * wb.d * es + 2 * wb.batch * wb.hq * wb.d * es
              + 4 * (2 * wb.batch + 1 + npages))
    w = Wrapper(torch.empty(256 << 20, dtype=torch.uint8, device=dev), "NHD")
    w.plan(wb.indptr, wb.indices, wb.last, wb.hq, wb.hkv, wb.d, wb.ps, q_data_type=wb.dtype,
           num_ctas=args.ctas, deterministic=not args.dynamic)
    out = torch.empty_like(wb.q)
    if args.profile_launches:  # counter runs: eager launches, then copies of the same byte count
        for _ in range(args.profile_launches):
            w.run(wb.q, wb.cache, out=out)
        nb = dbytes // 16 * 16
        src = torch.empty(nb // 4, dtype=torch.int32, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(args.profile_launches):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"profile_launches": args.profile_launches, "kernel_dispatches": args.profile_launches,
                          "algorithmic_bytes": dbytes, "copy_bytes": nb, "key": {"decode_ctas": w._ctas}}),
              flush=True)
        return None
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        w.run(wb.q, wb.cache, out=out)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        REP = 10
        with torch.cuda.graph(g, stream=stream):
            for _ in range(REP):
                w.run(wb.q, wb.cache, out=out)
        for _ in range(max(1, args.warmup // REP)):
            g.replay()
    t = graph_time(torch, stream, g, max(1, args.steps // REP), REP)
    gbs = dbytes / t / 1e9
    # CPU baseline on a bounded sample: the reference's gather + fp32 SDPA for 4 sequences
    import torch.nn.functional as F
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    lens = np.array(wb.kv_len)
    sample = [int(i) for i in np.argsort(lens)[len(lens) // 2: len(lens) // 2 + 4]]
    ks, vs, qs = [], [], []
    ip = wb.indptr.cpu().numpy()
    for b in sample:
        pages = wb.indices[ip[b]:ip[b + 1]].long()
        L = int(lens[b])
        ks.append(wb.cache[pages, 0].reshape(-1, wb.hkv, wb.d)[:L].cpu())
        vs.append(wb.cache[pages, 1].reshape(-1, wb.hkv, wb.d)[:L].cpu())
        qs.append(wb.q[b].cpu())
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        for k, v, q in zip(ks, vs, qs):
            kk = k.float().transpose(0, 1)[None]
            vv = v.float().transpose(0, 1)[None]
            F.scaled_dot_product_attention(q.float()[None, :, None, :], kk, vv, enable_gqa=True)
        times.append(time.perf_counter() - t0)
    sample_bytes = sum(int(lens[b]) for b in sample) * 2 * wb.hkv * wb.d * es
    result = {
        "metric": "paged decode attn GB/s (% HBM peak), long-context Llama-3.1-8B B=128",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "higher_is_better": True,
        "dtype": "bf16", "data": "synthetic (device-generated N(0,1) K/V/Q, random page permutation, NaN-poisoned pool)",
        "config": {"workload": "llama-3.1-8b long-context paged decode, 1 layer, B=128, ctx logU[1024,32768], "
                               "page 16, 32 q / 8 kv heads, head_dim 128, bf16, pool ~20 GB",
                   "batch": wb.batch, "kv_tokens": sum(wb.kv_len), "pages": npages, "pool_pages": wb.num_pages,
                   "decode_ctas": w._ctas, "decode_kernel": "mfma" if w._mfma else "valu"},
        "decode_us": round(t * 1e6, 3), "decode_bytes": dbytes,
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": recorded_traffic("llama31_8b_b128", dbytes, key={"decode_ctas": w._ctas})},
        "cpu_baseline": {"value": round(sample_bytes / statistics.median(times) / 1e9, 3), "unit": "GB/s",
                         "cores": cores, "kind": "port",
                         "sample": f"4 median-length sequences ({sum(int(lens[b]) for b in sample)} tokens): "
                                   "gather + fp32 SDPA, median of 3", "cpu_model": cpu_model()},
    }
    return result


MFMA_PEAK_TFLOPS = 2500.0  # dense fp16/bf16


def sampling(args, torch, dev):
    """Top-k / top-p sampling of one decode step's logits at Qwen2.5-3B's vocabulary: B = 128
    rows of 151,936 fp16 logits, top_k 50, top_p 0.9, the default device generator.  Bytes per
    call: the logits once plus the tokens out (the kernel's further passes over a row hit the
    caches)."""
    from ecahlang_amd.sampling import top_k_top_p_sampling_from_logits as sample
    B, V = 128, 151936
    g = torch.Generator().manual_seed(1006)
    x = (torch.randn(B, V, generator=g) * 3).half().to(dev)
    k = torch.full((B,), 50, dtype=torch.int32, device=dev)
    p = torch.full((B,), 0.9, dtype=torch.float32, device=dev)
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        sample(x, k, p)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        REP = 10
        with torch.cuda.graph(gr, stream=stream):
            for _ in range(REP):
                sample(x, k, p)
    t = graph_time(torch, stream, gr, max(1, args.steps // REP), REP)
    nbytes = B * V * 2 + B * 4
    gbs = nbytes / t / 1e9

    def timed(fn):
        with torch.cuda.stream(stream):
            fn()
            torch.cuda.synchronize()
            g2 = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g2, stream=stream):
                for _ in range(REP):
                    fn()
        return graph_time(torch, stream, g2, max(1, args.steps // REP), REP)

    # the reference's default request (top_k 0 -> whole vocabulary, top_p 1): plain multinomial
    t_default = timed(lambda: sample(x, 0, 1.0))
    # with the serving loop's scaling (main.py:483-487): repetition-penalty rows and temperature,
    # fused into the sampler against the eager `logits / mask_penalty[rows] / temperature`
    table = torch.ones(B, V, dtype=torch.float16, device=dev)
    table[:, ::97] = 1.0 / 1.1
    prow = torch.arange(B, dtype=torch.int32, device=dev)
    temp = torch.full((B,), 0.7, dtype=torch.float32, device=dev)
    t_fused = timed(lambda: sample(x, k, p, penalty=table, penalty_rows=prow, temperature=temp))
    t_eager = timed(lambda: sample(x / table[prow.long()] / temp.reshape(-1, 1), k, p))
    from ecahlang_amd.sampling import scale_logits
    t_scale = timed(lambda: scale_logits(x, table, prow, temp))
    # CPU baseline: torch's sort-based top-k / top-p sampling on this host, 8 rows
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    xc = x[:8].float().cpu()

    def cpu_sample(l):
        probs = torch.softmax(l, -1)
        vals, idx = probs.topk(50, dim=-1)
        vals = vals / vals.sum(-1, keepdim=True)
        c = vals.cumsum(-1)
        vals = torch.where(c - vals >= 0.9, torch.zeros_like(vals), vals)
        return idx.gather(-1, torch.multinomial(vals, 1))

    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        cpu_sample(xc)
        times.append(time.perf_counter() - t0)
    result = {
        "metric": "top-k/top-p sampling GB/s of logits (% HBM peak), Qwen2.5-3B vocabulary, B=128",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "higher_is_better": True, "dtype": "fp16",
        "data": "synthetic (seeded N(0,1)*3 logits)",
        "config": {"workload": "top_k_top_p_sampling_from_logits, 128 x 151936 fp16 logits, top_k 50, top_p 0.9",
                   "rows": B, "vocab": V},
        "sampling_us": round(t * 1e6, 3), "bytes": nbytes,
        "default_params_us": round(t_default * 1e6, 3),
        "scaled_fused_us": round(t_fused * 1e6, 3), "scaled_eager_us": round(t_eager * 1e6, 3),
        "scale_logits_us": round(t_scale * 1e6, 3),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None},
        "cpu_baseline": {"value": round(8 * V * 2 / statistics.median(times) / 1e9, 3), "unit": "GB/s",
                         "cores": cores, "kind": "port",
                         "sample": "8 rows: torch softmax + topk + cumsum nucleus + multinomial, median of 3",
                         "cpu_model": cpu_model()},
    }
    return result


def rope_bytes(hq, hkv, d, es) -> int:
    """Algorithmic bytes per token of the fused rotation + append: q read and written, k and v
    read and written into their pages, the token's cos and sin rows, batch index and position."""
    return 2 * es * d * (hq + 2 * hkv) + 2 * es * d + 8


def rope_append(args, torch, workloads, ops, dev):
    """The model's rotary embedding on the new tokens fused with the append, at Qwen2.5-3B
    shape (16 q / 2 kv heads, head_dim 128, fp16): the chunked-prefill batch (8 requests x
    512-token chunks, 4096 tokens) and the B = 64 decode step.  Compared with the unfused
    sequence the model and hook run today: transformers' apply_rotary_pos_emb, then the append."""
    import numpy as np
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb
    from oracle import kv_ref, rope_ref

    def cos_sin(positions, d):
        # the model's position embeddings: theta 1e6, fp32 angles, cast to the activations' dtype
        inv = 1.0 / (1000000.0 ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
        ang = positions.float().cpu()[:, None] * inv[None]
        emb = torch.cat((ang, ang), -1)
        return emb.cos().half(), emb.sin().half()

    stream = torch.cuda.Stream(device=dev)
    REP = 10

    def timed(fn):
        with torch.cuda.stream(stream):
            fn()
            torch.cuda.synchronize()
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr, stream=stream):
                for _ in range(REP):
                    fn()
        return graph_time(torch, stream, gr, max(1, args.steps // REP), REP)

    res = {}
    for name, wb in (("prefill", workloads.qwen25_3b_prefill()), ("decode", workloads.qwen25_3b_decode())):
        print(f"bench: rope + append, {name} batch", file=sys.stderr, flush=True)
        dv = wb.to(dev)
        cos, sin = cos_sin(wb.positions, wb.d)
        cd, sd = cos.to(dev), sin.to(dev)
        q_out = torch.empty_like(dv.q)

        def fused():
            ops.append_paged_kv_cache_with_rope(dv.q, dv.k_new, dv.v_new, cd, sd, dv.batch_indices,
                                                dv.positions, dv.cache, dv.indices, dv.indptr, dv.last,
                                                q_out=q_out)

        def unfused():
            qe, ke = apply_rotary_pos_emb(dv.q.transpose(0, 1)[None], dv.k_new.transpose(0, 1)[None],
                                          cd[None], sd[None])
            ops.append_paged_kv_cache(ke[0].transpose(0, 1), dv.v_new, dv.batch_indices, dv.positions,
                                      dv.cache, dv.indices, dv.indptr, dv.last)
            return qe

        if not args.no_check:  # both sequences leave identical bits
            fused()
            c1, q1 = dv.cache.clone(), q_out.clone()
            q2 = unfused()[0].transpose(0, 1)
            torch.cuda.synchronize()
            if not (torch.equal(c1.view(torch.int16), dv.cache.view(torch.int16))
                    and torch.equal(q1.view(torch.int16), q2.contiguous().view(torch.int16))):
                raise SystemExit("rope + append: fused and unfused results differ")
        tf, tu = timed(fused), timed(unfused)
        nnz = dv.q.shape[0]
        nbytes = nnz * rope_bytes(wb.hq, wb.hkv, wb.d, 2)
        res[name] = dict(tokens=nnz, fused_us=round(tf * 1e6, 3), unfused_us=round(tu * 1e6, 3),
                         bytes=nbytes, gbs=round(nbytes / tf / 1e9, 2))
        del dv
    # CPU baseline: the oracle (per-op rounded numpy rotation + scatter) on one 512-token chunk
    sb = workloads.build_batch([512], [512], 16, 2, 128, torch.float16, seed=3, fill_old=False)
    c, s = cos_sin(sb.positions, 128)
    iv = lambda t: t.view(torch.int16).numpy()
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        cb, sbits = iv(c)[:, None], iv(s)[:, None]
        rope_ref.rotate(iv(sb.q).view(np.uint16), cb.view(np.uint16), sbits.view(np.uint16), "float16")
        k_rot = rope_ref.rotate(iv(sb.k_new).view(np.uint16), cb.view(np.uint16), sbits.view(np.uint16), "float16")
        kv_ref.append(iv(sb.cache), k_rot.view(np.int16), iv(sb.v_new), sb.batch_indices.numpy(),
                      sb.positions.numpy(), sb.indices.numpy(), sb.indptr.numpy(), 16)
        times.append(time.perf_counter() - t0)
    cpu_gbs = 512 * rope_bytes(16, 2, 128, 2) / statistics.median(times) / 1e9
    p = res["prefill"]
    result = {
        "metric": "fused rotary embedding + paged K/V append GB/s (% HBM peak), Qwen2.5-3B, 4096-token chunked prefill",
        "value": p["gbs"], "unit": "GB/s", "n_gpus": 1, "higher_is_better": True, "dtype": "fp16",
        "data": "synthetic (seeded N(0,1)*0.5 activations, the model's cos/sin at the tokens' positions)",
        "config": {"workload": "append_paged_kv_cache_with_rope, 8 requests x 512-token chunks onto prefixes "
                               "U[0, 8192], Hq 16, Hkv 2, D 128, page 16; and the B=64 decode step",
                   "bytes_per_token": rope_bytes(16, 2, 128, 2)},
        "prefill": p, "decode": res["decode"],
        "speedup_vs_unfused": {k: round(v["unfused_us"] / v["fused_us"], 2) for k, v in res.items()},
        "roofline": {"bound": "hbm", "achieved": p["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(p["gbs"] / HBM_PEAK_GBS, 4), "traffic": None},
        "cpu_baseline": {"value": round(cpu_gbs, 3), "unit": "GB/s", "cores": 1, "kind": "port",
                         "sample": "one 512-token chunk: oracle rotation of q and k, then the oracle append "
                                   "(which also copies its 40-page pool), median of 3",
                         "cpu_model": cpu_model()},
    }
    return result


def bulk_append(args, torch, workloads, ops, dev):
    """append_paged_kv_cache (the reference's append, ecahlang/manager.py:153-185) of large
    token batches at Qwen2.5-3B shape (2 KV heads, head_dim 128, fp16): 8 requests x 512
    tokens (nnz 4096) and 128 requests x 512 tokens (nnz 65536), each onto a prefix of
    U[0, 4096] tokens, pages scattered over the pool.  Bytes per token: K and V rows read and
    written (4 * Hkv * D * 2) plus the token's batch index and position and its page-table
    entry (12)."""
    import numpy as np
    from oracle import kv_ref
    stream = torch.cuda.Stream(device=dev)
    res = {}
    for requests in (8, 128):
        g = torch.Generator().manual_seed(4000 + requests)
        prefix = torch.randint(0, 4097, (requests,), generator=g).tolist()
        wb = workloads.build_batch([p + 512 for p in prefix], [512] * requests, 16, 2, 128, torch.float16,
                                   seed=4100 + requests, fill_old=False)
        nnz = wb.k_new.shape[0]
        if requests == 128:
            host_big = wb
        print(f"bench: bulk append, nnz {nnz}", file=sys.stderr, flush=True)
        dv = wb.to(dev)

        def app():
            ops.append_paged_kv_cache(dv.k_new, dv.v_new, dv.batch_indices, dv.positions, dv.cache,
                                      dv.indices, dv.indptr, dv.last)

        before = None if args.no_check or requests == 8 else dv.cache.clone()
        with torch.cuda.stream(stream):
            app()
        torch.cuda.synchronize()
        ok = None
        if not args.no_check and requests == 8:  # bit-exact against the oracle on the whole pool
            iv = lambda t: t.view(torch.int16).cpu().numpy()
            want = kv_ref.append(iv(wb.cache), iv(wb.k_new), iv(wb.v_new), wb.batch_indices.numpy(),
                                 wb.positions.numpy(), wb.indices.numpy(), wb.indptr.numpy(), 16)
            ok = bool(np.array_equal(iv(dv.cache), want))
        elif before is not None:
            # bit-exact on the whole pool at full size: the pool before the launch with every
            # token's K and V rows written at its page and slot by torch's index_put
            ps = dv.cache.shape[2]
            pos, bi = dv.positions.long(), dv.batch_indices.long()
            page = dv.indices.long()[dv.indptr.long()[bi] + pos // ps]
            slot = pos % ps
            before[page, 0, slot] = dv.k_new
            before[page, 1, slot] = dv.v_new
            ok = bool(torch.equal(before.view(torch.int16), dv.cache.view(torch.int16)))
            del before
        if args.profile_launches and requests == 128:
            for _ in range(args.profile_launches):
                app()
            nb = append_bytes(wb) // 16 * 16
            src = torch.empty(nb // 4, dtype=torch.int32, device=dev).fill_(1)
            dst = torch.empty_like(src)
            for _ in range(args.profile_launches):
                dst.copy_(src)
            torch.cuda.synchronize()
            print(json.dumps({"profile_launches": args.profile_launches,
                              "kernel_dispatches": args.profile_launches, "algorithmic_bytes": append_bytes(wb),
                              "copy_bytes": nb}), flush=True)
            return None
        REP = 10
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            with torch.cuda.graph(gr, stream=stream):
                for _ in range(REP):
                    app()
        t = graph_time(torch, stream, gr, max(2, args.steps // (REP * 10)), REP)
        nbytes = append_bytes(wb)
        if requests == 128:
            traffic = measured_append_traffic(wb)
        res[nnz] = dict(requests=requests, tokens=nnz, us=round(t * 1e6, 3), bytes=nbytes,
                        gbs=round(nbytes / t / 1e9, 2), frac=round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4),
                        parity_bitexact=ok)
        del dv
    big = res[max(res)]
    # CPU baseline: the same 65,536-token append on the host cores with torch's index_put (the
    # page and slot of each token from the page table, then one scatter of the K rows and one of
    # the V rows into the pool), median of 3
    ncores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    prev_threads = torch.get_num_threads()
    torch.set_num_threads(ncores)
    cpool = host_big.cache.clone()
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        pos, bi = host_big.positions.long(), host_big.batch_indices.long()
        page = host_big.indices.long()[host_big.indptr.long()[bi] + pos // 16]
        slot = pos % 16
        cpool[page, 0, slot] = host_big.k_new
        cpool[page, 1, slot] = host_big.v_new
        times.append(time.perf_counter() - t0)
    cores_used = torch.get_num_threads()
    torch.set_num_threads(prev_threads)
    del cpool
    result = {
        "metric": "paged K/V append GB/s (% HBM peak), Qwen2.5-3B, 65536 tokens",
        "value": big["gbs"], "unit": "GB/s", "n_gpus": 1, "higher_is_better": True, "dtype": "fp16",
        "data": "synthetic (seeded N(0,1) K/V rows, random page permutation, NaN-poisoned pool)",
        "config": {"workload": "append_paged_kv_cache, 128 requests x 512 tokens (and 8 x 512) onto prefixes "
                               "U[0, 4096], Hkv 2, D 128, page 16",
                   "bytes_per_token": 4 * 2 * 128 * 2 + 12},
        "by_nnz": {str(k): v for k, v in sorted(res.items())},
        "roofline": {"bound": "hbm", "achieved": big["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": big["frac"], "traffic": traffic},
        "cpu_baseline": {"value": round(append_bytes(host_big) / statistics.median(times) / 1e9, 3), "unit": "GB/s",
                         "cores": cores_used, "kind": "port",
                         "sample": "the 65,536-token append itself: torch index_put of the K and V rows on the host "
                                   "cores, median of 3",
                         "cpu_model": cpu_model()},
    }
    return result


def step36(args, torch, workloads, dev):
    """The 36-layer decode step at Qwen2.5-3B attention shape, batch 128, on a shared
    2048-token prefix (workloads.SharedPrefixDecodeLoop): per step, the page-table step
    (append_tokens for every sequence, fill_cuda_graph_metadata), the plan, and 36 decodes, each
    with the layer's append of the step's token fused in (the reference's step makes each append
    a launch of its own).  By default the whole step is one graph replay and the host's part is
    advance_device_step (AutoKVCacheManager.begin_device_steps); with --host-steps the
    bookkeeping runs on the host per step, as the reference's loop does, and the graph holds
    the layers only.  The timed region of each step runs from before the host's part to the
    end of the batch change that follows the replay: 8 sequences retired and 8 new ones
    allocated on the prefix, and with device steps the new batch handed back to the device
    (begin_device_steps); writing the new sequences' tokens (the work of their prefill) follows
    the timed region.  batch_change_ms is that batch change alone.  graph_ms times the replay
    alone on alternate steps (their host part done before the first event, their batch change
    after the last); graph_back_to_back_ms replays the graph with the host enqueueing ahead."""
    import numpy as np
    steps, warmup = max(1, min(args.steps, 40)), max(1, min(args.warmup, 4))
    print("bench: building the 36-layer shared-prefix decode loop (B=128)", file=sys.stderr, flush=True)
    device_steps = not args.host_steps
    cascade = not args.no_cascade
    n_prof = args.profile_launches
    loop = workloads.SharedPrefixDecodeLoop(dev, max_steps=(n_prof or 2 * steps) + warmup + 2,
                                            device_steps=device_steps, cascade=cascade)
    for _ in range(warmup):
        loop.begin_step()
        loop.replay()
        loop.retire()
    torch.cuda.synchronize()
    step_key = {"layers": loop.layers, "batch": loop.batch, "prefix_tokens": loop.prefix_tokens,
                "device_steps": device_steps, "cascade": cascade}
    if n_prof:  # counter runs: n steps (36 decode launches each), then copies of a layer's unique bytes
        ub, lb = [], []
        for _ in range(n_prof):
            b = loop.step_bytes(ahead=1)
            ub.append(b["unique"])
            lb.append(b["logical"])
            loop.begin_step()
            loop.replay()
            loop.retire()
        unique, logical = int(np.mean(ub)), int(np.mean(lb))
        nb = unique // 16 * 16
        src = torch.empty(nb // 4, dtype=torch.int32, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(n_prof):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"profile_launches": n_prof, "kernel_dispatches": n_prof * loop.layers,
                          "algorithmic_bytes": unique, "logical_bytes": logical, "copy_bytes": nb,
                          "key": step_key}), flush=True)
        return None
    # a cyclic-garbage pass of the interpreter over everything torch has loaded can stall one
    # step's host bookkeeping by tens of ms; collect once and freeze the survivors first
    import gc
    gc.collect()
    gc.freeze()
    # Steps alternate between the timed step (host part, then replay) and the same kind of
    # step with the host part done before the first event (the replay alone: graph_ms), so the
    # two figures are taken on the same mix of batch states; each starts on an idle GPU.
    times, gtimes, rtimes, byts, gbyts = [], [], [], [], []
    with loop.on_stream():
        for i in range(2 * steps):
            full = i % 2 == 0
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e2 = torch.cuda.Event(enable_timing=True)
            if not full:
                loop.begin_step()
            else:
                sb = loop.step_bytes(ahead=1)  # (the lengths this step attends)
            loop.stream.synchronize()
            e0.record(loop.stream)
            if full:
                loop.begin_step()
            loop.replay()
            e1.record(loop.stream)
            if full:  # the batch change: 8 sequences freed, 8 allocated on the prefix, the new
                # batch handed to the device (their tokens, the prefill's work, come after)
                _, new = loop.retire(write_tokens=False)
                e2.record(loop.stream)
                e2.synchronize()
                times.append(e0.elapsed_time(e2) / 1e3)
                rtimes.append(e1.elapsed_time(e2) / 1e3)
                byts.append(sb)
                loop.write_tokens(new)
            else:
                e1.synchronize()
                gtimes.append(e0.elapsed_time(e1) / 1e3)
                gbyts.append(loop.step_bytes())
                loop.retire()
    # parity on the last step's layers 0 and 35, 8 sequences each, before the next step
    par = None
    if not args.no_check:
        loop.begin_step()
        loop.replay()
        torch.cuda.synchronize()
        par = step36_parity(loop, [0, loop.layers - 1], 8)
    # the graph replayed back to back, the host enqueueing ahead (each replay repeats the same
    # appends; with device steps each replay is one more step, whose pages the pool has room
    # for: nothing reads the loop's state after this)
    t_b2b = graph_time(torch, loop.stream, loop.graph, 4, 1)
    L = loop.layers
    t_step, t_graph = float(np.mean(times)), float(np.mean(gtimes))
    uniq = float(np.mean([b["unique"] for b in byts])) * L
    logical = float(np.mean([b["logical"] for b in byts])) * L
    gbs = uniq / t_step / 1e9
    gbs_graph = float(np.mean([b["unique"] for b in gbyts])) * L / t_graph / 1e9
    # CPU baseline: the reference's path (gather + fp32 SDPA per sequence, index_put append)
    # for one layer of 4 sequences
    import torch.nn.functional as F
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    cache0 = loop.mgr.kv_cache[0]
    m = loop.mgr
    sample = loop.ids[:4]
    ks, vs, qs = [], [], []
    for r, sid in enumerate(sample):
        n, _ = m._counts(sid)
        pages = m._table[m.batch_to_seq_len[sid], :n].long()
        Ls = m._seq_len(sid)
        ks.append(cache0[pages, 0].reshape(-1, loop.hkv, loop.d)[:Ls].cpu())
        vs.append(cache0[pages, 1].reshape(-1, loop.hkv, loop.d)[:Ls].cpu())
        qs.append(loop.q[0, r].cpu())
    ctimes = []
    for _ in range(3):
        t0 = time.perf_counter()
        for k, v, q in zip(ks, vs, qs):
            F.scaled_dot_product_attention(q.float()[None, :, None, :], k.float().transpose(0, 1)[None],
                                           v.float().transpose(0, 1)[None], enable_gqa=True)
        ctimes.append(time.perf_counter() - t0)
    sample_bytes = sum(k.numel() * 2 * 2 for k in ks)
    per_launch = recorded_traffic("qwen25_3b_step36", key=step_key)
    step_traffic = None if per_launch is None else per_launch * L
    result = {
        "metric": "36-layer decode step (attention path), unique KV GB/s (% HBM peak), Qwen2.5-3B B=128 shared prefix",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "higher_is_better": True,
        "dtype": "fp16", "data": "synthetic (device-generated N(0,1)*0.5, pages from the manager's pool, NaN-poisoned)",
        "config": {"workload": "qwen2.5-3b 36-layer decode step, B=128, 2048-token shared prefix + own suffix U[64,1024], "
                               + ("page-table step + plan + decode with the token's append fused in, per layer, "
                                  "in one graph (device steps)"
                                  if device_steps else "host page-table step + plan, graph-captured decode with the "
                                  "token's append fused in, per layer")
                               + ", 8 sequences retired per step",
                   "layers": L, "batch": loop.batch, "steps": steps, "warmup": warmup,
                   "pool_pages": loop.mgr.max_blocks, "device_steps": device_steps},
        "step_ms": round(t_step * 1e3, 4), "batch_change_ms": round(float(np.mean(rtimes)) * 1e3, 4),
        "graph_ms": round(t_graph * 1e3, 4),
        "graph_back_to_back_ms": round(t_b2b * 1e3, 4),
        "unique_bytes_per_step": int(uniq), "logical_bytes_per_step": int(logical),
        "graph_unique_gbs": round(gbs_graph, 2), "logical_gbs": round(logical / t_step / 1e9, 2),
        "parity": par,
        # (value and roofline share one denominator: the whole step; traffic is the HBM bytes of
        # the step's 36 decode launches from the counter record, which the record also states per
        # launch against a layer's unique and logical bytes)
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": step_traffic},
        "cpu_baseline": {"value": round(sample_bytes / statistics.median(ctimes) / 1e9, 3), "unit": "GB/s",
                         "cores": cores, "kind": "port",
                         "sample": f"layer 0, 4 sequences ({sum(k.shape[0] for k in ks)} tokens): gather + fp32 SDPA, median of 3",
                         "cpu_model": cpu_model()},
    }
    return result


def step36_parity(loop, layers, nseq):
    """The step's decode output of ``nseq`` sequences in each of ``layers`` against the
    oracle's attention over the same pages (read back), and the step's appended K/V in place."""
    import numpy as np
    import torch
    from oracle import kv_ref
    m = loop.mgr
    worst, ok = 0.0, True
    for layer in layers:
        cache = m.kv_cache[layer]
        for r in range(nseq):
            sid = loop.ids[r]
            n, _ = m._counts(sid)
            pages = m._table[m.batch_to_seq_len[sid], :n].long()
            L = m._seq_len(sid)
            kv = cache[pages].float().cpu().numpy()  # [n, 2, ps, hkv, d]
            k = kv[:, 0].reshape(-1, loop.hkv, loop.d)[:L]
            v = kv[:, 1].reshape(-1, loop.hkv, loop.d)[:L]
            # the appended token sits at position L - 1, bit for bit
            ok &= bool(torch.equal(cache[pages[(L - 1) // 16], 0, (L - 1) % 16].cpu(), loop.k[layer, r].cpu()))
            ok &= bool(torch.equal(cache[pages[(L - 1) // 16], 1, (L - 1) % 16].cpu(), loop.v[layer, r].cpu()))
            q = loop.q[layer, r:r + 1].float().cpu().numpy().astype(np.float64)
            ref = kv_ref._attend(q, k, v, [L], loop.d ** -0.5)[0]
            got = loop.out[layer, r].float().cpu().numpy()
            err = np.abs(got - ref)
            ok &= bool(np.all(err <= 2e-3 + 1e-2 * np.abs(ref)))
            worst = max(worst, float(err.max()))
    return {"max_abs_err": worst, "within_atol2e-3_rtol1e-2_and_append_bitexact": ok}


def chunked_prefill(args, torch, workloads, ops, dev):
    """Chunked prefill at Qwen2.5-3B shape: append each request's chunk, then causal ragged
    attention over prefix + chunk.  FLOPs count valid causal (query, key) pairs only:
    4 * Hq * D * sum_b (C * P_b + C (C + 1) / 2)."""
    import numpy as np
    from ecahlang_amd.wrappers import BatchPrefillWithPagedKVCacheWrapper
    print("bench: building Qwen2.5-3B chunked-prefill batch", file=sys.stderr, flush=True)
    wb = workloads.qwen25_3b_prefill()
    dv = wb.to(dev)
    ops.append_paged_kv_cache(dv.k_new, dv.v_new, dv.batch_indices, dv.positions, dv.cache, dv.indices,
                              dv.indptr, dv.last)
    w = BatchPrefillWithPagedKVCacheWrapper(torch.empty(128 << 20, dtype=torch.uint8, device=dev), "NHD")
    w.plan(dv.append_indptr, dv.indptr, dv.indices, dv.last, wb.hq, wb.hkv, wb.d, wb.ps, causal=True,
           q_data_type=wb.dtype)
    out = torch.empty_like(dv.q)
    if args.profile_launches:
        for _ in range(args.profile_launches):
            w.run(dv.q, dv.cache, out=out)
        torch.cuda.synchronize()
        print(json.dumps({"profile_launches": args.profile_launches, "work_items": w._n_items}), flush=True)
        return
    stream = torch.cuda.Stream(device=dev)

    def timed_graph(fn, reps, n, samples=5):
        with torch.cuda.stream(stream):
            fn()
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for _ in range(reps):
                    fn()
        return graph_time(torch, stream, g, n, reps, samples)

    t = timed_graph(lambda: w.run(dv.q, dv.cache, out=out), 10, max(1, args.steps // 10))
    t_valu = timed_graph(lambda: w.run(dv.q, dv.cache, out=out, force_valu=True), 1, 1, samples=1)
    C = wb.new_len[0]
    prefix = [L - n for L, n in zip(wb.kv_len, wb.new_len)]
    flops = 4 * wb.hq * wb.d * sum(C * p + C * (C + 1) // 2 for p in prefix)
    tfs = flops / t / 1e12
    # CPU baseline on a bounded sample (the reference's CPU path: gather, then causal SDPA with
    # the bottom-right offset, fp32) for the shortest request
    import torch.nn.functional as F
    from oracle import kv_ref
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    b = int(np.argmin(wb.kv_len))
    qo = wb.append_indptr.tolist()
    sample_q = wb.q[qo[b]:qo[b + 1]]
    kk, vv = kv_ref.gather(wb.cache.numpy() if wb.dtype == torch.float32 else wb.cache.float().numpy(),
                           wb.indices.numpy(), wb.indptr.numpy(), wb.last.numpy(), b, wb.ps)
    kk, vv = torch.from_numpy(kk).float(), torch.from_numpy(vv).float()
    L, qn = kk.shape[0], sample_q.shape[0]
    mask = torch.arange(L)[None, :] <= (torch.arange(qn)[:, None] + L - qn)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        F.scaled_dot_product_attention(sample_q.float().transpose(0, 1)[None], kk.transpose(0, 1)[None],
                                       vv.transpose(0, 1)[None], attn_mask=mask, enable_gqa=True)
        times.append(time.perf_counter() - t0)
    sample_flops = 4 * wb.hq * wb.d * (C * prefix[b] + C * (C + 1) // 2)
    result = {
        "metric": "chunked prefill attn TFLOP/s (% MFMA peak), Qwen2.5-3B 8 x 512-token chunks",
        "value": round(tfs, 2), "unit": "TFLOP/s", "n_gpus": 1, "higher_is_better": True,
        "dtype": "fp16", "data": "synthetic (seeded N(0,1)*0.5, random page permutation, NaN-poisoned pool)",
        "config": {"workload": "qwen2.5-3b chunked prefill, 1 layer, 8 requests x 512-token chunk onto prefix "
                               "U[0,8192], causal, page 16, 16 q / 2 kv heads, head_dim 128, fp16",
                   "requests": wb.batch, "q_rows": int(wb.q.shape[0]), "kv_tokens": sum(wb.kv_len),
                   "work_items": w._n_items, "split_groups": w._n_groups, "chunk_keys": w._chunk},
        "prefill_us": round(t * 1e6, 3), "prefill_valu_us": round(t_valu * 1e6, 3), "flops": flops,
        "roofline": {"bound": "mfma", "achieved": round(tfs, 2), "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tfs / MFMA_PEAK_TFLOPS, 4), "traffic": None},
        "cpu_baseline": {"value": round(sample_flops / statistics.median(times) / 1e12, 5), "unit": "TFLOP/s",
                         "cores": cores, "kind": "port",
                         "sample": f"request {b} ({qn} query rows over {L} keys): gather + fp32 causal SDPA, median of 3",
                         "cpu_model": cpu_model()},
    }
    return result


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(wb, reps=5):
    """The reference's CPU path on this host: torch index_put append, then per-sequence
    gather + fp32 SDPA (oracle.kv_ref.sdpa_decode)."""
    import torch
    from oracle import kv_ref

    n = min(len(os.sched_getaffinity(0)), 16)
    torch.set_num_threads(n)
    cache = wb.cache.clone()
    pos = wb.positions.long()
    pages = wb.indices[wb.indptr[wb.batch_indices.long()].long() + pos // wb.ps].long()
    slots = pos % wb.ps

    def do_append():
        cache[pages, 0, slots] = wb.k_new
        cache[pages, 1, slots] = wb.v_new

    def do_decode():
        return kv_ref.sdpa_decode(wb.q, cache, wb.indptr, wb.indices, wb.last, wb.ps)

    ta, td = [], []
    for i in range(reps + 2):
        t0 = time.perf_counter()
        do_append()
        t1 = time.perf_counter()
        do_decode()
        t2 = time.perf_counter()
        if i >= 2:
            ta.append(t1 - t0)
            td.append(t2 - t1)
    t_dec, t_app = statistics.median(td), statistics.median(ta)
    return {
        "value": round(decode_bytes(wb) / t_dec / 1e9, 3),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"full batch ({wb.batch} sequences, one layer): torch index_put append + "
                   f"per-sequence gather + fp32 SDPA, median of {reps}"),
        "decode_ms": round(t_dec * 1e3, 3),
        "append_mtok_s": round(wb.k_new.shape[0] / t_app / 1e6, 4),
        "cpu_model": cpu_model(),
    }


def parity(wb, out_dev, cache_dev=None):
    """The decode output against the float64 oracle on the oracle's appended cache; with
    cache_dev, that cache bit for bit against the device's after its append."""
    import numpy as np
    import torch
    from oracle import kv_ref

    iv = torch.int16
    raw = kv_ref.append(wb.cache.view(iv).numpy(), wb.k_new.view(iv).numpy(), wb.v_new.view(iv).numpy(),
                        wb.batch_indices.numpy(), wb.positions.numpy(), wb.indices.numpy(),
                        wb.indptr.numpy(), wb.ps)
    vals = torch.from_numpy(raw).view(wb.dtype).float().numpy()
    ref = kv_ref.decode(wb.q.float().numpy(), vals, wb.indptr.numpy(), wb.indices.numpy(),
                        wb.last.numpy(), wb.ps)
    got = out_dev.float().cpu().numpy()
    err = np.abs(got - ref)
    ok = bool(np.all(err <= 2e-3 + 1e-2 * np.abs(ref)))
    res = {"max_abs_err": float(err.max()), "within_atol2e-3_rtol1e-2": ok}
    if cache_dev is not None:
        res["append_bitexact"] = bool(np.array_equal(cache_dev.view(iv).cpu().numpy(), raw))
    return res


def extras(args, torch, runs):
    """The other hot-path workloads, each run in this process at its own default size after the
    headline's figures are taken, summarised as the line's "extras": chunked prefill (matrix-core
    bound), long-context decode, the 36-layer shared-prefix step and the bulk append.  Each
    entry carries that workload's own metric, value, roofline fraction and the times behind it;
    `bench.py --workload <name>` prints its full line."""
    sub = argparse.Namespace(**vars(args))
    sub.profile_launches, sub.ctas = 0, None
    keep = {
        "qwen25_3b_prefill": ("prefill_us", "prefill_valu_us", "flops"),
        "llama31_8b_b128": ("decode_us", "decode_bytes"),
        "qwen25_3b_step36": ("step_ms", "batch_change_ms", "graph_ms", "graph_back_to_back_ms", "graph_unique_gbs",
                             "parity"),
        "qwen25_3b_bulk_append": ("by_nnz",),
    }
    out = {}
    for name, fields in keep.items():
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        r = runs[name](sub)
        e = {"metric": r["metric"], "value": r["value"], "unit": r["unit"],
             "roofline_frac": r["roofline"]["frac"], "roofline_bound": r["roofline"]["bound"],
             "traffic": r["roofline"]["traffic"]}
        e.update({k: r[k] for k in fields})
        if name == "qwen25_3b_step36":
            e["device_steps"] = r["config"]["device_steps"]
        if "cpu_baseline" in r:
            e["cpu_baseline"] = {k: r["cpu_baseline"][k] for k in ("value", "unit", "cores", "kind")}
        out[name] = e
        print(f"bench: extras {name}: {e['value']} {e['unit']}", file=sys.stderr, flush=True)
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=4, help="layer pools rotated per step")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-check", action="store_true", help="skip the oracle parity check")
    ap.add_argument("--ctas", type=int, default=None, help="decode workgroups (default: one per CU)")
    ap.add_argument("--host-steps", action="store_true",
                    help="shared-prefix step: page-table bookkeeping on the host each step (the reference's loop)")
    ap.add_argument("--no-cascade", action="store_true",
                    help="shared-prefix step: plan without prefix items (every sequence reads the prefix, "
                         "kept in L2 by the hint)")
    ap.add_argument("--dynamic", action="store_true",
                    help="waves take pages on demand (faster, not bitwise reproducible)")
    ap.add_argument("--workload", default="qwen25_3b_b64",
                    choices=["qwen25_3b_b64", "llama31_8b_b128", "qwen25_3b_prefill", "qwen25_3b_step36",
                             "qwen25_3b_bulk_append",
                             "qwen25_3b_sampling", "qwen25_3b_rope_append"],
                    help="qwen25_3b_b64: the headline decode + append step (default); llama31_8b_b128: "
                         "long-context decode at Llama-3.1-8B shape, B=128, ~4.4 GB of K/V in a 20 GB pool "
                         "(decode only, generated on the device); qwen25_3b_prefill: chunked prefill, 8 "
                         "requests x 512-token chunks onto prefixes U[0, 8192] (the matrix-core roofline); "
                         "qwen25_3b_step36: the 36-layer graph-captured decode step, B=128, on a shared "
                         "2048-token prefix with pages allocated and freed by the device pool; "
                         "qwen25_3b_sampling: top-k/top-p sampling of 128 rows of the 151,936-token vocabulary; "
                         "qwen25_3b_rope_append: the model's rotary embedding fused with the append, "
                         "4096-token prefill chunk and B=64 decode step, against the unfused sequence; "
                         "qwen25_3b_bulk_append: the plain append of 4096 and 65536 tokens")
    ap.add_argument("--no-extras", action="store_true",
                    help="default workload only: skip the other workloads' summary (the line's 'extras')")
    ap.add_argument("--profile-launches", type=int, default=0, metavar="N",
                    help="for counter runs: N eager launches of the workload's kernel (the 36-layer "
                         "step: N steps), then N plain copies of its algorithmic byte count per launch "
                         "(the counters' calibration), then exit")
    ap.add_argument("--traffic-record", nargs=3, metavar=("FETCH_CSV", "WRITE_CSV", "PROFILE_LOG"),
                    help="write the workload's traffic record (profiles/*traffic.json) from the "
                         "counter_collection CSVs of a FETCH_SIZE and a WRITE_SIZE run of "
                         "--profile-launches and that run's output, then exit (no GPU needed)")
    args = ap.parse_args()
    if args.traffic_record:
        print(json.dumps(record_traffic(args.workload, *args.traffic_record)))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported "
              "(the paged-KV path is sharded by sequence across GPUs with no exchange; "
              "multi-GPU runs are not measured here)", file=sys.stderr)
        sys.exit(2)

    import torch
    from ecahlang_amd import ops, workloads
    from ecahlang_amd.wrappers import BatchDecodeWithPagedKVCacheWrapper

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    runs = {
        "qwen25_3b_b64": lambda a: headline(a, torch, workloads, ops, BatchDecodeWithPagedKVCacheWrapper, dev),
        "llama31_8b_b128": lambda a: long_context(a, torch, workloads, BatchDecodeWithPagedKVCacheWrapper, dev),
        "qwen25_3b_prefill": lambda a: chunked_prefill(a, torch, workloads, ops, dev),
        "qwen25_3b_step36": lambda a: step36(a, torch, workloads, dev),
        "qwen25_3b_sampling": lambda a: sampling(a, torch, dev),
        "qwen25_3b_rope_append": lambda a: rope_append(a, torch, workloads, ops, dev),
        "qwen25_3b_bulk_append": lambda a: bulk_append(a, torch, workloads, ops, dev),
    }
    result = runs[args.workload](args)
    if result is None:  # --profile-launches: the counter run prints its own record
        return
    if args.workload == "qwen25_3b_b64" and not args.no_extras:
        result["extras"] = extras(args, torch, runs)
    print(json.dumps(result), flush=True)


def headline(args, torch, workloads, ops, BatchDecodeWithPagedKVCacheWrapper, dev):
    """The default workload: append + decode of one Qwen2.5-3B layer at B = 64, rotated over
    --layers pools (the module docstring describes the line it returns)."""
    print("bench: building Qwen2.5-3B B=64 decode batch", file=sys.stderr, flush=True)
    wb = workloads.qwen25_3b_decode()
    NL = args.layers
    kv = torch.empty((NL,) + tuple(wb.cache.shape), dtype=wb.cache.dtype, device=dev)
    for l in range(NL):
        kv[l].copy_(wb.cache)
    dv = wb.to(dev)
    del dv.cache
    ws = torch.empty(128 << 20, dtype=torch.uint8, device=dev)
    w = BatchDecodeWithPagedKVCacheWrapper(ws, "NHD")
    w.plan(dv.indptr, dv.indices, dv.last, wb.hq, wb.hkv, wb.d, wb.ps, pos_encoding_mode="NONE",
           q_data_type=wb.dtype, num_ctas=args.ctas, deterministic=not args.dynamic)
    outs = [torch.empty_like(dv.q) for _ in range(NL)]

    def append(l):
        ops.append_paged_kv_cache(dv.k_new, dv.v_new, dv.batch_indices, dv.positions, kv[l],
                                  dv.indices, dv.indptr, dv.last)

    def decode(l):
        w.run(dv.q, kv[l], out=outs[l])

    # the vector-ALU kernel on the same batch, for comparison (its own default: 2 workgroups
    # per CU)
    wv = BatchDecodeWithPagedKVCacheWrapper(torch.empty(128 << 20, dtype=torch.uint8, device=dev), "NHD")
    wv.plan(dv.indptr, dv.indices, dv.last, wb.hq, wb.hkv, wb.d, wb.ps, pos_encoding_mode="NONE",
            q_data_type=wb.dtype, num_ctas=2 * w._ctas)

    def decode_valu(l):
        wv.run(dv.q, kv[l], out=outs[l], force_valu=True)

    def decode_append(l):  # the step's append fused into the decode launch
        w.run(dv.q, kv[l], out=outs[l], append_kv=(dv.k_new, dv.v_new))

    # eager warm-up; parity of the timed step's launch (the append fused into the decode) on
    # layer 0: the output against the oracle, the appended cache bit for bit, and the plain
    # decode of the appended cache bitwise equal to the fused output
    decode_append(0)
    fused_out = outs[0].clone()
    for l in range(NL):
        append(l)
        decode(l)
    torch.cuda.synchronize()
    par = None
    if not args.no_check:
        par = parity(wb, fused_out, kv[0])
        par["fused_equals_plain"] = bool(torch.equal(fused_out.view(torch.int16), outs[0].view(torch.int16)))
    print(f"bench: parity {par}", file=sys.stderr, flush=True)

    if args.profile_launches:
        n = args.profile_launches
        for i in range(n):
            append(i % NL)
            decode(i % NL)
        # plain copy of decode_bytes: reads and writes exactly that many bytes
        nb = decode_bytes(wb) // 16 * 16
        src = torch.empty(nb // 4, dtype=torch.int32, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(n):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"profile_launches": n, "kernel_dispatches": n, "algorithmic_bytes": decode_bytes(wb),
                          "copy_bytes": nb, "key": {"decode_ctas": w._ctas}}), flush=True)
        return None

    stream = torch.cuda.Stream(device=dev)

    def capture(fn):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            with torch.cuda.graph(g, stream=stream):
                fn()
        return g

    step_graphs = [capture(lambda l=l: decode_append(l)) for l in range(NL)]
    REP = 8  # launches per layer inside the per-kernel timing graphs
    dec_graph = capture(lambda: [decode(l) for _ in range(REP) for l in range(NL)])
    app_graph = capture(lambda: [append(l) for _ in range(REP) for l in range(NL)])
    fused_graph = capture(lambda: [decode_append(l) for _ in range(REP) for l in range(NL)])
    valu_graph = capture(lambda: [decode_valu(l) for l in range(NL)])
    torch.cuda.synchronize()

    def timed(fn, n):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            e0.record(stream)
            for i in range(n):
                fn(i)
            e1.record(stream)
        e1.synchronize()
        return e0.elapsed_time(e1) / 1e3

    # --- the contract's timed region: exactly K steps, after W warm-up steps
    with torch.cuda.stream(stream):
        for i in range(args.warmup):
            step_graphs[i % NL].replay()
    torch.cuda.synchronize()
    t_steps = timed(lambda i: step_graphs[i % NL].replay(), args.steps)
    torch.cuda.synchronize()

    # --- per-kernel averages: events around back-to-back graph-replayed launches of one
    # kernel, the median of 5 samples after a warm-up burst (the first milliseconds after the
    # GPU has idled run ~10 % slow, so a single sample taken then is not the kernel's rate)
    n_rep = max(3, args.steps // (REP * NL))

    t_dec = graph_time(torch, stream, dec_graph, n_rep, REP * NL)
    t_app = graph_time(torch, stream, app_graph, n_rep, REP * NL)
    t_fused = graph_time(torch, stream, fused_graph, n_rep, REP * NL)
    t_valu = graph_time(torch, stream, valu_graph, 1, NL, samples=1)
    torch.cuda.synchronize()

    dbytes = decode_bytes(wb)
    gbs = dbytes / t_dec / 1e9
    # the read rate a launch of the decode's size reaches here: the same bytes (four buffers in
    # turn), one workgroup per CU as the decode runs and the best of wider launches; and a 2 GiB
    # read for the sustained rate
    probe = {}
    for blocks in (w._ctas, 2 * w._ctas, 4 * w._ctas):
        probe[blocks] = dbytes / read_probe(torch, dev, stream, dbytes, NL, blocks) / 1e9
    best = max(probe, key=probe.get)
    large = 1 << 31
    large_gbs = large / read_probe(torch, dev, stream, large, 1, 4 * w._ctas, per_buf=8) / 1e9
    torch.cuda.synchronize()
    nnz = wb.k_new.shape[0]
    result = {
        "metric": "paged decode attn GB/s (% HBM peak) + KV append Mtok/s, Qwen2.5-3B B=64",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_steps / args.steps * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded N(0,1)*0.5 K/V/Q, random page permutation, NaN-poisoned pool)",
        "config": {
            "workload": "qwen2.5-3b paged decode, 1 layer, B=64, ctx U[512,4096], page 16, "
                        "16 q / 2 kv heads, head_dim 128, fp16, append 1 token/seq then decode "
                        "(one launch: the append fused into the decode)",
            "batch": wb.batch,
            "kv_tokens": sum(wb.kv_len),
            "pages": int(wb.indptr[-1]),
            "pool_pages": wb.num_pages,
            "layer_pools_rotated": NL,
            "decode_ctas": w._ctas,
            "decode_kernel": "mfma" if w._mfma else "valu",
        },
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "decode_us": round(t_dec * 1e6, 3),
        "decode_valu_us": round(t_valu * 1e6, 3),
        "decode_bytes": dbytes,
        "append_mtok_s": round(nnz / t_app / 1e6, 3),
        "append_us": round(t_app * 1e6, 3),
        "append_nnz": nnz,
        "decode_append_fused_us": round(t_fused * 1e6, 3),
        "hbm_read_probe": {
            "kernel": "pkv_probe_stream_read (1024-thread workgroups, 8 x 16-byte non-temporal loads in "
                      "flight per thread, contiguous slices)",
            "bytes": dbytes,
            "buffers_rotated": NL,
            "gbs_at_decode_ctas": round(probe[w._ctas], 2),
            "decode_ctas": w._ctas,
            "best_gbs": round(probe[best], 2),
            "best_blocks": best,
            "large_bytes": large,
            "large_gbs": round(large_gbs, 2),
            "decode_frac_of_best": round(gbs / probe[best], 4),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(wb, w),
        },
        "parity": par,
    }
    if not args.no_cpu:
        print("bench: CPU baseline", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(wb)
    return result


if __name__ == "__main__":
    main()
